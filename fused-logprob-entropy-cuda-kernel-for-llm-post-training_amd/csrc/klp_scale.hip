// klp_scale.hip — in-place scaling of a buffer by a float held in device
// memory (klp_scale_inplace), for gfx950.
//
// The fused GRPO step and the chunked LM head compute their gradients in the
// forward; the backward only multiplies them by the loss's upstream gradient.
// That scalar lives on the device; reading it on the host would stall the
// caller's stream (a synchronisation in every backward).  This kernel reads
// it itself.  The buffer may already hold the gradients scaled by the
// upstream gradient the caller declared in advance (`applied`, 1 when none
// was): when the scalar equals it (loss.backward() on the loss, or the
// declared 1 / gradient-accumulation steps) every workgroup returns at once
// and nothing is written; otherwise each element is multiplied in fp32 by
// scalar / applied (the scalar itself when applied is 1) and rounded once to
// its dtype (RNE), as torch's `tensor * float` does.
#include "klp_launch.h"

namespace klp {

namespace {

constexpr int kScaleThreads = 256;
constexpr int64_t kScaleMaxBlocks = 4096;

template <int DT>
__global__ __launch_bounds__(kScaleThreads) void klp_scale_kernel(ScaleParams p) {
    const float g = *p.scale;
    if (g == p.applied) return;
    const float s = g / p.applied;  // g itself when applied is 1
    typedef typename Traits<DT>::elem elem;
    constexpr int EPV = Traits<DT>::kPerVec;
    elem* e = static_cast<elem*>(p.data);
    const int64_t tid = static_cast<int64_t>(blockIdx.x) * kScaleThreads + threadIdx.x;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kScaleThreads;
    // Elements before the first 16-byte boundary and after the last whole
    // vector, one per thread.
    const int64_t tail_begin = p.head + p.nvec * EPV;
    if (tid < p.head + (p.n - tail_begin)) {
        const int64_t i = tid < p.head ? tid : tail_begin + (tid - p.head);
        e[i] = from_f32<DT>(to_f32<DT>(e[i]) * s);
    }
    u32x4* v = reinterpret_cast<u32x4*>(e + p.head);
    for (int64_t i = tid; i < p.nvec; i += stride) {
        float x[EPV];
        unpack<DT>(v[i], x);
#pragma unroll
        for (int j = 0; j < EPV; ++j) x[j] *= s;
        v[i] = pack<DT>(x);
    }
}

}  // namespace

hipError_t launch_scale(int dtype, const ScaleParams& p, hipStream_t stream) {
    const int64_t work = p.nvec > 0 ? p.nvec : 1;
    int64_t blocks = (work + kScaleThreads - 1) / kScaleThreads;
    if (blocks > kScaleMaxBlocks) blocks = kScaleMaxBlocks;
    const dim3 grid(static_cast<unsigned>(blocks));
    switch (dtype) {
        case kBF16: return launch_kernel(klp_scale_kernel<kBF16>, grid, dim3(kScaleThreads),
                                         stream, p);
        case kFP16: return launch_kernel(klp_scale_kernel<kFP16>, grid, dim3(kScaleThreads),
                                         stream, p);
        case kFP32: return launch_kernel(klp_scale_kernel<kFP32>, grid, dim3(kScaleThreads),
                                         stream, p);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace klp
