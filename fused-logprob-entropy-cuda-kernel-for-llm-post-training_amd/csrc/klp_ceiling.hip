// klp_ceiling.hip — calibration kernels: the memory access of the forward
// (klp_fwd_kernel) and of the backward (klp_bwd_kernel) without their
// arithmetic, over rows of the same size and with the same launch shapes.
//
//  klp_ceiling_read_kernel  non-temporal 16-byte loads of every row piece,
//                           consecutive lanes on consecutive 16-byte words,
//                           U loads per thread per iteration (the forward's
//                           body loop); the words are xor-folded and the fold
//                           is stored only if it equals a caller-given value,
//                           so the loads cannot be dropped and nothing else
//                           is written in practice.
//  klp_ceiling_copy_kernel  buffer loads over the row piece (temporal) and
//                           non-temporal 16-byte stores, pieces rounded up to
//                           8 vectors (the backward's body loop).
//
// Timed next to the real kernels on the same device, they give the read and
// copy rates this device reaches for this size and shape, against which the
// kernels' own rates are judged.  The reference has no counterpart (its
// roofline uses the device's nominal peak, bench/plot_roofline.py).
#include "klp_device.h"
#include "klp_launch.h"

namespace klp {

template <int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) void klp_ceiling_read_kernel(CeilingParams p) {
    constexpr int NTHREADS = WAVES * 64;
    const int tid = threadIdx.x;
    const int64_t b = blockIdx.x;
    const int64_t row = b / p.splits;
    const int64_t split = b - row * p.splits;
    const u32x4* vp =
        reinterpret_cast<const u32x4*>(static_cast<const char*>(p.src) + row * p.row_bytes);
    const int64_t nvec = p.row_bytes / 16;
    const int64_t per = (nvec + p.splits - 1) / p.splits;
    int64_t vb = split * per;
    int64_t ve = vb + per;
    if (vb > nvec) vb = nvec;
    if (ve > nvec) ve = nvec;

    u32x4 acc = u32x4{0u, 0u, 0u, 0u};
    const int64_t step = static_cast<int64_t>(NTHREADS) * U;
    int64_t i = vb + tid;
    const int64_t n_full = (ve - vb) / step;
    for (int64_t k = 0; k < n_full; ++k) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = load16<true>(vp + i + u * NTHREADS);
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u];
        i += step;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t idx = i + u * NTHREADS;
        if (idx < ve) acc ^= load16<true>(vp + idx);
    }
    const uint32_t fold = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
    if (fold == p.magic) p.sink[b] = fold;
}

template <int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) void klp_ceiling_copy_kernel(CeilingParams p) {
    constexpr int NTHREADS = WAVES * 64;
    const int tid = threadIdx.x;
    const int64_t b = blockIdx.x;
    const int64_t row = b / p.splits;
    const int64_t split = b - row * p.splits;
    const u32x4* vin =
        reinterpret_cast<const u32x4*>(static_cast<const char*>(p.src) + row * p.row_bytes);
    u32x4* vout = reinterpret_cast<u32x4*>(static_cast<char*>(p.dst) + row * p.row_bytes);
    const int64_t nvec = p.row_bytes / 16;
    int64_t per = (nvec + p.splits - 1) / p.splits;
    per = (per + 7) & ~int64_t{7};
    int64_t vb = split * per;
    int64_t ve = vb + per;
    if (vb > nvec) vb = nvec;
    if (ve > nvec) ve = nvec;

    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<u32x4*>(vin + vb), 0, static_cast<int>((ve - vb) * 16), 0x00020000);
    for (int64_t i0 = vb; i0 < ve; i0 += static_cast<int64_t>(NTHREADS) * U) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t idx = i0 + tid + u * NTHREADS;
            if (idx < ve)
                v[u] = __builtin_amdgcn_raw_buffer_load_b128(
                    rs, static_cast<int>((idx - vb) * 16), 0, 0);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t idx = i0 + tid + u * NTHREADS;
            if (idx < ve) __builtin_nontemporal_store(v[u], vout + idx);
        }
    }
}

template <int W, int U>
static hipError_t launch_ceiling_wu(bool copy, const CeilingParams& p, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(p.n_rows * p.splits));
    if (copy) return launch_kernel(klp_ceiling_copy_kernel<W, U>, grid, dim3(W * 64), stream, p);
    return launch_kernel(klp_ceiling_read_kernel<W, U>, grid, dim3(W * 64), stream, p);
}

hipError_t launch_ceiling(bool copy, const CeilingParams& p, int waves, int unroll,
                          hipStream_t stream) {
#define KLP_CEIL_CASE(W, U) \
    if (waves == W && unroll == U) return launch_ceiling_wu<W, U>(copy, p, stream);
    KLP_CEIL_CASE(1, 2)
    KLP_CEIL_CASE(1, 4)
    KLP_CEIL_CASE(2, 2)
    KLP_CEIL_CASE(2, 4)
    KLP_CEIL_CASE(4, 2)
    KLP_CEIL_CASE(4, 4)
    KLP_CEIL_CASE(8, 2)
    KLP_CEIL_CASE(8, 4)
    KLP_CEIL_CASE(16, 2)
    KLP_CEIL_CASE(16, 4)
#undef KLP_CEIL_CASE
    return hipErrorInvalidValue;
}

}  // namespace klp
