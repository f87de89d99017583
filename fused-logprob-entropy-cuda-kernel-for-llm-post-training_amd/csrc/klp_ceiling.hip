// klp_ceiling.hip — calibration kernels: the memory access of the forward
// (klp_fwd_kernel) and of the backward (klp_bwd_kernel) without their
// arithmetic, over rows of the same size and with the same launch shapes.
//
//  kRead       the forward's access: each row piece streamed through the
//              forward's ring of register sets (kFwdRing - 1 chunks of U
//              non-temporal 16-byte buffer loads per thread in flight,
//              consecutive lanes on consecutive 16-byte words); the words
//              are xor-folded and the fold is stored only if it equals a
//              caller-given value, so the loads cannot be dropped and
//              nothing else is written in practice.
//  kCopy       the backward's access: buffer loads over the row piece
//              (temporal) and non-temporal 16-byte stores, pieces rounded up
//              to 8 vectors, U vectors per thread per iteration.
//  kReadPieces the backward's loads alone (its loop, no stores; folded as
//              kRead).
//  kWrite      the backward's stores alone (its loop, no loads; each vector
//              written with its own index).
//
// Timed next to the real kernels on the same device, they give the read,
// copy, read-only and write-only rates this device reaches for this size
// and shape, against which the kernels' own rates are judged.  The
// reference has no counterpart (its roofline uses the device's nominal
// peak, bench/plot_roofline.py).
#include "klp_device.h"
#include "klp_launch.h"

namespace klp {

template <int U, int NTHREADS>
__device__ __forceinline__ void ring_load(u32x4* dst, const __amdgpu_buffer_rsrc_t rs, int c,
                                          int tid) {
#pragma unroll
    for (int u = 0; u < U; ++u)
        dst[u] = __builtin_amdgcn_raw_buffer_load_b128(
            rs, ((c * U + u) * NTHREADS + tid) * 16, 0, kBufNonTemporal);
}

template <int U>
__device__ __forceinline__ uint32_t fold(const u32x4* v) {
    uint32_t a = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) a ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    return a;
}

// The forward's ring (scan_row_piece in klp_forward.hip) with the
// arithmetic replaced by the fold; row pieces as the forward cuts them
// (ceil(nvec / splits) vectors, not rounded).
template <int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) void klp_ceiling_read_kernel(CeilingParams p) {
    constexpr int NTHREADS = WAVES * 64;
    constexpr int step = NTHREADS * U;
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

    // The host keeps (piece + kFwdRing chunks) * 16 bytes under 2^31.
    const int n_full = static_cast<int>((ve - vb) / step);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<u32x4*>(vp + vb), 0, n_full * step * 16, 0x00020000);
    uint32_t acc = 0;
    u32x4 set[kFwdRing][U];
#pragma unroll
    for (int r = 0; r < kFwdRing - 1; ++r) ring_load<U, NTHREADS>(set[r], rs, r, tid);
    __builtin_amdgcn_sched_barrier(0);
    int k = 0;
    for (; k + kFwdRing <= n_full; k += kFwdRing) {
#pragma unroll
        for (int r = 0; r < kFwdRing; ++r) {
            ring_load<U, NTHREADS>(set[(r + kFwdRing - 1) % kFwdRing], rs, k + r + kFwdRing - 1,
                                   tid);
            __builtin_amdgcn_sched_barrier(0);
            acc ^= fold<U>(set[r]);
        }
    }
#pragma unroll
    for (int r = 0; r < kFwdRing - 1; ++r)
        if (k + r < n_full) acc ^= fold<U>(set[r]);
    const int64_t i = vb + static_cast<int64_t>(n_full) * step + tid;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t idx = i + u * NTHREADS;
        if (idx < ve) {
            const u32x4 v = load16<true>(vp + idx);
            acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
        }
    }
    if (acc == p.magic) p.sink[b] = acc;
}

// The backward's loop (klp_bwd_kernel): pieces rounded up to 8 vectors, U
// buffer loads then U non-temporal stores per thread per iteration.
template <int WAVES, int U, int kMode>
__device__ __forceinline__ void pieces_body(const CeilingParams& p) {
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
    uint32_t acc = 0;
    for (int64_t i0 = vb; i0 < ve; i0 += static_cast<int64_t>(NTHREADS) * U) {
        u32x4 v[U];
        if constexpr (kMode != kCeilWrite) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int64_t idx = i0 + tid + u * NTHREADS;
                if (idx < ve)
                    v[u] = __builtin_amdgcn_raw_buffer_load_b128(
                        rs, static_cast<int>((idx - vb) * 16), 0, 0);
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t idx = i0 + tid + u * NTHREADS;
            if (idx < ve) {
                if constexpr (kMode == kCeilCopy) {
                    __builtin_nontemporal_store(v[u], vout + idx);
                } else if constexpr (kMode == kCeilReadPieces) {
                    acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
                } else {
                    const uint32_t w = static_cast<uint32_t>(idx);
                    __builtin_nontemporal_store(u32x4{w, w, w, w}, vout + idx);
                }
            }
        }
    }
    if constexpr (kMode == kCeilReadPieces)
        if (acc == p.magic) p.sink[b] = acc;
}

template <int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) void klp_ceiling_copy_kernel(CeilingParams p) {
    pieces_body<WAVES, U, kCeilCopy>(p);
}
template <int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) void klp_ceiling_read_pieces_kernel(CeilingParams p) {
    pieces_body<WAVES, U, kCeilReadPieces>(p);
}
template <int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) void klp_ceiling_write_kernel(CeilingParams p) {
    pieces_body<WAVES, U, kCeilWrite>(p);
}

template <int W, int U>
static hipError_t launch_ceiling_wu(int mode, const CeilingParams& p, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(p.n_rows * p.splits));
    switch (mode) {
        case kCeilRead:
            return launch_kernel(klp_ceiling_read_kernel<W, U>, grid, dim3(W * 64), stream, p);
        case kCeilCopy:
            return launch_kernel(klp_ceiling_copy_kernel<W, U>, grid, dim3(W * 64), stream, p);
        case kCeilReadPieces:
            return launch_kernel(klp_ceiling_read_pieces_kernel<W, U>, grid, dim3(W * 64), stream,
                                 p);
        case kCeilWrite:
            return launch_kernel(klp_ceiling_write_kernel<W, U>, grid, dim3(W * 64), stream, p);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_ceiling(int mode, const CeilingParams& p, int waves, int unroll,
                          hipStream_t stream) {
#define KLP_CEIL_CASE(W, U) \
    if (waves == W && unroll == U) return launch_ceiling_wu<W, U>(mode, p, stream);
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
