// klp_backward.hip — backward kernel for gfx950 (replaces the reference's
// fused_logprob_entropy_v1_backward_kernel, csrc/fused_logprob.cu:243-282).
//
// For every element of a row:
//   lp = x - lse,  p = exp(lp),
//   d  = p * (c0 - g_ent * lp) + (v == t ? g_logp : 0),
//   c0 = g_lse - g_logp - g_ent * H          (hoisted per row, as at :271)
// One 16-byte load and one 16-byte store per 16 bytes of logits; nothing else
// touches memory except eight per-row scalars.
//
// p is computed as 2^(x*log2e - lse*log2e) with lse*log2e split into a
// rounded head and its exact fma remainder, so the exponent carries one
// rounding.  A -inf logit gets a gradient of exactly 0 (p = 0), where the
// reference's 0 * inf gives NaN; lp is clamped for that.
//
// With a temperature T (BwdParams::scale = 1/T != 1) the logits are scaled by
// 1/T on load, as in the forward, and the gradient is multiplied by 1/T.
#include "klp_device.h"
#include "klp_launch.h"

namespace klp {

// The piece's 16-byte vectors [vb, ve) (the body of klp_bwd_kernel).
template <int DT, int WAVES, int U, bool kNtStore, bool kScaled, bool kLseNonNeg>
__device__ __forceinline__ void bwd_vectors(const BwdParams& p, const u32x4* vin, u32x4* vout,
                                            int64_t vb, int64_t ve, int64_t t_vec,
                                            int t_lane_elem, const RowGrad& g) {
    constexpr int NTHREADS = WAVES * 64;
    constexpr int EPV = Traits<DT>::kPerVec;
    const int tid = threadIdx.x;
    // Buffer loads through a descriptor over the piece, with 32-bit offsets
    // (the caller keeps pieces under 2 GiB): C4 3113-3132 us against
    // 3166-3195 us for global loads of the same policy, C2 equal.  Temporal
    // loads here (non-temporal in the forward): measured best for a forward
    // followed by a backward over the same logits.
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
            if (idx < ve) {
                float x[EPV];
                unpack<DT>(v[u], x);
#pragma unroll
                for (int j = 0; j < EPV; ++j)
                    x[j] = grad_elem<DT, kLseNonNeg>(kScaled ? x[j] * p.scale : x[j], g);
                if (idx == t_vec) {
#pragma unroll
                    for (int j = 0; j < EPV; ++j)
                        if (j == t_lane_elem) x[j] += g.g_logp;
                }
                if (kScaled) {
#pragma unroll
                    for (int j = 0; j < EPV; ++j) x[j] *= p.scale;
                }
                if constexpr (kNtStore) __builtin_nontemporal_store(pack<DT>(x), vout + idx);
                else vout[idx] = pack<DT>(x);
            }
        }
    }
}

template <int DT, int WAVES, int U, bool kNtStore, bool kScaled>
__global__ __launch_bounds__(WAVES * 64) void klp_bwd_kernel(BwdParams p) {
    typedef typename Traits<DT>::elem elem;
    constexpr int NTHREADS = WAVES * 64;
    constexpr int EPV = Traits<DT>::kPerVec;
    constexpr int ESZ = 16 / EPV;

    const int tid = threadIdx.x;
    const int64_t row = static_cast<int64_t>(blockIdx.x) / p.splits;
    const int split = static_cast<int>(static_cast<int64_t>(blockIdx.x) - row * p.splits);

    const int64_t vocab = p.vocab;
    const elem* rp = static_cast<const elem*>(p.logits) + row_offset(p.rm, row);
    elem* dp = static_cast<elem*>(p.d_logits) + row * vocab;
    const int64_t tgt = p.targets[row];

    const RowGrad g = row_grad(p.lse[row], p.entropy[row], p.g_logp ? p.g_logp[row] : 0.0f,
                               p.g_ent ? p.g_ent[row] : 0.0f, p.g_lse ? p.g_lse[row] : 0.0f);

    const uintptr_t in_addr = reinterpret_cast<uintptr_t>(rp);
    const uintptr_t out_addr = reinterpret_cast<uintptr_t>(dp);
    if (((in_addr ^ out_addr) & 15u) != 0) {
        // Input and output rows sit at different offsets within 16 bytes, so
        // they cannot both be read/written as aligned vectors: scalar path.
        const int64_t per = (vocab + p.splits - 1) / p.splits;
        int64_t b = static_cast<int64_t>(split) * per;
        int64_t e = b + per;
        if (e > vocab) e = vocab;
        for (int64_t v = b + tid; v < e; v += NTHREADS) {
            float x = to_f32<DT>(rp[v]);
            if (kScaled) x *= p.scale;
            float d = g.lse >= 0.0f ? grad_elem<DT, true>(x, g) : grad_elem<DT, false>(x, g);
            if (v == tgt) d += g.g_logp;
            if (kScaled) d *= p.scale;
            dp[v] = from_f32<DT>(d);
        }
        return;
    }

    int64_t head = static_cast<int64_t>(((16u - (in_addr & 15u)) & 15u) / ESZ);
    if (head > vocab) head = vocab;
    const int64_t nvec = (vocab - head) / EPV;
    const int64_t tail_begin = head + nvec * EPV;

    if (split == 0) {
        const int64_t n_edge = head + (vocab - tail_begin);
        if (tid < n_edge) {
            const int64_t v = (tid < head) ? tid : tail_begin + (tid - head);
            float x = to_f32<DT>(rp[v]);
            if (kScaled) x *= p.scale;
            float d = g.lse >= 0.0f ? grad_elem<DT, true>(x, g) : grad_elem<DT, false>(x, g);
            if (v == tgt) d += g.g_logp;
            if (kScaled) d *= p.scale;
            dp[v] = from_f32<DT>(d);
        }
    }

    const u32x4* vin = reinterpret_cast<const u32x4*>(rp + head);
    u32x4* vout = reinterpret_cast<u32x4*>(dp + head);
    // Pieces are whole multiples of 8 vectors (128 bytes, one cache line
    // when the row is line-aligned), so that no line is written, or read,
    // by two workgroups (C4's 18992-vector rows in 8 pieces would otherwise
    // split a line at every boundary: +1.2% HBM writes).
    int64_t per = (nvec + p.splits - 1) / p.splits;
    per = (per + 7) & ~int64_t{7};
    int64_t vb = static_cast<int64_t>(split) * per;
    int64_t ve = vb + per;
    if (vb > nvec) vb = nvec;
    if (ve > nvec) ve = nvec;

    // Vector index holding the target's one-hot term (or -1).
    const int64_t t_rel = tgt - head;
    const int64_t t_vec = (tgt >= head && tgt < tail_begin) ? t_rel / EPV : -1;
    const int t_lane_elem = (t_vec >= 0) ? static_cast<int>(t_rel - t_vec * EPV) : 0;

    // fp32 rows take their Fast2Sum operand order from the sign of lse
    // (grad_one_fp32): one branch per row, outside the element loop.
    if constexpr (DT == kFP32) {
        if (g.lse >= 0.0f)
            bwd_vectors<DT, WAVES, U, kNtStore, kScaled, true>(p, vin, vout, vb, ve, t_vec,
                                                               t_lane_elem, g);
        else
            bwd_vectors<DT, WAVES, U, kNtStore, kScaled, false>(p, vin, vout, vb, ve, t_vec,
                                                                t_lane_elem, g);
    } else {
        bwd_vectors<DT, WAVES, U, kNtStore, kScaled, true>(p, vin, vout, vb, ve, t_vec,
                                                           t_lane_elem, g);
    }
}

template <int DT, int WAVES, int U, bool kNtStore>
static hipError_t launch_bwd_t(const BwdParams& p, hipStream_t stream) {
    if (p.scale != 1.0f)
        return launch_kernel(klp_bwd_kernel<DT, WAVES, U, kNtStore, true>,
                             dim3(static_cast<unsigned>(p.n_rows * p.splits)),
                             dim3(WAVES * 64), stream, p);
    return launch_kernel(klp_bwd_kernel<DT, WAVES, U, kNtStore, false>,
                         dim3(static_cast<unsigned>(p.n_rows * p.splits)), dim3(WAVES * 64),
                         stream, p);
}

template <int DT>
static hipError_t launch_bwd_dt(const BwdParams& p, const BwdConfig& c, hipStream_t stream) {
    const bool nt = (c.flags & kFlagNtStore) != 0;
#define KLP_BWD_CASE(W, U)                                                     \
    if (c.waves == W && c.unroll == U)                                         \
        return nt ? launch_bwd_t<DT, W, U, true>(p, stream)                \
                  : launch_bwd_t<DT, W, U, false>(p, stream);
    KLP_BWD_CASE(4, 2)
    KLP_BWD_CASE(4, 4)
    KLP_BWD_CASE(8, 2)
    KLP_BWD_CASE(8, 4)
    KLP_BWD_CASE(16, 2)
    KLP_BWD_CASE(16, 4)
#undef KLP_BWD_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_bwd(int dtype, const BwdParams& p, const BwdConfig& c, hipStream_t stream) {
    switch (dtype) {
        case kBF16: return launch_bwd_dt<kBF16>(p, c, stream);
        case kFP16: return launch_bwd_dt<kFP16>(p, c, stream);
        case kFP32: return launch_bwd_dt<kFP32>(p, c, stream);
        default: return hipErrorInvalidValue;
    }
}

bool bwd_config_supported(const BwdConfig& c) {
    const bool w = (c.waves == 4 || c.waves == 8 || c.waves == 16);
    const bool u = (c.unroll == 2 || c.unroll == 4);
    return w && u && (c.flags & ~kFlagNtStore) == 0;
}

}  // namespace klp
