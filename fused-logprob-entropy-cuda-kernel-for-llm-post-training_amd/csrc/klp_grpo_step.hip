// klp_grpo_step.hip — the GRPO step's logprob forward, loss gradient and
// logprob backward in one pass over the logits, for gfx950.
//
// In a GRPO step the upstream gradient of a token's log-probability depends
// only on that token: d loss / d logp_t = w_t * dl_t(logp_t; old_t, A_t,
// ref_t) with a per-token weight w_t known in advance (mask / normaliser),
// and the entropy is not differentiated.  So once a row's logsumexp is known,
// its d_logits can be written at once (klp_bwd's formula with
// g_logp = w_t * dl_t, g_ent = g_lse = 0):
//   d[v] = (onehot(v == t) - p_v) * g_logp          (times 1/T).
// The unfused step reads the logits twice (forward, backward) and writes
// d_logits once; here one workgroup of 1024 threads keeps its whole row in
// registers, so the logits are read once: 2 passes of HBM traffic instead
// of 3.  A thread holds up to kGrpoStepMaxVec = 19 16-byte vectors (76 of the
// 128 VGPRs a 1024-thread workgroup allows; 20 spill): 304 KB per row, a
// bf16 row of V <= 155648 or an fp32 row of V <= 77824.
//
// Per workgroup (one row):
//  1. load the row into registers (16-byte buffer loads, non-temporal);
//  2. per-thread online (m, z, t) state (absorb(), as klp_fwd), the wave
//     reduction, and the 16 wave states through LDS, merged by wave 0 with
//     one DPP row reduction;
//  3. logprob, entropy, lse of the row; the GRPO terms of the token
//     (grpo_token_loss, shared with klp_grpo.hip; its inputs read at the
//     start); loss_tok = w_t * loss_t;
//  4. d_logits from the registers (klp_bwd's gradient, which with g_ent = 0
//     is p * (-g_logp) plus the one-hot term), non-temporal 16-byte buffer
//     stores.
// Rows too long for the registers, or whose start or length is not a whole
// number of 16-byte vectors, are rejected by the caller (KLP_EINVAL), which
// then runs the unfused kernels.
#include "klp_grpo_terms.h"
#include "klp_launch.h"

namespace klp {

namespace {

constexpr int kStepThreads = kGrpoStepThreads;
constexpr int kStepWaves = kStepThreads / 64;
constexpr int kCachePolicyNt = 2;  // the "nt" (non-temporal) cache-policy bit

// Raw buffer resource over one row of `bytes` bytes: lanes past the end read
// 0 without touching memory, and their stores are dropped.  Word 3
// (0x00020000) is the gfx9-family descriptor default for dword data.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0,
                                             static_cast<int>(bytes), 0x00020000);
}

}  // namespace

template <int DT, int NV, bool kScaled>
__global__ __launch_bounds__(kStepThreads) void klp_grpo_step_kernel(GrpoStepParams p) {
    typedef typename Traits<DT>::elem elem;
    constexpr int EPV = Traits<DT>::kPerVec;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t row = blockIdx.x;
    const elem* rp = static_cast<const elem*>(p.logits) + row_offset(p.rm, row);
    const uint32_t nvec = static_cast<uint32_t>(p.vocab / EPV);
    const uint32_t row_bytes = nvec * 16u;
    // Vectors k < n_full exist for every thread; vector n_full only for some.
    const int n_full = static_cast<int>(nvec / kStepThreads);
    const bool has_tail = static_cast<uint32_t>(tid) < nvec - n_full * kStepThreads;
    const uint32_t pad = Traits<DT>::kNegInfWord;

    // Vector k of this thread is the row's vector tid + k * kStepThreads.
    // Every load is issued, unconditionally: a load skipped on some path
    // leaves the number of loads in flight unknown, and the compiler then
    // waits for all of them before the first use (no overlap of the scan
    // with the row's arrival).  Past the row's end the buffer descriptor
    // returns zeros without a memory access.
    const __amdgpu_buffer_rsrc_t rs = row_rsrc(rp, row_bytes);
    // The loads are issued in the order the scan uses them (the scheduling
    // fences keep them so).
    u32x4 r[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        r[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, (tid + k * kStepThreads) * 16, 0,
                                                     kCachePolicyNt);
        __builtin_amdgcn_sched_barrier(0);
    }
    const int64_t tgt = p.targets[row];
    const bool has_t = tgt >= 0 && tgt < p.vocab;
    // The token's GRPO inputs, read now: their latency hides behind the
    // row's loads instead of stalling the workgroup after the reduction.
    const float wt = p.tok_weight[row];
    const float old_lp = p.old_logp[row];
    const float adv = p.adv[p.adv_per_token ? row : row / p.seq_len];
    const bool has_ref = p.ref_logp != nullptr && p.beta != 0.0f;
    const float ref_lp = has_ref ? p.ref_logp[row] : 0.0f;

    // Pass 1 over the registers.  A lane whose own values include -inf
    // redoes its scan with -inf excluded (the reference's sentinel rule,
    // csrc/fused_logprob.cu:142-143), as klp_fwd does.
    auto scan = [&](auto clamp_tag) {
        constexpr bool kClamp = decltype(clamp_tag)::value;
        Stat s = stat_empty();
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            if (k > n_full) break;
            // Vector k's work stays after vector k-1's: hoisting any of it
            // (the select below, say) makes the first wait one for the
            // whole row.
            __builtin_amdgcn_sched_barrier(0);
            float x[EPV];
            // Lanes past the row's end in vector n_full read zeros: -inf.
            unpack<DT>((k < n_full || has_tail) ? r[k] : u32x4{pad, pad, pad, pad}, x);
            if (kScaled) {
#pragma unroll
                for (int j = 0; j < EPV; ++j) x[j] *= p.scale;
            }
            if (k < n_full) absorb<EPV, kClamp>(s, x);
            else absorb<EPV, true>(s, x);  // padding of the last vector is -inf
        }
        return s;
    };
    Stat s = scan(std::false_type{});
    if (needs_clamped_rescan(s)) s = scan(std::true_type{});

    // The target logit comes from the registers: the thread holding it
    // publishes it (a global load issued after the row's loads would make
    // every wave wait for the whole row before its scan).
    __shared__ Stat wave_stat[kStepWaves];
    __shared__ float target_logit;
    __shared__ float row_vals[3];  // lse, entropy, g_logp
    if (has_t) {
        const int64_t tv = tgt / EPV;
        if (static_cast<int>(tv % kStepThreads) == tid) {
            const int kt = static_cast<int>(tv / kStepThreads);
            const int jt = static_cast<int>(tgt - tv * EPV);
            float xt = 0.0f;
#pragma unroll
            for (int k = 0; k < NV; ++k) {
                if (k == kt) {
                    float x[EPV];
                    unpack<DT>(r[k], x);
#pragma unroll
                    for (int j = 0; j < EPV; ++j)
                        if (j == jt) xt = x[j];
                }
            }
            target_logit = kScaled ? xt * p.scale : xt;
        }
    }
    s = wave_reduce(s);
    if (lane == 0) wave_stat[wave] = s;
    __syncthreads();
    // Wave 0 merges the 16 wave states (each of its 16-lane DPP rows reads
    // all of them and reduces them, every lane ending with the same bits),
    // computes the row's results and the token's GRPO terms, and hands the
    // backward's constants to the other waves through LDS.
    static_assert(kStepWaves == 16, "one wave state per lane of a DPP row");
    if (wave == 0) {
        const RowOut o =
            finalize(row_reduce(wave_stat[lane & 15]), has_t ? target_logit : 0.0f);
        // GRPO terms of this token (token-level importance weight).
        const TokenLoss tl =
            grpo_token_loss(p.eps_low, p.eps_high, p.beta, o.logp - old_lp, adv, o.logp,
                            ref_lp, has_ref);
        const float g_logp = wt * (tl.dw + tl.dlp);
        if (lane == 0) {
            p.logprob[row] = o.logp;
            p.entropy[row] = o.ent;
            if (p.lse) p.lse[row] = o.lse;
            p.loss_tok[row] = wt * tl.loss;
            row_vals[0] = o.lse;
            row_vals[1] = o.ent;
            row_vals[2] = g_logp;
        }
    }
    __syncthreads();

    // Pass 2: d_logits from the registers.
    const RowGrad g = row_grad(row_vals[0], row_vals[1], row_vals[2], 0.0f, 0.0f);
    // Stores past the row's end are dropped by the descriptor.
    const __amdgpu_buffer_rsrc_t ds =
        row_rsrc(static_cast<elem*>(p.d_logits) + row * p.vocab, row_bytes);
    // Vector index holding the target's one-hot term (or none).
    const uint32_t t_vec = has_t ? static_cast<uint32_t>(tgt / EPV) : 0xFFFFFFFFu;
    const int t_elem = has_t ? static_cast<int>(tgt % EPV) : 0;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const uint32_t i = tid + k * kStepThreads;
        if (k > n_full) break;
        float x[EPV];
        unpack<DT>(r[k], x);
        // klp_bwd's gradient with g_ent = g_lse = 0 (grad_one_logp_only).
#pragma unroll
        for (int j = 0; j < EPV; ++j)
            x[j] = grad_one_logp_only(kScaled ? x[j] * p.scale : x[j], g);
        if (i == t_vec) {
#pragma unroll
            for (int j = 0; j < EPV; ++j)
                if (j == t_elem) x[j] += g.g_logp;
        }
        if (kScaled) {
#pragma unroll
            for (int j = 0; j < EPV; ++j) x[j] *= p.scale;
        }
        __builtin_amdgcn_raw_buffer_store_b128(pack<DT>(x), ds, i * 16u, 0, kCachePolicyNt);
    }
}

template <int DT, int NV>
static hipError_t launch_step_nv(const GrpoStepParams& p, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(p.n_rows));
    if (p.scale != 1.0f)
        return launch_kernel(klp_grpo_step_kernel<DT, NV, true>, grid, dim3(kStepThreads), stream,
                             p);
    return launch_kernel(klp_grpo_step_kernel<DT, NV, false>, grid, dim3(kStepThreads), stream,
                         p);
}

template <int DT>
static hipError_t launch_step_dt(const GrpoStepParams& p, hipStream_t stream) {
    const int64_t nvec = p.vocab / Traits<DT>::kPerVec;
    const int64_t nv = (nvec + kStepThreads - 1) / kStepThreads;
    if (nv <= 4) return launch_step_nv<DT, 4>(p, stream);
    if (nv <= 8) return launch_step_nv<DT, 8>(p, stream);
    if (nv <= 12) return launch_step_nv<DT, 12>(p, stream);
    if (nv <= 16) return launch_step_nv<DT, 16>(p, stream);
    if (nv <= kGrpoStepMaxVec) return launch_step_nv<DT, kGrpoStepMaxVec>(p, stream);
    return hipErrorInvalidValue;
}

hipError_t launch_grpo_step(int dtype, const GrpoStepParams& p, hipStream_t stream) {
    switch (dtype) {
        case kBF16: return launch_step_dt<kBF16>(p, stream);
        case kFP16: return launch_step_dt<kFP16>(p, stream);
        case kFP32: return launch_step_dt<kFP32>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace klp
