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
//  1. load the row into registers (16-byte loads, non-temporal);
//  2. per-thread online (m, z, t) state (absorb(), as klp_fwd), the wave
//     reduction and the 16 waves in order through LDS;
//  3. logprob, entropy, lse of the row; the GRPO terms of the token
//     (grpo_token_loss, shared with klp_grpo.hip); loss_tok = w_t * loss_t;
//  4. d_logits from the registers (klp_bwd's gradient, which with g_ent = 0
//     is p * (-g_logp) plus the one-hot term), non-temporal 16-byte stores.
// Rows too long for the registers, or whose start or length is not a whole
// number of 16-byte vectors, are rejected by the caller (KLP_EINVAL), which
// then runs the unfused kernels.
#include "klp_grpo_terms.h"
#include "klp_launch.h"

namespace klp {

namespace {

constexpr int kStepThreads = kGrpoStepThreads;
constexpr int kStepWaves = kStepThreads / 64;

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
    // Vector k of this thread is the row's vector tid + k * kStepThreads.
    // Addresses are the workgroup-uniform row start plus a 32-bit byte
    // offset, so the compiler keeps one 64-bit base in scalar registers
    // instead of a 64-bit address per vector in vector registers.
    const char* rbase = reinterpret_cast<const char*>(rp);
    const uint32_t nvec = static_cast<uint32_t>(p.vocab / EPV);
    // Vectors k < n_full exist for every thread; vector n_full only for some.
    const int n_full = static_cast<int>(nvec / kStepThreads);

    u32x4 r[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const uint32_t i = tid + k * kStepThreads;
        const uint32_t w = Traits<DT>::kNegInfWord;
        r[k] = (i < nvec) ? load16<true>(reinterpret_cast<const u32x4*>(rbase + i * 16u))
                          : u32x4{w, w, w, w};
    }
    const int64_t tgt = p.targets[row];
    const bool has_t = tgt >= 0 && tgt < p.vocab;
    // The target logit is read directly, as in klp_fwd; issued early so that
    // its latency hides behind the scan.
    float x_target = 0.0f;
    if (tid == 0 && has_t) x_target = to_f32<DT>(rp[tgt]) * p.scale;

    // Pass 1 over the registers.  A lane whose own values include -inf
    // redoes its scan with -inf excluded (the reference's sentinel rule,
    // csrc/fused_logprob.cu:142-143), as klp_fwd does.
    auto scan = [&](auto clamp_tag) {
        constexpr bool kClamp = decltype(clamp_tag)::value;
        Stat s = stat_empty();
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            if (k > n_full) break;
            float x[EPV];
            unpack<DT>(r[k], x);
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

    __shared__ Stat wave_stat[kStepWaves];
    __shared__ float row_vals[3];  // lse, entropy, g_logp
    s = wave_reduce(s);
    if (lane == 0) wave_stat[wave] = s;
    __syncthreads();
    if (tid == 0) {
        Stat acc = wave_stat[0];
#pragma unroll
        for (int w = 1; w < kStepWaves; ++w) acc = combine(acc, wave_stat[w]);
        const RowOut o = finalize(acc, x_target);
        // GRPO terms of this token (token-level importance weight).
        const float wt = p.tok_weight[row];
        const int64_t b = row / p.seq_len;
        const float adv = p.adv_per_token ? p.adv[row] : p.adv[b];
        const bool has_ref = p.ref_logp != nullptr && p.beta != 0.0f;
        const TokenLoss tl = grpo_token_loss(p.eps_low, p.eps_high, p.beta,
                                             o.logp - p.old_logp[row], adv, o.logp,
                                             has_ref ? p.ref_logp[row] : 0.0f, has_ref);
        const float g_logp = wt * (tl.dw + tl.dlp);
        p.logprob[row] = o.logp;
        p.entropy[row] = o.ent;
        if (p.lse) p.lse[row] = o.lse;
        p.loss_tok[row] = wt * tl.loss;
        row_vals[0] = o.lse;
        row_vals[1] = o.ent;
        row_vals[2] = g_logp;
    }
    __syncthreads();

    // Pass 2: d_logits from the registers.
    const RowGrad g = row_grad(row_vals[0], row_vals[1], row_vals[2], 0.0f, 0.0f);
    char* dbase = reinterpret_cast<char*>(static_cast<elem*>(p.d_logits) + row * p.vocab);
    // Vector index holding the target's one-hot term (or none).
    const uint32_t t_vec = has_t ? static_cast<uint32_t>(tgt / EPV) : 0xFFFFFFFFu;
    const int t_elem = has_t ? static_cast<int>(tgt % EPV) : 0;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const uint32_t i = tid + k * kStepThreads;
        if (k > n_full || i >= nvec) break;
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
        __builtin_nontemporal_store(pack<DT>(x), reinterpret_cast<u32x4*>(dbase + i * 16u));
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
