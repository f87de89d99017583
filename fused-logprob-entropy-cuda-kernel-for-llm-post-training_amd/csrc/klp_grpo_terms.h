// klp_grpo_terms.h — the per-token terms of the GRPO policy loss, shared by
// the loss kernels (klp_grpo.hip) and the fused GRPO step (klp_grpo_step.hip).
// The loss is the one written out in the reference's
// examples/compare_one_step.py:232-236, with the KL term and the separate
// clip bounds of TRL's GRPOTrainer (see include/kernel_opt_hip.h, klp_grpo_fwd).
#pragma once

#include <hip/hip_runtime.h>

namespace klp {

struct TokenLoss {
    float loss;   // per-token loss
    float dw;     // d loss / d w (w = the log importance weight)
    float dlp;    // d loss / d lp through the KL term only
    float kl;     // KL estimate (0 when beta == 0 or no reference)
    float low;    // 1 if clipped at 1 - eps_low with A < 0
    float high;   // 1 if clipped at 1 + eps_high with A > 0
};

// w = log importance weight, adv = advantage, lp = new log-probability,
// lr = reference log-probability (used when has_ref).  The gradient follows
// PyTorch's conventions for the eager expression: a tie of min() sends half
// to each side, clamp() passes the gradient on its closed interval.
__device__ __forceinline__ TokenLoss grpo_token_loss(float eps_low, float eps_high, float beta,
                                                     float w, float adv, float lp, float lr,
                                                     bool has_ref) {
    TokenLoss r;
    const float lo_b = 1.0f - eps_low;
    const float hi_b = 1.0f + eps_high;
    const float c1 = expf(w);
    const float c2 = fminf(fmaxf(c1, lo_b), hi_b);
    const float a = c1 * adv;
    const float b = c2 * adv;
    // d a / d w = c1 * adv; d b / d w = c1 * adv inside [lo_b, hi_b], else 0.
    const float da = c1 * adv;
    const float db = (c1 >= lo_b && c1 <= hi_b) ? da : 0.0f;
    float dmin;
    if (a < b) dmin = da;
    else if (b < a) dmin = db;
    else dmin = 0.5f * da + 0.5f * db;
    r.loss = -fminf(a, b);
    r.dw = -dmin;
    r.kl = 0.0f;
    r.dlp = 0.0f;
    if (has_ref) {
        const float d = lr - lp;
        const float e = expf(d);
        r.kl = e - d - 1.0f;
        r.loss += beta * r.kl;
        r.dlp = beta * (1.0f - e);
    }
    r.low = (c1 < lo_b && adv < 0.0f) ? 1.0f : 0.0f;
    r.high = (c1 > hi_b && adv > 0.0f) ? 1.0f : 0.0f;
    return r;
}

}  // namespace klp
