/*
 * klp_oracle.c — CPU restatement of the reference's fused logprob/entropy
 * algorithm, in float64.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the HIP kernels are
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product (kernel_opt, the HIP library)
 * never calls it and has no CPU fallback.
 *
 * Every function follows a named part of the reference
 * (/root/reference/csrc/fused_logprob.cu):
 *   klp_oracle_bf16_to_f32 / f16_to_f32       to_float<T>       :37-51
 *   klp_oracle_round_bf16 / round_f16          from_float<T>     :53-67 (RNE)
 *   klp_oracle_forward                         v1 kernel         :156-227
 *       per-element combine() with the empty-sentinel rule    :135-154,183-188
 *       target captured where v == tgt, default 0           :180,185
 *       lse = m + log Z, logp = x_t - lse, H = log Z - T/Z    :221-224
 *   klp_oracle_forward_naive                   naive kernel      :79-112
 *       peeled first element, per-element recurrence
 *   klp_oracle_backward                        v1 backward       :233-282
 *       d = p (g_lse - g_logp - g_ent (log p + H)) + [v==t] g_logp
 *   `scale` (forward/backward): temperature 1/T fused into the load, see
 *       load_scaled(); scale = 1 is the reference computation.
 *
 * One deliberate difference, documented where it applies: in the backward a
 * -inf logit gets gradient 0 (its probability is exactly 0), where the
 * reference's 0 * inf yields NaN.
 *
 * How each function is pinned (tests/test_oracle.py): brute-force two-pass
 * float64 formulas, closed forms (uniform rows, two-element rows, a single
 * spike), invariants (shift, permutation, sum of gradients = g_lse), central
 * finite differences of the forward, the explicit softmax Jacobian, and
 * numpy/torch float16/bfloat16 conversions.  tests/test_oracle_mutants.py
 * rebuilds this file with planted mistakes (-DKLP_MUTANT=k) and checks that
 * every mutant fails at least one of those pins.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#ifndef KLP_MUTANT
#define KLP_MUTANT 0
#endif

enum { KLP_BF16 = 0, KLP_FP16 = 1, KLP_FP32 = 2 };

/* ------------------------------------------------------------------------ */
/* Conversions                                                               */
/* ------------------------------------------------------------------------ */

float klp_oracle_bf16_to_f32(uint16_t h) {
    uint32_t w = (uint32_t)h << 16;
    float f;
    memcpy(&f, &w, 4);
    return f;
}

float klp_oracle_f16_to_f32(uint16_t h) {
    const uint32_t sign = (h >> 15) & 1u;
    const uint32_t exp = (h >> 10) & 0x1Fu;
    const uint32_t man = h & 0x3FFu;
    double v;
    if (exp == 0x1F) {
        v = man ? NAN : INFINITY;
    } else if (exp == 0) {
        v = ldexp((double)man, -24); /* subnormal: man * 2^-24 */
    } else {
        v = ldexp((double)(man | 0x400u), (int)exp - 25);
    }
    return (float)(sign ? -v : v);
}

static double load_elem(const void* base, int dtype, int64_t idx) {
    switch (dtype) {
        case KLP_BF16: return klp_oracle_bf16_to_f32(((const uint16_t*)base)[idx]);
        case KLP_FP16: return klp_oracle_f16_to_f32(((const uint16_t*)base)[idx]);
        default: return ((const float*)base)[idx];
    }
}

/* Temperature: the kernels multiply each logit by scale = fp32(1/T) in fp32
 * as it is loaded (fusing the trainer's logits.div_(temperature),
 * reference python/kernel_opt/trainer.py:101).  The oracle applies the same
 * single fp32 rounding, then works in float64. */
static double load_scaled(const void* base, int dtype, int64_t idx, float scale) {
    const float x = (float)load_elem(base, dtype, idx);
#if KLP_MUTANT == 9 /* planted: temperature not applied */
    (void)scale;
    return x;
#else
    return (double)(x * scale);
#endif
}

/* Round a float64 to a binary format with `p` significant bits, minimum
 * normal exponent `emin` and largest finite value `maxf`, nearest-even,
 * keeping subnormals.  Returns the rounded value as a float64. */
static double round_format(double x, int p, int emin, double maxf) {
    if (isnan(x) || isinf(x) || x == 0.0) return x;
    int e;
    frexp(fabs(x), &e); /* |x| in [2^(e-1), 2^e) */
    e -= 1;
    if (e < emin) e = emin;
    const double ulp = ldexp(1.0, e - (p - 1));
#if KLP_MUTANT == 8 /* planted: truncation instead of nearest-even */
    const double r = trunc(x / ulp) * ulp;
#else
    const double r = rint(x / ulp) * ulp; /* rint: ties to even */
#endif
    if (fabs(r) > maxf) return x > 0 ? INFINITY : -INFINITY;
    return r;
}

uint16_t klp_oracle_round_bf16(double x) {
    if (isnan(x)) return 0x7FC0u;
    const double maxf = ldexp(255.0, 120); /* (2 - 2^-7) * 2^127 */
    const float r = (float)round_format(x, 8, -126, maxf);
    uint32_t w;
    memcpy(&w, &r, 4);
    return (uint16_t)(w >> 16);
}

uint16_t klp_oracle_round_f16(double x) {
    if (isnan(x)) return 0x7E00u;
    const double r = round_format(x, 11, -14, 65504.0);
    const uint16_t sign = (signbit(r) ? 0x8000u : 0u);
    const double a = fabs(r);
    if (isinf(a)) return sign | 0x7C00u;
    if (a < ldexp(1.0, -14)) return sign | (uint16_t)(a / ldexp(1.0, -24));
    int e;
    const double m = frexp(a, &e); /* a = m * 2^e, m in [0.5, 1) */
    const uint16_t exp_bits = (uint16_t)(e - 1 + 15);
    const uint16_t man = (uint16_t)((m * 2.0 - 1.0) * 1024.0);
    return sign | (uint16_t)(exp_bits << 10) | man;
}

/* Rounds `n` float64 values to `dtype` storage (bf16/f16 bits, or float). */
void klp_oracle_round(const double* x, int dtype, int64_t n, void* out) {
    for (int64_t i = 0; i < n; ++i) {
        switch (dtype) {
            case KLP_BF16: ((uint16_t*)out)[i] = klp_oracle_round_bf16(x[i]); break;
            case KLP_FP16: ((uint16_t*)out)[i] = klp_oracle_round_f16(x[i]); break;
            default: ((float*)out)[i] = (float)x[i]; break;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Row addressing                                                            */
/* ------------------------------------------------------------------------ */

static int64_t row_offset(int64_t r, int64_t rows_inner, int64_t stride_outer,
                          int64_t stride_inner) {
    const int64_t q = r / rows_inner;
    return q * stride_outer + (r - q * rows_inner) * stride_inner;
}

/* ------------------------------------------------------------------------ */
/* Forward                                                                   */
/* ------------------------------------------------------------------------ */

typedef struct {
    double m, Z, T;
} klp_state;

/* combine(), csrc/fused_logprob.cu:141-154, in float64. */
static klp_state combine(klp_state a, klp_state b) {
    if (b.m == -INFINITY) return a;
    if (a.m == -INFINITY) return b;
    const double m = fmax(a.m, b.m);
    const double d1 = a.m - m;
    const double d2 = b.m - m;
    const double s1 = exp(d1);
    const double s2 = exp(d2);
    klp_state r;
    r.m = m;
#if KLP_MUTANT == 1 /* planted: swapped scale factors */
    r.Z = s2 * a.Z + s1 * b.Z;
#else
    r.Z = s1 * a.Z + s2 * b.Z;
#endif
#if KLP_MUTANT == 2 /* planted: dropped d*Z correction term */
    r.T = s1 * a.T + s2 * (b.T + d2 * b.Z);
#else
    r.T = s1 * (a.T + d1 * a.Z) + s2 * (b.T + d2 * b.Z);
#endif
    return r;
}

/* Exported for the associativity tests: merges two states. */
void klp_oracle_combine(const double* a, const double* b, double* out) {
    klp_state sa = {a[0], a[1], a[2]};
    klp_state sb = {b[0], b[1], b[2]};
    klp_state r = combine(sa, sb);
    out[0] = r.m;
    out[1] = r.Z;
    out[2] = r.T;
}

/* State of one row segment [v0, v1), as the v1 kernel's per-thread loop. */
void klp_oracle_segment_state(const void* row, int dtype, int64_t v0, int64_t v1, double* out) {
    klp_state s = {-INFINITY, 0.0, 0.0};
    for (int64_t v = v0; v < v1; ++v) {
        klp_state e = {load_elem(row, dtype, v), 1.0, 0.0};
        s = combine(s, e);
    }
    out[0] = s.m;
    out[1] = s.Z;
    out[2] = s.T;
}

/* Outputs from a final state: csrc/fused_logprob.cu:221-224. */
void klp_oracle_finalize(const double* st, double x_target, double* logp, double* ent,
                         double* lse) {
    const double lz = log(st[1]);
    const double l = st[0] + lz;
#if KLP_MUTANT == 3 /* planted: wrong sign of the T/Z term */
    *ent = lz + st[2] / st[1];
#else
    *ent = lz - st[2] / st[1];
#endif
    *lse = l;
    *logp = x_target - l;
}

void klp_oracle_forward(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                        int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
                        const int64_t* targets, float scale, double* logp, double* ent,
                        double* lse) {
#pragma omp parallel for schedule(dynamic, 4)
    for (int64_t r = 0; r < n_rows; ++r) {
        const int64_t off = row_offset(r, rows_inner, stride_outer, stride_inner);
        const char* row = (const char*)logits + off * (dtype == KLP_FP32 ? 4 : 2);
        const int64_t tgt = targets[r];
        klp_state s = {-INFINITY, 0.0, 0.0};
        for (int64_t v = 0; v < vocab; ++v) {
            klp_state e = {load_scaled(row, dtype, v, scale), 1.0, 0.0};
            s = combine(s, e);
        }
        double st[3] = {s.m, s.Z, s.T};
        double x_target = 0.0;
#if KLP_MUTANT == 4 /* planted: target index off by one */
        if (tgt + 1 >= 0 && tgt + 1 < vocab) x_target = load_scaled(row, dtype, tgt + 1, scale);
#elif KLP_MUTANT == 10 /* planted: target logit not scaled */
        if (tgt >= 0 && tgt < vocab) x_target = load_elem(row, dtype, tgt);
#else
        if (tgt >= 0 && tgt < vocab) x_target = load_scaled(row, dtype, tgt, scale);
#endif
        klp_oracle_finalize(st, x_target, &logp[r], &ent[r], &lse[r]);
    }
}

/* Naive kernel, csrc/fused_logprob.cu:79-112: peeled first element, then the
 * scalar recurrence for every following element (no -inf guard, so a -inf
 * logit after the first makes T, and the entropy, NaN). */
void klp_oracle_forward_naive(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                              int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
                              const int64_t* targets, double* logp, double* ent, double* lse) {
#pragma omp parallel for schedule(dynamic, 4)
    for (int64_t r = 0; r < n_rows; ++r) {
        const int64_t off = row_offset(r, rows_inner, stride_outer, stride_inner);
        const char* row = (const char*)logits + off * (dtype == KLP_FP32 ? 4 : 2);
        const int64_t tgt = targets[r];
        const double x0 = load_elem(row, dtype, 0);
        double m = x0, Z = 1.0, T = 0.0;
        double x_target = (tgt == 0) ? x0 : 0.0;
        for (int64_t v = 1; v < vocab; ++v) {
            const double x = load_elem(row, dtype, v);
            if (v == tgt) x_target = x;
            const double m_new = fmax(m, x);
            const double delta = m - m_new;
            const double scale = exp(delta);
            const double v_new = x - m_new;
            const double e = exp(v_new);
            T = scale * (T + delta * Z) + v_new * e;
            Z = scale * Z + e;
            m = m_new;
        }
        const double lz = log(Z);
        lse[r] = m + lz;
        logp[r] = x_target - (m + lz);
        ent[r] = lz - T / Z;
    }
}

/* ------------------------------------------------------------------------ */
/* Backward                                                                  */
/* ------------------------------------------------------------------------ */

/* d_out is a dense [n_rows, vocab] float64 array.  g_* may be NULL (zero). */
void klp_oracle_backward(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                         int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
                         const int64_t* targets, float scale, const double* lse,
                         const double* ent, const double* g_logp, const double* g_ent,
                         const double* g_lse, double* d_out) {
#pragma omp parallel for schedule(dynamic, 4)
    for (int64_t r = 0; r < n_rows; ++r) {
        const int64_t off = row_offset(r, rows_inner, stride_outer, stride_inner);
        const char* row = (const char*)logits + off * (dtype == KLP_FP32 ? 4 : 2);
        const int64_t tgt = targets[r];
        const double gl = g_logp ? g_logp[r] : 0.0;
        const double ge = g_ent ? g_ent[r] : 0.0;
        const double gs = g_lse ? g_lse[r] : 0.0;
        /* const_part, csrc/fused_logprob.cu:271 */
#if KLP_MUTANT == 5 /* planted: wrong sign of the g_logp term */
        const double c0 = gs + gl - ge * ent[r];
#else
        const double c0 = gs - gl - ge * ent[r];
#endif
        double* d = d_out + r * vocab;
        for (int64_t v = 0; v < vocab; ++v) {
            const double x = load_scaled(row, dtype, v, scale);
            double val;
            if (x == -INFINITY) {
                val = 0.0; /* p = 0 exactly; the reference writes NaN (0 * inf) */
            } else {
                const double lp = x - lse[r];
                const double p = exp(lp);
#if KLP_MUTANT == 6 /* planted: dropped the g_ent * log p term */
                val = p * c0;
#else
                val = p * (c0 - ge * lp);
#endif
            }
#if KLP_MUTANT == 7 /* planted: wrong sign of the one-hot term */
            if (v == tgt) val -= gl;
#else
            if (v == tgt) val += gl;
#endif
#if KLP_MUTANT == 11 /* planted: chain-rule factor 1/T dropped */
            d[v] = val;
#else
            d[v] = val * (double)scale; /* d/dx = (1/T) d/dx' */
#endif
        }
    }
}
