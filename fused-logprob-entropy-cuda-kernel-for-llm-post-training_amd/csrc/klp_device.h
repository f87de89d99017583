// klp_device.h — device-side building blocks for the gfx950 kernels:
// dtype traits, 128-bit vector unpack/pack, row addressing, the online
// (max, sum-exp, sum-shifted-x*exp) state and its associative combine, and
// the wave64 reduction.
//
// Arithmetic is done in base 2 so that each element costs one v_exp_f32:
//   y = x * log2(e),   o = RN(m * log2(e))   (m = running max of x),
//   z = sum 2^(y - o),
//   t = sum (y - o) * 2^(y - o)          (<= 0).
// The reference carries the same three quantities in base e
// (csrc/fused_logprob.cu:13-27, PartialState :135-139); the final formulas
// below convert back to nats.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace klp {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kLn2 = 0.69314718055994530942f;
// Finite stand-in for -inf exponents: 2^kNegBig == 0 and kNegBig * 0 == 0,
// where -inf * 0 would be NaN.
constexpr float kNegBig = -1.0e30f;

enum : int { kBF16 = 0, kFP16 = 1, kFP32 = 2 };

template <int DT> struct Traits;
template <> struct Traits<kBF16> {
    typedef uint16_t elem;
    static constexpr int kPerVec = 8;
    static constexpr uint32_t kNegInfWord = 0xFF80FF80u;
};
template <> struct Traits<kFP16> {
    typedef uint16_t elem;
    static constexpr int kPerVec = 8;
    static constexpr uint32_t kNegInfWord = 0xFC00FC00u;
};
template <> struct Traits<kFP32> {
    typedef uint32_t elem;
    static constexpr int kPerVec = 4;
    static constexpr uint32_t kNegInfWord = 0xFF800000u;
};

// ---------------------------------------------------------------------------
// Conversions.  Up-conversion is exact.  Down-conversion rounds to nearest
// even and keeps fp16 subnormals (v_cvt_pk_bf16_f32 / v_cvt_f16_f32 under the
// default MODE register), matching __float2bfloat16 / __float2half in the
// reference (csrc/fused_logprob.cu:53-67).
// ---------------------------------------------------------------------------
template <int DT> __device__ __forceinline__ float to_f32(typename Traits<DT>::elem e);
template <> __device__ __forceinline__ float to_f32<kBF16>(uint16_t e) {
    return __uint_as_float(static_cast<uint32_t>(e) << 16);
}
template <> __device__ __forceinline__ float to_f32<kFP16>(uint16_t e) {
    return static_cast<float>(__builtin_bit_cast(_Float16, e));
}
template <> __device__ __forceinline__ float to_f32<kFP32>(uint32_t e) {
    return __uint_as_float(e);
}

template <int DT> __device__ __forceinline__ typename Traits<DT>::elem from_f32(float x);
template <> __device__ __forceinline__ uint16_t from_f32<kBF16>(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(x));
}
template <> __device__ __forceinline__ uint16_t from_f32<kFP16>(float x) {
    // The empty asm hides x's origin from instruction selection: a product
    // rounded straight to fp16 would otherwise become v_fma_mixlo_f16 a, b, +0,
    // which turns a -0 product into +0.
    asm("" : "+v"(x));
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}
template <> __device__ __forceinline__ uint32_t from_f32<kFP32>(float x) {
    return __float_as_uint(x);
}

// 16 bytes -> Traits<DT>::kPerVec floats, element order = memory order.
template <int DT> __device__ __forceinline__ void unpack(const u32x4 v, float* x);
template <> __device__ __forceinline__ void unpack<kBF16>(const u32x4 v, float* x) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        x[2 * j] = __uint_as_float(v[j] << 16);
        x[2 * j + 1] = __uint_as_float(v[j] & 0xFFFF0000u);
    }
}
template <> __device__ __forceinline__ void unpack<kFP16>(const u32x4 v, float* x) {
    // Whole-vector bit_cast: hipcc 7.2 miscompiles __builtin_bit_cast applied
    // to an element expression v[j] (it reads element 0 for every j).
    const f32x8 f = __builtin_convertvector(__builtin_bit_cast(f16x8, v), f32x8);
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = f[j];
}
template <> __device__ __forceinline__ void unpack<kFP32>(const u32x4 v, float* x) {
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = __uint_as_float(v[j]);
}

// kPerVec floats -> 16 bytes, round to nearest even.
template <int DT> __device__ __forceinline__ u32x4 pack(const float* x);
template <> __device__ __forceinline__ u32x4 pack<kBF16>(const float* x) {
    f32x8 f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = x[j];
    return __builtin_bit_cast(u32x4, __builtin_convertvector(f, bf16x8));
}
template <> __device__ __forceinline__ u32x4 pack<kFP16>(const float* x) {
    f32x8 f;
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = x[j];
    return __builtin_bit_cast(u32x4, __builtin_convertvector(f, f16x8));
}
template <> __device__ __forceinline__ u32x4 pack<kFP32>(const float* x) {
    u32x4 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = __float_as_uint(x[j]);
    return r;
}

template <bool kNonTemporal>
__device__ __forceinline__ u32x4 load16(const u32x4* p) {
    if constexpr (kNonTemporal) return __builtin_nontemporal_load(p);
    else return *p;
}

// Cache-policy operand of the raw buffer load builtins for a non-temporal
// load (the "nt" bit on gfx950, which __builtin_nontemporal_load also sets).
constexpr int kBufNonTemporal = 2;

// s_waitcnt immediate (gfx9 encoding) that waits for vmcnt 0 only: vmcnt
// bits [3:0] and [15:14] zero, expcnt [6:4] and lgkmcnt [11:8] at their
// maxima (no wait).
constexpr int kWaitVmcnt0 = 0x0F70;

__device__ __forceinline__ float fmax_nan(float a, float b) {
    // NaN-propagating maximum (v_maximum3_f32 on gfx950): a NaN logit turns
    // the running max, and with it every output of its row, into NaN.
    return __builtin_elementwise_maximum(a, b);
}

__device__ __forceinline__ float exp2_hw(float u) { return __builtin_amdgcn_exp2f(u); }

// ---------------------------------------------------------------------------
// Row addressing: row r starts at (r / rows_inner) * stride_outer +
// (r % rows_inner) * stride_inner elements.
// ---------------------------------------------------------------------------
struct RowMap {
    int64_t rows_inner;
    int64_t stride_outer;
    int64_t stride_inner;
};

__device__ __forceinline__ int64_t row_offset(const RowMap& rm, int64_t r) {
    if (r < rm.rows_inner) return r * rm.stride_inner;
    const int64_t q = r / rm.rows_inner;
    return q * rm.stride_outer + (r - q * rm.rows_inner) * rm.stride_inner;
}

// ---------------------------------------------------------------------------
// Online state.  Empty state: (m = -inf, z = 0, t = 0), the reference's
// sentinel (csrc/fused_logprob.cu:127-129).
// ---------------------------------------------------------------------------
struct Stat {
    float m;
    float z;
    float t;
};

__device__ __forceinline__ Stat stat_empty() { return Stat{-INFINITY, 0.0f, 0.0f}; }

// Associative merge; restates combine() of csrc/fused_logprob.cu:141-154
// (including its empty-side early returns) in base-2 units.
__device__ __forceinline__ Stat combine(const Stat a, const Stat b) {
    if (b.m == -INFINITY) return a;
    if (a.m == -INFINITY) return b;
    const float m = fmax_nan(a.m, b.m);
    const float o = m * kLog2e;
    const float da = a.m * kLog2e - o;  // <= 0
    const float db = b.m * kLog2e - o;  // <= 0
    const float sa = exp2_hw(da);
    const float sb = exp2_hw(db);
    Stat r;
    r.m = m;
    r.z = sa * a.z + sb * b.z;
    r.t = sa * fmaf(da, a.z, a.t) + sb * fmaf(db, b.z, b.t);
    return r;
}

// Absorb K values into the state: one rescale of (z, t) to the new maximum,
// then one exp2 per value.  With kClamp == false a -inf value makes t NaN
// (-inf * 0) while z stays finite; the caller detects that and redoes the
// values with kClamp == true, which maps -inf exponents to kNegBig.
template <int K, bool kClamp>
__device__ __forceinline__ void absorb(Stat& s, const float* x) {
    float c = s.m;
#pragma unroll
    for (int j = 0; j < K; ++j) c = fmax_nan(c, x[j]);
    const float o_raw = c * kLog2e;
    const float o = (c == -INFINITY) ? 0.0f : o_raw;
    const float d = (s.m == -INFINITY) ? kNegBig : fmax_nan(s.m * kLog2e - o_raw, kNegBig);
    const float sc = exp2_hw(d);
    float z0 = sc * s.z;
    float t0 = sc * fmaf(d, s.z, s.t);
    float z1 = 0.0f, t1 = 0.0f;
#pragma unroll
    for (int j = 0; j < K; ++j) {
        float u = fmaf(x[j], kLog2e, -o);
        if (kClamp) u = fmax_nan(u, kNegBig);
        const float e = exp2_hw(u);
        if (j & 1) {
            z1 += e;
            t1 = fmaf(u, e, t1);
        } else {
            z0 += e;
            t0 = fmaf(u, e, t0);
        }
    }
    s.m = c;
    s.z = z0 + z1;
    s.t = t0 + t1;
}

// True when the unclamped scan met a -inf value (t is NaN, z is not).
__device__ __forceinline__ bool needs_clamped_rescan(const Stat& s) {
    return __builtin_isnan(s.t) && !__builtin_isnan(s.z);
}

// The state of the partner lane under DPP control `Ctrl` (a lane move
// within a row of 16 lanes, a few cycles; no LDS round trip).
template <int Ctrl>
__device__ __forceinline__ Stat stat_dpp(const Stat& s) {
    Stat o;
    o.m = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s.m), Ctrl, 0xF, 0xF,
                                                     false));
    o.z = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s.z), Ctrl, 0xF, 0xF,
                                                     false));
    o.t = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(s.t), Ctrl, 0xF, 0xF,
                                                     false));
    return o;
}

__device__ __forceinline__ Stat stat_shfl_xor(const Stat& s, int off) {
    return Stat{__shfl_xor(s.m, off, 64), __shfl_xor(s.z, off, 64), __shfl_xor(s.t, off, 64)};
}

// Merge the states of the 16 lanes of each DPP row; every lane of the row
// returns the row's total.  combine() is commutative bit for bit, so both
// lanes of a pair compute the same merge and the result depends on nothing
// but the fixed pairing order: lanes are paired by DPP quad_perm [1,0,3,2],
// quad_perm [2,3,0,1], row_half_mirror and row_mirror (the partner always
// holds the other half of the group merged so far).
__device__ __forceinline__ Stat row_reduce(Stat s) {
    s = combine(s, stat_dpp<0xB1>(s));   // quad_perm [1, 0, 3, 2]
    s = combine(s, stat_dpp<0x4E>(s));   // quad_perm [2, 3, 0, 1]
    s = combine(s, stat_dpp<0x141>(s));  // row_half_mirror
    s = combine(s, stat_dpp<0x140>(s));  // row_mirror
    return s;
}

// Merge the states of all 64 lanes; every lane returns the total: the four
// rows by row_reduce, then across rows by xor-16 and xor-32 shuffles.
__device__ __forceinline__ Stat wave_reduce(Stat s) {
    s = row_reduce(s);
    s = combine(s, stat_shfl_xor(s, 16));
    s = combine(s, stat_shfl_xor(s, 32));
    return s;
}

// ---------------------------------------------------------------------------
// Flat reduction: the states of many lanes merged as one maximum, one rescale
// per lane to it and two sums, instead of a tree of pairwise combine() calls
// (each with two v_exp_f32 on the critical path).  Same value as the tree up
// to fp32 rounding; deterministic (fixed lane pairing).  At the end of a
// C2-sized forward (one 304 KB row per workgroup) the row's reduction is on
// the critical path: this form measured 0.5-1.0 us faster per launch than
// wave_reduce() with ds_bpermute shuffles.
// ---------------------------------------------------------------------------
template <int Ctrl>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), Ctrl, 0xF, 0xF, false));
}

// Maximum / sum over each row of 16 lanes; every lane of the row gets it.
__device__ __forceinline__ float row_max16(float v) {
    v = fmax_nan(v, dpp_f32<0xB1>(v));   // quad_perm [1, 0, 3, 2]
    v = fmax_nan(v, dpp_f32<0x4E>(v));   // quad_perm [2, 3, 0, 1]
    v = fmax_nan(v, dpp_f32<0x141>(v));  // row_half_mirror
    return fmax_nan(v, dpp_f32<0x140>(v));  // row_mirror
}
__device__ __forceinline__ float row_sum16(float v) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    return v + dpp_f32<0x140>(v);
}

// Across the four rows of a wave with v_permlane16_swap / v_permlane32_swap
// (called with both operands equal, the pair holds the two halves being
// paired: rows (0,1),(2,3), then lanes (l, l+32)); every lane gets the total.
__device__ __forceinline__ float xrow_max(float v) {
    const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    v = fmax_nan(__uint_as_float(q[0]), __uint_as_float(q[1]));
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return fmax_nan(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xrow_sum(float v) {
    const auto q = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    v = __uint_as_float(q[0]) + __uint_as_float(q[1]);
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// (z, t) of state s rescaled to the offset RN(m * log2e), m >= s.m (or m
// NaN); an empty state contributes zeros.
__device__ __forceinline__ void rescale_to(const Stat& s, float m, float& z, float& t) {
    const bool live = s.m != -INFINITY;
    const float d = live ? s.m * kLog2e - m * kLog2e : 0.0f;
    const float sc = live ? exp2_hw(d) : 0.0f;
    z = live ? sc * s.z : 0.0f;
    t = live ? sc * fmaf(d, s.z, s.t) : 0.0f;
}

// All 64 lanes; every lane returns the total.
__device__ __forceinline__ Stat wave_reduce_flat(const Stat s) {
    const float m = xrow_max(row_max16(s.m));
    float z, t;
    rescale_to(s, m, z, t);
    return Stat{m, xrow_sum(row_sum16(z)), xrow_sum(row_sum16(t))};
}

// The 16 lanes of each DPP row; every lane of the row returns its total.
__device__ __forceinline__ Stat row_reduce_flat(const Stat s) {
    const float m = row_max16(s.m);
    float z, t;
    rescale_to(s, m, z, t);
    return Stat{m, row_sum16(z), row_sum16(t)};
}

// Final per-row outputs (csrc/fused_logprob.cu:221-224 in base e):
//   lse     = m + ln z + (o - m*log2e) * ln2
//   entropy = ln z - ln2 * t / z
//   logprob = x_target - lse
// The middle term of lse undoes the rounding of o = RN(m*log2e); it is the
// exact product remainder, obtained with one fma.
struct RowOut {
    float logp;
    float ent;
    float lse;
};

__device__ __forceinline__ RowOut finalize(const Stat s, float x_target) {
    const float lnz = logf(s.z);
    float rho = 0.0f;
    if (s.m != -INFINITY) {
        const float o = s.m * kLog2e;
        rho = -fmaf(s.m, kLog2e, -o);
    }
    RowOut r;
    r.lse = s.m + fmaf(rho, kLn2, lnz);
    r.ent = fmaf(-kLn2, s.t / s.z, lnz);
    r.logp = x_target - r.lse;
    return r;
}

// Per-row constants of the backward (reference csrc/fused_logprob.cu:233-238,
// the hoisted constant at :271): c0 = g_lse - g_logp - g_ent * H, and lse
// times log2(e) split into a rounded head and its exact fma remainder.
struct RowGrad {
    float lse, lse_hi, lse_lo, g_ent, g_logp, c0;
};

__device__ __forceinline__ RowGrad row_grad(float lse, float ent, float g_logp, float g_ent,
                                            float g_lse) {
    RowGrad g;
    g.lse = lse;
    g.g_logp = g_logp;
    g.g_ent = g_ent;
    g.c0 = g_lse - g_logp - g_ent * ent;
    g.lse_hi = lse * kLog2e;
    g.lse_lo = fmaf(lse, kLog2e, -g.lse_hi);
    return g;
}

// Gradient with respect to the (temperature-scaled) logit x, without the
// one-hot term; the chain-rule factor 1/T for the unscaled logit is applied
// by the caller.  p = 2^(x*log2e - lse*log2e) with one rounding in the
// exponent; lp is clamped so that a -inf logit gives exactly 0.
__device__ __forceinline__ float grad_one(float x, const RowGrad& g) {
    const float lp = fmax_nan(x - g.lse, kNegBig);
    const float arg = fmaf(x, kLog2e, -g.lse_hi) - g.lse_lo;
    const float p = exp2_hw(arg);
    return p * fmaf(-g.g_ent, lp, g.c0);
}

// grad_one for a row with g_ent == 0: p * c0.  Equal in value to grad_one
// (fmaf(-0, lp, c0) == c0 for the clamped, finite lp; only the sign of a
// zero result can differ), in three fewer operations.
__device__ __forceinline__ float grad_one_logp_only(float x, const RowGrad& g) {
    const float arg = fmaf(x, kLog2e, -g.lse_hi) - g.lse_lo;
    return exp2_hw(arg) * g.c0;
}

// fp32 gradients.  An fp32 output resolves the exponent's rounding: the
// argument above (|arg| ~ 20 for typical rows, two roundings of ulp(20) / 2
// ~ 1e-6) moves p by several ulps.  Here the argument is carried exactly to
// well below one ulp of p:
//   x - lse          as dh + dl: dh = RN(x - lse) and dl its exact error by
//                    Fast2Sum, the larger operand first.  lse >= x for every
//                    logit of the row, so a row with lse >= 0 takes (-lse, x)
//                    (exact for every x >= -lse, i.e. all logits but those
//                    below -lse, whose p < e^(-2 lse) keeps the error of one
//                    rounding), and a row with lse < 0 takes (x, -lse), exact
//                    for every logit.  The order is a row-level choice
//                    (kLseNonNeg), not a per-element one;
//   (dh + dl) log2e  as ah = RN(dh log2e) and, in nats, the remainder
//                    c = (dh log2e - ah) ln2 + dl + dh (log2e's fp32 tail) ln2
//                    (log2e ln2 = 1 to within that tail);
//   p = 2^ah (1 + c),
// so p carries v_exp_f32's error and the saved lse's rounding only, and
// lp = dh + dl enters the entropy term with its remainder too.  -inf logits
// are clamped to kNegBig first (p = 0 exactly, every term finite).  Six more
// operations per element than grad_one.
constexpr float kLog2eTailLn2 = 1.3349758e-08f;  // (log2(e) - fp32(log2(e))) * ln 2

template <bool kLseNonNeg>
__device__ __forceinline__ float p_exact_arg(float x, float lse, float& dh, float& dl) {
    const float xc = fmax_nan(x, kNegBig);
    dh = xc - lse;
    if constexpr (kLseNonNeg) dl = xc - (dh + lse);
    else dl = -lse - (dh - xc);
    const float ah = dh * kLog2e;
    float c = fmaf(dh, kLog2e, -ah);
    c = fmaf(c, kLn2, dl);
    c = fmaf(dh, kLog2eTailLn2, c);
    const float e = exp2_hw(ah);
    return fmaf(e, c, e);
}

template <bool kLseNonNeg>
__device__ __forceinline__ float grad_one_fp32(float x, const RowGrad& g) {
    float dh, dl;
    const float p = p_exact_arg<kLseNonNeg>(x, g.lse, dh, dl);
    return p * fmaf(-g.g_ent, dl, fmaf(-g.g_ent, dh, g.c0));
}

template <bool kLseNonNeg>
__device__ __forceinline__ float grad_one_fp32_logp_only(float x, const RowGrad& g) {
    float dh, dl;
    return p_exact_arg<kLseNonNeg>(x, g.lse, dh, dl) * g.c0;
}

// The gradient of one logit of dtype DT: fp32 rows take the exact-argument
// form above, with the row's operand order kLseNonNeg (= lse >= 0); bf16 /
// fp16 rows, whose outputs do not resolve it, take grad_one.
template <int DT, bool kLseNonNeg>
__device__ __forceinline__ float grad_elem(float x, const RowGrad& g) {
    if constexpr (DT == kFP32) return grad_one_fp32<kLseNonNeg>(x, g);
    else return grad_one(x, g);
}
template <int DT, bool kLseNonNeg>
__device__ __forceinline__ float grad_elem_logp_only(float x, const RowGrad& g) {
    if constexpr (DT == kFP32) return grad_one_fp32_logp_only<kLseNonNeg>(x, g);
    else return grad_one_logp_only(x, g);
}

}  // namespace klp
