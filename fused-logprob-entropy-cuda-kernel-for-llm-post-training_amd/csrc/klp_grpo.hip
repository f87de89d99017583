// klp_grpo.hip — the GRPO policy loss over per-token log-probabilities
// ("K2 fused_grpo_loss" in the reference's plan, notes/PLAN.md:59; the loss
// itself is written out in examples/compare_one_step.py:232-236, and is the
// loss TRL's GRPOTrainer applies to the output of the fused logprob kernel).
//
// Per token (b, s) with mask m, advantage A, new / old / reference
// log-probabilities lp, lo, lr:
//   w     = lp - lo                      (token level), or the row's masked
//           mean of lp - lo              (sequence level),
//   c1    = exp(w),  c2 = clamp(c1, 1 - eps_low, 1 + eps_high),
//   loss  = -min(c1 * A, c2 * A) + beta * (exp(lr - lp) - (lr - lp) - 1).
// The batch loss is the masked sum of the per-token losses divided by
//   "grpo":  B * max(sum_s m, 1) per row (mean over rows of row means),
//   "bnpo":  max(sum m, 1) over the batch,
//   "fixed": a caller-given constant (TRL's dr_grpo and dapo normalisers).
// The gradient with respect to lp follows PyTorch's rules for the eager
// expression: at a tie of min() each side gets half, clamp() passes the
// gradient on its closed interval.
//
// Launches: klp_grpo_rows_kernel (one workgroup per row: row sums into the
// workspace), klp_grpo_finish_kernel (one workgroup: the batch sums in a
// fixed order, the loss and statistics), klp_grpo_bwd_kernel (one workgroup
// per row: the gradient, scaled by the upstream gradient of the loss).  All
// reductions have a fixed order, so results do not depend on timing.
#include <type_traits>

#include "klp_grpo_terms.h"
#include "klp_launch.h"

namespace klp {

namespace {

constexpr int kGrpoThreads = 256;

__device__ __forceinline__ float mask_at(const GrpoParams& p, int64_t i) {
    return p.mask ? p.mask[i] : 1.0f;
}

__device__ __forceinline__ float adv_at(const GrpoParams& p, int64_t b, int64_t i) {
    return p.adv_per_token ? p.adv[i] : p.adv[b];
}

__device__ __forceinline__ TokenLoss token_loss(const GrpoParams& p, float w, float adv,
                                                float lp, float lr, bool has_ref) {
    return grpo_token_loss(p.eps_low, p.eps_high, p.beta, w, adv, lp, lr, has_ref);
}

// Block-wide sums of K values, fixed order (xor-shuffle tree within waves,
// waves in order through LDS).  Every thread returns the totals.
template <int K>
__device__ __forceinline__ void block_sum(float (&v)[K]) {
    __shared__ float red[kGrpoThreads / 64][K];
    __shared__ float tot[K];
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) v[k] += __shfl_xor(v[k], off, 64);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    if (lane == 0)
#pragma unroll
        for (int k = 0; k < K; ++k) red[wave][k] = v[k];
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int k = 0; k < K; ++k) {
            float s = red[0][k];
            for (int w = 1; w < kGrpoThreads / 64; ++w) s += red[w][k];
            tot[k] = s;
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < K; ++k) v[k] = tot[k];
    __syncthreads();
}

// The row's log importance weight at sequence level: masked mean of lp - lo.
__device__ __forceinline__ void row_sequence_weight(const GrpoParams& p, int64_t b, float* w_row,
                                                    float* m_row) {
    const int64_t base = b * p.S;
    float v[2] = {0.0f, 0.0f};
    for (int64_t s = threadIdx.x; s < p.S; s += kGrpoThreads) {
        const float m = mask_at(p, base + s);
        v[0] += (p.logp[base + s] - p.old_logp[base + s]) * m;
        v[1] += m;
    }
    block_sum<2>(v);
    *m_row = v[1];
    *w_row = v[0] / fmaxf(v[1], 1.0f);
}

}  // namespace

// Workspace words per row, and at the end of the row block the batch sums
// written by klp_grpo_finish_kernel.
//   row b:  [0] sum loss*m  [1] sum m  [2] sum kl*m  [3] sum low*m
//           [4] sum high*m
//   tail :  [0] sum m over the batch
__global__ __launch_bounds__(kGrpoThreads) void klp_grpo_rows_kernel(GrpoParams p) {
    const int64_t b = blockIdx.x;
    const int64_t base = b * p.S;
    const bool has_ref = p.ref_logp != nullptr && p.beta != 0.0f;
    float w_row = 0.0f, m_row = 0.0f;
    if (p.level == KLP_GRPO_SEQUENCE) row_sequence_weight(p, b, &w_row, &m_row);
    float v[5] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t s = threadIdx.x; s < p.S; s += kGrpoThreads) {
        const int64_t i = base + s;
        const float m = mask_at(p, i);
        const float lp = p.logp[i];
        const float w = (p.level == KLP_GRPO_SEQUENCE) ? w_row : lp - p.old_logp[i];
        const TokenLoss t = token_loss(p, w, adv_at(p, b, i), lp,
                                       has_ref ? p.ref_logp[i] : 0.0f, has_ref);
        v[0] += t.loss * m;
        v[1] += m;
        v[2] += t.kl * m;
        v[3] += t.low * m;
        v[4] += t.high * m;
    }
    block_sum<5>(v);
    if (threadIdx.x == 0) {
        float* row = p.ws + b * kGrpoRowWords;
#pragma unroll
        for (int k = 0; k < 5; ++k) row[k] = v[k];
    }
}

// Batch sums in a fixed order: thread j adds rows j, j + 256, ... in order,
// then the block tree.  loss, then stats = {mean kl, low-clip fraction,
// high-clip fraction, clipped fraction}, each a masked mean over all tokens.
__global__ __launch_bounds__(kGrpoThreads) void klp_grpo_finish_kernel(GrpoParams p) {
    float v[6] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    for (int64_t b = threadIdx.x; b < p.B; b += kGrpoThreads) {
        const float* row = p.ws + b * kGrpoRowWords;
        // "grpo": mean over rows of the row's masked mean.
        v[0] += row[0] / fmaxf(row[1], 1.0f);
        v[1] += row[0];
        v[2] += row[1];
        v[3] += row[2];
        v[4] += row[3];
        v[5] += row[4];
    }
    block_sum<6>(v);
    if (threadIdx.x != 0) return;
    float loss;
    if (p.loss_type == KLP_GRPO_LOSS_GRPO) loss = v[0] / static_cast<float>(p.B);
    else if (p.loss_type == KLP_GRPO_LOSS_BNPO) loss = v[1] / fmaxf(v[2], 1.0f);
    else loss = v[1] / p.norm_const;
    const float den = fmaxf(v[2], 1.0f);
    p.loss[0] = loss;
    if (p.stats) {
        p.stats[0] = v[3] / den;
        p.stats[1] = v[4] / den;
        p.stats[2] = v[5] / den;
        p.stats[3] = (v[4] + v[5]) / den;
    }
    p.ws[p.B * kGrpoRowWords] = v[2];
}

// d loss / d lp for every token, times the upstream gradient of the loss
// (a device scalar, or 1 when null).  Reads the row sums of the forward.
__global__ __launch_bounds__(kGrpoThreads) void klp_grpo_bwd_kernel(GrpoParams p) {
    const int64_t b = blockIdx.x;
    const int64_t base = b * p.S;
    const bool has_ref = p.ref_logp != nullptr && p.beta != 0.0f;
    const float g = p.grad_loss ? p.grad_loss[0] : 1.0f;
    // Weight of a token's loss in the batch loss, per unit mask.
    float scale;
    if (p.loss_type == KLP_GRPO_LOSS_GRPO)
        scale = 1.0f / (static_cast<float>(p.B) * fmaxf(p.ws[b * kGrpoRowWords + 1], 1.0f));
    else if (p.loss_type == KLP_GRPO_LOSS_BNPO)
        scale = 1.0f / fmaxf(p.ws[p.B * kGrpoRowWords], 1.0f);
    else
        scale = 1.0f / p.norm_const;
    scale *= g;

    if (p.level == KLP_GRPO_SEQUENCE) {
        // Every token shares w = sum_s (lp - lo) m / max(sum m, 1): the
        // ratio term's gradient is (sum_s' scale m_s' dw_s') * m_s / max(sum m, 1).
        float w_row, m_row;
        row_sequence_weight(p, b, &w_row, &m_row);
        float v[1] = {0.0f};
        for (int64_t s = threadIdx.x; s < p.S; s += kGrpoThreads) {
            const int64_t i = base + s;
            const float m = mask_at(p, i);
            const TokenLoss t = token_loss(p, w_row, adv_at(p, b, i), p.logp[i],
                                           has_ref ? p.ref_logp[i] : 0.0f, has_ref);
            v[0] += t.dw * m;
        }
        block_sum<1>(v);
        const float row_term = v[0] * scale / fmaxf(m_row, 1.0f);
        for (int64_t s = threadIdx.x; s < p.S; s += kGrpoThreads) {
            const int64_t i = base + s;
            const float m = mask_at(p, i);
            const TokenLoss t = token_loss(p, w_row, adv_at(p, b, i), p.logp[i],
                                           has_ref ? p.ref_logp[i] : 0.0f, has_ref);
            p.d_logp[i] = row_term * m + t.dlp * m * scale;
        }
        return;
    }
    for (int64_t s = threadIdx.x; s < p.S; s += kGrpoThreads) {
        const int64_t i = base + s;
        const float m = mask_at(p, i);
        const float lp = p.logp[i];
        const TokenLoss t = token_loss(p, lp - p.old_logp[i], adv_at(p, b, i), lp,
                                       has_ref ? p.ref_logp[i] : 0.0f, has_ref);
        p.d_logp[i] = (t.dw + t.dlp) * m * scale;
    }
}

namespace {

constexpr int kWeightThreads = 256;
constexpr int kWeightWaves = kWeightThreads / 64;
// Elements a thread handles per step of the grid-wide loops (their loads are
// issued together).
constexpr int kWeightUnroll = 4;

// Mask element i as an integer: M is the mask's element type, void for no
// mask (all ones).
template <typename M>
__device__ __forceinline__ int64_t mask_value(const void* mask, int64_t i) {
    if constexpr (std::is_void_v<M>) {
        return 1;
    } else {
        return static_cast<int64_t>(static_cast<const M*>(mask)[i]);
    }
}

// The mask from element `offset` on (no mask stays none).
template <typename M>
__device__ __forceinline__ const void* mask_from(const void* mask, int64_t offset) {
    if constexpr (std::is_void_v<M>) {
        return nullptr;
    } else {
        return static_cast<const M*>(mask) + offset;
    }
}

// 64-bit integer sum over a wave (xor tree on the two 32-bit halves).
__device__ __forceinline__ int64_t wave_sum_i64(int64_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const int lo = __shfl_xor(static_cast<int>(static_cast<uint64_t>(v)), off, 64);
        const int hi = __shfl_xor(static_cast<int>(static_cast<uint64_t>(v) >> 32), off, 64);
        v += static_cast<int64_t>((static_cast<uint64_t>(static_cast<uint32_t>(hi)) << 32) |
                                  static_cast<uint32_t>(lo));
    }
    return v;
}

// Sum over the workgroup, returned to every thread.  `part` is reused by the
// caller's next call only after that call's first barrier, which every
// thread reaches after reading this call's result.
__device__ __forceinline__ int64_t block_sum_i64(int64_t v, int64_t* part) {
    const uint32_t tid = threadIdx.x;
    v = wave_sum_i64(v);
    __syncthreads();  // the previous call's readers are done with `part`
    if ((tid & 63u) == 0) part[tid >> 6] = v;
    __syncthreads();
    int64_t tot = 0;
#pragma unroll
    for (int w = 0; w < kWeightWaves; ++w) tot += part[w];
    return tot;
}

// Sum of mask[i] over the indices i = first + k * stride < n.
template <typename M>
__device__ __forceinline__ int64_t strided_mask_sum(const void* mask, int64_t first, int64_t stride,
                                                    int64_t n) {
    int64_t v = 0;
    int64_t i = first;
    for (; i + (kWeightUnroll - 1) * stride < n; i += kWeightUnroll * stride) {
        int64_t m[kWeightUnroll];
#pragma unroll
        for (int k = 0; k < kWeightUnroll; ++k) m[k] = mask_value<M>(mask, i + k * stride);
#pragma unroll
        for (int k = 0; k < kWeightUnroll; ++k) v += m[k];
    }
    for (; i < n; i += stride) v += mask_value<M>(mask, i);
    return v;
}

// weights[i] = mask[i] * r over the indices i = first + k * stride < n.
template <typename M>
__device__ __forceinline__ void strided_weights(const void* mask, float* weights, float r,
                                                int64_t first, int64_t stride, int64_t n) {
    int64_t i = first;
    for (; i + (kWeightUnroll - 1) * stride < n; i += kWeightUnroll * stride) {
        int64_t m[kWeightUnroll];
#pragma unroll
        for (int k = 0; k < kWeightUnroll; ++k) m[k] = mask_value<M>(mask, i + k * stride);
#pragma unroll
        for (int k = 0; k < kWeightUnroll; ++k)
            weights[i + k * stride] = static_cast<float>(m[k]) * r;
    }
    for (; i < n; i += stride) weights[i] = static_cast<float>(mask_value<M>(mask, i)) * r;
}

}  // namespace

// The GRPO step's token weights w = m / normaliser:
//   "grpo":  m * (1 / (max(row sum of m, 1) * B)), one workgroup per row
//            (klp_grpo_weights_rows_kernel);
//   "bnpo":  m * (1 / max(sum of m, 1)): per-workgroup partial sums into the
//            caller's workspace (klp_grpo_weights_partial_kernel), then every
//            workgroup adds the partials and writes its share
//            (klp_grpo_weights_kernel<.., kFromPartials>); a grid of one
//            workgroup sums and writes in one launch (kOwnSum);
//   fixed:   m * scale (klp_grpo_weights_kernel<.., kScaleGiven>).
// The mask's sums are taken exactly in 64-bit integers (so every workgroup of
// the "bnpo" pass gets the same total, in any order) and rounded once to
// float32; then the same float32 operations as the eager statement
// (grpo_step.grpo_token_weights) follow: the weights are its bits whenever
// those sums are below 2^24, as the sums of any 0 / 1 mask of fewer than
// 2^24 tokens are (the eager float32 sums of integers are exact there, in
// any order).  One instance per mask element type; every 64-bit index starts
// from the zero-extended thread and workgroup ids.
template <typename M>
__global__ __launch_bounds__(kWeightThreads) void klp_grpo_weights_rows_kernel(
    TokenWeightsParams p) {
    __shared__ int64_t part[kWeightWaves];
    const int64_t tid = static_cast<int64_t>(threadIdx.x);
    for (int64_t b = static_cast<int64_t>(blockIdx.x); b < p.B; b += gridDim.x) {
        const int64_t base = b * p.S;
        const void* row_mask = mask_from<M>(p.mask, base);
        const int64_t v = block_sum_i64(
            strided_mask_sum<M>(row_mask, tid, kWeightThreads, p.S), part);
        const float den = fmaxf(static_cast<float>(v), 1.0f) * static_cast<float>(p.B);
        const float r = 1.0f / den;
        strided_weights<M>(row_mask, p.weights + base, r, tid, kWeightThreads, p.S);
    }
}

template <typename M>
__global__ __launch_bounds__(kWeightThreads) void klp_grpo_weights_partial_kernel(
    TokenWeightsParams p) {
    __shared__ int64_t part[kWeightWaves];
    const int64_t n = p.B * p.S;
    const int64_t first =
        static_cast<int64_t>(blockIdx.x) * kWeightThreads + static_cast<int64_t>(threadIdx.x);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kWeightThreads;
    const int64_t v = block_sum_i64(strided_mask_sum<M>(p.mask, first, stride, n), part);
    if (threadIdx.x == 0) p.partial[blockIdx.x] = v;
}

// How klp_grpo_weights_kernel gets its factor: the fixed scale; 1 / the
// total of the partial sums a previous launch left (one per workgroup of the
// same grid); or 1 / the mask's total summed by the one workgroup itself.
enum WeightsTotal { kScaleGiven = 0, kFromPartials = 1, kOwnSum = 2 };

template <typename M, int kTotal>
__global__ __launch_bounds__(kWeightThreads) void klp_grpo_weights_kernel(TokenWeightsParams p) {
    const int64_t n = p.B * p.S;
    const int64_t first =
        static_cast<int64_t>(blockIdx.x) * kWeightThreads + static_cast<int64_t>(threadIdx.x);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kWeightThreads;
    float r = p.scale;
    if constexpr (kTotal != kScaleGiven) {
        __shared__ int64_t part[kWeightWaves];
        int64_t v = 0;
        if constexpr (kTotal == kFromPartials) {
            for (uint32_t j = threadIdx.x; j < gridDim.x; j += kWeightThreads) v += p.partial[j];
        } else {
            v = strided_mask_sum<M>(p.mask, first, stride, n);  // gridDim.x == 1
        }
        r = 1.0f / fmaxf(static_cast<float>(block_sum_i64(v, part)), 1.0f);
    }
    strided_weights<M>(p.mask, p.weights, r, first, stride, n);
}

namespace {

// Workgroups of the grid-wide passes: one step of kWeightUnroll elements
// per thread (its loads in flight together), at most kGrpoWeightsMaxBlocks;
// larger inputs loop.
unsigned weights_blocks(int64_t n) {
    const int64_t per_block = int64_t{kWeightThreads} * kWeightUnroll;
    int64_t g = (n + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > kGrpoWeightsMaxBlocks) g = kGrpoWeightsMaxBlocks;
    return static_cast<unsigned>(g);
}

template <typename M>
hipError_t launch_token_weights_mask(const TokenWeightsParams& p, hipStream_t stream) {
    const dim3 block(kWeightThreads);
    if (p.kind == 0) {
        const unsigned rows = static_cast<unsigned>(p.B < 65535 ? p.B : 65535);
        return launch_kernel(klp_grpo_weights_rows_kernel<M>, dim3(rows), block, stream, p);
    }
    const dim3 grid(weights_blocks(p.B * p.S));
    if (p.kind == 1) {
        if (grid.x == 1)  // one workgroup: it sums the mask itself, one launch
            return launch_kernel(klp_grpo_weights_kernel<M, kOwnSum>, grid, block, stream, p);
        const hipError_t e =
            launch_kernel(klp_grpo_weights_partial_kernel<M>, grid, block, stream, p);
        if (e != hipSuccess) return e;
        return launch_kernel(klp_grpo_weights_kernel<M, kFromPartials>, grid, block, stream, p);
    }
    return launch_kernel(klp_grpo_weights_kernel<M, kScaleGiven>, grid, block, stream, p);
}

}  // namespace

hipError_t launch_grpo_token_weights(const TokenWeightsParams& p, hipStream_t stream) {
    if (p.kind < 0 || p.kind > 2) return hipErrorInvalidValue;
    if (p.mask == nullptr) return launch_token_weights_mask<void>(p, stream);
    switch (p.mask_dtype) {
        case KLP_MASK_U8: return launch_token_weights_mask<uint8_t>(p, stream);
        case KLP_MASK_I32: return launch_token_weights_mask<int32_t>(p, stream);
        case KLP_MASK_I64: return launch_token_weights_mask<int64_t>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_grpo_fwd(const GrpoParams& p, hipStream_t stream) {
    hipError_t e = launch_kernel(klp_grpo_rows_kernel, dim3(static_cast<unsigned>(p.B)),
                                 dim3(kGrpoThreads), stream, p);
    if (e != hipSuccess) return e;
    return launch_kernel(klp_grpo_finish_kernel, dim3(1), dim3(kGrpoThreads), stream, p);
}

hipError_t launch_grpo_bwd(const GrpoParams& p, hipStream_t stream) {
    return launch_kernel(klp_grpo_bwd_kernel, dim3(static_cast<unsigned>(p.B)),
                         dim3(kGrpoThreads), stream, p);
}

}  // namespace klp
