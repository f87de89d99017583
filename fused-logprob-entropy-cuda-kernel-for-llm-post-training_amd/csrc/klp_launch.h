// klp_launch.h — kernel parameter blocks and launcher declarations shared by
// the kernel translation units and the C-ABI dispatcher (klp_abi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kernel_opt_hip.h"
#include "klp_device.h"

namespace klp {

// Depth of the forward's register ring: chunks are loaded kFwdRing - 1
// ahead of their use (klp_forward.hip).
constexpr int kFwdRing = 3;

struct FwdParams {
    const void* logits;
    RowMap rm;
    int64_t n_rows;
    int64_t vocab;
    const int64_t* targets;
    float* logprob;
    float* entropy;
    float* lse;
    // Split rows (splits > 1): [n_rows * splits] float4 (m, z, t, target
    // logit or 0) piece states and [n_rows] arrival counters, all zero
    // before the launch and left zero by it.
    float* partials;
    unsigned int* counters;
    int splits;
    float scale;      // 1 / temperature; logits are multiplied by it on load
    // Vocabulary shards (splits == 1 only): the row holds columns
    // [target_offset, target_offset + vocab) of the full vocabulary, and with
    // `state` non-null each row's float4 (m, z, t, target logit or 0) is
    // written there instead of the outputs.
    int64_t target_offset;
    float* state;
    // Last vocabulary chunk of klp_fwd_chunk (splits == 1, state null): the
    // earlier chunks' row states, [merge_count][n_rows] float4, merged in
    // chunk order with this launch's own before the outputs are written.
    // Null for every other launch.
    const float* merge_states;
    int64_t merge_count;
};

// Merge of per-shard row states (klp_fwd_shard_merge).
struct ShardMergeParams {
    const float* states;     // [n_shards][n_rows] float4
    int64_t n_shards;
    int64_t n_rows;
    const int64_t* targets;  // [n_rows], indices into the full vocabulary
    int64_t shard_vocab;     // columns per shard (the last may hold fewer)
    int64_t vocab;           // full vocabulary
    float* logprob;
    float* entropy;
    float* lse;
};

struct NaiveParams {
    const void* logits;
    RowMap rm;
    int64_t n_rows;
    int64_t vocab;
    const int64_t* targets;
    float* logprob;
    float* entropy;
    float* lse;
};

struct BwdParams {
    const void* logits;
    RowMap rm;
    int64_t n_rows;
    int64_t vocab;
    const int64_t* targets;
    const float* lse;
    const float* entropy;
    const float* g_logp;  // nullable
    const float* g_ent;   // nullable
    const float* g_lse;   // nullable
    void* d_logits;       // dense [n_rows, vocab]
    int splits;
    float scale;          // 1 / temperature (gradient is w.r.t. the unscaled logits)
};

// Launch shape: `waves` wave64s per workgroup, `unroll` 16-byte loads per
// thread per iteration, `splits` workgroups per row.  `flags` selects kernel
// variants: bit 0 (backward only) = non-temporal gradient stores.  The
// forward reads logits with non-temporal loads, the backward with ordinary
// ones.
struct FwdConfig {
    int waves;
    int unroll;
    int splits;
    int flags;
};
typedef FwdConfig BwdConfig;
constexpr int kFlagNtStore = 1;

template <typename... KArgs, typename... Args>
inline hipError_t launch_kernel(void (*kernel)(KArgs...), dim3 grid, dim3 block,
                                hipStream_t stream, Args... args) {
    hipLaunchKernelGGL(kernel, grid, block, 0, stream, args...);
    return hipGetLastError();
}

// GRPO loss (klp_grpo.hip).  Arrays are float32 [B, S] unless noted.
struct GrpoParams {
    const float* logp;
    const float* old_logp;
    const float* ref_logp;   // nullable
    const float* adv;        // [B], or [B, S] when adv_per_token
    const float* mask;       // nullable (all ones)
    int64_t B;
    int64_t S;
    float eps_low;
    float eps_high;
    float beta;
    float norm_const;
    int loss_type;           // klp_grpo_loss_type
    int level;               // klp_grpo_level
    int adv_per_token;
    float* ws;               // [B * kGrpoRowWords + 1]
    float* loss;             // forward: [1]
    float* stats;            // forward: [4], nullable
    const float* grad_loss;  // backward: device scalar, nullable (1)
    float* d_logp;           // backward: [B, S]
};
// Workspace words per row of the GRPO loss (5 used, padded).
constexpr int kGrpoRowWords = 8;

// Token weights of the GRPO step (klp_grpo_token_weights): a bool / uint8,
// int32 or int64 mask (or none: all ones) divided by the loss type's
// normaliser.
struct TokenWeightsParams {
    const void* mask;  // nullable (all ones)
    int mask_dtype;    // KLP_MASK_U8 / KLP_MASK_I32 / KLP_MASK_I64
    int kind;          // 0 "grpo", 1 "bnpo", 2 fixed (scale)
    int64_t B;
    int64_t S;
    float scale;       // kind 2: the normaliser's float32 reciprocal
    float* weights;    // [B, S]
    int64_t* partial;  // kind 1: one mask sum per workgroup (kGrpoWeightsMaxBlocks)
};
// Workgroups of the token-weights kernels' grid-wide passes at most; kind 1
// keeps one 64-bit partial sum per workgroup in the caller's workspace.
constexpr int kGrpoWeightsMaxBlocks = 1024;

// Row counter of the persistent GRPO step kernel (klp_grpo_step's `sched`):
// zero before a launch, and left zero by it.
struct StepSched {
    unsigned long long next;  // rows handed out after the first gridDim.x
    unsigned int done;        // workgroups past the last row
    unsigned int unused;
};

// Fused GRPO step (klp_grpo_step.hip): the row held in the registers of one
// workgroup.  Rows are token rows of a [B, S] batch (n_rows = B * S).
struct GrpoStepParams {
    const void* logits;
    RowMap rm;
    int64_t n_rows;
    int64_t vocab;
    const int64_t* targets;
    float scale;              // 1 / temperature
    const float* old_logp;    // [n_rows]
    const float* ref_logp;    // [n_rows], nullable
    const float* adv;         // [n_rows / seq_len], or [n_rows] when adv_per_token
    const float* tok_weight;  // [n_rows]: d batch-loss / d token-loss (mask / normaliser)
    int64_t seq_len;
    float eps_low;
    float eps_high;
    float beta;
    int adv_per_token;
    float grad_scale;         // multiplies every token's gradient (not its loss)
    float* logprob;           // [n_rows]
    float* entropy;           // [n_rows]
    float* lse;               // [n_rows], nullable
    float* loss_tok;          // [n_rows]: tok_weight * token loss
    void* d_logits;           // dense [n_rows, vocab], logits dtype
    StepSched* sched;         // nullable: one workgroup per row
};
// Most 16-byte vectors one thread of the step kernel holds (1024 threads).
constexpr int kGrpoStepMaxVec = 19;
constexpr int kGrpoStepThreads = 1024;
hipError_t launch_grpo_step(int dtype, const GrpoStepParams& p, hipStream_t stream);
// Rows from which launch_grpo_step runs the persistent kernel (given a
// counter) on the current device; -1 if unknown, 0 for unsupported rows.
int64_t grpo_step_persistent_min_rows(int dtype, int64_t vocab, bool scaled);

// In-place scaling by a device scalar (klp_scale_inplace): elements
// [0, head) and [head + nvec * per-vector, n) one by one, the nvec 16-byte
// vectors from element `head` (16-byte aligned) in between.
struct ScaleParams {
    void* data;
    int64_t n;
    int64_t head;
    int64_t nvec;
    const float* scale;       // device scalar g
    float applied;            // data holds values already scaled by this; factor g / applied
};

hipError_t launch_scale(int dtype, const ScaleParams& p, hipStream_t stream);

// Fused LM head forward (klp_lmhead.hip).
struct LmhParams {
    const uint16_t* hidden;  // bf16 [n_tokens, ld_hidden], first `dim` columns used
    int64_t ld_hidden;
    const uint16_t* weight;  // bf16 [vocab, ld_weight]
    int64_t ld_weight;
    int64_t n_tokens;
    int64_t vocab;
    int64_t dim;             // K, a multiple of 64
    const int64_t* targets;  // [n_tokens]
    float scale;             // 1 / temperature
    float* partials;         // [n_chunks, n_tokens] float4 (m, z, t, target logit)
    int64_t n_tblocks;       // ceil(n_tokens / 128)
    int64_t n_vtiles;        // ceil(vocab / 256)
    int64_t tiles_per_chunk;
    int64_t n_chunks;        // ceil(n_vtiles / tiles_per_chunk)
    float* logprob;
    float* entropy;
    float* lse;
    // d_logits (backward) only:
    const float* g_logp;     // nullable
    const float* g_ent;      // nullable
    const float* g_lse;      // nullable
    const float* saved_lse;  // [n_tokens], as the forward wrote it
    const float* saved_entropy;
    uint16_t* d_logits;      // bf16 [n_tokens, ld_d], ld_d a multiple of 4
    int64_t ld_d;
};
int64_t lmh_token_blocks(int64_t n_tokens);
int64_t lmh_vocab_tiles(int64_t vocab);
hipError_t launch_lmh_fwd(const LmhParams& p, hipStream_t stream);
hipError_t launch_lmh_dlogits(const LmhParams& p, hipStream_t stream);

// Calibration kernels (klp_ceiling.hip): rows of `row_bytes` (a multiple of
// 16) at `src` (and `dst`), 16-byte aligned and contiguous; `splits`
// workgroups per row.  Modes: the forward's ring read, and the backward's
// loop as a copy, its loads alone and its stores alone.
enum : int { kCeilRead = 0, kCeilCopy = 1, kCeilReadPieces = 2, kCeilWrite = 3 };
struct CeilingParams {
    const void* src;     // all modes but kCeilWrite
    void* dst;           // kCeilCopy, kCeilWrite
    int64_t n_rows;
    int64_t row_bytes;
    int64_t splits;
    uint32_t* sink;      // reads: [n_rows * splits], written when fold == magic
    uint32_t magic;
};
hipError_t launch_ceiling(int mode, const CeilingParams& p, int waves, int unroll,
                          hipStream_t stream);

hipError_t launch_fwd(int dtype, const FwdParams& p, const FwdConfig& c, hipStream_t stream);
hipError_t launch_shard_merge(const ShardMergeParams& p, hipStream_t stream);
hipError_t launch_fwd_naive(int dtype, const NaiveParams& p, hipStream_t stream);
hipError_t launch_bwd(int dtype, const BwdParams& p, const BwdConfig& c, hipStream_t stream);
hipError_t launch_grpo_fwd(const GrpoParams& p, hipStream_t stream);
hipError_t launch_grpo_bwd(const GrpoParams& p, hipStream_t stream);
hipError_t launch_grpo_token_weights(const TokenWeightsParams& p, hipStream_t stream);
bool fwd_config_supported(const FwdConfig& c);
bool bwd_config_supported(const BwdConfig& c);

}  // namespace klp
