/*
 * kernel_opt_hip.h — C ABI of the MI355X (gfx950) fused per-token
 * log-probability + entropy library (libkernel_opt_hip.so).
 *
 * This ABI replaces the pybind11 module `kernel_opt._C` of the reference
 * (csrc/bindings.cpp:17-27).  The three compute entry points correspond
 * one-to-one to the three functions that module exposes; argument meaning
 * and the out-parameter convention are the same, but tensors are passed as
 * raw device pointers plus sizes and strides, so no torch type crosses the
 * boundary.
 *
 * Conventions shared by every entry point
 * ---------------------------------------
 *  - `dtype` is a klp_dtype value and describes `logits` (and `d_logits`).
 *  - `n_rows` = N = product of the leading dims, `vocab` = V (last dim).
 *  - Row r of `logits` starts at element offset
 *        (r / rows_inner) * stride_outer + (r % rows_inner) * stride_inner
 *    from `logits`; elements inside a row are contiguous (unit stride).
 *    A contiguous [N, V] tensor is (rows_inner = N, stride_outer = 0,
 *    stride_inner = V).  The non-contiguous slice logits[:, :-1, :] of a
 *    [B, L, V] tensor is (rows_inner = L - 1, stride_outer = L * V,
 *    stride_inner = V).  Strides are in elements.
 *  - `targets` is int64 [N], contiguous.  A target outside [0, V) (for
 *    example an ignore index of -100) yields logprob = -lse and no one-hot
 *    term in the gradient, exactly as the reference kernels do.
 *  - Per-row outputs and saved/upstream tensors are float32 [N], contiguous.
 *  - Work is enqueued on `stream` (a hipStream_t; NULL = the legacy default
 *    stream).  No entry point synchronises, allocates or frees device
 *    memory.  N = 0 is a no-op that returns KLP_OK.
 *  - Every entry point returns a klp_status.  On failure a thread-local
 *    message is available from klp_last_error().
 */
#ifndef KERNEL_OPT_HIP_H
#define KERNEL_OPT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KLP_ABI_VERSION 1

typedef enum klp_dtype {
    KLP_BF16 = 0,
    KLP_FP16 = 1,
    KLP_FP32 = 2
} klp_dtype;

typedef enum klp_status {
    KLP_OK = 0,
    KLP_EINVAL = 1,       /* bad argument: null pointer, size, stride, alignment */
    KLP_EDTYPE = 2,       /* unsupported dtype */
    KLP_ELAUNCH = 3,      /* hipGetLastError() reported a failure after launch */
    KLP_EWORKSPACE = 4    /* workspace given but too small / misaligned */
} klp_status;

/* Version of this ABI (KLP_ABI_VERSION). */
int klp_abi_version(void);

/*
 * Copies the calling thread's last error message (NUL-terminated, truncated
 * to `len`) into `buf`.  Returns the full message length.
 */
size_t klp_last_error(char* buf, size_t len);

/*
 * Bytes of device workspace that klp_fwd can use to split each row across
 * several workgroups (split-row mode) for this problem size; 0 means the
 * dispatcher keeps one workgroup per row.  In split-row mode each row piece
 * writes its partial (max, sum-exp, sum-x-exp) state into the workspace and
 * counts itself in its row's arrival counter there; the piece that arrives
 * last merges the row's states in a fixed order (one kernel in all).
 *
 * The workspace must be zero-filled before its first use (with a fill
 * kernel, or hipMemset outside any graph capture); every call leaves it
 * zero-filled again, whatever the shapes of the calls that share it.
 * Launches that share one workspace must be ordered (same stream, or
 * synchronised): overlapping ones race on the counters.
 */
size_t klp_fwd_workspace_bytes(int dtype, int64_t n_rows, int64_t vocab);

/*
 * Forward: logprob[r] = logits[r, t_r] - lse[r], entropy[r] = -sum_v p log p,
 * lse[r] = logsumexp(logits[r]).  One streaming pass over each row.
 *
 * Replaces kernel_opt::fused_logprob_entropy_v1
 * (reference csrc/fused_logprob.cu:355-403, bound at csrc/bindings.cpp:21-23).
 *
 * `workspace` may be NULL (then one workgroup per row).  When it is not
 * NULL it must hold klp_fwd_workspace_bytes() bytes, be 16-byte aligned
 * and be zero-filled (see klp_fwd_workspace_bytes).
 */
int klp_fwd(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
            int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
            const int64_t* targets,
            float* logprob, float* entropy, float* lse,
            void* workspace, size_t workspace_bytes,
            void* stream);

/*
 * Naive forward: one thread per row, scalar recurrence.  Correctness anchor,
 * never fast.  Same outputs as klp_fwd up to fp32 rounding, except that, like
 * the reference naive kernel, a -inf logit after the first element of a row
 * makes that row's entropy NaN.
 *
 * Replaces kernel_opt::fused_logprob_entropy_naive
 * (reference csrc/fused_logprob.cu:405-458, bound at csrc/bindings.cpp:18-20).
 */
int klp_fwd_naive(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                  int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
                  const int64_t* targets,
                  float* logprob, float* entropy, float* lse,
                  void* stream);

/*
 * Backward: d_logits[r, v] = p_v * (g_lse - g_logp - g_ent * (log p_v + H))
 *                            + (v == t_r ? g_logp : 0),
 * p_v = exp(logits[r, v] - lse[r]), recomputed from the saved lse in one
 * read + one write pass.  `g_logp`, `g_ent` and `g_lse` may each be NULL,
 * meaning an all-zero upstream gradient (autograd's None).  `d_logits` is a
 * dense row-major [N, V] array of `dtype`, written with round-to-nearest-even.
 *
 * Replaces kernel_opt::fused_logprob_entropy_v1_backward
 * (reference csrc/fused_logprob.cu:284-346, bound at csrc/bindings.cpp:24-26).
 */
int klp_bwd(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
            int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
            const int64_t* targets,
            const float* lse, const float* entropy,
            const float* g_logp, const float* g_ent, const float* g_lse,
            void* d_logits,
            void* stream);

/*
 * Forward and backward with a sampling temperature T fused in: the logits are
 * multiplied by 1/T (rounded once to fp32) as they are loaded, and the
 * backward returns the gradient with respect to the unscaled logits (the
 * scaled-logit gradient times 1/T).  Saved lse/entropy passed to
 * klp_bwd_temp are those klp_fwd_temp produced with the same T.  No
 * counterpart in the reference kernels: they replace the GRPO trainer's
 * separate in-place `logits.div_(temperature)` pass (reference
 * python/kernel_opt/trainer.py:101) followed by the plain kernels.
 * T must be finite and > 0 (KLP_EINVAL otherwise); T = 1 equals
 * klp_fwd / klp_bwd exactly.  Other arguments as klp_fwd / klp_bwd.
 */
int klp_fwd_temp(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                 int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
                 const int64_t* targets, float temperature,
                 float* logprob, float* entropy, float* lse,
                 void* workspace, size_t workspace_bytes,
                 void* stream);

int klp_bwd_temp(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                 int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
                 const int64_t* targets, float temperature,
                 const float* lse, const float* entropy,
                 const float* g_logp, const float* g_ent, const float* g_lse,
                 void* d_logits,
                 void* stream);

/*
 * klp_fwd without a workspace argument, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation).  No counterpart in the reference.
 *
 * When the default launch shape splits rows (few rows of a long vocabulary),
 * the split-row workspace (piece states and row arrival counters) is a
 * scratch array of KLP_FWD_NOALLOC_SCRATCH_BYTES that the library keeps on
 * each GPU it runs on until the process ends; a problem whose workspace
 * would not fit is rejected with KLP_EWORKSPACE (the current dispatcher needs
 * at most 5 KiB: it splits only while rows x pieces <= 256).  The first call
 * on a device clears the array once (a synchronous hipMemset, so that first
 * call must not be made while a stream of that device is being captured);
 * every call leaves it zero-filled.  All calls on one GPU share that GPU's
 * array, so calls that overlap on one GPU (on other streams, from other
 * threads) race and must be ordered by the caller: overlapping calls can
 * also leave the array's counters non-zero, which breaks later calls.  The
 * array used is the current device's (hipGetDevice): `stream` must belong to
 * the current device.  Arguments and results as klp_fwd.
 */
#define KLP_FWD_NOALLOC_SCRATCH_BYTES 65536
int klp_fwd_noalloc(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                    int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
                    const int64_t* targets,
                    float* logprob, float* entropy, float* lse,
                    void* stream);

/*
 * Vocabulary shards (a vocab-parallel LM head: each rank holds columns
 * [vocab_offset, vocab_offset + vocab) of the logits).  No counterpart in the
 * reference, which has no multi-GPU path; these are the per-rank pieces of
 * the sharded forward:
 *   klp_fwd_shard writes, per row, the 16-byte online state of the row's
 *     shard, float4 (max, sum-exp, sum-x-exp in the kernels' base-2 units,
 *     target logit or 0), into `state` ([n_rows][4] float32, 16-byte
 *     aligned).  `targets` index the full vocabulary; the target logit is
 *     recorded by the shard that holds it.  Logits and temperature as
 *     klp_fwd_temp.
 *   klp_fwd_shard_merge merges the states of n_shards shards
 *     (`states` = [n_shards][n_rows][4], shard k holding columns
 *     [k * shard_vocab, min((k + 1) * shard_vocab, vocab))) in shard order
 *     and writes logprob, entropy, lse as klp_fwd.
 * Between the two, ranks exchange the 16-byte states (an all-gather); every
 * rank then merges in the same order and holds identical outputs.  The
 * backward needs no exchange: klp_bwd_temp on the shard, with the merged lse /
 * entropy and targets shifted by -vocab_offset (a target outside the shard
 * gets no one-hot term), writes the shard's d_logits.
 */
int klp_fwd_shard(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                  int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
                  const int64_t* targets, int64_t vocab_offset, float temperature,
                  float* state, void* stream);

int klp_fwd_shard_merge(const float* states, int64_t n_shards, int64_t n_rows,
                        const int64_t* targets, int64_t shard_vocab, int64_t vocab,
                        float* logprob, float* entropy, float* lse, void* stream);

/*
 * Vocabulary chunks on one GPU (the chunked LM head: the logits of one chunk
 * of columns exist at a time).  No counterpart in the reference, whose
 * Liger-style fused LM head is a stated follow-up it does not build
 * (docs/FINAL_REPORT.md:439-450).  Call it once per chunk, in chunk order on
 * one stream, with chunk `chunk_index` of `n_chunks` holding columns
 * [vocab_offset, vocab_offset + vocab) of the full vocabulary (chunks may
 * have any widths):
 *   chunk_index < n_chunks - 1: writes the rows' states to
 *     states[chunk_index] ([n_chunks][n_rows][4] float32, 16-byte aligned),
 *     as klp_fwd_shard does; the outputs are not read.
 *   chunk_index == n_chunks - 1: merges states[0 .. n_chunks - 2] (written
 *     by the earlier calls) in chunk order with its own chunk's and writes
 *     logprob, entropy and lse as klp_fwd; states[n_chunks - 1] is not used.
 * The outputs equal klp_fwd_shard on every chunk followed by
 * klp_fwd_shard_merge, bit for bit, in one launch fewer and without that
 * function's equal-width rule.
 */
int klp_fwd_chunk(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                  int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
                  const int64_t* targets, int64_t vocab_offset, float temperature,
                  float* states, int64_t chunk_index, int64_t n_chunks,
                  float* logprob, float* entropy, float* lse, void* stream);

/*
 * GRPO policy loss over per-token log-probabilities.  The reference plans it
 * as kernel "K2 fused_grpo_loss" (notes/PLAN.md:59) but ships it only as
 * eager PyTorch (examples/compare_one_step.py:232-236, the clipped surrogate
 * with a masked mean).  These entry points have no counterpart in
 * csrc/bindings.cpp.
 *
 * Inputs are float32, contiguous, [n_seqs, seq_len] (row b = one completion):
 *   logp      new per-token log-probabilities (the differentiated input);
 *   old_logp  log-probabilities of the sampling policy;
 *   ref_logp  reference-model log-probabilities, or NULL (no KL term);
 *   advantages [n_seqs], or [n_seqs, seq_len] when adv_per_token != 0;
 *   mask      completion mask (0 / 1 as float), or NULL for all ones.
 * Per token, with w = logp - old_logp (level KLP_GRPO_TOKEN) or the row's
 * masked mean of logp - old_logp (KLP_GRPO_SEQUENCE):
 *   c1 = exp(w), c2 = clamp(c1, 1 - eps_low, 1 + eps_high),
 *   loss_tok = -min(c1 * A, c2 * A) + beta * (exp(r - logp) - (r - logp) - 1)
 * with r = ref_logp (the KL term is dropped when ref_logp is NULL or
 * beta == 0).  The loss is the masked sum of loss_tok divided by:
 *   KLP_GRPO_LOSS_GRPO   n_seqs * max(row mask sum, 1), row by row;
 *   KLP_GRPO_LOSS_BNPO   max(batch mask sum, 1);
 *   KLP_GRPO_LOSS_FIXED  norm_const (> 0).
 * klp_grpo_fwd writes loss[0] and, if stats != NULL, stats[0..3] = masked
 * means of the KL estimate, of "clipped low" (c1 < 1 - eps_low and A < 0),
 * of "clipped high" (c1 > 1 + eps_high and A > 0), and of either.
 * klp_grpo_bwd writes d_logp = grad_loss[0] * d loss / d logp (grad_loss is
 * a device scalar, NULL meaning 1).  It reads the row sums klp_grpo_fwd left
 * in `workspace`: pass the same workspace, unchanged, with the same inputs.
 * Both need a workspace of klp_grpo_workspace_bytes(n_seqs) bytes, 4-byte
 * aligned, without initialisation.  eps_low and eps_high must be >= 0.
 */
typedef enum klp_grpo_loss_type {
    KLP_GRPO_LOSS_GRPO = 0,
    KLP_GRPO_LOSS_BNPO = 1,
    KLP_GRPO_LOSS_FIXED = 2
} klp_grpo_loss_type;

typedef enum klp_grpo_level {
    KLP_GRPO_TOKEN = 0,
    KLP_GRPO_SEQUENCE = 1
} klp_grpo_level;

size_t klp_grpo_workspace_bytes(int64_t n_seqs);

int klp_grpo_fwd(const float* logp, const float* old_logp, const float* ref_logp,
                 const float* advantages, const float* mask,
                 int64_t n_seqs, int64_t seq_len,
                 float eps_low, float eps_high, float beta, float norm_const,
                 int loss_type, int level, int adv_per_token,
                 float* loss, float* stats,
                 void* workspace, size_t workspace_bytes,
                 void* stream);

int klp_grpo_bwd(const float* logp, const float* old_logp, const float* ref_logp,
                 const float* advantages, const float* mask,
                 int64_t n_seqs, int64_t seq_len,
                 float eps_low, float eps_high, float beta, float norm_const,
                 int loss_type, int level, int adv_per_token,
                 const float* grad_loss, float* d_logp,
                 void* workspace, size_t workspace_bytes,
                 void* stream);

/*
 * Fused GRPO step: klp_fwd, the GRPO loss's per-token gradient and klp_bwd in
 * one pass over the logits.  No counterpart in the reference, whose trainer
 * runs the logprob kernel (python/kernel_opt/trainer.py:38-130), then the
 * eager loss (examples/compare_one_step.py:232-236), then the logprob
 * backward, one after another.  With token-level importance weights the
 * upstream gradient of a token's log-probability is
 * tok_weight * d loss_tok / d logp, known as soon as that token's logprob
 * is, so each workgroup keeps its row of logits in registers, computes
 * logprob / entropy / lse, then writes the row's d_logits at once: the
 * logits are read once instead of twice.
 *   logits, targets, temperature: as klp_fwd_temp (n_rows = n_seqs * seq_len
 *       token rows, row r of completion r / seq_len);
 *   old_logp, ref_logp (NULL: no KL term), advantages: as klp_grpo_fwd
 *       (advantages [n_rows / seq_len], or [n_rows] when adv_per_token);
 *   tok_weight [n_rows]: the weight of each token's loss in the batch loss,
 *       mask / normaliser (e.g. mask / max(sum mask, 1) for
 *       KLP_GRPO_LOSS_BNPO).
 *   grad_scale: the upstream gradient the caller will send into the batch
 *       loss, declared in advance (finite, non-zero): 1 for loss.backward();
 *       1 / k when a trainer divides the loss by k gradient-accumulation
 *       steps.  It multiplies the gradient, not loss_tok.
 * Writes logprob, entropy and (unless NULL) lse [n_rows] as klp_fwd;
 * loss_tok [n_rows] = tok_weight * loss_tok (the batch loss is their sum);
 * and d_logits (dense [n_rows, vocab], logits dtype, 16-byte aligned) =
 * grad_scale * d (sum loss_tok) / d logits, exactly klp_bwd's formula with
 * g_logp = tok_weight * d loss_tok / d logp * grad_scale (in that order, in
 * fp32) and g_ent = g_lse = 0.  The backward then applies the actual
 * upstream gradient with klp_rescale_inplace(d_logits, ..., grad_scale),
 * which writes nothing when the two are equal.
 * Only rows of at most klp_grpo_step_max_vocab(dtype) elements whose start
 * and length are whole 16-byte vectors are supported (row starts 16-byte
 * aligned, vocab * element size a multiple of 16); anything else returns
 * KLP_EINVAL, and the caller runs klp_fwd / klp_grpo_fwd / klp_grpo_bwd /
 * klp_bwd instead.
 * sched (nullable): KLP_GRPO_STEP_SCHED_BYTES of device memory, 8-byte
 * aligned, zero before the first call that gets it; every call leaves it
 * zero.  With it, batches of many rows longer than 64 KiB (8 or more rows
 * per resident workgroup) run on persistent workgroups that take rows from
 * a counter held there; without it, or for fewer or shorter rows, each row
 * has a workgroup of its own.
 * Results are the same bits either way.  Calls that share one must be
 * ordered (one stream): concurrent calls on one counter skip rows.
 */
#define KLP_GRPO_STEP_SCHED_BYTES 16

int64_t klp_grpo_step_max_vocab(int dtype);

int klp_grpo_step(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                  int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
                  const int64_t* targets, float temperature,
                  const float* old_logp, const float* ref_logp, const float* advantages,
                  const float* tok_weight, int64_t seq_len,
                  float eps_low, float eps_high, float beta, int adv_per_token,
                  float grad_scale, float* logprob, float* entropy, float* lse, float* loss_tok,
                  void* d_logits, void* sched, void* stream);

/*
 * The fused GRPO step's token weights from a mask, on the device: weights
 * [n_seqs, seq_len] float32 = m / normaliser with m the mask (NULL: all
 * ones) and the normaliser of `loss_type` (KLP_GRPO_LOSS_GRPO: n_seqs *
 * max(row sum of m, 1), row by row; KLP_GRPO_LOSS_BNPO: max(sum of m, 1);
 * KLP_GRPO_LOSS_FIXED: `scale` is the normaliser's float32 reciprocal), as
 * weights = m * (1 / normaliser).  No counterpart in the reference, whose
 * loss divides by the normaliser in eager PyTorch
 * (examples/compare_one_step.py:232-236); it replaces the chain of small
 * launches (row sums, clamp, scale, reciprocal, product) that computes
 * klp_grpo_step's tok_weight from the mask.  mask_dtype: KLP_MASK_U8 (bool
 * or uint8), KLP_MASK_I32, KLP_MASK_I64; the mask's sums are exact 64-bit
 * integer sums rounded once to float32, so the weights equal the float32
 * eager computation's bits whenever those sums are below 2^24 (any 0 / 1
 * mask of fewer than 2^24 tokens).  Floating-point masks are not taken.
 * workspace: KLP_GRPO_TOKEN_WEIGHTS_WORKSPACE_BYTES of device memory, 8-byte
 * aligned, for KLP_GRPO_LOSS_BNPO (per-workgroup partial sums of the mask;
 * its contents on entry do not matter); NULL is accepted for the other loss
 * types.  Calls that share one must be ordered (one stream).  The work is
 * spread over the device: one workgroup per row for KLP_GRPO_LOSS_GRPO, a
 * grid-wide pass (two for KLP_GRPO_LOSS_BNPO) otherwise.
 */
enum klp_mask_dtype {
    KLP_MASK_U8 = 0,
    KLP_MASK_I32 = 1,
    KLP_MASK_I64 = 2
};

#define KLP_GRPO_TOKEN_WEIGHTS_WORKSPACE_BYTES 8192

int klp_grpo_token_weights(const void* mask, int mask_dtype, int64_t n_seqs, int64_t seq_len,
                           int loss_type, float scale, float* weights, void* workspace,
                           void* stream);

/*
 * data[i] *= *scale for i in [0, n), in place, on the stream: each element is
 * multiplied in fp32 and rounded once to `dtype` (RNE), as torch's
 * `tensor * float` computes it.  `scale` is a device pointer read by the
 * kernel; when *scale == 1 nothing is written.  No counterpart in the
 * reference.  It is for gradients computed in the forward (klp_grpo_step's
 * d_logits; the chunked LM head's d_hidden and d_weight), whose backward only
 * applies the loss's upstream gradient: kept on the device, that scalar needs
 * no host synchronisation.  data aligned to its element size, n >= 0.
 */
int klp_scale_inplace(void* data, int dtype, int64_t n, const float* scale, void* stream);

/*
 * data[i] *= *scale / applied for i in [0, n), in place, on the stream, for
 * a buffer that already holds its values multiplied by `applied` (the
 * upstream gradient declared in advance, klp_grpo_step's grad_scale): when
 * *scale == applied nothing is written; otherwise each element is
 * multiplied in fp32 by fp32(*scale / applied) and rounded once to `dtype`
 * (RNE).  klp_scale_inplace is this with applied = 1 (the factor is then
 * *scale itself).  No counterpart in the reference.  applied finite and
 * non-zero; the rest as klp_scale_inplace.
 */
int klp_rescale_inplace(void* data, int dtype, int64_t n, const float* scale, float applied,
                        void* stream);

/*
 * Fused LM head + per-token logprob / entropy, forward.  No counterpart in the
 * reference, which names it as its follow-up (a Liger-style fused linear +
 * loss, docs/FINAL_REPORT.md:439-450): instead of logits = hidden @ weight^T
 * followed by klp_fwd, one MFMA GEMM folds each block of logits into the
 * online softmax state as it is produced, so the [n_tokens, vocab] logits
 * are never written.
 *   hidden  bf16 [n_tokens, ld_hidden] (first `dim` columns), 16-byte aligned;
 *   weight  bf16 [vocab, ld_weight] (nn.Linear layout), 16-byte aligned;
 *   dim a positive multiple of 64; ld_hidden, ld_weight >= dim, multiples of 8;
 *   targets int64 [n_tokens]; outputs float32 [n_tokens] as klp_fwd;
 *   temperature T > 0: logits are fp32(sum) * fp32(1/T).
 * Logits are the fp32 MFMA sums (not rounded to bf16 as a bf16 GEMM output
 * would be).  The workspace (klp_lmh_workspace_bytes bytes, 16-byte aligned,
 * no initialisation) holds per-(token, vocab chunk) partial states; launches
 * sharing one must be ordered on one stream.
 */
size_t klp_lmh_workspace_bytes(int64_t n_tokens, int64_t vocab, int64_t dim);

int klp_lmh_fwd(const void* hidden, int64_t ld_hidden, const void* weight, int64_t ld_weight,
                int64_t n_tokens, int64_t vocab, int64_t dim, const int64_t* targets,
                float temperature, float* logprob, float* entropy, float* lse,
                void* workspace, size_t workspace_bytes, void* stream);

/*
 * The backward's d_logits for the fused LM head: recomputes each block of
 * logits exactly as klp_lmh_fwd did (same MFMA order, hence the same fp32
 * values behind the saved lse / entropy) and writes
 *   d_logits[n, v] = klp_bwd's gradient of that logit (times 1/T),
 * rounded to bf16, into `d_logits` (bf16 [n_tokens, ld_d], 8-byte aligned,
 * ld_d >= vocab and a multiple of 4).  Columns vocab .. round_up(vocab, 4) - 1
 * are written with 0 (stores go out four columns at a time); columns past
 * them are not touched.
 * d_hidden = d_logits @ weight and d_weight = d_logits^T @ hidden are then
 * plain GEMMs for the caller.  lse / entropy are klp_lmh_fwd's outputs for
 * the same inputs and temperature; g_logp / g_ent / g_lse may be NULL.
 */
int klp_lmh_bwd_logits(const void* hidden, int64_t ld_hidden, const void* weight,
                       int64_t ld_weight, int64_t n_tokens, int64_t vocab, int64_t dim,
                       const int64_t* targets, float temperature, const float* lse,
                       const float* entropy, const float* g_logp, const float* g_ent,
                       const float* g_lse, void* d_logits, int64_t ld_d, void* stream);

/*
 * Test hook with no counterpart in the reference: the next `count` compute
 * calls on the calling thread return KLP_ELAUNCH without launching anything,
 * as if hipGetLastError() had reported a failure.  Lets the error path be
 * tested on machines without a GPU.  count = 0 disarms it.
 */
void klp_debug_fail_next_launches(int count);

#ifdef __cplusplus
}
#endif

#endif /* KERNEL_OPT_HIP_H */
