/*
 * kernel_opt_hip_tuning.h — launch-shape control for libkernel_opt_hip.so.
 *
 * None of these entry points has a counterpart in the reference (whose
 * launch shape is fixed: one 256-thread block per row,
 * csrc/fused_logprob.cu:313,376).  They exist for benchmarks, sweeps and
 * tests that must pin a launch shape (for example to exercise split-row mode
 * at a size where the default dispatcher would not choose it).  Results do
 * not depend on the launch shape beyond fp32 rounding of the reduction order.
 *
 * Conventions are those of kernel_opt_hip.h.  Supported shapes:
 * waves (wave64s per workgroup) in {1, 2, 4, 8, 16} for the forward and
 * {4, 8, 16} for the backward, unroll in {2, 4} (16-byte loads per thread per
 * iteration), splits in [1, 1024] (workgroups per row); the backward's row
 * pieces (vocab / splits, rounded up to 8 16-byte vectors) must stay under
 * 2 GiB (KLP_EINVAL otherwise).
 * `flags` selects kernel variants: forward: must be 0; backward: bit 0 =
 * non-temporal gradient stores.
 */
#ifndef KERNEL_OPT_HIP_TUNING_H
#define KERNEL_OPT_HIP_TUNING_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Workspace bytes klp_fwd_ex needs for `splits` workgroups per row. */
size_t klp_fwd_workspace_bytes_ex(int64_t n_rows, int splits);

/* klp_fwd with an explicit launch shape.  splits > 1 needs a zero-filled
 * workspace (see klp_fwd_workspace_bytes). */
int klp_fwd_ex(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
               int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
               const int64_t* targets,
               float* logprob, float* entropy, float* lse,
               void* workspace, size_t workspace_bytes,
               int waves, int unroll, int splits, int flags,
               void* stream);

/* klp_bwd with an explicit launch shape (splits need no workspace). */
int klp_bwd_ex(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
               int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
               const int64_t* targets,
               const float* lse, const float* entropy,
               const float* g_logp, const float* g_ent, const float* g_lse,
               void* d_logits,
               int waves, int unroll, int splits, int flags,
               void* stream);

/* The launch shape klp_fwd (which = 0) or klp_bwd (which = 1) would pick. */
void klp_default_config(int which, int dtype, int64_t n_rows, int64_t vocab,
                        int* waves, int* unroll, int* splits, int* flags);

/*
 * Fewest rows from which klp_grpo_step, given a `sched` counter, runs its
 * persistent kernel on the current device for rows of `vocab` elements of
 * `dtype` (temperature 1 or not: the two variants are separate kernels);
 * -1 if the device cannot be queried; 0 for an unsupported dtype or vocab,
 * and for rows of at most 64 KiB, which always run one row per workgroup.
 */
int64_t klp_grpo_step_persistent_min_rows(int dtype, int64_t vocab, int scaled);

/*
 * Calibration kernels: the memory access of klp_fwd (klp_ceiling_read) and
 * of klp_bwd (klp_ceiling_copy; its loads alone, klp_ceiling_read_pieces;
 * its stores alone, klp_ceiling_write) without their arithmetic, for
 * measuring the read, copy, read-only and write-only rates this device
 * reaches at the same size and launch shape.  No counterpart in the
 * reference, whose roofline is priced against the device's nominal peak
 * (bench/plot_roofline.py, bench/ncu_parse.py:183-212).
 *
 * `src` (and `dst`) hold n_rows contiguous rows of `row_bytes` bytes (a
 * positive multiple of 16), 16-byte aligned.  waves in {1, 2, 4, 8, 16},
 * unroll in {2, 4}, splits in [1, 1024] workgroups per row.
 *
 * klp_ceiling_read streams every row piece (ceil(row / splits) 16-byte
 * vectors) through the forward's ring: unroll non-temporal 16-byte buffer
 * loads per thread per chunk, two chunks in flight ahead of the one being
 * folded, as klp_fwd loads them.  It xor-folds the words; a workgroup
 * writes its fold to sink[workgroup] (n_rows * splits uint32) only when it
 * equals `magic`.
 * klp_ceiling_copy copies src to dst with ordinary 16-byte loads and
 * non-temporal 16-byte stores, pieces rounded up to 8 vectors, unroll loads
 * then unroll stores per thread per iteration (as klp_bwd does); pieces
 * must stay under 2 GiB.
 * klp_ceiling_read_pieces runs the same loop with the loads alone (folded
 * into `sink` as klp_ceiling_read does); klp_ceiling_write with the stores
 * alone (each 16-byte vector of dst gets its index within the row).
 */
int klp_ceiling_read(const void* src, int64_t n_rows, int64_t row_bytes,
                     int waves, int unroll, int splits,
                     uint32_t* sink, uint32_t magic, void* stream);
int klp_ceiling_copy(const void* src, void* dst, int64_t n_rows, int64_t row_bytes,
                     int waves, int unroll, int splits, void* stream);
int klp_ceiling_read_pieces(const void* src, int64_t n_rows, int64_t row_bytes,
                            int waves, int unroll, int splits,
                            uint32_t* sink, uint32_t magic, void* stream);
int klp_ceiling_write(void* dst, int64_t n_rows, int64_t row_bytes,
                      int waves, int unroll, int splits, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KERNEL_OPT_HIP_TUNING_H */
