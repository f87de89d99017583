// klp_abi.hip — the C ABI of libkernel_opt_hip.so (include/kernel_opt_hip.h,
// include/kernel_opt_hip_tuning.h).
//
// Host-side counterpart of the reference's torch-level dispatch
// (csrc/fused_logprob.cu:284-458): argument checks with the same messages
// where an equivalent check exists, launch-shape selection, launch on the
// caller's stream, and a hipGetLastError() check after every launch (the
// reference has none).  Nothing here allocates, frees or synchronises.
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <math.h>
#include <string.h>

#include <mutex>
#include <string>

#include "../../include/kernel_opt_hip.h"
#include "../../include/kernel_opt_hip_tuning.h"
#include "klp_launch.h"

// Scratch of klp_fwd_noalloc: the split-row workspace (piece states and row
// arrival counters), cleared once per device at set-up and left zero by every
// call.  Each GPU holds its own copy until the process ends.  In host code
// `scratch` is only a stand-in for the symbol: its address on a device comes
// from hipGetSymbolAddress (noalloc_scratch below) and only that address is
// ever passed to a kernel or to hipMemset.
static __device__ __align__(256) unsigned char scratch[KLP_FWD_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_last_error;
thread_local int g_fail_next = 0;


int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int ok() {
    g_last_error.clear();
    return KLP_OK;
}

int elem_bytes(int dtype) { return dtype == KLP_FP32 ? 4 : 2; }

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// Launch-shape targets.  Forward: grids of fewer than kFwdTargetWaves
// wave64s (16 per CU on 256 CUs) at 8 waves per row are "few rows", where
// rows are split across workgroups (up to kFwdSplitGrid of them, one per
// CU) to put more loads in flight.  Backward: see default_bwd_config.
constexpr int64_t kFwdTargetWaves = 4096;
constexpr int64_t kFwdSplitGrid = 256;
// Wave64s resident at 8 per SIMD on 256 CUs: a grid up to this size runs as
// one round of workgroups.
constexpr int64_t kFwdOneRoundWaves = 8192;
constexpr int64_t kBwdLargeGrid = 65536;
constexpr int64_t kBwdSmallGrid = 16384;
constexpr int kMaxSplits = 64;
// fp32 backward rows of 4-wave workgroups (C5: 128 pieces of one iteration).
constexpr int kMaxSplitsFp32 = 256;
// MI355X's Infinity Cache (256 MB, memory-side, shared by the XCDs).
constexpr int64_t kInfinityCacheBytes = int64_t{256} << 20;
// Backward grids of this many row pieces and more (512 per CU) take pieces
// of up to 33/32 of an iteration rather than at most one.
constexpr int64_t kBwdManyPieces = 131072;

// Shared checks of the row-addressed logits operand.
int check_rows(const void* logits, int dtype, int64_t n_rows, int64_t vocab, int64_t rows_inner,
               int64_t stride_outer, int64_t stride_inner, const int64_t* targets) {
    if (dtype != KLP_BF16 && dtype != KLP_FP16 && dtype != KLP_FP32)
        return fail(KLP_EDTYPE, "logits dtype must be bf16, fp16, or fp32");
    if (vocab < 1) return fail(KLP_EINVAL, "vocab (last dim of logits) must be >= 1, got %lld",
                               static_cast<long long>(vocab));
    if (n_rows < 0) return fail(KLP_EINVAL, "n_rows must be >= 0");
    if (n_rows == 0) return KLP_OK;
    if (logits == nullptr || targets == nullptr)
        return fail(KLP_EINVAL, "logits and targets must be non-null");
    if (!aligned(logits, elem_bytes(dtype)))
        return fail(KLP_EINVAL, "logits pointer is not aligned to its element size");
    if (!aligned(targets, 8)) return fail(KLP_EINVAL, "targets pointer is not 8-byte aligned");
    if (rows_inner < 1) return fail(KLP_EINVAL, "rows_inner must be >= 1");
    if (stride_inner < 0 || stride_outer < 0)
        return fail(KLP_EINVAL, "row strides must be non-negative");
    if (n_rows > (int64_t{1} << 31) - 1)
        return fail(KLP_EINVAL, "n_rows above 2^31-1 is not supported");
    return KLP_OK;
}

int check_f32(const float* p, const char* name) {
    if (p == nullptr) return fail(KLP_EINVAL, "%s must be non-null", name);
    if (!aligned(p, 4)) return fail(KLP_EINVAL, "%s is not 4-byte aligned", name);
    return KLP_OK;
}

int after_launch(hipError_t e, const char* what) {
    if (e != hipSuccess)
        return fail(KLP_ELAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
    return ok();
}

bool injected_failure(const char* what) {
    if (g_fail_next <= 0) return false;
    --g_fail_next;
    fail(KLP_ELAUNCH, "%s launch failed: injected failure (klp_debug_fail_next_launches)", what);
    return true;
}

int64_t body_vectors(int dtype, int64_t vocab) { return vocab / (16 / elem_bytes(dtype)); }

// Bytes of the largest vector piece of a backward row in `splits` pieces (the
// kernel rounds pieces up to 8 vectors); its buffer offsets are 32-bit, so
// this must stay under 2 GiB.
int64_t bwd_piece_bytes(int dtype, int64_t vocab, int64_t splits) {
    const int64_t per = (body_vectors(dtype, vocab) + splits - 1) / splits;
    return ((per + 7) & ~int64_t{7}) * 16;
}

// Bytes the forward's buffer loads address for one row piece: the piece's
// body vectors plus the kFwdRing chunks its ring may prefetch past them (out
// of range, never read); the offsets are 32-bit, so this must stay under
// 2 GiB.
int64_t fwd_piece_bytes(int dtype, int64_t vocab, const klp::FwdConfig& c) {
    const int64_t per = (body_vectors(dtype, vocab) + c.splits - 1) / c.splits;
    return (per + int64_t{klp::kFwdRing} * c.waves * 64 * c.unroll) * 16;
}

int check_fwd_piece(int dtype, int64_t vocab, const klp::FwdConfig& c) {
    if (fwd_piece_bytes(dtype, vocab, c) > int64_t{INT32_MAX})
        return fail(KLP_EINVAL,
                    "forward row pieces must be under 2 GiB (vocab %lld in %d pieces): use "
                    "more splits",
                    static_cast<long long>(vocab), c.splits);
    return KLP_OK;
}

klp::FwdConfig default_fwd_config(int dtype, int64_t n_rows, int64_t vocab) {
    klp::FwdConfig c;
    c.flags = 0;
    c.splits = 1;
    const int64_t nvec = body_vectors(dtype, vocab);
    // Up to 8 waves per row, fewer for short rows so that each thread keeps
    // at least 8 vectors (rows that short take few threads whatever the
    // batch: [65536, 9496] bf16, 2 waves 206 us vs 4 waves 272 us).
    int w = 8;
    while (w > 1 && int64_t{w} * 64 * 8 > nvec) w /= 2;
    if (w == 8 && n_rows * w < kFwdTargetWaves) {
        // Few rows of a long vocabulary: 8-wave workgroups, unroll 2, rows
        // split in a power of two of pieces while the grid stays within one
        // workgroup per CU and each thread keeps at least 3 vectors.  GPU
        // times with launches queued (one box; bf16 unless noted):
        //   [1, 152064]   8 pieces 5.4 us   (unsplit, 16 waves 9.8 us)
        //   [8, 152064]   8 pieces 5.9 us   (16 pieces 6.2, unsplit 10.0)
        //   [32, 152064]  8 pieces 7.3 us   (4 pieces 7.5, unsplit 10.9)
        //   [128, 152064] 2 pieces 10.9 us  (unsplit 11.5, 4 pieces 11.4)
        //   [16, 128256] fp16: 8 pieces 6.8 us (unsplit 9.9)
        //   [64, 262144] fp32: 4 pieces 13.8 us (unsplit 24.3, 8 pieces 14.5)
        // Unsplit, rows of at least 16384 vectors also take 8 waves
        // ([256, 152064]: 12.8 us vs 14.6 on 16 waves, unroll 4); shorter
        // ones 16 waves, unroll 4 (C1, [256, 32000] fp32: 5.9 us vs 6.4).
        int s = 1;
        while (s < kMaxSplits && n_rows * 2 * s <= kFwdSplitGrid &&
               nvec >= int64_t{3} * 8 * 64 * 2 * s)
            s *= 2;
        if (s > 1 || nvec >= 16384) {
            c.waves = 8;
            c.unroll = 2;
            c.splits = s;
        } else {
            c.waves = 16;
            c.unroll = 4;
        }
    } else if (n_rows * w <= kFwdOneRoundWaves) {
        // All workgroups resident at once (C2: 1024 rows x 8 waves, 8 waves
        // per SIMD): unroll 2 keeps a wave at 61 VGPRs (unroll 4: ~100, 4
        // waves per SIMD).  C2, one box: 8 waves unroll 2 48.1 us, 4 waves
        // unroll 4 48.9 us, 16 waves unroll 4 57.6 us.
        c.waves = w;
        c.unroll = 2;
    } else {
        // Several rounds of workgroups: unroll 4 for rows of at least 16
        // vectors per thread (C3 8 waves: unroll 4 301 us vs unroll 2 312 us;
        // a C4 vocab shard [32768, 18992], 4 waves: unroll 2 195 us vs 4
        // 206 us); fp32 rows on 4 waves (C5: 1204 us vs 1233 us on 8).
        c.waves = (dtype == KLP_FP32 && w > 4) ? 4 : w;
        c.unroll = (nvec / (int64_t{c.waves} * 64) >= 16) ? 4 : 2;
    }
    return c;
}

klp::BwdConfig default_bwd_config(int dtype, int64_t n_rows, int64_t vocab) {
    klp::BwdConfig c;
    c.waves = 16;
    c.unroll = 2;
    c.flags = klp::kFlagNtStore;
    c.splits = 1;
    const int64_t nvec = body_vectors(dtype, vocab);
    // Rows shorter than one iteration of 16 waves take fewer waves (down to
    // 4) rather than idle lanes (bf16 [65536, 9496]: 8 waves 403 us vs 16
    // waves 485 us; [8192, 4096]: 4 waves 22.6 us vs 48.7 us).
    while (c.waves > 4 && int64_t{c.waves} * 64 * c.unroll > nvec) c.waves /= 2;
    const int64_t tile = static_cast<int64_t>(c.waves) * 64 * c.unroll;
    // Pieces of at least 15/16 of one iteration (`tile` vectors, 32 KB),
    // a power of two of them per row.  Short-lived workgroups of one to two
    // iterations measured fastest for this mixed read/write stream (C3: 8
    // pieces 665 us vs 4 pieces 729 us; C5: 32 pieces 2925 us vs 8 3099 us).
    int64_t s = 1;
    while (s < kMaxSplits && nvec / (2 * s) >= tile - tile / 16) s *= 2;
    // Grids of many workgroups: the fewest pieces that keep every piece
    // within one iteration, if each still fills 7/8 of it (C4, 32768 rows:
    // 10 pieces of 0.93 iterations 3183 us vs 8 3356 us vs 12 3498 us).  On
    // smaller grids that was slower (C2, 1024 rows: 10 pieces 104.8-107.9 us
    // vs 8 103.6-104.5 us), and so were pieces far below one iteration.
    if (n_rows * s >= kBwdLargeGrid) {
        int64_t e = (nvec + tile - 1) / tile;
        if (e > kMaxSplits) e = kMaxSplits;
        if (e >= 1 && nvec / e >= tile - tile / 8) s = e;
    }
    // Small grids (up to kBwdSmallGrid workgroups of 16 waves: C1, C2) and
    // fp32 rows: 8-wave workgroups over twice the pieces, each the same
    // fraction of its iteration.  C2 [1024, 152064] bf16: 101.7 us against
    // 104.5-105.2 back to back, 101.4-101.9 against 102.1-103.0 flushed (two
    // boxes); C1 equal back to back, 14.4-14.8 against 15.4-15.7 flushed.
    // fp32 (half the arithmetic per byte of bf16 / fp16): C5 2829 against
    // 2895 us, [8192, 32000] 329 against 344, [32768, 32000] 1283 against
    // 1331, [4096, 152064] 802 against 825, [2048, 262144] 697 against 685.
    // Larger bf16 / fp16 grids keep 16 waves (C3 666 against 662 us, C4
    // 3251 against 3131 us).
    if (c.waves == 16 && (n_rows * s <= kBwdSmallGrid || dtype == KLP_FP32) &&
        2 * s <= kMaxSplits) {
        c.waves = 8;
        s *= 2;
        // fp32 rows halve again: 4-wave workgroups over twice the pieces.
        // C5 2742-2769 us against 2837-2839 (two boxes), [32768, 32000] 1280
        // against 1302, [8192, 32000] 322 against 326, [2048, 262144] 689
        // against 698, C1 10.1 against 10.4 back to back; [4096, 152064] and
        // [64, 32000] equal, [256, 152064] 46.1 against 45.6.
        if (dtype == KLP_FP32 && 2 * s <= kMaxSplitsFp32) {
            c.waves = 4;
            s *= 2;
        }
    }
    // bf16 / fp16 logits larger than the Infinity Cache: 4-wave workgroups
    // over pieces of about one iteration (512 vectors): the fewest pieces of
    // at most one iteration, or on grids of kBwdManyPieces pieces and more of
    // at most 33/32 of one (fewer workgroups to dispatch), if each fills 7/8
    // of an iteration.  The rules above leave Qwen's vocabularies at 1.16
    // iterations a piece.  Measured back to back / flushed / after a forward:
    //  - C2 [1024, 152064], 38 pieces of 504 vectors: 96.0-98.5 / 98.0-98.7 /
    //    97.2-98.3 us against 99.7-100.1 / 100.8-101.3 / 100.0-101.2 for 8
    //    waves x 16 (four boxes); 36 pieces of 528 ~1% slower than 38;
    //  - C4 [32768, 151936], 36 pieces of 528: 3007-3010 / 2997-2998 /
    //    2998-3001 us against 3185-3231 / 3094-3111 / 3155-3173 for 16 waves
    //    x 10 (two boxes); 38 pieces of 504 3085-3239 / 3143-3317 / 3109-3154;
    //  - C3 [8192, 128256] fp16, 31 pieces of 520: 642 / 653 / 648 us
    //    against 660 / 654 / 673 for 32 pieces and 663 / 679 / 668 for 16
    //    waves x 8;
    //  - against the previous shapes: [32768, 18992] 0.95-0.97x,
    //    [4096, 152064] 0.94-0.97x, [16384, 65536] 0.88-0.90x,
    //    [2048, 262144] 0.86-0.88x, fp16 [4096, 128256] 0.95-0.96x,
    //    [8192, 32000] 0.98-0.99x; [1024, 256000] 1.00-1.02x (at 63 pieces
    //    of at most one iteration).
    // Logits the cache holds keep the shapes above: their back-to-back
    // re-reads hit it, and smaller pieces measured up to 12% slower there
    // ([1024, 100352]: 13 pieces of 8 waves 66.8 against 59.6 us).
    if (dtype != KLP_FP32 && n_rows * vocab * elem_bytes(dtype) >= kInfinityCacheBytes) {
        const int64_t tile4 = int64_t{4} * 64 * 2;
        int64_t e = (nvec + tile4 - 1) / tile4;
        if (n_rows * e >= kBwdManyPieces) {
            const int64_t cap = tile4 + tile4 / 32;
            e = (nvec + cap - 1) / cap;
        }
        if (e >= 1 && e <= kMaxSplits && nvec / e >= tile4 - tile4 / 8) {
            c.waves = 4;
            c.unroll = 2;
            s = e;
        }
    }
    // Rows of more than 2 GiB per 64 pieces (never a real vocabulary) take
    // more pieces.
    while (s < 1024 && bwd_piece_bytes(dtype, vocab, s) > int64_t{INT32_MAX}) s *= 2;
    c.splits = static_cast<int>(s);
    return c;
}

// Split-row workspace: the pieces' float4 states, then one 32-bit arrival
// counter per row (rounded up to 16 bytes).
size_t partials_bytes(int64_t n_rows, int splits) {
    return static_cast<size_t>(n_rows) * static_cast<size_t>(splits) * 4 * sizeof(float);
}

size_t workspace_bytes_for(int64_t n_rows, int splits) {
    if (splits <= 1 || n_rows <= 0) return 0;
    const size_t counters = (static_cast<size_t>(n_rows) * sizeof(unsigned int) + 15) & ~size_t{15};
    return partials_bytes(n_rows, splits) + counters;
}

// 1/temperature rounded once to fp32; rejects temperatures that are not
// finite and positive.
bool scale_from_temperature(float temperature, float* scale) {
    if (!(temperature > 0.0f) || temperature == INFINITY) {
        fail(KLP_EINVAL, "temperature must be finite and > 0, got %g",
             static_cast<double>(temperature));
        return false;
    }
    *scale = static_cast<float>(1.0 / static_cast<double>(temperature));
    return true;
}

int check_grid(int64_t n_rows, int splits, int threads) {
    const int64_t blocks = n_rows * splits;
    if (blocks > (int64_t{1} << 31) - 1 || blocks * threads > (int64_t{1} << 32) - 1)
        return fail(KLP_EINVAL, "grid of %lld workgroups x %d threads is too large",
                    static_cast<long long>(blocks), threads);
    return KLP_OK;
}

int fwd_impl(const void* logits, int dtype, int64_t n_rows, int64_t vocab, int64_t rows_inner,
             int64_t stride_outer, int64_t stride_inner, const int64_t* targets, float* logprob,
             float* entropy, float* lse, void* workspace, size_t workspace_bytes,
             klp::FwdConfig cfg, float scale, void* stream) {
    int rc = check_rows(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner,
                        targets);
    if (rc != KLP_OK) return rc;
    if (n_rows == 0) return ok();
    if ((rc = check_f32(logprob, "logprob")) != KLP_OK) return rc;
    if ((rc = check_f32(entropy, "entropy")) != KLP_OK) return rc;
    if ((rc = check_f32(lse, "lse")) != KLP_OK) return rc;
    if (!klp::fwd_config_supported(cfg) || cfg.splits < 1 || cfg.splits > 1024 || cfg.flags != 0)
        return fail(KLP_EINVAL,
                    "unsupported forward launch shape (waves=%d unroll=%d splits=%d flags=%d)",
                    cfg.waves, cfg.unroll, cfg.splits, cfg.flags);
    if (cfg.splits > 1) {
        const size_t need = workspace_bytes_for(n_rows, cfg.splits);
        if (workspace == nullptr) {
            cfg.splits = 1;  // no workspace: one workgroup per row
        } else if (workspace_bytes < need || !aligned(workspace, 16)) {
            return fail(KLP_EWORKSPACE,
                        "workspace too small or not 16-byte aligned: have %zu bytes, need %zu",
                        workspace_bytes, need);
        }
    }
    if ((rc = check_fwd_piece(dtype, vocab, cfg)) != KLP_OK) return rc;
    if ((rc = check_grid(n_rows, cfg.splits, cfg.waves * 64)) != KLP_OK) return rc;

    klp::FwdParams p;
    p.logits = logits;
    p.rm = klp::RowMap{rows_inner, stride_outer, stride_inner};
    p.n_rows = n_rows;
    p.vocab = vocab;
    p.targets = targets;
    p.logprob = logprob;
    p.entropy = entropy;
    p.lse = lse;
    p.splits = cfg.splits;
    p.partials = (cfg.splits > 1) ? static_cast<float*>(workspace) : nullptr;
    p.counters = (cfg.splits > 1)
                     ? reinterpret_cast<unsigned int*>(static_cast<unsigned char*>(workspace) +
                                                       partials_bytes(n_rows, cfg.splits))
                     : nullptr;
    p.scale = scale;
    p.target_offset = 0;
    p.state = nullptr;
    p.merge_states = nullptr;
    p.merge_count = 0;
    if (injected_failure("forward")) return KLP_ELAUNCH;
    return after_launch(klp::launch_fwd(dtype, p, cfg, static_cast<hipStream_t>(stream)),
                        "forward");
}

int bwd_impl(const void* logits, int dtype, int64_t n_rows, int64_t vocab, int64_t rows_inner,
             int64_t stride_outer, int64_t stride_inner, const int64_t* targets, const float* lse,
             const float* entropy, const float* g_logp, const float* g_ent, const float* g_lse,
             void* d_logits, klp::BwdConfig cfg, float scale, void* stream) {
    int rc = check_rows(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner,
                        targets);
    if (rc != KLP_OK) return rc;
    if (n_rows == 0) return ok();
    if ((rc = check_f32(lse, "lse")) != KLP_OK) return rc;
    if ((rc = check_f32(entropy, "entropy")) != KLP_OK) return rc;
    if (g_logp && !aligned(g_logp, 4)) return fail(KLP_EINVAL, "g_logp is not 4-byte aligned");
    if (g_ent && !aligned(g_ent, 4)) return fail(KLP_EINVAL, "g_ent is not 4-byte aligned");
    if (g_lse && !aligned(g_lse, 4)) return fail(KLP_EINVAL, "g_lse is not 4-byte aligned");
    if (d_logits == nullptr) return fail(KLP_EINVAL, "d_logits must be non-null");
    if (!aligned(d_logits, elem_bytes(dtype)))
        return fail(KLP_EINVAL, "d_logits pointer is not aligned to its element size");
    if (!klp::bwd_config_supported(cfg) || cfg.splits < 1 || cfg.splits > 1024)
        return fail(KLP_EINVAL,
                    "unsupported backward launch shape (waves=%d unroll=%d splits=%d flags=%d)",
                    cfg.waves, cfg.unroll, cfg.splits, cfg.flags);
    if (bwd_piece_bytes(dtype, vocab, cfg.splits) > int64_t{INT32_MAX})
        return fail(KLP_EINVAL,
                    "backward row pieces must be under 2 GiB (vocab %lld in %d pieces): use "
                    "more splits",
                    static_cast<long long>(vocab), cfg.splits);
    if ((rc = check_grid(n_rows, cfg.splits, cfg.waves * 64)) != KLP_OK) return rc;

    klp::BwdParams p;
    p.logits = logits;
    p.rm = klp::RowMap{rows_inner, stride_outer, stride_inner};
    p.n_rows = n_rows;
    p.vocab = vocab;
    p.targets = targets;
    p.lse = lse;
    p.entropy = entropy;
    p.g_logp = g_logp;
    p.g_ent = g_ent;
    p.g_lse = g_lse;
    p.d_logits = d_logits;
    p.splits = cfg.splits;
    p.scale = scale;
    if (injected_failure("backward")) return KLP_ELAUNCH;
    return after_launch(klp::launch_bwd(dtype, p, cfg, static_cast<hipStream_t>(stream)),
                        "backward");
}

size_t grpo_workspace_bytes(int64_t n_seqs) {
    if (n_seqs <= 0) return 0;
    return (static_cast<size_t>(n_seqs) * klp::kGrpoRowWords + 1) * sizeof(float);
}

bool finite_nonneg(float v) { return v >= 0.0f && v != INFINITY; }

// Shared checks and parameter block of klp_grpo_fwd / klp_grpo_bwd.
int grpo_setup(const float* logp, const float* old_logp, const float* ref_logp,
               const float* advantages, const float* mask, int64_t n_seqs, int64_t seq_len,
               float eps_low, float eps_high, float beta, float norm_const, int loss_type,
               int level, int adv_per_token, void* workspace, size_t workspace_bytes,
               klp::GrpoParams* p) {
    if (n_seqs < 1 || n_seqs > (int64_t{1} << 31) - 1)
        return fail(KLP_EINVAL, "n_seqs must be in [1, 2^31-1], got %lld",
                    static_cast<long long>(n_seqs));
    if (seq_len < 0) return fail(KLP_EINVAL, "seq_len must be >= 0");
    int rc;
    if ((rc = check_f32(logp, "logp")) != KLP_OK) return rc;
    if ((rc = check_f32(old_logp, "old_logp")) != KLP_OK) return rc;
    if ((rc = check_f32(advantages, "advantages")) != KLP_OK) return rc;
    if (ref_logp && (rc = check_f32(ref_logp, "ref_logp")) != KLP_OK) return rc;
    if (mask && (rc = check_f32(mask, "mask")) != KLP_OK) return rc;
    if (!finite_nonneg(eps_low) || !finite_nonneg(eps_high))
        return fail(KLP_EINVAL, "eps_low and eps_high must be finite and >= 0");
    if (!(beta == beta) || beta == INFINITY || beta == -INFINITY)
        return fail(KLP_EINVAL, "beta must be finite");
    if (loss_type != KLP_GRPO_LOSS_GRPO && loss_type != KLP_GRPO_LOSS_BNPO &&
        loss_type != KLP_GRPO_LOSS_FIXED)
        return fail(KLP_EINVAL, "unknown loss_type %d", loss_type);
    if (loss_type == KLP_GRPO_LOSS_FIXED && !(norm_const > 0.0f && norm_const != INFINITY))
        return fail(KLP_EINVAL, "norm_const must be finite and > 0 for KLP_GRPO_LOSS_FIXED");
    if (level != KLP_GRPO_TOKEN && level != KLP_GRPO_SEQUENCE)
        return fail(KLP_EINVAL, "unknown importance level %d", level);
    const size_t need = grpo_workspace_bytes(n_seqs);
    if (workspace == nullptr || workspace_bytes < need || !aligned(workspace, 4))
        return fail(KLP_EWORKSPACE,
                    "workspace missing, too small or not 4-byte aligned: have %zu bytes, need %zu",
                    workspace_bytes, need);
    p->logp = logp;
    p->old_logp = old_logp;
    p->ref_logp = ref_logp;
    p->adv = advantages;
    p->mask = mask;
    p->B = n_seqs;
    p->S = seq_len;
    p->eps_low = eps_low;
    p->eps_high = eps_high;
    p->beta = beta;
    p->norm_const = norm_const;
    p->loss_type = loss_type;
    p->level = level;
    p->adv_per_token = adv_per_token != 0;
    p->ws = static_cast<float*>(workspace);
    p->loss = nullptr;
    p->stats = nullptr;
    p->grad_loss = nullptr;
    p->d_logp = nullptr;
    return KLP_OK;
}

// Fused LM head: vocab tiles per workgroup chunk, chosen so that the grid
// holds about four rounds of one workgroup per CU (256 CUs).
void lmh_plan(int64_t n_tokens, int64_t vocab, int64_t* tiles_per_chunk, int64_t* n_chunks) {
    const int64_t tb = klp::lmh_token_blocks(n_tokens);
    const int64_t vt = klp::lmh_vocab_tiles(vocab);
    int64_t tpc = (tb * vt) / (256 * 4);
    if (tpc < 1) tpc = 1;
    if (tpc > 16) tpc = 16;
    *tiles_per_chunk = tpc;
    *n_chunks = (vt + tpc - 1) / tpc;
}

size_t lmh_workspace_bytes(int64_t n_tokens, int64_t vocab) {
    if (n_tokens <= 0 || vocab <= 0) return 0;
    int64_t tpc, nc;
    lmh_plan(n_tokens, vocab, &tpc, &nc);
    return static_cast<size_t>(nc) * static_cast<size_t>(n_tokens) * 4 * sizeof(float);
}

int ceiling_impl(int mode, const void* src, void* dst, int64_t n_rows, int64_t row_bytes,
                 int waves, int unroll, int splits, uint32_t* sink, uint32_t magic,
                 void* stream) {
    static const char* const kWhat[] = {"ceiling read", "ceiling copy", "ceiling read pieces",
                                        "ceiling write"};
    const char* what = kWhat[mode];
    const bool reads = mode != klp::kCeilWrite;
    const bool writes = mode == klp::kCeilCopy || mode == klp::kCeilWrite;
    const bool folds = mode == klp::kCeilRead || mode == klp::kCeilReadPieces;
    if (n_rows < 0) return fail(KLP_EINVAL, "n_rows must be >= 0");
    if (row_bytes < 16 || row_bytes % 16 != 0)
        return fail(KLP_EINVAL, "row_bytes must be a positive multiple of 16, got %lld",
                    static_cast<long long>(row_bytes));
    if (n_rows == 0) return ok();
    if (reads && (src == nullptr || !aligned(src, 16)))
        return fail(KLP_EINVAL, "src must be non-null and 16-byte aligned");
    if (writes && (dst == nullptr || !aligned(dst, 16)))
        return fail(KLP_EINVAL, "dst must be non-null and 16-byte aligned");
    if (folds && (sink == nullptr || !aligned(sink, 4)))
        return fail(KLP_EINVAL, "sink must be non-null and 4-byte aligned");
    const bool w = (waves == 1 || waves == 2 || waves == 4 || waves == 8 || waves == 16);
    if (!w || (unroll != 2 && unroll != 4) || splits < 1 || splits > 1024)
        return fail(KLP_EINVAL, "unsupported launch shape (waves=%d unroll=%d splits=%d)", waves,
                    unroll, splits);
    const int64_t nvec = row_bytes / 16;
    if (mode == klp::kCeilRead) {
        // the ring's buffer offsets: the piece plus the prefetched chunks
        const int64_t per = (nvec + splits - 1) / splits;
        const int64_t ahead = int64_t{klp::kFwdRing} * unroll * waves * 64;
        if ((per + ahead) * 16 > int64_t{INT32_MAX})
            return fail(KLP_EINVAL, "row pieces must be under 2 GiB: use more splits");
    } else if (((nvec + splits - 1) / splits + 7) / 8 * 8 * 16 > int64_t{INT32_MAX}) {
        return fail(KLP_EINVAL, "row pieces must be under 2 GiB: use more splits");
    }
    int rc;
    if ((rc = check_grid(n_rows, splits, waves * 64)) != KLP_OK) return rc;
    klp::CeilingParams p;
    p.src = src;
    p.dst = dst;
    p.n_rows = n_rows;
    p.row_bytes = row_bytes;
    p.splits = splits;
    p.sink = sink;
    p.magic = magic;
    if (injected_failure(what)) return KLP_ELAUNCH;
    return after_launch(
        klp::launch_ceiling(mode, p, waves, unroll, static_cast<hipStream_t>(stream)), what);
}

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

int noalloc_scratch(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return fail(KLP_ELAUNCH, "hipGetDevice failed: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxScratchDevices)
        return fail(KLP_EINVAL, "device %d is beyond the %d the scratch table holds", dev,
                    kMaxScratchDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr)
            return fail(KLP_ELAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                        hipGetErrorString(e));
        // The split-row kernels need the scratch zero before their first
        // launch (and leave it zero): one synchronous clear per device.
        e = hipMemset(p, 0, KLP_FWD_NOALLOC_SCRATCH_BYTES);
        if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
        if (e != hipSuccess)
            return fail(KLP_ELAUNCH, "clearing the scratch failed on device %d: %s", dev,
                        hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return KLP_OK;
}

}  // namespace

extern "C" {

int klp_abi_version(void) { return KLP_ABI_VERSION; }

size_t klp_last_error(char* buf, size_t len) {
    const size_t n = g_last_error.size();
    if (buf != nullptr && len > 0) {
        const size_t c = n < len - 1 ? n : len - 1;
        memcpy(buf, g_last_error.data(), c);
        buf[c] = '\0';
    }
    return n;
}

void klp_debug_fail_next_launches(int count) { g_fail_next = count > 0 ? count : 0; }

size_t klp_fwd_workspace_bytes(int dtype, int64_t n_rows, int64_t vocab) {
    if (dtype != KLP_BF16 && dtype != KLP_FP16 && dtype != KLP_FP32) return 0;
    if (n_rows <= 0 || vocab < 1) return 0;
    const klp::FwdConfig c = default_fwd_config(dtype, n_rows, vocab);
    return workspace_bytes_for(n_rows, c.splits);
}

size_t klp_fwd_workspace_bytes_ex(int64_t n_rows, int splits) {
    return workspace_bytes_for(n_rows, splits);
}

int klp_fwd(const void* logits, int dtype, int64_t n_rows, int64_t vocab, int64_t rows_inner,
            int64_t stride_outer, int64_t stride_inner, const int64_t* targets, float* logprob,
            float* entropy, float* lse, void* workspace, size_t workspace_bytes, void* stream) {
    klp::FwdConfig cfg = default_fwd_config(dtype, n_rows, vocab);
    return fwd_impl(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner, targets,
                    logprob, entropy, lse, workspace, workspace_bytes, cfg, 1.0f, stream);
}

int klp_fwd_ex(const void* logits, int dtype, int64_t n_rows, int64_t vocab, int64_t rows_inner,
               int64_t stride_outer, int64_t stride_inner, const int64_t* targets, float* logprob,
               float* entropy, float* lse, void* workspace, size_t workspace_bytes, int waves,
               int unroll, int splits, int flags, void* stream) {
    klp::FwdConfig cfg;
    cfg.waves = waves;
    cfg.unroll = unroll;
    cfg.splits = splits;
    cfg.flags = flags;
    return fwd_impl(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner, targets,
                    logprob, entropy, lse, workspace, workspace_bytes, cfg, 1.0f, stream);
}

int klp_fwd_naive(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                  int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
                  const int64_t* targets, float* logprob, float* entropy, float* lse,
                  void* stream) {
    int rc = check_rows(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner,
                        targets);
    if (rc != KLP_OK) return rc;
    if (n_rows == 0) return ok();
    if ((rc = check_f32(logprob, "logprob")) != KLP_OK) return rc;
    if ((rc = check_f32(entropy, "entropy")) != KLP_OK) return rc;
    if ((rc = check_f32(lse, "lse")) != KLP_OK) return rc;
    klp::NaiveParams p;
    p.logits = logits;
    p.rm = klp::RowMap{rows_inner, stride_outer, stride_inner};
    p.n_rows = n_rows;
    p.vocab = vocab;
    p.targets = targets;
    p.logprob = logprob;
    p.entropy = entropy;
    p.lse = lse;
    if (injected_failure("naive forward")) return KLP_ELAUNCH;
    return after_launch(klp::launch_fwd_naive(dtype, p, static_cast<hipStream_t>(stream)),
                        "naive forward");
}

int klp_bwd(const void* logits, int dtype, int64_t n_rows, int64_t vocab, int64_t rows_inner,
            int64_t stride_outer, int64_t stride_inner, const int64_t* targets, const float* lse,
            const float* entropy, const float* g_logp, const float* g_ent, const float* g_lse,
            void* d_logits, void* stream) {
    klp::BwdConfig cfg = default_bwd_config(dtype, n_rows, vocab);
    return bwd_impl(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner, targets,
                    lse, entropy, g_logp, g_ent, g_lse, d_logits, cfg, 1.0f, stream);
}

int klp_fwd_temp(const void* logits, int dtype, int64_t n_rows, int64_t vocab, int64_t rows_inner,
                 int64_t stride_outer, int64_t stride_inner, const int64_t* targets,
                 float temperature, float* logprob, float* entropy, float* lse, void* workspace,
                 size_t workspace_bytes, void* stream) {
    float scale;
    if (!scale_from_temperature(temperature, &scale)) return KLP_EINVAL;
    klp::FwdConfig cfg = default_fwd_config(dtype, n_rows, vocab);
    return fwd_impl(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner, targets,
                    logprob, entropy, lse, workspace, workspace_bytes, cfg, scale, stream);
}

int klp_bwd_temp(const void* logits, int dtype, int64_t n_rows, int64_t vocab, int64_t rows_inner,
                 int64_t stride_outer, int64_t stride_inner, const int64_t* targets,
                 float temperature, const float* lse, const float* entropy, const float* g_logp,
                 const float* g_ent, const float* g_lse, void* d_logits, void* stream) {
    float scale;
    if (!scale_from_temperature(temperature, &scale)) return KLP_EINVAL;
    klp::BwdConfig cfg = default_bwd_config(dtype, n_rows, vocab);
    return bwd_impl(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner, targets,
                    lse, entropy, g_logp, g_ent, g_lse, d_logits, cfg, scale, stream);
}

int klp_bwd_ex(const void* logits, int dtype, int64_t n_rows, int64_t vocab, int64_t rows_inner,
               int64_t stride_outer, int64_t stride_inner, const int64_t* targets,
               const float* lse, const float* entropy, const float* g_logp, const float* g_ent,
               const float* g_lse, void* d_logits, int waves, int unroll, int splits,
               int flags, void* stream) {
    klp::BwdConfig cfg;
    cfg.waves = waves;
    cfg.unroll = unroll;
    cfg.splits = splits;
    cfg.flags = flags;
    return bwd_impl(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner, targets,
                    lse, entropy, g_logp, g_ent, g_lse, d_logits, cfg, 1.0f, stream);
}

void klp_default_config(int which, int dtype, int64_t n_rows, int64_t vocab, int* waves,
                        int* unroll, int* splits, int* flags) {
    klp::FwdConfig c = (which == 0) ? default_fwd_config(dtype, n_rows, vocab)
                                    : default_bwd_config(dtype, n_rows, vocab);
    if (waves) *waves = c.waves;
    if (unroll) *unroll = c.unroll;
    if (splits) *splits = c.splits;
    if (flags) *flags = c.flags;
}

size_t klp_grpo_workspace_bytes(int64_t n_seqs) { return grpo_workspace_bytes(n_seqs); }

int klp_grpo_fwd(const float* logp, const float* old_logp, const float* ref_logp,
                 const float* advantages, const float* mask, int64_t n_seqs, int64_t seq_len,
                 float eps_low, float eps_high, float beta, float norm_const, int loss_type,
                 int level, int adv_per_token, float* loss, float* stats, void* workspace,
                 size_t workspace_bytes, void* stream) {
    klp::GrpoParams p;
    int rc = grpo_setup(logp, old_logp, ref_logp, advantages, mask, n_seqs, seq_len, eps_low,
                        eps_high, beta, norm_const, loss_type, level, adv_per_token, workspace,
                        workspace_bytes, &p);
    if (rc != KLP_OK) return rc;
    if ((rc = check_f32(loss, "loss")) != KLP_OK) return rc;
    if (stats && (rc = check_f32(stats, "stats")) != KLP_OK) return rc;
    p.loss = loss;
    p.stats = stats;
    if (injected_failure("grpo forward")) return KLP_ELAUNCH;
    return after_launch(klp::launch_grpo_fwd(p, static_cast<hipStream_t>(stream)),
                        "grpo forward");
}

int klp_grpo_bwd(const float* logp, const float* old_logp, const float* ref_logp,
                 const float* advantages, const float* mask, int64_t n_seqs, int64_t seq_len,
                 float eps_low, float eps_high, float beta, float norm_const, int loss_type,
                 int level, int adv_per_token, const float* grad_loss, float* d_logp,
                 void* workspace, size_t workspace_bytes, void* stream) {
    klp::GrpoParams p;
    int rc = grpo_setup(logp, old_logp, ref_logp, advantages, mask, n_seqs, seq_len, eps_low,
                        eps_high, beta, norm_const, loss_type, level, adv_per_token, workspace,
                        workspace_bytes, &p);
    if (rc != KLP_OK) return rc;
    if ((rc = check_f32(d_logp, "d_logp")) != KLP_OK) return rc;
    if (grad_loss && (rc = check_f32(grad_loss, "grad_loss")) != KLP_OK) return rc;
    p.grad_loss = grad_loss;
    p.d_logp = d_logp;
    if (injected_failure("grpo backward")) return KLP_ELAUNCH;
    return after_launch(klp::launch_grpo_bwd(p, static_cast<hipStream_t>(stream)),
                        "grpo backward");
}

// One launch over a vocabulary shard or chunk (one workgroup per row):
// writes the rows' states to `state`, or, with `merge_states` non-null (the
// last chunk of klp_fwd_chunk), merges the earlier chunks' states with its
// own and writes the outputs.
static int shard_impl(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                      int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
                      const int64_t* targets, int64_t vocab_offset, float scale, float* state,
                      const float* merge_states, int64_t merge_count, float* logprob,
                      float* entropy, float* lse, void* stream, const char* what) {
    // One workgroup per row (the states are per row, not per piece).
    klp::FwdConfig cfg = default_fwd_config(dtype, n_rows, vocab);
    if (cfg.splits > 1) {
        cfg.waves = 16;
        cfg.splits = 1;
    }
    int rc;
    if ((rc = check_fwd_piece(dtype, vocab, cfg)) != KLP_OK) return rc;
    if ((rc = check_grid(n_rows, 1, cfg.waves * 64)) != KLP_OK) return rc;
    klp::FwdParams p;
    p.logits = logits;
    p.rm = klp::RowMap{rows_inner, stride_outer, stride_inner};
    p.n_rows = n_rows;
    p.vocab = vocab;
    p.targets = targets;
    p.logprob = logprob;
    p.entropy = entropy;
    p.lse = lse;
    p.splits = 1;
    p.partials = nullptr;
    p.counters = nullptr;
    p.scale = scale;
    p.target_offset = vocab_offset;
    p.state = state;
    p.merge_states = merge_states;
    p.merge_count = merge_count;
    if (injected_failure(what)) return KLP_ELAUNCH;
    return after_launch(klp::launch_fwd(dtype, p, cfg, static_cast<hipStream_t>(stream)), what);
}

int klp_fwd_shard(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                  int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
                  const int64_t* targets, int64_t vocab_offset, float temperature, float* state,
                  void* stream) {
    int rc = check_rows(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner,
                        targets);
    if (rc != KLP_OK) return rc;
    float scale;
    if (!scale_from_temperature(temperature, &scale)) return KLP_EINVAL;
    if (vocab_offset < 0) return fail(KLP_EINVAL, "vocab_offset must be >= 0");
    if (n_rows == 0) return ok();
    if (state == nullptr || !aligned(state, 16))
        return fail(KLP_EINVAL, "state must be non-null and 16-byte aligned");
    return shard_impl(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner,
                      targets, vocab_offset, scale, state, nullptr, 0, nullptr, nullptr, nullptr,
                      stream, "shard forward");
}

int klp_fwd_chunk(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                  int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
                  const int64_t* targets, int64_t vocab_offset, float temperature, float* states,
                  int64_t chunk_index, int64_t n_chunks, float* logprob, float* entropy,
                  float* lse, void* stream) {
    int rc = check_rows(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner,
                        targets);
    if (rc != KLP_OK) return rc;
    float scale;
    if (!scale_from_temperature(temperature, &scale)) return KLP_EINVAL;
    if (vocab_offset < 0) return fail(KLP_EINVAL, "vocab_offset must be >= 0");
    if (n_chunks < 1 || chunk_index < 0 || chunk_index >= n_chunks)
        return fail(KLP_EINVAL, "chunk_index (%lld) must lie in [0, n_chunks) (n_chunks %lld)",
                    static_cast<long long>(chunk_index), static_cast<long long>(n_chunks));
    if (n_rows == 0) return ok();
    if (states == nullptr || !aligned(states, 16))
        return fail(KLP_EINVAL, "states must be non-null and 16-byte aligned");
    if (n_chunks > (int64_t{1} << 62) / 16 / n_rows)
        return fail(KLP_EINVAL, "n_chunks * n_rows states overflow");
    if (chunk_index + 1 < n_chunks)
        return shard_impl(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner,
                          targets, vocab_offset, scale, states + chunk_index * n_rows * 4,
                          nullptr, 0, nullptr, nullptr, nullptr, stream, "chunk forward");
    if ((rc = check_f32(logprob, "logprob")) != KLP_OK) return rc;
    if ((rc = check_f32(entropy, "entropy")) != KLP_OK) return rc;
    if ((rc = check_f32(lse, "lse")) != KLP_OK) return rc;
    return shard_impl(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner,
                      targets, vocab_offset, scale, nullptr, states, n_chunks - 1, logprob,
                      entropy, lse, stream, "chunk forward");
}

int klp_fwd_shard_merge(const float* states, int64_t n_shards, int64_t n_rows,
                        const int64_t* targets, int64_t shard_vocab, int64_t vocab,
                        float* logprob, float* entropy, float* lse, void* stream) {
    if (n_rows < 0) return fail(KLP_EINVAL, "n_rows must be >= 0");
    if (n_shards < 1) return fail(KLP_EINVAL, "n_shards must be >= 1");
    if (shard_vocab < 1 || vocab < 1 || vocab > n_shards * shard_vocab ||
        vocab <= (n_shards - 1) * shard_vocab)
        return fail(KLP_EINVAL,
                    "vocab (%lld) must lie in ((n_shards - 1) * shard_vocab, n_shards * "
                    "shard_vocab] (n_shards %lld, shard_vocab %lld)",
                    static_cast<long long>(vocab), static_cast<long long>(n_shards),
                    static_cast<long long>(shard_vocab));
    if (n_rows == 0) return ok();
    if (n_rows > (int64_t{1} << 31) - 1)
        return fail(KLP_EINVAL, "n_rows above 2^31-1 is not supported");
    if (states == nullptr || !aligned(states, 16))
        return fail(KLP_EINVAL, "states must be non-null and 16-byte aligned");
    if (targets == nullptr || !aligned(targets, 8))
        return fail(KLP_EINVAL, "targets must be non-null and 8-byte aligned");
    int rc;
    if ((rc = check_f32(logprob, "logprob")) != KLP_OK) return rc;
    if ((rc = check_f32(entropy, "entropy")) != KLP_OK) return rc;
    if ((rc = check_f32(lse, "lse")) != KLP_OK) return rc;
    klp::ShardMergeParams p;
    p.states = states;
    p.n_shards = n_shards;
    p.n_rows = n_rows;
    p.targets = targets;
    p.shard_vocab = shard_vocab;
    p.vocab = vocab;
    p.logprob = logprob;
    p.entropy = entropy;
    p.lse = lse;
    if (injected_failure("shard merge")) return KLP_ELAUNCH;
    return after_launch(klp::launch_shard_merge(p, static_cast<hipStream_t>(stream)),
                        "shard merge");
}

int klp_scale_inplace(void* data, int dtype, int64_t n, const float* scale, void* stream) {
    return klp_rescale_inplace(data, dtype, n, scale, 1.0f, stream);
}

int klp_rescale_inplace(void* data, int dtype, int64_t n, const float* scale, float applied,
                        void* stream) {
    if (!(applied == applied) || applied == INFINITY || applied == -INFINITY || applied == 0.0f)
        return fail(KLP_EINVAL, "applied must be finite and non-zero, got %g",
                    static_cast<double>(applied));
    if (dtype != KLP_BF16 && dtype != KLP_FP16 && dtype != KLP_FP32)
        return fail(KLP_EDTYPE, "dtype must be bf16, fp16, or fp32");
    if (n < 0) return fail(KLP_EINVAL, "n must be >= 0");
    if (n == 0) return ok();
    const int esz = elem_bytes(dtype);
    if (data == nullptr || !aligned(data, esz))
        return fail(KLP_EINVAL, "data must be non-null and aligned to its element size");
    if (scale == nullptr || !aligned(scale, 4))
        return fail(KLP_EINVAL, "scale must be non-null and 4-byte aligned");
    klp::ScaleParams p;
    p.data = data;
    p.n = n;
    const uintptr_t addr = reinterpret_cast<uintptr_t>(data);
    p.head = static_cast<int64_t>(((16u - (addr & 15u)) & 15u) / esz);
    if (p.head > n) p.head = n;
    p.nvec = (n - p.head) / (16 / esz);
    p.scale = scale;
    p.applied = applied;
    if (injected_failure("scale")) return KLP_ELAUNCH;
    return after_launch(klp::launch_scale(dtype, p, static_cast<hipStream_t>(stream)), "scale");
}

int klp_grpo_token_weights(const void* mask, int mask_dtype, int64_t n_seqs, int64_t seq_len,
                           int loss_type, float scale, float* weights, void* workspace,
                           void* stream) {
    if (n_seqs < 0 || seq_len < 0) return fail(KLP_EINVAL, "n_seqs and seq_len must be >= 0");
    if (loss_type != KLP_GRPO_LOSS_GRPO && loss_type != KLP_GRPO_LOSS_BNPO &&
        loss_type != KLP_GRPO_LOSS_FIXED)
        return fail(KLP_EINVAL, "unknown loss_type %d", loss_type);
    if (mask != nullptr && mask_dtype != KLP_MASK_U8 && mask_dtype != KLP_MASK_I32 &&
        mask_dtype != KLP_MASK_I64)
        return fail(KLP_EDTYPE, "mask must be bool / uint8, int32 or int64");
    if (n_seqs > 0 && seq_len > INT64_MAX / n_seqs)
        return fail(KLP_EINVAL, "n_seqs * seq_len overflows");
    if (n_seqs * seq_len == 0) return ok();
    if (weights == nullptr || !aligned(weights, 4))
        return fail(KLP_EINVAL, "weights must be non-null and 4-byte aligned");
    if (mask != nullptr) {
        const size_t a = mask_dtype == KLP_MASK_I64 ? 8 : mask_dtype == KLP_MASK_I32 ? 4 : 1;
        if (!aligned(mask, a)) return fail(KLP_EINVAL, "mask must be aligned to its element size");
    }
    if (loss_type == KLP_GRPO_LOSS_FIXED && !(scale > 0.0f && scale < INFINITY))
        return fail(KLP_EINVAL, "scale (1 / normaliser) must be finite and > 0, got %g",
                    static_cast<double>(scale));
    if (loss_type == KLP_GRPO_LOSS_BNPO && (workspace == nullptr || !aligned(workspace, 8)))
        return fail(KLP_EINVAL,
                    "KLP_GRPO_LOSS_BNPO needs a workspace of KLP_GRPO_TOKEN_WEIGHTS_WORKSPACE_BYTES, "
                    "8-byte aligned");
    klp::TokenWeightsParams p;
    p.mask = mask;
    p.mask_dtype = mask_dtype;
    p.kind = loss_type;
    p.B = n_seqs;
    p.S = seq_len;
    p.scale = scale;
    p.weights = weights;
    p.partial = static_cast<int64_t*>(workspace);
    if (injected_failure("grpo_token_weights")) return KLP_ELAUNCH;
    return after_launch(klp::launch_grpo_token_weights(p, static_cast<hipStream_t>(stream)),
                        "grpo_token_weights");
}

static_assert(KLP_GRPO_TOKEN_WEIGHTS_WORKSPACE_BYTES ==
                  klp::kGrpoWeightsMaxBlocks * sizeof(int64_t),
              "the token weights' workspace holds one partial sum per workgroup");

int64_t klp_grpo_step_max_vocab(int dtype) {
    if (dtype != KLP_BF16 && dtype != KLP_FP16 && dtype != KLP_FP32) return 0;
    return int64_t{klp::kGrpoStepMaxVec} * klp::kGrpoStepThreads * (16 / elem_bytes(dtype));
}

int klp_grpo_step(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                  int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
                  const int64_t* targets, float temperature, const float* old_logp,
                  const float* ref_logp, const float* advantages, const float* tok_weight,
                  int64_t seq_len, float eps_low, float eps_high, float beta, int adv_per_token,
                  float grad_scale, float* logprob, float* entropy, float* lse, float* loss_tok,
                  void* d_logits, void* sched, void* stream) {
    int rc = check_rows(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner,
                        targets);
    if (rc != KLP_OK) return rc;
    float scale;
    if (!scale_from_temperature(temperature, &scale)) return KLP_EINVAL;
    if (n_rows == 0) return ok();
    if (seq_len < 1 || n_rows % seq_len != 0)
        return fail(KLP_EINVAL, "n_rows (%lld) must be a positive multiple of seq_len (%lld)",
                    static_cast<long long>(n_rows), static_cast<long long>(seq_len));
    if (vocab > klp_grpo_step_max_vocab(dtype))
        return fail(KLP_EINVAL, "vocab %lld exceeds the fused GRPO step's row capacity %lld",
                    static_cast<long long>(vocab),
                    static_cast<long long>(klp_grpo_step_max_vocab(dtype)));
    const int64_t esz = elem_bytes(dtype);
    if ((vocab * esz) % 16 != 0 || !aligned(logits, 16) || (stride_inner * esz) % 16 != 0 ||
        (n_rows > rows_inner && (stride_outer * esz) % 16 != 0))
        return fail(KLP_EINVAL,
                    "fused GRPO step needs 16-byte aligned rows whose length is a multiple of "
                    "16 bytes");
    if ((rc = check_f32(old_logp, "old_logp")) != KLP_OK) return rc;
    if ((rc = check_f32(advantages, "advantages")) != KLP_OK) return rc;
    if ((rc = check_f32(tok_weight, "tok_weight")) != KLP_OK) return rc;
    if (ref_logp && (rc = check_f32(ref_logp, "ref_logp")) != KLP_OK) return rc;
    if ((rc = check_f32(logprob, "logprob")) != KLP_OK) return rc;
    if ((rc = check_f32(entropy, "entropy")) != KLP_OK) return rc;
    if (lse && (rc = check_f32(lse, "lse")) != KLP_OK) return rc;
    if ((rc = check_f32(loss_tok, "loss_tok")) != KLP_OK) return rc;
    if (d_logits == nullptr || !aligned(d_logits, 16))
        return fail(KLP_EINVAL, "d_logits must be non-null and 16-byte aligned");
    if (!finite_nonneg(eps_low) || !finite_nonneg(eps_high))
        return fail(KLP_EINVAL, "eps_low and eps_high must be finite and >= 0");
    if (!(beta == beta) || beta == INFINITY || beta == -INFINITY)
        return fail(KLP_EINVAL, "beta must be finite");
    if (!(grad_scale == grad_scale) || grad_scale == INFINITY || grad_scale == -INFINITY ||
        grad_scale == 0.0f)
        return fail(KLP_EINVAL, "grad_scale must be finite and non-zero, got %g",
                    static_cast<double>(grad_scale));
    if (sched != nullptr && !aligned(sched, 8))
        return fail(KLP_EINVAL, "sched must be 8-byte aligned");
    if ((rc = check_grid(n_rows, 1, klp::kGrpoStepThreads)) != KLP_OK) return rc;

    klp::GrpoStepParams p;
    p.logits = logits;
    p.rm = klp::RowMap{rows_inner, stride_outer, stride_inner};
    p.n_rows = n_rows;
    p.vocab = vocab;
    p.targets = targets;
    p.scale = scale;
    p.old_logp = old_logp;
    p.ref_logp = ref_logp;
    p.adv = advantages;
    p.tok_weight = tok_weight;
    p.seq_len = seq_len;
    p.eps_low = eps_low;
    p.eps_high = eps_high;
    p.beta = beta;
    p.adv_per_token = adv_per_token != 0;
    p.grad_scale = grad_scale;
    p.logprob = logprob;
    p.entropy = entropy;
    p.lse = lse;
    p.loss_tok = loss_tok;
    p.d_logits = d_logits;
    p.sched = static_cast<klp::StepSched*>(sched);
    if (injected_failure("grpo step")) return KLP_ELAUNCH;
    return after_launch(klp::launch_grpo_step(dtype, p, static_cast<hipStream_t>(stream)),
                        "grpo step");
}

int64_t klp_grpo_step_persistent_min_rows(int dtype, int64_t vocab, int scaled) {
    return klp::grpo_step_persistent_min_rows(dtype, vocab, scaled != 0);
}

size_t klp_lmh_workspace_bytes(int64_t n_tokens, int64_t vocab, int64_t dim) {
    (void)dim;
    return lmh_workspace_bytes(n_tokens, vocab);
}

// Checks shared by klp_lmh_fwd and klp_lmh_bwd_logits; fills the GEMM part
// of `p`.  Returns KLP_OK, or an error (after fail()).
int lmh_setup(const void* hidden, int64_t ld_hidden, const void* weight, int64_t ld_weight,
              int64_t n_tokens, int64_t vocab, int64_t dim, const int64_t* targets,
              float temperature, klp::LmhParams* p) {
    if (n_tokens < 0) return fail(KLP_EINVAL, "n_tokens must be >= 0");
    if (vocab < 1) return fail(KLP_EINVAL, "vocab must be >= 1, got %lld",
                               static_cast<long long>(vocab));
    if (dim < 64 || dim % 64 != 0)
        return fail(KLP_EINVAL, "dim must be a positive multiple of 64, got %lld",
                    static_cast<long long>(dim));
    if (ld_hidden < dim || ld_weight < dim || ld_hidden % 8 != 0 || ld_weight % 8 != 0)
        return fail(KLP_EINVAL, "row strides must be >= dim and multiples of 8 elements");
    if (n_tokens > (int64_t{1} << 31) - 1 || vocab > (int64_t{1} << 31) - 1)
        return fail(KLP_EINVAL, "n_tokens and vocab must be below 2^31");
    float scale;
    if (!scale_from_temperature(temperature, &scale)) return KLP_EINVAL;
    if (n_tokens == 0) return KLP_OK;
    if (hidden == nullptr || weight == nullptr || targets == nullptr)
        return fail(KLP_EINVAL, "hidden, weight and targets must be non-null");
    if (!aligned(hidden, 16) || !aligned(weight, 16))
        return fail(KLP_EINVAL, "hidden and weight must be 16-byte aligned");
    if (!aligned(targets, 8)) return fail(KLP_EINVAL, "targets pointer is not 8-byte aligned");
    *p = klp::LmhParams{};
    p->hidden = static_cast<const uint16_t*>(hidden);
    p->ld_hidden = ld_hidden;
    p->weight = static_cast<const uint16_t*>(weight);
    p->ld_weight = ld_weight;
    p->n_tokens = n_tokens;
    p->vocab = vocab;
    p->dim = dim;
    p->targets = targets;
    p->scale = scale;
    p->n_tblocks = klp::lmh_token_blocks(n_tokens);
    p->n_vtiles = klp::lmh_vocab_tiles(vocab);
    lmh_plan(n_tokens, vocab, &p->tiles_per_chunk, &p->n_chunks);
    const int64_t blocks = (p->n_chunks + 7) / 8 * 8 * p->n_tblocks;
    if (blocks > (int64_t{1} << 31) - 1)
        return fail(KLP_EINVAL, "grid of %lld workgroups is too large",
                    static_cast<long long>(blocks));
    return KLP_OK;
}

int klp_lmh_bwd_logits(const void* hidden, int64_t ld_hidden, const void* weight,
                       int64_t ld_weight, int64_t n_tokens, int64_t vocab, int64_t dim,
                       const int64_t* targets, float temperature, const float* lse,
                       const float* entropy, const float* g_logp, const float* g_ent,
                       const float* g_lse, void* d_logits, int64_t ld_d, void* stream) {
    klp::LmhParams p;
    int rc = lmh_setup(hidden, ld_hidden, weight, ld_weight, n_tokens, vocab, dim, targets,
                       temperature, &p);
    if (rc != KLP_OK) return rc;
    if (n_tokens == 0) return ok();
    if ((rc = check_f32(lse, "lse")) != KLP_OK) return rc;
    if ((rc = check_f32(entropy, "entropy")) != KLP_OK) return rc;
    if (g_logp && (rc = check_f32(g_logp, "g_logp")) != KLP_OK) return rc;
    if (g_ent && (rc = check_f32(g_ent, "g_ent")) != KLP_OK) return rc;
    if (g_lse && (rc = check_f32(g_lse, "g_lse")) != KLP_OK) return rc;
    if (d_logits == nullptr || !aligned(d_logits, 8) || ld_d < vocab || ld_d % 4 != 0)
        return fail(KLP_EINVAL,
                    "d_logits must be non-null and 8-byte aligned, with a row stride >= vocab "
                    "and a multiple of 4 elements");
    p.saved_lse = lse;
    p.saved_entropy = entropy;
    p.g_logp = g_logp;
    p.g_ent = g_ent;
    p.g_lse = g_lse;
    p.d_logits = static_cast<uint16_t*>(d_logits);
    p.ld_d = ld_d;
    if (injected_failure("lm-head backward")) return KLP_ELAUNCH;
    return after_launch(klp::launch_lmh_dlogits(p, static_cast<hipStream_t>(stream)),
                        "lm-head backward");
}

int klp_lmh_fwd(const void* hidden, int64_t ld_hidden, const void* weight, int64_t ld_weight,
                int64_t n_tokens, int64_t vocab, int64_t dim, const int64_t* targets,
                float temperature, float* logprob, float* entropy, float* lse, void* workspace,
                size_t workspace_bytes, void* stream) {
    klp::LmhParams p;
    int rc = lmh_setup(hidden, ld_hidden, weight, ld_weight, n_tokens, vocab, dim, targets,
                       temperature, &p);
    if (rc != KLP_OK) return rc;
    if (n_tokens == 0) return ok();
    if ((rc = check_f32(logprob, "logprob")) != KLP_OK) return rc;
    if ((rc = check_f32(entropy, "entropy")) != KLP_OK) return rc;
    if ((rc = check_f32(lse, "lse")) != KLP_OK) return rc;
    const size_t need = lmh_workspace_bytes(n_tokens, vocab);
    if (workspace == nullptr || workspace_bytes < need || !aligned(workspace, 16))
        return fail(KLP_EWORKSPACE,
                    "workspace missing, too small or not 16-byte aligned: have %zu bytes, need %zu",
                    workspace_bytes, need);
    p.partials = static_cast<float*>(workspace);
    p.logprob = logprob;
    p.entropy = entropy;
    p.lse = lse;
    if (injected_failure("lm-head forward")) return KLP_ELAUNCH;
    return after_launch(klp::launch_lmh_fwd(p, static_cast<hipStream_t>(stream)),
                        "lm-head forward");
}

int klp_ceiling_read(const void* src, int64_t n_rows, int64_t row_bytes, int waves, int unroll,
                     int splits, uint32_t* sink, uint32_t magic, void* stream) {
    return ceiling_impl(klp::kCeilRead, src, nullptr, n_rows, row_bytes, waves, unroll, splits,
                        sink, magic, stream);
}

int klp_ceiling_copy(const void* src, void* dst, int64_t n_rows, int64_t row_bytes, int waves,
                     int unroll, int splits, void* stream) {
    return ceiling_impl(klp::kCeilCopy, src, dst, n_rows, row_bytes, waves, unroll, splits,
                        nullptr, 0, stream);
}

int klp_ceiling_read_pieces(const void* src, int64_t n_rows, int64_t row_bytes, int waves,
                            int unroll, int splits, uint32_t* sink, uint32_t magic,
                            void* stream) {
    return ceiling_impl(klp::kCeilReadPieces, src, nullptr, n_rows, row_bytes, waves, unroll,
                        splits, sink, magic, stream);
}

int klp_ceiling_write(void* dst, int64_t n_rows, int64_t row_bytes, int waves, int unroll,
                      int splits, void* stream) {
    return ceiling_impl(klp::kCeilWrite, nullptr, dst, n_rows, row_bytes, waves, unroll, splits,
                        nullptr, 0, stream);
}

int klp_fwd_noalloc(const void* logits, int dtype, int64_t n_rows, int64_t vocab,
                    int64_t rows_inner, int64_t stride_outer, int64_t stride_inner,
                    const int64_t* targets, float* logprob, float* entropy, float* lse,
                    void* stream) {
    int rc = check_rows(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner,
                        targets);
    if (rc != KLP_OK) return rc;
    if (n_rows == 0) return ok();
    const klp::FwdConfig cfg = default_fwd_config(dtype, n_rows, vocab);
    const size_t need = workspace_bytes_for(n_rows, cfg.splits);
    if (need > KLP_FWD_NOALLOC_SCRATCH_BYTES)
        return fail(KLP_EWORKSPACE,
                    "klp_fwd_noalloc: %lld rows in %d pieces need %zu bytes of split-row scratch, "
                    "more than the %d it holds; use klp_fwd with a workspace",
                    static_cast<long long>(n_rows), cfg.splits, need,
                    KLP_FWD_NOALLOC_SCRATCH_BYTES);
    void* ws = nullptr;
    if (need > 0 && (rc = noalloc_scratch(&ws)) != KLP_OK) return rc;
    return fwd_impl(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner, targets,
                    logprob, entropy, lse, ws, ws ? size_t{KLP_FWD_NOALLOC_SCRATCH_BYTES} : 0, cfg,
                    1.0f, stream);
}

}  // extern "C"
