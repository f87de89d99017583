// klp_abi.hip — the C ABI of libkernel_opt_hip.so (include/kernel_opt_hip.h,
// include/kernel_opt_hip_tuning.h).
//
// Host-side counterpart of the reference's torch-level dispatch
// (csrc/fused_logprob.cu:284-458): argument checks with the same messages
// where an equivalent check exists, launch-shape selection, launch on the
// caller's stream, and a hipGetLastError() check after every launch (the
// reference has none).  Nothing here allocates, frees or synchronises.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <string>

#include "../../include/kernel_opt_hip.h"
#include "../../include/kernel_opt_hip_tuning.h"
#include "klp_launch.h"

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

constexpr int64_t kTargetBlocks = 2048;  // 8 workgroups per CU on 256 CUs
constexpr int kMaxSplits = 32;

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

int default_fwd_splits(int dtype, int64_t n_rows, int64_t vocab, int threads, int unroll) {
    const int64_t nvec = body_vectors(dtype, vocab);
    int s = 1;
    // Split while the grid is short of kTargetBlocks and every thread still
    // gets at least two full iterations per piece.
    while (s < kMaxSplits && n_rows * s < kTargetBlocks &&
           nvec / (2 * s) >= static_cast<int64_t>(threads) * unroll * 2)
        s *= 2;
    return s;
}

klp::FwdConfig default_fwd_config(int dtype, int64_t n_rows, int64_t vocab) {
    klp::FwdConfig c;
    c.waves = 8;
    c.unroll = 4;
    c.nontemporal = true;
    c.splits = default_fwd_splits(dtype, n_rows, vocab, c.waves * 64, c.unroll);
    return c;
}

klp::BwdConfig default_bwd_config(int dtype, int64_t n_rows, int64_t vocab) {
    klp::BwdConfig c;
    c.waves = 4;
    c.unroll = 2;
    c.nontemporal = true;
    const int64_t nvec = body_vectors(dtype, vocab);
    int s = 1;
    while (s < kMaxSplits && n_rows * s < kTargetBlocks &&
           nvec / (2 * s) >= static_cast<int64_t>(c.waves) * 64 * c.unroll)
        s *= 2;
    c.splits = s;
    return c;
}

size_t workspace_bytes_for(int64_t n_rows, int splits) {
    if (splits <= 1 || n_rows <= 0) return 0;
    const size_t padded = static_cast<size_t>((n_rows + 7) / 8) * 8;
    const size_t partial_bytes = padded * static_cast<size_t>(splits) * 4 * sizeof(float);
    const size_t counter_bytes = ((padded * sizeof(unsigned) + 15) / 16) * 16;
    return partial_bytes + counter_bytes;
}

int check_grid(int64_t n_rows, int splits, int threads) {
    const int64_t blocks = (splits == 1) ? n_rows : ((n_rows + 7) / 8) * 8 * splits;
    if (blocks > (int64_t{1} << 31) - 1 || blocks * threads > (int64_t{1} << 32) - 1)
        return fail(KLP_EINVAL, "grid of %lld workgroups x %d threads is too large",
                    static_cast<long long>(blocks), threads);
    return KLP_OK;
}

int fwd_impl(const void* logits, int dtype, int64_t n_rows, int64_t vocab, int64_t rows_inner,
             int64_t stride_outer, int64_t stride_inner, const int64_t* targets, float* logprob,
             float* entropy, float* lse, void* workspace, size_t workspace_bytes,
             klp::FwdConfig cfg, void* stream) {
    int rc = check_rows(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner,
                        targets);
    if (rc != KLP_OK) return rc;
    if (n_rows == 0) return ok();
    if ((rc = check_f32(logprob, "logprob")) != KLP_OK) return rc;
    if ((rc = check_f32(entropy, "entropy")) != KLP_OK) return rc;
    if ((rc = check_f32(lse, "lse")) != KLP_OK) return rc;
    if (!klp::fwd_config_supported(cfg) || cfg.splits < 1 || cfg.splits > 1024)
        return fail(KLP_EINVAL, "unsupported forward launch shape (waves=%d unroll=%d splits=%d)",
                    cfg.waves, cfg.unroll, cfg.splits);
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
    p.partials = nullptr;
    p.counters = nullptr;
    if (cfg.splits > 1) {
        // Layout: [counters: padded rows x u32, rounded up to 16 B][partials:
        // padded rows x splits x float4].  The kernel leaves both zero.
        const size_t padded = static_cast<size_t>((n_rows + 7) / 8) * 8;
        const size_t counter_bytes = ((padded * sizeof(unsigned) + 15) / 16) * 16;
        p.counters = static_cast<unsigned*>(workspace);
        p.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + counter_bytes);
    }
    if (injected_failure("forward")) return KLP_ELAUNCH;
    return after_launch(klp::launch_fwd(dtype, p, cfg, static_cast<hipStream_t>(stream)),
                        "forward");
}

int bwd_impl(const void* logits, int dtype, int64_t n_rows, int64_t vocab, int64_t rows_inner,
             int64_t stride_outer, int64_t stride_inner, const int64_t* targets, const float* lse,
             const float* entropy, const float* g_logp, const float* g_ent, const float* g_lse,
             void* d_logits, klp::BwdConfig cfg, void* stream) {
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
        return fail(KLP_EINVAL, "unsupported backward launch shape (waves=%d unroll=%d splits=%d)",
                    cfg.waves, cfg.unroll, cfg.splits);
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
    if (injected_failure("backward")) return KLP_ELAUNCH;
    return after_launch(klp::launch_bwd(dtype, p, cfg, static_cast<hipStream_t>(stream)),
                        "backward");
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
                    logprob, entropy, lse, workspace, workspace_bytes, cfg, stream);
}

int klp_fwd_ex(const void* logits, int dtype, int64_t n_rows, int64_t vocab, int64_t rows_inner,
               int64_t stride_outer, int64_t stride_inner, const int64_t* targets, float* logprob,
               float* entropy, float* lse, void* workspace, size_t workspace_bytes, int waves,
               int unroll, int splits, int nontemporal, void* stream) {
    klp::FwdConfig cfg;
    cfg.waves = waves;
    cfg.unroll = unroll;
    cfg.splits = splits;
    cfg.nontemporal = nontemporal != 0;
    return fwd_impl(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner, targets,
                    logprob, entropy, lse, workspace, workspace_bytes, cfg, stream);
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
                    lse, entropy, g_logp, g_ent, g_lse, d_logits, cfg, stream);
}

int klp_bwd_ex(const void* logits, int dtype, int64_t n_rows, int64_t vocab, int64_t rows_inner,
               int64_t stride_outer, int64_t stride_inner, const int64_t* targets,
               const float* lse, const float* entropy, const float* g_logp, const float* g_ent,
               const float* g_lse, void* d_logits, int waves, int unroll, int splits,
               int nontemporal, void* stream) {
    klp::BwdConfig cfg;
    cfg.waves = waves;
    cfg.unroll = unroll;
    cfg.splits = splits;
    cfg.nontemporal = nontemporal != 0;
    return bwd_impl(logits, dtype, n_rows, vocab, rows_inner, stride_outer, stride_inner, targets,
                    lse, entropy, g_logp, g_ent, g_lse, d_logits, cfg, stream);
}

void klp_default_config(int which, int dtype, int64_t n_rows, int64_t vocab, int* waves,
                        int* unroll, int* splits, int* nontemporal) {
    klp::FwdConfig c = (which == 0) ? default_fwd_config(dtype, n_rows, vocab)
                                    : default_bwd_config(dtype, n_rows, vocab);
    if (waves) *waves = c.waves;
    if (unroll) *unroll = c.unroll;
    if (splits) *splits = c.splits;
    if (nontemporal) *nontemporal = c.nontemporal ? 1 : 0;
}

}  // extern "C"
