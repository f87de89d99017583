// klp_launch.h — kernel parameter blocks and launcher declarations shared by
// the kernel translation units and the C-ABI dispatcher (klp_abi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "klp_device.h"

namespace klp {

struct FwdParams {
    const void* logits;
    RowMap rm;
    int64_t n_rows;
    int64_t vocab;
    const int64_t* targets;
    float* logprob;
    float* entropy;
    float* lse;
    float* partials;  // [n_rows * splits] float4 (m, z, t, unused) when splits > 1
    int splits;
    float scale;      // 1 / temperature; logits are multiplied by it on load
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

hipError_t launch_fwd(int dtype, const FwdParams& p, const FwdConfig& c, hipStream_t stream);
hipError_t launch_fwd_naive(int dtype, const NaiveParams& p, hipStream_t stream);
hipError_t launch_bwd(int dtype, const BwdParams& p, const BwdConfig& c, hipStream_t stream);
bool fwd_config_supported(const FwdConfig& c);
bool bwd_config_supported(const BwdConfig& c);

}  // namespace klp
