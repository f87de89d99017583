// klp_forward.hip — forward kernels for gfx950.
//
//  klp_fwd_kernel        production forward (replaces the reference's
//                        fused_logprob_entropy_v1_kernel, csrc/fused_logprob.cu:156-227)
//  klp_fwd_naive_kernel  one thread per row, scalar recurrence (replaces
//                        fused_logprob_entropy_naive_kernel, :69-113)
//
// Production forward, per workgroup of WAVES wave64s:
//  - a workgroup owns one row, or one of `splits` contiguous pieces of a row;
//  - the row body is read with 16-byte loads (global_load_dwordx4), U per
//    thread per iteration, consecutive lanes on consecutive 16-byte words;
//    the few elements before the first 16-byte boundary and after the last
//    one (head / tail) are read as scalars by split 0;
//  - U vectors per thread form a chunk; chunks are loaded kFwdRing - 1 ahead
//    of their use into a ring of register sets (buffer loads), so that loads
//    stay in flight while a wave computes;
//  - every chunk costs one rescale plus one v_exp_f32 per element
//    (absorb() in klp_device.h);
//  - with a temperature T (FwdParams::scale = 1/T != 1) every logit is
//    multiplied by 1/T in fp32 as it is loaded, which fuses the GRPO trainer's
//    separate `logits.div_(temperature)` pass (reference trainer.py:101);
//  - lanes merge as one flat reduction (maximum, one rescale per lane, sums;
//    DPP within rows, v_permlane16/32_swap across them), the waves' states
//    through LDS by the same reduction in wave 0;
//  - split rows merge in the same launch: each piece stores its state in the
//    workspace and counts itself in the row's arrival counter (one
//    acquire-release atomic); the piece that arrives last merges all of the
//    row's states, lane k holding piece k, so the result does not depend on
//    which piece came last, then writes the outputs and puts the row's
//    workspace words back to zero for the next call.
#include "klp_device.h"
#include "klp_launch.h"

namespace klp {

// Chunk c of a workgroup's piece (U 16-byte vectors per thread, lanes on
// consecutive vectors) is loaded into register set c % kFwdRing, kFwdRing - 1
// chunks ahead of its use, by buffer loads over the piece's whole chunks:
// the loads of the next chunks stay in flight while a wave computes (a
// wave that loaded and then computed had nothing in flight while it
// computed), and prefetches past the last whole chunk are out of the
// buffer's range, so they read nothing and are never used.
template <int DT, bool kClamp, int U, bool kScaled>
__device__ __forceinline__ void absorb_chunk(Stat& s, const u32x4* v, float scale) {
    constexpr int EPV = Traits<DT>::kPerVec;
    float x[U * EPV];
#pragma unroll
    for (int u = 0; u < U; ++u) unpack<DT>(v[u], x + u * EPV);
    if (kScaled) {
#pragma unroll
        for (int j = 0; j < U * EPV; ++j) x[j] *= scale;
    }
    absorb<U * EPV, kClamp>(s, x);
}

template <int U, int NTHREADS>
__device__ __forceinline__ void load_chunk(u32x4* dst, const __amdgpu_buffer_rsrc_t rs, int c,
                                           int tid) {
#pragma unroll
    for (int u = 0; u < U; ++u)
        dst[u] = __builtin_amdgcn_raw_buffer_load_b128(
            rs, ((c * U + u) * NTHREADS + tid) * 16, 0, kBufNonTemporal);
}

template <int DT, bool kClamp, int U, int NTHREADS, bool kScaled>
__device__ __forceinline__ void scan_row_piece(Stat& s, const typename Traits<DT>::elem* rp,
                                               const u32x4* vp, int64_t head, int64_t tail_begin,
                                               int64_t vocab, bool with_edges, int64_t vb,
                                               int64_t ve, int tid, float scale) {
    // Scalar head / tail elements (fewer than 2 * EPV of them).
    if (with_edges) {
        const int64_t n_edge = head + (vocab - tail_begin);
        if (tid < n_edge) {
            const int64_t idx = (tid < head) ? tid : tail_begin + (tid - head);
            float x = to_f32<DT>(rp[idx]);
            if (kScaled) x *= scale;
            absorb<1, true>(s, &x);
        }
    }
    constexpr int step = NTHREADS * U;  // vectors per chunk
    // The host keeps (piece + kFwdRing chunks) * 16 bytes under 2^31, so
    // every buffer offset below fits in 32 bits.
    const int n_full = static_cast<int>((ve - vb) / step);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<u32x4*>(vp + vb), 0, n_full * step * 16, 0x00020000);
    u32x4 set[kFwdRing][U];
#pragma unroll
    for (int r = 0; r < kFwdRing - 1; ++r) load_chunk<U, NTHREADS>(set[r], rs, r, tid);
    __builtin_amdgcn_sched_barrier(0);
    int k = 0;
    for (; k + kFwdRing <= n_full; k += kFwdRing) {
#pragma unroll
        for (int r = 0; r < kFwdRing; ++r) {
            load_chunk<U, NTHREADS>(set[(r + kFwdRing - 1) % kFwdRing], rs, k + r + kFwdRing - 1,
                                    tid);
            // Keeps the prefetch ahead of the arithmetic: the scheduler would
            // otherwise sink it below to save registers.
            __builtin_amdgcn_sched_barrier(0);
            absorb_chunk<DT, kClamp, U, kScaled>(s, set[r], scale);
        }
    }
#pragma unroll
    for (int r = 0; r < kFwdRing - 1; ++r)
        if (k + r < n_full) absorb_chunk<DT, kClamp, U, kScaled>(s, set[r], scale);

    const int64_t i = vb + static_cast<int64_t>(n_full) * step + tid;
    if (i - tid < ve) {
        // Remainder: vectors past the end read as -inf, which the clamped
        // absorb ignores.
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t idx = i + u * NTHREADS;
            if (idx < ve) {
                v[u] = load16<true>(vp + idx);
            } else {
                const uint32_t w = Traits<DT>::kNegInfWord;
                v[u] = u32x4{w, w, w, w};
            }
        }
        absorb_chunk<DT, true, U, kScaled>(s, v, scale);
    }
}

__device__ __forceinline__ float readlane_f32(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Last chunk of a row set cut into vocabulary chunks (klp_fwd_chunk): wave 0
// merges the states of the earlier chunks, p.merge_states[k][row] for
// k < p.merge_count (written by the earlier chunks' launches on the same
// stream), in chunk order and then this chunk's own state `own` (lane 0's),
// the same sequence of combine() calls klp_fwd_shard_merge_kernel makes over
// the same states, so the outputs are bitwise equal to its.  The target logit
// is the one recorded by the chunk that holds the target: every other chunk
// records +0.0, so the last word whose bits are not all zero is taken (a
// target logit of +0.0 leaves +0.0, its own value).  Lanes load 64 states
// at a time; the combines run on lane-uniform values.
__device__ __forceinline__ void merge_chunks_final(const FwdParams& p, int64_t row,
                                                   const Stat own, float own_xt, int lane) {
    const float4* st = reinterpret_cast<const float4*>(p.merge_states);
    Stat acc = stat_empty();
    float xt = 0.0f;
    for (int64_t base = 0; base < p.merge_count; base += 64) {
        const int64_t k = base + lane;
        float4 q = make_float4(-INFINITY, 0.0f, 0.0f, 0.0f);
        if (k < p.merge_count) q = st[k * p.n_rows + row];
        const int cnt = static_cast<int>(p.merge_count - base < 64 ? p.merge_count - base : 64);
        for (int j = 0; j < cnt; ++j) {
            acc = combine(acc, Stat{readlane_f32(q.x, j), readlane_f32(q.y, j),
                                    readlane_f32(q.z, j)});
            const float w = readlane_f32(q.w, j);
            if (__float_as_uint(w) != 0u) xt = w;
        }
    }
    acc = combine(acc, Stat{readlane_f32(own.m, 0), readlane_f32(own.z, 0),
                            readlane_f32(own.t, 0)});
    const float w = readlane_f32(own_xt, 0);
    if (__float_as_uint(w) != 0u) xt = w;
    if (lane != 0) return;
    const RowOut o = finalize(acc, xt);
    p.logprob[row] = o.logp;
    p.entropy[row] = o.ent;
    p.lse[row] = o.lse;
}

// One workgroup's row (or row piece); the body of klp_fwd_kernel and of
// klp_fwd_chunk_final_kernel (kMergeChunks: the last chunk's launch of
// klp_fwd_chunk, which merges the chunks' states instead of writing its own).
template <int DT, int WAVES, int U, bool kSplit, bool kScaled, bool kMergeChunks>
__device__ __forceinline__ void fwd_row(const FwdParams& p) {
    typedef typename Traits<DT>::elem elem;
    constexpr int NTHREADS = WAVES * 64;
    constexpr int EPV = Traits<DT>::kPerVec;
    constexpr int ESZ = 16 / EPV;

    const int tid = threadIdx.x;
    const int64_t b = blockIdx.x;
    const int64_t row = kSplit ? b / p.splits : b;
    const int split = kSplit ? static_cast<int>(b - row * p.splits) : 0;

    const int64_t vocab = p.vocab;
    const elem* rp = static_cast<const elem*>(p.logits) + row_offset(p.rm, row);

    const uintptr_t addr = reinterpret_cast<uintptr_t>(rp);
    int64_t head = static_cast<int64_t>(((16u - (addr & 15u)) & 15u) / ESZ);
    if (head > vocab) head = vocab;
    const int64_t nvec = (vocab - head) / EPV;
    const int64_t tail_begin = head + nvec * EPV;
    const u32x4* vp = reinterpret_cast<const u32x4*>(rp + head);

    int64_t vb = 0, ve = nvec, per = nvec;
    if (kSplit) {
        per = (nvec + p.splits - 1) / p.splits;
        vb = static_cast<int64_t>(split) * per;
        ve = vb + per;
        if (vb > nvec) vb = nvec;
        if (ve > nvec) ve = nvec;
    }

    // The target logit is read directly (the reference captures it inside the
    // scan, csrc/fused_logprob.cu:180,185, leaving 0 for an out-of-range
    // target).  Issued before the scan so that its latency hides behind it.
    // With split rows the piece that scans the target's element reads it
    // (split 0 owns the scalar head and tail).
    float x_target = 0.0f;
    if (tid == 0) {
        const int64_t tgt = p.targets[row] - p.target_offset;
        if (tgt >= 0 && tgt < vocab) {
            bool mine = true;
            if (kSplit) {
                const int64_t owner =
                    (tgt < head || tgt >= tail_begin) ? 0 : ((tgt - head) / EPV) / per;
                mine = (owner == split);
            }
            if (mine) x_target = to_f32<DT>(rp[tgt]) * p.scale;
        }
    }

    Stat s = stat_empty();
    scan_row_piece<DT, false, U, NTHREADS, kScaled>(s, rp, vp, head, tail_begin, vocab,
                                                    split == 0, vb, ve, tid, p.scale);
    if (needs_clamped_rescan(s)) {
        // This lane met a -inf logit: redo its values with -inf excluded, as
        // the reference's sentinel rule does (csrc/fused_logprob.cu:142-143).
        s = stat_empty();
        scan_row_piece<DT, true, U, NTHREADS, kScaled>(s, rp, vp, head, tail_begin, vocab,
                                                       split == 0, vb, ve, tid, p.scale);
    }

    s = wave_reduce_flat(s);
    __shared__ Stat wave_stat[WAVES];
    const int lane = tid & 63;
    const int wave = tid >> 6;
    if (lane == 0) wave_stat[wave] = s;
    __syncthreads();
    // Wave 0 merges the WAVES states as one flat reduction over a DPP row
    // (lane l < WAVES holds state l).
    if (wave != 0) return;
    static_assert(WAVES <= 16, "one DPP row of states");
    const Stat r = row_reduce_flat(lane < WAVES ? wave_stat[lane] : stat_empty());

    if constexpr (kSplit) {
        // This piece's state (x_target is 0 except in the piece that read
        // the target logit), then its arrival.  The state's words are
        // device-scope atomic stores, which write through to the device's
        // coherence point; waiting for them (vmcnt 0) before the increment
        // orders them before the count without the L2 write-back a release
        // fence costs (which, once per workgroup, made grids of a few hundred
        // pieces several times slower).  The piece that counts last acquires
        // (one fence) before it reads the others.
        float4* part = reinterpret_cast<float4*>(p.partials) + row * p.splits;
        unsigned int* counter = p.counters + row;
        unsigned int arrived = 0;
        if (lane == 0) {
            float* slot = reinterpret_cast<float*>(part + split);
            __hip_atomic_store(slot + 0, r.m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(slot + 1, r.z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(slot + 2, r.t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(slot + 3, x_target, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
            __atomic_signal_fence(__ATOMIC_SEQ_CST);
            arrived = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        }
        arrived = __shfl(arrived, 0);
        if (arrived != static_cast<unsigned int>(p.splits - 1)) return;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        // Last piece of the row: lane k merges pieces k, k + 64, ... in
        // order, the lanes as one flat reduction; the target logit is the
        // sum of the pieces' x_target, all zero but the reader's.
        Stat acc = stat_empty();
        float xt = 0.0f;
        for (int k = lane; k < p.splits; k += 64) {
            const float4 q = part[k];
            acc = combine(acc, Stat{q.x, q.y, q.z});
            xt += q.w;
            float* slot = reinterpret_cast<float*>(part + k);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                __hip_atomic_store(slot + j, 0.0f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        const Stat m = wave_reduce_flat(acc);
        xt = xrow_sum(row_sum16(xt));
        if (lane != 0) return;
        __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const RowOut o = finalize(m, xt);
        p.logprob[row] = o.logp;
        p.entropy[row] = o.ent;
        p.lse[row] = o.lse;
        return;
    }
    if constexpr (kMergeChunks) {
        merge_chunks_final(p, row, r, x_target, lane);
        return;
    }
    if (lane != 0) return;  // thread 0 (it read the target logit)

    if (p.state) {
        // One vocabulary shard: the row's state, merged across shards by
        // klp_fwd_shard_merge_kernel.
        reinterpret_cast<float4*>(p.state)[row] = make_float4(r.m, r.z, r.t, x_target);
        return;
    }
    const RowOut o = finalize(r, x_target);
    p.logprob[row] = o.logp;
    p.entropy[row] = o.ent;
    p.lse[row] = o.lse;
}

template <int DT, int WAVES, int U, bool kSplit, bool kScaled>
__global__ __launch_bounds__(WAVES * 64) void klp_fwd_kernel(FwdParams p) {
    fwd_row<DT, WAVES, U, kSplit, kScaled, false>(p);
}

template <int DT, int WAVES, int U, bool kScaled>
__global__ __launch_bounds__(WAVES * 64) void klp_fwd_chunk_final_kernel(FwdParams p) {
    fwd_row<DT, WAVES, U, false, kScaled, true>(p);
}

// Merge of the row states of `n_shards` vocabulary shards, one thread per row,
// in shard order (the split-row combine across shards): the target logit comes
// from the shard that holds the target.
__global__ __launch_bounds__(256) void klp_fwd_shard_merge_kernel(ShardMergeParams p) {
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (row >= p.n_rows) return;
    const float4* st = reinterpret_cast<const float4*>(p.states);
    Stat acc = stat_empty();
    for (int64_t k = 0; k < p.n_shards; ++k) {
        const float4 q = st[k * p.n_rows + row];
        acc = combine(acc, Stat{q.x, q.y, q.z});
    }
    const int64_t tgt = p.targets[row];
    float x_target = 0.0f;
    if (tgt >= 0 && tgt < p.vocab) x_target = st[(tgt / p.shard_vocab) * p.n_rows + row].w;
    const RowOut o = finalize(acc, x_target);
    p.logprob[row] = o.logp;
    p.entropy[row] = o.ent;
    p.lse[row] = o.lse;
}

// Naive forward: restates the reference's one-thread-per-row recurrence with
// its peeled first element (csrc/fused_logprob.cu:79-112), in base e.
template <int DT>
__global__ __launch_bounds__(128) void klp_fwd_naive_kernel(NaiveParams p) {
    typedef typename Traits<DT>::elem elem;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (row >= p.n_rows) return;
    const elem* rp = static_cast<const elem*>(p.logits) + row_offset(p.rm, row);
    const int64_t tgt = p.targets[row];

    const float x0 = to_f32<DT>(rp[0]);
    float m = x0;
    float z = 1.0f;
    float t = 0.0f;
    float x_target = (tgt == 0) ? x0 : 0.0f;
    for (int64_t v = 1; v < p.vocab; ++v) {
        const float x = to_f32<DT>(rp[v]);
        if (v == tgt) x_target = x;
        const float m_new = fmaxf(m, x);
        const float delta = m - m_new;
        const float scale = expf(delta);
        const float v_new = x - m_new;
        const float e = expf(v_new);
        t = scale * (t + delta * z) + v_new * e;
        z = scale * z + e;
        m = m_new;
    }
    const float lnz = logf(z);
    const float lse = m + lnz;
    p.logprob[row] = x_target - lse;
    p.entropy[row] = lnz - t / z;
    p.lse[row] = lse;
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
template <int DT, int WAVES, int U, bool kScaled>
static hipError_t launch_fwd_t(const FwdParams& p, hipStream_t stream) {
    if (p.merge_states != nullptr)
        return launch_kernel(klp_fwd_chunk_final_kernel<DT, WAVES, U, kScaled>,
                             dim3(static_cast<unsigned>(p.n_rows)), dim3(WAVES * 64), stream, p);
    if (p.splits == 1)
        return launch_kernel(klp_fwd_kernel<DT, WAVES, U, false, kScaled>,
                             dim3(static_cast<unsigned>(p.n_rows)), dim3(WAVES * 64), stream, p);
    return launch_kernel(klp_fwd_kernel<DT, WAVES, U, true, kScaled>,
                         dim3(static_cast<unsigned>(p.n_rows * p.splits)), dim3(WAVES * 64),
                         stream, p);
}

template <int DT>
static hipError_t launch_fwd_dt(const FwdParams& p, const FwdConfig& c, hipStream_t stream) {
    const bool scaled = (p.scale != 1.0f);
#define KLP_FWD_CASE(W, U)                                                     \
    if (c.waves == W && c.unroll == U)                                         \
        return scaled ? launch_fwd_t<DT, W, U, true>(p, stream)                \
                      : launch_fwd_t<DT, W, U, false>(p, stream);
    KLP_FWD_CASE(1, 2)
    KLP_FWD_CASE(1, 4)
    KLP_FWD_CASE(2, 2)
    KLP_FWD_CASE(2, 4)
    KLP_FWD_CASE(4, 2)
    KLP_FWD_CASE(4, 4)
    KLP_FWD_CASE(8, 2)
    KLP_FWD_CASE(8, 4)
    KLP_FWD_CASE(16, 2)
    KLP_FWD_CASE(16, 4)
#undef KLP_FWD_CASE
    return hipErrorInvalidValue;
}

hipError_t launch_shard_merge(const ShardMergeParams& p, hipStream_t stream) {
    return launch_kernel(klp_fwd_shard_merge_kernel,
                         dim3(static_cast<unsigned>((p.n_rows + 255) / 256)), dim3(256), stream, p);
}

hipError_t launch_fwd(int dtype, const FwdParams& p, const FwdConfig& c, hipStream_t stream) {
    switch (dtype) {
        case kBF16: return launch_fwd_dt<kBF16>(p, c, stream);
        case kFP16: return launch_fwd_dt<kFP16>(p, c, stream);
        case kFP32: return launch_fwd_dt<kFP32>(p, c, stream);
        default: return hipErrorInvalidValue;
    }
}

bool fwd_config_supported(const FwdConfig& c) {
    const bool w = (c.waves == 1 || c.waves == 2 || c.waves == 4 || c.waves == 8 ||
                    c.waves == 16);
    const bool u = (c.unroll == 2 || c.unroll == 4);
    return w && u;
}

hipError_t launch_fwd_naive(int dtype, const NaiveParams& p, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>((p.n_rows + 127) / 128));
    switch (dtype) {
        case kBF16: return launch_kernel(klp_fwd_naive_kernel<kBF16>, grid, dim3(128), stream, p);
        case kFP16: return launch_kernel(klp_fwd_naive_kernel<kFP16>, grid, dim3(128), stream, p);
        case kFP32: return launch_kernel(klp_fwd_naive_kernel<kFP32>, grid, dim3(128), stream, p);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace klp
