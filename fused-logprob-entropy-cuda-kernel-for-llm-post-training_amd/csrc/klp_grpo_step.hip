// klp_grpo_step.hip — the GRPO step's logprob forward, loss gradient and
// logprob backward in one pass over the logits, for gfx950.
//
// In a GRPO step the upstream gradient of a token's log-probability depends
// only on that token: d loss / d logp_t = w_t * dl_t(logp_t; old_t, A_t,
// ref_t) with a per-token weight w_t known in advance (mask / normaliser),
// and the entropy is not differentiated.  So once a row's logsumexp is known,
// its d_logits can be written at once (klp_bwd's formula with
// g_logp = w_t * dl_t * c, g_ent = g_lse = 0):
//   d[v] = (onehot(v == t) - p_v) * g_logp          (times 1/T),
// where c (grad_scale) is the upstream gradient the caller will send into
// the loss, declared in advance (1 for loss.backward(); 1 / k when a
// trainer divides the loss by k gradient-accumulation steps), so that the
// backward has nothing left to do.
// The unfused step reads the logits twice (forward, backward) and writes
// d_logits once; here one workgroup of 1024 threads keeps its whole row in
// registers, so the logits are read once: 2 passes of HBM traffic instead
// of 3.  A thread holds up to kGrpoStepMaxVec = 19 16-byte vectors (76 of the
// 128 VGPRs a 1024-thread workgroup allows; 20 spill): 304 KB per row, a
// bf16 row of V <= 155648 or an fp32 row of V <= 77824.
//
// Per workgroup (one row):
//  1. load the row into registers (16-byte buffer loads, non-temporal);
//  2. per-thread online (m, z, t) state (absorb(), as klp_fwd), the wave
//     reduction, and the 16 wave states through LDS, merged by wave 0 with
//     one DPP row reduction;
//  3. logprob, entropy, lse of the row; the GRPO terms of the token
//     (grpo_token_loss, shared with klp_grpo.hip; its inputs read at the
//     start); loss_tok = w_t * loss_t;
//  4. d_logits from the registers (klp_bwd's gradient, which with g_ent = 0
//     is p * (-g_logp) plus the one-hot term), non-temporal 16-byte buffer
//     stores.
// Rows too long for the registers, or whose start or length is not a whole
// number of 16-byte vectors, are rejected by the caller (KLP_EINVAL), which
// then runs the unfused kernels.
//
// Two kernels run these steps: klp_grpo_step_kernel, one workgroup per row;
// and, for large bf16 batches of long rows when the caller passes a row
// counter, klp_grpo_step_rows_kernel, persistent workgroups that claim rows
// from the counter and load the next row under the current row's pass 2.
// Their outputs are the same bits.
#include "klp_grpo_terms.h"
#include "klp_launch.h"

namespace klp {

namespace {

constexpr int kStepThreads = kGrpoStepThreads;
constexpr int kStepWaves = kStepThreads / 64;
constexpr int kCachePolicyNt = 2;  // the "nt" (non-temporal) cache-policy bit

// Raw buffer resource over one row of `bytes` bytes: lanes past the end read
// 0 without touching memory, and their stores are dropped.  Word 3
// (0x00020000) is the gfx9-family descriptor default for dword data.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0,
                                             static_cast<int>(bytes), 0x00020000);
}

// A 16-byte non-temporal buffer store, then two wait states before the
// wave's next instruction.  A VALU write to the store's data registers in the
// cycles right after a buffer store whose offset is an SGPR reached memory in
// the store's place on gfx950: a pass 2 that reused each stored register at
// once for the next vector's unpack wrote that unpack's first dword instead of
// the gradient's in ~2% of its vectors.  The compiler puts wait states there
// only for a constant offset, so they are written here.
__device__ __forceinline__ void store_vec_nt(u32x4 v, __amdgpu_buffer_rsrc_t rs, uint32_t voff,
                                             uint32_t soff) {
    __builtin_amdgcn_raw_buffer_store_b128(v, rs, voff, soff, kCachePolicyNt);
    asm volatile("s_nop 1");
}

// The token's GRPO inputs.
struct RowInputs {
    int64_t tgt;
    float wt, old_lp, adv, ref_lp;
};

__device__ __forceinline__ RowInputs row_inputs(const GrpoStepParams& p, int64_t row,
                                                bool has_ref) {
    RowInputs in;
    in.tgt = p.targets[row];
    in.wt = p.tok_weight[row];
    in.old_lp = p.old_logp[row];
    in.adv = p.adv[p.adv_per_token ? row : row / p.seq_len];
    in.ref_lp = has_ref ? p.ref_logp[row] : 0.0f;
    return in;
}

// Pass 1 over the registers: the row's online (m, z, t) state.  A lane whose
// own values include -inf redoes its scan with -inf excluded (the reference's
// sentinel rule, csrc/fused_logprob.cu:142-143), as klp_fwd does.  Vector k
// of a thread is the row's vector tid + k * kStepThreads: vectors
// k < n_full exist for every thread, vector n_full only where has_tail.
template <int DT, int NV, bool kScaled>
__device__ __forceinline__ Stat scan_regs(const u32x4 (&r)[NV], int n_full, bool has_tail,
                                          float scale) {
    constexpr int EPV = Traits<DT>::kPerVec;
    constexpr uint32_t pad = Traits<DT>::kNegInfWord;
    auto scan = [&](auto clamp_tag) {
        constexpr bool kClamp = decltype(clamp_tag)::value;
        Stat s = stat_empty();
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            if (k > n_full) break;
            // Vector k's work stays after vector k-1's: hoisting any of it
            // (the select below, say) makes the first wait one for the
            // whole row.
            __builtin_amdgcn_sched_barrier(0);
            float x[EPV];
            // Lanes past the row's end in vector n_full read zeros: -inf.
            unpack<DT>((k < n_full || has_tail) ? r[k] : u32x4{pad, pad, pad, pad}, x);
            if (kScaled) {
#pragma unroll
                for (int j = 0; j < EPV; ++j) x[j] *= scale;
            }
            if (k < n_full) absorb<EPV, kClamp>(s, x);
            else absorb<EPV, true>(s, x);  // padding of the last vector is -inf
        }
        return s;
    };
    Stat s = scan(std::false_type{});
    if (needs_clamped_rescan(s)) s = scan(std::true_type{});
    return s;
}

// The target logit comes from the registers: the thread holding it
// publishes it (a global load issued after the row's loads would make every
// wave wait for the whole row before its scan).
template <int DT, int NV, bool kScaled>
__device__ __forceinline__ void publish_target(const u32x4 (&r)[NV], int64_t tgt, int tid,
                                               float scale, float* target_logit) {
    constexpr int EPV = Traits<DT>::kPerVec;
    const int64_t tv = tgt / EPV;
    if (static_cast<int>(tv % kStepThreads) != tid) return;
    const int kt = static_cast<int>(tv / kStepThreads);
    const int jt = static_cast<int>(tgt - tv * EPV);
    float xt = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        if (k == kt) {
            float x[EPV];
            unpack<DT>(r[k], x);
#pragma unroll
            for (int j = 0; j < EPV; ++j)
                if (j == jt) xt = x[j];
        }
    }
    *target_logit = kScaled ? xt * scale : xt;
}

// LDS of one workgroup.
struct StepShared {
    Stat wave_stat[kStepWaves];
    float target_logit;
    float row_vals[3];  // lse, entropy, g_logp
    int64_t next_row;   // persistent kernel: the workgroup's next row
};

// The row's results: the wave reduction (flat: one maximum, one rescale per
// lane, two sums), the 16 wave states through LDS, merged by wave 0 (each of
// its 16-lane DPP rows reads all of them and reduces them the same way, every
// lane ending with the same bits), which computes the
// row's results and the token's GRPO terms, writes them, and hands the
// backward's constants to the other waves through LDS.  Both barriers are
// here; `s` is this thread's state.  With kPublishNext, thread 0 also
// publishes `next_row` (its claim of the workgroup's next row) between the
// barriers: every wave read the previous one before the first.
template <bool kPublishNext>
__device__ __forceinline__ RowGrad row_results(const GrpoStepParams& p, int64_t row, Stat s,
                                               bool has_t, const RowInputs& in, bool has_ref,
                                               float eps_low, float eps_high, float beta,
                                               int64_t next_row, StepShared& sh) {
    const int lane = threadIdx.x & 63;
    // Uniform in the wave: an SGPR (as a VGPR it is one more register live
    // across the persistent kernel's loop).
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    s = wave_reduce_flat(s);
    if (lane == 0) sh.wave_stat[wave] = s;
    __syncthreads();
    static_assert(kStepWaves == 16, "one wave state per lane of a DPP row");
    if (wave == 0) {
        const RowOut o =
            finalize(row_reduce_flat(sh.wave_stat[lane & 15]), has_t ? sh.target_logit : 0.0f);
        // GRPO terms of this token (token-level importance weight).
        const TokenLoss tl = grpo_token_loss(eps_low, eps_high, beta, o.logp - in.old_lp,
                                             in.adv, o.logp, in.ref_lp, has_ref);
        const float g_logp = in.wt * (tl.dw + tl.dlp) * p.grad_scale;
        if (lane == 0) {
            if (kPublishNext) sh.next_row = next_row;
            sh.row_vals[0] = o.lse;
            sh.row_vals[1] = o.ent;
            sh.row_vals[2] = g_logp;
            p.logprob[row] = o.logp;
            p.entropy[row] = o.ent;
            if (p.lse) p.lse[row] = o.lse;
            p.loss_tok[row] = in.wt * tl.loss;
        }
    }
    __syncthreads();
    return row_grad(sh.row_vals[0], sh.row_vals[1], sh.row_vals[2], 0.0f, 0.0f);
}

// Pass 2 for one vector (the row's vector i): klp_bwd's gradient with
// g_ent = g_lse = 0 (grad_elem_logp_only), plus the one-hot term at the
// target (element t_elem of vector t_vec), times 1/T, packed to the dtype.
template <int DT, bool kScaled>
__device__ __forceinline__ u32x4 grad_vec(u32x4 v, uint32_t i, const RowGrad& g,
                                          uint32_t t_vec, int t_elem, float scale) {
    constexpr int EPV = Traits<DT>::kPerVec;
    float x[EPV];
    unpack<DT>(v, x);
    // fp32 rows: the operand order of klp_bwd's exact argument (the sign of
    // lse), so that the gradient is klp_bwd's bit for bit.
    if (DT != kFP32 || g.lse >= 0.0f) {
#pragma unroll
        for (int j = 0; j < EPV; ++j)
            x[j] = grad_elem_logp_only<DT, true>(kScaled ? x[j] * scale : x[j], g);
    } else {
#pragma unroll
        for (int j = 0; j < EPV; ++j)
            x[j] = grad_elem_logp_only<DT, false>(kScaled ? x[j] * scale : x[j], g);
    }
    if (i == t_vec) {
#pragma unroll
        for (int j = 0; j < EPV; ++j)
            if (j == t_elem) x[j] += g.g_logp;
    }
    if (kScaled) {
#pragma unroll
        for (int j = 0; j < EPV; ++j) x[j] *= scale;
    }
    return pack<DT>(x);
}

}  // namespace

// One workgroup per row.
template <int DT, int NV, bool kScaled>
__global__ __launch_bounds__(kStepThreads) void klp_grpo_step_kernel(GrpoStepParams p) {
    typedef typename Traits<DT>::elem elem;
    constexpr int EPV = Traits<DT>::kPerVec;
    const int tid = threadIdx.x;
    const int64_t row = blockIdx.x;
    const elem* rp = static_cast<const elem*>(p.logits) + row_offset(p.rm, row);
    const uint32_t nvec = static_cast<uint32_t>(p.vocab / EPV);
    const uint32_t row_bytes = nvec * 16u;
    const int n_full = static_cast<int>(nvec / kStepThreads);
    const bool has_tail = static_cast<uint32_t>(tid) < nvec - n_full * kStepThreads;

    // Every load is issued, unconditionally: a load skipped on some path
    // leaves the number of loads in flight unknown, and the compiler then
    // waits for all of them before the first use (no overlap of the scan
    // with the row's arrival).  Past the row's end the buffer descriptor
    // returns zeros without a memory access.  The loads are issued in the
    // order the scan uses them (the scheduling fences keep them so).
    const __amdgpu_buffer_rsrc_t rs = row_rsrc(rp, row_bytes);
    u32x4 r[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        r[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, (tid + k * kStepThreads) * 16, 0,
                                                     kCachePolicyNt);
        __builtin_amdgcn_sched_barrier(0);
    }
    // The token's GRPO inputs, read now: their latency hides behind the
    // row's loads instead of stalling the workgroup after the reduction.
    const bool has_ref = p.ref_logp != nullptr && p.beta != 0.0f;
    const RowInputs in = row_inputs(p, row, has_ref);
    const bool has_t = in.tgt >= 0 && in.tgt < p.vocab;

    const Stat s = scan_regs<DT, NV, kScaled>(r, n_full, has_tail, p.scale);
    __shared__ StepShared sh;
    if (has_t) publish_target<DT, NV, kScaled>(r, in.tgt, tid, p.scale, &sh.target_logit);
    const RowGrad g = row_results<false>(p, row, s, has_t, in, has_ref, p.eps_low, p.eps_high,
                                         p.beta, 0, sh);

    // Pass 2: d_logits from the registers.  Stores past the row's end are
    // dropped by the descriptor.
    const __amdgpu_buffer_rsrc_t ds =
        row_rsrc(static_cast<elem*>(p.d_logits) + row * p.vocab, row_bytes);
    const uint32_t t_vec = has_t ? static_cast<uint32_t>(in.tgt / EPV) : 0xFFFFFFFFu;
    const int t_elem = has_t ? static_cast<int>(in.tgt % EPV) : 0;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const uint32_t i = tid + k * kStepThreads;
        if (k <= n_full)
            store_vec_nt(grad_vec<DT, kScaled>(r[k], i, g, t_vec, t_elem, p.scale), ds, i * 16u,
                         0);
    }
}

// Persistent workgroups (one per CU the kernel fits) that take rows one
// after another, the next row from a counter (StepSched), so that a CU that
// streams faster gets more rows.  Once a row's gradient stores are issued,
// the next row's loads follow at once, into the same registers: the next
// row arrives while the workgroup would otherwise end and a new one start,
// and its scan runs as its vectors arrive.  The stores all go ahead of the
// loads: a CU writes, then reads, in long runs.  Refilling each register
// right after its own store instead (stores and loads alternating) measured
// 7% slower at bf16 [32768, 151936] (3601-3629 against 3339-3361 us), where
// the scan then ran on a row already in registers, with no memory traffic
// from the CU.
//
// The loads of each row are counted, not waited for as a whole: after a
// pass 2 the vector memory operations in flight are, oldest first, the next
// row's GRPO inputs, then stores 0 .. NV-1, then loads 0 .. NV-1; vector k of
// the next scan waits until at most NV - 1 - k of them remain.  The first
// row's loads follow the same pattern (behind NV stores that a zero-length
// descriptor drops), so the compiler's waits at the loop head are those of
// the steady state.
template <int DT, int NV, bool kScaled>
__global__ __launch_bounds__(kStepThreads) void klp_grpo_step_rows_kernel(GrpoStepParams p) {
    typedef typename Traits<DT>::elem elem;
    constexpr int EPV = Traits<DT>::kPerVec;
    const int tid = threadIdx.x;
    const uint32_t nvec = static_cast<uint32_t>(p.vocab / EPV);
    const uint32_t row_bytes = nvec * 16u;
    const uint32_t voff = static_cast<uint32_t>(tid) * 16u;
    const bool has_ref = p.ref_logp != nullptr && p.beta != 0.0f;
    __shared__ StepShared sh;

    // The first rows are rows 0 .. gridDim.x - 1; the counter hands out the
    // rest.  The first row's inputs are read before its logits: in the loop
    // they are vector loads (the loop's stores could alias them, which rules
    // out scalar loads), and the oldest in flight, so waiting for them waits
    // for no logits.
    int64_t row = blockIdx.x;
    RowInputs in = row_inputs(p, row, has_ref);
    __builtin_amdgcn_sched_barrier(0);
    u32x4 r[NV];
    {
        const elem* rp = static_cast<const elem*>(p.logits) + row_offset(p.rm, row);
        const __amdgpu_buffer_rsrc_t rs = row_rsrc(rp, row_bytes);
        const __amdgpu_buffer_rsrc_t none = row_rsrc(p.d_logits, 0u);
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            store_vec_nt(u32x4{0, 0, 0, 0}, none, voff, k * kStepThreads * 16);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            r[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, k * kStepThreads * 16,
                                                         kCachePolicyNt);
            __builtin_amdgcn_sched_barrier(0);
        }
    }

    for (;;) {
        // The row's inputs stay in VGPRs until here: a uniform value read by
        // a vector load is otherwise moved to an SGPR, with a wait, right
        // after its load.
        asm volatile("" : "+v"(in.tgt), "+v"(in.wt), "+v"(in.old_lp), "+v"(in.adv),
                     "+v"(in.ref_lp));
        // Row-length facts, recomputed per row: left loop-invariant, the
        // compiler keeps one lane mask per vector live across the loop and
        // spills.
        uint32_t nvec_o = nvec;
        asm volatile("" : "+s"(nvec_o));
        const int n_full = static_cast<int>(nvec_o / kStepThreads);
        const bool has_tail = static_cast<uint32_t>(tid) < nvec_o - n_full * kStepThreads;
        const bool has_t = in.tgt >= 0 && in.tgt < p.vocab;

        // Claim the row after this one now; the answer is needed after the
        // scan.  The opaque zero offset keeps the atomic out of the
        // compiler's wave-combining rewrite, which would wait for its result
        // (and so for the whole row's loads) at once.
        uint64_t claimed = 0;
        if (tid == 0) {
            uint32_t zero = 0;
            asm volatile("" : "+v"(zero));
            claimed = atomicAdd(&p.sched->next + zero, 1ull);
        }

        const Stat s = scan_regs<DT, NV, kScaled>(r, n_full, has_tail, p.scale);
        // The claim has arrived by now (the scan waited for every load, all
        // issued before it).  Consumed here on every path, it leaves no
        // pending result that a later wait would have to cover, with the
        // output stores in front of it.
        asm volatile("" : "+v"(claimed));
        if (has_t) publish_target<DT, NV, kScaled>(r, in.tgt, tid, p.scale, &sh.target_logit);
        // The clip bounds are recomputed per row rather than kept live (and
        // spilled) across the loop.
        float eps_low = p.eps_low, eps_high = p.eps_high, beta = p.beta;
        asm volatile("" : "+s"(eps_low), "+s"(eps_high), "+s"(beta));
        const RowGrad g = row_results<true>(
            p, row, s, has_t, in, has_ref, eps_low, eps_high, beta,
            static_cast<int64_t>(gridDim.x) + static_cast<int64_t>(claimed), sh);

        // The next row, and its inputs, read before pass 2's stores and
        // loads.  Past the last row the descriptor has length 0 (no memory
        // access).
        const int64_t next = sh.next_row;
        const bool more = next < p.n_rows;
        const int64_t nrow = more ? next : row;
        const RowInputs in_next = row_inputs(p, nrow, has_ref);
        __builtin_amdgcn_sched_barrier(0);
        const __amdgpu_buffer_rsrc_t ns = row_rsrc(
            static_cast<const elem*>(p.logits) + row_offset(p.rm, nrow), more ? row_bytes : 0u);

        // Pass 2: d_logits from the registers, then the next row's loads
        // into them, all issued at once behind the stores.  Every vector is
        // stored and loaded, past the row's end too (the descriptors drop
        // those stores and return zeros for those loads), which keeps the
        // count of operations in flight the same on every path.
        const __amdgpu_buffer_rsrc_t ds =
            row_rsrc(static_cast<elem*>(p.d_logits) + row * p.vocab, row_bytes);
        const uint32_t t_vec = has_t ? static_cast<uint32_t>(in.tgt / EPV) : 0xFFFFFFFFu;
        const int t_elem = has_t ? static_cast<int>(in.tgt % EPV) : 0;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const uint32_t i = tid + k * kStepThreads;
            store_vec_nt(grad_vec<DT, kScaled>(r[k], i, g, t_vec, t_elem, p.scale), ds, voff,
                         k * kStepThreads * 16);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            r[k] = __builtin_amdgcn_raw_buffer_load_b128(ns, voff, k * kStepThreads * 16,
                                                         kCachePolicyNt);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (!more) break;
        row = next;
        in = in_next;
    }
    // Every workgroup's last claim was past the end; the last of them to get
    // there leaves the counter at zero for the next launch.
    if (tid == 0 && atomicAdd(&p.sched->done, 1u) == gridDim.x - 1) {
        atomicExch(&p.sched->next, 0ull);
        atomicExch(&p.sched->done, 0u);
    }
}

// Where the persistent kernel runs (given a counter): rows of 8 or more
// vectors per thread (bf16 and fp16 V > 32768, fp32 V > 16384), from 8 rows
// per workgroup on.  Measured on one box against the one-row-per-workgroup
// kernel (us, same inputs, two runs each):
//   bf16 [32768, 151936]  3339-3342 against 3619-3620
//   bf16 [8192, 128256]    716-762  against 765-774
//   fp16 [8192, 128256]    703-704  against 789-791
//   bf16 [4096, 152064]    434      against 466-467
//   bf16 [4096, 65536]     189-190  against 206-211
//   fp32 [8192, 32000]     337-339  against 354-355
//   bf16 [2048, 152064]    230-234  against 236
//   bf16 [1024, 152064]    123-126  against 124   (4 rows per workgroup)
//   fp32 [256, 32000]       14.5    against 11-12  (1 row per workgroup)
//   bf16 [8192, 32000]     194-200  against 177   (4 vectors per thread: the
//                          one-row kernel fits two workgroups per CU there,
//                          the persistent one one).
constexpr int64_t kPersistMinRowsPerWorkgroup = 8;

template <int DT, int NV>
constexpr bool persistent_pays() {
    return NV >= 8;
}

// Workgroups of the persistent kernel: as many as are resident at once (CUs
// times workgroups per CU), or 0 if that cannot be found.
template <int DT, int NV, bool kScaled>
static int64_t persistent_workgroups() {
    static const int per_cu = [] {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &n, klp_grpo_step_rows_kernel<DT, NV, kScaled>, kStepThreads, 0) != hipSuccess)
            n = 0;
        return n;
    }();
    int dev = 0, cus = 0;
    if (per_cu <= 0 || hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    return static_cast<int64_t>(per_cu) * cus;
}

template <int DT, int NV, bool kScaled>
static int64_t persistent_min_rows() {
    if constexpr (persistent_pays<DT, NV>()) {
        const int64_t wgs = persistent_workgroups<DT, NV, kScaled>();
        return wgs > 0 ? kPersistMinRowsPerWorkgroup * wgs : -1;
    }
    return 0;
}

template <int DT, int NV, bool kScaled>
static hipError_t launch_step(const GrpoStepParams& p, hipStream_t stream) {
    if constexpr (persistent_pays<DT, NV>()) {
        const int64_t wgs = p.sched != nullptr ? persistent_workgroups<DT, NV, kScaled>() : 0;
        if (wgs > 0 && p.n_rows >= kPersistMinRowsPerWorkgroup * wgs)
            return launch_kernel(klp_grpo_step_rows_kernel<DT, NV, kScaled>,
                                 dim3(static_cast<unsigned>(wgs)), dim3(kStepThreads), stream, p);
    }
    return launch_kernel(klp_grpo_step_kernel<DT, NV, kScaled>,
                         dim3(static_cast<unsigned>(p.n_rows)), dim3(kStepThreads), stream, p);
}

template <int DT, int NV>
static hipError_t launch_step_nv(const GrpoStepParams& p, hipStream_t stream) {
    if (p.scale != 1.0f) return launch_step<DT, NV, true>(p, stream);
    return launch_step<DT, NV, false>(p, stream);
}

// The register capacity (16-byte vectors per thread) that rows of `vocab`
// elements take, or 0 for rows too long.
template <int DT>
static int capacity(int64_t vocab) {
    const int64_t nvec = vocab / Traits<DT>::kPerVec;
    const int64_t nv = (nvec + kStepThreads - 1) / kStepThreads;
    for (const int c : {4, 8, 12, 16, kGrpoStepMaxVec})
        if (nv <= c) return c;
    return 0;
}

template <int DT>
static hipError_t launch_step_dt(const GrpoStepParams& p, hipStream_t stream) {
    switch (capacity<DT>(p.vocab)) {
        case 4: return launch_step_nv<DT, 4>(p, stream);
        case 8: return launch_step_nv<DT, 8>(p, stream);
        case 12: return launch_step_nv<DT, 12>(p, stream);
        case 16: return launch_step_nv<DT, 16>(p, stream);
        case kGrpoStepMaxVec: return launch_step_nv<DT, kGrpoStepMaxVec>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

template <int DT, bool kScaled>
static int64_t persistent_min_rows_dt(int64_t vocab) {
    switch (capacity<DT>(vocab)) {
        case 4: return persistent_min_rows<DT, 4, kScaled>();
        case 8: return persistent_min_rows<DT, 8, kScaled>();
        case 12: return persistent_min_rows<DT, 12, kScaled>();
        case 16: return persistent_min_rows<DT, 16, kScaled>();
        case kGrpoStepMaxVec: return persistent_min_rows<DT, kGrpoStepMaxVec, kScaled>();
        default: return 0;
    }
}

template <int DT>
static int64_t persistent_min_rows_dt(int64_t vocab, bool scaled) {
    return scaled ? persistent_min_rows_dt<DT, true>(vocab) : persistent_min_rows_dt<DT, false>(vocab);
}

hipError_t launch_grpo_step(int dtype, const GrpoStepParams& p, hipStream_t stream) {
    switch (dtype) {
        case kBF16: return launch_step_dt<kBF16>(p, stream);
        case kFP16: return launch_step_dt<kFP16>(p, stream);
        case kFP32: return launch_step_dt<kFP32>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

int64_t grpo_step_persistent_min_rows(int dtype, int64_t vocab, bool scaled) {
    if (vocab < 1) return 0;
    switch (dtype) {
        case kBF16: return persistent_min_rows_dt<kBF16>(vocab, scaled);
        case kFP16: return persistent_min_rows_dt<kFP16>(vocab, scaled);
        case kFP32: return persistent_min_rows_dt<kFP32>(vocab, scaled);
        default: return 0;
    }
}

}  // namespace klp
