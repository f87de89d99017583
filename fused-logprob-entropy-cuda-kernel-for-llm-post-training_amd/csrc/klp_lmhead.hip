// klp_lmhead.hip — fused LM head + per-token logprob / entropy (forward, and
// the backward's d_logits), for gfx950.  The reference names this as its
// natural follow-up (a Liger-style fused linear + loss,
// docs/FINAL_REPORT.md:439-450) and does not build it.
//
//   logits[n, v] = scale * sum_k hidden[n, k] * weight[v, k]      (fp32)
//   logprob[n] = logits[n, t_n] - lse[n],  entropy[n], lse[n]  as klp_fwd
//
// without writing the [N, V] logits anywhere.  hidden is bf16 [N, D] and
// weight bf16 [V, D] (nn.Linear's layout), both K-contiguous.
//
// klp_lmh_kernel<false> (forward): one workgroup (4 waves, 2 x 2) per (token block of
// 256, vocab chunk of `tiles_per_chunk` tiles of 256 rows).  Per vocab tile
// it computes the 256 x 256 block of logits^T with v_mfma_f32_32x32x16_bf16,
// each wave a 128 x 128 part of it (16 accumulator blocks, 256 AGPRs):
//  - the transposed orientation puts vocab rows on the MFMA's M side, so a
//    lane's 16 accumulator values all belong to one token (its N column):
//    the online softmax update runs lane-locally, with no cross-lane
//    reduction until the end of the chunk;
//  - K advances in steps of 32 through a ring of 5 LDS stages (32 KB each,
//    all 160 KB of LDS), filled by direct global -> LDS copies
//    (global_load_lds_dwordx4, no register staging) 3-4 stages ahead of the
//    multiply; a slot is refilled once every wave is past the MFMAs of the
//    stage it held; the ring runs across tile boundaries;
//  - LDS rows are 64 bytes; the 16-byte chunk index is XOR-swizzled with
//    row bits 0..3 (swz_f) so that the MFMA operand reads are free of bank
//    conflicts;
//  - a stage's operands are read in two 16-column halves, ping-ponged: the
//    MFMAs of one half run while the other half is read from LDS (the next
//    stage's first half under the current stage's second), one barrier per
//    stage between the halves;
//  - after each tile the block's logits are folded into per-lane
//    (m, z, t) states (absorb() of klp_device.h) and the target logit is
//    captured if it lies in the tile.
// At the end of the chunk, lanes l and l+32 (same token) and the two waves
// of a token half merge; the chunk's partial state per token goes to the
// workspace.  klp_lmh_combine_kernel merges the chunks of each token (one
// wave per token, a fixed order) and applies the output formulas.
//
// klp_lmh_kernel<true> (backward) runs the same tiles and replaces the fold
// with the gradient of klp_bwd, written to d_logits as bf16.
//
// Workgroup order: workgroup b runs on XCD b % 8 (round-robin dispatch).
// Consecutive workgroups of one XCD take the token blocks of one vocab
// chunk, so the chunk's weight rows are fetched from HBM once per XCD and
// shared through its L2 by the token blocks running there together.
#include "klp_launch.h"

namespace klp {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kVB = 4;              // 32-row vocab blocks per wave
constexpr int kTB = 4;              // 32-token blocks per wave
constexpr int kBV = 2 * kVB * 32;   // vocab rows per tile (2 waves along vocab): 256
constexpr int kBT = 2 * kTB * 32;   // tokens per block (2 waves along tokens): 256
// K per LDS stage and LDS stages in the ring.  Measured: 64-wide stages (whole
// 128-byte lines per row, a ring of 2) and non-temporal / sc0 copies were no
// faster.
constexpr int kBK = 32;
constexpr int kRing = 5;
constexpr int kThreads = 256;
constexpr int kRowBytes = kBK * 2;
constexpr int kChunksPerRow = kRowBytes / 16;
constexpr int kWBytes = kBV * kRowBytes;
constexpr int kStageBytes = (kBV + kBT) * kRowBytes;
// One global_load_lds_dwordx4 moves 64 lanes x 16 B = 1 KB of LDS rows.
constexpr int kRowsPerCopy = 1024 / kRowBytes;
constexpr int kWCopies = kBV / kRowsPerCopy / (kThreads / 64);    // per wave per stage
constexpr int kHCopies = kBT / kRowsPerCopy / (kThreads / 64);
constexpr int kCopiesPerStage = kWCopies + kHCopies;              // vmcnt units per stage
static_assert(kRing * kStageBytes <= 160 * 1024, "LDS holds 160 KB");
static_assert(kCopiesPerStage * (kRing - 2) <= 63, "vmcnt counts up to 63");

// LDS byte offset of 16-byte chunk `c` of row `row`.  The chunk index is
// XOR-swizzled with f(row) (bits 0..3 of the row only): the MFMA operand
// reads (one chunk of 16 consecutive rows per pass) are then free of bank
// conflicts whether the LDS serves 8 or 16 lanes x 16 B per cycle.
__device__ __forceinline__ int swz_f(int row) {
    if constexpr (kChunksPerRow == 4) return ((row >> 1) & 3) ^ ((row >> 3) & 1);
    else return (row & 7) ^ ((row >> 3) & 1);
}
__device__ __forceinline__ int swz(int row, int c) {
    return row * kRowBytes + ((c ^ swz_f(row)) << 4);
}

// s_waitcnt with vmcnt = n (0..63) and no wait on the other counters.
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Wait until at most min(N, ahead) stages of copies issued after the
// current one are outstanding (vmcnt takes an immediate, hence the chain).
template <int N>
__device__ __forceinline__ void wait_stages(int ahead) {
    if constexpr (N > 0) {
        if (ahead >= N) {
            __builtin_amdgcn_s_waitcnt(waitcnt_vm(N * kCopiesPerStage));
            return;
        }
        wait_stages<N - 1>(ahead);
    } else {
        __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    }
}

}  // namespace

// kGrad == false: the forward (partial states per vocab chunk).
// kGrad == true: the backward's d_logits: the same logits tiles, turned into
// the gradient of klp_bwd (grad_one, klp_device.h) and written as bf16.
template <bool kGrad>
__global__ __launch_bounds__(kThreads) void klp_lmh_kernel(LmhParams p) {
    // The ring takes all 160 KB of LDS; the end-of-chunk merge reuses it.
    __shared__ __attribute__((aligned(1024))) unsigned char lds[kRing * kStageBytes];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wv = wave & 1;   // vocab half (128 rows) of the tile
    const int wt = wave >> 1;  // token half (128 tokens) of the block

    // Workgroup -> (token block, vocab chunk), XCD-aware (see above).
    const int64_t bid = blockIdx.x;
    const int64_t xcd = bid % 8;
    const int64_t local = bid / 8;
    const int64_t tb = local % p.n_tblocks;
    const int64_t chunk = (local / p.n_tblocks) * 8 + xcd;
    if (chunk >= p.n_chunks) return;  // padding workgroups of the last round

    const int64_t tok0 = tb * kBT;
    const int n_ksteps = static_cast<int>(p.dim / kBK);
    const int64_t tile_first = chunk * p.tiles_per_chunk;
    int64_t tile_end = tile_first + p.tiles_per_chunk;
    if (tile_end > p.n_vtiles) tile_end = p.n_vtiles;
    const int n_stages = static_cast<int>(tile_end - tile_first) * n_ksteps;

    // Copy slots.  Copy q of the W part covers tile rows q * kRowsPerCopy ..
    // + kRowsPerCopy - 1; this wave issues q = wave + 4j.  Lane l fills LDS
    // row q * kRowsPerCopy + l / kChunksPerRow, chunk l % kChunksPerRow, which
    // holds global chunk (l % kChunksPerRow) ^ swz_f(row) of that row (swz_f
    // reads row bits 0..3, the same for every j).  Rows past the end of the
    // matrix are clamped to its last row (valid memory; their logits are
    // masked or their outputs never written).
    const int lrow = lane / kChunksPerRow;
    const int gchunk = (lane % kChunksPerRow) ^ swz_f(wave * kRowsPerCopy + lrow);
    const uint16_t* hsrc[kHCopies];
#pragma unroll
    for (int j = 0; j < kHCopies; ++j) {
        int64_t n = tok0 + (wave + 4 * j) * kRowsPerCopy + lrow;
        if (n > p.n_tokens - 1) n = p.n_tokens - 1;
        hsrc[j] = p.hidden + n * p.ld_hidden + gchunk * 8;
    }

    Stat st[kTB];
    float xt[kTB];
    int64_t my_tgt[kTB];
    RowGrad rg[kTB];
#pragma unroll
    for (int j = 0; j < kTB; ++j) {
        st[j] = stat_empty();
        xt[j] = 0.0f;
        const int64_t tok = tok0 + wt * (kTB * 32) + j * 32 + (lane & 31);
        const bool ok = tok < p.n_tokens;
        my_tgt[j] = ok ? p.targets[tok] : -1;
        if constexpr (kGrad) {
            rg[j] = ok ? row_grad(p.saved_lse[tok], p.saved_entropy[tok],
                                  p.g_logp ? p.g_logp[tok] : 0.0f,
                                  p.g_ent ? p.g_ent[tok] : 0.0f, p.g_lse ? p.g_lse[tok] : 0.0f)
                       : row_grad(0.0f, 0.0f, 0.0f, 0.0f, 0.0f);
        }
    }

    // Copies.  Stages run across the chunk's tiles: global stage g is tile
    // tile_first + g / n_ksteps, K step g % n_ksteps, in ring slot g % kRing.
    // `issued` stages have been issued; the W sources of the tile being issued
    // are set once per tile and advanced by kBK columns per stage.
    int64_t iss_vt = tile_first;
    int iss_k = 0;
    int issued = 0;
    const uint16_t* wsrc[kWCopies];
    auto point_w = [&]() {
#pragma unroll
        for (int j = 0; j < kWCopies; ++j) {
            int64_t v = iss_vt * kBV + (wave + 4 * j) * kRowsPerCopy + lrow;
            if (v > p.vocab - 1) v = p.vocab - 1;
            wsrc[j] = p.weight + v * p.ld_weight + gchunk * 8;
        }
    };
    point_w();
    // Issue stages up to (not including) `limit`.  A slot may be refilled
    // once every wave is past the MFMAs of the stage it held: the callers
    // pass limit = h + 1 + kRing right after a barrier that follows stage h's
    // MFMAs (the operands of stage h + 1 may still be in flight from LDS, so
    // its slot stays untouched).
    auto issue_upto = [&](int limit) {
        if (limit > n_stages) limit = n_stages;
        while (issued < limit) {
            unsigned char* dst = lds + (issued % kRing) * kStageBytes;
            const int64_t koff = static_cast<int64_t>(iss_k) * kBK;
#pragma unroll
            for (int j = 0; j < kWCopies; ++j)
                __builtin_amdgcn_global_load_lds(wsrc[j] + koff, dst + (wave + 4 * j) * 1024, 16,
                                                 0, 0);
#pragma unroll
            for (int j = 0; j < kHCopies; ++j)
                __builtin_amdgcn_global_load_lds(hsrc[j] + koff,
                                                 dst + kWBytes + (wave + 4 * j) * 1024, 16, 0, 0);
            ++issued;
            if (++iss_k == n_ksteps) {
                iss_k = 0;
                ++iss_vt;
                point_w();
            }
        }
    };

    // Operands in two halves of the stage's K (16 columns each, one MFMA K
    // step), ping-ponged: the MFMAs of one half run while the other half's
    // operands are read from LDS.  Half 0 of the next stage is read under
    // half 1's MFMAs, so a stage's first MFMAs find their operands in
    // registers.  Two halves take the registers one whole stage did.
    static_assert(kBK == 32, "two 16-column halves per stage");
    bf16x8 ah[2][kVB], bh[2][kTB];
    auto read_half = [&](auto half_tag, int stage) {
        constexpr int H = decltype(half_tag)::value;
        const unsigned char* wl = lds + (stage % kRing) * kStageBytes;
        const unsigned char* hl = wl + kWBytes;
        const int c = H * 2 + (lane >> 5);
#pragma unroll
        for (int a = 0; a < kVB; ++a)
            ah[H][a] = *reinterpret_cast<const bf16x8*>(
                wl + swz(wv * (kVB * 32) + a * 32 + (lane & 31), c));
#pragma unroll
        for (int b = 0; b < kTB; ++b)
            bh[H][b] = *reinterpret_cast<const bf16x8*>(
                hl + swz(wt * (kTB * 32) + b * 32 + (lane & 31), c));
    };
    // Wait until stage `stage` has landed for this wave (at most the stages
    // issued after it outstanding, up to kRing - 2 of them), then the barrier
    // makes every wave's copies of it visible.
    auto sync_stage = [&](int stage) {
        wait_stages<kRing - 2>(issued - 1 - stage);
        __builtin_amdgcn_s_barrier();
    };
    constexpr int kReadsPerHalf = kVB + kTB;
    constexpr int kMfmaPerHalf = kVB * kTB;

    issue_upto(kRing);  // prologue: every slot is free
    int g = 0;          // global stage index, runs across tiles
    for (int64_t vt = tile_first; vt < tile_end; ++vt) {
        f32x16 acc[kVB][kTB];
#pragma unroll
        for (int a = 0; a < kVB; ++a)
#pragma unroll
            for (int b = 0; b < kTB; ++b)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;

        auto mfma_half = [&](auto half_tag) {
            constexpr int H = decltype(half_tag)::value;
#pragma unroll
            for (int a = 0; a < kVB; ++a)
#pragma unroll
                for (int b = 0; b < kTB; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[H][a], bh[H][b],
                                                                        acc[a][b], 0, 0, 0);
        };
        // One read per MFMA for the first kReadsPerHalf MFMAs, then the rest.
        auto interleave = [&]() {
#pragma unroll
            for (int i = 0; i < kReadsPerHalf; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one DS read
            }
            __builtin_amdgcn_sched_group_barrier(0x008, kMfmaPerHalf - kReadsPerHalf, 0);
        };
        using Half0 = std::integral_constant<int, 0>;
        using Half1 = std::integral_constant<int, 1>;
        // Stage g: half 0's MFMAs under half 1's reads; then, when stage g + 1
        // belongs to this tile, sync on it, top up the ring and read its half
        // 0 under half 1's MFMAs.
        auto step = [&](auto prefetch_tag) {
            constexpr bool kPrefetch = decltype(prefetch_tag)::value;
            read_half(Half1{}, g);
            mfma_half(Half0{});
            interleave();
            if constexpr (kPrefetch) {
                sync_stage(g + 1);
                // Stage g - 1's operand reads all completed before its MFMAs,
                // which are behind this barrier; stage g's may still be in flight.
                issue_upto(g + kRing);
                read_half(Half0{}, g + 1);
            }
            mfma_half(Half1{});
            if constexpr (kPrefetch) interleave();
            ++g;
        };

        // The tile's first stage: its half 0.
        sync_stage(g);
        issue_upto(g + kRing);  // stage g - 1's MFMAs are behind the barrier
        read_half(Half0{}, g);
        for (int kk = 0; kk + 1 < n_ksteps; ++kk) step(std::true_type{});
        // The tile's last stage reads nothing ahead: the pipeline drains at
        // the tile's end, so no operands are live across the epilogue.
        step(std::false_type{});

        const int64_t v0 = vt * kBV;
        if constexpr (kGrad) {
            // d_logits of the tile: accumulator r of block (a, b) holds tile
            // row wv*128 + a*32 + 8*(r/4) + 4*(lane/32) + r%4 of token column
            // b*32 + lane%32; rows 4q .. 4q + 3 go out as one 8-byte store.
            const int lrow0 = wv * (kVB * 32) + 4 * (lane >> 5);
#pragma unroll
            for (int b = 0; b < kTB; ++b) {
                const int64_t tok = tok0 + wt * (kTB * 32) + b * 32 + (lane & 31);
                if (tok >= p.n_tokens) continue;
                uint16_t* drow = p.d_logits + tok * p.ld_d;
#pragma unroll
                for (int a = 0; a < kVB; ++a) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int64_t vq = v0 + lrow0 + a * 32 + 8 * q;
                        if (vq >= p.vocab) continue;
                        float d[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            float g = grad_one(acc[a][b][4 * q + i] * p.scale, rg[b]);
                            if (vq + i == my_tgt[b]) g += rg[b].g_logp;
                            if (vq + i >= p.vocab) g = 0.0f;
                            d[i] = g * p.scale;
                        }
                        const bf16x2 lo = __builtin_convertvector(f32x2{d[0], d[1]}, bf16x2);
                        const bf16x2 hi = __builtin_convertvector(f32x2{d[2], d[3]}, bf16x2);
                        uint2 w;
                        w.x = __builtin_bit_cast(uint32_t, lo);
                        w.y = __builtin_bit_cast(uint32_t, hi);
                        *reinterpret_cast<uint2*>(drow + vq) = w;
                    }
                }
            }
            continue;
        }

        // Tile done: fold it into the lane's token states, one 32-row block
        // at a time.  Accumulator r of block (a, b) holds tile row
        // wv*128 + a*32 + 8*(r/4) + 4*(lane/32) + r%4 (vocab row v0 + that).
        const int64_t vlim64 = p.vocab - v0;
        const int vlim = vlim64 < kBV ? static_cast<int>(vlim64) : kBV;
        const int lrow0 = wv * (kVB * 32) + 4 * (lane >> 5);
#pragma unroll
        for (int b = 0; b < kTB; ++b) {
            const int64_t trel64 = my_tgt[b] - v0;
            const int trel = (trel64 >= 0 && trel64 < kBV) ? static_cast<int>(trel64) : -1;
#pragma unroll
            for (int a = 0; a < kVB; ++a) {
                float x[16];
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = lrow0 + a * 32 + 8 * (r / 4) + (r % 4);
                    const float val = acc[a][b][r] * p.scale;
                    x[r] = (row < vlim) ? val : -INFINITY;
                    if (row == trel) xt[b] = val;
                }
                absorb<16, true>(st[b], x);
            }
        }
    }

    if constexpr (kGrad) return;

    // Merge lane l with lane l + 32 (same token, other vocab rows), then the
    // two vocab-half waves of each token half through LDS (the ring's memory:
    // every wave is past its last read of it once all reach the barrier).
    __syncthreads();
    Stat (*merge_stat)[kBT] = reinterpret_cast<Stat (*)[kBT]>(lds);
    float (*merge_xt)[kBT] = reinterpret_cast<float (*)[kBT]>(lds + 2 * kBT * sizeof(Stat));
#pragma unroll
    for (int b = 0; b < kTB; ++b) {
        Stat o;
        o.m = __shfl_xor(st[b].m, 32, 64);
        o.z = __shfl_xor(st[b].z, 32, 64);
        o.t = __shfl_xor(st[b].t, 32, 64);
        const float oxt = __shfl_xor(xt[b], 32, 64);
        st[b] = (lane < 32) ? combine(st[b], o) : combine(o, st[b]);
        xt[b] += oxt;  // at most one of the two is non-zero
        if (lane < 32) {
            const int col = wt * (kTB * 32) + b * 32 + lane;
            merge_stat[wv][col] = st[b];
            merge_xt[wv][col] = xt[b];
        }
    }
    __syncthreads();
    if (tid < kBT) {
        const int64_t n = tok0 + tid;
        if (n < p.n_tokens) {
            const Stat s = combine(merge_stat[0][tid], merge_stat[1][tid]);
            float4* slot = reinterpret_cast<float4*>(p.partials) + chunk * p.n_tokens + n;
            *slot = make_float4(s.m, s.z, s.t, merge_xt[0][tid] + merge_xt[1][tid]);
        }
    }
}

// One wave per token: lane l merges chunks l, l + 64, l + 128, ... in order,
// the lanes then merge in the fixed xor-butterfly order of wave_reduce (so the
// result does not depend on timing), and lane 0 takes the target logit from
// the chunk that holds the target.
__global__ __launch_bounds__(256) void klp_lmh_combine_kernel(LmhParams p) {
    const int64_t n = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (n >= p.n_tokens) return;
    const float4* part = reinterpret_cast<const float4*>(p.partials);
    Stat acc = stat_empty();
    for (int64_t c = lane; c < p.n_chunks; c += 64) {
        const float4 q = part[c * p.n_tokens + n];
        acc = combine(acc, Stat{q.x, q.y, q.z});
    }
    acc = wave_reduce(acc);
    if (lane != 0) return;
    const int64_t tgt = p.targets[n];
    float x_target = 0.0f;
    if (tgt >= 0 && tgt < p.vocab) {
        const int64_t c = tgt / (static_cast<int64_t>(p.tiles_per_chunk) * kBV);
        x_target = part[c * p.n_tokens + n].w;
    }
    const RowOut o = finalize(acc, x_target);
    p.logprob[n] = o.logp;
    p.entropy[n] = o.ent;
    p.lse[n] = o.lse;
}

int64_t lmh_token_blocks(int64_t n_tokens) { return (n_tokens + kBT - 1) / kBT; }
int64_t lmh_vocab_tiles(int64_t vocab) { return (vocab + kBV - 1) / kBV; }

hipError_t launch_lmh_dlogits(const LmhParams& p, hipStream_t stream) {
    const int64_t chunks8 = (p.n_chunks + 7) / 8 * 8;
    return launch_kernel(klp_lmh_kernel<true>,
                         dim3(static_cast<unsigned>(chunks8 * p.n_tblocks)), dim3(kThreads),
                         stream, p);
}

hipError_t launch_lmh_fwd(const LmhParams& p, hipStream_t stream) {
    // Round the chunk count up to a multiple of 8 (one per XCD per round);
    // padding workgroups exit at once.
    const int64_t chunks8 = (p.n_chunks + 7) / 8 * 8;
    const int64_t blocks = chunks8 * p.n_tblocks;
    hipError_t e = launch_kernel(klp_lmh_kernel<false>, dim3(static_cast<unsigned>(blocks)),
                                 dim3(kThreads), stream, p);
    if (e != hipSuccess) return e;
    return launch_kernel(klp_lmh_combine_kernel,
                         dim3(static_cast<unsigned>((p.n_tokens + 3) / 4)), dim3(256), stream, p);
}

}  // namespace klp
