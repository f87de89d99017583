// klp_lmhead.hip — fused LM head + per-token logprob / entropy (forward),
// for gfx950.  The reference names this as its natural follow-up (a
// Liger-style fused linear + loss, docs/FINAL_REPORT.md:439-450) and does not
// build it.
//
//   logits[n, v] = scale * sum_k hidden[n, k] * weight[v, k]      (fp32)
//   logprob[n] = logits[n, t_n] - lse[n],  entropy[n], lse[n]  as klp_fwd
//
// without writing the [N, V] logits anywhere.  hidden is bf16 [N, D] and
// weight bf16 [V, D] (nn.Linear's layout), both K-contiguous.
//
// klp_lmh_fwd_kernel: one workgroup (4 waves) per (token block of 128,
// vocab chunk of `tiles_per_chunk` tiles of 256 rows).  Per vocab tile it
// computes the 256 x 128 block of logits^T with v_mfma_f32_32x32x16_bf16:
//  - the transposed orientation puts vocab rows on the MFMA's M side, so a
//    lane's 16 accumulator values all belong to one token (its N column):
//    the online softmax update runs lane-locally, with no cross-lane
//    reduction until the end of the chunk;
//  - K advances in steps of 64 through two LDS buffers (48 KB each):
//    global loads for step s+1 are issued into registers before step s is
//    multiplied, and written to the other buffer after it;
//  - LDS rows are 128 bytes; the 16-byte chunk index is XOR-swizzled with
//    the row index so that the MFMA operand reads of 8 consecutive rows hit
//    8 different bank groups;
//  - after each tile the block's logits are folded into per-lane
//    (m, z, t) states (absorb() of klp_device.h) and the target logit is
//    captured if it lies in the tile.
// At the end of the chunk, lanes l and l+32 (same token) and the two waves
// of a token half merge; the chunk's partial state per token goes to the
// workspace.  klp_lmh_combine_kernel merges the chunks of each token in
// chunk order (a fixed order) and applies the output formulas.
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

constexpr int kBV = 256;     // vocab rows per tile
constexpr int kBT = 128;     // tokens per block
constexpr int kBK = 64;      // K per LDS stage
constexpr int kThreads = 256;
constexpr int kRowBytes = kBK * 2;                       // 128
constexpr int kStageBytes = (kBV + kBT) * kRowBytes;     // 48 KB
constexpr int kWChunks = kBV * kRowBytes / 16 / kThreads;  // 16-byte loads per thread: 8
constexpr int kHChunks = kBT * kRowBytes / 16 / kThreads;  // 4

__device__ __forceinline__ int swz(int row, int chunk) {
    return row * kRowBytes + ((chunk ^ (row & 7)) << 4);
}

}  // namespace

__global__ __launch_bounds__(kThreads) void klp_lmh_fwd_kernel(LmhParams p) {
    __shared__ __attribute__((aligned(16))) unsigned char lds[2 * kStageBytes];
    __shared__ Stat merge_stat[2][kBT];
    __shared__ float merge_xt[2][kBT];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wv = wave & 1;   // vocab half (128 rows) of the tile
    const int wt = wave >> 1;  // token half (64 tokens) of the block

    // Workgroup -> (token block, vocab chunk), XCD-aware (see above).
    const int64_t bid = blockIdx.x;
    const int64_t xcd = bid % 8;
    const int64_t local = bid / 8;
    const int64_t tb = local % p.n_tblocks;
    const int64_t chunk = (local / p.n_tblocks) * 8 + xcd;
    if (chunk >= p.n_chunks) return;  // padding workgroups of the last round

    const int64_t tok0 = tb * kBT;
    const int64_t K = p.dim;
    const int n_ksteps = static_cast<int>(K / kBK);

    // This thread's global -> LDS copy slots: 16-byte chunk c of the stage,
    // row c / 8, column chunk c % 8.
    const uint16_t* hbase[kHChunks];
    bool hvalid[kHChunks];
#pragma unroll
    for (int j = 0; j < kHChunks; ++j) {
        const int c = tid + j * kThreads;
        const int64_t n = tok0 + c / 8;
        hvalid[j] = n < p.n_tokens;
        hbase[j] = p.hidden + (hvalid[j] ? n : 0) * p.ld_hidden + (c % 8) * 8;
    }

    // Per-lane states for the lane's two tokens (token block column
    // wt*64 + j*32 + lane%32, j = 0, 1).
    Stat st[2] = {stat_empty(), stat_empty()};
    float xt[2] = {0.0f, 0.0f};
    int64_t my_tok[2], my_tgt[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        my_tok[j] = tok0 + wt * 64 + j * 32 + (lane & 31);
        my_tgt[j] = (my_tok[j] < p.n_tokens) ? p.targets[my_tok[j]] : -1;
    }

    const int64_t tile_first = chunk * p.tiles_per_chunk;
    int64_t tile_end = tile_first + p.tiles_per_chunk;
    if (tile_end > p.n_vtiles) tile_end = p.n_vtiles;

    for (int64_t vt = tile_first; vt < tile_end; ++vt) {
        const int64_t v0 = vt * kBV;
        const uint16_t* wbase[kWChunks];
        bool wvalid[kWChunks];
#pragma unroll
        for (int j = 0; j < kWChunks; ++j) {
            const int c = tid + j * kThreads;
            const int64_t v = v0 + c / 8;
            wvalid[j] = v < p.vocab;
            wbase[j] = p.weight + (wvalid[j] ? v : 0) * p.ld_weight + (c % 8) * 8;
        }

        f32x16 acc[4][2];
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.0f;

        u32x4 wreg[kWChunks], hreg[kHChunks];
        auto gload = [&](int ks) {
            const int64_t koff = static_cast<int64_t>(ks) * kBK;
#pragma unroll
            for (int j = 0; j < kWChunks; ++j)
                wreg[j] = wvalid[j] ? *reinterpret_cast<const u32x4*>(wbase[j] + koff)
                                    : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (int j = 0; j < kHChunks; ++j)
                hreg[j] = hvalid[j] ? *reinterpret_cast<const u32x4*>(hbase[j] + koff)
                                    : u32x4{0u, 0u, 0u, 0u};
        };
        auto lstore = [&](int buf) {
            unsigned char* base = lds + buf * kStageBytes;
#pragma unroll
            for (int j = 0; j < kWChunks; ++j) {
                const int c = tid + j * kThreads;
                *reinterpret_cast<u32x4*>(base + swz(c / 8, c % 8)) = wreg[j];
            }
#pragma unroll
            for (int j = 0; j < kHChunks; ++j) {
                const int c = tid + j * kThreads;
                *reinterpret_cast<u32x4*>(base + kBV * kRowBytes + swz(c / 8, c % 8)) = hreg[j];
            }
        };
        auto compute = [&](int buf) {
            const unsigned char* wl = lds + buf * kStageBytes;
            const unsigned char* hl = wl + kBV * kRowBytes;
#pragma unroll
            for (int ks = 0; ks < kBK / 16; ++ks) {
                const int ch = ks * 2 + (lane >> 5);
                bf16x8 af[4], bfr[2];
#pragma unroll
                for (int a = 0; a < 4; ++a) {
                    const int row = wv * 128 + a * 32 + (lane & 31);
                    af[a] = *reinterpret_cast<const bf16x8*>(wl + swz(row, ch));
                }
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const int row = wt * 64 + b * 32 + (lane & 31);
                    bfr[b] = *reinterpret_cast<const bf16x8*>(hl + swz(row, ch));
                }
#pragma unroll
                for (int a = 0; a < 4; ++a)
#pragma unroll
                    for (int b = 0; b < 2; ++b)
                        acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[a], bfr[b],
                                                                           acc[a][b], 0, 0, 0);
            }
        };

        gload(0);
        lstore(0);
        __syncthreads();
        for (int ks = 0; ks < n_ksteps; ++ks) {
            const int buf = ks & 1;
            if (ks + 1 < n_ksteps) gload(ks + 1);
            compute(buf);
            if (ks + 1 < n_ksteps) lstore(buf ^ 1);
            __syncthreads();
        }

        // Fold the tile into the lane's token states.  Accumulator r of block
        // (a, b) holds vocab row v0 + wv*128 + a*32 + 8*(r/4) + 4*(lane/32) + r%4.
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            float x[64];
#pragma unroll
            for (int a = 0; a < 4; ++a)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int64_t v = v0 + wv * 128 + a * 32 + 8 * (r / 4) + 4 * (lane >> 5) +
                                      (r % 4);
                    const float val = acc[a][b][r] * p.scale;
                    x[a * 16 + r] = (v < p.vocab) ? val : -INFINITY;
                    if (v == my_tgt[b]) xt[b] = val;
                }
            absorb<64, true>(st[b], x);
        }
    }

    // Merge lane l with lane l + 32 (same token, other vocab rows), then the
    // two vocab-half waves of each token half through LDS.
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        Stat o;
        o.m = __shfl_xor(st[b].m, 32, 64);
        o.z = __shfl_xor(st[b].z, 32, 64);
        o.t = __shfl_xor(st[b].t, 32, 64);
        const float oxt = __shfl_xor(xt[b], 32, 64);
        st[b] = (lane < 32) ? combine(st[b], o) : combine(o, st[b]);
        xt[b] += oxt;  // at most one of the two is non-zero
        if (lane < 32) {
            const int col = wt * 64 + b * 32 + lane;
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

// One thread per token: merge the chunks in chunk order, take the target
// logit from the chunk that holds the target.
__global__ __launch_bounds__(256) void klp_lmh_combine_kernel(LmhParams p) {
    const int64_t n = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (n >= p.n_tokens) return;
    const float4* part = reinterpret_cast<const float4*>(p.partials);
    Stat acc = stat_empty();
    for (int64_t c = 0; c < p.n_chunks; ++c) {
        const float4 q = part[c * p.n_tokens + n];
        acc = combine(acc, Stat{q.x, q.y, q.z});
    }
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

hipError_t launch_lmh_fwd(const LmhParams& p, hipStream_t stream) {
    // Round the chunk count up to a multiple of 8 (one per XCD per round);
    // padding workgroups exit at once.
    const int64_t chunks8 = (p.n_chunks + 7) / 8 * 8;
    const int64_t blocks = chunks8 * p.n_tblocks;
    hipError_t e = launch_kernel(klp_lmh_fwd_kernel, dim3(static_cast<unsigned>(blocks)),
                                 dim3(kThreads), stream, p);
    if (e != hipSuccess) return e;
    return launch_kernel(klp_lmh_combine_kernel,
                         dim3(static_cast<unsigned>((p.n_tokens + 255) / 256)), dim3(256),
                         stream, p);
}

}  // namespace klp
