// attn.h -- the attention of a batch of prompt tokens over the latent cache, a query tile
// at a time (infer.c:1017-1058 for every token of the batch: scores of the absorbed and
// rotated queries against every cached entry up to the token's own position, softmax,
// the softmax-weighted sum of compressed entries).
//
// k_attn_chunk (dense.h) takes one token per block and reads the token's whole cache
// prefix, so a batch of n tokens streams the cache n times and computes on the vector
// ALUs. Here a block takes AQ_T tokens of one head against one chunk of positions: each
// staged cache entry serves the block's AQ_T query rows, and both products run on
// v_mfma_f32_16x16x4_f32 (fp32 operands, fp32 accumulation, like glm.c's own fp32 sums
// up to the order of the additions). The per-chunk maximum, sum of exponentials and
// weighted sum go to the same partial-result slots k_attn_merge reads, so the merge is
// shared with the per-token path.
#pragma once

#include "common.h"
#include "dense.h"

#define AQ_T 64        // query tokens per block (one head): four 16-row MFMA tiles
#define AQ_P 16        // cache positions per staged tile
#define AQ_BLOCK 1024  // sixteen waves, four per SIMD
#define AQ_KQ_MAX 576  // widest staged entry (kv + rope)
#define AQ_STAGES 3    // staged tiles: two in flight while one is used
#define AQ_BLOCKS_PER_CU 3  // blocks per CU the position chunks aim at (one block fits a CU at a time; with
                            // k_attn_tile16's longest-first order, 3 beat 5 by ~1 %: fewer partial results)
#define AQ_SLOTS (AQ_P * (AQ_KQ_MAX / 4 + 1) + 64)  // 16-byte slots of a stage (one wave's DMA past the rows)

typedef float aq_f4 __attribute__((ext_vector_type(4)));

struct AttnTileArgs {
    AttnArgs a;  // a.pos = the batch's first position, a.nblk = chunks per token
    int n;       // tokens in the batch
    int chunk;   // positions per chunk
};

// 16-byte DMA rounds (AQ_BLOCK slots each) of a staged tile: AQ_P rows of kq/4 + 1 slots
// (one slot of padding makes the row stride odd in 16-byte units, so the rows' reads
// spread over the banks).
__host__ __device__ constexpr int aq_rounds(int kq) { return (AQ_P * (kq / 4 + 1) + AQ_BLOCK - 1) / AQ_BLOCK; }

__device__ static inline aq_f4 aq_mfma(float a, float b, aq_f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Block (chunk c, query tile, head h): tokens t0 .. t0 + AQ_T of the batch (at positions
// pos + t) against positions [c chunk, (c + 1) chunk) that any of them attends. Waves:
// the scores of a 16-position tile are split by 16-row quarter (w / 4) and by quarter of
// the entry's 16-column groups (w % 4), the four column quarters summed in shared memory;
// the weighted sum's 16x16 output blocks (four row quarters x kv / 16 column blocks) go
// round robin over the sixteen waves. Staging: a tile is NR rounds of 16-byte DMAs (a
// wave whose slots of the last round lie past the tile's skips it), not tracked by the
// compiler, so each wait is an exact count per wave: the tile before the last is waited
// for with one tile's DMAs still in flight.
template <int NR>
__global__ __launch_bounds__(AQ_BLOCK) void k_attn_tile(AttnTileArgs g) {
    __shared__ __align__(16) float ks[AQ_STAGES][AQ_SLOTS * 4];
    __shared__ __align__(16) float sp[4][AQ_T][AQ_P + 4];  // the column quarters' partial scores
    __shared__ __align__(16) float ps[AQ_T][AQ_P + 4];     // exponentials (rows padded: 5 slots)
    __shared__ float run_m[AQ_T], run_l[AQ_T], corr[AQ_T];
    const AttnArgs &a = g.a;
    const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, lg = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = blockIdx.x, t0 = AQ_T * blockIdx.y, h = blockIdx.z;
    const int kv = a.kv, rope = a.rope, KQ = kv + rope, H = a.H, nch = a.nblk;
    const int tl = min(g.n, t0 + AQ_T);    // the tile's tokens t0 .. tl - 1
    const int r0 = c * g.chunk;
    const int r1 = min(r0 + g.chunk, a.pos + tl);  // the chunk's positions any of them attends
    auto slot = [&](int t) { return ((size_t)t * nch + c) * H + h; };  // partial-result slot of token t
    if (r0 >= r1) {
        // no position here for any of the tile's tokens: empty partials, which the merge
        // weights by zero (it reads this chunk for tokens whose chunk count exceeds c)
        for (int i = tid; i < (tl - t0) * kv; i += AQ_BLOCK) a.part_ctx[slot(t0 + i / kv) * kv + i % kv] = 0.0f;
        if (tid < tl - t0) {
            a.part_ml[slot(t0 + tid) * 2] = -INFINITY;
            a.part_ml[slot(t0 + tid) * 2 + 1] = 0.0f;
        }
        return;
    }
    const int ksd4 = KQ / 4 + 1;  // 16-byte slots per staged row
    const int nslot = AQ_P * ksd4;
    const int ntile = (r1 - r0 + AQ_P - 1) / AQ_P;
    const bool last_round = AQ_BLOCK * (NR - 1) + 64 * w < nslot;  // the wave takes part in round NR - 1

    // the thread's DMA slots: round r writes slot AQ_BLOCK r + 64 w + lane = (row n, 16-byte
    // column d / 4), packed as n << 20 | (d in the rope part) << 19 | the part's column
    unsigned src[NR];
#pragma unroll
    for (int r = 0; r < NR; r++) {
        const int sl = AQ_BLOCK * r + 64 * w + lane, n = sl / ksd4, d = 4 * (sl % ksd4);
        const unsigned row = n < AQ_P ? n : 0;  // slots past the tile's rows load row 0 into the tail
        src[r] = d < kv ? row << 20 | (unsigned)d : d < KQ ? row << 20 | 1u << 19 | (unsigned)(d - kv) : row << 20;
    }
    auto issue = [&](int stage, int s0) {
#pragma unroll
        for (int r = 0; r < NR; r++) {
            if (r + 1 < NR || last_round) {
                // (opaque here, so that the addresses are formed per request rather than
                // hoisted out of the tile loop as 64-bit values that do not fit the registers)
                asm volatile("" : "+v"(src[r]));
                const int s = min(s0 + (int)(src[r] >> 20), r1 - 1);  // positions past the chunk: any entry (masked)
                const bool pe = (src[r] >> 19) & 1;
                const float *p = (pe ? a.pe + (size_t)s * rope : a.comp + (size_t)s * kv) + (src[r] & 0x7ffffu);
                dma16_untracked(gbl((const void *)p), (lds_void *)&ks[stage][4 * (AQ_BLOCK * r + 64 * w)]);
            }
        }
    };

    // the lane's query values for the scores: row 16 rb + l16, the column quarter's groups
    const int rb = w >> 2, q = w & 3, nu = KQ / 16;
    const int tq = min(t0 + 16 * rb + l16, g.n - 1);  // rows past the batch: any token (masked)
    constexpr int NQ = (AQ_KQ_MAX / 16 + 3) / 4;
    aq_f4 qa[NQ];
    {
        const float *qsrc = a.q_abs + ((size_t)tq * H + h) * kv, *psrc = a.q_pe + ((size_t)tq * H + h) * rope;
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            const int u = q + 4 * i, d = 16 * u + 4 * lg;
            const aq_f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
            qa[i] = u >= nu ? zero : d < kv ? *(const aq_f4 *)(qsrc + d) : *(const aq_f4 *)(psrc + d - kv);
        }
        // the queries are waited for here, once: inside the tile loop a pending load from
        // before the loop would make the compiler wait for every load at each iteration
#pragma unroll
        for (int i = 0; i < NQ; i++) asm volatile("" ::"v"(qa[i]));
    }
    if (tid < AQ_T) {
        run_m[tid] = -INFINITY;
        run_l[tid] = 0.0f;
    }
    issue(0, r0);
    if (ntile > 1) issue(1, r0 + AQ_P);

    aq_f4 acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = (aq_f4){0.0f, 0.0f, 0.0f, 0.0f};

    for (int j = 0; j < ntile; j++) {
        const int s0 = r0 + AQ_P * j;
        const float *kt = ks[j % AQ_STAGES];
        if (j + 1 < ntile) {
            if (last_round)
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NR) : "memory");
            else
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NR - 1) : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        // tile j is in shared memory (every wave's part), and every wave is done with tile
        // j - 1, whose stage the request below refills
        __syncthreads();
        if (j + 2 < ntile) issue((j + 2) % AQ_STAGES, s0 + 2 * AQ_P);
        {
            // partial scores: lane holds rows 16 rb + 4 lg + r, position l16; MFMA k index
            // (lane group lg) = column 16 u + 4 lg + e of the entry
            aq_f4 d = {0.0f, 0.0f, 0.0f, 0.0f};
            const float *kr = kt + 4 * ksd4 * l16 + 4 * lg;
#pragma unroll
            for (int i = 0; i < NQ; i++) {
                const int u = q + 4 * i;
                if (u < nu) {
                    const aq_f4 kb = *(const aq_f4 *)(kr + 16 * u);
                    d = aq_mfma(qa[i].x, kb.x, d);
                    d = aq_mfma(qa[i].y, kb.y, d);
                    d = aq_mfma(qa[i].z, kb.z, d);
                    d = aq_mfma(qa[i].w, kb.w, d);
                }
            }
#pragma unroll
            for (int r = 0; r < 4; r++) sp[q][16 * rb + 4 * lg + r][l16] = d[r];
        }
        __syncthreads();
        {
            // softmax step: thread = (row tid / 16, position tid % 16), a 16-lane DPP row per row
            const int row = tid >> 4, p = tid & 15, t = t0 + row, s = s0 + p;
            float v = (sp[0][row][p] + sp[1][row][p]) + (sp[2][row][p] + sp[3][row][p]);
            v = __fmul_rn(v, a.kq_scale);
            if (t >= tl || s >= r1 || s > a.pos + t) v = -INFINITY;  // causal, and past the chunk
            const float mo = run_m[row], mn = fmaxf(mo, row_max_dpp_f(v));
            const float e = mn == -INFINITY ? 0.0f : expf(__fsub_rn(v, mn));
            const float l = row_sum_dpp_f(e);
            ps[row][p] = e;
            if (p == 0) {
                const float cr = mn == -INFINITY ? 1.0f : expf(__fsub_rn(mo, mn));  // 0 while mo is -inf
                run_m[row] = mn;
                run_l[row] = fmaf(run_l[row], cr, l);
                corr[row] = cr;
            }
        }
        __syncthreads();
        // weighted sum: the wave's blocks are row quarter w % 4 and column blocks w / 4 + 4 i
        // (16 columns each); MFMA k index (lane group lg) = position 4 lg + e of the tile
        {
            const int rh = w & 3;
            aq_f4 cr;
#pragma unroll
            for (int r = 0; r < 4; r++) cr[r] = corr[16 * rh + 4 * lg + r];
            const aq_f4 pa = *(const aq_f4 *)&ps[16 * rh + l16][4 * lg];
            const float *vr = kt + 4 * ksd4 * (4 * lg) + 16 * (w >> 2) + l16;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                if ((w >> 2) + 4 * i < kv / 16) {
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[i][r] = __fmul_rn(acc[i][r], cr[r]);
                    const float *v = vr + 64 * i;
                    acc[i] = aq_mfma(pa.x, v[0], acc[i]);
                    acc[i] = aq_mfma(pa.y, v[4 * ksd4], acc[i]);
                    acc[i] = aq_mfma(pa.z, v[8 * ksd4], acc[i]);
                    acc[i] = aq_mfma(pa.w, v[12 * ksd4], acc[i]);
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int cb = (w >> 2) + 4 * i;
        if (cb < kv / 16) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int t = t0 + 16 * (w & 3) + 4 * lg + r;
                if (t < tl) a.part_ctx[slot(t) * kv + 16 * cb + l16] = acc[i][r];
            }
        }
    }
    if (tid < tl - t0) {
        a.part_ml[slot(t0 + tid) * 2] = run_m[tid];
        a.part_ml[slot(t0 + tid) * 2 + 1] = run_l[tid];
    }
}
