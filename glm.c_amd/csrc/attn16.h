// attn16.h -- the batch attention of attn.h (infer.c:1017-1058) on fp16 matrix cores with
// fp32-like accuracy: k_attn_tile's work split (AQ_T tokens of one head against a chunk
// of positions, AQ_P positions a tile, the same partial-result slots for k_attn_merge),
// with both products on v_mfma_f32_16x16x32_f16 / 16x16x16_f16 over operands split into
// fp16 hi and lo (x = hi + lo to ~22 bits, as the expert GEMMs split their activations):
// a product of two split operands is hi.hi + hi.lo + lo.hi in fp32 (the dropped lo.lo is
// ~2^-22 of it). fp32 MFMA runs at 157 TFLOP/s on MI355X, fp16 at 2.5 PFLOP/s, so the three
// fp16 products cost about a fifth of one fp32 product.
//
// The cache entries come in the split form attn_prep_run writes once per position (dense.h:
// ksp rows scaled by 2^-e[p], vsp blocks of the compressed part transposed), so the 16 query
// tiles x heads that read a position do not each convert it: a tile's rows and its
// transposed block land in shared memory by DMA, two tiles in flight. Each token's query
// row is split once per block, scaled by 2^-eq; a score is the MFMA's sum times 2^(eq + e[p]).
// For the weighted sum the tile's exponentials are scaled by 2^(e[p] - eT), eT the tile's
// largest e over the positions it attends (so the weights stay <= 1); the tile's sum starts
// from zero on the matrix cores and joins the running fp32 sum as acc = acc * corr + sum * 2^eT.
//
// A tile: the scores (waves by 16-row quarter and quarter of the 32-column steps, summed in
// shared memory), the softmax step as in k_attn_tile, and the weighted sum (16x16 output
// blocks round robin over the waves).
#pragma once

#include "attn.h"

#define A16_NKS (AQ_KQ_MAX / 32)  // 32-column steps of the widest entry
#define A16_NQS ((A16_NKS + 3) / 4)  // steps a wave's quarter holds at most
#define A16_PS 20                  // halves a row of the exponentials' planes: 16 + 4, an odd count of 8-byte units
#define A16_KB (AQ_P * SPL_KROW * 2)             // bytes of a stage's rows
#define A16_VB (2 * AT_KV_MAX * 16 * 2)          // bytes of a stage's transposed block at the widest kv
#define A16_STAGE (A16_KB + A16_VB)
// A timing point (k: 0 start, 1 queries ready, then per tile 2 landed, 3 scores, 4 softmax,
// 5 weighted sum); empty unless a timing build defines it.
#ifndef A16_STAMP
#define A16_STAMP(k, j)
#endif
static_assert(AQ_P == 16, "one ksp row a wave's share of the DMA, and a 16-position K dimension for the weighted sum");
static_assert(AQ_BLOCK == 1024 && AQ_T == 64, "16 waves: four 16-row quarters by four column quarters");
static_assert(AQ_KQ_MAX == SPL_KCOLS, "the split rows hold the widest entry");
static_assert(A16_KB % 16 == 0 && A16_STAGE % 16 == 0, "16-byte DMA slots");

typedef _Float16 a16_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 a16_h4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(AQ_BLOCK) void k_attn_tile16(AttnTileArgs g) {
    __shared__ __align__(16) uint8_t stg[2][A16_STAGE];        // tiles j and j + 1: rows, then the block
    __shared__ __align__(16) float sp[4][AQ_T][AQ_P];         // the column quarters' partial scores
    __shared__ __align__(16) _Float16 pp[2][AQ_T * A16_PS];   // the exponentials' hi and lo planes
    __shared__ float run_m[AQ_T], run_l[AQ_T], corr[AQ_T];
    __shared__ int eq_s[AQ_T], et_s;
    const AttnArgs &a = g.a;
    const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, lg = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    // blocks dispatched longest first, so that short ones fill the CUs at the end: chunk by
    // chunk (the earlier chunks are the full ones), and in a chunk the later token tiles
    // (which attend more of its positions) first, the heads of a tile in a row
    const int L = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z), per = gridDim.y * gridDim.z;
    const int c = L / per, t0 = AQ_T * (gridDim.y - 1 - (L % per) / gridDim.z), h = (L % per) % gridDim.z;
    const int kv = a.kv, rope = a.rope, KQ = kv + rope, H = a.H, nch = a.nblk;
    const int tl = min(g.n, t0 + AQ_T);    // the tile's tokens t0 .. tl - 1
    const int r0 = c * g.chunk;
    const int r1 = min(r0 + g.chunk, a.pos + tl);  // the chunk's positions any of them attends
    auto slot = [&](int t) { return ((size_t)t * nch + c) * H + h; };  // partial-result slot of token t
    if (r0 >= r1) {
        for (int i = tid; i < (tl - t0) * kv; i += AQ_BLOCK) a.part_ctx[slot(t0 + i / kv) * kv + i % kv] = 0.0f;
        if (tid < tl - t0) {
            a.part_ml[slot(t0 + tid) * 2] = -INFINITY;
            a.part_ml[slot(t0 + tid) * 2 + 1] = 0.0f;
        }
        return;
    }
    A16_STAMP(0, 0);
    const int nks = (KQ + 31) / 32;   // 32-column steps (ksp holds zeros past KQ)
    const int ntile = (r1 - r0 + AQ_P - 1) / AQ_P;

    // a tile by DMA into stage st: its 16 ksp rows (contiguous), then its vsp block (4 kv
    // 16-byte slots); 64 slots per wave and round, the last round's lanes past the data idle.
    // The wave's count of DMA instructions is the same for every tile (nd below).
    constexpr int NKS = A16_KB / 16;
    const int nvs = 4 * kv;
    const int nd = 2 + (2048 + 64 * w < NKS ? 1 : 0) + (64 * w < nvs ? 1 : 0) + (1024 + 64 * w < nvs ? 1 : 0);
    auto issue = [&](int s0, int st) {
        const uint8_t *ks = reinterpret_cast<const uint8_t *>(a.ksp + (size_t)s0 * SPL_KROW);
        const uint8_t *vs = reinterpret_cast<const uint8_t *>(a.vsp + (size_t)(s0 >> 4) * 2 * kv * 16);
        int ln = lane;
        asm volatile("" : "+v"(ln));  // (addresses formed per request, not hoisted out of the loop)
#pragma unroll
        for (int r = 0; r < 3; r++) {
            const int b0 = 1024 * r + 64 * w;
            if (b0 < NKS && b0 + ln < NKS) dma16_untracked(gbl((const void *)(ks + 16 * (b0 + ln))), (lds_void *)(stg[st] + 16 * b0));
        }
#pragma unroll
        for (int r = 0; r < 2; r++) {
            const int b0 = 1024 * r + 64 * w;
            if (b0 < nvs) dma16_untracked(gbl((const void *)(vs + 16 * (b0 + ln))), (lds_void *)(stg[st] + A16_KB + 16 * b0));
        }
    };
    issue(r0, 0);  // before the queries' loads: the two share a round trip
    if (ntile > 1) issue(r0 + AQ_P, 1);

    // the queries: the lane's operand columns (row 16 rb + l16, steps q + 4 i, columns 32 s +
    // 8 lg .. + 7, each 8-column group inside one part since kv and KQ are multiples of 16)
    // as float4 pairs, all requested at once; the row's exponent from the four waves that
    // hold its column quarters (16 rows x 4 quarters, through shared memory)
    const int rb = w >> 2, q = w & 3;
    float4 qv[A16_NQS][2];
    {
        const int tq = min(t0 + 16 * rb + l16, g.n - 1);  // rows past the batch: any token (masked)
        const float *qa = a.q_abs + ((size_t)tq * H + h) * kv, *qp = a.q_pe + ((size_t)tq * H + h) * rope - kv;
#pragma unroll
        for (int i = 0; i < A16_NQS; i++) {
            const int col = 32 * (q + 4 * i) + 8 * lg;
            const bool on = q + 4 * i < nks && col < KQ;
            const float *src = col < kv ? qa + col : qp + col;
            qv[i][0] = on ? *(const float4 *)src : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            qv[i][1] = on ? *(const float4 *)(src + 4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < A16_NQS; i++)
#pragma unroll
            for (int k = 0; k < 2; k++)
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(qv[i][k].x), fabsf(qv[i][k].y)), fmaxf(fabsf(qv[i][k].z), fabsf(qv[i][k].w))));
        sp[q][16 * rb + l16][lg] = mx;  // the row's maximum over its columns: four lane groups in each of four waves
    }
    if (tid < AQ_T) {
        run_m[tid] = -INFINITY;
        run_l[tid] = 0.0f;
    }
    __syncthreads();
    if (tid < AQ_T) {
        float mx = 0.0f;
#pragma unroll
        for (int qq = 0; qq < 4; qq++)
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) mx = fmaxf(mx, sp[qq][tid][g4]);
        eq_s[tid] = spl_exp(mx);
    }
    __syncthreads();
    a16_h8 qh[A16_NQS], ql[A16_NQS];
    {
        const int e = eq_s[16 * rb + l16];
#pragma unroll
        for (int i = 0; i < A16_NQS; i++) {
            const float xs[8] = {qv[i][0].x, qv[i][0].y, qv[i][0].z, qv[i][0].w, qv[i][1].x, qv[i][1].y, qv[i][1].z, qv[i][1].w};
#pragma unroll
            for (int k = 0; k < 8; k++) {
                _Float16 hi, lo;
                spl_split(ldexpf(xs[k], -e), hi, lo);
                qh[i][k] = hi;
                ql[i][k] = lo;
            }
        }
    }
    int eqd[4];  // the exponents of the score rows the lane holds: tokens 16 rb + 4 lg + r
#pragma unroll
    for (int r = 0; r < 4; r++) eqd[r] = eq_s[16 * rb + 4 * lg + r];
    A16_STAMP(1, 0);


    aq_f4 acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = (aq_f4){0.0f, 0.0f, 0.0f, 0.0f};

    for (int j = 0; j < ntile; j++) {
        const int s0 = r0 + AQ_P * j;
        const uint8_t *sb = stg[j & 1];
        const _Float16 *K = reinterpret_cast<const _Float16 *>(sb), *V = reinterpret_cast<const _Float16 *>(sb + A16_KB);
        // tile j has landed (this wave's DMAs of tile j + 1, issued after, may still be in flight)
        if (j + 1 < ntile) {
            switch (nd) {
            case 2: asm volatile("s_waitcnt vmcnt(2)" ::: "memory"); break;
            case 3: asm volatile("s_waitcnt vmcnt(3)" ::: "memory"); break;
            case 4: asm volatile("s_waitcnt vmcnt(4)" ::: "memory"); break;
            default: asm volatile("s_waitcnt vmcnt(5)" ::: "memory"); break;
            }
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        at_barrier();  // every wave's part of tile j (shared memory only: the next tile's DMA stays in flight)
        A16_STAMP(2, j);
        {
            // partial scores: lane holds rows 16 rb + 4 lg + r, position l16
            aq_f4 d = {0.0f, 0.0f, 0.0f, 0.0f};
            const _Float16 *kr = K + l16 * SPL_KROW + 8 * lg + 32 * q;  // step q + 4 i at + 128 i, lo at + SPL_KCOLS
#pragma unroll
            for (int i = 0; i < A16_NQS; i++) {
                const int s = q + 4 * i;
                if (s < nks) {
                    const a16_h8 bh = *(const a16_h8 *)(kr + 128 * i);
                    const a16_h8 bl = *(const a16_h8 *)(kr + 128 * i + SPL_KCOLS);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[i], bh, d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[i], bl, d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[i], bh, d, 0, 0, 0);
                }
            }
            const int ekp = *(const int *)(K + l16 * SPL_KROW + SPL_KEXP);
#pragma unroll
            for (int r = 0; r < 4; r++) sp[q][16 * rb + 4 * lg + r][l16] = ldexpf(d[r], eqd[r] + ekp);
        }
        at_barrier();
        A16_STAMP(3, j);
        {
            // softmax step: thread = (row tid / 16, position tid % 16), a 16-lane DPP row per row
            const int row = tid >> 4, p = tid & 15, t = t0 + row, s = s0 + p;
            float v = (sp[0][row][p] + sp[1][row][p]) + (sp[2][row][p] + sp[3][row][p]);
            v = __fmul_rn(v, a.kq_scale);
            const bool in = s < r1;
            if (t >= tl || !in || s > a.pos + t) v = -INFINITY;  // causal, and past the chunk
            const float mo = run_m[row], mn = fmaxf(mo, row_max_dpp_f(v));
            const float e = mn == -INFINITY ? 0.0f : expf(__fsub_rn(v, mn));
            const float l = row_sum_dpp_f(e);
            const int ep = *(const int *)(K + p * SPL_KROW + SPL_KEXP);
            const int eT = (int)row_max_dpp_f((float)(in ? ep : SPL_EMPTY));  // the same in every row
            _Float16 hi, lo;
            spl_split(ldexpf(e, ep - eT), hi, lo);
            pp[0][row * A16_PS + p] = hi;
            pp[1][row * A16_PS + p] = lo;
            if (p == 0) {
                const float cr = mn == -INFINITY ? 1.0f : expf(__fsub_rn(mo, mn));  // 0 while mo is -inf
                run_m[row] = mn;
                run_l[row] = fmaf(run_l[row], cr, l);
                corr[row] = cr;
                if (row == 0) et_s = eT;
            }
        }
        at_barrier();
        A16_STAMP(4, j);
        {
            // weighted sum: the wave's blocks are row quarter w % 4 and column blocks w / 4 + 4 i
            const int rh = w & 3;
            aq_f4 cr;
#pragma unroll
            for (int r = 0; r < 4; r++) cr[r] = corr[16 * rh + 4 * lg + r];
            const float sv = ldexpf(1.0f, et_s);
            const a16_h4 ah = *(const a16_h4 *)&pp[0][(16 * rh + l16) * A16_PS + 4 * lg];
            const a16_h4 al = *(const a16_h4 *)&pp[1][(16 * rh + l16) * A16_PS + 4 * lg];
            const _Float16 *vh = V + (16 * (w >> 2) + l16) * 16 + 4 * lg;  // block i at + 1024 i
            const _Float16 *vl = vh + kv * 16;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int cb = (w >> 2) + 4 * i;
                if (cb < kv / 16) {
                    const a16_h4 bh = *(const a16_h4 *)(vh + 1024 * i), bl = *(const a16_h4 *)(vl + 1024 * i);
                    aq_f4 d = {0.0f, 0.0f, 0.0f, 0.0f};
                    d = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bh, d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bl, d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bh, d, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[i][r] = fmaf(d[r], sv, __fmul_rn(acc[i][r], cr[r]));
                }
            }
        }
        at_barrier();  // every wave is done with stage j % 2 and the exponentials' planes
        A16_STAMP(5, j);
        if (j + 2 < ntile) issue(s0 + 2 * AQ_P, j & 1);
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
