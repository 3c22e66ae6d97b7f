// attn16.h -- the batch attention of attn.h (infer.c:1017-1058) on fp16 matrix cores with
// fp32-like accuracy: k_attn_tile's work split (AQ_T tokens of one head against a chunk
// of positions, AQ_P positions a tile, the same partial-result slots for k_attn_merge),
// with both products on v_mfma_f32_16x16x32_f16 / 16x16x16_f16 over operands split into
// fp16 hi and lo (x = hi + lo to ~22 bits, as the expert GEMMs split their activations):
// a product of two split operands is hi.hi + hi.lo + lo.hi in fp32 (the dropped lo.lo is
// ~2^-22 of it). fp32 MFMA runs at 157 TFLOP/s on MI355X, fp16 at 2.5 PFLOP/s, so the three
// fp16 products cost about a fifth of one fp32 product.
//
// fp16's range needs exponents: each token's query row is scaled by 2^-eq (max below
// 2^15) and each staged cache row by 2^-ek (kv and rope parts together, for the scores);
// a score is the MFMA's sum times 2^(eq + ek). For the weighted sum the compressed part
// of row p is scaled by its own 2^-ev[p], and the tile's exponentials by 2^(ev[p] - eV),
// eV the tile's largest ev (so the weights stay <= 1); the tile's sum starts from zero on
// the matrix cores and joins the running fp32 sum as acc = acc * corr + sum * 2^eV.
//
// A tile's rows are loaded to registers (one row a wave, requested while the tile before
// is used), converted to the split planes in shared memory (kp: [position][column] for the
// scores' B operand; vp: [column][position] for the weighted sum's), then: the
// scores (waves by 16-row quarter and quarter of the 32-column steps, summed in shared
// memory), the softmax step as in k_attn_tile, and the weighted sum (16x16 output blocks
// round robin over the waves).
#pragma once

#include "attn.h"

#define A16_KQS 584    // halves a kp row: 576 + 8, an odd count of 16-byte units (the 16 rows' reads miss no bank)
#define A16_VS 20      // halves a vp row: 16 positions + 4, an odd count of 8-byte units
#define A16_PS 20      // halves a pp row (the same)
#define A16_NKS (AQ_KQ_MAX / 32)  // 32-column steps of the widest entry
#define A16_NQS ((A16_NKS + 3) / 4)  // steps a wave's quarter holds at most
#define A16_NJ (AQ_KQ_MAX / 64)   // a row's 64-column groups (one per lane and load)
#define A16_EMPTY (-1000)         // exponent of an all-zero row
// A timing point (k: 0 start, 1 queries ready, then per tile 2 converted, 3 scores, 4 softmax,
// 5 weighted sum); empty unless a timing build defines it.
#ifndef A16_STAMP
#define A16_STAMP(k, j)
#endif
static_assert(AQ_P == 16, "one wave per staged row, and a 16-position K dimension for the weighted sum");
static_assert(AQ_BLOCK == 1024 && AQ_T == 64, "16 waves: four 16-row quarters by four column quarters");

typedef _Float16 a16_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 a16_h4 __attribute__((ext_vector_type(4)));

// The exponent e with |x| 2^-e < 2^15 for every |x| <= mx (A16_EMPTY when mx is 0).
__device__ static inline int a16_exp(float mx) {
    if (!(mx > 0.0f)) return A16_EMPTY;
    int k;
    (void)frexpf(mx, &k);  // mx < 2^k
    return k - 15;
}

// x = hi + lo: hi the nearest fp16, lo the nearest fp16 to the (exact) remainder.
__device__ static inline void a16_split(float x, _Float16 &hi, _Float16 &lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

__global__ __launch_bounds__(AQ_BLOCK) void k_attn_tile16(AttnTileArgs g) {
    // each pair of planes in one array (lo at a fixed offset from hi), so that every read of
    // a product takes one base address and immediate offsets
    __shared__ __align__(16) _Float16 kp[2][AQ_P * A16_KQS];
    __shared__ __align__(16) _Float16 vp[2][AT_KV_MAX * A16_VS];
    __shared__ __align__(16) _Float16 pp[2][AQ_T * A16_PS];
    __shared__ __align__(16) float sp[4][AQ_T][AQ_P + 4];  // the column quarters' partial scores
    __shared__ float run_m[AQ_T], run_l[AQ_T], corr[AQ_T];
    __shared__ int ek_s[AQ_P], ev_s[AQ_P], eq_s[AQ_T], ev_tile;
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
        for (int i = tid; i < (tl - t0) * kv; i += AQ_BLOCK) a.part_ctx[slot(t0 + i / kv) * kv + i % kv] = 0.0f;
        if (tid < tl - t0) {
            a.part_ml[slot(t0 + tid) * 2] = -INFINITY;
            a.part_ml[slot(t0 + tid) * 2 + 1] = 0.0f;
        }
        return;
    }
    A16_STAMP(0, 0);
    const int nks = (KQ + 31) / 32;   // 32-column steps (columns past KQ are zeros)
    const int ncol = 32 * nks;        // columns of the kp planes that the steps read
    const int ntile = (r1 - r0 + AQ_P - 1) / AQ_P;

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
        // the row's maximum over its columns: four lane groups in each of four waves
        sp[q][16 * rb + l16][lg] = mx;
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
        eq_s[tid] = a16_exp(mx);
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
                a16_split(ldexpf(xs[k], -e), hi, lo);
                qh[i][k] = hi;
                ql[i][k] = lo;
            }
        }
    }
    int eqd[4];  // the exponents of the score rows the lane holds: tokens 16 rb + 4 lg + r
#pragma unroll
    for (int r = 0; r < 4; r++) eqd[r] = eq_s[16 * rb + 4 * lg + r];

    // a tile's rows: wave w loads position s0 + w, lane columns lane + 64 j (zeros past the
    // chunk and past KQ)
    // (the lane index passes through an opaque copy per call, so that its 64-bit addresses
    // are formed per request rather than hoisted out of the tile loop, where they would not
    // fit the registers)
    float xr[A16_NJ];
    auto load = [&](int s0) {
        const int pos = s0 + w;
        const bool ok = pos < r1;
        int ln = lane;
        asm volatile("" : "+v"(ln));
        const float *cr = a.comp + (size_t)pos * kv + ln, *pr = a.pe + (size_t)pos * rope + (ln - kv);
#pragma unroll
        for (int j = 0; j < A16_NJ; j++) {
            const int col = ln + 64 * j;
            xr[j] = ok && col < KQ ? (col < kv ? cr[64 * j] : pr[64 * j]) : 0.0f;
        }
    };
    load(r0);
    A16_STAMP(1, 0);

    aq_f4 acc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = (aq_f4){0.0f, 0.0f, 0.0f, 0.0f};

    for (int j = 0; j < ntile; j++) {
        const int s0 = r0 + AQ_P * j;
        {
            // the row of position s0 + w into the planes: kp scaled by its exponent over the
            // whole row, vp (the kv part) by its exponent over that part
            float mk = 0.0f, mv = 0.0f;
#pragma unroll
            for (int jj = 0; jj < A16_NJ; jj++) {
                const int col = lane + 64 * jj;
                mk = fmaxf(mk, fabsf(xr[jj]));
                if (col < kv) mv = fmaxf(mv, fabsf(xr[jj]));
            }
            const int ek = a16_exp(wave_max_dpp_f(mk)), ev = a16_exp(wave_max_dpp_f(mv));
            if (lane == 0) {
                ek_s[w] = ek;
                ev_s[w] = ev;
            }
            int ln = lane;
            asm volatile("" : "+v"(ln));
            _Float16 *khr = &kp[0][w * A16_KQS + ln], *klr = &kp[1][w * A16_KQS + ln];
            _Float16 *vhr = &vp[0][ln * A16_VS + w], *vlr = &vp[1][ln * A16_VS + w];
#pragma unroll
            for (int jj = 0; jj < A16_NJ; jj++) {
                const int col = ln + 64 * jj;
                if (col < ncol) {
                    _Float16 hi, lo;
                    a16_split(ldexpf(xr[jj], -ek), hi, lo);
                    khr[64 * jj] = hi;
                    klr[64 * jj] = lo;
                }
                if (col < kv) {
                    _Float16 hi, lo;
                    a16_split(ldexpf(xr[jj], -ev), hi, lo);
                    vhr[64 * A16_VS * jj] = hi;
                    vlr[64 * A16_VS * jj] = lo;
                }
            }
        }
        if (j + 1 < ntile) load(s0 + AQ_P);  // in flight while this tile is used
        at_barrier();  // (shared memory only: __syncthreads() would wait for that load)
        A16_STAMP(2, j);
        {
            // partial scores: lane holds rows 16 rb + 4 lg + r, position l16
            aq_f4 d = {0.0f, 0.0f, 0.0f, 0.0f};
            const _Float16 *kr = &kp[0][l16 * A16_KQS + 8 * lg + 32 * q];  // step q + 4 i at + 128 i
#pragma unroll
            for (int i = 0; i < A16_NQS; i++) {
                const int s = q + 4 * i;
                if (s < nks) {
                    const a16_h8 bh = *(const a16_h8 *)(kr + 128 * i);
                    const a16_h8 bl = *(const a16_h8 *)(kr + 128 * i + AQ_P * A16_KQS);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[i], bh, d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(qh[i], bl, d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ql[i], bh, d, 0, 0, 0);
                }
            }
            const int ekp = ek_s[l16];
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
            if (t >= tl || s >= r1 || s > a.pos + t) v = -INFINITY;  // causal, and past the chunk
            const float mo = run_m[row], mn = fmaxf(mo, row_max_dpp_f(v));
            const float e = mn == -INFINITY ? 0.0f : expf(__fsub_rn(v, mn));
            const float l = row_sum_dpp_f(e);
            const int evp = ev_s[p];
            const int eV = (int)row_max_dpp_f((float)evp);  // the tile's largest (the same in every row)
            _Float16 hi, lo;
            a16_split(ldexpf(e, evp - eV), hi, lo);
            pp[0][row * A16_PS + p] = hi;
            pp[1][row * A16_PS + p] = lo;
            if (p == 0) {
                const float cr = mn == -INFINITY ? 1.0f : expf(__fsub_rn(mo, mn));  // 0 while mo is -inf
                run_m[row] = mn;
                run_l[row] = fmaf(run_l[row], cr, l);
                corr[row] = cr;
                if (row == 0) ev_tile = eV;
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
            const float sv = ldexpf(1.0f, ev_tile);
            const a16_h4 ah = *(const a16_h4 *)&pp[0][(16 * rh + l16) * A16_PS + 4 * lg];
            const a16_h4 al = *(const a16_h4 *)&pp[1][(16 * rh + l16) * A16_PS + 4 * lg];
            const _Float16 *vr = &vp[0][(16 * (w >> 2) + l16) * A16_VS + 4 * lg];  // block i at + 64 A16_VS i
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const int cb = (w >> 2) + 4 * i;
                if (cb < kv / 16) {
                    const a16_h4 bh = *(const a16_h4 *)(vr + 64 * A16_VS * i);
                    const a16_h4 bl = *(const a16_h4 *)(vr + 64 * A16_VS * i + AT_KV_MAX * A16_VS);
                    aq_f4 d = {0.0f, 0.0f, 0.0f, 0.0f};
                    d = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bh, d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, bl, d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x16f16(al, bh, d, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[i][r] = fmaf(d[r], sv, __fmul_rn(acc[i][r], cr[r]));
                }
            }
        }
        at_barrier();  // the next tile overwrites the planes, the scores and the exponents
        A16_STAMP(5, j);
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
