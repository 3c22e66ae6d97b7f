// dense.h -- glm.c's decode forward outside the MoE layers, on the GPU: the Q8_0
// matrix-vector products (matvec_q80_rows, infer.c:765-786) of MLA attention, of layer
// 0's dense FFN and of the LM head; the latent-cache attention (infer.c:978-1065); the
// embedding row (infer.c:1807-1810). Everything is fp32 as in glm.c; the inputs of the
// products that glm.c normalises first (rmsnorm, infer.c:746-752) are normalised on
// load with glm.c's own operations, so they equal glm.c's normalised vectors bit for bit.
#pragma once

#include "common.h"

#define DM_BLOCK 256

// ---- Q8_0 matrix . vector ---------------------------------------------------------
//
// A row's dot product belongs to LPR lanes (16 or 64): lane sl of the row takes the
// 16-column units sl, sl + LPR, ... (U of them, so cols <= 16 LPR U), and keeps the
// activations of those units in registers for every row it visits. Each unit's 16
// products are summed and scaled by its group's scale (a unit lies inside one group: the
// group size is a multiple of 16). A wave holds 64 / LPR rows at a time and strides over
// the matrix's row groups, so its loads are 16 contiguous bytes per lane per unit.

enum { GV_PLAIN = 0, GV_RESID = 1, GV_PAIR = 2 };

struct GemvArgs {
    const int8_t *q, *q2;  // [rows][cols] Q8_0 values; q2 the second matrix of GV_PAIR
    const float *s, *s2;   // [rows][cols / gs] fp32 scales
    const float *x;        // input: rows of group g (x_rows rows each) read x + g * x_stride
    const float *norm;     // optional, one shared input: the input is rmsnorm(x) * norm
    const float *resid;    // GV_RESID: y = resid + dot (infer.c:1061, 1083)
    float *y;              // GV_PAIR: y = silu(dot) * dot2 (infer.c:1078-1080)
    int rows, cols, gs, x_rows, x_stride;
    int bx, by, br;        // a batch (grid y): token t's x, y and resid start t*bx, t*by, t*br floats in
    // GV_PLAIN only: a second matrix over the same input, its rows after the first's
    // (rows a multiple of the kernel's rows per wave): yb = qb . x
    const int8_t *qb;
    const float *sb;
    float *yb;
    int rows_b, by_b;
};

// Sum over each 16-lane row of a wave in fp64, to every lane of the row.
__device__ static inline double row_sum_dpp_d(double v) {
    v += dpp_d<DPP_QUAD_1032>(v, 0.0);
    v += dpp_d<DPP_QUAD_2301>(v, 0.0);
    v += dpp_d<DPP_ROW_HALF_MIRROR>(v, 0.0);
    v += dpp_d<DPP_ROW_MIRROR>(v, 0.0);
    return v;
}

// The lane's U units of the input of group g, normalised when a.norm is set.
template <int LPR, int U>
__device__ static inline void gv_load_x(const GemvArgs &a, int g, float (&xv)[U][16]) {
    const int sl = (threadIdx.x & 63) % LPR, nunits = a.cols >> 4;
    const float *x = a.x + (size_t)g * a.x_stride;
#pragma unroll
    for (int m = 0; m < U; m++) {
        const int u = sl + LPR * m;
        const bool on = u < nunits;
        const float4 *p = (const float4 *)(x + 16 * (on ? u : 0));
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const float4 f = p[v];
            xv[m][4 * v + 0] = on ? f.x : 0.0f;
            xv[m][4 * v + 1] = on ? f.y : 0.0f;
            xv[m][4 * v + 2] = on ? f.z : 0.0f;
            xv[m][4 * v + 3] = on ? f.w : 0.0f;
        }
    }
    if (!a.norm) return;
    // infer.c:746-752: fp64 sum of squares (every lane group holds the whole input),
    // fp32 mean, 1 / sqrtf, then x * inv * w
    double ss = 0.0;
#pragma unroll
    for (int m = 0; m < U; m++)
#pragma unroll
        for (int k = 0; k < 16; k++) ss += (double)xv[m][k] * (double)xv[m][k];
    ss = row_sum_dpp_d(ss);
    if (LPR == 64) ss = (readlane_d(ss, 0) + readlane_d(ss, 16)) + (readlane_d(ss, 32) + readlane_d(ss, 48));
    const float mean = (float)(ss / (double)a.cols);
    const float inv = __fdiv_rn(1.0f, sqrt_rn_f32(__fadd_rn(mean, 1e-5f)));
#pragma unroll
    for (int m = 0; m < U; m++) {
        const int u = sl + LPR * m;
        const bool on = u < nunits;
        const float4 *w = (const float4 *)(a.norm + 16 * (on ? u : 0));
#pragma unroll
        for (int v = 0; v < 4; v++) {
            const float4 f = w[v];
            const float wv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
            for (int k = 0; k < 4; k++) xv[m][4 * v + k] = __fmul_rn(__fmul_rn(xv[m][4 * v + k], inv), wv[k]);
        }
    }
}

// The lane's units of row r of a matrix: 16 int8 values and their group's scale each.
template <int U>
struct GvRow {
    u32x4 q[U];
    float s[U];
};

template <int LPR, int U>
__device__ static inline void gv_fetch(const int8_t *q, const float *s, int r, const GemvArgs &a, GvRow<U> &w) {
    const int sl = (threadIdx.x & 63) % LPR, nunits = a.cols >> 4, ng = a.cols / a.gs;
#pragma unroll
    for (int m = 0; m < U; m++) {
        const int u = sl + LPR * m, uc = u < nunits ? u : 0;
        w.q[m] = *gbl((const u32x4 *)(q + (size_t)r * a.cols + 16 * (size_t)uc));
        w.s[m] = *gbl(s + (size_t)r * ng + (16 * uc) / a.gs);
    }
}

// The lane's share of a fetched row's dot product with its units.
template <int LPR, int U>
__device__ static inline float gv_dot(const GvRow<U> &w, const GemvArgs &a, const float (&xv)[U][16]) {
    const int sl = (threadIdx.x & 63) % LPR, nunits = a.cols >> 4;
    float acc = 0.0f;
#pragma unroll
    for (int m = 0; m < U; m++) {
        const unsigned wd[4] = {w.q[m].x, w.q[m].y, w.q[m].z, w.q[m].w};
        float part = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; k++) part = fmaf((float)(int8_t)(wd[k >> 2] >> (8 * (k & 3))), xv[m][k], part);
        if (sl + LPR * m < nunits) acc = fmaf(part, w.s[m], acc);
    }
    return acc;
}

// Sum over the row's LPR lanes, to every lane of them.
template <int LPR>
__device__ static inline float gv_reduce(float v) {
    v = row_sum_dpp_f(v);
    if (LPR == 64) v = (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
    return v;
}

// The product over blocks bx of nbx (grid x) and token blockIdx.y of a batch.
template <int LPR, int U, int MODE>
__device__ __attribute__((always_inline)) static void gemv_run(GemvArgs a, int bx, int nbx) {
    constexpr int RPW = 64 / LPR;  // rows per wave at a time
    {
        const size_t t = blockIdx.y;  // the token of a batch
        a.x += t * (size_t)a.bx;
        a.y += t * (size_t)a.by;
        if (MODE == GV_RESID) a.resid += t * (size_t)a.br;
    }
    if (MODE == GV_PLAIN && a.rows_b) a.yb += blockIdx.y * (size_t)a.by_b;
    const int lane = threadIdx.x & 63, sub = lane / LPR, sl = lane % LPR;
    const int wave = bx * (DM_BLOCK / 64) + (threadIdx.x >> 6), nwaves = nbx * (DM_BLOCK / 64);
    const int rows_all = a.rows + (MODE == GV_PLAIN ? a.rows_b : 0);
    const int nrg = (rows_all + RPW - 1) / RPW;
    float xv[U][16];
    int xg = -1;  // the input group xv holds
    for (int rg = wave; rg < nrg; rg += nwaves) {
        // the row group's weights are requested before the input is loaded and normalised
        int r = rg * RPW + sub, n = a.rows;
        const int8_t *q = a.q;
        const float *s = a.s;
        float *y = a.y;
        if (MODE == GV_PLAIN && r >= a.rows) {  // the second matrix (whole row groups)
            r -= a.rows;
            n = a.rows_b;
            q = a.qb;
            s = a.sb;
            y = a.yb;
        }
        const int rc = r < n ? r : n - 1;
        GvRow<U> w, w2;
        gv_fetch<LPR, U>(q, s, rc, a, w);
        if (MODE == GV_PAIR) gv_fetch<LPR, U>(a.q2, a.s2, rc, a, w2);
        const int g = (rg * RPW) / a.x_rows;  // x_rows is a multiple of RPW: one group per row group
        if (g != xg) {
            gv_load_x<LPR, U>(a, g, xv);
            xg = g;
        }
        const float d = gv_reduce<LPR>(gv_dot<LPR, U>(w, a, xv));
        float out = d;
        if (MODE == GV_PAIR) {
            const float d2 = gv_reduce<LPR>(gv_dot<LPR, U>(w2, a, xv));
            out = __fmul_rn(__fdiv_rn(d, __fadd_rn(1.0f, expf(-d))), d2);
        }
        if (sl == 0 && r < n) {
            if (MODE == GV_RESID) out = __fadd_rn(a.resid[r], d);
            y[r] = out;
        }
    }
}

template <int LPR, int U, int MODE>
__global__ __launch_bounds__(DM_BLOCK) void k_gemv(GemvArgs a) {
    gemv_run<LPR, U, MODE>(a, blockIdx.x, gridDim.x);
}

// ---- embedding --------------------------------------------------------------------

// x = row `token` of the Q8_0 embedding table, dequantised (infer.c:754-763, 1807-1810).
__global__ __launch_bounds__(DM_BLOCK) void k_embed(const int8_t *__restrict__ tq, const float *__restrict__ ts, int token,
                                                    int dim, int gs, float *__restrict__ x) {
    const int i = blockIdx.x * DM_BLOCK + threadIdx.x;
    if (i >= dim) return;
    x[i] = __fmul_rn((float)tq[(size_t)token * dim + i], ts[(size_t)token * (dim / gs) + i / gs]);
}

// The embedding rows of a batch: token blockIdx.y's row into x + blockIdx.y * dim; a token
// outside the vocabulary takes row 0, as infer.c:1781 does.
__global__ __launch_bounds__(DM_BLOCK) void k_embed_batch(const int8_t *__restrict__ tq, const float *__restrict__ ts,
                                                          const int32_t *__restrict__ tokens, int vocab, int dim, int gs,
                                                          float *__restrict__ x) {
    const int i = blockIdx.x * DM_BLOCK + threadIdx.x;
    if (i >= dim) return;
    int token = tokens[blockIdx.y];
    if (token < 0 || token >= vocab) token = 0;
    x[(size_t)blockIdx.y * dim + i] = __fmul_rn((float)tq[(size_t)token * dim + i], ts[(size_t)token * (dim / gs) + i / gs]);
}

// ---- MLA attention over the latent cache ------------------------------------------

#define AT_TILE 36   // cache positions staged at a time by k_attn_chunk
#define AT_HG 16     // most heads per block of k_attn_chunk
#define AT_KV_MAX 512
#define AT_ROPE_MAX 64
#define AT_KS (AT_KV_MAX + AT_ROPE_MAX + 4)  // LDS row stride of a staged entry at the largest shape
#define AT_MAX_PARTS 1024                   // most position ranges (partial results) per head
#define AT_PREFILL_RANGES 8                 // position ranges per token of a batch
#define AT_BLOCK 1024                       // threads of k_attn_chunk

struct AttnArgs {
    const float *kv_a;     // [kv + rope]: the kv_a product of this position
    const float *kv_norm;  // [kv]
    const float *q_full;   // [H][head_k]: nope part, then rope part
    const float *rope_cs;  // [cap][rope / 2][2]: cos, sin of glm.c's angles (computed on the host with libm)
    float *comp, *pe;      // this layer's latent cache, [cap][kv] and [cap][rope]
    float *q_pe;           // [H][rope]
    const float *q_abs;    // [H][kv]
    float *part_ctx;       // [nblk][H][kv]
    float *part_ml;        // [nblk][H][2]: a range's maximum score and its sum of exponentials
    float *ctx;            // [H][kv]
    int H, kv, rope, head_k, nope, pos;
    int hg;                // heads per block of k_attn_chunk (<= AT_HG)
    int nblk;              // position ranges of k_attn_chunk (blocks per head group), <= AT_MAX_PARTS
    float kq_scale;
    // this layer's cache entries in split fp16 form for the batch attention on matrix cores
    // (null: not kept): ksp [cap16][SPL_KROW] halves, a row per position (see below); vsp
    // [cap16 / 16][2][kv][16] halves, the compressed part transposed in blocks of 16 positions
    _Float16 *ksp, *vsp;
};

// The split form of a cache entry (the matrix cores' operands, written once per position
// by attn_prep_run): x = hi + lo, fp16 each, of the entry scaled by 2^-e, e the exponent with
// max |entry| 2^-e < 2^15 (SPL_EMPTY for a zero entry). A ksp row is the kv + rope columns'
// hi (SPL_KCOLS halves, zeros past kv + rope), then their lo, then e (an int), then
// padding to SPL_KROW halves, an odd count of 16-byte units so that rows read together fall
// in distinct banks. vsp holds the compressed part's hi and lo planes transposed by blocks
// of 16 positions: block b, plane, column c, position slot s at ((b * 2 + plane) * kv + c) * 16 + s.
#define SPL_KCOLS 576
#define SPL_KEXP (2 * SPL_KCOLS)   // half index of the exponent in a ksp row
#define SPL_KROW (2 * SPL_KCOLS + 8)
#define SPL_EMPTY (-1000)
static_assert((SPL_KROW * 2 / 16) % 2 == 1, "a ksp row is an odd count of 16-byte units");

// The exponent e with |x| 2^-e < 2^15 for every |x| <= mx (SPL_EMPTY when mx is 0).
__device__ static inline int spl_exp(float mx) {
    if (!(mx > 0.0f)) return SPL_EMPTY;
    int k;
    (void)frexpf(mx, &k);  // mx < 2^k
    return k - 15;
}

// x = hi + lo: hi the nearest fp16, lo the nearest fp16 to the (exact) remainder.
__device__ static inline void spl_split(float x, _Float16 &hi, _Float16 &lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// The split form of the entry row[0 .. kv + rope) (the block's shared memory, written before
// a barrier) into ksp row kr and vsp slot vb (kv + rope <= SPL_KCOLS, kv <= the vsp planes'
// width: the host's checks); rmax: DM_BLOCK / 64 floats of shared memory.
__device__ __attribute__((always_inline)) static void spl_store(const float *row, int kv, int rope, _Float16 *kr,
                                                                _Float16 *vb, float *rmax) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, KQ = kv + rope;
    float mx = 0.0f;
    for (int i = tid; i < KQ; i += DM_BLOCK) mx = fmaxf(mx, fabsf(row[i]));
    mx = wave_max_dpp_f(mx);
    if (lane == 0) rmax[w] = mx;
    __syncthreads();
    const int e = spl_exp(fmaxf(fmaxf(rmax[0], rmax[1]), fmaxf(rmax[2], rmax[3])));
    for (int i = tid; i < SPL_KCOLS; i += DM_BLOCK) {
        _Float16 hi = (_Float16)0.0f, lo = (_Float16)0.0f;
        if (i < KQ) spl_split(ldexpf(row[i], -e), hi, lo);
        kr[i] = hi;
        kr[SPL_KCOLS + i] = lo;
        if (i < kv) {
            vb[(size_t)i * 16] = hi;
            vb[((size_t)kv + i) * 16] = lo;
        }
    }
    if (tid < (SPL_KROW - SPL_KEXP) / 2) ((int *)(kr + SPL_KEXP))[tid] = tid == 0 ? e : 0;
}
static_assert(DM_BLOCK == 256, "spl_store joins four waves' maxima");

// The position's cache entry and the heads' rotated queries (infer.c:1000-1016): the
// compressed kv normalised (rmsnorm over kv values), the rope part of kv_a and of every
// head's query rotated by the position's angles. One block for token t of a batch, at
// position pos + t (its kv_a, q_full and q_pe t token strides on).
__device__ __attribute__((always_inline)) static void attn_prep_run(AttnArgs a, int t) {
    __shared__ double red[DM_BLOCK / 64];
    __shared__ float row[SPL_KCOLS];  // the entry, for its split form
    __shared__ float rmax[DM_BLOCK / 64];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    {
        a.kv_a += (size_t)t * (a.kv + a.rope);
        a.q_full += (size_t)t * a.H * a.head_k;
        a.q_pe += (size_t)t * a.H * a.rope;
        a.pos += t;
    }
    double ss = 0.0;
    for (int i = tid; i < a.kv; i += DM_BLOCK) ss += (double)a.kv_a[i] * (double)a.kv_a[i];
    ss = wave_sum_dpp(ss);
    if (lane == 0) red[w] = ss;
    __syncthreads();
    ss = (red[0] + red[1]) + (red[2] + red[3]);
    const float mean = (float)(ss / (double)a.kv);
    const float inv = __fdiv_rn(1.0f, sqrt_rn_f32(__fadd_rn(mean, 1e-5f)));
    float *comp = a.comp + (size_t)a.pos * a.kv, *pe = a.pe + (size_t)a.pos * a.rope;
    for (int i = tid; i < a.kv; i += DM_BLOCK) {
        const float v = __fmul_rn(__fmul_rn(a.kv_a[i], inv), a.kv_norm[i]);
        comp[i] = v;
        if (i < SPL_KCOLS) row[i] = v;
    }
    const float *cs = a.rope_cs + (size_t)a.pos * a.rope;  // rope/2 pairs of (cos, sin)
    const int half = a.rope >> 1;
    // infer.c:964-976 on kv_a's rope part (pair 0 .. half-1) and each head's (pairs half ..)
    for (int j = tid; j < (a.H + 1) * half; j += DM_BLOCK) {
        const int h = j / half - 1, i = j % half;
        const float *src = h < 0 ? a.kv_a + a.kv : a.q_full + (size_t)h * a.head_k + a.nope;
        float *dst = h < 0 ? pe : a.q_pe + (size_t)h * a.rope;
        const float c = cs[2 * i], s = cs[2 * i + 1], x0 = src[2 * i], x1 = src[2 * i + 1];
        const float y0 = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, s)), y1 = __fadd_rn(__fmul_rn(x0, s), __fmul_rn(x1, c));
        dst[2 * i] = y0;
        dst[2 * i + 1] = y1;
        if (h < 0 && a.kv + 2 * i + 1 < SPL_KCOLS) {
            row[a.kv + 2 * i] = y0;
            row[a.kv + 2 * i + 1] = y1;
        }
    }
    if (!a.ksp) return;  // a decode step: the host marks the position for k_spl_fill
    __syncthreads();
    spl_store(row, a.kv, a.rope, a.ksp + (size_t)a.pos * SPL_KROW, a.vsp + (size_t)(a.pos >> 4) * 2 * a.kv * 16 + (a.pos & 15),
              rmax);
}

// Positions p0 + blockIdx.x of attention layer blockIdx.y: the split form from the fp32
// entry (the same values attn_prep_run splits), for positions a decode step wrote without it.
__global__ __launch_bounds__(DM_BLOCK) void k_spl_fill(const float *comp, const float *pe, _Float16 *ksp, _Float16 *vsp,
                                                      size_t cap, size_t capt, int kv, int rope, int p0) {
    __shared__ float row[SPL_KCOLS];
    __shared__ float rmax[DM_BLOCK / 64];
    const int p = p0 + blockIdx.x, l = blockIdx.y;
    const float *ce = comp + ((size_t)l * cap + p) * kv, *re = pe + ((size_t)l * cap + p) * rope;
    for (int i = threadIdx.x; i < kv + rope; i += DM_BLOCK) row[i] = i < kv ? ce[i] : re[i - kv];
    __syncthreads();
    spl_store(row, kv, rope, ksp + ((size_t)l * capt + p) * SPL_KROW,
              vsp + (size_t)l * capt * 2 * kv + (size_t)(p >> 4) * 2 * kv * 16 + (p & 15), rmax);
}

// The query side of a token's attention in one launch: the absorbed queries q_abs = k_b_h .
// q_nope_h (the k_b product, blocks 0 .. gridDim.x - 2) and, on the last block of the
// row, k_attn_prep's cache entry and rotated queries. The two read q_full and kv_a only.
template <int LPR, int U>
__global__ __launch_bounds__(DM_BLOCK) void k_attn_query(GemvArgs kb, AttnArgs aa) {
    if (blockIdx.x + 1 < gridDim.x)
        gemv_run<LPR, U, GV_PLAIN>(kb, blockIdx.x, gridDim.x - 1);
    else
        attn_prep_run(aa, blockIdx.y);
}

// Token t of a batch (grid z) at position pos + t: its queries, context and partial results
// t token strides on (nblk ranges of partials per token).
__device__ __attribute__((always_inline)) static void attn_token(AttnArgs &a, int t) {
    if (t == 0) return;
    a.pos += t;
    a.q_abs += (size_t)t * a.H * a.kv;
    a.q_pe += (size_t)t * a.H * a.rope;
    a.ctx += (size_t)t * a.H * a.kv;
    a.part_ctx += (size_t)t * a.nblk * a.H * a.kv;
    a.part_ml += (size_t)t * a.nblk * a.H * 2;
}

// Float DPP move within a row (bound_ctrl off: an inactive source lane gives 0).
template <int CTRL>
__device__ static inline float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Reduce-scatter over each 16-lane row: every lane holds v[0..7]; afterwards lanes s and
// s ^ 1 of the row hold the row's sum of v[s >> 1]. Each step pairs a lane with one whose
// index differs in the next bit down (across the row, then within each half, then within
// quads), keeps the half of its values whose index has its own bit and adds the partner's
// copy of that half; the last step adds the pair's two sums. 8 adds and DPP moves per lane
// instead of 8 row sums of 4 steps each.
__device__ static inline float row_reduce_scatter8(const float (&v)[8], int s) {
    const bool b3 = (s & 8) != 0, b2 = (s & 4) != 0, b1 = (s & 2) != 0;
    float u[4], x[2];
#pragma unroll
    for (int m = 0; m < 4; m++) u[m] = (b3 ? v[m + 4] : v[m]) + dpp_f<DPP_ROW_MIRROR>(b3 ? v[m] : v[m + 4]);
#pragma unroll
    for (int m = 0; m < 2; m++) x[m] = (b2 ? u[m + 2] : u[m]) + dpp_f<DPP_ROW_HALF_MIRROR>(b2 ? u[m] : u[m + 2]);
    const float y = (b1 ? x[1] : x[0]) + dpp_f<DPP_QUAD_2301>(b1 ? x[0] : x[1]);
    return y + dpp_f<DPP_QUAD_1032>(y);
}

// A block barrier after this wave's shared-memory accesses only: global loads still in
// flight (the next tile's) are not waited for, as __syncthreads()'s release fence would.
__device__ static inline void at_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

#define AT_HB 2  // heads per thread in k_attn_chunk's scores and weighted sum
#define AT_TB 4  // cache positions per thread in its scores
static_assert(AT_HB * AT_TB == 8, "row_reduce_scatter8 takes eight scores per lane");

// Position range blockIdx.x of nblk (an even split of 0 .. pos) for heads hg * blockIdx.y ..
// (infer.c:1029-1051, split into ranges and merged by k_attn_merge). The heads' queries are
// staged in LDS once and the range's cache entries AT_TILE at a time; the loads of the
// first tile go out with the queries' and each later tile's while the one before it is
// scored, so a range waits on memory once. Each score is the absorbed query against the
// compressed entry plus the rotated parts, times 1/sqrt(head_k): a 16-lane row takes
// AT_HB heads x AT_TB positions, each lane a sixteenth of the columns, so every value it
// reads from LDS serves two or four products, and a reduce-scatter leaves one score per
// lane pair. Pairs of heads spread the work over 10 of the 16 waves at 10 heads. Per
// head the block keeps the range's running maximum and sum of exponentials and the
// exponential-weighted sum of compressed entries, rescaled when the maximum grows; a
// thread of that sum takes one float4 of the entry for AT_HB heads, four positions per
// step. The LDS holds one block per CU, so the block is 16 waves wide, and the host sizes
// nblk so that a head group's ranges fill the CUs once. A batch of tokens takes grid z
// (attn_token), each token min(nblk, its positions) ranges.
__global__ __launch_bounds__(AT_BLOCK) void k_attn_chunk(AttnArgs a) {
    __shared__ __align__(16) float ks[AT_TILE * AT_KS];
    __shared__ __align__(16) float qs[AT_HG * (AT_KV_MAX + AT_ROPE_MAX)];
    __shared__ __align__(16) float sc[AT_HG][AT_TILE];
    __shared__ float run_m[AT_HG], run_l[AT_HG], corr[AT_HG];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    attn_token(a, blockIdx.z);
    const int b = blockIdx.x, h0 = a.hg * blockIdx.y, nh = min(a.hg, a.H - h0);
    const int P = a.pos + 1, nb = min(a.nblk, P);
    if (b >= nb) return;  // a prefill token with fewer positions than ranges
    const int r0 = (int)((long long)b * P / nb), r1 = (int)((long long)(b + 1) * P / nb);
    const int kv = a.kv, rope = a.rope, KQ = kv + rope;
    const int qsd = (KQ + 3) & ~3;          // a row of either, rounded up to whole float4s
    const int ksd = ((KQ + 31) & ~31) + 4;  // entry row stride: 4 mod 32 keeps row-wise b128 reads apart
    const int kv4 = kv >> 2, r2 = rope >> 1, n4 = qsd >> 2;
    constexpr int NQ = (AT_HG * AT_KV_MAX / 4 + AT_BLOCK - 1) / AT_BLOCK;      // float4s of absorbed queries
    constexpr int NR = (AT_HG * AT_ROPE_MAX / 2 + AT_BLOCK - 1) / AT_BLOCK;    // float2s of rotated queries
    constexpr int NC = (AT_TILE * AT_KV_MAX / 4 + AT_BLOCK - 1) / AT_BLOCK;    // float4s of a tile's entries
    constexpr int NP = (AT_TILE * AT_ROPE_MAX / 2 + AT_BLOCK - 1) / AT_BLOCK;  // float2s of its rope parts
    float4 vc[NC];
    float2 vp[NP];
    auto fetch = [&](int t0) {  // a tile's loads into vc, vp
        const int nt = min(AT_TILE, r1 - t0);
        const float4 *gc = reinterpret_cast<const float4 *>(a.comp + (size_t)t0 * kv);
        const float2 *gp = reinterpret_cast<const float2 *>(a.pe + (size_t)t0 * rope);
#pragma unroll
        for (int k = 0; k < NC; k++) {
            const int i = tid + AT_BLOCK * k;
            vc[k] = i < nt * kv4 ? gc[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int k = 0; k < NP; k++) {
            const int i = tid + AT_BLOCK * k;
            vp[k] = i < nt * r2 ? gp[i] : make_float2(0.0f, 0.0f);
        }
    };
    {
        const float4 *gq = reinterpret_cast<const float4 *>(a.q_abs + (size_t)h0 * kv);
        const float2 *gr = reinterpret_cast<const float2 *>(a.q_pe + (size_t)h0 * rope);
        float4 vq[NQ];
        float2 vr[NR];
#pragma unroll
        for (int k = 0; k < NQ; k++) {
            const int i = tid + AT_BLOCK * k;
            vq[k] = i < nh * kv4 ? gq[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int k = 0; k < NR; k++) {
            const int i = tid + AT_BLOCK * k;
            vr[k] = i < nh * r2 ? gr[i] : make_float2(0.0f, 0.0f);
        }
        fetch(r0);
#pragma unroll
        for (int k = 0; k < NQ; k++) {
            const int i = tid + AT_BLOCK * k;
            if (i < nh * kv4) *reinterpret_cast<float4 *>(&qs[(i / kv4) * qsd + 4 * (i % kv4)]) = vq[k];
        }
#pragma unroll
        for (int k = 0; k < NR; k++) {
            const int i = tid + AT_BLOCK * k;
            if (i < nh * r2) *reinterpret_cast<float2 *>(&qs[(i / r2) * qsd + kv + 2 * (i % r2)]) = vr[k];
        }
        if (qsd > KQ && tid < nh) {  // zeros up to the float4 boundary (rope % 4 == 2)
            qs[tid * qsd + KQ] = 0.0f;
            qs[tid * qsd + KQ + 1] = 0.0f;
        }
        if (tid < AT_HG) {
            run_m[tid] = -INFINITY;
            run_l[tid] = 0.0f;
        }
    }
    const int ngh = (nh + AT_HB - 1) / AT_HB;  // head groups of AT_HB
    const int sg = tid >> 4, sl = tid & 15;    // scores: the thread's 16-lane row and its lane in it
    const int wq = tid % kv4, wh = tid / kv4;  // weighted sum: the entry's float4 and the head group
    const bool summer = wh < ngh;
    float4 acc[AT_HB];
#pragma unroll
    for (int x = 0; x < AT_HB; x++) acc[x] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int t0 = r0; t0 < r1; t0 += AT_TILE) {
        const int nt = min(AT_TILE, r1 - t0);
#pragma unroll
        for (int k = 0; k < NC; k++) {
            const int i = tid + AT_BLOCK * k;
            if (i < nt * kv4) *reinterpret_cast<float4 *>(&ks[(i / kv4) * ksd + 4 * (i % kv4)]) = vc[k];
        }
#pragma unroll
        for (int k = 0; k < NP; k++) {
            const int i = tid + AT_BLOCK * k;
            if (i < nt * r2) *reinterpret_cast<float2 *>(&ks[(i / r2) * ksd + kv + 2 * (i % r2)]) = vp[k];
        }
        if (qsd > KQ && tid < nt) {
            ks[tid * ksd + KQ] = 0.0f;
            ks[tid * ksd + KQ + 1] = 0.0f;
        }
        at_barrier();
        if (t0 + AT_TILE < r1) fetch(t0 + AT_TILE);  // in flight while this tile is used
        // scores: row sg takes heads AT_HB gh .. and positions AT_TB gt .. (rows past nh or nt
        // read LDS rows inside the buffers and are not written)
        const int ngt = (nt + AT_TB - 1) / AT_TB;
        for (int g = sg; g < ngh * ngt; g += AT_BLOCK / 16) {
            const int gh = g % ngh, gt = g / ngh;
            const float *qr = qs + AT_HB * gh * qsd, *kr = ks + AT_TB * gt * ksd;
            float d[AT_HB * AT_TB];
#pragma unroll
            for (int i = 0; i < AT_HB * AT_TB; i++) d[i] = 0.0f;
            for (int j = sl; j < n4; j += 16) {
                float4 q4[AT_HB];
#pragma unroll
                for (int x = 0; x < AT_HB; x++) q4[x] = *reinterpret_cast<const float4 *>(qr + x * qsd + 4 * j);
#pragma unroll
                for (int y = 0; y < AT_TB; y++) {  // one entry at a time: fewer live registers
                    const float4 k4 = *reinterpret_cast<const float4 *>(kr + y * ksd + 4 * j);
#pragma unroll
                    for (int x = 0; x < AT_HB; x++) {
                        float s = d[AT_TB * x + y];
                        s = fmaf(q4[x].x, k4.x, s);
                        s = fmaf(q4[x].y, k4.y, s);
                        s = fmaf(q4[x].z, k4.z, s);
                        d[AT_TB * x + y] = fmaf(q4[x].w, k4.w, s);
                    }
                }
            }
            const float v = row_reduce_scatter8(d, sl);
            const int h = AT_HB * gh + (sl >> 3), t = AT_TB * gt + ((sl >> 1) & 3);
            if ((sl & 1) == 0 && h < nh && t < nt) sc[h][t] = __fmul_rn(v, a.kq_scale);
        }
        at_barrier();
        // per head (a wave each): the tile's maximum, the running maximum and sum of
        // exponentials, exp(score - running maximum) for the tile (lane = position; zeros
        // past nt, which the weighted sum reads in its last step)
        for (int h = w; h < nh; h += AT_BLOCK / 64) {
            const float v = lane < nt ? sc[h][lane] : -INFINITY;
            const float mo = run_m[h], mn = fmaxf(mo, wave_max_dpp_f(v));
            const float e = lane < nt ? expf(__fsub_rn(v, mn)) : 0.0f;
            const float l = gv_reduce<64>(e);
            const float cr = mo == -INFINITY ? 0.0f : expf(__fsub_rn(mo, mn));  // the earlier tiles' rescale
            if (lane < AT_TILE) sc[h][lane] = e;
            if (lane == 0) {
                run_m[h] = mn;
                run_l[h] = fmaf(run_l[h], cr, l);
                corr[h] = cr;
            }
        }
        at_barrier();
        if (summer) {
#pragma unroll
            for (int x = 0; x < AT_HB; x++) {  // head groups past nh rescale rows that are not stored
                const float cr = corr[AT_HB * wh + x];
                acc[x].x = __fmul_rn(acc[x].x, cr);
                acc[x].y = __fmul_rn(acc[x].y, cr);
                acc[x].z = __fmul_rn(acc[x].z, cr);
                acc[x].w = __fmul_rn(acc[x].w, cr);
            }
            for (int t = 0; t < nt; t += 4) {
                float4 k4[4];
#pragma unroll
                for (int y = 0; y < 4; y++)
                    k4[y] = t + y < nt ? *reinterpret_cast<const float4 *>(&ks[(t + y) * ksd + 4 * wq])
                                       : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
                for (int x = 0; x < AT_HB; x++) {
                    const float4 p = *reinterpret_cast<const float4 *>(&sc[AT_HB * wh + x][t]);
                    const float pv[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
                    for (int y = 0; y < 4; y++) {
                        acc[x].x = fmaf(pv[y], k4[y].x, acc[x].x);
                        acc[x].y = fmaf(pv[y], k4[y].y, acc[x].y);
                        acc[x].z = fmaf(pv[y], k4[y].z, acc[x].z);
                        acc[x].w = fmaf(pv[y], k4[y].w, acc[x].w);
                    }
                }
            }
        }
        at_barrier();  // the next tile overwrites ks and sc
    }
    if (summer) {
#pragma unroll
        for (int x = 0; x < AT_HB; x++) {
            const int h = AT_HB * wh + x;
            if (h < nh) *reinterpret_cast<float4 *>(&a.part_ctx[((size_t)b * a.H + h0 + h) * kv + 4 * wq]) = acc[x];
        }
    }
    if (tid < nh) {
        a.part_ml[((size_t)b * a.H + h0 + tid) * 2] = run_m[tid];
        a.part_ml[((size_t)b * a.H + h0 + tid) * 2 + 1] = run_l[tid];
    }
}

// Head blockIdx.x, entries 64 * blockIdx.y ..: the ranges' partial sums merged (each
// weighted by exp(its max - the overall max)) and divided by the total sum of exponentials,
// the softmax-weighted sum of compressed entries (infer.c:1038-1051). The block's four
// waves take every fourth range, eight loads in flight each.
__global__ __launch_bounds__(DM_BLOCK) void k_attn_merge(AttnArgs a) {
    __shared__ float wgt[AT_MAX_PARTS];
    __shared__ float red[DM_BLOCK / 64];
    __shared__ float part[DM_BLOCK / 64][64];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = blockIdx.x;
    attn_token(a, blockIdx.z);
    const int nc = min(a.nblk, a.pos + 1);  // the position ranges of k_attn_chunk
    float m = -INFINITY;
    for (int c = tid; c < nc; c += DM_BLOCK) m = fmaxf(m, a.part_ml[((size_t)c * a.H + h) * 2]);
    m = wave_max_dpp_f(m);
    if (lane == 0) red[w] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float l = 0.0f;
    for (int c = tid; c < nc; c += DM_BLOCK) {
        const float e = expf(__fsub_rn(a.part_ml[((size_t)c * a.H + h) * 2], m));
        wgt[c] = e;
        l = fmaf(a.part_ml[((size_t)c * a.H + h) * 2 + 1], e, l);
    }
    l = gv_reduce<64>(l);
    if (lane == 0) red[w] = l;
    __syncthreads();
    l = (red[0] + red[1]) + (red[2] + red[3]);
    const int d = 64 * blockIdx.y + lane;
    const float *pc = a.part_ctx + (size_t)h * a.kv + d;
    const size_t cs = (size_t)a.H * a.kv;  // one chunk's stride
    float s = 0.0f;
    int c = w;
    for (; c + 28 < nc; c += 32) {
        float v[8];
#pragma unroll
        for (int k = 0; k < 8; k++) v[k] = pc[(size_t)(c + 4 * k) * cs];
#pragma unroll
        for (int k = 0; k < 8; k++) s = fmaf(wgt[c + 4 * k], v[k], s);
    }
    for (; c < nc; c += 4) s = fmaf(wgt[c], pc[(size_t)c * cs], s);
    part[w][lane] = s;
    __syncthreads();
    if (w == 0) {
        const float t = (part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]);
        a.ctx[(size_t)h * a.kv + d] = __fmul_rn(t, __fdiv_rn(1.0f, l));
    }
}

// k_attn_merge for at most AM_SMALL ranges per token (the batch attention's position chunks,
// attn.h): one wave per (token, head), lane l taking columns l + 64 j, with the same operations
// in the same order as k_attn_merge (a range per lane for the maximum and the sum; per column
// the ranges w and w + 4 of "wave" w, then (s0 + s1) + (s2 + s3)), so its results are
// bit-identical, in one wave instead of a block of four per 64 columns and three barriers.
#define AM_SMALL 8
__global__ __launch_bounds__(DM_BLOCK) void k_attn_merge_small(AttnArgs a0, int n) {
    const int lane = threadIdx.x & 63, pair = blockIdx.x * (DM_BLOCK / 64) + (threadIdx.x >> 6);
    if (pair >= n * a0.H) return;
    const int t = pair / a0.H, h = pair % a0.H;
    AttnArgs a = a0;
    attn_token(a, t);
    const int nc = min(a.nblk, a.pos + 1);  // <= AM_SMALL (the caller's guarantee)
    const float raw = lane < nc ? a.part_ml[((size_t)lane * a.H + h) * 2] : -INFINITY;
    const float m = wave_max_dpp_f(fmaxf(-INFINITY, raw));
    float e = 0.0f, lp = 0.0f;
    if (lane < nc) {
        e = expf(__fsub_rn(raw, m));
        lp = fmaf(a.part_ml[((size_t)lane * a.H + h) * 2 + 1], e, 0.0f);
    }
    const float l = __fadd_rn(__fadd_rn(gv_reduce<64>(lp), 0.0f), __fadd_rn(0.0f, 0.0f));
    float wgt[AM_SMALL];
#pragma unroll
    for (int c = 0; c < AM_SMALL; c++) wgt[c] = readlane_f(e, c);
    const float inv = __fdiv_rn(1.0f, l);
    const size_t cs = (size_t)a.H * a.kv;  // one range's stride
    const float *pc = a.part_ctx + (size_t)h * a.kv;
    for (int d = lane; d < a.kv; d += 64) {
        float v[AM_SMALL];
#pragma unroll
        for (int c = 0; c < AM_SMALL; c++) v[c] = c < nc ? pc[(size_t)c * cs + d] : 0.0f;
        float sw[4];
#pragma unroll
        for (int w = 0; w < 4; w++) {
            float sv = 0.0f;
            if (w < nc) sv = fmaf(wgt[w], v[w], sv);
            if (w + 4 < nc) sv = fmaf(wgt[w + 4], v[w + 4], sv);
            sw[w] = sv;
        }
        a.ctx[(size_t)h * a.kv + d] = __fmul_rn(__fadd_rn(__fadd_rn(sw[0], sw[1]), __fadd_rn(sw[2], sw[3])), inv);
    }
}
