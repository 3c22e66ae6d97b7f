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

// The lane's share of row r's dot product with its units.
template <int LPR, int U>
__device__ static inline float gv_dot(const int8_t *q, const float *s, int r, const GemvArgs &a, const float (&xv)[U][16]) {
    const int sl = (threadIdx.x & 63) % LPR, nunits = a.cols >> 4, ng = a.cols / a.gs;
    u32x4 qv[U];
    float sv[U];
#pragma unroll
    for (int m = 0; m < U; m++) {
        const int u = sl + LPR * m, uc = u < nunits ? u : 0;
        qv[m] = *gbl((const u32x4 *)(q + (size_t)r * a.cols + 16 * (size_t)uc));
        sv[m] = *gbl(s + (size_t)r * ng + (16 * uc) / a.gs);
    }
    float acc = 0.0f;
#pragma unroll
    for (int m = 0; m < U; m++) {
        const unsigned wd[4] = {qv[m].x, qv[m].y, qv[m].z, qv[m].w};
        float part = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; k++) part = fmaf((float)(int8_t)(wd[k >> 2] >> (8 * (k & 3))), xv[m][k], part);
        if (sl + LPR * m < nunits) acc = fmaf(part, sv[m], acc);
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

template <int LPR, int U, int MODE>
__global__ __launch_bounds__(DM_BLOCK) void k_gemv(GemvArgs a) {
    constexpr int RPW = 64 / LPR;  // rows per wave at a time
    {
        const size_t t = blockIdx.y;  // the token of a batch
        a.x += t * (size_t)a.bx;
        a.y += t * (size_t)a.by;
        if (MODE == GV_RESID) a.resid += t * (size_t)a.br;
    }
    const int lane = threadIdx.x & 63, sub = lane / LPR, sl = lane % LPR;
    const int wave = blockIdx.x * (DM_BLOCK / 64) + (threadIdx.x >> 6), nwaves = gridDim.x * (DM_BLOCK / 64);
    const int nrg = (a.rows + RPW - 1) / RPW;
    float xv[U][16];
    int xg = -1;  // the input group xv holds
    for (int rg = wave; rg < nrg; rg += nwaves) {
        const int g = (rg * RPW) / a.x_rows;  // x_rows is a multiple of RPW: one group per row group
        if (g != xg) {
            gv_load_x<LPR, U>(a, g, xv);
            xg = g;
        }
        const int r = rg * RPW + sub, rc = r < a.rows ? r : a.rows - 1;
        const float d = gv_reduce<LPR>(gv_dot<LPR, U>(a.q, a.s, rc, a, xv));
        float out = d;
        if (MODE == GV_PAIR) {
            const float d2 = gv_reduce<LPR>(gv_dot<LPR, U>(a.q2, a.s2, rc, a, xv));
            out = __fmul_rn(__fdiv_rn(d, __fadd_rn(1.0f, expf(-d))), d2);
        }
        if (sl == 0 && r < a.rows) {
            if (MODE == GV_RESID) out = __fadd_rn(a.resid[r], d);
            a.y[r] = out;
        }
    }
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

#define AT_CH 64   // cache positions per chunk of k_attn_part (one per lane in its softmax)
#define AT_HG 8    // heads per block of k_attn_part
#define AT_KV_MAX 512
#define AT_ROPE_MAX 64

struct AttnArgs {
    const float *kv_a;     // [kv + rope]: the kv_a product of this position
    const float *kv_norm;  // [kv]
    const float *q_full;   // [H][head_k]: nope part, then rope part
    const float *rope_cs;  // [cap][rope / 2][2]: cos, sin of glm.c's angles (computed on the host with libm)
    float *comp, *pe;      // this layer's latent cache, [cap][kv] and [cap][rope]
    float *q_pe;           // [H][rope]
    const float *q_abs;    // [H][kv]
    float *part_ctx;       // [chunks][H][kv]
    float *part_ml;        // [chunks][H][2]: chunk maximum and its sum of exponentials
    float *ctx;            // [H][kv]
    int H, kv, rope, head_k, nope, pos;
    float kq_scale;
};

// The position's cache entry and the heads' rotated queries (infer.c:1000-1016): the
// compressed kv normalised (rmsnorm over kv values), the rope part of kv_a and of every
// head's query rotated by the position's angles. One block per token: block t of a batch
// takes token t at position pos + t (its kv_a, q_full and q_pe t token strides on).
__global__ __launch_bounds__(DM_BLOCK) void k_attn_prep(AttnArgs a) {
    __shared__ double red[DM_BLOCK / 64];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    {
        const int t = blockIdx.x;
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
    for (int i = tid; i < a.kv; i += DM_BLOCK) comp[i] = __fmul_rn(__fmul_rn(a.kv_a[i], inv), a.kv_norm[i]);
    const float *cs = a.rope_cs + (size_t)a.pos * a.rope;  // rope/2 pairs of (cos, sin)
    const int half = a.rope >> 1;
    // infer.c:964-976 on kv_a's rope part (pair 0 .. half-1) and each head's (pairs half ..)
    for (int j = tid; j < (a.H + 1) * half; j += DM_BLOCK) {
        const int h = j / half - 1, i = j % half;
        const float *src = h < 0 ? a.kv_a + a.kv : a.q_full + (size_t)h * a.head_k + a.nope;
        float *dst = h < 0 ? pe : a.q_pe + (size_t)h * a.rope;
        const float c = cs[2 * i], s = cs[2 * i + 1], x0 = src[2 * i], x1 = src[2 * i + 1];
        dst[2 * i] = __fsub_rn(__fmul_rn(x0, c), __fmul_rn(x1, s));
        dst[2 * i + 1] = __fadd_rn(__fmul_rn(x0, s), __fmul_rn(x1, c));
    }
}

// Chunk c (AT_CH positions) of heads AT_HG * blockIdx.y ..: every score (the absorbed
// query against the compressed entry plus the rotated parts, times 1/sqrt(head_k)), the
// chunk's maximum and sum of exponentials per head, and its exponential-weighted sum of
// compressed entries (infer.c:1017-1051, split into chunks and merged by k_attn_combine).
__global__ __launch_bounds__(DM_BLOCK) void k_attn_part(AttnArgs a) {
    __shared__ float qs[AT_HG][AT_KV_MAX + AT_ROPE_MAX];
    __shared__ float sc[AT_HG][AT_CH];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int c = blockIdx.x, h0 = AT_HG * blockIdx.y, nh = min(AT_HG, a.H - h0);
    const int t0 = c * AT_CH, nt = min(AT_CH, a.pos + 1 - t0), KQ = a.kv + a.rope;
    for (int j = tid; j < nh * KQ; j += DM_BLOCK) {
        const int h = j / KQ, i = j % KQ;
        qs[h][i] = i < a.kv ? a.q_abs[(size_t)(h0 + h) * a.kv + i] : a.q_pe[(size_t)(h0 + h) * a.rope + (i - a.kv)];
    }
    __syncthreads();
    // scores: a wave per position, lane l holding entries l, l + 64, .. of it
    const int nk = a.kv >> 6;
    for (int t = w; t < nt; t += DM_BLOCK / 64) {
        const float *kc = a.comp + (size_t)(t0 + t) * a.kv, *kp = a.pe + (size_t)(t0 + t) * a.rope;
        float cv[AT_KV_MAX / 64];
#pragma unroll
        for (int k = 0; k < AT_KV_MAX / 64; k++) cv[k] = k < nk ? kc[lane + 64 * k] : 0.0f;
        const float pv = lane < a.rope ? kp[lane] : 0.0f;
        for (int h = 0; h < nh; h++) {
            float part = lane < a.rope ? __fmul_rn(qs[h][a.kv + lane], pv) : 0.0f;
#pragma unroll
            for (int k = 0; k < AT_KV_MAX / 64; k++)
                if (k < nk) part = fmaf(qs[h][lane + 64 * k], cv[k], part);
            const float sum = gv_reduce<64>(part);
            if (lane == 0) sc[h][t] = __fmul_rn(sum, a.kq_scale);
        }
    }
    __syncthreads();
    // per head: the chunk's maximum, exp(score - max) and their sum (lane = position)
    for (int h = w; h < nh; h += DM_BLOCK / 64) {
        const float v = lane < nt ? sc[h][lane] : -INFINITY;
        const float m = wave_max_dpp_f(v);
        const float e = lane < nt ? expf(__fsub_rn(v, m)) : 0.0f;
        const float l = gv_reduce<64>(e);
        sc[h][lane] = e;
        if (lane == 0) {
            a.part_ml[((size_t)c * a.H + h0 + h) * 2] = m;
            a.part_ml[((size_t)c * a.H + h0 + h) * 2 + 1] = l;
        }
    }
    __syncthreads();
    // the chunk's weighted sum of compressed entries: thread j owns entries j and j + 256
    float acc[AT_HG][AT_KV_MAX / DM_BLOCK];
#pragma unroll
    for (int h = 0; h < AT_HG; h++)
#pragma unroll
        for (int k = 0; k < AT_KV_MAX / DM_BLOCK; k++) acc[h][k] = 0.0f;
    for (int t = 0; t < nt; t++) {
        const float *kc = a.comp + (size_t)(t0 + t) * a.kv;
        float cv[AT_KV_MAX / DM_BLOCK];
#pragma unroll
        for (int k = 0; k < AT_KV_MAX / DM_BLOCK; k++) cv[k] = tid + DM_BLOCK * k < a.kv ? kc[tid + DM_BLOCK * k] : 0.0f;
#pragma unroll
        for (int h = 0; h < AT_HG; h++)
            if (h < nh)
#pragma unroll
                for (int k = 0; k < AT_KV_MAX / DM_BLOCK; k++) acc[h][k] = fmaf(sc[h][t], cv[k], acc[h][k]);
    }
#pragma unroll
    for (int h = 0; h < AT_HG; h++)
        if (h < nh)
#pragma unroll
            for (int k = 0; k < AT_KV_MAX / DM_BLOCK; k++)
                if (tid + DM_BLOCK * k < a.kv) a.part_ctx[((size_t)c * a.H + h0 + h) * a.kv + tid + DM_BLOCK * k] = acc[h][k];
}

// Head blockIdx.x: the chunks merged (each weighted by exp(its max - the overall max)) and
// divided by the total sum of exponentials: the softmax-weighted sum of compressed entries.
__global__ __launch_bounds__(DM_BLOCK) void k_attn_combine(AttnArgs a) {
    __shared__ float wgt[1024];
    __shared__ float red[DM_BLOCK / 64];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = blockIdx.x;
    const int nc = (a.pos + AT_CH) / AT_CH;  // chunks over positions 0 .. pos
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
    const float inv = __fdiv_rn(1.0f, l);
    for (int d = tid; d < a.kv; d += DM_BLOCK) {
        float s = 0.0f;
        for (int c = 0; c < nc; c++) s = fmaf(wgt[c], a.part_ctx[((size_t)c * a.H + h) * a.kv + d], s);
        a.ctx[(size_t)h * a.kv + d] = __fmul_rn(s, inv);
    }
}
