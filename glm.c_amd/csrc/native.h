// native.h -- the expert path for checkpoints in glm.c's own Q8_0 form: any group size that
// is a multiple of 16 and fp32 scales as the exporter writes them (scale = max|w| / 127,
// which fp16 cannot hold in general). The matrices stay in the checkpoint layout, int8
// [rows][cols] with fp32 scales [rows][cols/gs] (infer.c:707-739); a context in this form
// runs these kernels for every T (the tiled decode and prefill kernels assume gs = 32 and
// fp16-exact scales).
//
// A matrix row's dot product is one wave's: the row is cut into 16-column units, lane l
// takes units l and l + 64 (cols <= 2048), and a unit lies inside one group, so each unit's
// sum of q*x is scaled by its group's scale and accumulated (infer.c:765-786 sums a whole
// group before scaling; the order differs only in fp32 rounding). The activation units a
// lane needs are the same for every row, so they stay in its registers.
#pragma once

#include "common.h"

#define NV_BLOCK 256
#define NV_UNITS 2  // 16-column units per lane: cols <= 2048

struct NativeArgs {
    const uint8_t *experts;  // the layer's experts, expert e at e * stride (the shared one at E)
    size_t stride, off_gq, off_uq, off_dq, off_gs, off_us, off_ds;
    int D, F, E, K, S, gs, flags;
};

// Lane's units of a row of `cols` columns: 16 activations each from x (fp32, global).
__device__ static inline void nv_load_x(const float *x, int cols, float (&xv)[NV_UNITS][16]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int m = 0; m < NV_UNITS; m++) {
        const int u = lane + 64 * m;
        const bool on = u < (cols >> 4);
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
}

// One row's requests: the lane's units of int8 weights and their groups' scales.
struct NvRow {
    u32x4 q[NV_UNITS];
    float s[NV_UNITS];
};

__device__ static inline void nv_row_load(const int8_t *q, const float *s, int cols, int gs, NvRow &r) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int m = 0; m < NV_UNITS; m++) {
        const int u = lane + 64 * m, uc = u < (cols >> 4) ? u : 0;  // clamped; masked in nv_row_dot
        r.q[m] = *gbl((const u32x4 *)(q + 16 * (size_t)uc));
        r.s[m] = *gbl(s + (16 * uc) / gs);
    }
}

// The row's dot product with the lane's activation units, summed over the wave (every lane).
__device__ static inline float nv_row_dot(const NvRow &r, const float (&xv)[NV_UNITS][16], int cols) {
    const int lane = threadIdx.x & 63;
    float acc = 0.0f;
#pragma unroll
    for (int m = 0; m < NV_UNITS; m++) {
        const unsigned w[4] = {r.q[m].x, r.q[m].y, r.q[m].z, r.q[m].w};
        float part = 0.0f;
#pragma unroll
        for (int k = 0; k < 16; k++) part = fmaf((float)(int8_t)(w[k >> 2] >> (8 * (k & 3))), xv[m][k], part);
        if (lane + 64 * m < (cols >> 4)) acc = fmaf(part, r.s[m], acc);
    }
    acc = row_sum_dpp_f(acc);
    return (readlane_f(acc, 0) + readlane_f(acc, 16)) + (readlane_f(acc, 32) + readlane_f(acc, 48));
}

// Expert of slot s of token t: the routed slot's expert (or -1: none), E for the shared one.
__device__ static inline int nv_expert(const NativeArgs &a, const int *topk_idx, int t, int s) {
    if (s == a.K) return a.E;
    if (a.flags & GMOE_FLAG_NO_ROUTED) return -1;
    return topk_idx[(size_t)t * a.K + s];
}

// h[t][s][r] = silu(g_r) * u_r (infer.c:1184-1188, 1199-1202) for rows 16 bx .. 16 bx + 15 of
// slot s = by's expert, token t = bz; 0 for a slot without an expert. Wave w: 4 rows.
__global__ __launch_bounds__(NV_BLOCK) void k_native_gate_up(NativeArgs a, const float *__restrict__ xn,
                                                             const int *__restrict__ topk_idx, float *__restrict__ h) {
    const int s = blockIdx.y, t = blockIdx.z, w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int NS = a.K + a.S, D = a.D, F = a.F;
    const int e = nv_expert(a, topk_idx, t, s);
    const int r0 = 16 * blockIdx.x + 4 * w;
    float *hout = h + ((size_t)t * NS + s) * F;
    if (e < 0) {
        if (lane < 4) hout[r0 + lane] = 0.0f;
        return;
    }
    float xv[NV_UNITS][16];
    nv_load_x(xn + (size_t)t * D, D, xv);
    const uint8_t *base = a.experts + (size_t)e * a.stride;
    const int8_t *gq = (const int8_t *)(base + a.off_gq), *uq = (const int8_t *)(base + a.off_uq);
    const float *gsc = (const float *)(base + a.off_gs), *usc = (const float *)(base + a.off_us);
    const int ng = D / a.gs;
    NvRow rg[4], ru[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        nv_row_load(gq + (size_t)(r0 + i) * D, gsc + (size_t)(r0 + i) * ng, D, a.gs, rg[i]);
        nv_row_load(uq + (size_t)(r0 + i) * D, usc + (size_t)(r0 + i) * ng, D, a.gs, ru[i]);
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float g = nv_row_dot(rg[i], xv, D), u = nv_row_dot(ru[i], xv, D);
        if (lane == 0) hout[r0 + i] = g / (1.0f + expf(-g)) * u;
    }
}

// y[t][s][r] = down_e row r . h[t][s] (infer.c:1190, 1204) for rows 4 bx .. 4 bx + 3 (one per
// wave) of slot by, token bz; 0 for a slot without an expert.
__global__ __launch_bounds__(NV_BLOCK) void k_native_down(NativeArgs a, const float *__restrict__ h,
                                                          const int *__restrict__ topk_idx, float *__restrict__ y) {
    const int s = blockIdx.y, t = blockIdx.z, w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int NS = a.K + a.S, D = a.D, F = a.F;
    const int e = nv_expert(a, topk_idx, t, s), r = 4 * blockIdx.x + w;
    float *yout = y + ((size_t)t * NS + s) * D;
    if (e < 0) {
        if (lane == 0) yout[r] = 0.0f;
        return;
    }
    float xv[NV_UNITS][16];
    nv_load_x(h + ((size_t)t * NS + s) * F, F, xv);
    const uint8_t *base = a.experts + (size_t)e * a.stride;
    NvRow rd;
    nv_row_load((const int8_t *)(base + a.off_dq) + (size_t)r * F, (const float *)(base + a.off_ds) + (size_t)r * (F / a.gs),
                F, a.gs, rd);
    const float v = nv_row_dot(rd, xv, F);
    if (lane == 0) yout[r] = v;
}

// x_out = x_in + (shared + sum_k w_k y_k) per token in glm.c's order (infer.c:1192,
// 1212-1214), with the observables shared_out and routed_out.
__global__ __launch_bounds__(NV_BLOCK) void k_native_combine(NativeArgs a, const float *__restrict__ y,
                                                             const int *__restrict__ topk_idx,
                                                             const float *__restrict__ topk_ws, const float *x_in,
                                                             float *x_out, float *shared_out, float *routed_out) {
    const int t = blockIdx.y, r = blockIdx.x * NV_BLOCK + threadIdx.x, NS = a.K + a.S, D = a.D;
    if (r >= D) return;
    const float *yt = y + (size_t)t * NS * D;
    float acc = 0.0f;
    if (!(a.flags & GMOE_FLAG_NO_ROUTED)) {
        for (int k = 0; k < a.K; k++)
            if (topk_idx[(size_t)t * a.K + k] >= 0)
                acc = __fadd_rn(acc, __fmul_rn(topk_ws[(size_t)t * a.K + k], yt[(size_t)k * D + r]));
    }
    const float shv = a.S ? yt[(size_t)a.K * D + r] : 0.0f;
    const size_t o = (size_t)t * D + r;
    const float xo = __fadd_rn(x_in[o], __fadd_rn(shv, acc));
    shared_out[o] = shv;
    routed_out[o] = acc;
    x_out[o] = xo;
}
