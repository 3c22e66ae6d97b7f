// experts.h -- expert products for one token per block row: gate/up with SwiGLU
// (infer.c:1184-1188, 1197-1202) and down with the weighted combine and residual
// (infer.c:1190-1192, 1205, 1212-1214).
//
// Each block owns one 16-row panel of one expert matrix (or of gate and up together)
// and one token. Its four waves split the columns; each wave streams 1 KB chunks of
// the tiled q plane (one dwordx4 per lane) and feeds each 32-column block to
// v_mfma_i32_16x16x32_i8 with the activation digits as the A operand (rows 0..2 =
// digits, k = the block's 32 columns). Lanes 0..15 then rebuild that block's fp32 dot
// for their row and apply the fp16 block scale and the digit exponent.
#pragma once

#include "common.h"

struct ExpertArgs {
    const uint8_t *experts;  // layer base: expert e at experts + e * stride, shared expert at index E
    size_t stride;
    size_t off_gq, off_uq, off_dq, off_gs, off_us, off_ds;
    int D, F, E, K, S;
    int flags;
};

#define EX_BLOCK 256
#define EX_WAVES 4

// Digit form of n activations (n a multiple of 32) into shared memory:
// dig[j*n + i] = digit j of v[i], dexp[i/32] = block exponent.
__device__ static inline void load_digits(const float *__restrict__ v, int n, int8_t *dig, int *dexp) {
    for (int i0 = threadIdx.x * 8; i0 < n; i0 += EX_BLOCK * 8) {
        float vals[8];
        float mx = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            vals[k] = v[i0 + k];
            mx = fmaxf(mx, fabsf(vals[k]));
        }
        mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
        const int e = digit_exponent(mx);
        unsigned long long w0 = 0, w1 = 0, w2 = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            int8_t a, b, c;
            split_digits(vals[k], e, &a, &b, &c);
            w0 |= (unsigned long long)(uint8_t)a << (8 * k);
            w1 |= (unsigned long long)(uint8_t)b << (8 * k);
            w2 |= (unsigned long long)(uint8_t)c << (8 * k);
        }
        *(unsigned long long *)(dig + i0) = w0;
        *(unsigned long long *)(dig + n + i0) = w1;
        *(unsigned long long *)(dig + 2 * n + i0) = w2;
        if ((threadIdx.x & 3) == 0) dexp[i0 >> 5] = e;
    }
}

__device__ static inline long chunk_half(const u32x4 &c, int h) {
    return h == 0 ? (long)(((unsigned long long)c.y << 32) | c.x) : (long)(((unsigned long long)c.w << 32) | c.z);
}

// One block of 32 columns: the three digit dots of every weight row via one MFMA.
// Lanes 0..15 hold their row's dots in d[0..2]; the other lanes hold rows 4.. of the
// product, whose A rows are zero, so their d are zero.
__device__ static inline v4i mfma_digits(long A, long B) {
    const v4i zero = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, zero, 0, 0, 0);
}

// acc += (block dot) * fp16 scale * 2^dexp, on every lane without branching (lanes >= 16
// add zeros and are never read).
__device__ static inline void mfma_accumulate(const v4i &d, __half sc, int dexp, float &acc) {
    acc = fmaf(digits_to_float(d[0], d[1], d[2]), ldexpf(__half2float(sc), dexp), acc);
}

__device__ static inline void mfma_block(long A, long B, __half sc, int dexp, int lane, float &acc) {
    (void)lane;
    mfma_accumulate(mfma_digits(A, B), sc, dexp, acc);
}

// A wave's share of one 16-row panel: the chunks [w*cpw, (w+1)*cpw) of one or two
// matrices, cpw = cols/64/4 <= NB, and for lanes 0..15 (the panel's rows) the fp16
// scales of those chunks' blocks (two per chunk, one dword). All loads are issued
// together so a panel costs one memory latency.
template <int NMAT, int NB>
struct PanelRegs {
    u32x4 q[NMAT][NB];
    unsigned s[NMAT][NB];
};

template <int NMAT, int NB>
__device__ static inline void panel_load(PanelRegs<NMAT, NB> &r, const uint8_t *q0, const __half *s0,
                                         const uint8_t *q1, const __half *s1, int p, int cols) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int nchunks = cols >> 6, nblocks = cols >> 5, cpw = nchunks >> 2;
    const int j0 = w * cpw;
    const uint8_t *qs[2] = {q0, q1};
    const __half *ss[2] = {s0, s1};
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
        const GM_GLOBAL u32x4 *qp = gbl((const u32x4 *)(qs[m] + ((size_t)p * nchunks + j0) * GM_CHUNK_BYTES)) + lane;
        const GM_GLOBAL unsigned *sp = gbl((const unsigned *)(ss[m] + ((size_t)p * 16 + (lane & 15)) * nblocks + 2 * j0));
#pragma unroll
        for (int u = 0; u < NB; u++) {
            if (u < cpw) {
                r.q[m][u] = __builtin_nontemporal_load(qp + (size_t)u * 64);
                r.s[m][u] = lane < 16 ? __builtin_nontemporal_load(sp + u) : 0u;
            }
        }
    }
}

// Partial dot products of the wave's chunks with the activation digits `dig`
// ([3][cols] int8) and block exponents `dexp`; lanes 0..15 get their row's sums.
template <int NMAT, int NB>
__device__ static inline void panel_compute(const PanelRegs<NMAT, NB> &r, int cols, const int8_t *dig,
                                            const int *dexp, float *out) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int cpw = (cols >> 6) >> 2, j0 = w * cpw;
    const int m = lane & 15, kofs = 8 * (lane >> 4);
    float acc[NMAT];
#pragma unroll
    for (int i = 0; i < NMAT; i++) acc[i] = 0.0f;
#pragma unroll
    for (int u = 0; u < NB; u++) {
        if (u < cpw) {
            // Both blocks' digit rows and exponents are read before the first product, without
            // branches, so the shared-memory reads overlap. Lanes with m >= 3 read row 0 and
            // use zeros.
            long A[2];
            int de[2];
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const int b = 2 * (j0 + u) + hh;
                const long av = *(const long *)(dig + (m < 3 ? m : 0) * cols + 32 * b + kofs);
                A[hh] = m < 3 ? av : 0;
                de[hh] = dexp[b];
            }
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
#pragma unroll
                for (int i = 0; i < NMAT; i++) {
                    const unsigned sw = r.s[i][u];
                    const __half sc = __ushort_as_half((unsigned short)(hh ? (sw >> 16) : (sw & 0xffffu)));
                    mfma_block(A[hh], chunk_half(r.q[i][u], hh), sc, de[hh], lane, acc[i]);
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < NMAT; i++) out[i] = acc[i];
}

// The q chunks of panel_load without the scales, for callers that stage a panel's
// scales in shared memory with one wide load per lane (panel_compute_sc).
template <int NMAT, int NB>
__device__ static inline void panel_load_q(PanelRegs<NMAT, NB> &r, const uint8_t *q0, const uint8_t *q1, int p,
                                           int cols) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int nchunks = cols >> 6, cpw = nchunks >> 2;
    const int j0 = w * cpw;
    const uint8_t *qs[2] = {q0, q1};
    const GM_GLOBAL u32x4 *qp[2];
#pragma unroll
    for (int m = 0; m < NMAT; m++) qp[m] = gbl((const u32x4 *)(qs[m] + ((size_t)p * nchunks + j0) * GM_CHUNK_BYTES)) + lane;
    // chunk u of every matrix before chunk u + 1 of any: consumers can start on u early
#pragma unroll
    for (int u = 0; u < NB; u++)
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
            if (u < cpw) r.q[m][u] = __builtin_nontemporal_load(qp[m] + (size_t)u * 64);
            else r.q[m][u] = u32x4{0u, 0u, 0u, 0u};  // defined operands for branch-free consumers
        }
}

// panel_load_q without branches: exactly NB loads per matrix and wave whatever cols is
// (chunks past cpw reload the wave's first chunk; their scales must be zero), so that the
// compiler can wait for chunk u's loads alone.
template <int NMAT, int NB>
__device__ static inline void panel_load_q_all(PanelRegs<NMAT, NB> &r, const uint8_t *q0, const uint8_t *q1, int p,
                                               int cols) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int nchunks = cols >> 6, cpw = nchunks >> 2;
    const int j0 = w * cpw;
    const uint8_t *qs[2] = {q0, q1};
    const GM_GLOBAL u32x4 *qp[2];
#pragma unroll
    for (int m = 0; m < NMAT; m++) qp[m] = gbl((const u32x4 *)(qs[m] + ((size_t)p * nchunks + j0) * GM_CHUNK_BYTES)) + lane;
#pragma unroll
    for (int u = 0; u < NB; u++)
#pragma unroll
        for (int m = 0; m < NMAT; m++) r.q[m][u] = __builtin_nontemporal_load(qp[m] + (size_t)(u < cpw ? u : 0) * 64);
}

// panel_compute with the panel's fp16 scales in shared memory: sc[m] holds matrix m's
// [16 rows][cols/32] scales of the panel.
template <int NMAT, int NB>
__device__ static inline void panel_compute_sc(const PanelRegs<NMAT, NB> &r, int cols, const int8_t *dig,
                                               const int *dexp, const unsigned short *const *sc, float *out) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int cpw = (cols >> 6) >> 2, j0 = w * cpw, nblocks = cols >> 5;
    const int m = lane & 15, kofs = 8 * (lane >> 4);
    float acc[NMAT];
#pragma unroll
    for (int i = 0; i < NMAT; i++) acc[i] = 0.0f;
#pragma unroll
    for (int u = 0; u < NB; u++) {
        if (u < cpw) {
            long A[2];
            int de[2];
            unsigned short sv[NMAT][2];
#pragma unroll
            for (int hh = 0; hh < 2; hh++) {
                const int b = 2 * (j0 + u) + hh;
                const long av = *(const long *)(dig + (m < 3 ? m : 0) * cols + 32 * b + kofs);
                A[hh] = m < 3 ? av : 0;
                de[hh] = dexp[b];
#pragma unroll
                for (int i = 0; i < NMAT; i++) sv[i][hh] = sc[i][m * nblocks + b];
            }
            v4i d[2][NMAT];
#pragma unroll
            for (int hh = 0; hh < 2; hh++)
#pragma unroll
                for (int i = 0; i < NMAT; i++) d[hh][i] = mfma_digits(A[hh], chunk_half(r.q[i][u], hh));
#pragma unroll
            for (int hh = 0; hh < 2; hh++)
#pragma unroll
                for (int i = 0; i < NMAT; i++) mfma_accumulate(d[hh][i], __ushort_as_half(sv[i][hh]), de[hh], acc[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < NMAT; i++) out[i] = acc[i];
}

// Column tiling used by the expert kernels: cols/64 chunks split evenly over 4 waves.
#define EX_NB_MAX 8  // chunks per wave in registers: cols <= 2048

// One 16-row panel p of a down matrix in the column-slice layout. Each wave takes the
// 32-column blocks [w*bpw, (w+1)*bpw); for block b, lane l holds the MFMA B operand:
// row 16p + l%16, columns 32b + 8*(l/16) .. +8, which is 8 bytes of slice 2b + (l/32).
// Lanes 0..15 also hold their row's fp16 scale of block b.
#define EX_BB_MAX 16  // blocks per wave: cols <= 2048
template <int NB>
struct SliceRegs {
    unsigned long long q[NB];
    unsigned short s[NB];
};

template <int NB>
__device__ static inline void slice_panel_load(SliceRegs<NB> &r, const uint8_t *q, const __half *s, int p, int rows,
                                               int cols) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int bpw = (cols >> 5) >> 2, b0 = w * bpw;
    const int row = p * 16 + (lane & 15), kq = lane >> 4;
    const GM_GLOBAL uint8_t *qg = gbl(q) + (size_t)row * 16 + 8 * (kq & 1);
    const GM_GLOBAL unsigned short *sg = gbl((const unsigned short *)s) + row;
#pragma unroll
    for (int u = 0; u < NB; u++) {
        if (u < bpw) {
            const int b = b0 + u;
            r.q[u] = __builtin_nontemporal_load((const GM_GLOBAL unsigned long long *)(qg + (size_t)(2 * b + (kq >> 1)) * rows * 16));
            r.s[u] = lane < 16 ? sg[(size_t)b * rows] : (unsigned short)0;
        }
    }
}

// Partial dots of the wave's blocks with the activation digits; lanes 0..15 get their row's sum.
template <int NB>
__device__ static inline float slice_panel_compute(const SliceRegs<NB> &r, int cols, const int8_t *dig,
                                                   const int *dexp) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int bpw = (cols >> 5) >> 2, b0 = w * bpw;
    const int m = lane & 15, kofs = 8 * (lane >> 4);
    float acc = 0.0f;
#pragma unroll
    for (int u = 0; u < NB; u++) {
        if (u < bpw) {
            const int b = b0 + u;
            const long av = *(const long *)(dig + (m < 3 ? m : 0) * cols + 32 * b + kofs);
            mfma_block(m < 3 ? av : 0, (long)r.q[u], __ushort_as_half(r.s[u]), dexp[b], lane, acc);
        }
    }
    return acc;
}

// grid (F/16, K+S, T): h[t][slot][F] = silu(gate . xn) * (up . xn) for the slot's expert.
__global__ __launch_bounds__(EX_BLOCK) void k_gate_up(ExpertArgs a, const float *__restrict__ xn,
                                                      const int *__restrict__ topk_idx, float *__restrict__ h) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float part[EX_WAVES][2][16];
    const int p = blockIdx.x, slot = blockIdx.y, t = blockIdx.z;
    const int D = a.D, F = a.F, K = a.K, nslots = a.K + a.S;
    int e = a.E;
    if (slot < K) {
        if (a.flags & 1) return;
        e = topk_idx[(size_t)t * K + slot];
        if (e < 0) return;
    }
    int8_t *dig = (int8_t *)smem;
    int *dexp = (int *)(smem + 3 * D);
    const uint8_t *base = a.experts + (size_t)e * a.stride;
    PanelRegs<2, EX_NB_MAX> pr;
    panel_load<2, EX_NB_MAX>(pr, base + a.off_gq, (const __half *)(base + a.off_gs), base + a.off_uq,
                             (const __half *)(base + a.off_us), p, D);
    load_digits(xn + (size_t)t * D, D, dig, dexp);
    __syncthreads();
    float gu[2];
    panel_compute<2, EX_NB_MAX>(pr, D, dig, dexp, gu);
    const float g = gu[0], u = gu[1];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane < 16) {
        part[w][0][lane] = g;
        part[w][1][lane] = u;
    }
    __syncthreads();
    if (threadIdx.x < 16) {
        const int l = threadIdx.x;
        const float gs = ((part[0][0][l] + part[1][0][l]) + part[2][0][l]) + part[3][0][l];
        const float us = ((part[0][1][l] + part[1][1][l]) + part[2][1][l]) + part[3][1][l];
        const float act = gs / (1.0f + expf(-gs));
        h[((size_t)t * nslots + slot) * F + (size_t)p * 16 + l] = act * us;
    }
}

struct CombineArgs {
    const int *topk_idx;      // [T][K]
    const float *topk_ws;     // [T][K] weights * routed_scale
    float *y;                 // [T][K+S][D] per-slot down outputs
    unsigned *panel_counter;  // [T][D/16], zero between launches
    const float *x_in;        // [T][D]
    float *x_out;             // [T][D]
    float *shared_out;        // [T][D]
    float *routed_out;        // [T][D]
};

// grid (D/16, K+S, T): y[t][slot] = down . h[t][slot]; the last slot block of each
// (token, panel) forms x_out = x_in + (shared + sum_k w_k y_k) for the panel's rows.
__global__ __launch_bounds__(EX_BLOCK) void k_down_combine(ExpertArgs a, CombineArgs c, const float *__restrict__ h) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float part[EX_WAVES][16];
    __shared__ int s_last;
    const int p = blockIdx.x, slot = blockIdx.y, t = blockIdx.z;
    const int D = a.D, F = a.F, K = a.K, nslots = a.K + a.S;
    const int routed_on = !(a.flags & 1);
    int e = a.E;
    bool valid = true;
    if (slot < K) {
        e = c.topk_idx[(size_t)t * K + slot];
        valid = routed_on && e >= 0;
    }
    if (valid) {
        int8_t *dig = (int8_t *)smem;
        int *dexp = (int *)(smem + 3 * F);
        const uint8_t *base = a.experts + (size_t)e * a.stride;
        SliceRegs<EX_BB_MAX> sr;
        slice_panel_load<EX_BB_MAX>(sr, base + a.off_dq, (const __half *)(base + a.off_ds), p, D, F);
        load_digits(h + ((size_t)t * nslots + slot) * F, F, dig, dexp);
        __syncthreads();
        const float yv = slice_panel_compute<EX_BB_MAX>(sr, F, dig, dexp);
        const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
        if (lane < 16) part[w][lane] = yv;
        __syncthreads();
        if (threadIdx.x < 16) {
            const int l = threadIdx.x;
            c.y[((size_t)t * nslots + slot) * D + (size_t)p * 16 + l] =
                ((part[0][l] + part[1][l]) + part[2][l]) + part[3][l];
        }
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = (atomicAdd(&c.panel_counter[(size_t)t * (D >> 4) + p], 1u) == (unsigned)(nslots - 1));
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    if (threadIdx.x == 0) c.panel_counter[(size_t)t * (D >> 4) + p] = 0u;
    if (threadIdx.x < 16) {
        const int r = p * 16 + threadIdx.x;
        float acc = 0.0f;
        if (routed_on) {
            for (int k = 0; k < K; k++) {
                if (c.topk_idx[(size_t)t * K + k] < 0) continue;
                const float yk = c.y[((size_t)t * nslots + k) * D + r];
                acc = __fadd_rn(acc, __fmul_rn(c.topk_ws[(size_t)t * K + k], yk));
            }
        }
        const float sh = a.S ? c.y[((size_t)t * nslots + K) * D + r] : 0.0f;
        const size_t o = (size_t)t * D + r;
        c.routed_out[o] = acc;
        c.shared_out[o] = sh;
        c.x_out[o] = __fadd_rn(c.x_in[o], __fadd_rn(sh, acc));
    }
}
