// gemm.h -- the dense Q8_0 products of a prefill batch (matvec_q80_rows, infer.c:765-786,
// for every token of the batch) as MFMA GEMMs: each weight panel is read once per tile of
// up to QG_TT tokens instead of once per token.
//
//   k_norm_split  each token's input row, normalised as glm.c normalises it when the
//                 product takes rmsnorm(x) * w (infer.c:746-752), in the split form of the
//                 grouped expert GEMMs (grouped.h): fp16 hi and lo with one exponent per row;
//   k_gemm_q8     y[t][r] = sum_g s[r][g] * (q[r][g] . x_t[g]) for a tile of 64 rows of the
//                 matrix (four waves of 16) and up to QG_TT tokens, with epilogues for glm.c's
//                 SwiGLU pair (infer.c:1078-1080) and residual add (infer.c:1061, 1083).
//
// Weights stay in glm.c's row-major Q8_0 form with fp32 scales, which the decode products
// (dense.h) read too. Per 32-column block (v_mfma_f32_16x16x32_f16, group sizes that are
// multiples of 32) or 16-column group (v_mfma_f32_16x16x16_f16, group size 16): the
// block's int8 weights converted to fp16 exactly, two MFMAs (hi, then lo of the inputs)
// into one fp32 accumulator, and one fma applying the group's fp32 scale into the running
// fp32 sum; 2^e at the end. The inputs carry 22 significant bits, so each product is
// within ~2^-21 of fp32's.
//
// Per-head products (k_b and v_b, whose row groups of x_rows rows read their own slice of
// the input, x_stride apart) run as groups: a block's rows lie inside one group.
//
// Block order is XCD-aware: the blocks of one 64-row panel (its token tiles) are dispatched
// on one XCD in a row, so the panel is fetched from HBM once and then read from that XCD's L2.
#pragma once

#include <type_traits>

#include "common.h"

#define QG_BLOCK 256
#define QG_TT 32                // tokens per tile (two A tiles of 16): twice the blocks of 64-token
                                // tiles, which leave most CUs idle at a 512-token batch's small matrices
#define QG_KC 64                // columns per staged chunk
#define QG_RB (QG_KC * 2)       // bytes of one staged row (one plane of one token)
#define QG_RG (QG_RB / 16)      // 16-byte groups per staged row
#define QG_XCD 8                // XCDs the dispatcher deals blocks over, round robin
#define QG_GEMM_MIN_TOKENS 8    // smaller batches take the per-token products (dense.h)

enum { QG_PLAIN = 0, QG_RESID = 1, QG_PAIR = 2 };

struct QgArgs {
    const int8_t *q, *q2;      // [rows][cols] int8 (q2: up, for QG_PAIR)
    const float *s, *s2;       // [rows][cols / gs] fp32 scales
    const __half *xs;          // split inputs [n][2][xcols]: hi, lo
    const int *xe;             // [n] their exponents
    const __half *zeros;       // 16 bytes of zeros (staged past the last column)
    float *y;                  // y[t * ldy + r]
    const float *resid;        // QG_RESID: y = resid[t * ldr + r] + dot
    int rows, cols, gs, n, xcols, ldy, ldr;
    int x_rows, x_stride;      // row group g (x_rows rows) reads split columns g * x_stride ..
    int bpg, groups, tiles;    // 64-row blocks per group, groups, token tiles
};

typedef _Float16 qg_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 qg_h4 __attribute__((ext_vector_type(4)));
typedef float qg_f4 __attribute__((ext_vector_type(4)));
typedef float qg_f2 __attribute__((ext_vector_type(2)));
typedef unsigned qg_u2 __attribute__((ext_vector_type(2)));

// ---- the inputs' split form ---------------------------------------------------------

// One block per token row t of x (row t at x + t * ldx, n columns, n a multiple of 8):
// v = rmsnorm(x) * norm when norm is given (glm.c's operations: fp64 sum of squares, fp32
// mean, 1 / sqrtf of mean + 1e-5, then (x * inv) * w), else v = x; then
// sp[t][0][:] = fp16(v 2^-e), sp[t][1][:] = fp16(v 2^-e - hi), ex[t] = e, with e from
// max |v| so that the row's largest value sits near 2^14.
#define QG_SPLIT_MAX 40  // row values a thread holds: rows of up to 40 x QG_BLOCK = 10240 columns
// NK: the values a thread holds (n <= NK x QG_BLOCK; the launch takes the fewest of 2, 8,
// 20, 40 that hold the row, so a 2048-column row issues 8 loads a thread, not 40; the
// values past n add nothing, so every NK gives the same bits)
template <int NK>
__global__ __launch_bounds__(QG_BLOCK) void k_norm_split(const float *__restrict__ x, int ldx, int n,
                                                         const float *__restrict__ norm, __half *__restrict__ sp,
                                                         int *__restrict__ ex) {
    __shared__ double red_d[QG_BLOCK / 64];
    __shared__ float red_f[QG_BLOCK / 64];
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const float *src = x + (size_t)t * ldx;
    // the row read once: thread tid holds columns tid + QG_BLOCK k
    float v[NK], nw[NK];
#pragma unroll
    for (int k = 0; k < NK; k++) {
        const int i = tid + QG_BLOCK * k;
        v[k] = i < n ? src[i] : 0.0f;
        nw[k] = norm && i < n ? norm[i] : 0.0f;
    }
    float inv = 1.0f;
    if (norm) {
        double ss = 0.0;
#pragma unroll
        for (int k = 0; k < NK; k++)
            if (tid + QG_BLOCK * k < n) ss += (double)v[k] * (double)v[k];
        ss = wave_sum_dpp(ss);
        if (lane == 0) red_d[w] = ss;
        __syncthreads();
        ss = (red_d[0] + red_d[1]) + (red_d[2] + red_d[3]);
        const float mean = (float)(ss / (double)n);
        inv = __fdiv_rn(1.0f, sqrt_rn_f32(__fadd_rn(mean, 1e-5f)));
#pragma unroll
        for (int k = 0; k < NK; k++) v[k] = __fmul_rn(__fmul_rn(v[k], inv), nw[k]);
    }
    float mx = 0.0f;
#pragma unroll
    for (int k = 0; k < NK; k++)
        if (tid + QG_BLOCK * k < n) mx = fmaxf(mx, fabsf(v[k]));
    mx = wave_max_f(mx);
    if (lane == 0) red_f[w] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red_f[0], red_f[1]), fmaxf(red_f[2], red_f[3]));
    int e = 0;
    if (mx > 0.0f && isfinite(mx)) {
        int k;
        (void)frexpf(mx, &k);
        e = k - 14;
    }
    if (tid == 0) ex[t] = e;
    __half *hi = sp + (size_t)t * 2 * n, *lo = hi + n;
#pragma unroll
    for (int k = 0; k < NK; k++) {
        const int i = tid + QG_BLOCK * k;
        if (i < n) {
            const float xs = ldexpf(v[k], -e);
            const __half h = __float2half_rn(xs);
            hi[i] = h;
            lo[i] = __float2half_rn(xs - __half2float(h));
        }
    }
}

// ---- the GEMM -----------------------------------------------------------------------

// Eight (or four) int8 weights as fp16, exactly: byte b becomes the fp16 with bits
// 0x64 (b ^ 0x80) = 1152 + q, and one packed subtract removes the 1152.
__device__ static inline unsigned qg_pair(unsigned u, unsigned sel) {
    return __builtin_amdgcn_perm(0x64646464u, u ^ 0x80808080u, sel);
}
__device__ static inline qg_h8 qg_i8_to_h8(unsigned lo, unsigned hi) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 off = {(_Float16)1152.0f, (_Float16)1152.0f};
    const unsigned w[4] = {qg_pair(lo, 0x07010700u), qg_pair(lo, 0x07030702u), qg_pair(hi, 0x07010700u),
                           qg_pair(hi, 0x07030702u)};
    qg_h8 r;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const h2 v = __builtin_bit_cast(h2, w[k]) - off;
        r[2 * k] = v[0];
        r[2 * k + 1] = v[1];
    }
    return r;
}
__device__ static inline qg_h4 qg_i8_to_h4(unsigned u) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 off = {(_Float16)1152.0f, (_Float16)1152.0f};
    const h2 a = __builtin_bit_cast(h2, qg_pair(u, 0x07010700u)) - off;
    const h2 b = __builtin_bit_cast(h2, qg_pair(u, 0x07030702u)) - off;
    qg_h4 r = {a[0], a[1], b[0], b[1]};
    return r;
}

// 4 bytes from global memory into shared memory: lane l's at dst + 4 l, by a DMA that the
// compiler does not count (the caller waits on vmcnt).
__device__ static inline void dma4_untracked(const GM_GLOBAL void *src, lds_void *dst) {
    const unsigned m0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)dst);
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(m0) : "memory", "m0");
}

// One stage of the chunk pipeline in shared memory: every operand of a chunk of QG_KC
// columns arrives by DMA that the compiler does not track, so its only waits are the
// pipeline's exact vmcnt counts. (Weights loaded into registers instead make the compiler
// wait, at the pipeline loop's join, for every outstanding load, the next chunk's
// included.)
//   act  [QG_TT tokens][2 planes][QG_KC] fp16, row r = 2 token + plane, its 16-byte groups
//        XOR-swizzled by token % 8 so that an A-operand read (16 tokens) spreads over the banks;
//   w    [NM matrices][64 rows][QG_KC] int8, row r's 16-byte groups swizzled by (r / 4) % 4;
//   s    [NM][256] fp32: row r's scales of the chunk's NB blocks at r NB + b.
template <int NM>
struct QgStageBuf {
    uint8_t act[QG_TT * 2 * QG_RB];
    uint8_t w[NM][64 * QG_KC];
    float s[NM][QG_BLOCK];
};

// Per-thread sources of a tile's DMA: NA activation slots (16 bytes), and for each matrix
// one weight slot (16 bytes of row t / 4 of the panel) and one scale slot (4 bytes).
template <int NA>
struct QgSrc {
    const __half *act[NA];  // the slot's activation row at column 0
    int act_col[NA];        // the slot's first column within a chunk
    int w_row, w_col;       // panel row (clamped) and column of the weight slot within a chunk
    int s_row, s_blk;       // panel row (clamped) and block of the scale slot
};

template <int NA, int KB>
__device__ static inline QgSrc<NA> qg_src_init(const QgArgs &a, int t0, int c_off, int row0, int nrows) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    QgSrc<NA> g;
#pragma unroll
    for (int it = 0; it < NA; it++) {
        const int s = 64 * w + QG_BLOCK * it + lane, r = s / QG_RG, p = s % QG_RG, tok = r >> 1;
        const int j = p ^ (tok & 7);  // the slot holds logical group j of its row
        const int t = t0 + tok < a.n ? t0 + tok : a.n - 1;
        g.act[it] = a.xs + ((size_t)t * 2 + (r & 1)) * a.xcols + c_off;
        g.act_col[it] = 8 * j;
    }
    const int wr = tid >> 2, wg = (tid & 3) ^ ((wr >> 2) & 3);  // slot tid holds group wg of row wr
    g.w_row = row0 + (wr < nrows ? wr : 0);
    g.w_col = 16 * wg;
    constexpr int NB = QG_KC / KB;
    const int sr = tid / NB;
    g.s_row = row0 + (sr < nrows ? sr : 0);  // slots past the panel's 64 rows (NB = 2) load row 0
    g.s_blk = tid % NB;
    return g;
}

template <int NA, int KB, int NM>
__device__ static inline void qg_issue(const QgArgs &a, const QgSrc<NA> &g, QgStageBuf<NM> &sb, int c0) {
    const int w = threadIdx.x >> 6;
#pragma unroll
    for (int it = 0; it < NA; it++) {
        const int c = c0 + g.act_col[it];
        const __half *src = c < a.cols ? g.act[it] + c : a.zeros;  // past the last column: zeros
        dma16_untracked(gbl((const void *)src), (lds_void *)(sb.act + 16 * (64 * w + QG_BLOCK * it)));
    }
    const int ng = a.cols / a.gs;
    const int cw = c0 + g.w_col < a.cols ? c0 + g.w_col : 0;  // past the last column: any weights
    const int cs = c0 + KB * g.s_blk;
    const int gi = cs < a.cols ? cs / a.gs : 0;
#pragma unroll
    for (int m = 0; m < NM; m++) {
        const int8_t *q = m ? a.q2 : a.q;
        const float *s = m ? a.s2 : a.s;
        dma16_untracked(gbl((const void *)(q + (size_t)g.w_row * a.cols + cw)), (lds_void *)(sb.w[m] + 1024 * w));
        dma4_untracked(gbl((const void *)(s + (size_t)g.s_row * ng + gi)), (lds_void *)(sb.s[m] + 64 * w));
    }
}

// KB = 32: A operand of A tile i, plane pl, block b of the chunk: lane l holds token
// 16 i + l % 16, columns 32 b + 8 (l / 16) .. +8.
__device__ static inline qg_h8 qg_a8(const uint8_t *act, int i, int pl, int b) {
    const int lane = threadIdx.x & 63, tok = 16 * i + (lane & 15), r = 2 * tok + pl;
    const int j = 4 * b + (lane >> 4), p = j ^ (tok & 7);
    return *(const qg_h8 *)(act + r * QG_RB + 16 * p);
}
// KB = 16: columns 16 b + 4 (l / 16) .. +4.
__device__ static inline qg_h4 qg_a4(const uint8_t *act, int i, int pl, int b) {
    const int lane = threadIdx.x & 63, tok = 16 * i + (lane & 15), r = 2 * tok + pl;
    const int col = 16 * b + 4 * (lane >> 4), j = col >> 3, p = j ^ (tok & 7);
    return *(const qg_h4 *)(act + r * QG_RB + 16 * p + 2 * (col & 7));
}
// The lane's weight bytes of panel row r, columns c .. c + n (n = 8 or 4, inside a group).
__device__ static inline const uint8_t *qg_w(const uint8_t *w, int r, int c) {
    const int g = (c >> 4) ^ ((r >> 2) & 3);
    return w + r * QG_KC + 16 * g + (c & 15);
}

template <int NA, int KB>
__device__ static inline void qg_mma(const uint8_t *act, const uint8_t *wm, const float *sm, const QgArgs &a, int c0,
                                     int r, float (*acc)[4]) {
    const qg_f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    const int lane = threadIdx.x & 63;
    constexpr int NB = QG_KC / KB;
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const float sc = c0 + KB * b < a.cols ? sm[r * NB + b] : 0.0f;
        if (KB == 32) {
            const qg_u2 q = *(const qg_u2 *)qg_w(wm, r, 32 * b + 8 * (lane >> 4));
            const qg_h8 B = qg_i8_to_h8(q.x, q.y);
#pragma unroll
            for (int i = 0; i < NA; i++) {
                qg_f4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(qg_a8(act, i, 0, b), B, zero, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(qg_a8(act, i, 1, b), B, d, 0, 0, 0);
#pragma unroll
                for (int k = 0; k < 4; k++) acc[i][k] = fmaf(d[k], sc, acc[i][k]);
            }
        } else {
            const unsigned q = *(const unsigned *)qg_w(wm, r, 16 * b + 4 * (lane >> 4));
            const qg_h4 B = qg_i8_to_h4(q);
#pragma unroll
            for (int i = 0; i < NA; i++) {
                qg_f4 d = __builtin_amdgcn_mfma_f32_16x16x16f16(qg_a4(act, i, 0, b), B, zero, 0, 0, 0);
                d = __builtin_amdgcn_mfma_f32_16x16x16f16(qg_a4(act, i, 1, b), B, d, 0, 0, 0);
#pragma unroll
                for (int k = 0; k < 4; k++) acc[i][k] = fmaf(d[k], sc, acc[i][k]);
            }
        }
    }
}

// The tile of block (panel, token tile): wave w takes rows 16 w .. +16 of the panel. The
// chunks run double-buffered: chunk kc + 1's operands are requested before chunk kc is
// multiplied; each step waits for exactly the loads issued before the prefetch (vmcnt)
// and then on the block (s_barrier), so the prefetch stays in flight.
template <int NA, int KB, int MODE, int NM>
__device__ __attribute__((always_inline)) static void qg_tile(const QgArgs &a, int panel, int tt,
                                                             QgStageBuf<NM> (&buf)[2]) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int g = panel / a.bpg, rb = panel % a.bpg;
    const int row0 = g * a.x_rows + 64 * rb;                         // the panel's first row
    const int left = min(a.x_rows - 64 * rb, a.rows - row0);
    const int nrows = left < 64 ? left : 64;                         // its rows (of 64)
    const int pr = 16 * w + (lane & 15);                             // the lane's panel row
    const bool row_on = pr < nrows;
    const int t0 = QG_TT * tt;
    const QgSrc<NA> src = qg_src_init<NA, KB>(a, t0, g * a.x_stride, row0, nrows);
    constexpr int LOADS = NA + 2 * NM;  // DMA per chunk and thread
    float acc[NA][4], acc2[NA][4];
#pragma unroll
    for (int i = 0; i < NA; i++)
#pragma unroll
        for (int k = 0; k < 4; k++) acc[i][k] = acc2[i][k] = 0.0f;
    const int nkc = (a.cols + QG_KC - 1) / QG_KC;
    auto compute = [&](const QgStageBuf<NM> &sb, int kc) {
        qg_mma<NA, KB>(sb.act, sb.w[0], sb.s[0], a, kc * QG_KC, pr, acc);
        if (NM == 2) qg_mma<NA, KB>(sb.act, sb.w[NM - 1], sb.s[NM - 1], a, kc * QG_KC, pr, acc2);
    };
    qg_issue<NA, KB, NM>(a, src, buf[0], 0);
    for (int kc = 0; kc < nkc; kc++) {
        if (kc + 1 < nkc) {
            qg_issue<NA, KB, NM>(a, src, buf[(kc + 1) & 1], (kc + 1) * QG_KC);
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LOADS) : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        __builtin_amdgcn_s_barrier();  // every wave's part of chunk kc has landed
        compute(buf[kc & 1], kc);
        __builtin_amdgcn_s_barrier();  // every wave is done with the stage before its refill
    }
    // lane l holds tokens 16 i + 4 (l / 16) + k of panel row pr
    const int r = row0 + pr;
#pragma unroll
    for (int i = 0; i < NA; i++)
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int t = t0 + 16 * i + 4 * (lane >> 4) + k;
            if (row_on && t < a.n) {
                const int e = a.xe[t];
                const float v = ldexpf(acc[i][k], e);
                float out;
                if (MODE == QG_PAIR) {
                    const float u = ldexpf(acc2[i][k], e);
                    out = v / (1.0f + expf(-v)) * u;  // infer.c:1078-1080
                } else if (MODE == QG_RESID) {
                    out = a.resid[(size_t)t * a.ldr + r] + v;  // infer.c:1061, 1083
                } else {
                    out = v;
                }
                a.y[(size_t)t * a.ldy + r] = out;
            }
        }
}

// f(NA) with NA the tile's A-tile count (1..4, block-uniform) as a compile-time constant.
template <int N, typename Body>
__device__ __attribute__((always_inline)) static inline void qg_with_na(int na, Body &&f) {
    if constexpr (N > 1) {
        if (na < N) {
            qg_with_na<N - 1>(na, f);
            return;
        }
    }
    f(std::integral_constant<int, N>{});
}

// Grid: one block per (64-row panel, token tile), in XCD-aware order: linear block id b
// runs on XCD b % 8, which takes panels xcd, xcd + 8, ... (its weights stay in its L2); its
// blocks take token tile 0 for each of those panels, then tile 1, ..., so that the blocks
// resident together share their tokens' inputs in L2 (walking one panel's tiles before the
// next streamed the whole input once per panel: 603 MB fetched per attn_out call of a
// 1024-token batch, for 31.5 MB of weights and inputs).
template <int KB, int MODE>
__global__ __launch_bounds__(QG_BLOCK) void k_gemm_q8(QgArgs a) {
    constexpr int NM = MODE == QG_PAIR ? 2 : 1;
    __shared__ __align__(16) QgStageBuf<NM> buf[2];
    const int b = blockIdx.x, xcd = b % QG_XCD, k = b / QG_XCD;
    const int ppx = (a.bpg * a.groups + QG_XCD - 1) / QG_XCD;  // panels per XCD
    const int panel = (k % ppx) * QG_XCD + xcd, tt = k / ppx;
    if (panel >= a.bpg * a.groups) return;
    const int left = a.n - QG_TT * tt;
    const int na = __builtin_amdgcn_readfirstlane(left >= QG_TT ? QG_TT / 16 : (left + 15) >> 4);
    qg_with_na<QG_TT / 16>(na, [&](auto NA) { qg_tile<decltype(NA)::value, KB, MODE, NM>(a, panel, tt, buf); });
}
