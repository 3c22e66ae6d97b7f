// grouped.h -- prefill (T > 1): the expert products as grouped GEMMs over the per-expert
// token lists (lists that glm.c never materialises, since it routes prompt tokens one at
// a time, infer.c:2190-2233).
//
// Per layer: the router (router.h) and the dispatch (dispatch.h, which also cuts every
// list into tiles of GP_TOK tokens) run first. Then
//   k_act_split    xn of every token as fp16 hi/lo with one exponent per token;
//   k_group_gu     per (tile, 64 rows of F): g and u for the tile's tokens (fp16 MFMA,
//                  fp32 scale per 32-column block), h = silu(g) * u (infer.c:1184-1188,
//                  1199-1202), stored per list row;
//   k_act_split    h in the same form;
//   k_group_down   per (tile, 64 rows of D): y = down . h for the tile's tokens
//                  (infer.c:1190, 1205), stored per list row;
//   k_token_combine  x' = x + (shared + sum_k w_k y_k) per token, in glm.c's order
//                  (infer.c:1192, 1212-1214).
// Each expert's weights are read once per tile (once for the typical expert, whose list
// fits one tile), so the layer reads the touched experts' 10 MB each, not T times.
//
// Arithmetic: fp16 MFMA (v_mfma_f32_16x16x32_f16) with fp32 accumulation. A row v (xn
// of a token, or h of one list row) is scaled by 2^-e (e from max|v|, so the row's
// maximum sits near 2^14) and split into fp16 hi = fp16(v 2^-e) and lo = fp16(v 2^-e -
// hi): 22 bits per element. The int8 weights are exact in fp16 (converted in registers
// by a byte permute into 1024 + q + 128 and one packed subtract), so a 32-column block's
// two MFMAs (hi, then lo into the same accumulator) give its dot in fp32, which one
// v_fma_mix scales by the block's fp16 scale into the running fp32 sum; 2^e is applied
// once at the end. Errors are ~2^-22 of each element, fp32-like.
#pragma once

#include <type_traits>

#include "common.h"
#include "dispatch.h"
#include "experts.h"

#define GP_KC 128             // columns per K chunk staged in shared memory
#define GP_NB (GP_KC / 32)    // quant blocks per chunk
#define GP_BLOCK 256
#define GP_OCC 3              // blocks per CU the GEMMs are built for (32 KB of LDS each)

// Split form of `rows` rows of n values (n a multiple of 8): sp[r][0][:] = hi and
// sp[r][1][:] = lo (fp16), ex[r] the exponent. One block per row; rows past *n_rows
// (when given) are skipped.
__global__ __launch_bounds__(GP_BLOCK) void k_act_split(const float *__restrict__ v, int n, int rows,
                                                        const int *__restrict__ n_rows, __half *__restrict__ sp,
                                                        int *__restrict__ ex) {
    __shared__ float red[GP_BLOCK / 64];
    const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    if (r >= (n_rows ? *n_rows : rows)) return;
    const float *src = v + (size_t)r * n;
    float mx = 0.0f;
    for (int i = tid * 8; i < n; i += GP_BLOCK * 8) {
        const float4 a = *(const float4 *)(src + i), b = *(const float4 *)(src + i + 4);
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
    }
    mx = wave_max_f(mx);
    if (lane == 0) red[w] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e = 0;
    if (mx > 0.0f && isfinite(mx)) {
        int k;
        (void)frexpf(mx, &k);  // mx < 2^k
        e = k - 14;            // the scaled row stays below 2^14
    }
    if (tid == 0) ex[r] = e;
    __half *hi = sp + (size_t)r * 2 * n, *lo = hi + n;
    for (int i = tid * 8; i < n; i += GP_BLOCK * 8) {
        const float4 a = *(const float4 *)(src + i), b = *(const float4 *)(src + i + 4);
        const float xs[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        unsigned hw[4], lw[4];  // eight halves of each plane, one 16-byte store each
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float x0 = ldexpf(xs[2 * k], -e), x1 = ldexpf(xs[2 * k + 1], -e);
            const __half h0 = __float2half_rn(x0), h1 = __float2half_rn(x1);
            const __half l0 = __float2half_rn(x0 - __half2float(h0)), l1 = __float2half_rn(x1 - __half2float(h1));
            hw[k] = (unsigned)__half_as_ushort(h0) | ((unsigned)__half_as_ushort(h1) << 16);
            lw[k] = (unsigned)__half_as_ushort(l0) | ((unsigned)__half_as_ushort(l1) << 16);
        }
        *(uint4 *)(hi + i) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        *(uint4 *)(lo + i) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
    }
}

struct GroupArgs {
    const uint8_t *experts;  // layer base: expert e at experts + e * stride, shared at E
    size_t stride, off_gq, off_uq, off_dq, off_gs, off_us, off_ds;
    int D, F, E, T, TK;      // TK = rows of routed pairs (T*K); shared rows follow
    const GpTile *tiles;
    const int *n_tiles;
    const int *tokens;       // [TK] token of each routed list row
    const __half *aspl;      // activations split: [token or list row][2 (hi, lo)][cols]
    const int *aexp;
    float *out;              // [TK + T][cols out] per list row
};

// Token (for the gate/up input) of list row `row`.
__device__ static inline int gp_token(const GroupArgs &a, int row) {
    return row < a.TK ? a.tokens[row] : row - a.TK;
}

typedef __attribute__((address_space(3))) void gp_lds_void;

typedef _Float16 gp_h8 __attribute__((ext_vector_type(8)));
typedef float gp_f4 __attribute__((ext_vector_type(4)));

// Staging of a tile's inputs, chunk by chunk, into [GP_TOK * 2 rows][GP_KC] fp16 of
// shared memory, row r = 2 (input) + plane (hi, lo). The 16-byte groups of row r are
// stored XOR-swizzled by input % 16, so the A-operand reads (16 inputs, 16 bytes each)
// hit 16 different bank groups. A tile body for NA A tiles (16 NA inputs) stages rows
// 0 .. 32 NA - 1 only: each thread fills gp_stage_iters(NA) slots per chunk, whose source
// addresses are fixed per tile (the row's start plus the slot's logical group), so a
// chunk costs exactly that many loads per thread.
#define GP_RB (GP_KC * 2)            // bytes per staged row
#define GP_RG (GP_RB / 16)           // 16-byte groups per staged row
#define GP_NA_MAX (GP_TOK / 16)      // A tiles (16 inputs each) per tile
static_assert(16 * 2 * GP_RG == 2 * GP_BLOCK, "an A tile's staged rows take two slots per thread");
__host__ __device__ constexpr int gp_stage_iters(int na) { return 2 * na; }
template <int NA>
struct GpStage {
    const __half *src[gp_stage_iters(NA)];
};

// src_row(i): the activation row of input i (clamped to a valid row past the count).
template <int NA, typename RowOf>
__device__ static inline GpStage<NA> gp_stage_init(const __half *spl, int cols, RowOf src_row) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    GpStage<NA> g;
#pragma unroll
    for (int it = 0; it < gp_stage_iters(NA); it++) {
        const int s = 64 * w + GP_BLOCK * it + lane, r = s / GP_RG, p = s % GP_RG, j = p ^ ((r >> 1) & 15);
        g.src[it] = spl + ((size_t)src_row(r >> 1) * 2 + (r & 1)) * cols + 8 * j;
    }
    return g;
}

template <int NA>
__device__ static inline void gp_stage(const GpStage<NA> &g, uint8_t *buf, int c0) {
    const int w = threadIdx.x >> 6;
#pragma unroll
    for (int it = 0; it < gp_stage_iters(NA); it++)
        __builtin_amdgcn_global_load_lds((const GM_GLOBAL void *)gbl(g.src[it] + c0),
                                         (gp_lds_void *)(buf + 16 * (64 * w + GP_BLOCK * it)), 16, 0, 0);
}

// The A operand of A tile i (inputs 16i..16i+15), plane pl, for 32-column block b of
// the staged chunk: lane l holds input 16i + l % 16, columns 32b + 8(l / 16) .. +8.
__device__ static inline gp_h8 gp_a(const uint8_t *buf, int i, int pl, int b) {
    const int lane = threadIdx.x & 63;
    const int in = 16 * i + (lane & 15), r = 2 * in + pl;
    const int j = 4 * b + (lane >> 4), p = j ^ (in & 15);
    return *(const gp_h8 *)(buf + r * GP_RB + 16 * p);
}

// Eight int8 weights (two dwords) as fp16, exactly: each byte b becomes the fp16 with
// bits 0x64 (b ^ 0x80) = 1152 + q, and one packed subtract removes the 1152.
__device__ static inline gp_h8 gp_i8_to_h8(unsigned lo, unsigned hi) {
    const unsigned u0 = lo ^ 0x80808080u, u1 = hi ^ 0x80808080u;
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 off = {(_Float16)1152.0f, (_Float16)1152.0f};
    unsigned w[4];
    w[0] = __builtin_amdgcn_perm(0x64646464u, u0, 0x07010700u);  // bytes: u0.b0, 0x64, u0.b1, 0x64
    w[1] = __builtin_amdgcn_perm(0x64646464u, u0, 0x07030702u);
    w[2] = __builtin_amdgcn_perm(0x64646464u, u1, 0x07010700u);
    w[3] = __builtin_amdgcn_perm(0x64646464u, u1, 0x07030702u);
    gp_h8 r;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        h2 v = __builtin_bit_cast(h2, w[k]) - off;
        r[2 * k] = v[0];
        r[2 * k + 1] = v[1];
    }
    return r;
}

// acc[i][0..3] += the block dots of the lane's four inputs of A tile i (i < NA), times
// scale s. NA is a compile-time count: a data-dependent exit between these MFMAs and the
// accumulation would put the accumulation in a join block, where the compiler's wait
// states before reading an MFMA result only cover the fall-through path (seen on gfx950:
// the first reads after the branch got the registers' old contents).
template <int NA>
__device__ static inline void gp_block(const uint8_t *buf, int b, gp_h8 B, float s, float (*acc)[4]) {
    const gp_f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < NA; i++) {
        gp_f4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(gp_a(buf, i, 0, b), B, zero, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(gp_a(buf, i, 1, b), B, d, 0, 0, 0);
#pragma unroll
        for (int k = 0; k < 4; k++) acc[i][k] = fmaf(d[k], s, acc[i][k]);
    }
}

// f(NA) for the tile's A-tile count na (1 .. GP_NA_MAX, block-uniform) as a compile-time
// constant: one branch per block, before any of the tile's work.
template <int N, typename Body>
__device__ __attribute__((always_inline)) static inline void gp_with_na(int na, Body &&f) {
    if constexpr (N > 1) {
        if (na < N) {
            gp_with_na<N - 1>(na, f);
            return;
        }
    }
    f(std::integral_constant<int, N>{});
}

// Chunk pipeline of the grouped GEMMs. A chunk's weights are requested into one of the
// register sets and its activations into one of the shared-memory buffers while earlier
// chunks are multiplied: k_group_down keeps one chunk in flight (two sets, the loop
// unrolled by two), k_group_gu two (three sets and buffers, unrolled by three; its
// gate and up weights make it the larger stream: 162 -> 151 us at T=512, while a third set
// in k_group_down, at 159 VGPRs and three blocks per CU, was slower), so that the register
// sets rotate without copies. Barriers are plain s_barrier after an exact vmcnt wait:
// __syncthreads() carries a release fence that waits for every outstanding load, the
// prefetch included, which would serialise the pipeline.
__device__ static inline void gp_barrier() { __builtin_amdgcn_s_barrier(); }

typedef uint8_t gp_abuf_t[2][GP_TOK * 2 * GP_RB];
typedef uint8_t gp_abuf3_t[3][GP_TOK * 2 * GP_RB];  // k_group_gu: two chunks in flight

// k_group_gu: grid (F/64, max tiles). Wave w computes rows 64 p + 16 w .. +16 of F, gate
// and up, for the tile's inputs, and from them h = silu(g) * u.
typedef unsigned gp_sw __attribute__((ext_vector_type(GP_NB / 2)));  // a chunk's GP_NB fp16 block scales
typedef float gp_s4 __attribute__((ext_vector_type(4)));
template <bool G16>
struct GuRegs {
    u32x4 q[2][GP_NB / 2];  // gate, up: the chunk's 64-column pieces
    gp_sw s[2];             // gate, up: the chunk's block scales
};
template <>
struct GuRegs<true> {       // group size 16: fp32 scales
    u32x4 q[2][GP_NB / 2];
    gp_s4 s[2][GP_NB / 2];  // gate, up: per 64-column piece, the row's four (gm_s16_offset order)
};
// loads per chunk and thread
__host__ __device__ constexpr int gp_gu_loads(int na, bool g16) {
    return 2 * (GP_NB / 2) + (g16 ? 2 * (GP_NB / 2) : 2) + gp_stage_iters(na);
}

// The B operand of one block split by its 16-column groups: lanes 0..31 hold k 0..15 (the
// first group), lanes 32..63 k 16..31; each half keeps its own lanes and zeros elsewhere,
// so that two MFMAs give the two groups' dots apart.
__device__ static inline void gp_split16(gp_h8 B, gp_h8 &B0, gp_h8 &B1) {
    const bool first = (threadIdx.x & 63) < 32;
    const gp_h8 z = {};
    B0 = first ? B : z;
    B1 = first ? z : B;
}

template <int NA, bool G16>
__device__ __attribute__((always_inline)) static inline void gp_gu_tile(const GroupArgs &a, const GpTile &tl, gp_abuf3_t &abuf) {
    const int p = blockIdx.x;
    const int D = a.D, F = a.F, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int nchunks = D >> 6, nblocks = D >> 5;
    const uint8_t *base = a.experts + (size_t)tl.e * a.stride;
    const int P = 4 * p + w;  // the wave's 16-row panel of gate and of up
    const GM_GLOBAL u32x4 *qg = gbl((const u32x4 *)(base + a.off_gq + (size_t)P * nchunks * GM_CHUNK_BYTES)) + lane;
    const GM_GLOBAL u32x4 *qu = gbl((const u32x4 *)(base + a.off_uq + (size_t)P * nchunks * GM_CHUNK_BYTES)) + lane;
    const int row = 16 * P + (lane & 15);
    // the row's fp16 scales, one chunk's blocks per load; at group size 16 the row's four
    // fp32 scales of each 64-column piece (gm_s16_offset: piece c at 16 c + row % 16)
    const GM_GLOBAL gp_sw *sg = gbl((const gp_sw *)(base + a.off_gs + (size_t)row * nblocks * 2));
    const GM_GLOBAL gp_sw *su = gbl((const gp_sw *)(base + a.off_us + (size_t)row * nblocks * 2));
    const GM_GLOBAL gp_s4 *sg16 = gbl((const gp_s4 *)(base + a.off_gs + (size_t)P * D * 4)) + (lane & 15);
    const GM_GLOBAL gp_s4 *su16 = gbl((const gp_s4 *)(base + a.off_us + (size_t)P * D * 4)) + (lane & 15);
    auto src_row = [&](int i) { return gp_token(a, tl.row + (i < tl.count ? i : 0)); };
    const GpStage<NA> stg = gp_stage_init<NA>(a.aspl, D, src_row);
    const int nkc = D / GP_KC;  // K chunks

    float ag[NA][4], au[NA][4];
#pragma unroll
    for (int i = 0; i < NA; i++)
#pragma unroll
        for (int k = 0; k < 4; k++) ag[i][k] = au[i][k] = 0.0f;
    auto issue = [&](GuRegs<G16> &r, int kc) {  // gp_gu_loads(NA, G16) loads
#pragma unroll
        for (int u = 0; u < GP_NB / 2; u++) {
            r.q[0][u] = qg[(size_t)((GP_NB / 2) * kc + u) * 64];
            r.q[1][u] = qu[(size_t)((GP_NB / 2) * kc + u) * 64];
        }
        if constexpr (G16) {
#pragma unroll
            for (int u = 0; u < GP_NB / 2; u++) {
                r.s[0][u] = sg16[(size_t)((GP_NB / 2) * kc + u) * 16];
                r.s[1][u] = su16[(size_t)((GP_NB / 2) * kc + u) * 16];
            }
        } else {
            r.s[0] = sg[kc];
            r.s[1] = su[kc];
        }
        gp_stage<NA>(stg, abuf[kc % 3], kc * GP_KC);
    };
    auto compute = [&](const GuRegs<G16> &r, int kc) {
        const uint8_t *buf = abuf[kc % 3];
#pragma unroll
        for (int b = 0; b < GP_NB; b++) {
#pragma unroll
            for (int m = 0; m < 2; m++) {
                const u32x4 c = r.q[m][b >> 1];
                const gp_h8 B = (b & 1) ? gp_i8_to_h8(c.z, c.w) : gp_i8_to_h8(c.x, c.y);
                if constexpr (G16) {
                    // the block's first group scales lanes 0..31's half of B, its second 32..63's
                    const gp_s4 s4 = r.s[m][b >> 1];
                    gp_h8 B0, B1;
                    gp_split16(B, B0, B1);
                    gp_block<NA>(buf, b, B0, (b & 1) ? s4.y : s4.x, m ? au : ag);
                    gp_block<NA>(buf, b, B1, (b & 1) ? s4.w : s4.z, m ? au : ag);
                } else {
                    const unsigned s2 = r.s[m][b >> 1];
                    const float sc = __half2float(__ushort_as_half((unsigned short)((b & 1) ? s2 >> 16 : s2 & 0xffffu)));
                    gp_block<NA>(buf, b, B, sc, m ? au : ag);
                }
            }
        }
    };
    // one step: chunk kc's data is in (r, buffer kc % 3); chunk kc + 2's is requested into rn
    // (into the registers and buffer chunk kc - 1 used), so that two chunks are in flight
    // while one is multiplied; the wait leaves the later chunks' loads outstanding
    auto step = [&](GuRegs<G16> &r, GuRegs<G16> &rn, int kc) {
        if (kc + 2 < nkc) {
            issue(rn, kc + 2);
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * gp_gu_loads(NA, G16)) : "memory");
        } else if (kc + 1 < nkc) {
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(gp_gu_loads(NA, G16)) : "memory");
        } else {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        gp_barrier();  // every wave's part of chunk kc's activations is in shared memory
        compute(r, kc);
        gp_barrier();  // every wave is done with buffer kc % 3 before it is refilled
    };
    GuRegs<G16> r0, r1, r2;
    issue(r0, 0);
    if (nkc > 1) issue(r1, 1);
    for (int kc = 0; kc < nkc; kc += 3) {
        step(r0, r2, kc);
        if (kc + 1 < nkc) step(r1, r0, kc + 1);
        if (kc + 2 < nkc) step(r2, r1, kc + 2);
    }
    // lane l holds inputs 16i + 4(l/16) + k, row l % 16 of the wave's panel
    const int f = 16 * P + (lane & 15);
#pragma unroll
    for (int i = 0; i < NA; i++)
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int in = 16 * i + 4 * (lane >> 4) + k;
            if (in < tl.count) {
                const int e = a.aexp[src_row(in)];
                const float g = ldexpf(ag[i][k], e), u = ldexpf(au[i][k], e);
                a.out[(size_t)(tl.row + in) * F + f] = g / (1.0f + expf(-g)) * u;
            }
        }
}

template <bool G16>
__global__ __launch_bounds__(GP_BLOCK, G16 ? 2 : GP_OCC) void k_group_gu(GroupArgs a) {
    __shared__ __align__(16) gp_abuf3_t abuf;
    if ((int)blockIdx.y >= *a.n_tiles) return;
    const GpTile tl = a.tiles[blockIdx.y];
    gp_with_na<GP_NA_MAX>(__builtin_amdgcn_readfirstlane((tl.count + 15) >> 4),
                          [&](auto NA) { gp_gu_tile<decltype(NA)::value, G16>(a, tl, abuf); });
}

// k_group_down: grid (D/64, max tiles). Wave w computes D rows 64 p + 16 w .. +16 for the
// tile's inputs (list rows), from h's split form; down is in the column-slice layout.
template <bool G16>
struct DnRegs {
    unsigned long long q[GP_NB];  // the chunk's blocks: 8 bytes of the row each
    unsigned short s[GP_NB];
};
template <>
struct DnRegs<true> {             // group size 16: the row's fp32 scales of both groups of each block
    unsigned long long q[GP_NB];
    float s[GP_NB][2];
};
// loads per chunk and thread
__host__ __device__ constexpr int gp_dn_loads(int na, bool g16) { return (g16 ? 3 : 2) * GP_NB + gp_stage_iters(na); }

template <int NA, bool G16>
__device__ __attribute__((always_inline)) static inline void gp_down_tile(const GroupArgs &a, const GpTile &tl, gp_abuf_t &abuf) {
    const int p = blockIdx.x;
    const int D = a.D, F = a.F, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const uint8_t *base = a.experts + (size_t)tl.e * a.stride;
    const int row = 64 * p + 16 * w + (lane & 15), qh = lane >> 4;
    // B operand of block b (F columns 32b + 8 qh .. +8): slice 2b + qh/2, half qh % 2
    const GM_GLOBAL uint8_t *qd = gbl(base + a.off_dq) + (size_t)row * 16 + 8 * (qh & 1);
    const GM_GLOBAL unsigned short *sd = gbl((const unsigned short *)(base + a.off_ds)) + row;
    const GM_GLOBAL float *sd16 = gbl((const float *)(base + a.off_ds)) + row;  // gm_ds16_offset: [F/16][D]
    auto src_row = [&](int i) { return tl.row + (i < tl.count ? i : 0); };
    const GpStage<NA> stg = gp_stage_init<NA>(a.aspl, F, src_row);
    const int nkc = F / GP_KC;
    float acc[NA][4];
#pragma unroll
    for (int i = 0; i < NA; i++)
#pragma unroll
        for (int k = 0; k < 4; k++) acc[i][k] = 0.0f;
    auto issue = [&](DnRegs<G16> &r, int kc) {  // gp_dn_loads(NA, G16) loads
#pragma unroll
        for (int b = 0; b < GP_NB; b++) {
            const int blk = GP_NB * kc + b;
            r.q[b] = *(const GM_GLOBAL unsigned long long *)(qd + ((size_t)(2 * blk + (qh >> 1)) * D) * 16);
            if constexpr (G16) {
                r.s[b][0] = sd16[(size_t)(2 * blk) * D];
                r.s[b][1] = sd16[(size_t)(2 * blk + 1) * D];
            } else {
                r.s[b] = sd[(size_t)blk * D];
            }
        }
        gp_stage<NA>(stg, abuf[kc & 1], kc * GP_KC);
    };
    auto compute = [&](const DnRegs<G16> &r, int kc) {
        const uint8_t *buf = abuf[kc & 1];
#pragma unroll
        for (int b = 0; b < GP_NB; b++) {
            const gp_h8 B = gp_i8_to_h8((unsigned)r.q[b], (unsigned)(r.q[b] >> 32));
            if constexpr (G16) {
                gp_h8 B0, B1;
                gp_split16(B, B0, B1);
                gp_block<NA>(buf, b, B0, r.s[b][0], acc);
                gp_block<NA>(buf, b, B1, r.s[b][1], acc);
            } else {
                gp_block<NA>(buf, b, B, __half2float(__ushort_as_half(r.s[b])), acc);
            }
        }
    };
    auto step = [&](DnRegs<G16> &r, DnRegs<G16> &rn, int kc) {
        issue(rn, kc + 1);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(gp_dn_loads(NA, G16)) : "memory");
        gp_barrier();
        compute(r, kc);
        gp_barrier();
    };
    auto last = [&](DnRegs<G16> &r, int kc) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        gp_barrier();
        compute(r, kc);
    };
    DnRegs<G16> r0, r1;
    issue(r0, 0);
    int kc = 0;
    for (; kc + 2 < nkc; kc += 2) {
        step(r0, r1, kc);
        step(r1, r0, kc + 1);
    }
    if (nkc - kc == 2) {
        step(r0, r1, kc);
        last(r1, kc + 1);
    } else {
        last(r0, kc);
    }
#pragma unroll
    for (int i = 0; i < NA; i++)
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int in = 16 * i + 4 * (lane >> 4) + k;
            if (in < tl.count) {
                const int r = tl.row + in;
                a.out[(size_t)r * D + row] = ldexpf(acc[i][k], a.aexp[r]);
            }
        }
}

template <bool G16>
__global__ __launch_bounds__(GP_BLOCK, GP_OCC) void k_group_down(GroupArgs a) {
    __shared__ __align__(16) gp_abuf_t abuf;
    if ((int)blockIdx.y >= *a.n_tiles) return;
    const GpTile tl = a.tiles[blockIdx.y];
    gp_with_na<GP_NA_MAX>(__builtin_amdgcn_readfirstlane((tl.count + 15) >> 4),
                          [&](auto NA) { gp_down_tile<decltype(NA)::value, G16>(a, tl, abuf); });
}

struct TokenCombineArgs {
    const int *topk_idx;   // [T][K]
    const float *topk_ws;  // [T][K] weights * routed_scale
    const int *pair_row;   // [T][K] list row of (token, slot)
    const float *y;        // [TK + T][D]
    const float *x_in;
    float *x_out, *shared_out, *routed_out;
    int D, K, TK, routed_on;
};

// grid (D/1024, T): x' = x + (shared + sum_k fl(w_k y_k)) in top-k order (infer.c:1192,
// 1212-1214), with the shared and routed sums kept as observables; four consecutive
// elements per thread (D is a multiple of 256), in 16-byte loads and stores when the
// caller's x_in and x_out are 16-byte aligned (VEC), else element by element.
template <bool VEC>
__global__ __launch_bounds__(GP_BLOCK) void k_token_combine(TokenCombineArgs a) {
    const int t = blockIdx.y, d = 4 * (blockIdx.x * GP_BLOCK + threadIdx.x);
    if (d >= a.D) return;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (a.routed_on) {
        for (int k = 0; k < a.K; k++) {
            if (a.topk_idx[t * a.K + k] < 0) continue;
            const float4 yk = *(const float4 *)&a.y[(size_t)a.pair_row[t * a.K + k] * a.D + d];
            const float w = a.topk_ws[t * a.K + k], yv[4] = {yk.x, yk.y, yk.z, yk.w};
#pragma unroll
            for (int c = 0; c < 4; c++) acc[c] = __fadd_rn(acc[c], __fmul_rn(w, yv[c]));
        }
    }
    const float4 sh4 = *(const float4 *)&a.y[(size_t)(a.TK + t) * a.D + d];
    const size_t o = (size_t)t * a.D + d;
    *(float4 *)&a.routed_out[o] = make_float4(acc[0], acc[1], acc[2], acc[3]);
    *(float4 *)&a.shared_out[o] = sh4;
    const float shv[4] = {sh4.x, sh4.y, sh4.z, sh4.w};
    if (VEC) {
        const float4 x4 = *(const float4 *)&a.x_in[o];
        *(float4 *)&a.x_out[o] = make_float4(__fadd_rn(x4.x, __fadd_rn(shv[0], acc[0])), __fadd_rn(x4.y, __fadd_rn(shv[1], acc[1])),
                                             __fadd_rn(x4.z, __fadd_rn(shv[2], acc[2])), __fadd_rn(x4.w, __fadd_rn(shv[3], acc[3])));
    } else {
#pragma unroll
        for (int c = 0; c < 4; c++) a.x_out[o + c] = __fadd_rn(a.x_in[o + c], __fadd_rn(shv[c], acc[c]));
    }
}
