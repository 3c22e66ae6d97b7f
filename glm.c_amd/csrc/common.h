// common.h -- device-side helpers and the HBM layout of Q8_0 expert weights.
//
// Tiled Q8_0 layout. A matrix W[R][C] (int8, one fp16 scale per 32-column block)
// is stored as two planes:
//   q plane: 16-row panels; inside a panel, 64-column chunks of 1 KB. Byte 16*l + 8*h + i
//            of chunk (p, j) is W[16p + l%16][64j + 32h + 8*(l/16) + i] (l = lane 0..63,
//            h = 0..1, i = 0..7). One dwordx4 load per lane reads a whole chunk, and its
//            two 8-byte halves are exactly the B operands of two v_mfma_i32_16x16x32_i8
//            (lane l = row l%16, k = 8*(l/16)..+8), one per 32-column quantisation block.
//   s plane: fp16 scale of (row r, block b) at r*(C/32) + b (row-major), so the row a
//            lane owns has the scales of any run of consecutive blocks side by side.
// One expert = gate, up, down q planes then their s planes, 34 bytes per 32 weights.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#define GM_TILE_ROWS 16
#define GM_QBLOCK 32
#define GM_CHUNK_COLS 64
#define GM_CHUNK_BYTES 1024
#define GM_MAX_E 256
#define GM_MAX_K 8
#define GM_MAX_DIM 8192
#define GM_MAX_COLS 2048  // widest matrix row the expert kernels hold in registers

// Global-memory (address space 1) views. Pointers read from memory (the layer table)
// are generic to the compiler, which then emits flat loads; flat loads also count
// against lgkmcnt, so an LDS wait would stall on every outstanding weight load.
#define GM_GLOBAL __attribute__((address_space(1)))
template <typename T>
__device__ static inline const GM_GLOBAL T *gbl(const T *p) {
    return (const GM_GLOBAL T *)p;
}

// s_waitcnt immediate (gfx9 encoding) for vmcnt(0) alone: expcnt and lgkmcnt at their
// maxima. Passed to __builtin_amdgcn_s_waitcnt, which the compiler's wait insertion sees,
// unlike an asm wait.
#define GM_WAIT_VM0 0x0F70

typedef int v4i __attribute__((ext_vector_type(4)));

typedef __attribute__((address_space(3))) void lds_void;

// One 16-byte piece per lane from global memory straight into shared memory (lane l at
// dst + 16 l), issued by inline assembly, which the compiler does not see as a
// shared-memory DMA: with a global_load_lds of its own in flight, the compiler waits for
// all of a wave's loads before using any loaded register or reading shared memory, which
// would serialise whatever is streamed behind it. The caller waits (vmcnt) before reading
// `dst`.
__device__ static inline void dma16_untracked(const GM_GLOBAL void *src, lds_void *dst) {
    const unsigned m0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)dst);
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(m0) : "memory", "m0");
}
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__host__ __device__ static inline size_t gm_q_offset(int r, int c, int cols) {
    const int p = r >> 4, j = c >> 6;
    const int lane = (r & 15) + 16 * ((c & 31) >> 3);
    const int half = (c & 63) >> 5;
    return ((size_t)p * (size_t)(cols >> 6) + (size_t)j) * GM_CHUNK_BYTES + (size_t)lane * 16 + (size_t)half * 8 +
           (size_t)(c & 7);
}

__host__ __device__ static inline size_t gm_s_offset(int r, int b, int cols) {
    return (size_t)r * (size_t)(cols >> 5) + (size_t)b;
}

// Down matrices ([D rows][F cols]) use the column-slice layout instead: slice j holds
// columns 16j..16j+15 of every row, 16 bytes per row, rows in order, and the fp16
// scales are block-major [F/32][D]. A decode item that owns 16 columns of F then reads
// its D x 16 slice as one contiguous, fully coalesced run.
#define GM_LAYOUT_PANELS 0
#define GM_LAYOUT_SLICES 1
__host__ __device__ static inline size_t gm_dq_offset(int r, int c, int rows) {
    return ((size_t)(c >> 4) * (size_t)rows + (size_t)r) * 16 + (size_t)(c & 15);
}
__host__ __device__ static inline size_t gm_ds_offset(int r, int b, int rows) {
    return (size_t)b * (size_t)rows + (size_t)r;
}

// Group size 16 with fp32 scales (the exporter's form), q planes as above. Gate/up scales:
// panel p (16 rows) holds [cols/64 chunks][16 rows][2 groups][2 blocks] fp32, so that a
// 64-column chunk's 64 scales are one run, row r's four of them contiguous, ordered (first
// group of block 0, of block 1, second group of block 0, of block 1). Group g of a row is
// columns 16g..16g+15: chunk g/4, block (g/2)%2, group g%2 of its block.
__host__ __device__ static inline size_t gm_s16_offset(int r, int g, int cols) {
    const int p = r >> 4, m = r & 15, c = g >> 2, hb = (g >> 1) & 1, h = g & 1;
    return (size_t)p * (size_t)cols + (size_t)((((c * 16 + m) * 2 + h) * 2) + hb);
}
// Down scales at group size 16: [F/16 slices][D rows] fp32, one scale per slice row.
__host__ __device__ static inline size_t gm_ds16_offset(int r, int g, int rows) {
    return (size_t)g * (size_t)rows + (size_t)r;
}

// Correctly rounded fp32 square root. The fp32 intrinsic lowers to v_sqrt_f32, which is
// not always correctly rounded; the fp64 lowering is (Newton-refined), and rounding a
// correctly rounded fp64 root to fp32 is exact-rounding since 53 >= 2*24 + 2.
__device__ static inline float sqrt_rn_f32(float a) { return (float)sqrt((double)a); }

// ---------------------------------------------------------------- reductions
//
// Cross-lane traffic uses DPP row operations (no LDS round trip) within each 16-lane
// row and v_readlane across the four rows; ds_bpermute-based shuffles take ~100 clocks
// each and a six-step chain of them dominated the router's latency.

#define DPP_QUAD_1032 0xB1  // quad_perm [1,0,3,2]
#define DPP_QUAD_2301 0x4E  // quad_perm [2,3,0,1]
#define DPP_ROW_HALF_MIRROR 0x141
#define DPP_ROW_MIRROR 0x140
#define DPP_ROW_SHR(n) (0x110 + (n))

template <int CTRL>
__device__ static inline double dpp_d(double v, double fill) {
    const int2 a = *(int2 *)&v, f = *(int2 *)&fill;
    int2 r;
    r.x = __builtin_amdgcn_update_dpp(f.x, a.x, CTRL, 0xF, 0xF, false);
    r.y = __builtin_amdgcn_update_dpp(f.y, a.y, CTRL, 0xF, 0xF, false);
    return *(double *)&r;
}

__device__ static inline double readlane_d(double v, int lane) {
    const int2 a = *(int2 *)&v;
    int2 r;
    r.x = __builtin_amdgcn_readlane(a.x, lane);
    r.y = __builtin_amdgcn_readlane(a.y, lane);
    return *(double *)&r;
}

// Sum over the 64 lanes of a wave, returned to every lane (wave-uniform).
__device__ static inline double wave_sum_dpp(double v) {
    v += dpp_d<DPP_QUAD_1032>(v, 0.0);
    v += dpp_d<DPP_QUAD_2301>(v, 0.0);
    v += dpp_d<DPP_ROW_HALF_MIRROR>(v, 0.0);
    v += dpp_d<DPP_ROW_MIRROR>(v, 0.0);
    return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}

// Maximum over the 64 lanes of a wave, returned to every lane (wave-uniform). NaN
// inputs are ignored, as fmax ignores them.
__device__ static inline double wave_max_dpp(double v) {
    v = fmax(v, dpp_d<DPP_QUAD_1032>(v, -INFINITY));
    v = fmax(v, dpp_d<DPP_QUAD_2301>(v, -INFINITY));
    v = fmax(v, dpp_d<DPP_ROW_HALF_MIRROR>(v, -INFINITY));
    v = fmax(v, dpp_d<DPP_ROW_MIRROR>(v, -INFINITY));
    return fmax(fmax(readlane_d(v, 0), readlane_d(v, 16)), fmax(readlane_d(v, 32), readlane_d(v, 48)));
}

__device__ static inline float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Maximum over the 64 lanes of a wave, returned to every lane (wave-uniform), by DPP.
__device__ static inline float wave_max_dpp_f(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(v), DPP_QUAD_1032, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(v), DPP_QUAD_2301, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(v), DPP_ROW_HALF_MIRROR, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(v), DPP_ROW_MIRROR, 0xF, 0xF, false)));
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

// Maximum over each 16-lane row of a wave, returned to every lane of the row, by DPP.
__device__ static inline float row_max_dpp_f(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(v), DPP_QUAD_1032, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(v), DPP_QUAD_2301, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(v), DPP_ROW_HALF_MIRROR, 0xF, 0xF, false)));
    return fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(-INFINITY), __float_as_int(v), DPP_ROW_MIRROR, 0xF, 0xF, false)));
}

// Sum over each 16-lane row of a wave, returned to every lane of the row, by DPP: quads,
// then pairs of quads, then the two halves (the same order in every lane: fp32 addition
// commutes).
__device__ static inline float row_sum_dpp_f(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP_QUAD_1032, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP_QUAD_2301, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP_ROW_HALF_MIRROR, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP_ROW_MIRROR, 0xF, 0xF, false));
    return v;
}

// Inclusive prefix sum over the lanes of a wave, in lane order.
__device__ static inline double wave_incl_scan_dpp(double v) {
    v += dpp_d<DPP_ROW_SHR(1)>(v, 0.0);
    v += dpp_d<DPP_ROW_SHR(2)>(v, 0.0);
    v += dpp_d<DPP_ROW_SHR(4)>(v, 0.0);
    v += dpp_d<DPP_ROW_SHR(8)>(v, 0.0);
    const double r0 = readlane_d(v, 15), r1 = readlane_d(v, 31), r2 = readlane_d(v, 47);
    const int row = (threadIdx.x & 63) >> 4;
    double off = 0.0;
    if (row >= 1) off += r0;
    if (row >= 2) off += r1;
    if (row >= 3) off += r2;
    return v + off;
}

// Block-wide sum of doubles for a 256-thread block, to every thread; `red` holds 4
// doubles of shared memory.
__device__ static inline double block_sum_fast(double v, double *red) {
    v = wave_sum_dpp(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return ((red[0] + red[1]) + red[2]) + red[3];
}

__device__ static inline double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ static inline float wave_max_f(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Block-wide sum of doubles for a 256-thread block; every thread gets the total.
// `red` must hold 4 doubles of shared memory. Summation order is fixed.
__device__ static inline double block_sum_d(double v, double *red) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    v = wave_sum_d(v);
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    double t = ((red[0] + red[1]) + red[2]) + red[3];
    return t;
}

// Block-wide exclusive prefix sum of doubles (256 threads) in thread order.
__device__ static inline double block_exclusive_scan_d(double v, double *red, double *total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    double incl = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        double n = __shfl_up(incl, o, 64);
        if (lane >= o) incl += n;
    }
    __syncthreads();
    if (lane == 63) red[w] = incl;
    __syncthreads();
    double base = 0.0;
    for (int i = 0; i < w; i++) base += red[i];
    *total = ((red[0] + red[1]) + red[2]) + red[3];
    return base + incl - v;
}

// ---------------------------------------------------------------- int8 digit form
//
// A block of 32 fp32 activations is written exactly-enough as 2^e * X with X integer,
// |X| <= 8323072 = 127*2^16 + 127*2^8 (22-23 significant bits relative to the block
// maximum), and X is split into balanced base-256 digits d0, d1, d2 in [-128, 127]:
// X = d0 + 256*d1 + 65536*d2. An int8 MFMA then gives each digit's dot product with a
// weight block exactly in int32, and the block dot is rebuilt in fp32.

__device__ static inline int digit_exponent(float maxabs) {
    if (!(maxabs > 0.0f) || !isfinite(maxabs)) return 0;
    int k;
    float m = frexpf(maxabs, &k);  // maxabs = m * 2^k, m in [0.5, 1)
    // m * 2^23 <= 8323072 keeps the top digit within int8; otherwise use one bit less.
    return (m * 8388608.0f <= 8323072.0f) ? k - 23 : k - 22;
}

__device__ static inline void split_digits(float v, int e, int8_t *d0, int8_t *d1, int8_t *d2) {
    int X = (int)rintf(ldexpf(v, -e));
    int a0 = ((X + 128) & 255) - 128;
    int X1 = (X - a0) >> 8;
    int a1 = ((X1 + 128) & 255) - 128;
    int a2 = (X1 - a1) >> 8;
    *d0 = (int8_t)a0;
    *d1 = (int8_t)a1;
    *d2 = (int8_t)a2;
}

// Two-digit form for the prefill kernels: X = rint(v * 2^-e) with |X| <= 32639, so that
// X = d0 + 256 d1 with balanced int8 digits (d0 in [-128, 127], d1 in [-128, 127]).
__device__ static inline int digit_exponent2(float maxabs) {
    if (!(maxabs > 0.0f) || !isfinite(maxabs)) return 0;
    int k;
    const float m = frexpf(maxabs, &k);  // maxabs = m * 2^k, m in [0.5, 1)
    return (m * 32768.0f <= 32639.0f) ? k - 15 : k - 14;
}

__device__ static inline void split_digits2(float v, int e, int8_t *d0, int8_t *d1) {
    const int X = (int)rintf(ldexpf(v, -e));
    const int a0 = ((X + 128) & 255) - 128;
    *d0 = (int8_t)a0;
    *d1 = (int8_t)((X - a0) >> 8);
}

// fp32 value of D0 + 256*D1 + 65536*D2 for int32 digit dots (|Di| < 2^20).
__device__ static inline float digits_to_float(int D0, int D1, int D2) {
    int lo = D0 + (D1 << 8);  // |lo| < 2^29
    return fmaf((float)D2, 65536.0f, (float)lo);
}
