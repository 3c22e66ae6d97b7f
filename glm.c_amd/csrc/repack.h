// repack.h -- one-time upload repack from glm.c's checkpoint layout (int8 [rows][cols],
// fp32 scales [rows][cols/32]; infer.c:707-739) into the tiled Q8_0 layout of common.h.
#pragma once

#include "common.h"

// One thread per 16-byte unit of the q plane, for n_mat matrices of rows x cols laid
// out back to back in `raw`; matrix m goes to dst + m * dst_stride, in the tiled panel
// layout or (GM_LAYOUT_SLICES) the column-slice layout.
__global__ void k_repack_q(const int8_t *__restrict__ raw, uint8_t *__restrict__ dst, size_t dst_stride, int rows,
                           int cols, int n_mat, int layout) {
    const size_t units = (size_t)rows * cols / 16;
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= units * (size_t)n_mat) return;
    const int m = (int)(gid / units);
    const size_t u = gid % units;
    if (layout == GM_LAYOUT_SLICES) {
        const int r = (int)(u % rows), j = (int)(u / rows);
        const u32x4 v = *(const u32x4 *)(raw + (size_t)m * rows * cols + (size_t)r * cols + 16 * (size_t)j);
        *(u32x4 *)(dst + (size_t)m * dst_stride + u * 16) = v;
        return;
    }
    const int lane = (int)(u & 63);
    const size_t pj = u >> 6;
    const int nch = cols >> 6;
    const int j = (int)(pj % nch), p = (int)(pj / nch);
    const int r = p * 16 + (lane & 15);
    const int c0 = 64 * j + 8 * (lane >> 4);
    const int8_t *src = raw + (size_t)m * rows * cols + (size_t)r * cols;
    const uint2 lo = *(const uint2 *)(src + c0);
    const uint2 hi = *(const uint2 *)(src + c0 + 32);
    u32x4 v;
    v.x = lo.x;
    v.y = lo.y;
    v.z = hi.x;
    v.w = hi.y;
    *(u32x4 *)(dst + (size_t)m * dst_stride + u * 16) = v;
}

// One thread per scale; counts scales whose fp16 rounding is not exact (inexact: optional).
__global__ void k_repack_s(const float *__restrict__ raw, uint8_t *__restrict__ dst, size_t dst_stride, int rows,
                           int cols, int n_mat, int layout, unsigned long long *inexact) {
    const int nb = cols >> 5;
    const size_t per = (size_t)rows * nb;
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= per * (size_t)n_mat) return;
    const int m = (int)(gid / per);
    const size_t i = gid % per;
    const int r = (int)(i / nb), b = (int)(i % nb);
    const float s = raw[gid];
    const __half hs = __float2half_rn(s);
    if (inexact && __half2float(hs) != s) atomicAdd(inexact, 1ull);
    __half *out = (__half *)(dst + (size_t)m * dst_stride);
    out[layout == GM_LAYOUT_SLICES ? gm_ds_offset(r, b, rows) : gm_s_offset(r, b, cols)] = hs;
}

// Group size 16: one thread per fp32 scale (raw [rows][cols/16], glm.c's order), copied as
// it is into gm_s16_offset's panel runs or (GM_LAYOUT_SLICES) gm_ds16_offset's slice rows.
__global__ void k_repack_s16(const float *__restrict__ raw, uint8_t *__restrict__ dst, size_t dst_stride, int rows,
                             int cols, int n_mat, int layout) {
    const int ng = cols >> 4;
    const size_t per = (size_t)rows * ng;
    const size_t gid = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= per * (size_t)n_mat) return;
    const int m = (int)(gid / per);
    const size_t i = gid % per;
    const int r = (int)(i / ng), g = (int)(i % ng);
    float *out = (float *)(dst + (size_t)m * dst_stride);
    out[layout == GM_LAYOUT_SLICES ? gm_ds16_offset(r, g, rows) : gm_s16_offset(r, g, cols)] = raw[gid];
}
