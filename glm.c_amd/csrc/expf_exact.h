// expf_exact.h -- the host C library's expf, bit for bit, on the GPU.
//
// glm.c scores experts with p = 1.0f / (1.0f + expf(-logit)) using libm's expf
// (infer.c:1104-1107) and orders them by p + bias with a strict `>`
// (infer.c:1110-1135), so two experts can be ordered by expf's last bit. The exact
// router replay therefore needs libm's results, not merely accurate ones.
//
// expf_libm(x) rounds a double-precision exp(x) (error far below 2^-40 relative) to
// fp32. That is the correctly rounded result, which libm's expf also returns except
// where exp(x) lies within its internal error of a midpoint between two floats. Those
// inputs, and every input where two accurate double results could round to different
// floats, were measured once against libm over all 2^32 fp32 inputs
// (host/expf_table.c, data/expf_exceptions.bin): the generated gm_expf_* arrays list
// them with the neighbour libm picks. Every input libm rounds away from the correctly
// rounded value lies within 2^-9 ulp of a midpoint, so only inputs within 2^-7 ulp
// (GM_EXPF_NEAR_LOG2) consult the table: ~1.6 % of inputs, a bucket index and a short
// binary search.
#pragma once

#include "expf_table.inc"  // GM_EXPF_N, GM_EXPF_NEAR_LOG2, gm_expf_keys/up/index (generated)

__device__ static float expf_libm(float x) {
    if (!(x < 89.0f)) return x > 0.0f ? __builtin_inff() : x;  // overflow, +inf; NaN stays NaN
    if (x < -104.0f) return 0.0f;                               // exp(x) < 2^-150 rounds to zero
    const double d = exp((double)x);
    // d on the fp32 grid: d = (fl + frac) * 2^ue with fl an integer and 0 <= frac < 1
    int ex;
    (void)frexp(d, &ex);
    const int ue = ex - 24 < -149 ? -149 : ex - 24;
    const double q = ldexp(d, -ue), fl = floor(q), frac = q - fl;
    float r = (float)d;
    if (fabs(frac - 0.5) < ldexp(1.0, -(int)GM_EXPF_NEAR_LOG2)) {
        const unsigned key = __float_as_uint(x);
        unsigned lo = gm_expf_index[key >> 16], hi = gm_expf_index[(key >> 16) + 1];
        while (lo < hi) {
            const unsigned mid = (lo + hi) >> 1;
            if (gm_expf_keys[mid] < key)
                lo = mid + 1;
            else
                hi = mid;
        }
        if (lo < GM_EXPF_N && gm_expf_keys[lo] == key) {
            const bool up = (gm_expf_up[lo >> 5] >> (lo & 31)) & 1u;
            r = (float)ldexp(up ? fl + 1.0 : fl, ue);
        }
    }
    return r;
}

// glm.c's router probability 1 / (1 + expf(-s)) in fp32, bit for bit (infer.c:1105).
__device__ static inline float sigmoid_libm(float s) { return __fdiv_rn(1.0f, __fadd_rn(1.0f, expf_libm(-s))); }
