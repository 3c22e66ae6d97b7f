// router.h -- RMSNorm, sigmoid router and top-k selection (infer.c:1098-1145).
//
// glm.c's router is a sequential fp32 dot per expert (infer.c:916-925), and its
// RMSNorm sums squares sequentially in fp64 (infer.c:746-752). Replaying those chains
// on a GPU costs thousands of dependent adds, so the fast path instead
//  * computes the sum of squares in parallel fp64 and proves that the sequential sum
//    rounds to the same fp32 mean (otherwise replays the chain, rare), which makes
//    xn bit-identical to the CPU's;
//  * computes each router logit S exactly enough in fp64, with a rigorous bound B on
//    |fl32-sequential(S) - S| (a posteriori bound from the fp64 prefix sums), turns
//    [S-B, S+B] into an interval that must contain the CPU's selection score
//    p + bias (allowing for expf, the add and the divide in fp32), and accepts the
//    top-k only when the intervals order the chosen experts strictly.
// When the proof fails the last block replays every expert's fp32 chain exactly and
// runs glm.c's insertion top-k on it; only a tie within the last bits of libm's expf
// could then still differ, and that case is counted in stats[GM_STAT_UNRESOLVED].
#pragma once

#include "common.h"

enum { GM_STAT_NORM_EXACT = 0, GM_STAT_ROUTE_EXACT = 1, GM_STAT_UNRESOLVED = 2, GM_STAT_COUNT = 4 };

struct RouterArgs {
    const float *x;            // [T][D]
    const float *norm_w;       // [D]
    const float *gate_inp;     // [E][D]
    const float *bias;         // [E]
    float *xn;                 // [T][D]
    double2 *stage;            // [T][E]  (S, B)
    unsigned *tok_counter;     // [T], zero between launches
    float *router_prob;        // [T][E]
    int *topk_idx;             // [T][K]
    float *topk_w;             // [T][K] normalised
    float *topk_ws;            // [T][K] normalised * routed_scale
    int *hist_idx;             // [T][K] per-layer copy
    float *hist_w;             // [T][K]
    unsigned long long *stats; // [GM_STAT_COUNT]
    int D, E, K;
    float eps, routed_scale;
    int force_exact;           // GMOE_FLAG_EXACT_ROUTER: skip the certificate, always replay
};

// (float) of the sequential fp64 mean of squares, decided from a parallel fp64 sum.
__device__ static float certified_mean_sq(const float *xt, int D, double *red, float *lds_mean, bool count_stat,
                                          unsigned long long *stats) {
    double ss = 0.0;
    for (int i = threadIdx.x; i < D; i += blockDim.x) {
        double v = (double)xt[i];
        ss += v * v;
    }
    ss = block_sum_d(ss, red);
    const double v = ss / (double)D;
    const double rho = (double)D * 0x1p-52;  // >= error of both the sequential and our sum
    const float lo = (float)(v * (1.0 - rho)), hi = (float)(v * (1.0 + rho));
    if (lo == hi) return lo;
    __syncthreads();
    if (threadIdx.x == 0) {
        double s = 0.0;
        for (int i = 0; i < D; i++) {
            double q = (double)xt[i];
            s += q * q;
        }
        *lds_mean = (float)(s / (double)D);
        if (count_stat) atomicAdd(&stats[GM_STAT_NORM_EXACT], 1ull);
    }
    __syncthreads();
    return *lds_mean;
}

// Interval of fl32(p + b) where p = fl32(1 / fl32(1 + expf(-s))) and s in [S-B, S+B].
// The sigmoid bounds are evaluated in fp32 at the interval ends rounded outwards; the
// GPU's expf and the CPU's libm expf are both within 2 ulp, the add and the divide round
// once each, so p moves by less than 2^-20 relative -- widened to 2^-19 for margin, and
// one more ulp for the final add.
// The last step of selection_interval, from the sigmoids plo, phi at the interval ends.
__device__ static inline void selection_bounds(double plo, double phi, float bias, double *lo, double *hi) {
    const double dp = 0x1p-19;
    const double vlo = plo * (1.0 - dp) + (double)bias;
    const double vhi = phi * (1.0 + dp) + (double)bias;
    *lo = vlo - fabs(vlo) * 0x1p-22 - 0x1p-148;
    *hi = vhi + fabs(vhi) * 0x1p-22 + 0x1p-148;
}

__device__ static inline void selection_interval(double S, double B, float bias, double *lo, double *hi) {
    const float slo = __double2float_rd(S - B), shi = __double2float_ru(S + B);
    const double plo = (double)(1.0f / (1.0f + expf(-slo)));
    const double phi = (double)(1.0f / (1.0f + expf(-shi)));
    const double dp = 0x1p-19;
    const double vlo = plo * (1.0 - dp) + (double)bias;
    const double vhi = phi * (1.0 + dp) + (double)bias;
    *lo = vlo - fabs(vlo) * 0x1p-22 - 0x1p-148;
    *hi = vhi + fabs(vhi) * 0x1p-22 + 0x1p-148;
}

// Wave-wide argmax over (key desc, index asc); lanes hold candidates in registers.
__device__ static inline void wave_argmax(double key, int idx, double *bkey, int *bidx) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        double k2 = __shfl_xor(key, o, 64);
        int i2 = __shfl_xor(idx, o, 64);
        if (k2 > key || (k2 == key && i2 < idx)) {
            key = k2;
            idx = i2;
        }
    }
    *bkey = key;
    *bidx = idx;
}

#define RT_BLOCK 256
#define RT_MAX_PER 32  // D <= 256 * 32

__global__ __launch_bounds__(RT_BLOCK) void k_norm_router(RouterArgs a) {
    extern __shared__ float s_xn[];  // [D]
    __shared__ double red[4];
    __shared__ float s_mean;
    __shared__ int s_last;
    const int e = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const int D = a.D, E = a.E, K = a.K;
    const float *xt = a.x + (size_t)t * D;

    // ---- RMSNorm, bit-identical to infer.c:746-752
    const float mean = certified_mean_sq(xt, D, red, &s_mean, e == 0, a.stats);
    const float inv = __fdiv_rn(1.0f, sqrt_rn_f32(__fadd_rn(mean, a.eps)));
    for (int i = tid; i < D; i += RT_BLOCK) {
        float v = __fmul_rn(__fmul_rn(xt[i], inv), a.norm_w[i]);
        s_xn[i] = v;
        if (e == 0) a.xn[(size_t)t * D + i] = v;
    }
    __syncthreads();

    // ---- router logit of expert e in fp64 plus the bound on the fp32 chain error
    const float *g = a.gate_inp + (size_t)e * D;
    const int per = (D + RT_BLOCK - 1) / RT_BLOCK;
    double p[RT_MAX_PER];
    double seg = 0.0, seg_abs = 0.0;
#pragma unroll
    for (int j = 0; j < RT_MAX_PER; j++) {
        if (j < per) {
            const int i = tid * per + j;
            const double pj = (i < D) ? (double)g[i] * (double)s_xn[i] : 0.0;
            p[j] = pj;
            seg += pj;
            seg_abs += fabs(pj);
        }
    }
    double S;
    double run = block_exclusive_scan_d(seg, red, &S);
    double prefix_abs = 0.0;
#pragma unroll
    for (int j = 0; j < RT_MAX_PER; j++) {
        if (j < per) {
            run += p[j];
            if (tid * per + j < D) prefix_abs += fabs(run);
        }
    }
    const double sum_prefix_abs = block_sum_d(prefix_abs, red);
    const double sum_abs = block_sum_d(seg_abs, red);
    if (tid == 0) {
        const double u = 0x1p-24, n = (double)D;
        const double gamma = n * u / (1.0 - n * u);
        double B = u * (1.0 + u) * sum_abs + u * sum_prefix_abs + n * u * gamma * sum_abs;
        B = B * (1.0 + 0x1p-30) + 0x1p-40 * sum_abs + n * 0x1p-149;
        a.stage[(size_t)t * E + e] = make_double2(S, B);
    }

    // ---- the last block of token t selects
    __threadfence();
    __syncthreads();
    if (tid == 0) s_last = (atomicAdd(&a.tok_counter[t], 1u) == (unsigned)(E - 1));
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    if (tid == 0) a.tok_counter[t] = 0u;

    __shared__ double s_lo[GM_MAX_E], s_hi[GM_MAX_E], s_mid[GM_MAX_E];
    __shared__ float s_p[GM_MAX_E], s_sel[GM_MAX_E];
    __shared__ int s_idx[GM_MAX_K];
    __shared__ int s_ok;
    for (int i = tid; i < E; i += RT_BLOCK) {
        const double2 sb = a.stage[(size_t)t * E + i];
        double lo, hi;
        selection_interval(sb.x, sb.y, a.bias[i], &lo, &hi);
        s_lo[i] = lo;
        s_hi[i] = hi;
        s_mid[i] = 0.5 * (lo + hi);
        s_p[i] = (float)(1.0 / (1.0 + exp(-sb.x)));
    }
    __syncthreads();

    if (tid < 64) {
        // K rounds of wave argmax over the midpoints; then check strict separation.
        unsigned long long taken = 0ull;  // bit i: lane-local candidate i taken (E <= 256 -> 4 per lane)
        int ok = !a.force_exact;
        double prev_lo = 0.0;
        const int kk = K < E ? K : E;
        for (int k = 0; k < kk; k++) {
            double best = -INFINITY;
            int bi = 0x7fffffff;
            for (int c = 0; c < 4; c++) {
                const int i = tid + 64 * c;
                if (i < E && !((taken >> c) & 1ull)) {
                    const double m = s_mid[i];
                    if (m > best || (m == best && i < bi)) {
                        best = m;
                        bi = i;
                    }
                }
            }
            double wk;
            int wi;
            wave_argmax(best, bi, &wk, &wi);
            if (wi == 0x7fffffff || !(wk == wk)) {
                ok = 0;
                break;
            }
            if ((wi & 63) == tid) taken |= 1ull << (wi >> 6);
            if (k > 0 && !(prev_lo > s_hi[wi])) ok = 0;
            prev_lo = s_lo[wi];
            if (tid == 0) s_idx[k] = wi;
        }
        if (ok && kk < E) {
            // the last chosen must beat every expert left out
            double mx = -INFINITY;
            for (int c = 0; c < 4; c++) {
                const int i = tid + 64 * c;
                if (i < E && !((taken >> c) & 1ull)) mx = fmax(mx, s_hi[i]);
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) mx = fmax(mx, __shfl_xor(mx, o, 64));
            if (!(prev_lo > mx)) ok = 0;
        }
        if (tid == 0) {
            s_ok = ok;
            for (int k = kk; k < K; k++) s_idx[k] = -1;
        }
    }
    __syncthreads();

    if (!s_ok) {
        // ---- exact replay: sequential fp32 chains (infer.c:916-925), glm.c's insertion top-k
        for (int i = tid; i < E; i += RT_BLOCK) {
            const float *gi = a.gate_inp + (size_t)i * D;
            float chain = 0.0f;
            for (int j = 0; j < D; j++) chain = __fadd_rn(chain, __fmul_rn(gi[j], s_xn[j]));
            const float pr = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-chain)));
            s_p[i] = pr;
            s_sel[i] = __fadd_rn(pr, a.bias[i]);
        }
        __syncthreads();
        if (tid == 0) {
            atomicAdd(&a.stats[GM_STAT_ROUTE_EXACT], 1ull);
            int idx[GM_MAX_K];
            for (int k = 0; k < K; k++) idx[k] = -1;
            for (int i = 0; i < E; i++) {
                const float sc = s_sel[i];
                int at = -1;
                for (int k = 0; k < K && at < 0; k++) {
                    const float held = idx[k] >= 0 ? s_sel[idx[k]] : -INFINITY;
                    if (sc > held) at = k;
                }
                if (at < 0) continue;
                for (int k = K - 1; k > at; k--) idx[k] = idx[k - 1];
                idx[at] = i;
            }
            // GPU expf may differ from libm's by an ulp: flag orderings decided that closely.
            int unresolved = 0;
            for (int k = 0; k < K; k++) {
                if (idx[k] < 0) continue;
                const float a0 = s_sel[idx[k]];
                const float tol = 4.0f * fmaxf(fabsf(a0), 1e-30f) * 0x1p-23f + 4.0f * 0x1p-24f;
                for (int i = 0; i < E; i++) {
                    if (i == idx[k]) continue;
                    bool above = false;
                    for (int q = 0; q < k; q++) above |= (idx[q] == i);
                    if (above) continue;
                    if (fabsf(s_sel[i] - a0) <= tol) unresolved = 1;
                }
            }
            if (unresolved) atomicAdd(&a.stats[GM_STAT_UNRESOLVED], 1ull);
            for (int k = 0; k < K; k++) s_idx[k] = idx[k];
        }
        __syncthreads();
    }

    if (tid == 0) {
        // weights: unbiased probabilities, normalised as infer.c:1136-1145
        float w[GM_MAX_K];
        float total = 0.0f;
        for (int k = 0; k < K; k++) {
            w[k] = s_idx[k] >= 0 ? s_p[s_idx[k]] : -1e30f;
            if (s_idx[k] >= 0) total = __fadd_rn(total, w[k]);
        }
        if (total > 0.0f) {
            const float denom = total < 6.103515625e-5f ? 6.103515625e-5f : total;
            const float inv_d = __fdiv_rn(1.0f, denom);
            for (int k = 0; k < K; k++) w[k] = __fmul_rn(w[k], inv_d);
        }
        for (int k = 0; k < K; k++) {
            const size_t o = (size_t)t * K + k;
            a.topk_idx[o] = s_idx[k];
            a.topk_w[o] = w[k];
            a.topk_ws[o] = __fmul_rn(w[k], a.routed_scale);
            a.hist_idx[o] = s_idx[k];
            a.hist_w[o] = w[k];
        }
    }
    for (int i = tid; i < E; i += RT_BLOCK) a.router_prob[(size_t)t * E + i] = s_p[i];
}
