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
// When the proof fails the block replays every expert's fp32 chain exactly, with libm's
// own expf results (expf_exact.h), and runs glm.c's insertion top-k on it: the same
// scores bit for bit, so the same experts in the same order, ties to the lower index.
#pragma once

#include "common.h"
#include "expf_exact.h"

enum { GM_STAT_NORM_EXACT = 0, GM_STAT_ROUTE_EXACT = 1, GM_STAT_ROUTE_SUBSET = 2, GM_STAT_COUNT = 4 };

struct RouterArgs {
    const float *x;            // [T][D]
    const float *norm_w;       // [D]
    const float *gate_inp;     // [E][D]
    const float *bias;         // [E]
    float *xn;                 // [T][D]
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

#define RT_SEL_C (GM_MAX_E / 64)  // experts per lane in a one-wave selection
#define RT_BLOCK 256
#define RT_XT 160                 // scratch of the exact replay: RT_XT x 64 floats (exact_router uses two
                                  // 16 KB gate tiles; exact_router_subset holds five 2048-column rows at once)

// Certified top-k on one wave, over C chunks of 64 experts whose results are in
// registers (lane l: experts l + 64c; w0 = fp32 bits of lo | hi << 32, w1 = fp32 bits
// of p): the K best interval midpoints are taken one at a time (a wave maximum, then the
// lowest lane holding it), and the result is certified when each chosen interval lies
// strictly above the next chosen one and the last chosen lies strictly above every
// expert left out. glm.c's insertion top-k (infer.c:1110-1135) orders strictly by
// value, so it must then pick the same experts in the same order. Lane 0 writes the
// top-k to idx / wk (unnormalised p), their sum to *total and the verdict to *sel_ok;
// with p_out, every probability goes there too.
template <int C>
__device__ __attribute__((always_inline)) static void certified_select(int E, int K, int tid, const unsigned long long *w0,
                                                                       const unsigned long long *w1, float *p_out, int *idx,
                                                                       float *wk_out, int *sel_ok, float *total_out) {
    float lo[C], hi[C], pr[C], key[C];
    bool bad = false;
#pragma unroll
    for (int c = 0; c < C; c++) {
        const int e = tid + 64 * c;
        const bool valid = e < E;
        lo[c] = valid ? __uint_as_float((unsigned)w0[c]) : -INFINITY;
        hi[c] = valid ? __uint_as_float((unsigned)(w0[c] >> 32)) : -INFINITY;
        pr[c] = valid ? __uint_as_float((unsigned)w1[c]) : 0.0f;
        if (valid) bad |= !(isfinite(lo[c]) && isfinite(hi[c]));
        key[c] = valid ? 0.5f * lo[c] + 0.5f * hi[c] : -INFINITY;
        if (p_out && valid) p_out[e] = pr[c];
    }
    bool cert = __ballot(bad) == 0;
    float prev_lo = 0.0f, total = 0.0f;
    for (int k = 0; k < K; k++) {
        float bm = key[0];
        int bc = 0;
#pragma unroll
        for (int c = 1; c < C; c++)
            if (key[c] > bm) {
                bm = key[c];
                bc = c;
            }
        const float gm = wave_max_dpp_f(bm);
        int ek = -1;
        float wk = -1e30f;
        if (gm > -INFINITY) {  // fewer than K experts leave the rest at -1 (infer.c:1110-1113)
            const int ls = __ffsll(__ballot(bm == gm)) - 1;
            const int cs = __builtin_amdgcn_readlane(bc, ls);
            float ml = lo[0], mh = hi[0], mp = pr[0];
#pragma unroll
            for (int c = 1; c < C; c++)
                if (bc == c) {
                    ml = lo[c];
                    mh = hi[c];
                    mp = pr[c];
                }
            const float lk = readlane_f(ml, ls), hk = readlane_f(mh, ls);
            if (k > 0 && !(prev_lo > hk)) cert = false;
            prev_lo = lk;
            ek = ls + 64 * cs;
            wk = readlane_f(mp, ls);
            total = __fadd_rn(total, wk);
#pragma unroll
            for (int c = 0; c < C; c++)
                if (tid == ls && c == cs) key[c] = -INFINITY;
        }
        if (tid == 0) {
            idx[k] = ek;
            wk_out[k] = wk;
        }
    }
    // the last chosen must lie above every expert left out (chosen ones now hold -inf)
    float rest = -INFINITY;
#pragma unroll
    for (int c = 0; c < C; c++)
        if (key[c] > -INFINITY) rest = fmaxf(rest, hi[c]);
    rest = wave_max_dpp_f(rest);
    if (rest > -INFINITY && !(prev_lo > rest)) cert = false;
    if (tid == 0) {
        *sel_ok = cert;
        *total_out = total;
    }
}

__device__ __attribute__((always_inline)) static void exact_topk(int E, int K, int tid, const float *p, const float *sel,
                                                                 int *idx, float *wk_out, unsigned long long *stats);

// glm.c's router replayed exactly in fp32 (infer.c:916-938, 1104-1145) by one block of
// 256 threads, for the xn in shared memory: every probability into p and selection
// score into sel (shared, [E]), the top-k into idx and its normalised weights into wk
// (shared, [K]). prod is 32 KB of shared scratch (16-byte aligned). Counts the replay in stats.
__device__ __attribute__((always_inline)) static void exact_router(int D, int E, int K, int tid, const float *gate_inp, const float *bias_p,
                                    const float *xn, float (*prod)[64], float *p, float *sel, int *idx, float *wk_out,
                                    unsigned long long *stats) {
    const GM_GLOBAL float *bias = gbl(bias_p);
    // infer.c:916-925 for 64 experts at a time: lane e of wave 0 forms fl(g * xn) and adds
    // it to its expert's chain, column by column. The gate rows reach shared memory in
    // tiles of 64 columns by DMA from every wave, [64 experts][16 four-column groups] with
    // group g of row e at slot g ^ (e % 16), two tiles in flight (prod's 32 KB); the chain
    // reads the next four groups before adding the current ones.
    const int lane = tid & 63, w = tid >> 6;
    float4(*gt)[1024] = (float4(*)[1024])prod;
    const int ntile = D / 64;
    for (int eb = 0; eb < E; eb += 64) {
        const int ne = E - eb < 64 ? E - eb : 64;
        auto stage = [&](int j, int buf) {  // 1024 pieces of 16 bytes: four per lane
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int unit = (4 * w + i) * 64 + lane, e = unit >> 4, g = (unit & 15) ^ (e & 15);
                const int ee = eb + (e < ne ? e : 0);
                dma16_untracked(gbl(gate_inp + (size_t)ee * D + 64 * j + 4 * g), (lds_void *)(gt[buf] + (4 * w + i) * 64));
            }
        };
        stage(0, 0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        float chain = 0.0f;
        for (int j = 0; j < ntile; j++) {
            if (j + 1 < ntile) stage(j + 1, (j + 1) & 1);
            if (w == 0) {
                const float4 *gb = gt[j & 1] + lane * 16;
                const float4 *xb = (const float4 *)(xn + 64 * j);
                float4 ga[4], xa[4], gn[4], xq[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    ga[u] = gb[u ^ (lane & 15)];
                    xa[u] = xb[u];
                }
#pragma unroll
                for (int g0 = 0; g0 < 16; g0 += 4) {
#pragma unroll
                    for (int u = 0; u < 4; u++) {  // the next four groups (the last batch re-reads the first)
                        const int gg = g0 + 4 < 16 ? g0 + 4 + u : u;
                        gn[u] = gb[gg ^ (lane & 15)];
                        xq[u] = xb[gg];
                    }
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        chain = __fadd_rn(chain, __fmul_rn(ga[u].x, xa[u].x));
                        chain = __fadd_rn(chain, __fmul_rn(ga[u].y, xa[u].y));
                        chain = __fadd_rn(chain, __fmul_rn(ga[u].z, xa[u].z));
                        chain = __fadd_rn(chain, __fmul_rn(ga[u].w, xa[u].w));
                    }
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        ga[u] = gn[u];
                        xa[u] = xq[u];
                    }
                }
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the next tile is in shared memory
            __syncthreads();                                    // and wave 0 is done with this one
        }
        if (tid < ne) {
            const float pr = sigmoid_libm(chain);  // infer.c:1105, libm's expf bits
            p[eb + tid] = pr;
            sel[eb + tid] = __fadd_rn(pr, bias[eb + tid]);
        }
    }
    __syncthreads();
    exact_topk(E, K, tid, p, sel, idx, wk_out, stats);
}

// The exact replay restricted to the experts that can still be chosen: with L the K-th
// largest lower end of the selection intervals (w0[e] = fp32 bits of lo | hi << 32), at
// least K experts score at least L, so an expert whose upper end lies below L scores
// strictly below the K-th best and is never chosen; the others (U, hi >= L: the K
// best-placed ones and those they overlap) are replayed exactly. Then glm.c's insertion
// top-k over U's exact scores picks glm.c's experts in glm.c's order, ties to the lower
// index, and their weights are the exact ones. For |U| <= RT_SUB_MAX the rows of U fit the
// scratch `prod` (cap floats, at least RT_SUB_MAX x 260) in column tiles, the
// intervals w0 (read before the scratch is written, so they may lie in it) are no longer
// needed, every thread forms the products
// fl(g * xn) in place, and lane u of wave 0 runs expert U[u]'s sequential chain over them:
// ~2 K dependent adds instead of the full replay's 64 chains fed tile by tile. p keeps
// the certified probabilities of the experts outside U (they are never chosen). Returns
// false, before touching any output, when |U| is larger (the caller then runs
// exact_router); block-uniform.
#define RT_SUB_MAX 8
static_assert(RT_XT * 64 >= RT_SUB_MAX * 260, "the batch routers' replay scratch holds RT_SUB_MAX padded 256-column rows");
template <int NV>  // 16-byte groups a chain lane reads at once (a multiple of 4 that divides 64)
__device__ __attribute__((always_inline)) static bool exact_router_subset(int D, int E, int K, int tid,
                                                                          const float *gate_inp, const float *bias_p,
                                                                          const float *xn, float (*prod)[64],
                                                                          const unsigned long long *w0, float *p, float *sel,
                                                                          int *idx, float *wk_out, unsigned long long *stats,
                                                                          int *s_u, int *s_nu, int cap) {
    const int lane = tid & 63, w = tid >> 6;
    if (w == 0) {
        const int nch = (E + 63) >> 6;
        float lo[RT_SEL_C], hi[RT_SEL_C];
#pragma unroll
        for (int c = 0; c < RT_SEL_C; c++) {
            const int e = lane + 64 * c;
            const bool valid = c < nch && e < E;
            lo[c] = valid ? __uint_as_float((unsigned)w0[e]) : -INFINITY;
            hi[c] = valid ? __uint_as_float((unsigned)(w0[e] >> 32)) : -INFINITY;
            if (lo[c] != lo[c]) lo[c] = -INFINITY;  // never certified, so never the bound
            if (hi[c] != hi[c]) hi[c] = INFINITY;
        }
        // L: the K-th largest lower end (K rounds of a wave maximum, one entry removed each)
        float rem[RT_SEL_C], L = -INFINITY;
#pragma unroll
        for (int c = 0; c < RT_SEL_C; c++) rem[c] = lo[c];
        for (int k = 0; k < K; k++) {
            float bm = rem[0];
#pragma unroll
            for (int c = 1; c < RT_SEL_C; c++) bm = fmaxf(bm, rem[c]);
            L = wave_max_dpp_f(bm);
            int ls = -1, cs = 0;
#pragma unroll
            for (int c = 0; c < RT_SEL_C; c++) {
                const unsigned long long m = __ballot(rem[c] == L);
                if (ls < 0 && m != 0ull) {
                    ls = __ffsll(m) - 1;
                    cs = c;
                }
            }
#pragma unroll
            for (int c = 0; c < RT_SEL_C; c++)
                if (lane == ls && c == cs) rem[c] = -INFINITY;
        }
        // U in ascending expert order
        int nu = 0;
#pragma unroll
        for (int c = 0; c < RT_SEL_C; c++) {
            const bool in = c < nch && lane + 64 * c < E && hi[c] >= L;
            const unsigned long long m = __ballot(in);
            const int pos = nu + __popcll(m & ((1ull << lane) - 1ull));
            if (in && pos < RT_SUB_MAX) s_u[pos] = lane + 64 * c;
            nu += __popcll(m);
        }
        if (lane == 0) *s_nu = nu;
    }
    __syncthreads();
    const int nu = *s_nu;
    if (nu > RT_SUB_MAX) return false;
    if (tid == 0) atomicAdd(&stats[GM_STAT_ROUTE_SUBSET], 1ull);
    const GM_GLOBAL float *bias = gbl(bias_p);
    // rows of U in the scratch, tile by tile: [nu][tc + 4] floats, the 4 floats of padding
    // putting row u's groups 16 u bytes further round the banks, so that the chain lanes'
    // reads (one group of each row, at the same column) miss no bank with no address
    // arithmetic beyond an add (an XOR swizzle of the groups instead took the chain from
    // ~7.7 to ~10.6 cycles an add, its address work issuing between the dependent adds)
    float *buf = &prod[0][0];
    // columns per tile: the widest of D, 1024, 512, 256 whose nu padded rows fit the scratch
    // (a multiple of 256, as D is, so that every tile's groups fill whole 64-lane DMAs)
    int tc_max = D;
    if (nu * (tc_max + 4) > cap) tc_max = D < 1024 ? D : 1024;
    if (nu * (tc_max + 4) > cap) tc_max = D < 512 ? D : 512;
    if (nu * (tc_max + 4) > cap) tc_max = 256;
    float chain = 0.0f;
    for (int c0 = 0; c0 < D; c0 += tc_max) {
        const int tc = D - c0 < tc_max ? D - c0 : tc_max, ng = tc >> 2, rs = tc + 4;  // D is a multiple of 256
        for (int s = tid; s < nu * ng; s += RT_BLOCK) {  // slot s: row s / ng, group s % ng (64 of one row a wave)
            const int u = s / ng, q = s % ng;
            const int ee = s_u[u];
            dma16_untracked(gbl(gate_inp + (size_t)ee * D + c0 + 4 * q), (lds_void *)(buf + (size_t)u * rs + 4 * (q & ~63)));
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        for (int s = tid; s < nu * ng; s += RT_BLOCK) {  // the products in place (infer.c:922), slot by slot
            const int u = s / ng, q = s % ng;
            float4 *pe = (float4 *)(buf + (size_t)u * rs + 4 * q);
            const float4 v = *pe, xv = *(const float4 *)(xn + c0 + 4 * q);
            *pe = make_float4(__fmul_rn(v.x, xv.x), __fmul_rn(v.y, xv.y), __fmul_rn(v.z, xv.z), __fmul_rn(v.w, xv.w));
        }
        __syncthreads();
        if (w == 0 && lane < nu) {  // infer.c:916-925: the sequential chain of expert U[lane]
            const float *row = buf + (size_t)lane * rs;
            for (int q0 = 0; q0 < ng; q0 += NV) {  // ng is a multiple of 64
                // NV groups' reads at once, so that the LDS latency is paid once per 4 NV adds
                float4 v[NV];
#pragma unroll
                for (int j = 0; j < NV; j++) v[j] = *(const float4 *)(row + 4 * (q0 + j));
#pragma unroll
                for (int j = 0; j < NV; j++) {
                    chain = __fadd_rn(chain, v[j].x);
                    chain = __fadd_rn(chain, v[j].y);
                    chain = __fadd_rn(chain, v[j].z);
                    chain = __fadd_rn(chain, v[j].w);
                }
            }
        }
        __syncthreads();  // the chains are done with the tile before the next one lands
    }
    for (int e = tid; e < E; e += RT_BLOCK) sel[e] = -INFINITY;  // outside U: never chosen
    __syncthreads();
    if (w == 0 && lane < nu) {
        const int e = s_u[lane];
        const float pr = sigmoid_libm(chain);  // infer.c:1105, libm's expf bits
        p[e] = pr;
        sel[e] = __fadd_rn(pr, bias[e]);
    }
    __syncthreads();
    exact_topk(E, K, tid, p, sel, idx, wk_out, stats);
    return true;
}

// glm.c's insertion top-k (infer.c:1110-1135) on wave 0 of the block, from every expert's
// probability p and selection score sel (shared memory): the K largest sel by (value desc,
// index asc) among values above -inf (NaN is never inserted), by K wave-maximum rounds with
// the lowest lane winning ties, chunk c of lane l holding expert l + 64c; their unbiased
// p, normalised (infer.c:1136-1145), into idx / wk_out (shared, [K]). Counts the replay in
// stats. Ends with a barrier.
__device__ __attribute__((always_inline)) static void exact_topk(int E, int K, int tid, const float *p, const float *sel,
                                                                 int *idx, float *wk_out, unsigned long long *stats) {
    const int lane = tid & 63, w = tid >> 6;
    if (w == 0) {
        const int nch = (E + 63) >> 6;
        float key[RT_SEL_C], pv[RT_SEL_C];
#pragma unroll
        for (int c = 0; c < RT_SEL_C; c++) {
            const int e = lane + 64 * c;
            const bool valid = c < nch && e < E;
            const float v = valid ? sel[e] : -INFINITY;
            key[c] = v == v ? v : -INFINITY;
            pv[c] = valid ? p[e] : 0.0f;
        }
        float total = 0.0f;
        for (int k = 0; k < K; k++) {
            float bm = key[0];
#pragma unroll
            for (int c = 1; c < RT_SEL_C; c++) bm = fmaxf(bm, key[c]);
            const float gm = wave_max_dpp_f(bm);
            int ek = -1;
            float wk = -1e30f;
            if (gm > -INFINITY) {
                // the lowest expert index holding the maximum: chunks in index order
                int ls = -1, cs = 0;
#pragma unroll
                for (int c = 0; c < RT_SEL_C; c++) {
                    const unsigned long long m = __ballot(key[c] == gm);
                    if (ls < 0 && m != 0ull) {
                        ls = __ffsll(m) - 1;
                        cs = c;
                    }
                }
                float mp = pv[0];
#pragma unroll
                for (int c = 1; c < RT_SEL_C; c++)
                    if (cs == c) mp = pv[c];
                ek = ls + 64 * cs;
                wk = readlane_f(mp, ls);
                total = __fadd_rn(total, wk);
#pragma unroll
                for (int c = 0; c < RT_SEL_C; c++)
                    if (lane == ls && c == cs) key[c] = -INFINITY;
            }
            if (lane == 0) {
                idx[k] = ek;
                wk_out[k] = wk;
            }
        }
        if (lane == 0) {
            atomicAdd(&stats[GM_STAT_ROUTE_EXACT], 1ull);
            if (total > 0.0f) {
                // normalisation of infer.c:1136-1145
                const float denom = total < 6.103515625e-5f ? 6.103515625e-5f : total;
                const float inv_d = __fdiv_rn(1.0f, denom);
                for (int k = 0; k < K; k++) wk_out[k] = __fmul_rn(wk_out[k], inv_d);
            }
        }
    }
    __syncthreads();
}

#define RT_CPL_MAX (GM_MAX_COLS / 64)  // router columns per lane

// grid (T): the router of one token per block. RMSNorm bit-identical to infer.c:746-752
// (certified_mean_sq); every expert's fp64 logit with the bound of its fp32 chain, wave
// w taking experts w, w + 4, ... and lane l the D/64 consecutive columns from l D/64 (so
// a wave scan yields the chain's partial sums in glm.c's order); then, one thread per
// expert, the bounds and selection intervals; then the certified top-k on wave 0
// (certified_select) or, when it fails or is forced, the exact replay (exact_router).
// Outputs as infer.c:1098-1145 leaves them: xn, probabilities, top-k, normalised weights
// (and times routed_scale).
//
// The loop over experts is what the kernel's time goes to (512 tokens x 64 experts of
// wave work, the SIMDs shared by three blocks), so only the estimate S = sum p_k uses
// fp64 (exact products, fp64 sums and scan). The bound's terms, sum |p_k| and the sum of
// the partial sums' magnitudes, are taken in fp32 and then enlarged by their own rounding
// bound: for the lane's m columns, with r_k the fp32 running sum started from fl(R_0),
// R_0 the exact sum before the lane, and q_k = fl(p_k),
//   sum_k |R_k| <= T + m u (|R_0| + A + (1 + u) T),
//   T = sum_k |r_k| <= fl-sum * (1 + 2(m+1)u), A = sum_k |p_k| <= fl-sum |q_k| * (1 + 2(m+2)u)
// (each fp32 add or product errs by at most u relative, plus 2^-150 absolute below the
// normal range, counted as 2m 2^-149).
__global__ __launch_bounds__(RT_BLOCK) void k_router_tok(RouterArgs a) {
    __shared__ __align__(16) float s_xn[GM_MAX_COLS];
    __shared__ __align__(16) float s_prod[RT_XT][64];  // exact replay scratch
    __shared__ double red[4];
    __shared__ float s_mean, s_total;
    __shared__ unsigned long long s_w0[GM_MAX_E], s_w1[GM_MAX_E];
    __shared__ float s_p[GM_MAX_E], s_sel[GM_MAX_E], s_wk[GM_MAX_K];
    __shared__ int s_idx[GM_MAX_K], s_ok, s_u[RT_SUB_MAX], s_nu;
    __shared__ double s_S[GM_MAX_E];
    __shared__ float s_sp[GM_MAX_E], s_sa[GM_MAX_E];
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int D = a.D, E = a.E, K = a.K, cpl = D >> 6;
    const float *xt = a.x + (size_t)t * D;

    const float mean = certified_mean_sq(xt, D, red, &s_mean, true, a.stats);
    const float inv = __fdiv_rn(1.0f, sqrt_rn_f32(__fadd_rn(mean, a.eps)));
    for (int i = tid; i < D; i += RT_BLOCK) {
        const float v = __fmul_rn(__fmul_rn(xt[i], inv), a.norm_w[i]);
        s_xn[i] = v;
        a.xn[(size_t)t * D + i] = v;
    }
    __syncthreads();

    // the lane's columns of xn in registers, and each expert's gate row one expert ahead
    float xr[RT_CPL_MAX];
#pragma unroll
    for (int q = 0; q < RT_CPL_MAX / 4; q++) {
        const float4 v = q < cpl / 4 ? *(const float4 *)&s_xn[lane * cpl + 4 * q] : make_float4(0.f, 0.f, 0.f, 0.f);
        xr[4 * q] = v.x;
        xr[4 * q + 1] = v.y;
        xr[4 * q + 2] = v.z;
        xr[4 * q + 3] = v.w;
    }
    auto load_row = [&](int e, float4 *g) {
        const float4 *src = (const float4 *)(a.gate_inp + (size_t)(e < E ? e : 0) * D + lane * cpl);
#pragma unroll
        for (int q = 0; q < RT_CPL_MAX / 4; q++) g[q] = q < cpl / 4 ? src[q] : make_float4(0.f, 0.f, 0.f, 0.f);
    };
    float4 gc[RT_CPL_MAX / 4], gn[RT_CPL_MAX / 4];
    load_row(w, gc);
    for (int e = w; e < E; e += 4) {
        load_row(e + 4, gn);
        float g[RT_CPL_MAX];
#pragma unroll
        for (int q = 0; q < RT_CPL_MAX / 4; q++) {
            g[4 * q] = gc[q].x;
            g[4 * q + 1] = gc[q].y;
            g[4 * q + 2] = gc[q].z;
            g[4 * q + 3] = gc[q].w;
        }
        // xn stays 32 floats: kept opaque here so that its fp64 conversions are not
        // hoisted out of the loop as 32 live doubles
#pragma unroll
        for (int j = 0; j < RT_CPL_MAX; j++) asm volatile("" : "+v"(xr[j]));
        // pass 1: the lane's segment sum (products in fp64 are exact) and the wave's
        // exclusive prefix R_0; pass 2, in fp32: the running sum's magnitudes and |q_k|
        double seg = 0.0;
#pragma unroll
        for (int j = 0; j < RT_CPL_MAX; j++) seg += (double)g[j] * (double)xr[j];
        const double incl = wave_incl_scan_dpp(seg), r0 = incl - seg;
        float run = (float)r0, steps = 0.0f, sabs = 0.0f;
#pragma unroll
        for (int j = 0; j < RT_CPL_MAX; j++) {
            if (j < cpl) {
                const float q = __fmul_rn(g[j], xr[j]);
                run = __fadd_rn(run, q);
                steps = __fadd_rn(steps, fabsf(run));
                sabs = __fadd_rn(sabs, fabsf(q));
            }
        }
        const double u = 0x1p-24, m = (double)cpl;
        const double T = (double)steps * (1.0 + 2.0 * (m + 1.0) * u), A = (double)sabs * (1.0 + 2.0 * (m + 2.0) * u);
        const double spl = T + m * u * (fabs(r0) * (1.0 + 0x1p-40) + A + (1.0 + u) * T) + 2.0 * m * 0x1p-149;
        const double S = readlane_d(incl, 63);
        const double sp = wave_sum_dpp(spl), sa = wave_sum_dpp(A);
        if (lane == 0) {
            s_S[e] = S;
            s_sp[e] = __double2float_ru(sp);
            s_sa[e] = __double2float_ru(sa);
        }
#pragma unroll
        for (int q = 0; q < RT_CPL_MAX / 4; q++) gc[q] = gn[q];
    }
    __syncthreads();
    // every expert's bound and selection interval, one thread each
    for (int e = tid; e < E; e += RT_BLOCK) {
        const double S = s_S[e], sp = (double)s_sp[e], sa = (double)s_sa[e];
        const double u = 0x1p-24, n = (double)D;
        const double gamma = n * u / (1.0 - n * u);
        const double emax = gamma * sa;  // a priori bound on every partial sum's error
        double B = u * (1.0 + u) * sa + u * (sp + n * emax + u * sa);
        B = B * (1.0 + 0x1p-30) + 0x1p-40 * sa + n * 0x1p-149;
        double lo, hi;
        selection_interval(S, B, a.bias[e], &lo, &hi);
        float lo_f = __double2float_rd(lo), hi_f = __double2float_ru(hi);
        if (!(lo_f <= hi_f)) {  // NaN: an interval that is never certified
            lo_f = -INFINITY;
            hi_f = INFINITY;
        }
        s_w0[e] = (unsigned long long)__float_as_uint(lo_f) | ((unsigned long long)__float_as_uint(hi_f) << 32);
        s_w1[e] = (unsigned long long)__float_as_uint(1.0f / (1.0f + expf(-(float)S)));
    }
    __syncthreads();

    if (tid < 64) {
        unsigned long long w0[RT_SEL_C], w1[RT_SEL_C];
#pragma unroll
        for (int c = 0; c < RT_SEL_C; c++) {
            const int e = tid + 64 * c < E ? tid + 64 * c : E - 1;
            w0[c] = s_w0[e];
            w1[c] = s_w1[e];
        }
        if (E <= 64)
            certified_select<1>(E, K, tid, w0, w1, s_p, s_idx, s_wk, &s_ok, &s_total);
        else
            certified_select<RT_SEL_C>(E, K, tid, w0, w1, s_p, s_idx, s_wk, &s_ok, &s_total);
        if (tid == 0 && a.force_exact) s_ok = 0;
    }
    __syncthreads();
    if (s_ok) {
        if (tid < K) {  // normalisation of infer.c:1136-1145
            const float total = s_total;
            float wk = s_wk[tid];
            if (total > 0.0f) {
                const float denom = total < 6.103515625e-5f ? 6.103515625e-5f : total;
                wk = __fmul_rn(wk, __fdiv_rn(1.0f, denom));
            }
            s_wk[tid] = wk;
        }
        __syncthreads();
    } else if (a.force_exact || !exact_router_subset<16>(D, E, K, tid, a.gate_inp, a.bias, s_xn, s_prod, s_w0, s_p, s_sel,
                                                     s_idx, s_wk, a.stats, s_u, &s_nu, RT_XT * 64)) {
        exact_router(D, E, K, tid, a.gate_inp, a.bias, s_xn, s_prod, s_p, s_sel, s_idx, s_wk, a.stats);
    }
    if (tid < K) {
        const size_t o = (size_t)t * K + tid;
        a.topk_idx[o] = s_idx[tid];
        a.topk_w[o] = s_wk[tid];
        a.topk_ws[o] = __fmul_rn(s_wk[tid], a.routed_scale);
        a.hist_idx[o] = s_idx[tid];
        a.hist_w[o] = s_wk[tid];
    }
    for (int i = tid; i < E; i += RT_BLOCK) a.router_prob[(size_t)t * E + i] = s_p[i];
}

// ---------------------------------------------------------------- the router of T > 1, in three kernels
//
// For E <= 64 the router of a batch runs as k_rt_norm (rmsnorm, one block per token),
// k_rt_dots (the logits' sums) and k_rt_select (bounds, certified top-k, exact replay),
// rather than k_router_tok's one block per token: there, each expert's dot is a
// wave-wide reduction, and its fp64 scans and sums leave the SIMDs issue-bound.
// k_rt_dots gives every (token, expert, quarter of D) its own thread, which runs the
// quarter's columns in order: one fp64 FMA chain P_k (the estimate; products exact, each
// step rounds once), the sum of |P_k| in fp64 and the sum of |g_k x_k| in fp32.
// k_rt_select joins the quarters: S = t_0 + t_1 + t_2 + t_3 in order, and the bound's
// sum of the chain's partial-sum magnitudes, with Q_q the exact sum before quarter q and
// L_k the running sum inside it, as sum_{k in q} |Q_q + L_k| <= (D/4) |Q_q| + sum |L_k|.
struct RtParts {
    double *t;   // [T][4][E] quarter sums
    double *sp;  // [T][4][E] quarter sums of |running sum|
    float *sa;   // [T][4][E] quarter sums of |g x| (fp32)
};

// grid (ceil(T/4)): xn of token 4 blockIdx.x + w on wave w (infer.c:746-752),
// bit-identical to glm.c: lane l holds the row's D/64 consecutive values from l D/64, the
// mean of squares is certified from the wave's fp64 sum (relative error below D 2^-52)
// or else replayed in order by lane 0, and xn is formed from the registers.
__global__ __launch_bounds__(RT_BLOCK) void k_rt_norm(RouterArgs a, int T) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, t = 4 * blockIdx.x + w, D = a.D;
    if (t >= T) return;  // wave-uniform
    const int per = D / 64;  // a multiple of 4, at most RT_CPL_MAX
    const float *xt = a.x + (size_t)t * D;
    float xv[RT_CPL_MAX];
    if (((uintptr_t)a.x & 15) == 0) {  // the caller's x: 16-byte loads when aligned
#pragma unroll
        for (int q = 0; q < RT_CPL_MAX / 4; q++) {
            const float4 v = q < per / 4 ? *(const float4 *)(xt + lane * per + 4 * q) : make_float4(0.f, 0.f, 0.f, 0.f);
            xv[4 * q] = v.x;
            xv[4 * q + 1] = v.y;
            xv[4 * q + 2] = v.z;
            xv[4 * q + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < RT_CPL_MAX; j++) xv[j] = j < per ? xt[lane * per + j] : 0.0f;
    }
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < RT_CPL_MAX; j++) ss += (double)xv[j] * (double)xv[j];
    ss = wave_sum_dpp(ss);
    const double v = ss / (double)D, rho = (double)D * 0x1p-52;
    float mean = (float)(v * (1.0 - rho));
    if (mean != (float)(v * (1.0 + rho))) {  // wave-uniform
        double sq = 0.0;
        if (lane == 0) {
            for (int i = 0; i < D; i++) sq += (double)xt[i] * (double)xt[i];
            atomicAdd(&a.stats[GM_STAT_NORM_EXACT], 1ull);
        }
        mean = (float)(readlane_d(sq, 0) / (double)D);
    }
    const float inv = __fdiv_rn(1.0f, sqrt_rn_f32(__fadd_rn(mean, a.eps)));
#pragma unroll
    for (int q = 0; q < RT_CPL_MAX / 4; q++)
        if (q < per / 4) {
            const float4 nw = *(const float4 *)(a.norm_w + lane * per + 4 * q);
            *(float4 *)(a.xn + (size_t)t * D + lane * per + 4 * q) =
                make_float4(__fmul_rn(__fmul_rn(xv[4 * q], inv), nw.x), __fmul_rn(__fmul_rn(xv[4 * q + 1], inv), nw.y),
                            __fmul_rn(__fmul_rn(xv[4 * q + 2], inv), nw.z), __fmul_rn(__fmul_rn(xv[4 * q + 3], inv), nw.w));
        }
}

#define RT_QMAX (GM_MAX_COLS / 4)  // columns per quarter

// grid (ceil(T/4), 4): wave w takes token 4 blockIdx.x + w, lane e expert e, over the
// columns of quarter blockIdx.y. The gate rows come through shared memory in tiles of
// 64 columns, [64 experts][16 four-column groups] with group g of row e at slot
// g ^ (e % 16) (so that the 64 lanes' reads of one group spread over the banks), two
// tiles in flight; xn's quarter of the block's tokens is staged once.
#define RT_DOT_STAGES 3  // router-row tiles in shared memory: two in flight while one is used
__global__ __launch_bounds__(RT_BLOCK) void k_rt_dots(RouterArgs a, RtParts p, int T) {
    __shared__ __align__(16) float4 gt[RT_DOT_STAGES][64 * 16];
    __shared__ __align__(16) float xs[4 * RT_QMAX];  // the block's 4 tokens' quarters, Lq floats apart
    const int tg = blockIdx.x, q = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int D = a.D, E = a.E, Lq = D / 4, c0 = q * Lq, ntile = Lq / 64;
    const int t = 4 * tg + w;
    // The quarters by DMA too, issued first: Lq pieces of 16 bytes (Lq / 4 a row), 64 to a
    // wave's DMA, dealt round the waves. A token past T reads token T - 1 (its sums are not stored).
    for (int s = w; s < Lq / 64; s += 4) {
        const int piece = 64 * s + lane, tw = piece / (Lq / 4), k = 4 * (piece - tw * (Lq / 4));
        const int tt = min(4 * tg + tw, T - 1);
        dma16_untracked(gbl(a.xn + (size_t)tt * D + c0 + k), (lds_void *)(xs + 256 * s));
    }
    auto stage = [&](int j, int buf) {  // 1024 pieces of 16 bytes: four per lane
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int unit = (4 * w + i) * 64 + lane, e = unit >> 4, g = (unit & 15) ^ (e & 15);
            const int ee = e < E ? e : 0;
            dma16_untracked(gbl(a.gate_inp + (size_t)ee * D + c0 + 64 * j + 4 * g), (lds_void *)(gt[buf] + (4 * w + i) * 64));
        }
    };
    // tiles of 64 columns, two ahead. Each stage() is four DMAs a thread; the waits below
    // count them in order, so vmcnt(4) after stage(1) also covers the quarters' DMAs.
    // The barriers are s_barrier in inline assembly after an exact wait (with the shared-memory
    // stores and reads done): __syncthreads() would also wait for the DMAs still in flight.
    stage(0, 0);
    if (ntile > 1) {
        stage(1, 1);
        asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    } else {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    double acc = 0.0, sp = 0.0;
    float sa = 0.0f;
    for (int j = 0; j < ntile; j++) {
        if (j + 2 < ntile) stage(j + 2, (j + 2) % RT_DOT_STAGES);
        const float4 *gb = gt[j % RT_DOT_STAGES] + lane * 16;
        const float *xw = xs + w * Lq + 64 * j;
#pragma unroll
        for (int g = 0; g < 16; g++) {
            const float4 gv = gb[g ^ (lane & 15)];
            const float4 xv = *(const float4 *)(xw + 4 * g);
            const float gg[4] = {gv.x, gv.y, gv.z, gv.w}, xx[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                acc = fma((double)gg[c], (double)xx[c], acc);
                sp += fabs(acc);
                sa = fmaf(fabsf(gg[c]), fabsf(xx[c]), sa);
            }
        }
        // tile j + 1 is in shared memory (tile j + 2's DMAs may still be in flight), and after
        // the barrier every wave is done with tile j, whose buffer tile j + 3 refills
        if (j + 2 < ntile)
            asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        else
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    if (t < T && lane < E) {
        const size_t o = ((size_t)t * 4 + q) * E + lane;
        p.t[o] = acc;
        p.sp[o] = sp;
        p.sa[o] = sa;
    }
}

// grid (T): the quarters joined into each expert's estimate and bound (one thread per
// expert), the selection intervals, the certified top-k and, when it fails or is
// forced, the exact replay; outputs as k_router_tok.
__global__ __launch_bounds__(RT_BLOCK) void k_rt_select(RouterArgs a, RtParts p) {
    __shared__ __align__(16) float s_xn[GM_MAX_COLS];
    __shared__ __align__(16) float s_prod[RT_XT][64];  // exact replay scratch
    __shared__ float s_total;
    __shared__ unsigned long long s_w0[64], s_w1[64];
    __shared__ float s_p[GM_MAX_E], s_sel[GM_MAX_E], s_wk[GM_MAX_K];
    __shared__ int s_idx[GM_MAX_K], s_ok, s_u[RT_SUB_MAX], s_nu;
    const int t = blockIdx.x, tid = threadIdx.x;
    const int D = a.D, E = a.E, K = a.K;
    if (tid < E) {
        const int e = tid;
        const size_t o = (size_t)t * 4 * E + e;
        const double t0 = p.t[o], t1 = p.t[o + E], t2 = p.t[o + 2 * E], t3 = p.t[o + 3 * E];
        const double S = ((t0 + t1) + t2) + t3;
        const double q1 = t0, q2 = t0 + t1, q3 = q2 + t2, Lq = (double)(D / 4);
        const double u = 0x1p-24, n = (double)D;
        // (fp64 roundings of the running sums and of these sums: a relative 2^-40)
        const double sp = (p.sp[o] + (Lq * fabs(q1) + p.sp[o + E]) + (Lq * fabs(q2) + p.sp[o + 2 * E]) +
                           (Lq * fabs(q3) + p.sp[o + 3 * E])) * (1.0 + 0x1p-40);
        // each quarter's fp32 sum of |g x| (exact products inside the fma) errs by at most
        // (D/4) u relative; below the normal range by 2^-150 a step
        const double sa = (((double)p.sa[o] + (double)p.sa[o + E]) + ((double)p.sa[o + 2 * E] + (double)p.sa[o + 3 * E])) *
                              (1.0 + 2.0 * Lq * u) + n * 0x1p-149;
        const double gamma = n * u / (1.0 - n * u);
        const double emax = gamma * sa;  // a priori bound on every partial sum's error
        double B = u * (1.0 + u) * sa + u * (sp + n * emax + u * sa);
        B = B * (1.0 + 0x1p-30) + 0x1p-40 * sa + n * 0x1p-149;
        double lo, hi;
        selection_interval(S, B, a.bias[e], &lo, &hi);
        float lo_f = __double2float_rd(lo), hi_f = __double2float_ru(hi);
        if (!(lo_f <= hi_f)) {  // NaN: an interval that is never certified
            lo_f = -INFINITY;
            hi_f = INFINITY;
        }
        s_w0[e] = (unsigned long long)__float_as_uint(lo_f) | ((unsigned long long)__float_as_uint(hi_f) << 32);
        s_w1[e] = (unsigned long long)__float_as_uint(1.0f / (1.0f + expf(-(float)S)));
    }
    __syncthreads();
    if (tid < 64) {
        unsigned long long w0[1], w1[1];
        w0[0] = s_w0[tid < E ? tid : E - 1];
        w1[0] = s_w1[tid < E ? tid : E - 1];
        certified_select<1>(E, K, tid, w0, w1, s_p, s_idx, s_wk, &s_ok, &s_total);
        if (tid == 0 && a.force_exact) s_ok = 0;
    }
    __syncthreads();
    if (s_ok) {
        if (tid < K) {  // normalisation of infer.c:1136-1145
            const float total = s_total;
            float wk = s_wk[tid];
            if (total > 0.0f) {
                const float denom = total < 6.103515625e-5f ? 6.103515625e-5f : total;
                wk = __fmul_rn(wk, __fdiv_rn(1.0f, denom));
            }
            s_wk[tid] = wk;
        }
        __syncthreads();
    } else {
        for (int i = tid; i < D; i += RT_BLOCK) s_xn[i] = a.xn[(size_t)t * D + i];
        __syncthreads();
        if (a.force_exact || !exact_router_subset<16>(D, E, K, tid, a.gate_inp, a.bias, s_xn, s_prod, s_w0, s_p, s_sel, s_idx,
                                                  s_wk, a.stats, s_u, &s_nu, RT_XT * 64))
            exact_router(D, E, K, tid, a.gate_inp, a.bias, s_xn, s_prod, s_p, s_sel, s_idx, s_wk, a.stats);
    }
    if (tid < K) {
        const size_t o = (size_t)t * K + tid;
        a.topk_idx[o] = s_idx[tid];
        a.topk_w[o] = s_wk[tid];
        a.topk_ws[o] = __fmul_rn(s_wk[tid], a.routed_scale);
        a.hist_idx[o] = s_idx[tid];
        a.hist_w[o] = s_wk[tid];
    }
    for (int i = tid; i < E; i += RT_BLOCK) a.router_prob[(size_t)t * E + i] = s_p[i];
}
