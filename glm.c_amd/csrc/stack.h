// stack.h -- persistent decode kernel: T=1 through a run of MoE layers in one launch.
//
// A decode step is a chain of small, strictly dependent phases per layer
// (infer.c:1087-1216):  x -> rmsnorm + router -> top-k -> gate/up (K+1 experts) ->
// down (K+1 experts) + combine -> x'.  Each phase moves 1-35 MB, a few microseconds of
// HBM time, so kernel boundaries (~2 us each on this GPU) would cost as much as the
// work. Instead one grid of co-resident blocks walks a per-layer work list in
// topological order:
//   router items   2 experts each: rmsnorm (bit-exact) + fp64 logits and error bounds;
//                  every routed item then certifies the top-k itself (see router.h)
//   gate/up items  (slot, 16-row panel): gate and up rows of one expert panel
//   down items     (slot, 16-row panel of D): h = silu(gate) * up, then down; the last
//                  slot item of a panel forms x' = x + (shared + sum_k w_k y_k)
// Blocks have roles (router, shared expert, routed experts) and walk the layers in
// order; an item only waits for items of the same or an earlier layer that come before
// it in their role's order, so with all blocks resident some unfinished item can always run.
//
// Memory ordering without cache flushes. Every activation buffer is per layer and is
// written exactly once per launch, by write-through (agent-scope) stores; a producer
// waits for its stores to complete (s_waitcnt) before bumping a monotonic counter, and a
// consumer polls the counter (agent-scope loads, bounded spin, then an error flag instead
// of a hang) before reading. Since no cache line of a per-layer buffer is touched before
// it is produced, and caches start clean at a kernel boundary, consumers may read it with
// ordinary cached loads: each XCD fetches it from memory once, into its own L2.
#pragma once

#include "common.h"
#include "experts.h"
#include "router.h"

#define SK_BLOCK 256
#define SK_MAX_SLOTS 9           // K + 1 <= 9
#define SK_SPIN_LIMIT (1u << 22) // polls before a wait is declared dead (~seconds)
#define SK_TRACE_STAMPS 16
#define SK_RX 4                  // experts per router item: one per wave

// Counters sit 64 words (256 bytes) apart: polls of one never share a cache line, or a
// memory channel's hot spot, with another.
#define SKC_PAD 64
enum { SKC_ROUTER = 0, SKC_DIG = 2, SKC_X = 3, SKC_GATE = 4, SKC_PANEL = 16 };
#define SKC(i) ((i) * SKC_PAD)
// per-layer flags of the exact top-k replay, after the D/16 panel counters
#define SKC_CLAIM(np, li) SKC(SKC_PANEL + (np) + 2 * (li))
#define SKC_EXACT(np, li) SKC(SKC_PANEL + (np) + 2 * (li) + 1)

struct StackLayer {
    const uint8_t *experts;
    const float *norm;
    const float *gate_inp;
    const float *bias;
    int has_routed;
    int pad;
};

// Per-layer workspace: one region of `ws_layer_bytes` per layer of the launch.
struct StackWs {
    size_t x, xn, dig, dexp, stage, ex_idx, ex_w, ex_p, g, u, y;  // byte offsets inside a layer region
};

struct StackArgs {
    const StackLayer *layers;  // [n_layers], relative to first_layer
    int n_layers, first_layer;
    const float *x_in;
    float *x_out;
    int D, F, E, K, flags;
    float eps, routed_scale;
    size_t stride, off_gq, off_uq, off_dq, off_gs, off_us, off_ds;
    uint8_t *ws;               // per-layer workspace base
    size_t ws_layer_bytes;
    StackWs o;
    // observables of the most recent layer, written through
    float *xn;                 // [D]
    float *router_prob;        // [E]
    int *topk_idx;             // [K]
    float *topk_w;             // [K]
    float *shared_out;         // [D]
    float *routed_out;         // [D]
    int *hist_idx;             // + layer * hist_stride
    float *hist_w;
    int hist_stride;
    unsigned *ctr;             // counters, zero at launch
    unsigned long long *stats;
    int *error;                // nonzero: a wait timed out
    unsigned long long *trace; // optional: SK_TRACE_STAMPS timestamps per item (see k_moe_stack)
    int shared_blocks;         // blocks in the shared-expert role
};

template <typename T>
__device__ static inline T *ws_at(const StackArgs &a, int li, size_t off) {
    return (T *)(a.ws + (size_t)li * a.ws_layer_bytes + off);
}

__device__ static inline void st_f(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ static inline void st_i(int *p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ static inline void st_d(double *p, double v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ static inline void st_u64(unsigned long long *p, unsigned long long v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ static inline unsigned ld_u(const unsigned *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

struct SkShared {
    union {
        struct {  // router item: xn at padded positions, see rpad()
            float xn[GM_MAX_COLS + GM_MAX_COLS / 32];
        } r;
        struct {  // top-k selection and its exact replay
            double lo[GM_MAX_E], hi[GM_MAX_E], mid[GM_MAX_E];
            float p[GM_MAX_E], sel[GM_MAX_E];
            float xn[GM_MAX_COLS];
            float prod[64][17];  // products of 64 experts x 16 columns
        } s;
        struct {  // expert panels
            int8_t dig[3 * GM_MAX_COLS];
            int dexp[GM_MAX_COLS / 32];
            float part[EX_WAVES][16];
            float part2[EX_WAVES][16];
        } g;
    } u;
    double red[4];
    float mean;
    unsigned old;
    int ok, sel_ok;
    float total;
    int idx[GM_MAX_K];
    float wk[GM_MAX_K], ws[GM_MAX_K];
    long trace_item;
    unsigned long long *trace;
};

// All of this block's write-through stores have completed; then thread 0 bumps `c`.
// With `need_old` the previous counter value is returned to every thread.
__device__ static inline unsigned publish(unsigned *c, SkShared &sh, bool need_old) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        if (need_old) sh.old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!need_old) return 0;
    __syncthreads();
    return sh.old;
}

// Block-wide wait until *c >= target. Returns false if the wait timed out or another
// block already failed (the caller then returns from the kernel).
__device__ static inline bool wait_ge(const unsigned *c, unsigned target, int *error, SkShared &sh) {
    if (threadIdx.x == 0) {
        int ok = 1;
        unsigned spins = 0;
        while (ld_u(c) < target) {
            if (__hip_atomic_load(error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                ok = 0;
                break;
            }
            if (++spins > SK_SPIN_LIMIT) {
                __hip_atomic_store(error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(8);  // ~512 clocks between polls
        }
        sh.ok = ok;
        if (sh.trace) sh.trace[SK_TRACE_STAMPS * sh.trace_item + 1] = wall_clock64();
    }
    __syncthreads();
    return sh.ok != 0;
}

// Diagnostic stamp k of the current item (thread 0, when tracing).
__device__ static inline void sk_stamp(SkShared &sh, int k) {
    if (sh.trace && threadIdx.x == 0) sh.trace[SK_TRACE_STAMPS * sh.trace_item + k] = wall_clock64();
}

// ---------------------------------------------------------------- router item
#define SK_RCOLS 32  // router columns per lane: D <= 64 * 32

// Column i = l * cpl + j of the router's normalised activations (lane l's segment of cpl
// columns) sits at l * (cpl + 1) + j in shared memory. cpl is a multiple of 4, so cpl + 1
// is odd and the 64 lanes reading their own segments start on 64 different banks instead
// of sharing two.
__device__ static inline int rpad(int i, int cpl) { return i + i / cpl; }

__device__ __attribute__((always_inline)) static bool sk_router_item(const StackArgs &a, const StackLayer &L,
                                                                     int layer, int li, int r0, SkShared &sh) {
    const int D = a.D, E = a.E, tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int per = D / SK_BLOCK;  // norm columns per thread, D a multiple of 256
    const int cpl = D / 64;        // router columns per lane
    const int e = r0 * SK_RX + w;  // this wave's expert
    // The router row and the norm weights do not depend on x: fetch them before waiting.
    // Every load is unconditional (indices past the end are clamped and the values
    // replaced by zeros afterwards), so all of them are in flight at once.
    float gw[SK_RCOLS], nw[8];
    const GM_GLOBAL float *nrm = gbl(L.norm);
#pragma unroll
    for (int j = 0; j < 8; j++) nw[j] = nrm[tid * per + (j < per ? j : 0)];
    {
        const GM_GLOBAL float *g = gbl(L.gate_inp + (size_t)(e < E ? e : 0) * D + (size_t)lane * cpl);
#pragma unroll
        for (int j = 0; j < SK_RCOLS; j++) gw[j] = g[j < cpl ? j : 0];
#pragma unroll
        for (int j = 0; j < SK_RCOLS; j++) gw[j] = j < cpl ? gw[j] : 0.0f;
    }
    if (li > 0 && !wait_ge(&a.ctr[SKC(SKC_X)], (unsigned)li * (D >> 4), a.error, sh)) return false;
    const float *xsrc = li == 0 ? a.x_in : ws_at<float>(a, li, a.o.x);

    // rmsnorm, bit-identical to infer.c:746-752. Thread tid holds columns tid*per..+per,
    // inside lane tid/4's router segment (cpl = 4 * per).
    const int xn_at = (tid >> 2) * (cpl + 1) + (tid & 3) * per;
    float xv[8];
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < 8; j++) xv[j] = xsrc[tid * per + (j < per ? j : 0)];
#pragma unroll
    for (int j = 0; j < 8; j++)
        if (j < per) ss += (double)xv[j] * (double)xv[j];
    ss = block_sum_fast(ss, sh.red);
    sk_stamp(sh, 11);
    const double v = ss / (double)D, rho = (double)D * 0x1p-52;
    const float mlo = (float)(v * (1.0 - rho)), mhi = (float)(v * (1.0 + rho));
    float mean = mlo;
    if (mlo != mhi) {
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (j < per) sh.u.r.xn[xn_at + j] = xv[j];
        __syncthreads();
        if (tid == 0) {
            double sq = 0.0;
            for (int i = 0; i < D; i++) sq += (double)sh.u.r.xn[rpad(i, cpl)] * (double)sh.u.r.xn[rpad(i, cpl)];
            sh.mean = (float)(sq / (double)D);
            if (r0 == 0) atomicAdd(&a.stats[GM_STAT_NORM_EXACT], 1ull);
        }
        __syncthreads();
        mean = sh.mean;
        __syncthreads();
    }
    const float inv = __fdiv_rn(1.0f, sqrt_rn_f32(__fadd_rn(mean, a.eps)));
#pragma unroll
    for (int j = 0; j < 8; j++)
        if (j < per) {
            xv[j] = __fmul_rn(__fmul_rn(xv[j], inv), nw[j]);
            sh.u.r.xn[xn_at + j] = xv[j];
        }
    __syncthreads();

    if (r0 == 0) {
        // publish xn and its digit form for this layer's gate/up items: 8 consecutive
        // columns per thread, four threads per 32-column block
        int8_t *dig = ws_at<int8_t>(a, li, a.o.dig);
        int *dexp = ws_at<int>(a, li, a.o.dexp);
        float *wxn = ws_at<float>(a, li, a.o.xn);
        for (int i0 = tid * 8; i0 < D; i0 += SK_BLOCK * 8) {
            float vals[8];
            float mx = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                vals[j] = sh.u.r.xn[rpad(i0 + j, cpl)];
                mx = fmaxf(mx, fabsf(vals[j]));
                st_f(a.xn + i0 + j, vals[j]);
                st_f(wxn + i0 + j, vals[j]);
            }
            mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
            const int ex = digit_exponent(mx);
            unsigned long long w0 = 0, w1 = 0, w2 = 0;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                int8_t d0, d1, d2;
                split_digits(vals[j], ex, &d0, &d1, &d2);
                w0 |= (unsigned long long)(uint8_t)d0 << (8 * j);
                w1 |= (unsigned long long)(uint8_t)d1 << (8 * j);
                w2 |= (unsigned long long)(uint8_t)d2 << (8 * j);
            }
            st_u64((unsigned long long *)(dig + i0), w0);
            st_u64((unsigned long long *)(dig + D + i0), w1);
            st_u64((unsigned long long *)(dig + 2 * D + i0), w2);
            if ((tid & 3) == 0) st_i(dexp + (i0 >> 5), ex);
        }
        publish(&a.ctr[SKC(SKC_DIG)], sh, false);
        sk_stamp(sh, 12);
    }

    // Logit of expert e in fp64, and a rigorous bound on how far glm.c's sequential fp32
    // chain (infer.c:916-925) can be from it. Lane l owns columns [l*cpl, (l+1)*cpl), so
    // the exact partial sums S_k run in lane order.
    // gw[j] is 0 for j >= cpl, so those terms add exact zeros
    float xr[SK_RCOLS];
#pragma unroll
    for (int j = 0; j < SK_RCOLS; j++) xr[j] = sh.u.r.xn[lane * (cpl + 1) + j];  // <= 63 * 33 + 31
#pragma unroll
    for (int j = 0; j < SK_RCOLS; j++) xr[j] = j < cpl ? xr[j] : 0.0f;  // neighbours' or unset words
    double seg = 0.0, seg_abs = 0.0;
#pragma unroll
    for (int j = 0; j < SK_RCOLS; j++) {
        const double pj = (double)gw[j] * (double)xr[j];
        seg += pj;
        seg_abs += fabs(pj);
    }
    const double incl = wave_incl_scan_dpp(seg);
    double run = incl - seg, steps = 0.0;
#pragma unroll
    for (int j = 0; j < SK_RCOLS; j++) {
        run += (double)gw[j] * (double)xr[j];
        steps += fabs(run);
    }
    const double S = readlane_d(incl, 63);
    const double sp = wave_sum_dpp(steps), sa = wave_sum_dpp(seg_abs);
    sk_stamp(sh, 13);
    if (lane == 0 && e < E) {
        const double u = 0x1p-24, n = (double)D;
        const double gamma = n * u / (1.0 - n * u);
        const double emax = gamma * sa;  // a priori bound on every partial sum's error
        // step k rounds |fl(s_{k-1}) + fl(p_k)| <= |S_k| + emax + u|p_k| by at most u times
        // that, and each product adds u|p_k|
        double B = u * (1.0 + u) * sa + u * (sp + n * emax + u * sa);
        B = B * (1.0 + 0x1p-30) + 0x1p-40 * sa + n * 0x1p-149;
        double2 *stage = ws_at<double2>(a, li, a.o.stage);
        st_d(&stage[e].x, S);
        st_d(&stage[e].y, B);
    }
    sk_stamp(sh, 5);
    publish(&a.ctr[SKC(SKC_ROUTER)], sh, false);
    return true;
}

// Top-k of layer li (infer.c:1108-1145) into sh.idx / sh.wk (normalised) / sh.ws (times
// routed_scale) from the router items' (S, B) table, and the router probabilities of all
// experts into sh.u.s.p.
//
// Fast path, wave 0 alone: lane l holds experts l + 64c. The K best interval midpoints are
// taken one at a time (a wave maximum, then the lowest lane holding it), and the result is
// certified when each chosen interval lies strictly above the next chosen one and the
// last chosen lies strictly above every expert left out. glm.c's insertion top-k orders
// strictly by value, so it must then pick the same experts in the same order. Otherwise,
// or when any interval is not finite, one block replays the fp32 router exactly.
#define SK_SEL_C (GM_MAX_E / 64)

__device__ __attribute__((always_inline)) static bool sk_select(const StackArgs &a, const StackLayer &L, int li, SkShared &sh) {
    const int D = a.D, E = a.E, K = a.K, tid = threadIdx.x;
    const int n_items = (E + SK_RX - 1) / SK_RX;
    if (!wait_ge(&a.ctr[SKC(SKC_ROUTER)], (unsigned)(li + 1) * n_items, a.error, sh)) return false;
    sk_stamp(sh, 8);
    const GM_GLOBAL float *bias = gbl(L.bias);
    if (tid < 64) {
        const double2 *stage = ws_at<double2>(a, li, a.o.stage);
        double2 sb[SK_SEL_C];
        float bb[SK_SEL_C];
#pragma unroll
        for (int c = 0; c < SK_SEL_C; c++) {  // all loads in flight at once
            const int e = tid + 64 * c < E ? tid + 64 * c : E - 1;
            sb[c] = stage[e];
            bb[c] = bias[e];
        }
        double lo[SK_SEL_C], hi[SK_SEL_C], mid[SK_SEL_C];
        float pr[SK_SEL_C];
        bool bad = false;
#pragma unroll
        for (int c = 0; c < SK_SEL_C; c++) {
            lo[c] = hi[c] = mid[c] = -INFINITY;
            pr[c] = 0.0f;
            if (64 * c < E) {  // wave-uniform
                const int e = tid + 64 * c;
                double l, h;
                selection_interval(sb[c].x, sb[c].y, bb[c], &l, &h);
                const float pe = 1.0f / (1.0f + expf(-(float)sb[c].x));
                if (e < E) {
                    sh.u.s.p[e] = pe;
                    bad |= !(isfinite(l) && isfinite(h));
                    lo[c] = l;
                    hi[c] = h;
                    mid[c] = 0.5 * (l + h);
                    pr[c] = pe;
                }
            }
        }
        bool ok = __ballot(bad) == 0;
        double prev_lo = 0.0;
        float total = 0.0f;
        for (int k = 0; k < K; k++) {
            double bm = mid[0];
            int bc = 0;
#pragma unroll
            for (int c = 1; c < SK_SEL_C; c++)
                if (mid[c] > bm) {
                    bm = mid[c];
                    bc = c;
                }
            const double gm = wave_max_dpp(bm);
            int ek = -1;
            float wk = -1e30f;
            if (gm > -INFINITY) {  // fewer than K experts leave the rest at -1 (infer.c:1110-1113)
                const int ls = __ffsll(__ballot(bm == gm)) - 1;
                const int cs = __builtin_amdgcn_readlane(bc, ls);
                double ml = lo[0], mh = hi[0];
                float mp = pr[0];
#pragma unroll
                for (int c = 1; c < SK_SEL_C; c++)
                    if (bc == c) {
                        ml = lo[c];
                        mh = hi[c];
                        mp = pr[c];
                    }
                const double lk = readlane_d(ml, ls), hk = readlane_d(mh, ls);
                if (k > 0 && !(prev_lo > hk)) ok = false;
                prev_lo = lk;
                ek = ls + 64 * cs;
                wk = readlane_f(mp, ls);
                total = __fadd_rn(total, wk);
#pragma unroll
                for (int c = 0; c < SK_SEL_C; c++)
                    if (tid == ls && c == cs) mid[c] = -INFINITY;
            }
            if (tid == 0) {
                sh.idx[k] = ek;
                sh.wk[k] = wk;
            }
        }
        // the last chosen must lie above every expert left out (chosen ones now hold -inf)
        double rest = -INFINITY;
#pragma unroll
        for (int c = 0; c < SK_SEL_C; c++)
            if (mid[c] > -INFINITY) rest = fmax(rest, hi[c]);
        rest = wave_max_dpp(rest);
        if (rest > -INFINITY && !(prev_lo > rest)) ok = false;
        if (tid == 0) {
            sh.sel_ok = ok;
            sh.total = total;
        }
    }
    __syncthreads();
    int *ex_idx = ws_at<int>(a, li, a.o.ex_idx);
    float *ex_w = ws_at<float>(a, li, a.o.ex_w);
    float *ex_p = ws_at<float>(a, li, a.o.ex_p);
    const int NPD = D >> 4;
    if (sh.sel_ok) {
        // normalisation of infer.c:1137-1145
        if (tid < K) {
            const float total = sh.total;
            if (total > 0.0f) {
                const float denom = total < 6.103515625e-5f ? 6.103515625e-5f : total;
                sh.wk[tid] = __fmul_rn(sh.wk[tid], __fdiv_rn(1.0f, denom));
            }
        }
    } else {
        // The proof failed: one block replays glm.c's router exactly, the others wait for it.
        if (tid == 0)
            sh.old = __hip_atomic_fetch_add(&a.ctr[SKC_CLAIM(NPD, li)], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        if (sh.old == 0) {
            const float *wxn = ws_at<float>(a, li, a.o.xn);
            for (int i = tid; i < D; i += SK_BLOCK) sh.u.s.xn[i] = wxn[i];
            // infer.c:916-925 for every expert, 16 columns at a time: all threads form the
            // products fl(g * xn), then lane e adds its expert's 16 in order.
            float chain[GM_MAX_E / 64];
            for (int c = 0; c < GM_MAX_E / 64; c++) chain[c] = 0.0f;
            const GM_GLOBAL float *gi = gbl(L.gate_inp);
            for (int eb = 0; eb < E; eb += 64) {
                const int ne = E - eb < 64 ? E - eb : 64;
                for (int c0 = 0; c0 < D; c0 += 16) {
                    __syncthreads();
                    for (int i = tid; i < ne * 16; i += SK_BLOCK) {
                        const int er = i >> 4, cc = i & 15;
                        sh.u.s.prod[er][cc] = __fmul_rn(gi[(size_t)(eb + er) * D + c0 + cc], sh.u.s.xn[c0 + cc]);
                    }
                    __syncthreads();
                    if (tid < ne) {
                        float acc = chain[eb >> 6];
                        for (int cc = 0; cc < 16; cc++) acc = __fadd_rn(acc, sh.u.s.prod[tid][cc]);
                        chain[eb >> 6] = acc;
                    }
                }
                __syncthreads();
                if (tid < ne) {
                    const float pr = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-chain[eb >> 6])));
                    sh.u.s.p[eb + tid] = pr;
                    sh.u.s.sel[eb + tid] = __fadd_rn(pr, bias[eb + tid]);
                }
            }
            __syncthreads();
            if (tid == 0) {
                atomicAdd(&a.stats[GM_STAT_ROUTE_EXACT], 1ull);
                int idx[GM_MAX_K];
                for (int k = 0; k < K; k++) idx[k] = -1;
                for (int i = 0; i < E; i++) {
                    const float sc = sh.u.s.sel[i];
                    int at = -1;
                    for (int k = 0; k < K && at < 0; k++) {
                        const float held = idx[k] >= 0 ? sh.u.s.sel[idx[k]] : -INFINITY;
                        if (sc > held) at = k;
                    }
                    if (at < 0) continue;
                    for (int k = K - 1; k > at; k--) idx[k] = idx[k - 1];
                    idx[at] = i;
                }
                // libm's expf may differ from the GPU's by an ulp: flag orders decided that closely
                int unresolved = 0;
                for (int k = 0; k < K; k++) {
                    if (idx[k] < 0) continue;
                    const float a0 = sh.u.s.sel[idx[k]];
                    const float tol = 4.0f * fmaxf(fabsf(a0), 1e-30f) * 0x1p-23f + 4.0f * 0x1p-24f;
                    for (int i = 0; i < E; i++) {
                        if (i == idx[k]) continue;
                        bool above = false;
                        for (int q = 0; q < k; q++) above |= (idx[q] == i);
                        if (!above && fabsf(sh.u.s.sel[i] - a0) <= tol) unresolved = 1;
                    }
                }
                if (unresolved) atomicAdd(&a.stats[GM_STAT_UNRESOLVED], 1ull);
                float total = 0.0f;
                for (int k = 0; k < K; k++) {
                    sh.idx[k] = idx[k];
                    sh.wk[k] = idx[k] >= 0 ? sh.u.s.p[idx[k]] : -1e30f;
                    if (idx[k] >= 0) total = __fadd_rn(total, sh.wk[k]);
                }
                if (total > 0.0f) {
                    const float denom = total < 6.103515625e-5f ? 6.103515625e-5f : total;
                    const float inv_d = __fdiv_rn(1.0f, denom);
                    for (int k = 0; k < K; k++) sh.wk[k] = __fmul_rn(sh.wk[k], inv_d);
                }
                for (int k = 0; k < K; k++) {
                    st_i(ex_idx + k, sh.idx[k]);
                    st_f(ex_w + k, sh.wk[k]);
                }
            }
            for (int i = tid; i < E; i += SK_BLOCK) st_f(ex_p + i, sh.u.s.p[i]);
            publish(&a.ctr[SKC_EXACT(NPD, li)], sh, false);
        } else {
            if (!wait_ge(&a.ctr[SKC_EXACT(NPD, li)], 1u, a.error, sh)) return false;
            if (tid < K) {
                sh.idx[tid] = ex_idx[tid];
                sh.wk[tid] = ex_w[tid];
            }
            for (int i = tid; i < E; i += SK_BLOCK) sh.u.s.p[i] = ex_p[i];
        }
    }
    __syncthreads();
    if (tid < K) sh.ws[tid] = __fmul_rn(sh.wk[tid], a.routed_scale);
    __syncthreads();
    sk_stamp(sh, 3);
    return true;
}

// Observables of layer `layer` (top-k, weights, router probabilities), written through
// right after sk_select.
__device__ static void sk_write_routing(const StackArgs &a, int layer, SkShared &sh) {
    const int tid = threadIdx.x;
    if (tid < a.K) {
        st_i(a.topk_idx + tid, sh.idx[tid]);
        st_f(a.topk_w + tid, sh.wk[tid]);
        st_i(a.hist_idx + (size_t)layer * a.hist_stride + tid, sh.idx[tid]);
        st_f(a.hist_w + (size_t)layer * a.hist_stride + tid, sh.wk[tid]);
    }
    for (int i = tid; i < a.E; i += SK_BLOCK) st_f(a.router_prob + i, sh.u.s.p[i]);
}

// ---------------------------------------------------------------- gate / up item
__device__ __attribute__((always_inline)) static bool sk_gate_up_item(const StackArgs &a, const StackLayer &L, int li,
                                                                      int slot, int p, int e, SkShared &sh) {
    const int D = a.D, F = a.F;
    if (e >= 0) {
        const uint8_t *base = L.experts + (size_t)e * a.stride;
        PanelRegs<2, EX_NB_MAX> pr;
        panel_load<2, EX_NB_MAX>(pr, base + a.off_gq, (const __half *)(base + a.off_gs), base + a.off_uq,
                                 (const __half *)(base + a.off_us), p, D);
        if (!wait_ge(&a.ctr[SKC(SKC_DIG)], (unsigned)(li + 1), a.error, sh)) return false;
        const unsigned long long *dig = ws_at<unsigned long long>(a, li, a.o.dig);
        const int *dexp = ws_at<int>(a, li, a.o.dexp);
        for (int i = threadIdx.x; i < (3 * D) / 8; i += SK_BLOCK) ((unsigned long long *)sh.u.g.dig)[i] = dig[i];
        for (int i = threadIdx.x; i < D / 32; i += SK_BLOCK) sh.u.g.dexp[i] = dexp[i];
        __syncthreads();
        sk_stamp(sh, 6);
        float gu[2];
        panel_compute<2, EX_NB_MAX>(pr, D, sh.u.g.dig, sh.u.g.dexp, gu);
        sk_stamp(sh, 4);
        const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
        if (lane < 16) {
            sh.u.g.part[w][lane] = gu[0];
            sh.u.g.part2[w][lane] = gu[1];
        }
        __syncthreads();
        if (threadIdx.x < 16) {
            const int l = threadIdx.x;
            float *go = ws_at<float>(a, li, a.o.g) + (size_t)slot * F;
            float *uo = ws_at<float>(a, li, a.o.u) + (size_t)slot * F;
            st_f(go + (size_t)p * 16 + l, ((sh.u.g.part[0][l] + sh.u.g.part[1][l]) + sh.u.g.part[2][l]) + sh.u.g.part[3][l]);
            st_f(uo + (size_t)p * 16 + l, ((sh.u.g.part2[0][l] + sh.u.g.part2[1][l]) + sh.u.g.part2[2][l]) + sh.u.g.part2[3][l]);
        }
    }
    sk_stamp(sh, 5);
    publish(&a.ctr[SKC(SKC_GATE + slot)], sh, false);
    return true;
}

// ---------------------------------------------------------------- down item (+ combine)
// Down item of `slot` (expert e, -1 when idle) and 16-row panel p. A routed slot stores its
// output already multiplied by its routing weight, w_e * y (infer.c:1189-1192), and an idle
// slot stores zeros, so the combine needs no routing: adding +0.0 to the running sum,
// which is never -0.0, leaves it unchanged, as skipping the slot does.
__device__ __attribute__((always_inline)) static bool sk_down_item(const StackArgs &a, const StackLayer &L, int li, int slot,
                                                                   int p, int e, bool routed_on, SkShared &sh) {
    const int D = a.D, F = a.F, K = a.K, NS = a.K + 1;
    if (e >= 0) {
        const uint8_t *base = L.experts + (size_t)e * a.stride;
        PanelRegs<1, EX_NB_MAX> pr;
        panel_load<1, EX_NB_MAX>(pr, base + a.off_dq, (const __half *)(base + a.off_ds), nullptr, nullptr, p, F);
        if (!wait_ge(&a.ctr[SKC(SKC_GATE + slot)], (unsigned)(li + 1) * (F >> 4), a.error, sh)) return false;
        // h = silu(gate) * up (infer.c:1188, 1202), then its digit form in shared memory
        const float *gs = ws_at<float>(a, li, a.o.g) + (size_t)slot * F;
        const float *us = ws_at<float>(a, li, a.o.u) + (size_t)slot * F;
        for (int i0 = threadIdx.x * 8; i0 < F; i0 += SK_BLOCK * 8) {
            float vals[8];
            float mx = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const float gv = gs[i0 + k];
                vals[k] = gv / (1.0f + expf(-gv)) * us[i0 + k];
                mx = fmaxf(mx, fabsf(vals[k]));
            }
            mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
            const int ex = digit_exponent(mx);
            unsigned long long w0 = 0, w1 = 0, w2 = 0;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                int8_t d0, d1, d2;
                split_digits(vals[k], ex, &d0, &d1, &d2);
                w0 |= (unsigned long long)(uint8_t)d0 << (8 * k);
                w1 |= (unsigned long long)(uint8_t)d1 << (8 * k);
                w2 |= (unsigned long long)(uint8_t)d2 << (8 * k);
            }
            *(unsigned long long *)(sh.u.g.dig + i0) = w0;
            *(unsigned long long *)(sh.u.g.dig + F + i0) = w1;
            *(unsigned long long *)(sh.u.g.dig + 2 * F + i0) = w2;
            if ((threadIdx.x & 3) == 0) sh.u.g.dexp[i0 >> 5] = ex;
        }
        __syncthreads();
        sk_stamp(sh, 6);
        float yv;
        panel_compute<1, EX_NB_MAX>(pr, F, sh.u.g.dig, sh.u.g.dexp, &yv);
        sk_stamp(sh, 4);
        const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
        if (lane < 16) sh.u.g.part[w][lane] = yv;
        __syncthreads();
        if (threadIdx.x < 16) {
            const int l = threadIdx.x;
            float *y = ws_at<float>(a, li, a.o.y) + (size_t)slot * D;
            const float yv = ((sh.u.g.part[0][l] + sh.u.g.part[1][l]) + sh.u.g.part[2][l]) + sh.u.g.part[3][l];
            st_f(y + (size_t)p * 16 + l, slot < K ? __fmul_rn(sh.ws[slot], yv) : yv);
        }
    } else if (routed_on && slot < K && threadIdx.x < 16) {
        st_f(ws_at<float>(a, li, a.o.y) + (size_t)slot * D + (size_t)p * 16 + threadIdx.x, 0.0f);
    }
    sk_stamp(sh, 5);
    const unsigned old = publish(&a.ctr[SKC(SKC_PANEL + p)], sh, true);
    sk_stamp(sh, 7);
    if (old != (unsigned)((li + 1) * NS - 1)) return true;
    // last slot of this panel: combine (infer.c:1192, 1212-1214)
    if (threadIdx.x < 16) {
        const int r = p * 16 + threadIdx.x;
        const float *y = ws_at<float>(a, li, a.o.y);
        float acc = 0.0f;
        if (routed_on) {
            float yk[GM_MAX_K];
#pragma unroll
            for (int k = 0; k < GM_MAX_K; k++) yk[k] = y[(size_t)(k < K ? k : 0) * D + r];
#pragma unroll
            for (int k = 0; k < GM_MAX_K; k++)
                if (k < K) acc = __fadd_rn(acc, yk[k]);
        }
        const float shv = y[(size_t)K * D + r];
        const float xr = (li == 0 ? a.x_in : ws_at<float>(a, li, a.o.x))[r];
        st_f(a.routed_out + r, acc);
        st_f(a.shared_out + r, shv);
        float *xo = li == a.n_layers - 1 ? a.x_out : ws_at<float>(a, li + 1, a.o.x);
        st_f(xo + r, __fadd_rn(xr, __fadd_rn(shv, acc)));
    }
    publish(&a.ctr[SKC(SKC_X)], sh, false);
    return true;
}

__global__ __launch_bounds__(SK_BLOCK) void k_stack_reset(unsigned *ctr, int n, int *error) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) ctr[i] = 0u;
    if (threadIdx.x == 0) *error = 0;
}

__device__ static inline unsigned long long sk_now() { return wall_clock64(); }


// Block roles. The first n_router blocks compute the router items, the next
// a.shared_blocks blocks the shared expert, the rest the routed experts; each role walks
// the layers in order, so a block never holds an item that is ready later than the
// items other blocks of its role are waiting to start.
__global__ __launch_bounds__(SK_BLOCK, 2) void k_moe_stack(StackArgs a) {
    __shared__ SkShared sh;
    sh.trace = a.trace;
    const int K = a.K, NS = K + 1;
    const int NPF = a.F >> 4, NPD = a.D >> 4;
    const int NR = (a.E + SK_RX - 1) / SK_RX, NSB = a.shared_blocks, NWB = (int)gridDim.x - NR - NSB;
    const int per_layer = NR + NS * NPF + NS * NPD;  // trace numbering of one layer's items
    const int b = blockIdx.x;
    for (int li = 0; li < a.n_layers; li++) {
        const StackLayer L = a.layers[li];
        const int layer = a.first_layer + li;
        const long base = (long)li * per_layer;
        bool ok = true;
#define SK_ITEM(idx, call)                                                              \
    do {                                                                                \
        sh.trace_item = base + (idx);                                                   \
        if (a.trace && threadIdx.x == 0) a.trace[SK_TRACE_STAMPS * sh.trace_item] = sk_now(); \
        ok = (call);                                                                    \
        if (!ok) return;                                                                \
        if (a.trace && threadIdx.x == 0) a.trace[SK_TRACE_STAMPS * sh.trace_item + 2] = sk_now(); \
        __syncthreads();                                                                \
    } while (0)
        const bool routed_on = !(a.flags & 1) && L.has_routed;
        if (b < NR) {
            SK_ITEM(b, sk_router_item(a, L, layer, li, b, sh));
        } else if (b < NR + NSB) {
            const int sb = b - NR;
            for (int p = sb; p < NPF; p += NSB) SK_ITEM(NR + p, sk_gate_up_item(a, L, li, K, p, a.E, sh));
            for (int p = sb; p < NPD; p += NSB) SK_ITEM(NR + NPF + p, sk_down_item(a, L, li, K, p, a.E, routed_on, sh));
        } else {
            const int wb = b - NR - NSB;
            // the first routed block records the routing, also when routed experts are off
            if (routed_on || wb == 0) {
                sh.trace_item = base + NR + NPF + NPD + wb;
                if (!sk_select(a, L, li, sh)) return;
                if (wb == 0) sk_write_routing(a, layer, sh);
            }
            for (int i = wb; i < K * NPF; i += NWB) {
                const int slot = i / NPF;
                SK_ITEM(NR + NPF + NPD + i, sk_gate_up_item(a, L, li, slot, i % NPF, routed_on ? sh.idx[slot] : -1, sh));
            }
            for (int i = wb; i < K * NPD; i += NWB) {
                const int slot = i / NPD;
                SK_ITEM(NR + NPF + NPD + K * NPF + i,
                        sk_down_item(a, L, li, slot, i % NPD, routed_on ? sh.idx[slot] : -1, routed_on, sh));
            }
        }
#undef SK_ITEM
        (void)ok;
    }
}
