// stack.h -- persistent decode kernel: T=1 through a run of MoE layers in one launch.
//
// A decode step is a chain of small, strictly dependent phases per layer
// (infer.c:1087-1216):  x -> rmsnorm + router -> top-k -> gate/up (5 experts) ->
// down (5 experts) + combine -> x'.  Each phase moves 1-35 MB, a few microseconds of
// HBM time, so kernel boundaries (~2 us each on this GPU) would cost as much as the
// work. Instead one grid of co-resident blocks walks a per-layer work list in
// topological order:
//   router items     one per expert: rmsnorm (bit-exact) + fp64 logit and error bound;
//                    the item finishing last certifies the top-k (router.h)
//   gate/up items    (slot, 16-row panel): shared expert first (needs only xn), then
//                    the K routed experts; h = silu(gate) * up
//   down items       (slot, 16-row panel of D); the last slot item of a panel forms
//                    x' = x + (shared + sum_k w_k y_k) for its 16 rows
// Block b takes items b, b+G, b+2G, ... ; every dependency of an item has a smaller
// index, so with all blocks resident the lowest unfinished item can always run.
//
// Cross-block data (x, xn digits, top-k, h, y, router partials) moves through
// agent-scope relaxed atomic loads and stores (coherent across the XCDs' L2s without
// whole-cache writeback/invalidate); each producer waits for its stores to complete
// (s_waitcnt) before bumping a monotonic counter, and consumers poll counters with a
// bounded spin that turns a missed dependency into an error flag instead of a hang.
#pragma once

#include "common.h"
#include "experts.h"
#include "router.h"

#define SK_BLOCK 256
#define SK_MAX_SLOTS 9           // K + 1 <= 9
#define SK_SPIN_LIMIT (1u << 22) // polls before a wait is declared dead (~seconds)

// Counters sit 64 words (256 bytes) apart so that polls of one never share a cache
// line, or a memory channel's hot spot, with another.
#define SKC_PAD 64
enum { SKC_ROUTER = 0, SKC_SEL = 1, SKC_DIG = 2, SKC_X = 3, SKC_GATE = 4, SKC_PANEL = 16 };
#define SKC(i) ((i) * SKC_PAD)

struct StackLayer {
    const uint8_t *experts;
    const float *norm;
    const float *gate_inp;
    const float *bias;
    int has_routed;
    int pad;
};

struct StackArgs {
    const StackLayer *layers;  // [n_layers], relative to first_layer
    int n_layers, first_layer;
    const float *x_in;
    float *x;  // running activation = output
    int D, F, E, K, flags;
    float eps, routed_scale;
    size_t stride, off_gq, off_uq, off_dq, off_gs, off_us, off_ds;
    double2 *stage;       // [E]
    int8_t *dig;          // [3][D] digits of xn
    int *dexp;            // [D/32]
    float *xn;            // [D]
    int *topk_idx;        // [K]
    float *topk_w;        // [K]
    float *topk_ws;       // [K]
    float *router_prob;   // [E]
    int *hist_idx;        // + layer * hist_stride
    float *hist_w;
    int hist_stride;
    float *h;             // [K+1][F]
    float *y;             // [K+1][D]
    float *shared_out;    // [D]
    float *routed_out;    // [D]
    unsigned *ctr;        // counters, zero at launch
    unsigned long long *stats;
    int *error;           // nonzero: a wait timed out
    unsigned long long *trace;  // optional: 3 timestamps per item (picked, deps ready, done)
};

__device__ static inline float ld_f(const float *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ static inline int ld_i(const int *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ static inline void st_f(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ static inline void st_i(int *p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ static inline unsigned ld_u(const unsigned *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ static inline unsigned long long ld_u64(const unsigned long long *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ static inline void st_u64(unsigned long long *p, unsigned long long v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// All of this block's coherent stores have completed; then thread 0 bumps `c`.
// Returns the previous counter value to every thread.
__device__ static inline unsigned publish(unsigned *c, unsigned *s_old) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) *s_old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    return *s_old;
}

struct SkShared {
    union {
        struct {
            float xn[2048];
            double lo[GM_MAX_E], hi[GM_MAX_E], mid[GM_MAX_E];
            float p[GM_MAX_E], sel[GM_MAX_E];
        } r;
        struct {
            int8_t dig[3 * 2048];
            int dexp[64];
            float part[EX_WAVES][2][16];
        } g;
    } u;
    double red[4];
    float mean;
    unsigned old;
    int ok, last, sel_ok;
    int idx[GM_MAX_K];
    int expert;
    long trace_item;
    unsigned long long *trace;
};

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
        if (sh.trace) sh.trace[3 * sh.trace_item + 1] = wall_clock64();
    }
    __syncthreads();
    return sh.ok != 0;
}


// ---------------------------------------------------------------- router item
__device__ static bool sk_router_item(const StackArgs &a, const StackLayer &L, int layer, int li, int e, SkShared &sh) {
    const int D = a.D, E = a.E, K = a.K, tid = threadIdx.x;
    const int per = D / SK_BLOCK;  // D is a multiple of 256 here
    // The router row and the norm weights do not depend on x: fetch them before waiting.
    float gw[8], nw[8];
    const GM_GLOBAL float *g = gbl(L.gate_inp + (size_t)e * D);
    const GM_GLOBAL float *nrm = gbl(L.norm);
#pragma unroll
    for (int j = 0; j < 8; j++) {
        if (j < per) {
            gw[j] = g[tid * per + j];
            nw[j] = nrm[tid * per + j];
        }
    }
    if (li > 0 && !wait_ge(&a.ctr[SKC(SKC_X)], (unsigned)li * (D >> 4), a.error, sh)) return false;
    const float *xsrc = li == 0 ? a.x_in : a.x;
    // rmsnorm, bit-identical to infer.c:746-752, on coherent loads of x
    float xv[8];
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        if (j < per) xv[j] = ld_f(xsrc + tid * per + j);
    }
#pragma unroll
    for (int j = 0; j < 8; j++) {
        if (j < per) {
            sh.u.r.xn[tid * per + j] = xv[j];
            ss += (double)xv[j] * (double)xv[j];
        }
    }
    ss = block_sum_d(ss, sh.red);
    const double v = ss / (double)D, rho = (double)D * 0x1p-52;
    const float mlo = (float)(v * (1.0 - rho)), mhi = (float)(v * (1.0 + rho));
    float mean = mlo;
    if (mlo != mhi) {
        if (tid == 0) {
            double s = 0.0;
            for (int i = 0; i < D; i++) s += (double)sh.u.r.xn[i] * (double)sh.u.r.xn[i];
            sh.mean = (float)(s / (double)D);
            if (e == 0) atomicAdd(&a.stats[GM_STAT_NORM_EXACT], 1ull);
        }
        __syncthreads();
        mean = sh.mean;
    }
    const float inv = __fdiv_rn(1.0f, sqrt_rn_f32(__fadd_rn(mean, a.eps)));
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 8; j++) {
        if (j < per) {
            xv[j] = __fmul_rn(__fmul_rn(xv[j], inv), nw[j]);
            sh.u.r.xn[tid * per + j] = xv[j];
        }
    }
    __syncthreads();

    if (e == 0) {
        // publish xn and its digit form for the gate/up items of this layer
        for (int i0 = tid * 8; i0 < D; i0 += SK_BLOCK * 8) {
            float vals[8];
            float mx = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                vals[k] = sh.u.r.xn[i0 + k];
                mx = fmaxf(mx, fabsf(vals[k]));
                st_f(a.xn + i0 + k, vals[k]);
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
            st_u64((unsigned long long *)(a.dig + i0), w0);
            st_u64((unsigned long long *)(a.dig + D + i0), w1);
            st_u64((unsigned long long *)(a.dig + 2 * D + i0), w2);
            if ((tid & 3) == 0) st_i(a.dexp + (i0 >> 5), ex);
        }
        publish(&a.ctr[SKC(SKC_DIG)], &sh.old);
    }

    // logit of expert e in fp64 and the bound on glm.c's sequential fp32 chain
    double p[8];
    double seg = 0.0, seg_abs = 0.0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        if (j < per) {
            p[j] = (double)gw[j] * (double)xv[j];
            seg += p[j];
            seg_abs += fabs(p[j]);
        }
    }
    double S;
    double run = block_exclusive_scan_d(seg, sh.red, &S);
    double prefix_abs = 0.0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        if (j < per) {
            run += p[j];
            prefix_abs += fabs(run);
        }
    }
    const double sum_prefix_abs = block_sum_d(prefix_abs, sh.red);
    const double sum_abs = block_sum_d(seg_abs, sh.red);
    if (tid == 0) {
        const double u = 0x1p-24, n = (double)D;
        const double gamma = n * u / (1.0 - n * u);
        double B = u * (1.0 + u) * sum_abs + u * sum_prefix_abs + n * u * gamma * sum_abs;
        B = B * (1.0 + 0x1p-30) + 0x1p-40 * sum_abs + n * 0x1p-149;
        __hip_atomic_store((double *)&a.stage[e].x, S, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store((double *)&a.stage[e].y, B, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    const unsigned old = publish(&a.ctr[SKC(SKC_ROUTER)], &sh.old);
    if (old != (unsigned)((li + 1) * E - 1)) return true;

    // ---- this block finished the layer's last router item: select the top-k
    for (int i = tid; i < E; i += SK_BLOCK) {
        const double S_i = __hip_atomic_load((double *)&a.stage[i].x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const double B_i = __hip_atomic_load((double *)&a.stage[i].y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        double lo, hi;
        selection_interval(S_i, B_i, gbl(L.bias)[i], &lo, &hi);
        sh.u.r.lo[i] = lo;
        sh.u.r.hi[i] = hi;
        sh.u.r.mid[i] = 0.5 * (lo + hi);
        sh.u.r.p[i] = (float)(1.0 / (1.0 + exp(-S_i)));
    }
    __syncthreads();
    if (tid < 64) {
        unsigned long long taken = 0ull;
        int ok = 1;
        double prev_lo = 0.0;
        const int kk = K < E ? K : E;
        for (int k = 0; k < kk; k++) {
            double best = -INFINITY;
            int bi = 0x7fffffff;
            for (int c = 0; c < 4; c++) {
                const int i = tid + 64 * c;
                if (i < E && !((taken >> c) & 1ull)) {
                    const double m = sh.u.r.mid[i];
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
            if (k > 0 && !(prev_lo > sh.u.r.hi[wi])) ok = 0;
            prev_lo = sh.u.r.lo[wi];
            if (tid == 0) sh.idx[k] = wi;
        }
        if (ok && kk < E) {
            double mx = -INFINITY;
            for (int c = 0; c < 4; c++) {
                const int i = tid + 64 * c;
                if (i < E && !((taken >> c) & 1ull)) mx = fmax(mx, sh.u.r.hi[i]);
            }
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) mx = fmax(mx, __shfl_xor(mx, o, 64));
            if (!(prev_lo > mx)) ok = 0;
        }
        if (tid == 0) {
            sh.sel_ok = ok;
            for (int k = kk; k < K; k++) sh.idx[k] = -1;
        }
    }
    __syncthreads();
    if (!sh.sel_ok) {
        for (int i = tid; i < E; i += SK_BLOCK) {
            const GM_GLOBAL float *gi = gbl(L.gate_inp + (size_t)i * D);
            float chain = 0.0f;
            for (int j = 0; j < D; j++) chain = __fadd_rn(chain, __fmul_rn(gi[j], sh.u.r.xn[j]));
            const float pr = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-chain)));
            sh.u.r.p[i] = pr;
            sh.u.r.sel[i] = __fadd_rn(pr, gbl(L.bias)[i]);
        }
        __syncthreads();
        if (tid == 0) {
            atomicAdd(&a.stats[GM_STAT_ROUTE_EXACT], 1ull);
            int idx[GM_MAX_K];
            for (int k = 0; k < K; k++) idx[k] = -1;
            for (int i = 0; i < E; i++) {
                const float sc = sh.u.r.sel[i];
                int at = -1;
                for (int k = 0; k < K && at < 0; k++) {
                    const float held = idx[k] >= 0 ? sh.u.r.sel[idx[k]] : -INFINITY;
                    if (sc > held) at = k;
                }
                if (at < 0) continue;
                for (int k = K - 1; k > at; k--) idx[k] = idx[k - 1];
                idx[at] = i;
            }
            int unresolved = 0;
            for (int k = 0; k < K; k++) {
                if (idx[k] < 0) continue;
                const float a0 = sh.u.r.sel[idx[k]];
                const float tol = 4.0f * fmaxf(fabsf(a0), 1e-30f) * 0x1p-23f + 4.0f * 0x1p-24f;
                for (int i = 0; i < E; i++) {
                    if (i == idx[k]) continue;
                    bool above = false;
                    for (int q = 0; q < k; q++) above |= (idx[q] == i);
                    if (!above && fabsf(sh.u.r.sel[i] - a0) <= tol) unresolved = 1;
                }
            }
            if (unresolved) atomicAdd(&a.stats[GM_STAT_UNRESOLVED], 1ull);
            for (int k = 0; k < K; k++) sh.idx[k] = idx[k];
        }
        __syncthreads();
    }
    if (tid == 0) {
        float w[GM_MAX_K];
        float total = 0.0f;
        for (int k = 0; k < K; k++) {
            w[k] = sh.idx[k] >= 0 ? sh.u.r.p[sh.idx[k]] : -1e30f;
            if (sh.idx[k] >= 0) total = __fadd_rn(total, w[k]);
        }
        if (total > 0.0f) {
            const float denom = total < 6.103515625e-5f ? 6.103515625e-5f : total;
            const float inv_d = __fdiv_rn(1.0f, denom);
            for (int k = 0; k < K; k++) w[k] = __fmul_rn(w[k], inv_d);
        }
        for (int k = 0; k < K; k++) {
            st_i(a.topk_idx + k, sh.idx[k]);
            st_f(a.topk_w + k, w[k]);
            st_f(a.topk_ws + k, __fmul_rn(w[k], a.routed_scale));
            a.hist_idx[(size_t)layer * a.hist_stride + k] = sh.idx[k];
            a.hist_w[(size_t)layer * a.hist_stride + k] = w[k];
        }
    }
    for (int i = tid; i < E; i += SK_BLOCK) a.router_prob[i] = sh.u.r.p[i];
    publish(&a.ctr[SKC(SKC_SEL)], &sh.old);
    return true;
}

// Expert index of `slot` for the current layer, or -1 when the slot is idle.
__device__ static inline int sk_slot_expert(const StackArgs &a, const StackLayer &L, int slot) {
    if (slot == a.K) return a.E;
    if ((a.flags & 1) || !L.has_routed) return -1;
    return ld_i(a.topk_idx + slot);
}

// ---------------------------------------------------------------- gate/up item
__device__ static bool sk_gate_up_item(const StackArgs &a, const StackLayer &L, int li, int slot, int p, SkShared &sh) {
    const int D = a.D, F = a.F;
    if (slot < a.K && !wait_ge(&a.ctr[SKC(SKC_SEL)], (unsigned)(li + 1), a.error, sh)) return false;
    const int e = sk_slot_expert(a, L, slot);
    if (e >= 0) {
        const uint8_t *base = L.experts + (size_t)e * a.stride;
        PanelRegs<2, EX_NB_MAX> pr;
        panel_load<2, EX_NB_MAX>(pr, base + a.off_gq, (const __half *)(base + a.off_gs), base + a.off_uq,
                                 (const __half *)(base + a.off_us), p, D);
        if (slot == a.K && !wait_ge(&a.ctr[SKC(SKC_DIG)], (unsigned)(li + 1), a.error, sh)) return false;
        for (int i = threadIdx.x; i < (3 * D) / 8; i += SK_BLOCK)
            ((unsigned long long *)sh.u.g.dig)[i] = ld_u64((const unsigned long long *)a.dig + i);
        for (int i = threadIdx.x; i < D / 32; i += SK_BLOCK) sh.u.g.dexp[i] = ld_i(a.dexp + i);
        __syncthreads();
        float gu[2];
        panel_compute<2, EX_NB_MAX>(pr, D, sh.u.g.dig, sh.u.g.dexp, gu);
        const float g = gu[0], u = gu[1];
        const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
        if (lane < 16) {
            sh.u.g.part[w][0][lane] = g;
            sh.u.g.part[w][1][lane] = u;
        }
        __syncthreads();
        if (threadIdx.x < 16) {
            const int l = threadIdx.x;
            const float gs = ((sh.u.g.part[0][0][l] + sh.u.g.part[1][0][l]) + sh.u.g.part[2][0][l]) + sh.u.g.part[3][0][l];
            const float us = ((sh.u.g.part[0][1][l] + sh.u.g.part[1][1][l]) + sh.u.g.part[2][1][l]) + sh.u.g.part[3][1][l];
            st_f(a.h + (size_t)slot * F + (size_t)p * 16 + l, gs / (1.0f + expf(-gs)) * us);
        }
    }
    publish(&a.ctr[SKC(SKC_GATE + slot)], &sh.old);
    return true;
}

// ---------------------------------------------------------------- down item (+ combine)
__device__ static bool sk_down_item(const StackArgs &a, const StackLayer &L, int li, int slot, int p, SkShared &sh) {
    const int D = a.D, F = a.F, K = a.K, NS = a.K + 1;
    if (slot < K && !wait_ge(&a.ctr[SKC(SKC_SEL)], (unsigned)(li + 1), a.error, sh)) return false;
    const int e = sk_slot_expert(a, L, slot);
    if (e >= 0) {
        const uint8_t *base = L.experts + (size_t)e * a.stride;
        PanelRegs<1, EX_NB_MAX> pr;
        panel_load<1, EX_NB_MAX>(pr, base + a.off_dq, (const __half *)(base + a.off_ds), nullptr, nullptr, p, F);
        if (!wait_ge(&a.ctr[SKC(SKC_GATE + slot)], (unsigned)(li + 1) * (F >> 4), a.error, sh)) return false;
        // digits of h[slot] into shared memory
        const float *hs = a.h + (size_t)slot * F;
        for (int i0 = threadIdx.x * 8; i0 < F; i0 += SK_BLOCK * 8) {
            float vals[8];
            float mx = 0.0f;
#pragma unroll
            for (int k = 0; k < 8; k++) {
                vals[k] = ld_f(hs + i0 + k);
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
        float yv;
        panel_compute<1, EX_NB_MAX>(pr, F, sh.u.g.dig, sh.u.g.dexp, &yv);
        const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
        if (lane < 16) sh.u.g.part[w][0][lane] = yv;
        __syncthreads();
        if (threadIdx.x < 16) {
            const int l = threadIdx.x;
            st_f(a.y + (size_t)slot * D + (size_t)p * 16 + l,
                 ((sh.u.g.part[0][0][l] + sh.u.g.part[1][0][l]) + sh.u.g.part[2][0][l]) + sh.u.g.part[3][0][l]);
        }
    }
    const unsigned old = publish(&a.ctr[SKC(SKC_PANEL + p)], &sh.old);
    if (old != (unsigned)((li + 1) * NS - 1)) return true;
    // last slot of this panel: combine (infer.c:1192, 1212-1214)
    if (threadIdx.x < 16) {
        const int r = p * 16 + threadIdx.x;
        float acc = 0.0f;
        if (!(a.flags & 1) && L.has_routed) {
            for (int k = 0; k < K; k++) {
                if (ld_i(a.topk_idx + k) < 0) continue;
                acc = __fadd_rn(acc, __fmul_rn(ld_f(a.topk_ws + k), ld_f(a.y + (size_t)k * D + r)));
            }
        }
        const float shv = ld_f(a.y + (size_t)K * D + r);
        const float xr = ld_f((li == 0 ? a.x_in : a.x) + r);
        a.routed_out[r] = acc;
        a.shared_out[r] = shv;
        st_f(a.x + r, __fadd_rn(xr, __fadd_rn(shv, acc)));
    }
    publish(&a.ctr[SKC(SKC_X)], &sh.old);
    return true;
}

__global__ __launch_bounds__(SK_BLOCK) void k_stack_reset(unsigned *ctr, int n, int *error) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) ctr[i] = 0u;
    if (threadIdx.x == 0) *error = 0;
}

__device__ static inline unsigned long long sk_now() { return wall_clock64(); }

__global__ __launch_bounds__(SK_BLOCK) void k_moe_stack(StackArgs a) {
    __shared__ SkShared sh;
    const int E = a.E, K = a.K, NS = K + 1;
    const int NPF = a.F >> 4, NPD = a.D >> 4;
    const int n_router = E, n_gate = NS * NPF, n_down = NS * NPD;
    const int per_layer = n_router + n_gate + n_down;
    const long total = (long)per_layer * a.n_layers;
    for (long it = blockIdx.x; it < total; it += gridDim.x) {
        const int li = (int)(it / per_layer);
        int r = (int)(it % per_layer);
        const StackLayer L = a.layers[li];
        const int layer = a.first_layer + li;
        if (a.trace && threadIdx.x == 0) a.trace[3 * it] = sk_now();
        sh.trace_item = it;
        sh.trace = a.trace;
        bool ok;
        if (r < n_router) {
            ok = sk_router_item(a, L, layer, li, r, sh);
        } else if ((r -= n_router) < n_gate) {
            // shared expert's panels first: they need only xn, not the top-k
            const int slot = (r / NPF + K) % NS;
            ok = sk_gate_up_item(a, L, li, slot, r % NPF, sh);
        } else {
            r -= n_gate;
            const int slot = (r / NPD + K) % NS;
            ok = sk_down_item(a, L, li, slot, r % NPD, sh);
        }
        if (!ok) return;
        if (a.trace && threadIdx.x == 0) a.trace[3 * it + 2] = sk_now();
        __syncthreads();
    }
}
