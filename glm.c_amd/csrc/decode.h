// decode.h -- the row-owner decode kernel: T=1 through a run of MoE layers in one launch
// (k_moe_decode), for shapes whose expert items fit the grid (see dk_fits).
//
// Each layer (infer.c:1087-1216) is three dependent phases, separated by device-wide flags
// (X, H) and the selection entries:
//
//  1. x of the layer is complete (X). The router finishers turn the layer's router
//     records (below) into each expert's certified selection entry (router.h), while every
//     block with an expert item computes xn and its digit form from x itself (the rmsnorm of
//     infer.c:746-752, bit-identical).
//  2. Every block takes the top-k from the entries (the certified selection, or the exact
//     replay's result). Expert items -- 16 rows of gate and up of one expert, K routed slots
//     and the shared expert -- form h = silu(g) * u for their rows and publish it in digit
//     form, and arrives on H. The shared expert's weights are requested before x exists, the
//     routed ones right after the selection.
//  3. Every block owns DK_ROWS consecutive rows of D. With the routing known (a block with a
//     routed item: once its h is out) it requests those rows of each selected expert's down
//     matrix into shared memory; after H it reads h, forms its rows of y for every slot
//     (int8 dot4 on h's digits), the residual combine
//     x' = x + (shared + sum_k w_k y_k) (infer.c:1192, 1212-1214), and from x' and the next
//     layer's router and norm rows that layer's router record, and arrives on X.
//
// Router records. glm.c's logit is a sequential fp32 chain over p_i = g_i * xn_i with
// xn_i = fl(fl(x_i * inv) * w_i) (infer.c:746-752, 916-925). Since inv is one scalar, the
// logit is inv * sum_i g_i w_i x_i up to xn's two roundings, and that sum splits by rows:
// the owner of rows 4q..4q+3 stores, per expert, the fp64 sum sigma_q of t_i = g_i w_i x_i
// over its rows, lambda_q >= sum_j |t_4q + ... + t_4q+j| and mu_q >= sum |t_i|, plus the
// rows' sum of x^2. A finisher then needs only a scan over the pieces: the estimate
// S = inv * sum sigma, sum |p_i| <= inv * sum mu (1 + kappa), and each partial sum of the
// chain |S_k| <= inv (|prefix_q| + |L_q,j|) + slack, which give the same bound on the fp32
// chain's error as the row-serial router (router.h), widened by xn's roundings (kappa ~ 2^-23)
// and the fp64 sums' (~D 2^-52). Underflow in xn's roundings adds at most 2^-150 (1+u) nu_e
// with nu_e = sum |g_i| (|w_i| + 1), computed at upload.
//
// Signalling is stack.h's: write-through stores, counters nobody polls, a write-once flag
// per layer and phase (X, H), bounded waits that set the error flag instead of hanging.
// Every wait is on work of the same layer or the one before that other blocks produce
// without waiting on the waiter, and all blocks are resident (one block per SIMD pair), so
// the schedule cannot deadlock. (Arrivals without the returned count, with every waiter
// polling all first-level counters, were slower: 512 blocks polling 16 lines each turn
// those lines into hot spots that the increments queue behind.)
#pragma once

#include "stack.h"

#define DK_ROWS 4    // rows of D per owner block
#define DK_PAIRS 2   // (slot, 16-column slice) pairs of the down projection per thread: 2 * 256 >= items
#define DK_HREC 64   // bytes of one item's h record: digit rows 0, 1, 2 (16 bytes each), the exponent
#define DK_RC_MAX (GM_MAX_E / 64)

// per-layer flags (SKF slots) and counters (SKC) of this kernel
enum { DKF_SEL = SKF_SEL, DKF_SELW = SKF_SELW, DKF_X = 3 };
enum { DKC_X = SKC_X, DKC_X2 = SKC_X2 };

// Router record of one owner piece and expert (16 bytes): fp64 sum of t_i over the piece's
// rows, and upper bounds of the sums of |partial sums| and |t_i|, rounded up to fp32.
struct DkRec {
    double sigma;
    float lam, mu;
};

// Router finisher blocks: a power of two, enough for one expert per wave (four per block)
// where the blocks left after the items allow, and at most 64.
__host__ __device__ static inline int dk_finishers(int G, int E, int K, int F) {
    const int free_blocks = G - (K + 1) * (F >> 4);
    int nf = 1;
    while (4 * nf < E && nf * 2 <= SK_NR_MAX && nf * 2 <= free_blocks) nf *= 2;
    return nf;
}

// Whether a shape runs on this kernel with a grid of G blocks: one block per expert item
// and per router finisher, DK_ROWS rows of D per block, 2 down pairs per thread.
__host__ __device__ static inline bool dk_fits(int G, int D, int F, int E, int K) {
    const int items = (K + 1) * (F >> 4);
    return D % 256 == 0 && D <= GM_MAX_COLS && F % 256 == 0 && F <= GM_MAX_COLS && E >= 1 && E <= GM_MAX_E &&
           K >= 1 && K <= GM_MAX_K && items + 1 <= G && items <= DK_PAIRS * SK_BLOCK && D / DK_ROWS <= G &&
           (D / DK_ROWS) % SK_NPART == 0 && (K + 1) * DK_ROWS * (F >> 4) * 4 <= (int)(sizeof(u32x4) * GM_MAX_COLS);
}

// Entry li of the launch's layer table, read through the constant address space: the host
// writes the table before the launch and the kernel never does, so scalar loads may read it
// and its pointers live in scalar registers. (Loaded by vector loads, their first use after
// a burst of weight requests would wait for the whole burst: the memory counter retires
// loads in order.)
__device__ static inline StackLayer dk_layer(const StackArgs &a, int li) {
    const __attribute__((address_space(4))) StackLayer *t = (const __attribute__((address_space(4))) StackLayer *)a.layers + li;
    StackLayer L;
    L.experts = t->experts;
    L.norm = t->norm;
    L.gate_inp = t->gate_inp;
    L.bias = t->bias;
    L.nu = t->nu;
    L.has_routed = t->has_routed;
    L.pad = 0;
    return L;
}

// Trace stamps go to shared memory (thread 0 only) and out once per layer (dk_trace_flush):
// a global store per stamp would sit in the memory counter, and the next wait for a load
// would wait for the store to reach memory as well.
__device__ static inline void dk_stamp(SkShared &sh, int k) {
    if (sh.dk_trace && threadIdx.x == 0) sh.stamps[k] = wall_clock64();
}
__device__ static inline void dk_trace_flush(SkShared &sh) {
    const int t = threadIdx.x;  // threads 0 .. SK_TRACE_STAMPS - 1: wave 0, the stamping wave
    if (sh.dk_trace && t < SK_TRACE_STAMPS) {
        const unsigned long long v = sh.stamps[t];
        if (v) sh.dk_trace[SK_TRACE_STAMPS * sh.trace_item + t] = v;
        sh.stamps[t] = 0ull;
    }
}

// Two-level count of a phase's arrivals (n per layer, n / SK_NPART on each first-level
// counter), then the layer's flag, after every store of this block has completed.
__device__ static inline void dk_arrive(const StackArgs &a, int c0, int c2, int idx, unsigned per_ctr, int li,
                                        unsigned *flag) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0 && add_u(&a.ctr[SKC(c0 + idx % SK_NPART)]) + 1u == (unsigned)(li + 1) * per_ctr &&
        add_u(&a.ctr[SKC(c2)]) + 1u == (unsigned)(li + 1) * SK_NPART)
        st_u(flag, 1u);
}

// ---------------------------------------------------------------- rmsnorm and digits
//
// xn of layer li (infer.c:746-752, bit-identical: sk_inv_rms) from x of the layer. With
// `digits`, its digit form goes to sh.xn_r as [3][D] int8 with one exponent in
// sh.xe_local (the A operands of the gate/up MFMAs); otherwise the fp32 xn goes to sh.xn_r
// (for the exact router replay). With `obs`, the fp32 xn is also written to a.xn.
__device__ __attribute__((always_inline)) static void dk_xn(const StackArgs &a, const StackLayer &L, int li,
                                                            bool digits, bool obs, SkShared &sh) {
    const int D = a.D, per = D / SK_BLOCK, tid = phase_tid(), lane = tid & 63, w = tid >> 6;
    const Seg nw = load_seg(gbl(L.norm) + tid * per, per);
    Seg xs = load_seg(ws_at<float>(a, li, a.o.x) + tid * per, per);
    float *xv = xs.v;
    const float inv = sk_inv_rms(a, xv, (float *)sh.dslice, false, sh);
    float mloc = 0.0f;
#pragma unroll
    for (int j = 0; j < SK_PER_MAX; j++) {
        xv[j] = j < per ? __fmul_rn(__fmul_rn(xv[j], inv), nw.v[j]) : 0.0f;
        mloc = fmaxf(mloc, fabsf(xv[j]));
    }
    if (obs) {
#pragma unroll
        for (int j = 0; j < SK_PER_MAX; j++)
            if (j < per) st_f(a.xn + tid * per + j, xv[j]);
    }
    if (!digits) {
#pragma unroll
        for (int j = 0; j < SK_PER_MAX; j++)
            if (j < per) sh.xn_r[tid * per + j] = xv[j];
        __syncthreads();
        return;
    }
    mloc = wave_max_dpp_f(mloc);
    if (lane == 0) sh.mxw[w] = mloc;
    __syncthreads();
    const int ex = digit_exponent(fmaxf(fmaxf(sh.mxw[0], sh.mxw[1]), fmaxf(sh.mxw[2], sh.mxw[3])));
    int8_t *dig = (int8_t *)sh.xn_r;
    if (per == SK_PER_MAX) {
        unsigned long long w0 = 0, w1 = 0, w2 = 0;
#pragma unroll
        for (int j = 0; j < SK_PER_MAX; j++) {
            int8_t d0, d1, d2;
            split_digits(xv[j], ex, &d0, &d1, &d2);
            w0 |= (unsigned long long)(uint8_t)d0 << (8 * j);
            w1 |= (unsigned long long)(uint8_t)d1 << (8 * j);
            w2 |= (unsigned long long)(uint8_t)d2 << (8 * j);
        }
        unsigned long long *dg = (unsigned long long *)dig;
        dg[tid] = w0;
        dg[D / 8 + tid] = w1;
        dg[2 * (D / 8) + tid] = w2;
    } else {
#pragma unroll
        for (int j = 0; j < SK_PER_MAX; j++) {
            if (j < per) {
                int8_t d0, d1, d2;
                split_digits(xv[j], ex, &d0, &d1, &d2);
                dig[tid * per + j] = d0;
                dig[D + tid * per + j] = d1;
                dig[2 * D + tid * per + j] = d2;
            }
        }
    }
    if (tid == 0) sh.xe_local = ex;
    __syncthreads();
}

// ---------------------------------------------------------------- router finisher
//
// One wave per expert: wave w of finisher block f takes experts f + NF (w + 4 n), n = 0, 1,
// ... (NF = a.n_router blocks). Lane l holds the records of pieces l ppl .. l ppl + ppl - 1
// (ppl = D / 4 / 64 consecutive pieces; the records of an expert are contiguous), so the
// scan over pieces is a lane-serial one inside a lane and one wave scan across lanes, with
// no block barrier. Every wave also reduces the pieces' sums of squares for inv itself.
#define DK_PPL (GM_MAX_COLS / DK_ROWS / 64)

// The per-expert constants of a finisher wave's first expert, loaded before x exists.
struct DkFinPre {
    double nu;
    float bias;
};

__device__ static inline void dk_fin_pre(const StackArgs &a, const StackLayer &L, int f, DkFinPre &fp) {
    const int e = f + a.n_router * (phase_tid() >> 6);
    const int ec = e < a.E ? e : 0;
    fp.nu = gbl(L.nu)[ec];
    fp.bias = gbl(L.bias)[ec];
}

// Expert e's selection entry from the lane's records rv (see the top of this file), stored
// as stack.h's stage entries (8 copies, stage_pos). `inv` is the layer's 1/sqrt(mean + eps).
__device__ __attribute__((always_inline)) static void dk_finish_expert(const StackArgs &a, int li, int e, float inv,
                                                                       double nu, float bias, const u32x4 (&rv)[DK_PPL]) {
    const int D = a.D, ppl = D / DK_ROWS / 64, lane = phase_tid() & 63;
    double sg[DK_PPL], tl = 0.0, m = 0.0;
#pragma unroll
    for (int k = 0; k < DK_PPL; k++) {
        sg[k] = k < ppl ? __longlong_as_double((long long)(((unsigned long long)rv[k].y << 32) | rv[k].x)) : 0.0;
        tl += sg[k];
        if (k < ppl) m += (double)__uint_as_float(rv[k].w);
    }
    const double incl = wave_incl_scan_dpp(tl), total = readlane_d(incl, 63);
    // sum over the lane's pieces of 4 |prefix before the piece| + lambda
    double pre = incl - tl, c = 0.0;
#pragma unroll
    for (int k = 0; k < DK_PPL; k++) {
        if (k < ppl) {
            c += 4.0 * fabs(pre) + (double)__uint_as_float(rv[k].z);
            pre += sg[k];
        }
    }
    const double cterm = wave_sum_dpp(c), mterm = wave_sum_dpp(m);
    const double u = 0x1p-24, n = (double)D, id = (double)inv;
    const double kap = (2.0 * u + u * u + 0x1p-53) * (1.0 + 0x1p-40);
    const double M = mterm * (1.0 + 0x1p-40), C = cterm * (1.0 + 0x1p-40);
    const double absv = 0x1p-150 * (1.0 + u) * nu;
    const double S = id * total;
    const double sa = id * M * (1.0 + kap) + absv;                           // >= sum |p_i|
    const double sp = id * C + n * (id * M * (n * 0x1p-51 + kap) + absv);    // >= sum_k |S_k|
    const double est = id * M * (n * 0x1p-52 + kap) + absv + 0x1p-52 * fabs(S);  // >= |S - sum p_i|
    const double gamma = n * u / (1.0 - n * u);
    const double emax = gamma * sa;
    double B = u * (1.0 + u) * sa + u * (sp + n * emax + u * sa) + est;
    B = B * (1.0 + 0x1p-30) + 0x1p-40 * sa + n * 0x1p-149;
    // the two interval ends and p on lanes 0, 1, 2
    const float arg = lane == 0 ? f32_rd(S - B) : lane == 1 ? f32_ru(S + B) : (float)S;
    const float sgm = 1.0f / (1.0f + expf(-arg));
    const float plo = readlane_f(sgm, 0), phi = readlane_f(sgm, 1), p = readlane_f(sgm, 2);
    if (lane < SK_STAGE_COPIES) {
        double lo, hi;
        selection_bounds((double)plo, (double)phi, bias, &lo, &hi);
        float lo_f = f32_rd(lo), hi_f = f32_ru(hi);
        if (!(lo_f <= hi_f)) {  // NaN: an interval that never certifies
            lo_f = -INFINITY;
            hi_f = INFINITY;
        }
        const int pe = stage_pos(e, a.n_router);
        st_u64(stage_plane(a, li, lane, 1) + pe, (unsigned long long)__float_as_uint(p));
        st_u64(stage_plane(a, li, lane, 0) + pe,
               (unsigned long long)__float_as_uint(lo_f) | ((unsigned long long)__float_as_uint(hi_f) << 32));
    }
}

// Finisher block f of layer li: each wave its experts' entries, after the layer's inv from
// the pieces' sums of squares (certified as sk_inv_rms certifies, else the sequential fp64
// sum replayed by the wave). The sums of squares and the first expert's records are all
// requested before anything waits.
__device__ __attribute__((always_inline)) static void dk_finish(const StackArgs &a, const StackLayer &L, int li, int f,
                                                                const DkFinPre &fp, SkShared &sh) {
    const int D = a.D, E = a.E, NF = a.n_router, NP = D / DK_ROWS, ppl = NP / 64;
    const int lane = phase_tid() & 63, w = phase_tid() >> 6, q0 = lane * ppl;
    const GM_GLOBAL double *xsq = gbl(ws_at<double>(a, li, a.o.xsq));
    static_assert(sizeof(DkRec) == sizeof(u32x4), "a router record is one 16-byte load");
    const GM_GLOBAL u32x4 *rec = gbl((const u32x4 *)ws_at<DkRec>(a, li, a.o.rec));
    // clamped rather than skipped (pieces k >= ppl are masked where they are used): a
    // register written by a load waits for no earlier load
    double xs[DK_PPL];
#pragma unroll
    for (int k = 0; k < DK_PPL; k++) xs[k] = xsq[q0 + (k < ppl ? k : 0)];
    float inv = 0.0f;
    bool first = true;
    for (int e = f + NF * w; e < E; e += 4 * NF) {
        u32x4 rv[DK_PPL];
#pragma unroll
        for (int k = 0; k < DK_PPL; k++) rv[k] = rec[(size_t)e * NP + q0 + (k < ppl ? k : 0)];
        if (first) {
            double ss = 0.0;
#pragma unroll
            for (int k = 0; k < DK_PPL; k++)
                if (k < ppl) ss += xs[k];
            ss = wave_sum_dpp(ss);
            const double v = ss / (double)D, rho = (double)D * 0x1p-52;
            const float mlo = (float)(v * (1.0 - rho)), mhi = (float)(v * (1.0 + rho));
            float mean = mlo;
            if (mlo != mhi) {  // wave-uniform
                float mv = 0.0f;
                if (lane == 0) {
                    const float *x = ws_at<float>(a, li, a.o.x);
                    double s2 = 0.0;
                    for (int i = 0; i < D; i++) s2 += (double)x[i] * (double)x[i];
                    mv = (float)(s2 / (double)D);
                    if (f == 0 && w == 0) atomicAdd(&a.stats[GM_STAT_NORM_EXACT], 1ull);
                }
                mean = readlane_f(mv, 0);
            }
            inv = __fdiv_rn(1.0f, sqrt_rn_f32(__fadd_rn(mean, a.eps)));
            dk_stamp(sh, 16);
        }
        double nu;
        float bias;
        if (first) {
            nu = fp.nu;
            bias = fp.bias;
        } else {
            nu = gbl(L.nu)[e];
            bias = gbl(L.bias)[e];
        }
        dk_finish_expert(a, li, e, inv, nu, bias, rv);
        first = false;
    }
}

// ---------------------------------------------------------------- router records
//
// Router rows of one owner for the records of a layer: thread t holds gate_inp[e][r0 + t%4]
// for e = t/4 + 64c, and norm[r0 + t%4].
struct DkRouter {
    float g[DK_RC_MAX];
    float wn;
};

__device__ static inline void dk_router_rows(const StackArgs &a, const StackLayer &L, int r0, DkRouter &rr) {
    const int tid = phase_tid(), i = tid & 3, eq = tid >> 2;
    rr.wn = gbl(L.norm)[r0 + i];
#pragma unroll
    for (int c = 0; c < DK_RC_MAX; c++) {
        const int e = eq + 64 * c;
        rr.g[c] = e < a.E ? gbl(L.gate_inp)[(size_t)e * a.D + r0 + i] : 0.0f;
    }
}

// Records of layer li for rows r0..r0+3 whose new values are xr4[0..3] (shared memory), and
// their sum of squares.
__device__ __attribute__((always_inline)) static void dk_records(const StackArgs &a, int li, int b, int r0,
                                                                 const DkRouter &rr, const float *xr4) {
    const int tid = phase_tid(), i = tid & 3, eq = tid >> 2, E = a.E;
    const double xv = (double)xr4[i];
    DkRec *rec = ws_at<DkRec>(a, li, a.o.rec) + b;  // [E][D/4]: an expert's pieces contiguous
#pragma unroll
    for (int c = 0; c < DK_RC_MAX; c++) {
        const int e = eq + 64 * c;
        if (64 * c < E) {  // block-uniform
            const double t = (double)rr.g[c] * (double)rr.wn * xv;
            // rows 0..3 of the piece are lanes 4m..4m+3: partial sums in row order
            double incl = t;
            const double u1 = __shfl_up(incl, 1, 4);
            if (i >= 1) incl += u1;
            const double u2 = __shfl_up(incl, 2, 4);
            if (i >= 2) incl += u2;
            double lam = fabs(incl), mu = fabs(t);
            lam += __shfl_xor(lam, 1, 4);
            lam += __shfl_xor(lam, 2, 4);
            mu += __shfl_xor(mu, 1, 4);
            mu += __shfl_xor(mu, 2, 4);
            const double sig = __shfl(incl, 3, 4);
            if (i == 0 && e < E) {
                const float lf = f32_ru(lam * (1.0 + 0x1p-50)), mf = f32_ru(mu * (1.0 + 0x1p-50));
                DkRec *re = rec + (size_t)e * (a.D / DK_ROWS);
                st_u64((unsigned long long *)&re->sigma, (unsigned long long)__double_as_longlong(sig));
                st_u64((unsigned long long *)&re->lam,
                       (unsigned long long)__float_as_uint(lf) | ((unsigned long long)__float_as_uint(mf) << 32));
            }
        }
    }
    if (tid == 0) {
        double s = 0.0;
#pragma unroll
        for (int j = 0; j < DK_ROWS; j++) s += (double)xr4[j] * (double)xr4[j];
        st_d(ws_at<double>(a, li, a.o.xsq) + b, s);
    }
}

// ---------------------------------------------------------------- expert items
//
// One item's gate/up weights in registers: panel j's chunks of this wave (panel_load_q)
// and, for lanes 0..15 (row lane), the fp16 scales of those chunks' blocks, two per dword.
struct DkItem {
    PanelRegs<2, EX_NB_MAX> pr;
    unsigned sg[EX_NB_MAX], su[EX_NB_MAX];
};

__device__ __attribute__((always_inline)) static void dk_item_load(const StackArgs &a, const StackLayer &L, int e, int j,
                                                                   DkItem &it) {
    const int D = a.D, tid = phase_tid(), lane = tid & 63, w = tid >> 6, m = lane & 15;
    const int cpw = D >> 8, j0 = w * cpw;
    const uint8_t *base = L.experts + (size_t)e * a.stride;
    // row m's scales of blocks 2 j0 .. (panel j's s plane is [16 rows][D/32] fp16: D bytes)
    const size_t so = (size_t)j * D + (size_t)m * (D / 16) + 4 * (size_t)j0;
    if (cpw == EX_NB_MAX) {
        const GM_GLOBAL u32x4 *pg = gbl((const u32x4 *)(base + a.off_gs + so));
        const GM_GLOBAL u32x4 *pu = gbl((const u32x4 *)(base + a.off_us + so));
        const u32x4 g0 = pg[0], g1 = pg[1], u0 = pu[0], u1 = pu[1];
        const unsigned sgv[EX_NB_MAX] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
        const unsigned suv[EX_NB_MAX] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
#pragma unroll
        for (int u = 0; u < EX_NB_MAX; u++) {
            it.sg[u] = sgv[u];
            it.su[u] = suv[u];
        }
    } else {
        const GM_GLOBAL unsigned *pg = gbl((const unsigned *)(base + a.off_gs + so));
        const GM_GLOBAL unsigned *pu = gbl((const unsigned *)(base + a.off_us + so));
#pragma unroll
        for (int u = 0; u < EX_NB_MAX; u++) {
            it.sg[u] = u < cpw ? pg[u] : 0u;
            it.su[u] = u < cpw ? pu[u] : 0u;
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // the scales are requested before the chunks
    // panel j's 1 KB chunks j0 .. j0 + cpw - 1 of gate and up (one dwordx4 per lane each),
    // chunk u of both matrices before chunk u + 1; chunks past cpw are zeros
    const size_t co = ((size_t)j * (D >> 6) + j0) * GM_CHUNK_BYTES;
    const GM_GLOBAL u32x4 *qg = gbl((const u32x4 *)(base + a.off_gq + co)) + lane;
    const GM_GLOBAL u32x4 *qu = gbl((const u32x4 *)(base + a.off_uq + co)) + lane;
#pragma unroll
    for (int u = 0; u < EX_NB_MAX; u++) {
        it.pr.q[0][u] = u < cpw ? __builtin_nontemporal_load(qg + (size_t)u * 64) : u32x4{0u, 0u, 0u, 0u};
        it.pr.q[1][u] = u < cpw ? __builtin_nontemporal_load(qu + (size_t)u * 64) : u32x4{0u, 0u, 0u, 0u};
    }
}

// Item (slot, j) of layer li: gate and up rows 16j..16j+15 dotted with xn's digits
// (gu_products_r), h = silu(g) * u (infer.c:1184-1188, 1199-1202) for those rows, stored
// as its digit form with one exponent: the h record (DK_HREC bytes), 16 dwords of three
// digit bytes each under a marker byte, exponent + 128. The launch starts with the records
// zeroed, so a reader knows a dword has arrived when it is nonzero: no count, no flag. An
// idle item (no expert in the slot) writes nothing, and nobody reads its record.
__device__ __attribute__((always_inline)) static void dk_item(const StackArgs &a, int li, int slot, int j, bool live,
                                                              const DkItem &it, SkShared &sh) {
    const int D = a.D, NPF = a.F >> 4, tid = phase_tid(), lane = tid & 63, w = tid >> 6, m = lane & 15;
    if (live) {
        const int cpw = D >> 8, j0 = w * cpw;
        const int8_t *drow = (const int8_t *)sh.xn_r + (m < 3 ? m : 0) * D + 64 * j0 + 8 * (lane >> 4);
        long A[EX_NB_MAX][2];
#pragma unroll
        for (int u = 0; u < EX_NB_MAX; u++) {
            const int uu = u < cpw ? u : 0;  // chunks past cpw have zero scales
            A[u][0] = *(const long *)(drow + 64 * uu);
            A[u][1] = *(const long *)(drow + 64 * uu + 32);
        }
        float gu[2];
        gu_products_r<EX_NB_MAX>(it.pr, A, it.sg, it.su, gu);
        if (lane < 16) {
            sh.u.g.part[w][0][lane] = gu[0];
            sh.u.g.part[w][1][lane] = gu[1];
        }
        __syncthreads();
        dk_stamp(sh, 5);
        if (tid < 64) {
            const int xe = sh.xe_local, r = lane & 15;
            const float g = ldexpf(((sh.u.g.part[0][0][r] + sh.u.g.part[1][0][r]) + sh.u.g.part[2][0][r]) + sh.u.g.part[3][0][r], xe);
            const float u = ldexpf(((sh.u.g.part[0][1][r] + sh.u.g.part[1][1][r]) + sh.u.g.part[2][1][r]) + sh.u.g.part[3][1][r], xe);
            const float h = g / (1.0f + expf(-g)) * u;
            int ex = digit_exponent(row_max_dpp_f(fabsf(h)));  // lanes 0..15: the item's rows
            ex = ex < -127 ? -127 : ex;  // the marker's range (below 2^-150, the values are lost anyway)
            int8_t d0, d1, d2;
            split_digits(h, ex, &d0, &d1, &d2);
            uint8_t *hb = (uint8_t *)sh.hrec;  // the 48 digit bytes: rows 0..15 of digit 0, 1, 2
            if (lane < 16) {
                hb[lane] = (uint8_t)d0;
                hb[16 + lane] = (uint8_t)d1;
                hb[32 + lane] = (uint8_t)d2;
            }
            asm volatile("" ::: "memory");  // one wave's shared-memory operations complete in order
            if (lane < 8) {
                // word `lane`: digit bytes 6 lane .. 6 lane + 5, three to a dword, each dword
                // topped by the marker (ex + 128, never 0)
                const unsigned mk = (unsigned)(ex + 128) << 24;
                const uint8_t *bp = hb + 6 * lane;
                const unsigned lo = (unsigned)bp[0] | ((unsigned)bp[1] << 8) | ((unsigned)bp[2] << 16) | mk;
                const unsigned hi = (unsigned)bp[3] | ((unsigned)bp[4] << 8) | ((unsigned)bp[5] << 16) | mk;
                unsigned long long *dst = (unsigned long long *)(ws_at<uint8_t>(a, li, a.o.h) + (size_t)(slot * NPF + j) * DK_HREC);
                st_u64(dst + lane, (unsigned long long)lo | ((unsigned long long)hi << 32));
            }
        }
    }
    dk_stamp(sh, 12);
}

// ---------------------------------------------------------------- down projection, combine
//
// The owner's down pairs: pair pi = (slot pi / (F/16), slice pi % (F/16)) holds the
// slice's 16 weights of rows r0..r0+3 (64 contiguous bytes; the row-group layout of
// common.h puts an owner's slices of one matrix in a row), staged in shared memory at
// sh.dslice[4 pi + i] by DMA that the compiler does not count (so that no wait of the
// layer's expert item includes them). Thread t computes
// pairs t + 256 k; sc[k] holds their four rows' fp16 scales of the slice's 32-column block.
// pi / NPF for pair indices pi < 2^12 and NPF <= 128, by a float product: the quotient's
// fractional part lies in [1/(2 NPF), 1 - 1/(2 NPF)] after adding 1/2, far above the
// product's rounding error (a few 2^-24 of a value below 2^12).
__device__ static inline int dk_slot(int pi, float rnpf) { return (int)(((float)pi + 0.5f) * rnpf); }

struct DkDown {
    unsigned long long sc[DK_PAIRS];
};

// Issues the down pairs of the routed slots (the experts of idx; none when !routed_on) and
// the shared expert's slot K.
__device__ __attribute__((always_inline)) static void dk_down_load(const StackArgs &a, const StackLayer &L, int r0,
                                                                   bool routed_on, const int *idx, SkShared &sh,
                                                                   DkDown &dd) {
    const int K = a.K, NPF = a.F >> 4, NPAIR = (K + 1) * NPF, tid = phase_tid();
    const int lane = tid & 63;
    // piece z = 4 pi + i of the layer's pairs; DMA chunk c covers pieces 64c..64c+63, which
    // lie in one slot (a slot has F/256 chunks). Of the at most DK_PAIRS * SK_BLOCK / 16
    // chunks, wave w takes w, w + 4, ...: at most DK_PAIRS * SK_BLOCK / 64, unrolled (a loop
    // here would make the compiler wait for every load in flight before entering it). s and
    // cr (the chunk within the slot) are wave-uniform and advance by subtraction.
    const int cps = a.F >> 8, nch = NPAIR / 16;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    int s = 0, cr = w;
#pragma unroll
    for (int q = 0; q < 3; q++)
        if (cr >= cps) cr -= cps, s++;
#pragma unroll
    for (int t = 0; t < DK_PAIRS * SK_BLOCK / 64; t++) {
        const int c = w + 4 * t;
        if (c < nch) {
            const int e = s == K ? a.E : (routed_on ? idx[s] : -1);
            if (e >= 0) {
                // the chunk's 16 slices of the owner's 4 rows: 1 KB in a row (row-group layout)
                const uint8_t *base = L.experts + (size_t)e * a.stride + a.off_rq;
                dma16_untracked(gbl((const u32x4 *)base) + ((size_t)(r0 >> 2) * NPF + 16 * cr) * 4 + lane,
                                (lds_void *)(sh.dslice + 64 * c));
            }
        }
        cr += 4;
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (cr >= cps) cr -= cps, s++;
    }
    const float rnpf = 1.0f / (float)NPF;
    // the scales by loads whatever the slot (a dead pair reads the shared expert's and is
    // never used): a register written by a load waits for no earlier load, while a zero
    // written by an ALU op would wait for every load still in flight
#pragma unroll
    for (int k = 0; k < DK_PAIRS; k++) {
        const int pi = tid + SK_BLOCK * k, pc = pi < NPAIR ? pi : 0, s = dk_slot(pc, rnpf), j = pc - s * NPF;
        const int ei = s == K ? a.E : (routed_on ? idx[s] : -1);
        const uint8_t *base = L.experts + (size_t)(ei >= 0 ? ei : a.E) * a.stride + a.off_rs;
        dd.sc[k] = *gbl((const unsigned long long *)base + (size_t)(r0 >> 2) * (a.F >> 5) + (j >> 1));
    }
}

// After flag H of layer li: rows r0..r0+3 of y for every slot from h (int8 dot4 on its
// digits), then x' = x + (shared + sum_k w_k y_k) in glm.c's order (infer.c:1192,
// 1212-1214), into x of layer li + 1 (or x_out and the observables after the last layer),
// and into xr4 (shared memory) for the next layer's records.
__device__ __attribute__((always_inline)) static bool dk_down(const StackArgs &a, int li, int r0, bool routed_on,
                                                              const DkDown &dd, float xr, float *xr4, SkShared &sh) {
    const int K = a.K, NS = K + 1, NPF = a.F >> 4, NPAIR = NS * NPF, tid = phase_tid();
    const float rnpf = 1.0f / (float)NPF;
    // this wave's down-pair DMA (the wait's barrier: every wave's), and every other load: by the
    // builtin, which the compiler sees (after an asm wait it would still count the loads as
    // pending and wait for them again at the next write of their registers)
    __builtin_amdgcn_s_waitcnt(GM_WAIT_VM0);
    dk_stamp(sh, 13);
    if (routed_on && !sh.sel_ok) dk_stamp(sh, 11);
    if (routed_on && !sh.sel_ok && !sk_read_weights(a, li, sh)) return false;
    // the h records of the live pairs, polled until every dword has its marker (coherent
    // 8-byte loads: a record's words arrive in any order, each one whole)
    const unsigned long long *hbase = ws_at<unsigned long long>(a, li, a.o.h);
    unsigned long long hw[DK_PAIRS][8];
    bool live[DK_PAIRS], need[DK_PAIRS];
#pragma unroll
    for (int k = 0; k < DK_PAIRS; k++) {
        const int pi = tid + SK_BLOCK * k, s = dk_slot(pi, rnpf);
        live[k] = pi < NPAIR && (s == K || (routed_on && sh.idx[s] >= 0));
        need[k] = live[k];
#pragma unroll
        for (int c = 0; c < 8; c++) hw[k][c] = 0ull;
    }
    {
        unsigned spins = 0;
        bool alive = true;
        for (;;) {
            bool miss = false;
#pragma unroll
            for (int k = 0; k < DK_PAIRS; k++) {
                if (need[k]) {
                    const unsigned long long *hp = hbase + (size_t)(tid + SK_BLOCK * k) * (DK_HREC / 8);
                    bool full = true;
#pragma unroll
                    for (int c = 0; c < 8; c++) {
                        hw[k][c] = __hip_atomic_load(hp + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        full &= (unsigned)hw[k][c] != 0u && (unsigned)(hw[k][c] >> 32) != 0u;
                    }
                    need[k] = !full;
                    miss |= !full;
                }
            }
            if (__ballot(miss) == 0) break;
            if (__hip_atomic_load(a.error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) || ++spins > sh.spin_limit) {
                if ((tid & 63) == 0) __hip_atomic_store(a.error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                alive = false;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (!alive) sh.ok = 0;  // a write of 0 by any wave; read after the barrier
        dk_stamp(sh, 6);
        __syncthreads();
        if (!sh.ok) return false;
    }
    // digit ints q = 0..11 (bytes 4q..4q+3 of the 48-byte stream, byte n in dword n / 3 at
    // n % 3) from the record's dwords; the exponent from any marker
    u32x4 hr[DK_PAIRS][4];
#pragma unroll
    for (int k = 0; k < DK_PAIRS; k++) {
        unsigned dw[16];
#pragma unroll
        for (int c = 0; c < 8; c++) {
            dw[2 * c] = (unsigned)hw[k][c];
            dw[2 * c + 1] = (unsigned)(hw[k][c] >> 32);
        }
        unsigned q4[12];
#pragma unroll
        for (int q = 0; q < 12; q++) {
            const int d0 = (4 * q) / 3;
            unsigned sel = 0;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int n = 4 * q + t;
                sel |= (unsigned)((n / 3 == d0 ? 0 : 4) + n % 3) << (8 * t);
            }
            q4[q] = __builtin_amdgcn_perm(dw[d0 + 1 < 16 ? d0 + 1 : 15], dw[d0], sel);
        }
        hr[k][0] = u32x4{q4[0], q4[1], q4[2], q4[3]};
        hr[k][1] = u32x4{q4[4], q4[5], q4[6], q4[7]};
        hr[k][2] = u32x4{q4[8], q4[9], q4[10], q4[11]};
        hr[k][3] = u32x4{(unsigned)((int)(dw[0] >> 24) - 128), 0u, 0u, 0u};
    }
    // v[k][i]: pair tid + 256 k's product for row i (0 for a dead pair or none); the sums
    // over each 16 consecutive pairs (within one slot: F/16 is a multiple of 16) by DPP, into
    // gsum[i][g] for pair group g (xn's digits in sh.xn_r are no longer needed)
    const int NG = NPAIR / 16;
    float *gsum = sh.xn_r;
#pragma unroll
    for (int k = 0; k < DK_PAIRS; k++) {
        const int pi = tid + SK_BLOCK * k;
        const int hexp = (int)hr[k][3].x;
        const int hd[3][4] = {{(int)hr[k][0].x, (int)hr[k][0].y, (int)hr[k][0].z, (int)hr[k][0].w},
                              {(int)hr[k][1].x, (int)hr[k][1].y, (int)hr[k][1].z, (int)hr[k][1].w},
                              {(int)hr[k][2].x, (int)hr[k][2].y, (int)hr[k][2].z, (int)hr[k][2].w}};
        float v[DK_ROWS];
#pragma unroll
        for (int i = 0; i < DK_ROWS; i++) {
            v[i] = 0.0f;
            if (live[k]) {
                const u32x4 dq = sh.dslice[4 * pi + i];
                const int wq[4] = {(int)dq.x, (int)dq.y, (int)dq.z, (int)dq.w};
                int acc[3];
#pragma unroll
                for (int d = 0; d < 3; d++) {
                    int sacc = 0;
#pragma unroll
                    for (int q = 0; q < 4; q++) sacc = __builtin_amdgcn_sdot4(wq[q], hd[d][q], sacc, false);
                    acc[d] = sacc;
                }
                const unsigned short sc16 = (unsigned short)(dd.sc[k] >> (16 * i));
                v[i] = digits_to_float(acc[0], acc[1], acc[2]) * ldexpf(__half2float(__ushort_as_half(sc16)), hexp);
            }
            v[i] = row_sum_dpp_f(v[i]);
        }
        if ((pi & 15) == 0 && pi < NPAIR) {
#pragma unroll
            for (int i = 0; i < DK_ROWS; i++) gsum[i * NG + (pi >> 4)] = v[i];
        }
    }
    __syncthreads();
    dk_stamp(sh, 19);
    if (tid < DK_ROWS) {
        // y[s][i] = the slot's group sums in order; x' = x + (shared + sum_k w_k y_k)
        const int i = tid, r = r0 + i, gps = NPF / 16;
        const float *g = gsum + i * NG;
        float acc = 0.0f, shv = 0.0f;
        for (int s = 0; s < NS; s++) {
            float y = g[s * gps];
            for (int u = 1; u < gps; u++) y += g[s * gps + u];
            if (s == K)
                shv = y;
            else if (routed_on && sh.idx[s] >= 0)
                acc = __fadd_rn(acc, __fmul_rn(sh.ws[s], y));
        }
        const float xo = __fadd_rn(xr, __fadd_rn(shv, acc));
        if (li == a.n_layers - 1) {
            st_f(a.x_out + r, xo);
            st_f(a.shared_out + r, shv);
            st_f(a.routed_out + r, acc);
        } else {
            st_f(ws_at<float>(a, li + 1, a.o.x) + r, xo);
        }
        xr4[i] = xo;
    }
    __syncthreads();
    return true;
}

// ---------------------------------------------------------------- exact replay
//
// Finisher 0, when the certified selection fails: glm.c's router replayed exactly
// (infer.c:916-938, 1104-1145) and its top-k published as the SEL words and the weights
// (the SELW flag follows the layer's observables). One lane per expert adds fl(g * xn)
// column by column in fp32, reading its gate row from global memory (16 columns a step,
// the next step's loads in flight) and xn (fp32) from shared memory: few registers, so the
// rare replay (~2 % of layers) does not set the register budget of the whole kernel.
__device__ __attribute__((always_inline)) static void dk_replay(const StackArgs &a, const StackLayer &L, int li,
                                                                SkShared &sh) {
    dk_xn(a, L, li, false, false, sh);
    const int D = a.D, E = a.E, K = a.K, tid = phase_tid();
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4 *x4 = (const f32x4 *)sh.xn_r;
    for (int e = tid; e < E; e += SK_BLOCK) {
        const GM_GLOBAL f32x4 *g = gbl((const f32x4 *)(L.gate_inp + (size_t)e * D));
        float chain = 0.0f;
        f32x4 gn[4];
#pragma unroll
        for (int u = 0; u < 4; u++) gn[u] = g[u];
        for (int c = 0; c < D / 4; c += 4) {
            f32x4 gv[4];
#pragma unroll
            for (int u = 0; u < 4; u++) gv[u] = gn[u];
            if (c + 4 < D / 4) {
#pragma unroll
                for (int u = 0; u < 4; u++) gn[u] = g[c + 4 + u];
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const f32x4 xv = x4[c + u];
                chain = __fadd_rn(chain, __fmul_rn(gv[u].x, xv.x));
                chain = __fadd_rn(chain, __fmul_rn(gv[u].y, xv.y));
                chain = __fadd_rn(chain, __fmul_rn(gv[u].z, xv.z));
                chain = __fadd_rn(chain, __fmul_rn(gv[u].w, xv.w));
            }
        }
        const float pr = sigmoid_libm(chain);  // infer.c:1105, libm's expf bits
        sh.u.s.p[e] = pr;
        sh.u.s.sel[e] = __fadd_rn(pr, gbl(L.bias)[e]);
    }
    __syncthreads();
    exact_topk(E, K, tid, sh.u.s.p, sh.u.s.sel, sh.idx, sh.wk, a.stats);
    if (tid < K) sh.ws[tid] = __fmul_rn(sh.wk[tid], a.routed_scale);
    if (tid < SK_SEL_WORDS) {
        unsigned long long word = 0;
        for (int q = 0; q < 4; q++) {
            const int k = 4 * tid + q;
            const unsigned v = k < K ? (unsigned)(sh.idx[k] + 2) : 1u;
            word |= (unsigned long long)v << (16 * q);
        }
        st_u64((unsigned long long *)&a.ctr[SKF(li, DKF_SEL) + 2 * tid], word);
    }
    if (tid < K) st_f(ws_at<float>(a, li, a.o.ex_w) + tid, sh.wk[tid]);
    __syncthreads();
}

// ---------------------------------------------------------------- selection
//
// The layer's routing from the stage entries, in every block. Wave 0 polls its XCD's copy
// until no word is unset (as sk_stage_select); the experts are then ranked by interval
// midpoint, ties to the lower index (each wave counts, for every expert, the larger keys
// among a quarter of the experts), and the K best in rank order are certified as
// certified_select certifies them: each chosen interval strictly above the next chosen one,
// the last strictly above every expert left out. glm.c's insertion top-k
// (infer.c:1110-1135) orders strictly by value, so it then picks the same experts in the
// same order. The weights are normalised as infer.c:1137-1145 does. With keep_p every
// probability goes to sh.u.s.p. Scratch: sh.dslice, unused until the owner's down pairs
// are requested.
struct DkSelScratch {
    unsigned long long ck[GM_MAX_E];  // order key: midpoint's order bits, then ~e; 0 past E
    int part[4][GM_MAX_E];            // larger keys among wave w's quarter
    int sel_e[GM_MAX_K];                   // by rank: expert, interval, probability
    float sel_lo[GM_MAX_K], sel_hi[GM_MAX_K], sel_p[GM_MAX_K];
};
static_assert(sizeof(DkSelScratch) <= sizeof(u32x4) * GM_MAX_COLS, "the selection scratch fits the down slices");

// C: chunks of 64 experts per lane (1 when E <= 64), so that the common shape runs no code
// for the chunks it does not have.
template <int C>
__device__ __attribute__((always_inline)) static bool dk_select_c(const StackArgs &a, int li, bool keep_p, SkShared &sh) {
    const int E = a.E, K = a.K, tid = phase_tid(), lane = tid & 63, w = tid >> 6;
    DkSelScratch &ss = *(DkSelScratch *)sh.dslice;
    // wave 0's entries (expert lane + 64 c), kept in registers through the ranking
    float lo[C], hi[C], pr[C];
    bool anybad = false;
    if (w == 0) {
        const int cpy = blockIdx.x % SK_STAGE_COPIES;
        const unsigned long long *sw0 = stage_plane(a, li, cpy, 0), *sw1 = stage_plane(a, li, cpy, 1);
        unsigned long long w0[C], w1[C];
        int pe[C];
#pragma unroll
        for (int c = 0; c < C; c++) pe[c] = stage_pos(lane + 64 * c < E ? lane + 64 * c : E - 1, a.n_router);
        unsigned spins = 0;
        bool alive = true;
        for (;;) {
            bool miss = false;
#pragma unroll
            for (int c = 0; c < C; c++) {
                w0[c] = __hip_atomic_load(sw0 + pe[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                w1[c] = __hip_atomic_load(sw1 + pe[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                miss |= (w0[c] == SK_UNSET) | (w1[c] == SK_UNSET);
            }
            if (__ballot(miss) == 0) break;
            if (__hip_atomic_load(a.error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) || ++spins > a.spin_limit) {
                if (lane == 0) __hip_atomic_store(a.error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                alive = false;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        dk_stamp(sh, 8);
        bool bad = false;
#pragma unroll
        for (int c = 0; c < C; c++) {
            const int e = lane + 64 * c;
            const bool valid = e < E;
            lo[c] = __uint_as_float((unsigned)w0[c]);
            hi[c] = __uint_as_float((unsigned)(w0[c] >> 32));
            pr[c] = __uint_as_float((unsigned)w1[c]);
            bad |= valid && !(isfinite(lo[c]) && isfinite(hi[c]));
            const unsigned kb = __float_as_uint(0.5f * lo[c] + 0.5f * hi[c]);
            const unsigned ko = (kb & 0x80000000u) ? ~kb : (kb | 0x80000000u);  // float order as unsigned order
            // experts past E rank last (key 0)
            ss.ck[e] = valid ? ((unsigned long long)ko << 32) | (unsigned)~e : 0ull;
            if (keep_p && valid) sh.u.s.p[e] = pr[c];
        }
        if (lane < K) ss.sel_e[lane] = -1;  // fewer than K experts leave the rest at -1 (infer.c:1110-1113)
        anybad = __ballot(bad) != 0;
        if (lane == 0) sh.ok = alive;
    }
    __syncthreads();
    if (!sh.ok) return false;
    {
        // wave w counts the larger keys among 16 C of them (keys past E are 0: never larger)
        unsigned long long my[C];
        int cnt[C];
#pragma unroll
        for (int c = 0; c < C; c++) {
            my[c] = ss.ck[lane + 64 * c];
            cnt[c] = 0;
        }
#pragma unroll 1
        for (int g = 0; g < C; g++) {  // 16 keys at a time, every read issued before the compares
            unsigned long long kj[16];
#pragma unroll
            for (int t = 0; t < 16; t++) kj[t] = ss.ck[16 * (C * w + g) + t];
#pragma unroll
            for (int t = 0; t < 16; t++)
#pragma unroll
                for (int c = 0; c < C; c++) cnt[c] += kj[t] > my[c] ? 1 : 0;
        }
#pragma unroll
        for (int c = 0; c < C; c++) ss.part[w][lane + 64 * c] = cnt[c];
    }
    __syncthreads();
    if (w == 0) {
        int rk[C];
#pragma unroll
        for (int c = 0; c < C; c++) {
            rk[c] = (ss.part[0][lane + 64 * c] + ss.part[1][lane + 64 * c]) +
                    (ss.part[2][lane + 64 * c] + ss.part[3][lane + 64 * c]);
            if (rk[c] < K && lane + 64 * c < E) {
                ss.sel_e[rk[c]] = lane + 64 * c;
                ss.sel_lo[rk[c]] = lo[c];
                ss.sel_hi[rk[c]] = hi[c];
                ss.sel_p[rk[c]] = pr[c];
            }
        }
        // one wave's shared-memory operations complete in order: only the compiler must not
        // move the reads below above the writes
        asm volatile("" ::: "memory");
        const float lo_last = ss.sel_lo[K - 1];
        bool fail = false;
#pragma unroll
        for (int c = 0; c < C; c++) {
            const int r = rk[c];
            if (lane + 64 * c < E) {
                const int rn = r + 1 < K ? r + 1 : K - 1;
                const bool has_next = r + 1 < K && ss.sel_e[rn] >= 0;
                fail |= has_next && !(lo[c] > ss.sel_hi[rn]);
                fail |= r >= K && !(lo_last > hi[c]);
            }
        }
        const bool cert = __ballot(fail) == 0 && !anybad && !(a.flags & GMOE_FLAG_EXACT_ROUTER);
        // lane k < K: the k-th chosen expert; the sum of the chosen weights in rank order
        const int kk = lane < K ? lane : 0;
        const int ek = ss.sel_e[kk];
        const float pk = ss.sel_p[kk];
        float total = 0.0f;
        for (int k = 0; k < K; k++) {
            const int e = __builtin_amdgcn_readlane(ek, k);
            if (e >= 0) total = __fadd_rn(total, readlane_f(pk, k));
        }
        // normalisation of infer.c:1137-1145 (when the selection is certified)
        const bool norm = cert && total > 0.0f;
        const float r = norm ? __fdiv_rn(1.0f, total < 6.103515625e-5f ? 6.103515625e-5f : total) : 1.0f;
        if (lane < K) {
            const float wk0 = ek >= 0 ? pk : -1e30f, wk = norm ? __fmul_rn(wk0, r) : wk0;
            sh.idx[lane] = ek;
            sh.wk[lane] = wk;
            if (cert) sh.ws[lane] = __fmul_rn(wk, a.routed_scale);
        }
        if (lane == 0) {
            sh.total = total;
            sh.sel_ok = cert;
        }
    }
    __syncthreads();
    return true;
}

__device__ __attribute__((always_inline)) static bool dk_select(const StackArgs &a, int li, bool keep_p, SkShared &sh) {
    return a.E <= 64 ? dk_select_c<1>(a, li, keep_p, sh) : dk_select_c<SK_SEL_C>(a, li, keep_p, sh);
}

// ---------------------------------------------------------------- the kernel
//
// Block roles (G blocks): routed items (slot s, panel j) on blocks s * F/16 + j; router
// finishers on the next NF blocks; shared-expert items on the last F/16 blocks; every block
// b < D / DK_ROWS owns rows 4b..4b+3. With two blocks per CU (b and b + G/2), each CU holds
// one or two routed items, or a routed item and a finisher or shared item.
__device__ __attribute__((always_inline)) static bool dk_run(const StackArgs &a, SkShared &sh) {
    const int G = (int)gridDim.x, b = blockIdx.x, K = a.K, NPF = a.F >> 4;
    const int NRI = K * NPF, NF = a.n_router, SB0 = G - NPF;
    const bool routed_item = b < NRI, finisher = b >= NRI && b < NRI + NF, shared_item = b >= SB0;
    const bool owner = b < a.D / DK_ROWS;
    const int r0 = DK_ROWS * b;
    if (!routed_item && !finisher && !shared_item && !owner) return true;
    const int fin = b - NRI;                       // finisher index
    const int slot = routed_item ? b / NPF : K;    // item slot
    const int jp = routed_item ? b % NPF : b - SB0;  // item panel
    float *xr4 = sh.xr4;                           // the owner's new rows
    // prologue: the owners put x_in's rows into layer 0's x and write layer 0's records
    if (owner) {
        DkRouter rr;
        dk_router_rows(a, dk_layer(a, 0), r0, rr);
        if (phase_tid() < DK_ROWS) {
            const float v = a.x_in[r0 + phase_tid()];
            st_f(ws_at<float>(a, 0, a.o.x) + r0 + phase_tid(), v);
            xr4[phase_tid()] = v;
        }
        __syncthreads();
        dk_records(a, 0, b, r0, rr, xr4);
        dk_arrive(a, DKC_X, DKC_X2, b, (unsigned)(a.D / DK_ROWS / SK_NPART), 0, &a.ctr[SKF(0, DKF_X)]);
    }
    for (int li = 0; li < a.n_layers; li++) {
        const StackLayer L = dk_layer(a, li);
        const StackLayer Ln = dk_layer(a, li + 1 < a.n_layers ? li + 1 : li);
        const int layer = a.first_layer + li;
        const bool routed_on = !(a.flags & GMOE_FLAG_NO_ROUTED) && L.has_routed;
        const bool last = li == a.n_layers - 1;
        if (threadIdx.x == 0) sh.trace_item = (long)li * G + b;
        dk_stamp(sh, 0);
        DkItem it;
        DkDown dd;
        DkFinPre fp;
        // the shared expert's gate/up weights and the finisher's constants do not depend on x
        if (shared_item) dk_item_load(a, L, a.E, jp, it);
        if (finisher) dk_fin_pre(a, L, fin, fp);
        if (!wait_ge(&a.ctr[SKF(li, DKF_X)], 1u, a.error, sh)) return false;
        dk_stamp(sh, 10);
        if (finisher) {
            dk_finish(a, L, li, fin, fp, sh);
            dk_stamp(sh, 2);
        }
        // the routing: finisher 0 decides it (replaying the router when the certificate
        // fails) and writes the layer's observables; the others take it from the entries
        if (finisher && fin == 0) {
            if (!dk_select(a, li, true, sh)) return false;
            if (!sh.sel_ok) dk_replay(a, L, li, sh);
            sk_write_routing(a, layer, sh);
            if (!sh.sel_ok) signal(&a.ctr[SKF(li, DKF_SELW)]);
        }
        if (routed_item || shared_item) dk_xn(a, L, li, true, last && b == 0, sh);
        dk_stamp(sh, 9);
        if (shared_item) dk_item(a, li, K, jp, true, it, sh);
        if (!(finisher && fin == 0)) {
            if (!dk_select(a, li, false, sh)) return false;
            if (!sh.sel_ok && !sk_read_topk(a, li, sh)) return false;
        }
        dk_stamp(sh, 3);
        const bool item_live = routed_on && routed_item && sh.idx[slot] >= 0;
        if (item_live) dk_item_load(a, L, sh.idx[slot], jp, it);
        // an owner with a routed item requests its down rows after the item's products: the
        // gate/up weights that every item waits for then have the memory system to themselves
        if (owner && !routed_item) dk_down_load(a, L, r0, routed_on, sh.idx, sh, dd);
        __builtin_amdgcn_sched_barrier(0);  // every weight request issued before the products
        dk_stamp(sh, 4);
        if (routed_item) {
            dk_item(a, li, slot, jp, item_live, it, sh);
            if (owner) dk_down_load(a, L, r0, routed_on, sh.idx, sh, dd);
        }
        if (owner) {
            // the next layer's router rows and this layer's x rows, fetched while the items finish
            DkRouter rr;
            if (!last) dk_router_rows(a, Ln, r0, rr);
            const float xr = phase_tid() < DK_ROWS ? ws_at<float>(a, li, a.o.x)[r0 + phase_tid()] : 0.0f;
            if (!dk_down(a, li, r0, routed_on, dd, xr, xr4, sh)) return false;
            dk_stamp(sh, 20);
            if (!last) {
                dk_records(a, li + 1, b, r0, rr, xr4);
                dk_stamp(sh, 21);
                dk_arrive(a, DKC_X, DKC_X2, b, (unsigned)(a.D / DK_ROWS / SK_NPART), li + 1, &a.ctr[SKF(li + 1, DKF_X)]);
            }
            dk_stamp(sh, 7);
        }
        dk_trace_flush(sh);
    }
    return true;
}

__global__ __launch_bounds__(SK_BLOCK, 2) void k_moe_decode(StackArgs a) {
    __shared__ SkShared sh;
    if (threadIdx.x == 0) {
        sh.trace = nullptr;  // stack.h's global stamps off: this kernel stamps through shared memory
        sh.dk_trace = a.trace;
        sh.ok = 1;
        sh.zero = 0u;
        sh.spin_limit = a.spin_limit;
        sh.trace_item = 0;
    }
    if (threadIdx.x < SK_TRACE_STAMPS) sh.stamps[threadIdx.x] = 0ull;
    __syncthreads();
    if (!dk_run(a, sh) && threadIdx.x == 0)
        __hip_atomic_store(a.error_host, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
