// relay.h -- k_moe_relay: the persistent decode kernel (T=1 through a run of MoE layers in
// one launch) whose phases hand their results to each other as tagged values that the
// consumers poll directly, with no counters or flags in between.
//
// A handoff through a counter costs a wait for the producer's stores to be acknowledged,
// one or two atomic round trips and a flag store before the consumer can even issue its
// reads (about 2.3 us per handoff on MI355X); a consumer that polls the data itself sees
// each value about 0.7 us after its store. Every per-layer buffer that crosses blocks --
// x, the expert items' partial sums and the router records -- is therefore written with a
// parity bit in the lowest bit of every 32- or 64-bit word. Each workspace layer's parity
// lives in device memory and is flipped by the launch's reset kernel for the layers the
// launch runs (so a captured and replayed launch flips it too), and a launch writes every
// word of the layers it runs, so before the store lands a word still holds the other
// parity. A reader re-reads until every word it needs carries the current parity, then
// clears the bit.
// (x and the items' partial sums are rounded to an even significand, with no direction on
// average (rl_even), at every layer, so their values do not depend on the tag; the launch's
// final x is rounded the same way, so one launch of n layers gives the bits of n launches
// of one.) The stage entries keep stack.h's reset-to-unset form.
//
// Roles (G blocks, two per CU: blocks b and b + G/2 share a CU):
//  * routed items, blocks 0 .. K*F/16-1: poll x, compute xn and its digit form themselves
//    (the rmsnorm of infer.c:746-752, bit-identical), poll the stage entries and rank them
//    (the certified top-k of infer.c:1110-1145), then run their item: 16 rows of F of the
//    slot's expert (gate/up, SwiGLU, the down slice: infer.c:1166-1195), a partial y over
//    all D rows;
//  * shared items, the next F/16 blocks: poll x, request the shared expert's weights, form
//    the digits while they stream, run the item (infer.c:1197-1206);
//  * finisher blocks: one wave per expert polls that expert's router records, finishes
//    the certified logit interval and stores the expert's stage entry (router.h); finisher
//    0 also certifies the top-k, writes the layer's observables and, when the certificate
//    fails, replays glm.c's router exactly (exact_router) and publishes its top-k;
//  * combine chunks (D/16 of the routed blocks, after their item; on the CUs that carry
//    one routed item rather than two): poll the chunk's partial sums, form
//    x' = x + (shared + sum_k w_k y_k) for its 16 rows (infer.c:1192, 1212-1214) and from
//    x' the next layer's router records for those rows.
//
// Router records. glm.c's logit is a sequential fp32 chain over p_i = g_i * xn_i with
// xn_i = fl(fl(x_i * inv) * w_i) (infer.c:746-752, 916-925). Since inv is one scalar, the
// logit is inv * sum_i g_i w_i x_i up to xn's two roundings, and that sum splits by rows:
// the combine of chunk c stores, per expert, the fp64 sum sigma_c of t_i = g_i w_i x_i over
// its rows, lambda_c >= sum over the chunk's rows of |t_16c + ... + t_i| and
// mu_c >= sum |t_i|, plus the rows' sum of x^2. The finisher then needs only a scan over
// the chunks for the estimate inv * sum sigma and for every partial sum of the chain
// |S_k| <= inv (|prefix before chunk c| + partial inside it) + slack, which gives the
// bound of router.h on the fp32 chain's error, widened by xn's roundings and the fp64
// sums'.
//
// Every wait is bounded (an error flag instead of a hang). Every wait is on data of the
// same or an earlier layer that another role produces without waiting on the waiter, and
// all blocks are resident, so the schedule cannot deadlock.
#pragma once

#include "stack.h"

#define RL_ROWS 16       // rows of D per combine chunk and router record
#define RL_FIN_MAX 16    // finisher blocks (four experts at a time each)
#define RL_PPL 2         // combine chunks (router records) per lane of a finisher wave: D <= 64 * 2 * 16

// Router record of one chunk and expert (16 bytes): the fp64 sum of t_i over the chunk's
// rows, and upper bounds of the sums of |partial sums| and |t_i|, rounded up to fp32.
struct RlRec {
    double sigma;
    float lam, mu;
};

// Entry li of the launch's layer table, read through the constant address space: the host
// writes the table before the launch and the kernel never does, so scalar loads may read it
// and its pointers live in scalar registers. (Loaded by vector loads, their first use after
// a burst of weight requests would wait for the whole burst: the memory counter retires
// loads in order.)
__device__ static inline StackLayer rl_layer(const StackArgs &a, int li) {
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

// ---------------------------------------------------------------- tags

// The launch's parities (StackArgs::par_dev, as k_stack_reset left them), read once per block.
static __shared__ unsigned long long rl_par_sh[SK_MAX_LAYERS / 64];
__device__ static inline unsigned rl_par(const StackArgs &a, int li) {
    const int q = a.par_base + li;
    return (unsigned)(rl_par_sh[q >> 6] >> (q & 63)) & 1u;
}
// v rounded to an even significand, the value a tagged word carries: an odd significand
// goes to the neighbour whose bit 1 is clear (round half to even one bit up), so the
// rounding has no direction on average (|error| <= 1 ulp, mean 0). In bits, odd b becomes
// (b + 1) with its two lowest bits cleared (b + 1 when bit 1 was set, b - 1 when it was
// not) and even b stays: four integer operations, no branch. (Like any rounding up, the
// largest finite value can become infinity; x and the partial sums stay far below it.)
__device__ static inline float rl_even(float v) {
    const unsigned b = __float_as_uint(v), m = b & 1u;
    return __uint_as_float((b + m) & ~(m | (m << 1)));
}
__device__ static inline unsigned rl_tag(float v, unsigned p) { return __float_as_uint(rl_even(v)) | p; }
__device__ static inline float rl_untag(unsigned b) { return __uint_as_float(b & ~1u); }
__device__ static inline unsigned long long rl_tag_d(double v, unsigned p) {
    return ((unsigned long long)__double_as_longlong(v) & ~1ull) | p;
}
__device__ static inline double rl_untag_d(unsigned long long b) { return __longlong_as_double((long long)(b & ~1ull)); }
// Tag of a nonnegative upper bound, moved up (never down) to the next value of parity p.
__device__ static inline unsigned rl_tag_up(float v, unsigned p) {
    const unsigned b = __float_as_uint(v);
    return (b & 1u) == p ? b : b + 1u;
}
__device__ static inline unsigned long long ldc_u64(const void *p) {
    return __hip_atomic_load((const unsigned long long *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ static inline unsigned ldc_u32(const void *p) {
    return __hip_atomic_load((const unsigned *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ static inline bool lsb2_ok(unsigned long long w, unsigned p) {
    return ((unsigned)w & 1u) == p && ((unsigned)(w >> 32) & 1u) == p;
}

// One failed wait of any thread fails the block; false if the kernel must end.
__device__ __attribute__((always_inline)) static bool rl_block_ok(bool ok, SkShared &sh) {
    if (!ok) sh.ok = 0;
    __syncthreads();
    return sh.ok != 0;
}

// Another poll round allowed? Sets the error flag when the wait has gone on too long or
// another block already failed. Both are checked every 32nd round only: the error word's
// load is a memory round trip of its own, which would double every round's latency.
__device__ __attribute__((always_inline)) static bool rl_spin(const StackArgs &a, unsigned &spins) {
    const int mode = a.rl_poll;
    if (mode == 0 || (++spins & 31u) == 0u) {
        if (mode == 0) ++spins;
        if (__hip_atomic_load(a.error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return false;
        if (spins > a.spin_limit) {
            __hip_atomic_store(a.error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
    }
    __builtin_amdgcn_s_sleep(1);
    if (mode == 2)
        for (int i = 0; i < 15; i++) __builtin_amdgcn_s_sleep(1);
    return true;
}

#define RL_CW 16  // words per thread and poll batch

// Polls n <= RL_CW 8-byte words src[i * stride] until both halves of each carry parity p
// (each round re-reads only the words still missing); their values with the tags cleared
// into val. False if the wait gave up.
__device__ __attribute__((always_inline)) static bool rl_poll_words(const StackArgs &a, const unsigned long long *src,
                                                                    int stride, int n, unsigned p,
                                                                    unsigned long long (&val)[RL_CW]) {
    unsigned pend = n >= 32 ? ~0u : (1u << n) - 1u;
    unsigned spins = 0;
    for (;;) {
#pragma unroll
        for (int i = 0; i < RL_CW; i++)
            if ((pend >> i) & 1u) val[i] = ldc_u64(src + (size_t)i * stride);
#pragma unroll
        for (int i = 0; i < RL_CW; i++)
            if (((pend >> i) & 1u) && lsb2_ok(val[i], p)) pend &= ~(1u << i);
        if (!pend) break;
        if (!rl_spin(a, spins)) return false;
    }
#pragma unroll
    for (int i = 0; i < RL_CW; i++) val[i] &= ~0x0000000100000001ull;
    return true;
}

// ---------------------------------------------------------------- x

// x of layer li, rows [r0, r0 + n) (n in {1, 2, 4, 8}, r0 a multiple of n) into v: the
// launch's input for li == 0, otherwise polled until every value carries the layer's
// parity. False if the wait gave up.
// With `gate`, lane 0 of each wave first polls one word of x (in chunk blockIdx % (D/16),
// so that the blocks spread over the chunks' lines) and the wave reads the rest only once
// that word has arrived: the combine chunks all finish within a microsecond or so of each
// other, and a block that starts waiting long before that then costs 8 bytes a poll
// instead of all of x.
__device__ __attribute__((always_inline)) static bool rl_poll_x(const StackArgs &a, int li, int r0, int n, float *v, bool gate = false) {
    if (li == 0) {
        const Seg s = load_seg(a.x_in + r0, n);
#pragma unroll
        for (int j = 0; j < SK_PER_MAX; j++)
            if (j < n) v[j] = s.v[j];
        return true;
    }
    const float *x = ws_at<float>(a, li, a.o.x) + r0;
    const unsigned p = rl_par(a, li);
    unsigned spins = 0;
    if (gate) {
        const float *g = ws_at<float>(a, li, a.o.x) + RL_ROWS * (blockIdx.x % (a.D / RL_ROWS));
        bool ok = true;
        if ((threadIdx.x & 63) == 0) {
            while (!lsb2_ok(ldc_u64(g), p))
                if (!rl_spin(a, spins)) {
                    ok = false;
                    break;
                }
        }
        if (__ballot(!ok) != 0) return false;
        spins = 0;
    }
    for (;;) {
        unsigned b[SK_PER_MAX];
        if (n >= 2) {
#pragma unroll
            for (int k = 0; k < SK_PER_MAX / 2; k++)
                if (2 * k < n) {
                    const unsigned long long w = ldc_u64(x + 2 * k);
                    b[2 * k] = (unsigned)w;
                    b[2 * k + 1] = (unsigned)(w >> 32);
                }
        } else {
            b[0] = ldc_u32(x);
        }
        bool miss = false;
#pragma unroll
        for (int j = 0; j < SK_PER_MAX; j++)
            if (j < n) miss |= (b[j] & 1u) != p;
        if (!miss) {
#pragma unroll
            for (int j = 0; j < SK_PER_MAX; j++)
                if (j < n) v[j] = rl_untag(b[j]);
            return true;
        }
        if (!rl_spin(a, spins)) return false;
    }
}

// xn of layer li (bit-identical to infer.c:746-752) from this thread's D/256 values xv of
// x and of the norm weights nw: with `digits`, its digit form into sh.xn_r as [3][D] int8 with one exponent in
// sh.xe_local (the gate/up MFMAs' A operands); otherwise the fp32 xn into sh.xn_r. Ends
// with a barrier.
template <bool FULL>
__device__ __attribute__((always_inline)) static void rl_xn(const StackArgs &a, const Seg &nw, float *xv, bool digits,
                                                            SkShared &sh) {
    const int D = FULL ? GM_MAX_COLS : a.D, per = D / SK_BLOCK, tid = phase_tid(), lane = tid & 63, w = tid >> 6;
    const float inv = sk_inv_rms(a, xv, sh.xn_r, false, sh);
    float mloc = 0.0f;
#pragma unroll
    for (int j = 0; j < SK_PER_MAX; j++) {
        xv[j] = j < per ? __fmul_rn(__fmul_rn(xv[j], inv), nw.v[j]) : 0.0f;
        mloc = fmaxf(mloc, fabsf(xv[j]));
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

// ---------------------------------------------------------------- selection
//
// The layer's routing from the stage entries, in every wave of the block: each wave polls
// its XCD's copy (lane l: experts l + 64c) until no word is unset, then counts, for each of
// its experts, the larger keys (interval midpoint, ties to the lower index) among a
// quarter of the experts; the four counts give every expert's rank. The K best in rank
// order are certified as certified_select certifies them (each chosen interval strictly
// above the next chosen one, the last strictly above every expert left out): glm.c's
// insertion top-k orders strictly by value, so it then picks the same experts in the same
// order. Every wave derives the result itself. Results: sh.idx, sh.wk (normalised as
// infer.c:1137-1145 when certified), sh.ws (times routed_scale), sh.sel_ok, sh.total; with
// keep_p every probability into sh.u.s.p. Returns the expert of `slot` (-1 for none or an
// uncertified selection). `cnt` is four waves' counts of shared scratch.
template <int C>
__device__ __attribute__((always_inline)) static bool rl_select_c(const StackArgs &a, int li, bool keep_p, int slot,
                                                                  int *slot_e, SkShared &sh) {
    const int E = a.E, K = a.K, tid = phase_tid(), lane = tid & 63, w = tid >> 6;
    // wave 0 polls its XCD's copy of the entries and hands them to the other waves
    // [2][E] after the [4][E] counts below (the item's slice buffer, not yet in use)
    unsigned long long(*ent)[GM_MAX_E] = (unsigned long long(*)[GM_MAX_E])((int *)sh.dslice + 4 * GM_MAX_E);
    if (w == 0) {
        const int cpy = blockIdx.x % SK_STAGE_COPIES;
        const unsigned long long *sw0 = stage_plane(a, li, cpy, 0), *sw1 = stage_plane(a, li, cpy, 1);
        unsigned spins = 0;
        for (;;) {
            bool miss = false;
            unsigned long long v0[C], v1[C];
#pragma unroll
            for (int c = 0; c < C; c++) {
                const int e = lane + 64 * c;
                if (e < E) {
                    v0[c] = ldc_u64(sw0 + e);
                    v1[c] = ldc_u64(sw1 + e);
                    miss |= (v0[c] == SK_UNSET) | (v1[c] == SK_UNSET);
                }
            }
            if (__ballot(miss) == 0) {
#pragma unroll
                for (int c = 0; c < C; c++) {
                    const int e = lane + 64 * c;
                    if (e < E) {
                        ent[0][e] = v0[c];
                        ent[1][e] = v1[c];
                    }
                }
                break;
            }
            if (!rl_spin(a, spins)) {
                sh.ok = 0;
                break;
            }
        }
        sk_stamp(sh, 8);
    }
    __syncthreads();
    if (!sh.ok) return false;
    unsigned long long w0[C], w1[C];
#pragma unroll
    for (int c = 0; c < C; c++) {
        const int e = lane + 64 * c;
        w0[c] = e < E ? ent[0][e] : 0ull;
        w1[c] = e < E ? ent[1][e] : 0ull;
    }
    float lo[C], hi[C], pr[C];
    unsigned key[C];
    bool bad = false;
#pragma unroll
    for (int c = 0; c < C; c++) {
        const int e = lane + 64 * c;
        const bool valid = e < E;
        lo[c] = __uint_as_float((unsigned)w0[c]);
        hi[c] = __uint_as_float((unsigned)(w0[c] >> 32));
        pr[c] = __uint_as_float((unsigned)w1[c]);
        bad |= valid && !(isfinite(lo[c]) && isfinite(hi[c]));
        // midpoint in unsigned order, low 8 bits replaced by ~e: ties (and midpoints within
        // 2^-16 relative, whose intervals overlap anyway) go to the lower index, so a
        // misordered pair is never certified. Experts past E get key 0.
        const unsigned kb = __float_as_uint(0.5f * lo[c] + 0.5f * hi[c]);
        const unsigned ko = (kb & 0x80000000u) ? ~kb : (kb | 0x80000000u);
        key[c] = valid ? ((ko & ~255u) | (unsigned)(255 - e)) : 0u;
        if (keep_p && valid && w == 0) sh.u.s.p[e] = pr[c];
    }
    // this wave's quarter of the experts: 16 C of them
    int cnt[C];
#pragma unroll
    for (int c = 0; c < C; c++) cnt[c] = 0;
#pragma unroll
    for (int g = 0; g < C; g++) {
#pragma unroll
        for (int t = 0; t < 16; t++) {
            const unsigned kj = (unsigned)__builtin_amdgcn_readlane((int)key[g], 16 * w + t);
#pragma unroll
            for (int c = 0; c < C; c++) cnt[c] += kj > key[c] ? 1 : 0;
        }
    }
    int(*part)[GM_MAX_E] = (int(*)[GM_MAX_E])sh.dslice;  // [4][E] counts (the item's slice buffer, not yet in use)
#pragma unroll
    for (int c = 0; c < C; c++) part[w][lane + 64 * c] = cnt[c];
    if (w == 0) sk_stamp(sh, 18);
    __syncthreads();
    int rk[C];
#pragma unroll
    for (int c = 0; c < C; c++) {
        const int e = lane + 64 * c;
        rk[c] = (part[0][e] + part[1][e]) + (part[2][e] + part[3][e]);
        if (e >= E) rk[c] = 1 << 20;
    }
    // the K chosen, in rank order (wave-uniform): expert, interval and probability
    bool cert = __ballot(bad) == 0 && !(a.flags & GMOE_FLAG_EXACT_ROUTER);
    int my_e = -1;
    float my_w = -1e30f, prev_lo = 0.0f, total = 0.0f;
    for (int k = 0; k < K; k++) {
        int ek = -1;
        float lk = 0.0f, hk = 0.0f, pk = -1e30f;
#pragma unroll
        for (int c = 0; c < C; c++) {
            const unsigned long long m = __ballot(rk[c] == k);
            if (m) {
                const int ls = __ffsll(m) - 1;
                ek = ls + 64 * c;
                lk = readlane_f(lo[c], ls);
                hk = readlane_f(hi[c], ls);
                pk = readlane_f(pr[c], ls);
            }
        }
        if (ek >= 0) {  // fewer than K experts leave the rest at -1 (infer.c:1110-1113)
            if (k > 0 && !(prev_lo > hk)) cert = false;
            prev_lo = lk;
            total = __fadd_rn(total, pk);
        }
        if (lane == k) {
            my_e = ek;
            my_w = pk;
        }
    }
    // the last chosen must lie strictly above every expert left out
    float rest = -INFINITY;
#pragma unroll
    for (int c = 0; c < C; c++)
        if (rk[c] >= K && lane + 64 * c < E) rest = fmaxf(rest, hi[c]);
    rest = wave_max_dpp_f(rest);
    if (rest > -INFINITY && !(prev_lo > rest)) cert = false;
    const bool norm = cert && total > 0.0f;
    const float r = norm ? __fdiv_rn(1.0f, total < 6.103515625e-5f ? 6.103515625e-5f : total) : 1.0f;
    const float wk = norm && my_e >= 0 ? __fmul_rn(my_w, r) : my_w;
    if (w == 0) {
        if (lane < K) {
            sh.idx[lane] = my_e;
            sh.wk[lane] = wk;
            sh.ws[lane] = __fmul_rn(wk, a.routed_scale);
        }
        if (lane == 0) {
            sh.total = total;
            sh.sel_ok = cert;
        }
    }
    *slot_e = cert && slot >= 0 && slot < K ? __builtin_amdgcn_readlane(my_e, slot) : -1;
    if (w == 0) sk_stamp(sh, 3);
    __syncthreads();  // the results in shared memory, and the counts read before the scratch is reused
    return true;
}


// ---------------------------------------------------------------- expert item
//
// The weights of item (slot, j) of expert e: the down scales and the down slice (D rows x
// 16 bytes) to shared memory by DMA that the compiler does not count, then (D == 2048) the
// gate/up scales and the 64 KB of gate/up chunks to registers by ordinary loads, so that
// the compiler waits for each chunk by itself; for narrower D the gate/up scales go to
// shared memory by DMA as well and the chunks to registers.
struct RlItem {
    PanelRegs<2, EX_NB_MAX> pr;
    u32x4 g0, g1, u0, u1;  // D == 2048: row (lane & 15)'s gate/up scales of the wave's blocks
};

template <bool FULL, bool G16>
__device__ __attribute__((always_inline)) static void rl_item_request(const StackArgs &a, const StackLayer &L, int e,
                                                                      int j, RlItem &it, SkShared &sh) {
    const int D = FULL ? GM_MAX_COLS : a.D, tid = phase_tid(), lane = tid & 63, w = tid >> 6, wave0 = tid & ~63;
    const uint8_t *base = L.experts + (size_t)e * a.stride;
    const GM_GLOBAL u32x4 *qs = gbl((const u32x4 *)(base + a.off_dq)) + (size_t)j * D + tid;
    const int o = 1024 * w + 16 * lane;
    const int c = D / SK_BLOCK;
    if (G16) {
        // group size 16: the slice's D fp32 down scales (4 KB per 16 bytes a thread), then the
        // wave's own run of each gate/up scale panel (D bytes: its chunks' 64 scales each),
        // then the down slice, all by DMA that the compiler does not count; last the gate/up
        // chunks to registers (FULL: all of them, branch-free, so that the compiler waits for
        // each chunk by itself)
        const uint8_t *ds = base + a.off_ds + (size_t)j * D * 4;
#pragma unroll
        for (int h = 0; h < 2; h++)
            if (o + 4096 * h < 4 * D) dma16_untracked(gbl(ds + o + 4096 * h), (lds_void *)((uint8_t *)sh.sc16_d + 4096 * h + 1024 * w));
        const size_t pw = (size_t)j * D * 4 + (size_t)w * D;  // bytes: panel j, then the wave's run
#pragma unroll
        for (int mt = 0; mt < 2; mt++)
#pragma unroll
            for (int i = 0; i < 2; i++)
                if (64 * i + lane < D / 16)
                    dma16_untracked(gbl(base + (mt ? a.off_us : a.off_gs) + pw + 16 * (64 * i + lane)),
                                    (lds_void *)((uint8_t *)sh.sc16_gu + (2 * w + mt) * D + 1024 * i));
#pragma unroll
        for (int i = 0; i < SK_PER_MAX; i++)
            if (FULL || i < c) dma16_untracked(qs + (size_t)i * SK_BLOCK, (lds_void *)(sh.dslice + i * SK_BLOCK + wave0));
        __builtin_amdgcn_sched_barrier(0);
        if (FULL) panel_load_q_all<2, EX_NB_MAX>(it.pr, base + a.off_gq, base + a.off_uq, j, D);
        else panel_load_q<2, EX_NB_MAX>(it.pr, base + a.off_gq, base + a.off_uq, j, D);
    } else if (FULL) {
        const int m = lane & 15, j0 = w * EX_NB_MAX;
        dma16_untracked(gbl(base + a.off_ds + (size_t)(j >> 1) * D * 2 + o), (lds_void *)((uint8_t *)sh.sc_d + 1024 * w));
#pragma unroll
        for (int i = 0; i < SK_PER_MAX; i++)
            dma16_untracked(qs + (size_t)i * SK_BLOCK, (lds_void *)(sh.dslice + i * SK_BLOCK + wave0));
        const size_t so = (size_t)j * D + (size_t)m * (D / 16) + 4 * j0;
        const GM_GLOBAL u32x4 *pg = gbl((const u32x4 *)(base + a.off_gs + so));
        const GM_GLOBAL u32x4 *pu = gbl((const u32x4 *)(base + a.off_us + so));
        it.g0 = pg[0];
        it.g1 = pg[1];
        it.u0 = pu[0];
        it.u1 = pu[1];
        __builtin_amdgcn_sched_barrier(0);  // the scales are requested before the chunks
        panel_load_q_all<2, EX_NB_MAX>(it.pr, base + a.off_gq, base + a.off_uq, j, D);
    } else {
        if (o < 2 * D) {
            const uint8_t *src = o < D ? base + a.off_gs + (size_t)j * D + o : base + a.off_us + (size_t)j * D + (o - D);
            dma16_untracked(gbl(src), (lds_void *)((uint8_t *)sh.sc_gu + 1024 * w));
            dma16_untracked(gbl(base + a.off_ds + (size_t)(j >> 1) * D * 2 + o), (lds_void *)((uint8_t *)sh.sc_d + 1024 * w));
        }
#pragma unroll
        for (int i = 0; i < SK_PER_MAX; i++)
            if (i < c) dma16_untracked(qs + (size_t)i * SK_BLOCK, (lds_void *)(sh.dslice + i * SK_BLOCK + wave0));
        panel_load_q<2, EX_NB_MAX>(it.pr, base + a.off_gq, base + a.off_uq, j, D);
    }
    __builtin_amdgcn_sched_barrier(0);  // every request issued before anything that follows
}

// Item (slot, j) of layer li on expert e (-1: an idle slot, whose partials are zeros):
// g, u = gate, up rows 16j..16j+15 . xn (infer.c:1184-1185, 1199-1200) on the digits in
// sh.xn_r, h = silu(g) * u (:1188, :1202), and the partial y = down[:, 16j..16j+16) . h
// over all D rows (:1190, :1205), stored tagged at piece (j, slot) of every combine chunk:
// chunk r/16 holds [F/16][K+1][16] floats, so each 16 lanes store one 64-byte piece.
template <bool FULL, bool G16>
__device__ __attribute__((always_inline)) static void rl_item_compute(const StackArgs &a, int li, int slot, int j, int e,
                                                                      const RlItem &it, SkShared &sh) {
    const int D = FULL ? GM_MAX_COLS : a.D, NPF = a.F >> 4, NS = a.K + 1, tid = phase_tid(), lane = tid & 63, w = tid >> 6;
    const int c = D / SK_BLOCK;
    const unsigned p = rl_par(a, li);
    const size_t ychunk = (size_t)NPF * NS * RL_ROWS;
    float *yp = ws_at<float>(a, li, a.o.ypart) + (size_t)(j * NS + slot) * RL_ROWS + (tid & (RL_ROWS - 1)) +
                (size_t)(tid / RL_ROWS) * ychunk;
    if (e < 0) {
#pragma unroll
        for (int i = 0; i < SK_PER_MAX; i++)
            if (i < c) __hip_atomic_store((unsigned *)(yp + (size_t)i * (SK_BLOCK / RL_ROWS) * ychunk), p, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    float gu[2];
    if (G16) {
        // the wave's scale runs (issued before its 16 chunk loads) have landed: every load but
        // the chunks is done
        if (FULL) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * EX_NB_MAX) : "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const float *sg16 = sh.sc16_gu + (2 * w) * (D / 4), *su16 = sh.sc16_gu + (2 * w + 1) * (D / 4);
        gu_products16<EX_NB_MAX>(it.pr, D, FULL ? EX_NB_MAX : D >> 8, (const int8_t *)sh.xn_r, sg16, su16, gu);
        // the down slice and scales (not counted by the compiler) are in shared memory before
        // the barrier below
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else if (FULL) {
        const int m = lane & 15, j0 = w * EX_NB_MAX;
        const int8_t *drow = (const int8_t *)sh.xn_r + (m < 3 ? m : 0) * D + 64 * j0 + 8 * (lane >> 4);
        long A[EX_NB_MAX][2];
#pragma unroll
        for (int u = 0; u < EX_NB_MAX; u++) {
            A[u][0] = *(const long *)(drow + 64 * u);
            A[u][1] = *(const long *)(drow + 64 * u + 32);
        }
        const unsigned sg[EX_NB_MAX] = {it.g0.x, it.g0.y, it.g0.z, it.g0.w, it.g1.x, it.g1.y, it.g1.z, it.g1.w};
        const unsigned su[EX_NB_MAX] = {it.u0.x, it.u0.y, it.u0.z, it.u0.w, it.u1.x, it.u1.y, it.u1.z, it.u1.w};
        gu_products_r<EX_NB_MAX>(it.pr, A, sg, su, gu);
        // the down slice and scales (not counted by the compiler) are in shared memory before
        // the barrier below
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();  // every wave's scales and slice rows are in shared memory
        gu_products<EX_NB_MAX>(it.pr, D, (const int8_t *)sh.xn_r, sh.sc_gu, sh.sc_gu + D / 2, &sh.zero, gu);
    }
    if (lane < 16) {
        sh.u.g.part[w][0][lane] = gu[0];
        sh.u.g.part[w][1][lane] = gu[1];
    }
    __syncthreads();
    if (tid < 16) {
        // SwiGLU of the 16 rows, then their digit form with one exponent
        const int xe = sh.xe_local;
        const float g = ldexpf(((sh.u.g.part[0][0][tid] + sh.u.g.part[1][0][tid]) + sh.u.g.part[2][0][tid]) + sh.u.g.part[3][0][tid], xe);
        const float u = ldexpf(((sh.u.g.part[0][1][tid] + sh.u.g.part[1][1][tid]) + sh.u.g.part[2][1][tid]) + sh.u.g.part[3][1][tid], xe);
        const float h = g / (1.0f + expf(-g)) * u;
        const int ex = digit_exponent(row_max_dpp_f(fabsf(h)));
        int8_t d0, d1, d2;
        split_digits(h, ex, &d0, &d1, &d2);
        int8_t *hb = (int8_t *)sh.u.g.hd;
        hb[tid] = d0;
        hb[16 + tid] = d1;
        hb[32 + tid] = d2;
        if (tid == 0) sh.u.g.hexp = ex;
    }
    __syncthreads();
    sk_stamp(sh, 4);
    int h4[12];
#pragma unroll
    for (int q = 0; q < 12; q++) h4[q] = sh.u.g.hd[q];
    const int hexp = sh.u.g.hexp;
    u32x4 dqs[SK_PER_MAX];
    unsigned scs[SK_PER_MAX];  // the rows' fp16 scales, or (G16) their fp32 scales' bits
#pragma unroll
    for (int i = 0; i < SK_PER_MAX; i++) {
        dqs[i] = sh.dslice[i * SK_BLOCK + tid];
        scs[i] = G16 ? __float_as_uint(sh.sc16_d[i * SK_BLOCK + tid]) : (unsigned)sh.sc_d[i * SK_BLOCK + tid];
    }
#pragma unroll
    for (int i = 0; i < SK_PER_MAX; i++) asm volatile("" ::"v"(dqs[i]), "v"(scs[i]));
#pragma unroll
    for (int i = 0; i < SK_PER_MAX; i++) {
        if (i < c) {
            const u32x4 dq = dqs[i];
            const int wq[4] = {(int)dq.x, (int)dq.y, (int)dq.z, (int)dq.w};
            int acc[3];
#pragma unroll
            for (int d = 0; d < 3; d++) {
                int s = 0;
#pragma unroll
                for (int q = 0; q < 4; q++) s = __builtin_amdgcn_sdot4(wq[q], h4[4 * d + q], s, false);
                acc[d] = s;
            }
            const float sd = G16 ? __uint_as_float(scs[i]) : __half2float(__ushort_as_half((unsigned short)scs[i]));
            const float f = digits_to_float(acc[0], acc[1], acc[2]) * ldexpf(sd, hexp);
            __hip_atomic_store((unsigned *)(yp + (size_t)i * (SK_BLOCK / RL_ROWS) * ychunk), rl_tag(f, p), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    sk_stamp(sh, 5);
}

// ---------------------------------------------------------------- router records
//
// Records of layer li (its router and norm rows gr, wn) for chunk c, whose 16 rows of x are
// xc[0..15] (shared memory): thread t takes expert t/4 + 64 m and rows 4 (t%4) .. +3. The
// rows' partial sums run in order inside the thread and as a scan across its quad.
typedef float rl_f32x4 __attribute__((ext_vector_type(4)));
struct RlRouter {
    rl_f32x4 g[GM_MAX_E / 64];
    rl_f32x4 wn;
};

__device__ __attribute__((always_inline)) static void rl_router_rows(const StackArgs &a, const StackLayer &L, int c, RlRouter &rr) {
    const int tid = phase_tid(), q = tid & 3, eq = tid >> 2, r = RL_ROWS * c + 4 * q;
    rr.wn = *(const GM_GLOBAL rl_f32x4 *)(gbl(L.norm) + r);
#pragma unroll
    for (int m = 0; m < GM_MAX_E / 64; m++) {
        const int e = eq + 64 * m;
        const int ec = e < a.E ? e : 0;  // rows past E are loaded (in bounds) and never stored
        rr.g[m] = *(const GM_GLOBAL rl_f32x4 *)(gbl(L.gate_inp) + (size_t)ec * a.D + r);
    }
}

__device__ __attribute__((always_inline)) static void rl_records(const StackArgs &a, int li, int c, const RlRouter &rr,
                                                                 const float *xc) {
    const int tid = phase_tid(), q = tid & 3, eq = tid >> 2, E = a.E, NCH = a.D / RL_ROWS;
    const unsigned p = rl_par(a, li);
    const double x0 = xc[4 * q], x1 = xc[4 * q + 1], x2 = xc[4 * q + 2], x3 = xc[4 * q + 3];
    RlRec *rec = ws_at<RlRec>(a, li, a.o.rec);  // [E][D/16]: an expert's chunks contiguous
#pragma unroll
    for (int m = 0; m < GM_MAX_E / 64; m++) {
        const int e = eq + 64 * m;
        if (64 * m < E) {  // block-uniform
            const rl_f32x4 g = rr.g[m];
            const double t0 = (double)g.x * (double)rr.wn.x * x0, t1 = (double)g.y * (double)rr.wn.y * x1;
            const double t2 = (double)g.z * (double)rr.wn.z * x2, t3 = (double)g.w * (double)rr.wn.w * x3;
            const double l0 = t0, l1 = l0 + t1, l2 = l1 + t2, l3 = l2 + t3;  // inside the thread, in row order
            // inclusive prefix of the quad's thread sums, in row order (DPP quad_perm: lane q
            // reads lane q-1, then lane q-2)
            double incl = l3;
            const double s1 = dpp_d<0x90>(incl, 0.0);  // quad_perm [0,0,1,2]
            if (q >= 1) incl += s1;
            const double s2 = dpp_d<0x40>(incl, 0.0);  // quad_perm [0,0,0,1]
            if (q >= 2) incl += s2;
            const double ex = incl - l3;
            double lam = (fabs(ex + l0) + fabs(ex + l1)) + (fabs(ex + l2) + fabs(ex + l3));
            double mu = (fabs(t0) + fabs(t1)) + (fabs(t2) + fabs(t3));
            lam += dpp_d<DPP_QUAD_1032>(lam, 0.0);
            mu += dpp_d<DPP_QUAD_1032>(mu, 0.0);
            lam += dpp_d<DPP_QUAD_2301>(lam, 0.0);
            mu += dpp_d<DPP_QUAD_2301>(mu, 0.0);
            const double sig = dpp_d<0xFF>(incl, 0.0);  // quad_perm [3,3,3,3]
            if (q == 0 && e < E) {
                const float lf = f32_ru(lam * (1.0 + 0x1p-50)), mf = f32_ru(mu * (1.0 + 0x1p-50));
                RlRec *re = rec + (size_t)e * NCH + c;
                st_u64((unsigned long long *)&re->sigma, rl_tag_d(sig, p));
                st_u64((unsigned long long *)&re->lam,
                       (unsigned long long)rl_tag_up(lf, p) | ((unsigned long long)rl_tag_up(mf, p) << 32));
            }
        }
    }
    if (tid == 0) {
        double s = 0.0;
#pragma unroll
        for (int r = 0; r < RL_ROWS; r++) s += (double)xc[r] * (double)xc[r];
        st_u64(ws_at<unsigned long long>(a, li, a.o.xsq) + c, rl_tag_d(s, p));
    }
}

// ---------------------------------------------------------------- combine
//
// Chunk c of layer li: its partial sums, [F/16][K+1][16] floats, summed per (slot, row) in
// a fixed order, then x' = x + (shared + sum_k w_k y_k) in glm.c's order for the chunk's 16
// rows, rounded to an even significand, stored tagged for layer li + 1 (or plainly into
// x_out with the observables after the last layer), and the next layer's records for the
// rows. Thread (g, q) of the block, g a (slot, row pair) and q < Q = 256 / (8 (K+1)), polls
// the pair's 8-byte words of pieces j = q, q + Q, ... (re-read until tagged with the
// layer's parity) and sums them in j order in registers; the Q sums of a pair are then
// added in q order.
__device__ __attribute__((always_inline)) static bool rl_combine(const StackArgs &a, const StackLayer &Ln, int li, int c,
                                                                 bool routed_on, SkShared &sh) {
    const int K = a.K, NS = K + 1, NPF = a.F >> 4, tid = phase_tid();
    const bool last = li == a.n_layers - 1;
    RlRouter rr;
    if (!last) rl_router_rows(a, Ln, c, rr);
    // the residual rows (polled; already complete, since this block read x for its digits)
    if (tid < RL_ROWS / 2) {
        float v2[2];
        if (!rl_poll_x(a, li, RL_ROWS * c + 2 * tid, 2, v2)) sh.ok = 0;
        sh.xres[2 * tid] = v2[0];
        sh.xres[2 * tid + 1] = v2[1];
    }
    const unsigned p = rl_par(a, li);
    const int G2 = NS * (RL_ROWS / 2), Q = SK_BLOCK / G2;
    const int g = tid / Q, q = tid - g * Q, s = g / (RL_ROWS / 2), r2 = g % (RL_ROWS / 2);
    const int nj = tid < G2 * Q ? (NPF - q + Q - 1) / Q : 0;  // pieces j = q + Q i, i < nj
    const unsigned long long *src =
        ws_at<unsigned long long>(a, li, a.o.ypart) + (size_t)c * NPF * NS * (RL_ROWS / 2) + (size_t)(q * NS + s) * (RL_ROWS / 2) + r2;
    const int stride = Q * NS * (RL_ROWS / 2);  // words from piece j to piece j + Q
    float acc0 = 0.0f, acc1 = 0.0f;
    bool ok = true;
    for (int i0 = 0; i0 < nj && ok; i0 += RL_CW) {
        const int nb = nj - i0 < RL_CW ? nj - i0 : RL_CW;
        unsigned long long val[RL_CW];
        ok = rl_poll_words(a, src + (size_t)i0 * stride, stride, nb, p, val);
        if (ok) {
#pragma unroll
            for (int i = 0; i < RL_CW; i++)
                if (i < nb) {
                    acc0 += __uint_as_float((unsigned)val[i]);
                    acc1 += __uint_as_float((unsigned)(val[i] >> 32));
                }
        }
    }
    float(*part)[2] = (float(*)[2])sh.u.c.acc;  // [G2 * Q][2]
    if (tid < G2 * Q) {
        part[tid][0] = acc0;
        part[tid][1] = acc1;
    }
    if (!rl_block_ok(ok, sh)) return false;
    sk_stamp(sh, 1);
    if (tid < 2 * G2) {
        const int gg = tid >> 1, h = tid & 1;
        float y = part[gg * Q][h];
        for (int qq = 1; qq < Q; qq++) y += part[gg * Q + qq][h];
        sh.u.c.y[gg / (RL_ROWS / 2)][2 * (gg % (RL_ROWS / 2)) + h] = y;
    }
    __syncthreads();
    sk_stamp(sh, 19);
    float *xc = sh.xn_r;  // the chunk's new rows, for the records (xn's digits are no longer needed)
    if (tid < RL_ROWS) {
        const int r = c * RL_ROWS + tid;
        const float xr = sh.xres[tid];
        float acc = 0.0f;
        if (routed_on) {
#pragma unroll
            for (int k = 0; k < GM_MAX_K; k++)
                if (k < K && sh.idx[k] >= 0) acc = __fadd_rn(acc, __fmul_rn(sh.ws[k], sh.u.c.y[k][tid]));
        }
        const float shv = sh.u.c.y[K][tid];
        // the launch's output too, so that one launch of n layers equals n launches of one
        const float xo = rl_even(__fadd_rn(xr, __fadd_rn(shv, acc)));
        if (last) {
            st_f(a.x_out + r, xo);
            st_f(a.shared_out + r, shv);
            st_f(a.routed_out + r, acc);
        } else {
            __hip_atomic_store((unsigned *)(ws_at<float>(a, li + 1, a.o.x) + r), rl_tag(xo, rl_par(a, li + 1)),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        xc[tid] = xo;
    }
    __syncthreads();
    sk_stamp(sh, 20);
    if (!last) rl_records(a, li + 1, c, rr, xc);
    sk_stamp(sh, 5);
    __syncthreads();  // xc and the residual rows are reused by the next layer
    return true;
}

// ---------------------------------------------------------------- finisher
//
// Expert e's stage entry for layer li from its records (one wave): lane l holds chunks
// l*ppl .. l*ppl + ppl - 1 (records of an expert are contiguous), polled until tagged with
// the layer's parity, together with those chunks' sums of squares. The estimate is
// S = inv * sum sigma; with M >= sum_c mu_c and C >= sum_c (16 |prefix before c| + lambda_c)
// (the prefixes from a lane-serial plus wave scan), sum |p_i| <= inv M (1 + kappa) and
// sum_k |S_k| <= inv C + slack, where kappa covers xn's two roundings and the product's.
// Returns false if a wait gave up.
__device__ __attribute__((always_inline)) static bool rl_finish_expert(const StackArgs &a, const StackLayer &L, int li,
                                                                       int e, SkShared &sh) {
    const int D = a.D, NCH = D / RL_ROWS, lane = phase_tid() & 63;
    const int ppl = NCH > 64 ? NCH / 64 : 1;
    const unsigned p = rl_par(a, li);
    const unsigned long long *rec = (const unsigned long long *)(ws_at<RlRec>(a, li, a.o.rec) + (size_t)e * NCH);
    const unsigned long long *xsq = ws_at<unsigned long long>(a, li, a.o.xsq);
    // the expert's constants before the wait, so that no round trip follows it
    const double nu = gbl(L.nu)[e];
    const float bias = gbl(L.bias)[e];
    unsigned long long rs[RL_PPL], rl[RL_PPL], rq[RL_PPL];
    {
        unsigned spins = 0;
        // one record first (lane 0; the chunks' records land within a microsecond or so of
        // each other), then all of them
        bool ok = true;
        if (lane == 0)
            while ((ldc_u64(rec + 2 * (e % NCH)) & 1u) != p)
                if (!rl_spin(a, spins)) {
                    ok = false;
                    break;
                }
        if (__ballot(!ok) != 0) return false;
        sk_stamp(sh, 14);
        spins = 0;
        // then every record and sum of squares of the lane's chunks
        for (;;) {
            bool miss = false;
#pragma unroll
            for (int k = 0; k < RL_PPL; k++) {
                const int ci = lane * ppl + k;
                if (k < ppl && ci < NCH) {
                    rs[k] = ldc_u64(rec + 2 * ci);
                    rl[k] = ldc_u64(rec + 2 * ci + 1);
                    rq[k] = ldc_u64(xsq + ci);
                    miss |= ((unsigned)rs[k] & 1u) != p || !lsb2_ok(rl[k], p) || ((unsigned)rq[k] & 1u) != p;
                } else {
                    rs[k] = rl[k] = rq[k] = 0ull;
                }
            }
            if (__ballot(miss) == 0) break;
            if (!rl_spin(a, spins)) return false;
        }
    }
    sk_stamp(sh, 15);
    // inv: the sum of squares certified as sk_inv_rms certifies it (the tags move each
    // chunk's sum by at most 2^-52 of itself), else the sequential fp64 sum replayed by lane 0
    double sg[RL_PPL], tl = 0.0, m = 0.0, ssq = 0.0;
#pragma unroll
    for (int k = 0; k < RL_PPL; k++) {
        const bool on = k < ppl && lane * ppl + k < NCH;
        sg[k] = on ? rl_untag_d(rs[k]) : 0.0;
        tl += sg[k];
        if (on) {
            m += (double)rl_untag((unsigned)(rl[k] >> 32));
            ssq += rl_untag_d(rq[k]);
        }
    }
    ssq = wave_sum_dpp(ssq);
    const double v = ssq / (double)D, rho = (double)(D + 2) * 0x1p-52;
    const float mlo = (float)(v * (1.0 - rho)), mhi = (float)(v * (1.0 + rho));
    float mean = mlo;
    if (mlo != mhi) {  // wave-uniform: the sequential sum, by lane 0 (rare)
        float mv = 0.0f;
        bool ok = true;
        if (lane == 0) {
            double s2 = 0.0;
            for (int i = 0; i < D && ok; i++) {
                float xi;
                ok = rl_poll_x(a, li, i, 1, &xi);
                s2 += (double)xi * (double)xi;
            }
            mv = (float)(s2 / (double)D);
            if (ok) atomicAdd(&a.stats[GM_STAT_NORM_EXACT], 1ull);
        }
        if (__ballot(!ok) != 0) return false;
        mean = readlane_f(mv, 0);
    }
    const float inv = __fdiv_rn(1.0f, sqrt_rn_f32(__fadd_rn(mean, a.eps)));
    sk_stamp(sh, 16);
    const double incl = wave_incl_scan_dpp(tl), total = readlane_d(incl, 63);
    double pre = incl - tl, cs = 0.0;
#pragma unroll
    for (int k = 0; k < RL_PPL; k++) {
        if (k < ppl && lane * ppl + k < NCH) {
            cs += (double)RL_ROWS * fabs(pre) + (double)rl_untag((unsigned)rl[k]);
            pre += sg[k];
        }
    }
    const double cterm = wave_sum_dpp(cs), mterm = wave_sum_dpp(m);
    const double u = 0x1p-24, n = (double)D, id = (double)inv;
    const double kap = (2.0 * u + u * u + 0x1p-53) * (1.0 + 0x1p-40);
    const double M = mterm * (1.0 + 0x1p-40), Cb = cterm * (1.0 + 0x1p-40);
    const double absv = 0x1p-150 * (1.0 + u) * nu;
    const double S = id * total;
    const double sa = id * M * (1.0 + kap) + absv;                              // >= sum |p_i|
    const double sp = id * Cb + n * (id * M * (n * 0x1p-51 + kap) + absv);      // >= sum_k |S_k|
    // >= |S - sum p_i|: xn's roundings, the fp64 sums and the tags on the sigmas
    const double est = id * M * ((n + 2.0) * 0x1p-52 + kap) + absv + 0x1p-52 * fabs(S);
    const double gamma = n * u / (1.0 - n * u);
    const double emax = gamma * sa;
    double B = u * (1.0 + u) * sa + u * (sp + n * emax + u * sa) + est;
    B = B * (1.0 + 0x1p-30) + 0x1p-40 * sa + n * 0x1p-149;
    sk_stamp(sh, 17);
    // the two interval ends and p on lanes 0, 1, 2
    const float arg = lane == 0 ? f32_rd(S - B) : lane == 1 ? f32_ru(S + B) : (float)S;
    const float sgm = 1.0f / (1.0f + expf(-arg));
    const float plo = readlane_f(sgm, 0), phi = readlane_f(sgm, 1), pv = readlane_f(sgm, 2);
    sk_stamp(sh, 21);
    if (lane < SK_STAGE_COPIES) {
        double lo, hi;
        selection_bounds((double)plo, (double)phi, bias, &lo, &hi);
        float lo_f = f32_rd(lo), hi_f = f32_ru(hi);
        if (!(lo_f <= hi_f)) {  // NaN: an interval that never certifies
            lo_f = -INFINITY;
            hi_f = INFINITY;
        }
        st_u64(stage_plane(a, li, lane, 1) + e, (unsigned long long)__float_as_uint(pv));
        st_u64(stage_plane(a, li, lane, 0) + e,
               (unsigned long long)__float_as_uint(lo_f) | ((unsigned long long)__float_as_uint(hi_f) << 32));
    }
    sk_stamp(sh, 22);
    return true;
}

// Finisher block 0's routing duties for layer li after its entries: the certified top-k
// (or the exact replay of glm.c's router when it fails: the SEL words, then the weights
// under SELW), the layer's observables, and after the last layer xn.
template <bool FULL, int C>
__device__ __attribute__((always_inline)) static bool rl_route(const StackArgs &a, const StackLayer &L, int li, int layer,
                                                               SkShared &sh) {
    const int tid = phase_tid();
    int dummy;
    if (!rl_select_c<C>(a, li, true, -1, &dummy, sh)) return false;
    const bool last = li == a.n_layers - 1;
    if (!sh.sel_ok || last) {
        // xn (fp32) in sh.xn_r: x polled by every thread
        float xv[SK_PER_MAX];
        const int per = (FULL ? GM_MAX_COLS : a.D) / SK_BLOCK;
        const Seg nw = load_seg(gbl(L.norm) + tid * per, per);
        if (!rl_block_ok(rl_poll_x(a, li, tid * per, per, xv), sh)) return false;
        rl_xn<FULL>(a, nw, xv, false, sh);
        if (last)
            for (int i = tid; i < a.D; i += SK_BLOCK) st_f(a.xn + i, sh.xn_r[i]);
    }
    if (!sh.sel_ok) {
        // glm.c's router replayed on the experts that can still be chosen, from the intervals
        // rl_select_c left in the slice buffer (the whole replay when forced, when more than
        // RT_SUB_MAX experts overlap the K-th, and above 128 experts, where the inlined subset
        // code pushes this kernel into hundreds of bytes of scratch)
        const unsigned long long *ent0 = (const unsigned long long *)((const int *)sh.dslice + 4 * GM_MAX_E);
        constexpr int RL_SUB_NV = 4;  // the chains' reads in flight: few registers in this kernel
        static_assert(sizeof(sh.dslice) / sizeof(float) >= RT_SUB_MAX * 260, "the replay's rows fit the slice buffer");
        if (C <= 2 && !(a.flags & GMOE_FLAG_EXACT_ROUTER) &&
            exact_router_subset<RL_SUB_NV>(a.D, a.E, a.K, tid, L.gate_inp, L.bias, sh.xn_r, (float(*)[64])sh.dslice, ent0,
                                sh.u.s.p, sh.u.s.sel, sh.idx, sh.wk, a.stats, sh.u.s.su, &sh.u.s.nu,
                                (int)(sizeof(sh.dslice) / sizeof(float)))) {
            if (tid < a.K) sh.ws[tid] = __fmul_rn(sh.wk[tid], a.routed_scale);
            __syncthreads();
        } else {
            sk_exact_select(a, L, sh);
        }
        if (tid < SK_SEL_WORDS) {
            unsigned long long word = 0;
            for (int q = 0; q < 4; q++) {
                const int k = 4 * tid + q;
                const unsigned v = k < a.K ? (unsigned)(sh.idx[k] + 2) : 1u;
                word |= (unsigned long long)v << (16 * q);
            }
            st_u64((unsigned long long *)&a.ctr[SKF(li, SKF_SEL) + 2 * tid], word);
        }
        if (tid < a.K) st_f(ws_at<float>(a, li, a.o.ex_w) + tid, sh.wk[tid]);
    }
    sk_write_routing(a, layer, sh);
    if (!sh.sel_ok) signal(&a.ctr[SKF(li, SKF_SELW)]);
    __syncthreads();
    return true;
}

// ---------------------------------------------------------------- the kernel

// Block roles of a grid of G blocks for the shape (shared with the host).
struct RlRoles {
    int nri, nsi, nfb, nch, cb0;  // routed items, shared items, finisher blocks, combine chunks, first combine block
};
__host__ __device__ static inline RlRoles rl_roles(int G, int D, int F, int E, int K) {
    RlRoles r;
    r.nri = K * (F >> 4);
    r.nsi = F >> 4;
    r.nfb = (E + 3) / 4 < RL_FIN_MAX ? (E + 3) / 4 : RL_FIN_MAX;
    r.nch = D / RL_ROWS;
    // combine chunks on the routed blocks that finish their items last: the second blocks of
    // the CUs that carry two routed items (G/2 ..), whose weights arrive behind their CU
    // mates', so that they start polling the partial sums when nearly all have landed
    const int half = G / 2;
    r.cb0 = r.nri >= half + r.nch ? half : 0;
    return r;
}
// Whether the shape runs on k_moe_relay with G blocks.
__host__ __device__ static inline bool rl_fits(int G, int D, int F, int E, int K) {
    const RlRoles r = rl_roles(G, D, F, E, K);
    return D % 256 == 0 && D <= GM_MAX_COLS && F % 256 == 0 && F <= GM_MAX_COLS && E >= 1 && E <= GM_MAX_E && K >= 1 &&
           K <= GM_MAX_K && r.nri + r.nsi + r.nfb <= G && r.nch <= r.nri && D / RL_ROWS <= 64 * RL_PPL &&
           (K + 1) * (RL_ROWS / 2) <= SK_BLOCK;
}

template <bool FULL, int C, bool G16>
__device__ __attribute__((always_inline)) static bool rl_run(const StackArgs &a, SkShared &sh) {
    const int G = (int)gridDim.x, b = blockIdx.x, K = a.K, NPF = a.F >> 4, D = FULL ? GM_MAX_COLS : a.D, per = D / SK_BLOCK;
    const RlRoles R = rl_roles(G, D, a.F, a.E, K);
    const bool routed = b < R.nri, shared = b >= R.nri && b < R.nri + R.nsi;
    const bool fin = b >= R.nri + R.nsi && b < R.nri + R.nsi + R.nfb;
    const int fb = b - R.nri - R.nsi;
    const int cc = b - a.rl_cb0;  // combine chunk
    const bool combine = routed && cc >= 0 && cc < R.nch;
    const int slot = routed ? b / NPF : K, jp = routed ? b % NPF : b - R.nri;
    const int per_layer = R.nri + R.nsi + R.nch + R.nfb;  // trace items of a layer
    if (!routed && !shared && !fin) return true;
    const int tid = phase_tid();
    // a poll limit of 0 (a host diagnostic) fails the launch at once: with every wait
    // bounded, every block still exits
    if (a.spin_limit == 0) {
        if (tid == 0) __hip_atomic_store(a.error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return false;
    }
    // prologue: layer 0's records from the launch's input
    if (combine) {
        RlRouter rr;
        rl_router_rows(a, rl_layer(a, 0), cc, rr);
        if (tid < RL_ROWS) sh.xn_r[tid] = a.x_in[cc * RL_ROWS + tid];
        __syncthreads();
        rl_records(a, 0, cc, rr, sh.xn_r);
        __syncthreads();
    }
    for (int li = 0; li < a.n_layers; li++) {
        const StackLayer L = rl_layer(a, li);
        const StackLayer Ln = rl_layer(a, li + 1 < a.n_layers ? li + 1 : li);
        const int layer = a.first_layer + li;
        const bool routed_on = !(a.flags & GMOE_FLAG_NO_ROUTED) && L.has_routed;
        const long base = (long)li * per_layer;
        if (routed || shared) {
            if (tid == 0) sh.trace_item = base + (routed ? b : R.nri + jp);
            if (a.trace && tid == 0) trace_put(a.trace, SK_TRACE_STAMPS * sh.trace_item);
            float xv[SK_PER_MAX];
            const Seg nw = load_seg(gbl(L.norm) + tid * per, per);  // before the wait: no round trip after it
            if (!rl_block_ok(rl_poll_x(a, li, tid * per, per, xv, true), sh)) return false;
            sk_stamp(sh, 1);
            RlItem it;
            if (shared) {
                // the norm rows have arrived (requested before the wait): the count of the loads
                // the compiler waits on below must not include the item's DMA
                __builtin_amdgcn_s_waitcnt(GM_WAIT_VM0);
                rl_item_request<FULL, G16>(a, L, a.E, jp, it, sh);
                rl_xn<FULL>(a, nw, xv, true, sh);
                sk_stamp(sh, 11);
                rl_item_compute<FULL, G16>(a, li, K, jp, a.E, it, sh);
            } else {
                rl_xn<FULL>(a, nw, xv, true, sh);
                sk_stamp(sh, 11);
                int e = -1;
                if (!rl_select_c<C>(a, li, false, slot, &e, sh)) return false;
                if (!sh.sel_ok) {
                    if (!sk_read_topk(a, li, sh)) return false;
                    e = sh.idx[slot];
                }
                if (!routed_on) e = -1;
                if (e >= 0) rl_item_request<FULL, G16>(a, L, e, jp, it, sh);
                rl_item_compute<FULL, G16>(a, li, slot, jp, e, it, sh);
            }
            if (a.trace && tid == 0) trace_put(a.trace, SK_TRACE_STAMPS * sh.trace_item + 2);
            __syncthreads();
            if (combine) {
                if (tid == 0) sh.trace_item = base + R.nri + R.nsi + cc;
                if (a.trace && tid == 0) trace_put(a.trace, SK_TRACE_STAMPS * sh.trace_item);
                if (routed_on && !sh.sel_ok && !sk_read_weights(a, li, sh)) return false;
                if (!rl_combine(a, Ln, li, cc, routed_on, sh)) return false;
                if (a.trace && tid == 0) trace_put(a.trace, SK_TRACE_STAMPS * sh.trace_item + 2);
            }
        } else {
            if (tid == 0) sh.trace_item = base + R.nri + R.nsi + R.nch + fb;
            if (a.trace && tid == 0) trace_put(a.trace, SK_TRACE_STAMPS * sh.trace_item);
            const int w = tid >> 6;
            bool ok = true;
            for (int e = 4 * fb + w; e < a.E && ok; e += 4 * R.nfb) ok = rl_finish_expert(a, L, li, e, sh);
            if (!rl_block_ok(ok, sh)) return false;
            sk_stamp(sh, 13);
            if (fb == 0 && !rl_route<FULL, C>(a, L, li, layer, sh)) return false;
            if (a.trace && tid == 0) trace_put(a.trace, SK_TRACE_STAMPS * sh.trace_item + 2);
        }
    }
    return true;
}

// FULL: D == 2048 (a row of xn fills the item's registers exactly); C: chunks of 64 experts
// per lane in the selection (E <= 64 C); G16: experts at group size 16 with fp32 scales.
template <bool FULL, int C, bool G16>
__global__ __launch_bounds__(SK_BLOCK, 2) void k_moe_relay(StackArgs a) {
    __shared__ SkShared sh;
    if (threadIdx.x == 0) {
        sh.trace = a.trace;
        sh.ok = 1;
        sh.zero = 0u;
        sh.spin_limit = a.spin_limit;
        sh.trace_item = 0;
    }
    if (threadIdx.x < SK_MAX_LAYERS / 64) rl_par_sh[threadIdx.x] = a.par_dev[threadIdx.x];
    __syncthreads();
    if (!rl_run<FULL, C, G16>(a, sh) && threadIdx.x == 0)
        __hip_atomic_store(a.error_host, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Zeroes n16 16-byte words at p: the fixed workspace of gmoe_forward_layers_noalloc before
// each of its launches (its previous user may have been another context or kernel, whose
// words carry no parity of ours), parities included. A kernel rather than a memset, so
// that a captured call replays it.
__global__ __launch_bounds__(256) void k_relay_zero(u32x4 *p, size_t n16) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256) p[i] = u32x4{0u, 0u, 0u, 0u};
}
