// stack.h -- persistent decode kernel: T=1 through a run of MoE layers in one launch.
//
// A decode step is a chain of small, strictly dependent phases per layer
// (infer.c:1087-1216). Each phase moves 0.5-40 MB, a few microseconds of HBM time, so
// kernel boundaries (~2 us each on this GPU) would cost as much as the work. One grid
// of co-resident blocks walks the layers instead, with three roles:
//
//   router blocks (n_router, <= 64)  per layer: rmsnorm (bit-exact) and the fp64 logit
//       of their experts with a rigorous bound on glm.c's fp32 chain, turned into a
//       selection interval; block 0 also publishes xn in digit form. Later in the same
//       layer they certify the top-k and run the combine: 32 rows of
//       x' = x + (shared + sum_k w_k y_k) per chunk.
//   shared-expert blocks   expert items of the shared expert. They need no routing, so
//       their weights are requested while the router is still running.
//   routed blocks          certify the top-k (wave 0), then one expert item each.
//
// An expert item owns 16 rows j of F for one expert: gate and up rows (int8 MFMA on the
// digit form of xn), h = silu(g) * u for those 16 rows, and h times the matching 16
// columns of down (dot4 on h's digit form), a partial y over all D rows. The combine
// sums the F/16 partials of each expert in a fixed order. Every item's weights (68 KB
// of gate/up, 36 KB of down with scales) are requested at once, as soon as the top-k is
// known, and h never leaves the block.
//
// Memory ordering without cache flushes. Every activation buffer is per layer and is
// written exactly once per launch, by write-through (agent-scope) stores; a producer
// waits for its stores to complete (s_waitcnt) before bumping a monotonic counter, and a
// consumer polls the counter (agent-scope loads, bounded spin, then an error flag instead
// of a hang) before reading. Since no cache line of a per-layer buffer is touched before
// it is produced, and caches start clean at a kernel boundary, consumers may read it with
// ordinary cached loads: each XCD fetches it from memory once, into its own L2.
//
// Blocks walk the layers in order and every wait is on work of the same or an earlier
// layer that some other role produces without waiting on the waiter, so with all blocks
// resident the schedule cannot deadlock.
#pragma once

#include "common.h"
#include "experts.h"
#include "router.h"

#define SK_BLOCK 256
#define SK_SPIN_LIMIT (1u << 22)               // default polls before a wait is declared dead (~seconds)
#define SK_TRACE_STAMPS 32
#define SK_NR_MAX 64                           // router blocks
#define SK_RX_MAX (GM_MAX_E / SK_NR_MAX)       // experts per router block
#define SK_PER_MAX (GM_MAX_COLS / SK_BLOCK)    // columns (router) or rows (down) per thread
#define SK_NPART 16                            // completion counters of the expert items
#define SK_CROWS 16                            // rows per combine chunk (a 64-byte piece of one item's partials)
#define SK_CGROUPS (SK_BLOCK / SK_CROWS)       // partial sums per row in the combine
#define SK_MAX_LAYERS 256

// Signalling. Producers count their arrivals on counters that nobody polls; the producer
// whose atomic returns the last count of a layer then writes that layer's flag, once, and
// consumers poll the flag. Polling a word that is also receiving hundreds of atomics
// slows those atomics down badly (the phase's completion then arrives microseconds
// late); polling a word that is written once costs nothing measurable. Every counter and
// flag sits 64 words (256 bytes) from the next. The expert items count on SK_NPART
// counters, whose last arrivals count on a second level; the items of group A (see
// sk_early_slots) count a second time on counters of their own, for the PARTA flag.
#define SKC_PAD 64
enum {
    SKC_DIG = 0, SKC_X2 = 1, SKC_PART2 = 2, SKC_PA2 = 3, SKC_PART = 4, SKC_PA = SKC_PART + SK_NPART,
    SKC_X = SKC_PA + SK_NPART, SKC_FIXED = SKC_X + SK_NPART
};
enum { SKF_SEL = 0, SKF_SELW = 1, SKF_DIG = 2, SKF_PART = 3, SKF_X = 4, SKF_PARTA = 5, SKF_PER_LAYER = 6 };
#define SKC(i) ((i) * SKC_PAD)
#define SKF(li, f) SKC(SKC_FIXED + SKF_PER_LAYER * (li) + (f))  // per-layer flags
// The SEL flag carries the top-k itself, so that its consumers need nothing else: one
// 64-bit word per four slots, 16 bits per slot holding expert + 2 (never zero, so a word
// is either unwritten or complete).
#define SK_SEL_WORDS ((GM_MAX_K + 3) / 4)
static_assert(2 * SK_SEL_WORDS <= SKC_PAD, "the SEL words must fit in the flag's padding");
#define SK_CTR_WORDS(n_layers) SKF(n_layers, 0)
#define GM_STACK_COUNTERS SK_CTR_WORDS(SK_MAX_LAYERS)

struct StackLayer {
    const uint8_t *experts;
    const float *norm;
    const float *gate_inp;
    const float *bias;
    const double *nu;  // [E]: sum_i |gate_inp[e][i]| (|norm[i]| + 1), rounded up (the router bound's underflow term)
    int has_routed;
    int pad;
};

// Expert e's router result, written once per launch by its router block into two words
// that the launch's reset set to SK_UNSET: w0 = fp32 bits of lo | hi << 32, the certified
// selection interval [lo, hi] of sel = p + bias rounded outward; w1 = fp32 bits of p.
// Each word is stored and loaded whole (64-bit, single-copy atomic), so a reader that sees
// neither word unset has the final entry, with no counter or flag in between.
// The router block stores its entries in SK_STAGE_COPIES copies (4 KB apart), and a reader
// polls the copy of its XCD (blockIdx % 8, the dispatch order): 384 readers on one copy
// make the entries visible ~1.3 us later than 48 readers on each of eight. Within a copy
// the entries sit in two planes of GM_MAX_E words (all w0, then all w1) at stage_pos(e), which
// puts the entries of one XCD's router blocks (b % 8 alike) in the same lines.
#define SK_UNSET (~0ull)
#define SK_STAGE_COPIES 8
#define SK_STAGE_COPY_WORDS 512

// Per-layer workspace: one region of `ws_layer_bytes` per layer of the launch.
struct StackWs {
    size_t x, xn, dig, dexp, stage, ex_w, ypart;  // byte offsets inside a layer region
    size_t rec, xsq;                              // relay.h: router records, the chunks' sums of squares
};

struct StackArgs {
    const StackLayer *layers;  // [n_layers], relative to first_layer
    int n_layers, first_layer;
    const float *x_in;
    float *x_out;
    int D, F, E, K, flags;
    float eps, routed_scale;
    size_t stride, off_gq, off_uq, off_dq, off_gs, off_us, off_ds;  // down in the column-slice layout
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
    int *error;                // nonzero: a wait timed out (device word, cleared by k_stack_reset)
    int *error_host;           // host-visible copy, set by a failing block and left for the host to clear
    unsigned spin_limit;       // polls before a wait gives up (SK_SPIN_LIMIT unless the host lowers it)
    unsigned long long *trace; // optional: SK_TRACE_STAMPS timestamps per item (see k_moe_stack)
    int n_router;              // router blocks: a power of two, <= min(E, 64)
    int shared_blocks;         // blocks in the shared-expert role
    unsigned long long *par_dev;  // relay.h: [SK_MAX_LAYERS / 64] words, bit li = the parity of workspace layer li;
                                  // k_stack_reset flips the launch's layers before the kernel reads them
    int rl_cb0;                // relay.h: the routed block that runs combine chunk 0
    int rl_poll;               // relay.h: polling policy (rl_spin)
    int par_base;              // relay.h: parity bit of the launch's first workspace layer (ws and ctr point at it)
};

template <typename T>
__device__ static inline T *ws_at(const StackArgs &a, int li, size_t off) {
    return (T *)(a.ws + (size_t)li * a.ws_layer_bytes + off);
}
// Position of expert e (computed by router block e % NR) within a stage plane.
__device__ static inline int stage_pos(int e, int NR) {
    const int b = e % NR, x = e / NR;
    return NR >= 8 ? (b % 8) * (NR / 8) + b / 8 + NR * x : e;
}
// Copy c's plane (0: w0, 1: w1) of layer li's stage entries.
__device__ static inline unsigned long long *stage_plane(const StackArgs &a, int li, int c, int plane) {
    return ws_at<unsigned long long>(a, li, a.o.stage) + (size_t)c * SK_STAGE_COPY_WORDS + plane * GM_MAX_E;
}
static_assert(2 * GM_MAX_E <= SK_STAGE_COPY_WORDS, "a stage copy holds two planes of GM_MAX_E words");

// fp32 of v rounded toward -inf or +inf: the round-to-nearest conversion lies within one
// ulp of v, so one step toward v from its wrong side gives the directed rounding (also
// at overflow, inf -> FLT_MAX; NaN stays NaN), without a rounding-mode switch.
__device__ static inline float f32_rd(double v) {
    const float f = (float)v;
    return (double)f > v ? nextafterf(f, -INFINITY) : f;
}
__device__ static inline float f32_ru(double v) {
    const float f = (float)v;
    return (double)f < v ? nextafterf(f, INFINITY) : f;
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

// One trace stamp (the 100 MHz wall clock) at t[idx], through a global rather than a flat
// store: a flat store also counts against lgkmcnt, so the wave's next shared-memory wait
// would wait for the store to reach memory, and the stamp would slow what it measures.
__device__ static inline void trace_put(unsigned long long *t, long idx) {
    *(GM_GLOBAL unsigned long long *)(t + idx) = wall_clock64();
}

// The small fields first and the scale buffers last: shared-memory instructions reach 64 KB
// past their base register, and the block holds ~71 KB.
struct SkShared {
    double red[4];
    float mxw[4];  // per-wave max |xn|
    float mean, total;
    unsigned old;
    int ok, sel_ok;
    unsigned zero;  // 0 for the kernel's life (an always-zero operand of gu_products)
    int xe_local;   // exponent of a routed block's own digits of xn (sk_local_digits)
    unsigned spin_limit;
    float xres[16]; // relay.h: a combine chunk's residual rows
    int idx[GM_MAX_K];
    float wk[GM_MAX_K], ws[GM_MAX_K];
    long trace_item;
    unsigned long long *trace;
    union {
        struct {  // router item
            double wv[4][SK_RX_MAX][3];  // per wave: segment total, sum |S_k|, sum |p|
        } r;
        struct {  // top-k selection and its exact replay
            float p[GM_MAX_E], sel[GM_MAX_E];
            int su[RT_SUB_MAX], nu;  // the subset replay's experts (k_moe_relay)
        } s;
        struct {  // expert item
            int8_t dig[3 * GM_MAX_COLS];
            int dexp[GM_MAX_COLS / 32];
            float part[EX_WAVES][2][16];
            int hd[12];  // digit rows of h: 3 x 16 int8, four per word
            int hexp;
        } g;
        struct {  // combine
            float acc[SK_BLOCK / (2 * SK_CROWS)][GM_MAX_K + 1][SK_CROWS];
            float y[GM_MAX_K + 1][SK_CROWS];
        } c;
    } u;
    float xn_r[GM_MAX_COLS];    // a router item's xn (kept through the top-k and its replay)
    u32x4 dslice[GM_MAX_COLS];  // an expert item's down columns, D rows x 16 bytes
    union {
        struct {
            __attribute__((aligned(16))) unsigned short sc_gu[2 * GM_MAX_COLS / 2];  // its gate and up panel scales, [2][16][D/32]
            unsigned short sc_d[GM_MAX_COLS];  // its down scales, one per row
        };
        struct {  // group size 16 (k_moe_relay only): fp32 scales
            // per wave, gate then up: the wave's chunks of the panel's scale runs (gm_s16_offset)
            __attribute__((aligned(16))) float sc16_gu[2 * 16 * GM_MAX_COLS / 16];
            float sc16_d[GM_MAX_COLS];  // the item's down scales, one per row
        };
    };
};

__device__ static inline void st_u(unsigned *p, unsigned v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ static inline unsigned add_u(unsigned *p) { return __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// Group A of a layer's expert items: the routed slots 0..KA-1, whose items run on the first
// block of each CU (blocks b < G/2 hold items 0 .. G/2 - n_router - 1 when every routed
// block runs one item), and the shared expert's. Their data arrives microseconds before
// that of the items on the CUs' second blocks, so they count on their own flag and their
// partials lie apart, and the combine sums them while the rest still stream.
__device__ static inline int sk_early_slots(const StackArgs &a) {
    const int G = (int)gridDim.x, NR = a.n_router, NSB = a.shared_blocks, NPF = a.F >> 4;
    const int P = (G / 2 >= NR && G / 2 + NSB <= G) ? G / 2 : NR;  // as in k_moe_stack
    if (G - NR - NSB < a.K * NPF || P <= NR) return 0;
    const int ka = (P - NR) / NPF;
    return ka < a.K ? ka : a.K;
}

// Position of `slot` among a chunk's partials: slots 0..KA-1, the shared expert's (slot K),
// then slots KA..K-1; group A is positions 0..KA.
__device__ static inline int sk_pos(int slot, int K, int KA) { return slot < KA ? slot : slot == K ? KA : slot + 1; }

// Offset (floats) of (j, position)'s 16 rows inside a combine chunk's partials: group A as
// [F/16][KA+1][16], then group B as [F/16][K-KA][16], each contiguous.
__device__ static inline int sk_piece(int j, int pos, int NPF, int NS, int NA) {
    return pos < NA ? (j * NA + pos) * SK_CROWS : (NPF * NA + j * (NS - NA) + (pos - NA)) * SK_CROWS;
}

// All of this block's write-through stores have completed; then thread 0 sets `flag`.
__device__ static inline void signal(unsigned *flag) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) st_u(flag, 1u);
}

// All of this block's write-through stores have completed; then thread 0 counts the
// arrival on `c`, and if it is the `target`-th it sets `flag`. Every earlier arrival came
// after its own stores completed, so the flag implies all of them.
__device__ static inline void arrive(unsigned *c, unsigned target, unsigned *flag) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0 && add_u(c) + 1u == target) st_u(flag, 1u);
}

// Bounded spin of one thread until *c >= target; false if it timed out or another block
// already failed.
__device__ static inline bool spin_ge(const unsigned *c, unsigned target, int *error, unsigned limit) {
    unsigned spins = 0;
    while (ld_u(c) < target) {
        if (__hip_atomic_load(error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) return false;
        if (++spins > limit) {
            __hip_atomic_store(error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
        __builtin_amdgcn_s_sleep(2);  // ~128 clocks between polls
    }
    return true;
}

// Block-wide wait until *c >= target (a flag: target 1). Returns false if the wait timed
// out or another block already failed (the caller then returns from the kernel).
__device__ static inline bool wait_ge(const unsigned *c, unsigned target, int *error, SkShared &sh) {
    if (threadIdx.x == 0) {
        sh.ok = spin_ge(c, target, error, sh.spin_limit);
        if (sh.trace) trace_put(sh.trace, SK_TRACE_STAMPS * sh.trace_item + 1);
    }
    __syncthreads();
    return sh.ok != 0;
}

// threadIdx.x, opaque to the optimiser. The phases of the layer loop take their thread
// index from this, so that the many addresses derived from it are computed in the phase
// that uses them rather than hoisted out of the loop and kept live (spilled) throughout.
__device__ static inline int phase_tid() {
    int t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// Diagnostic stamp k of the current item (thread 0, when tracing).
__device__ static inline void sk_stamp(SkShared &sh, int k) {
    if (sh.trace && threadIdx.x == 0) trace_put(sh.trace, SK_TRACE_STAMPS * sh.trace_item + k);
}

// Copy `nbytes` (a multiple of 16) from global memory straight into shared memory, 1 KB
// per wave instruction. Completion is this wave's vmcnt.
__device__ static inline void dma_copy(void *dst, const void *src, int nbytes) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    for (int off = 1024 * w; off < nbytes; off += 1024 * (SK_BLOCK / 64))
        if (off + 16 * lane < nbytes)
            __builtin_amdgcn_global_load_lds((const GM_GLOBAL void *)gbl((const uint8_t *)src + off + 16 * lane),
                                             (lds_void *)((uint8_t *)dst + off), 16, 0, 0);
}


// ---------------------------------------------------------------- top-k selection
//
// Top-k of layer li (infer.c:1108-1145) into sh.idx / sh.wk (normalised) / sh.ws (times
// routed_scale), from the stage entries, by every block that needs it (each routed block
// and router block 0), with no signal in between: wave 0 polls the entries until none is
// unset, lane l holding experts l + 64c.
//
// The K best interval midpoints are taken one at a time (a wave maximum, then the lowest
// lane holding it), and the result is certified when each chosen interval lies strictly
// above the next chosen one and the last chosen lies strictly above every expert left
// out. glm.c's insertion top-k orders strictly by value, so it must then pick the same
// experts in the same order. Every block sees the same entries and so reaches the same
// verdict; when it is "not certified" (or an interval is not finite), router block 0
// replays the fp32 router exactly (sk_exact_select) and the others wait for its result.
// Returns false if the wait timed out or another block failed; sh.sel_ok = certified.
#define SK_SEL_C RT_SEL_C

// The certified selection of the layer (certified_select) into sh.
template <int C>
__device__ __attribute__((always_inline)) static void sk_select_rounds(const StackArgs &a, const unsigned long long *w0,
                                                                       const unsigned long long *w1, bool keep_p,
                                                                       SkShared &sh) {
    certified_select<C>(a.E, a.K, phase_tid(), w0, w1, keep_p ? sh.u.s.p : nullptr, sh.idx, sh.wk, &sh.sel_ok, &sh.total);
}

__device__ __attribute__((always_inline)) static bool sk_stage_select(const StackArgs &a, int li, bool keep_p,
                                                                      SkShared &sh) {
    const int E = a.E, K = a.K, tid = phase_tid();
    if (tid < 64) {
        const int cpy = blockIdx.x % SK_STAGE_COPIES;
        const unsigned long long *sw0 = stage_plane(a, li, cpy, 0), *sw1 = stage_plane(a, li, cpy, 1);
        const int nch = (E + 63) >> 6;
        unsigned long long w0[SK_SEL_C], w1[SK_SEL_C];
        unsigned spins = 0;
        bool alive = true;
        for (;;) {
            bool miss = false;
#pragma unroll
            for (int c = 0; c < SK_SEL_C; c++) {
                const int e = tid + 64 * c < E ? tid + 64 * c : E - 1;
                if (c < nch) {
                    const int pe = stage_pos(e, a.n_router);
                    w0[c] = __hip_atomic_load(sw0 + pe, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    w1[c] = __hip_atomic_load(sw1 + pe, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    miss |= (w0[c] == SK_UNSET) | (w1[c] == SK_UNSET);
                } else {
                    w0[c] = w1[c] = 0ull;
                }
            }
            if (__ballot(miss) == 0) break;
            if (__hip_atomic_load(a.error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) || ++spins > a.spin_limit) {
                if (tid == 0) __hip_atomic_store(a.error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                alive = false;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (sh.trace && tid == 0) trace_put(sh.trace, SK_TRACE_STAMPS * sh.trace_item + 8);
        if (nch == 1)
            sk_select_rounds<1>(a, w0, w1, keep_p, sh);
        else
            sk_select_rounds<SK_SEL_C>(a, w0, w1, keep_p, sh);
        if (tid == 0 && (a.flags & GMOE_FLAG_EXACT_ROUTER)) sh.sel_ok = 0;
        if (tid == 0) sh.ok = alive;
    }
    __syncthreads();
    if (!sh.ok) return false;
    if (sh.sel_ok && tid < K) {
        // normalisation of infer.c:1137-1145
        const float total = sh.total;
        float wk = sh.wk[tid];
        if (total > 0.0f) {
            const float denom = total < 6.103515625e-5f ? 6.103515625e-5f : total;
            wk = __fmul_rn(wk, __fdiv_rn(1.0f, denom));
        }
        sh.wk[tid] = wk;
        sh.ws[tid] = __fmul_rn(wk, a.routed_scale);
    }
    __syncthreads();
    sk_stamp(sh, 3);
    return true;
}

// glm.c's router replayed exactly (exact_router) for layer li, by the router block whose
// xn is in sh.xn_r, when the certified selection failed: the top-k into sh.idx / sh.wk /
// sh.ws and every probability into sh.u.s.p.
__device__ static void sk_exact_select(const StackArgs &a, const StackLayer &L, SkShared &sh) {
    const int tid = phase_tid();
    exact_router(a.D, a.E, a.K, tid, L.gate_inp, L.bias, sh.xn_r, (float(*)[64])sh.dslice, sh.u.s.p, sh.u.s.sel, sh.idx,
                 sh.wk, a.stats);
    if (tid < a.K) sh.ws[tid] = __fmul_rn(sh.wk[tid], a.routed_scale);
    __syncthreads();
}

// Observables of layer `layer` (top-k, weights, router probabilities), written through
// by the block that selected the top-k.
__device__ static void sk_write_routing(const StackArgs &a, int layer, SkShared &sh) {
    const int tid = phase_tid();
    if (tid < a.K) {
        st_i(a.topk_idx + tid, sh.idx[tid]);
        st_f(a.topk_w + tid, sh.wk[tid]);
        st_i(a.hist_idx + (size_t)layer * a.hist_stride + tid, sh.idx[tid]);
        st_f(a.hist_w + (size_t)layer * a.hist_stride + tid, sh.wk[tid]);
    }
    for (int i = tid; i < a.E; i += SK_BLOCK) st_f(a.router_prob + i, sh.u.s.p[i]);
}

// p[0..per) and zeros after, with the widest loads that `per` (a power of two <=
// SK_PER_MAX, p aligned to 4 * per bytes) allows, returned by value so that it lives in
// registers.
struct Seg {
    float v[SK_PER_MAX];
};
template <typename P>
__device__ static inline Seg load_seg(P p, int per) {
    static_assert(SK_PER_MAX == 8, "load_seg covers segments of up to 8 floats");
    Seg r;
    if (per == 8) {
        const float4 a0 = ((const float4 *)p)[0], a1 = ((const float4 *)p)[1];
        r.v[0] = a0.x; r.v[1] = a0.y; r.v[2] = a0.z; r.v[3] = a0.w;
        r.v[4] = a1.x; r.v[5] = a1.y; r.v[6] = a1.z; r.v[7] = a1.w;
    } else if (per == 4) {
        const float4 a0 = ((const float4 *)p)[0];
        r.v[0] = a0.x; r.v[1] = a0.y; r.v[2] = a0.z; r.v[3] = a0.w;
        r.v[4] = r.v[5] = r.v[6] = r.v[7] = 0.0f;
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) r.v[j] = j < per ? p[j] : 0.0f;
    }
    return r;
}

// ---------------------------------------------------------------- rmsnorm
//
// 1 / sqrt(mean + eps) of glm.c's rmsnorm (infer.c:746-752) for the thread's D/256
// consecutive values xv of x: mean = (float)(sum / D) of the sequential fp64 sum of squares,
// certified from the parallel sum (whose relative error is below D * 2^-52), else replayed
// in order by thread 0 from `scratch` (D floats of shared memory). `stat`: count a replay.
__device__ __attribute__((always_inline)) static float sk_inv_rms(const StackArgs &a, const float *xv, float *scratch,
                                                                  bool stat, SkShared &sh) {
    const int D = a.D, per = D / SK_BLOCK, tid = phase_tid();
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < SK_PER_MAX; j++)
        if (j < per) ss += (double)xv[j] * (double)xv[j];
    ss = block_sum_fast(ss, sh.red);
    const double v = ss / (double)D, rho = (double)D * 0x1p-52;
    const float mlo = (float)(v * (1.0 - rho)), mhi = (float)(v * (1.0 + rho));
    float mean = mlo;
    if (mlo != mhi) {
#pragma unroll
        for (int j = 0; j < SK_PER_MAX; j++)
            if (j < per) scratch[tid * per + j] = xv[j];
        __syncthreads();
        if (tid == 0) {
            double sq = 0.0;
            for (int i = 0; i < D; i++) sq += (double)scratch[i] * (double)scratch[i];
            sh.mean = (float)(sq / (double)D);
            if (stat) atomicAdd(&a.stats[GM_STAT_NORM_EXACT], 1ull);
        }
        __syncthreads();
        mean = sh.mean;
        __syncthreads();
    }
    return __fdiv_rn(1.0f, sqrt_rn_f32(__fadd_rn(mean, a.eps)));
}

// ---------------------------------------------------------------- router item
//
// Block b: rmsnorm of x (every router block, bit-identical to infer.c:746-752) and the
// logits of experts b, b + NR, ... (infer.c:916-938) in fp64. Thread t owns the `per`
// consecutive columns [t*per, (t+1)*per), so the exact partial sums S_k of glm.c's
// sequential chain run in thread order: a block-wide scan yields them, and with them
// the bound on the chain's rounding error (router.h). Each expert's result is stored
// as its selection interval and probability.
__device__ __attribute__((always_inline)) static bool sk_router_item(const StackArgs &a, const StackLayer &L, int layer,
                                                                     int li, int b, SkShared &sh) {
    const int D = a.D, E = a.E, NR = a.n_router, tid = phase_tid();
    const int lane = tid & 63, w = tid >> 6;
    const int per = D / SK_BLOCK;
    const int nx = (E - b + NR - 1) / NR;
    // The norm and router weights do not depend on x: fetch them before waiting on x, but
    // after the previous layer's expert items are done. A CU's vector memory path is
    // shared by its two blocks, and these requests issued during the routed weight burst
    // would queue the other block (an expert item) behind them for microseconds.
    if (li > 0 && !wait_ge(&a.ctr[SKF(li - 1, SKF_PART)], 1u, a.error, sh)) return false;
    const Seg nw = load_seg(gbl(L.norm) + tid * per, per);
    // the selection biases of this block's experts, for lanes 4x of the bound tail below
    const float bias_x = tid < 4 * nx ? gbl(L.bias)[b + (tid >> 2) * NR] : 0.0f;
    Seg gw[SK_RX_MAX];
#pragma unroll
    for (int x = 0; x < SK_RX_MAX; x++) {
        if (x < nx) {  // block-uniform
            gw[x] = load_seg(gbl(L.gate_inp) + (size_t)(b + x * NR) * D + tid * per, per);
        } else {
#pragma unroll
            for (int j = 0; j < SK_PER_MAX; j++) gw[x].v[j] = 0.0f;
        }
    }
    if (li > 0 && !wait_ge(&a.ctr[SKF(li - 1, SKF_X)], 1u, a.error, sh)) return false;
    Seg xs = load_seg((li == 0 ? a.x_in : ws_at<float>(a, li, a.o.x)) + tid * per, per);
    float *xv = xs.v;
    const float inv = sk_inv_rms(a, xv, sh.xn_r, b == 0, sh);
    sk_stamp(sh, 11);
#pragma unroll
    for (int j = 0; j < SK_PER_MAX; j++) xv[j] = j < per ? __fmul_rn(__fmul_rn(xv[j], inv), nw.v[j]) : 0.0f;

    float mloc = 0.0f;
#pragma unroll
    for (int j = 0; j < SK_PER_MAX; j++)
        if (j < per) {
            sh.xn_r[tid * per + j] = xv[j];
            mloc = fmaxf(mloc, fabsf(xv[j]));
        }
    mloc = (float)wave_max_dpp((double)mloc);
    if (lane == 0) sh.mxw[w] = mloc;
    __syncthreads();
    // Products in fp64 are exact (24 + 24 bits). Pass 1: this thread's segment sums and
    // the block-wide exclusive prefix, in column order.
    double sabs[SK_RX_MAX] = {0.0}, pre[SK_RX_MAX] = {0.0};
#pragma unroll
    for (int x = 0; x < SK_RX_MAX; x++) {
        if (x >= nx) break;  // block-uniform
        double s = 0.0, sa = 0.0;
#pragma unroll
        for (int j = 0; j < SK_PER_MAX; j++) {
            const double pj = (double)gw[x].v[j] * (double)xv[j];
            s += pj;
            sa += fabs(pj);
        }
        sabs[x] = sa;
        const double incl = wave_incl_scan_dpp(s);
        pre[x] = incl - s;
        if (lane == 63) sh.u.r.wv[w][x][0] = incl;
    }
    __syncthreads();
    // Pass 2: |S_k| after each column, with the waves before this one added in
#pragma unroll
    for (int x = 0; x < SK_RX_MAX; x++) {
        if (x >= nx) break;  // block-uniform
        double off = 0.0;
        for (int v2 = 0; v2 < w; v2++) off += sh.u.r.wv[v2][x][0];
        double run = off + pre[x], steps = 0.0;
#pragma unroll
        for (int j = 0; j < SK_PER_MAX; j++) {
            run += (double)gw[x].v[j] * (double)xv[j];
            steps += fabs(run);
        }
        const double sp = wave_sum_dpp(steps), sa = wave_sum_dpp(sabs[x]);
        if (lane == 0) {
            sh.u.r.wv[w][x][1] = sp;
            sh.u.r.wv[w][x][2] = sa;
        }
    }
    __syncthreads();
    sk_stamp(sh, 13);
    // The bound and the three sigmoids of each expert's entry (interval ends and p) on
    // three lanes of wave 0, lane 4x + r (r < 3) for expert x.
    if (tid < 64) {
        const int x = (tid >> 2) < nx ? tid >> 2 : 0, r = tid & 3, e = b + x * NR;
        const double S = ((sh.u.r.wv[0][x][0] + sh.u.r.wv[1][x][0]) + sh.u.r.wv[2][x][0]) + sh.u.r.wv[3][x][0];
        const double sp = ((sh.u.r.wv[0][x][1] + sh.u.r.wv[1][x][1]) + sh.u.r.wv[2][x][1]) + sh.u.r.wv[3][x][1];
        const double sa = ((sh.u.r.wv[0][x][2] + sh.u.r.wv[1][x][2]) + sh.u.r.wv[2][x][2]) + sh.u.r.wv[3][x][2];
        const double u = 0x1p-24, n = (double)D;
        const double gamma = n * u / (1.0 - n * u);
        const double emax = gamma * sa;  // a priori bound on every partial sum's error
        // step k rounds |fl(s_{k-1}) + fl(p_k)| <= |S_k| + emax + u|p_k| by at most u times
        // that, and each product adds u|p_k|
        double B = u * (1.0 + u) * sa + u * (sp + n * emax + u * sa);
        B = B * (1.0 + 0x1p-30) + 0x1p-40 * sa + n * 0x1p-149;
        const float arg = r == 0 ? f32_rd(S - B) : r == 1 ? f32_ru(S + B) : (float)S;
        const float sg = 1.0f / (1.0f + expf(-arg));
        // lanes 4x + 1 and 4x + 2 of the quad, to lane 4x (quad_perm [1,1,2,3] and [2,1,2,3])
        const float phi = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sg), 0xE5, 0xF, 0xF, false));
        const float p = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(sg), 0xE6, 0xF, 0xF, false));
        if (r == 0 && (tid >> 2) < nx) {
            double lo, hi;
            selection_bounds((double)sg, (double)phi, bias_x, &lo, &hi);
            float lo_f = f32_rd(lo), hi_f = f32_ru(hi);
            if (!(lo_f <= hi_f)) {  // NaN: an interval that is never certified
                lo_f = -INFINITY;
                hi_f = INFINITY;
            }
            const int pe = stage_pos(e, NR);
            const unsigned long long v0 = (unsigned long long)__float_as_uint(lo_f) | ((unsigned long long)__float_as_uint(hi_f) << 32);
#pragma unroll
            for (int cp = 0; cp < SK_STAGE_COPIES; cp++) {
                st_u64(stage_plane(a, li, cp, 1) + pe, (unsigned long long)__float_as_uint(p));
                st_u64(stage_plane(a, li, cp, 0) + pe, v0);
            }
        }
    }
    sk_stamp(sh, 5);
    // This block's share of xn and its digit form for the layer's expert items: 32-column
    // blocks q = b, b + NR, ... (every router block holds all of xn). Thread t takes
    // columns 8 (t % 4) .. +8 of block b + NR (t / 4). All of xn shares one exponent (from
    // its max |xn|, which every router block finds alike), so that an expert item's block
    // dots need only their weight scales. The DIG flag covers these stores.
    {
        const int ex = digit_exponent(fmaxf(fmaxf(sh.mxw[0], sh.mxw[1]), fmaxf(sh.mxw[2], sh.mxw[3])));
        const int q = b + NR * (tid >> 2);
        if (q < D / 32) {
            int8_t *dig = ws_at<int8_t>(a, li, a.o.dig);
            int *dexp = ws_at<int>(a, li, a.o.dexp);
            float *wxn = ws_at<float>(a, li, a.o.xn);
            const int i0 = 32 * q + 8 * (tid & 3);
            float vals[8];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                vals[j] = sh.xn_r[i0 + j];
                st_f(a.xn + i0 + j, vals[j]);
                st_f(wxn + i0 + j, vals[j]);
            }
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
            if ((tid & 3) == 0) st_i(dexp + q, ex);
        }
    }
    sk_stamp(sh, 12);
    arrive(&a.ctr[SKC(SKC_DIG)], (unsigned)(li + 1) * NR, &a.ctr[SKF(li, SKF_DIG)]);

    // Router block 0 also selects the top-k, writes the layer's observables, and when the
    // selection is not certified replays the router exactly and publishes the result: the
    // SEL words first (the routed blocks wait on them), then the weights under SELW.
    if (b == 0) {
        if (!sk_stage_select(a, li, true, sh)) return false;
        if (!sh.sel_ok) {
            sk_exact_select(a, L, sh);
            if (tid < SK_SEL_WORDS) {
                unsigned long long word = 0;
                for (int q = 0; q < 4; q++) {
                    const int k = 4 * tid + q;
                    const unsigned v = k < a.K ? (unsigned)(sh.idx[k] + 2) : 1u;
                    word |= (unsigned long long)v << (16 * q);
                }
                st_u64((unsigned long long *)&a.ctr[SKF(li, SKF_SEL) + 2 * tid], word);
            }
            float *ex_w = ws_at<float>(a, li, a.o.ex_w);
            if (tid < a.K) st_f(ex_w + tid, sh.wk[tid]);
        }
        sk_write_routing(a, layer, sh);
        if (!sh.sel_ok) signal(&a.ctr[SKF(li, SKF_SELW)]);
    }
    return true;
}

// The top-k of layer li from the SEL words (published by the exact replay), into sh.idx.
__device__ static inline bool sk_read_topk(const StackArgs &a, int li, SkShared &sh) {
    const int tid = threadIdx.x;
    if (tid == 0) {
        const int nw = (a.K + 3) / 4;
        bool ok = true;
        for (int wd = 0; wd < nw && ok; wd++) {
            const unsigned long long *p = (const unsigned long long *)&a.ctr[SKF(li, SKF_SEL) + 2 * wd];
            unsigned spins = 0;
            unsigned long long v;
            while ((v = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) == 0ull) {
                if (__hip_atomic_load(a.error, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) || ++spins > a.spin_limit) {
                    __hip_atomic_store(a.error, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ok = false;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
            for (int q = 0; q < 4 && ok; q++)
                if (4 * wd + q < a.K) sh.idx[4 * wd + q] = (int)((v >> (16 * q)) & 0xffffu) - 2;
        }
        sh.ok = ok;
        if (sh.trace) trace_put(sh.trace, SK_TRACE_STAMPS * sh.trace_item + 8);
    }
    __syncthreads();
    return sh.ok != 0;
}

// The normalised weights of the exact replay's top-k (published after the SEL words),
// into sh.wk / sh.ws.
__device__ static inline bool sk_read_weights(const StackArgs &a, int li, SkShared &sh) {
    if (!wait_ge(&a.ctr[SKF(li, SKF_SELW)], 1u, a.error, sh)) return false;
    const int tid = phase_tid();
    if (tid < a.K) {
        const float wk = ws_at<float>(a, li, a.o.ex_w)[tid];
        sh.wk[tid] = wk;
        sh.ws[tid] = __fmul_rn(wk, a.routed_scale);
    }
    __syncthreads();
    return true;
}

// ---------------------------------------------------------------- a routed block's own digits
//
// xn of layer li in its digit form, computed by a routed block itself while the router
// blocks run: the same rmsnorm of the same x, so the same xn as theirs. The digits go to
// sh.xn_r's space as [3][D] int8 (thread t: columns 8t .. 8t + 7), the exponent to
// sh.xe_local. The block's expert items then wait for nothing of the router's but the
// routing, and their weight requests have nothing queued ahead of them. D == GM_MAX_COLS.
__device__ __attribute__((always_inline)) static bool sk_local_digits(const StackArgs &a, const StackLayer &L, int li,
                                                                     SkShared &sh) {
    const int D = a.D, per = D / SK_BLOCK, tid = phase_tid(), lane = tid & 63, w = tid >> 6;
    const Seg nw = load_seg(gbl(L.norm) + tid * per, per);
    if (li > 0 && !wait_ge(&a.ctr[SKF(li - 1, SKF_X)], 1u, a.error, sh)) return false;
    Seg xs = load_seg((li == 0 ? a.x_in : ws_at<float>(a, li, a.o.x)) + tid * per, per);
    float *xv = xs.v;
    const float inv = sk_inv_rms(a, xv, (float *)sh.dslice, false, sh);
    float mloc = 0.0f;
#pragma unroll
    for (int j = 0; j < SK_PER_MAX; j++) {
        xv[j] = __fmul_rn(__fmul_rn(xv[j], inv), nw.v[j]);
        mloc = fmaxf(mloc, fabsf(xv[j]));
    }
    mloc = wave_max_dpp_f(mloc);
    if (lane == 0) sh.mxw[w] = mloc;
    __syncthreads();
    const int ex = digit_exponent(fmaxf(fmaxf(sh.mxw[0], sh.mxw[1]), fmaxf(sh.mxw[2], sh.mxw[3])));
    unsigned long long w0 = 0, w1 = 0, w2 = 0;
#pragma unroll
    for (int j = 0; j < SK_PER_MAX; j++) {
        int8_t d0, d1, d2;
        split_digits(xv[j], ex, &d0, &d1, &d2);
        w0 |= (unsigned long long)(uint8_t)d0 << (8 * j);
        w1 |= (unsigned long long)(uint8_t)d1 << (8 * j);
        w2 |= (unsigned long long)(uint8_t)d2 << (8 * j);
    }
    unsigned long long *dig = (unsigned long long *)sh.xn_r;
    dig[tid] = w0;
    dig[D / 8 + tid] = w1;
    dig[2 * (D / 8) + tid] = w2;
    if (tid == 0) sh.xe_local = ex;
    return true;  // the routing wait that follows ends with a barrier
}

// ---------------------------------------------------------------- expert item
//
// Gate and up rows [16j, 16j+16) of one expert dotted with xn, in units of 2^e where e is
// the single exponent of xn's digit form `dig` ([3][cols] int8). Wave w takes the 64-column
// chunks [w*cpw, (w+1)*cpw) held in `r`; each 32-column block is one MFMA per matrix (A =
// the three digit rows, B = the 16 weight rows), whose int dots lanes 0..15 turn into their
// row's fp32 block dot and scale by the block's fp16 scale (scg, scu: [16 rows][cols/32]).
// Rows 3..15 of A do not reach rows 0..2 of the product, so lanes 3..15 read digit row 0
// unmasked. Chunks past cpw (cols below 2048) read chunk 0's digits with zero scales
// (`zero`: a shared word that holds 0). The digits and scales are read before the first
// product; chunk u's products are then done before chunk u + 1's weights are touched, so
// that while the weights are still arriving each chunk waits only for its own loads.
// Lanes 0..15 return their row's sums.
// The gate/up products from register operands: A[u] = the two 8-byte digit pieces of
// chunk u for this lane (row lane & 15, column group lane >> 4), sg[u] and su[u] = the fp16
// scales of chunk u's two blocks for row lane & 15. Chunk u's products and their sums are
// done before chunk u + 1's weights are touched, so that while the weights are still
// arriving each chunk waits only for its own loads. Lanes 0..15 return their row's sums.
template <int NB>
__device__ static inline void gu_products_r(const PanelRegs<2, NB> &r, const long (&A)[NB][2], const unsigned (&sg)[NB],
                                            const unsigned (&su)[NB], float out[2]) {
    float ag = 0.0f, au = 0.0f;
    u32x4 qg = r.q[0][0], qu = r.q[1][0];
#pragma unroll
    for (int u = 0; u < NB; u++) {
        const v4i g0 = mfma_digits(A[u][0], chunk_half(qg, 0));
        const v4i g1 = mfma_digits(A[u][1], chunk_half(qg, 1));
        const v4i u0 = mfma_digits(A[u][0], chunk_half(qu, 0));
        const v4i u1 = mfma_digits(A[u][1], chunk_half(qu, 1));
        ag = fmaf(digits_to_float(g0[0], g0[1], g0[2]), __half2float(__ushort_as_half((unsigned short)(sg[u] & 0xffffu))), ag);
        ag = fmaf(digits_to_float(g1[0], g1[1], g1[2]), __half2float(__ushort_as_half((unsigned short)(sg[u] >> 16))), ag);
        au = fmaf(digits_to_float(u0[0], u0[1], u0[2]), __half2float(__ushort_as_half((unsigned short)(su[u] & 0xffffu))), au);
        au = fmaf(digits_to_float(u1[0], u1[1], u1[2]), __half2float(__ushort_as_half((unsigned short)(su[u] >> 16))), au);
        // the sums here on every lane (not sunk to the lanes that use them), and chunk u + 1's
        // weights taken only now (so that its products are not hoisted above these)
        if (u + 1 < NB) {
            qg = r.q[0][u + 1];
            qu = r.q[1][u + 1];
        }
        asm volatile("" : "+v"(ag), "+v"(au), "+v"(qg), "+v"(qu));
    }
    out[0] = ag;
    out[1] = au;
}

// Gate and up rows [16j, 16j+16) of one expert dotted with xn, in units of 2^e where e is
// the single exponent of xn's digit form `dig` ([3][cols] int8, in shared memory). Wave w
// takes the 64-column chunks [w*cpw, (w+1)*cpw) held in `r`; each 32-column block is one
// MFMA per matrix (A = the three digit rows, B = the 16 weight rows), whose int dots lanes
// 0..15 turn into their row's fp32 block dot and scale by the block's fp16 scale (scg, scu:
// [16 rows][cols/32], in shared memory). Rows 3..15 of A do not reach rows 0..2 of the
// product, so lanes 3..15 read digit row 0 unmasked. Chunks past cpw (cols below 2048) read
// chunk 0's digits with zero scales (`zero`: a shared word that holds 0).
template <int NB>
__device__ static inline void gu_products(const PanelRegs<2, NB> &r, int cols, const int8_t *dig,
                                          const unsigned short *scg, const unsigned short *scu, const unsigned *zero,
                                          float out[2]) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int cpw = cols >> 8, j0 = w * cpw, nblocks = cols >> 5;
    const int m = lane & 15;
    const int8_t *drow = dig + (m < 3 ? m : 0) * cols + 64 * j0 + 8 * (lane >> 4);
    const unsigned *pg = (const unsigned *)(scg + m * nblocks + 2 * j0);
    const unsigned *pu = (const unsigned *)(scu + m * nblocks + 2 * j0);
    long A[NB][2];
    unsigned sg[NB], su[NB];
#pragma unroll
    for (int u = 0; u < NB; u++) {
        const bool on = u < cpw;
        A[u][0] = *(const long *)(drow + 64 * (on ? u : 0));
        A[u][1] = *(const long *)(drow + 64 * (on ? u : 0) + 32);
        sg[u] = *(on ? pg + u : zero);
        su[u] = *(on ? pu + u : zero);
    }
    gu_products_r<NB>(r, A, sg, su, out);
}

// gu_products at group size 16 with fp32 scales: the two 16-column groups of every
// 32-column block get their own scale. A's rows 0..2 hold the digits of the block's first
// 16 columns (zeros in its last 16) and rows 4..6 those of its last 16 (zeros in its first),
// so the one MFMA per block and matrix leaves the first group's three digit dots on lanes
// 0..15 and the second group's on lanes 16..31 (rows 4..6 of the product), each lane
// scaling by its own group's scale; lanes 0..15 end with the sum of both. Rows 3 and 7..15
// of the product are never read. sg16 / su16: the wave's scale runs in shared memory,
// [cpw chunks][16 rows][2 groups][2 blocks] each; chunks past cpw read chunk 0 and add zero.
template <int NB>
__device__ static inline void gu_products16(const PanelRegs<2, NB> &r, int cols, int cpw, const int8_t *dig,
                                            const float *sg16, const float *su16, float out[2]) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, m = lane & 15, kq = lane >> 4;
    const int j0 = w * cpw;
    const int dr = (m & 3) < 3 ? (m & 3) : 0;      // the digit row of A row m (rows 3, 7: any)
    const bool on = (m < 4) == (kq < 2);           // rows 0..3 take k 0..15, rows 4..7 k 16..31
    const int8_t *drow = dig + dr * cols + 64 * j0 + 8 * kq;
    const int so = 2 * (2 * m + (kq & 1));         // the lane's (row, group) pair in a chunk's run
    float ag = 0.0f, au = 0.0f;
    u32x4 qg = r.q[0][0], qu = r.q[1][0];
#pragma unroll
    for (int u = 0; u < NB; u++) {
        const bool in = u < cpw;
        const int uu = in ? u : 0;
        const long a0 = *(const long *)(drow + 64 * uu), a1 = *(const long *)(drow + 64 * uu + 32);
        const float2 sgv = *(const float2 *)(sg16 + 64 * uu + so), suv = *(const float2 *)(su16 + 64 * uu + so);
        const long A0 = on ? a0 : 0, A1 = on ? a1 : 0;
        const float sg0 = in ? sgv.x : 0.0f, sg1 = in ? sgv.y : 0.0f, su0 = in ? suv.x : 0.0f, su1 = in ? suv.y : 0.0f;
        const v4i g0 = mfma_digits(A0, chunk_half(qg, 0));
        const v4i g1 = mfma_digits(A1, chunk_half(qg, 1));
        const v4i u0 = mfma_digits(A0, chunk_half(qu, 0));
        const v4i u1 = mfma_digits(A1, chunk_half(qu, 1));
        ag = fmaf(digits_to_float(g0[0], g0[1], g0[2]), sg0, ag);
        ag = fmaf(digits_to_float(g1[0], g1[1], g1[2]), sg1, ag);
        au = fmaf(digits_to_float(u0[0], u0[1], u0[2]), su0, au);
        au = fmaf(digits_to_float(u1[0], u1[1], u1[2]), su1, au);
        if (u + 1 < NB) {
            qg = r.q[0][u + 1];
            qu = r.q[1][u + 1];
        }
        asm volatile("" : "+v"(ag), "+v"(au), "+v"(qg), "+v"(qu));
    }
    out[0] = ag + __shfl_xor(ag, 16, 64);
    out[1] = au + __shfl_xor(au, 16, 64);
}

// Rows [16j, 16j+16) of F for expert e in `slot` (-1: idle slot, nothing to compute):
// g, u = gate, up rows . xn (infer.c:1184-1185, 1199-1200), h = silu(g) * u (:1188, :1202),
// and the partial y = down[:, 16j..16j+16) . h over all D rows (:1190, :1205), stored at
// ypart[slot][j]. Thread t owns the down rows t + 256 i.
// LOCAL (routed items, whose block computed xn's digits itself, sk_local_digits) on a
// full-width layer: the gate/up chunks are the last requests, and the products of chunk u
// start as soon as chunk u has arrived. Otherwise (shared items, which start before xn
// exists, and narrower layers) the weights are requested first and the router blocks'
// digits once the DIG flag is seen.
template <bool LOCAL>
__device__ __attribute__((always_inline)) static bool sk_expert_item(const StackArgs &a, const StackLayer &L, int li,
                                                                     int slot, int j, int e, SkShared &sh) {
    const int D = a.D, F = a.F, NPF = F >> 4, tid = phase_tid();
    if (e >= 0) {
        const uint8_t *base = L.experts + (size_t)e * a.stride;
        const int c = D / SK_BLOCK, wave0 = tid & ~63, lane = tid & 63, w = tid >> 6;
        const GM_GLOBAL u32x4 *qs = gbl((const u32x4 *)(base + a.off_dq)) + (size_t)j * D + tid;
        const int o = 1024 * w + 16 * lane;  // this lane's 16 bytes of the item's scale runs
        PanelRegs<2, EX_NB_MAX> pr;
        float gu[2];
        int xe;  // the exponent of all of xn's digits
        if (LOCAL && D == GM_MAX_COLS) {
            // The down scales and the down slice go to shared memory first (row t + 256 i of
            // the slice lands at dslice[t + 256 i]), by DMA that the compiler does not count,
            // then the gate/up scales and chunks to registers: the compiler then waits for each
            // chunk by itself.
            const int m = lane & 15, j0 = w * EX_NB_MAX;
            dma16_untracked(gbl(base + a.off_ds + (size_t)(j >> 1) * D * 2 + o),
                            (lds_void *)((uint8_t *)sh.sc_d + 1024 * w));  // o < 2 D here
#pragma unroll
            for (int i = 0; i < SK_PER_MAX; i++)
                dma16_untracked(qs + (size_t)i * SK_BLOCK, (lds_void *)(sh.dslice + i * SK_BLOCK + wave0));
            // row m's scales of blocks 2 j0 .. 2 j0 + 15 (panel j's plane is [16 rows][D/32])
            const size_t so = (size_t)j * D + (size_t)m * (D / 16) + 4 * j0;
            const GM_GLOBAL u32x4 *pg = gbl((const u32x4 *)(base + a.off_gs + so));
            const GM_GLOBAL u32x4 *pu = gbl((const u32x4 *)(base + a.off_us + so));
            const u32x4 g0 = pg[0], g1 = pg[1], u0 = pu[0], u1 = pu[1];
            __builtin_amdgcn_sched_barrier(0);  // the scales are requested before the chunks
            panel_load_q_all<2, EX_NB_MAX>(pr, base + a.off_gq, base + a.off_uq, j, D);
            __builtin_amdgcn_sched_barrier(0);  // every request issued before any product
            // the block's own digits (rows 3..15 of A do not reach the sums: lanes m >= 3
            // read row 0)
            const int8_t *drow = (const int8_t *)sh.xn_r + (m < 3 ? m : 0) * D + 64 * j0 + 8 * (lane >> 4);
            long A[EX_NB_MAX][2];
#pragma unroll
            for (int u = 0; u < EX_NB_MAX; u++) {
                A[u][0] = *(const long *)(drow + 64 * u);
                A[u][1] = *(const long *)(drow + 64 * u + 32);
            }
            const unsigned sg[EX_NB_MAX] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
            const unsigned su[EX_NB_MAX] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
            gu_products_r<EX_NB_MAX>(pr, A, sg, su, gu);
            xe = sh.xe_local;
            // the down slice and scales (not counted by the compiler) are in shared memory
            // before the barrier below
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        } else {
            // Every weight of the item is requested before anything waits: the gate/up chunks
            // to registers, the down slice and all scales straight to shared memory. The
            // digits follow once the DIG flag is seen.
            if (o < 2 * D) {
                // gate then up scales of panel j (D bytes each, contiguous in their s planes),
                // then the down scales of column block j/2 (one fp16 per row, 2D bytes)
                const uint8_t *src = o < D ? base + a.off_gs + (size_t)j * D + o : base + a.off_us + (size_t)j * D + (o - D);
                __builtin_amdgcn_global_load_lds((const GM_GLOBAL void *)gbl(src), (lds_void *)((uint8_t *)sh.sc_gu + 1024 * w),
                                                 16, 0, 0);
                __builtin_amdgcn_global_load_lds((const GM_GLOBAL void *)gbl(base + a.off_ds + (size_t)(j >> 1) * D * 2 + o),
                                                 (lds_void *)((uint8_t *)sh.sc_d + 1024 * w), 16, 0, 0);
            }
            panel_load_q<2, EX_NB_MAX>(pr, base + a.off_gq, base + a.off_uq, j, D);
#pragma unroll
            for (int i = 0; i < SK_PER_MAX; i++)
                if (i < c)
                    __builtin_amdgcn_global_load_lds((const GM_GLOBAL void *)(qs + (size_t)i * SK_BLOCK),
                                                     (lds_void *)(sh.dslice + i * SK_BLOCK + wave0), 16, 0, 0);
            if (!wait_ge(&a.ctr[SKF(li, SKF_DIG)], 1u, a.error, sh)) return false;  // digits of xn ready
            dma_copy(sh.u.g.dig, ws_at<unsigned long long>(a, li, a.o.dig), 3 * D);
            dma_copy(sh.u.g.dexp, ws_at<int>(a, li, a.o.dexp), D / 8);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();  // every wave's digits, scales and slice rows are in shared memory
            sk_stamp(sh, 6);
            gu_products<EX_NB_MAX>(pr, D, sh.u.g.dig, sh.sc_gu, sh.sc_gu + D / 2, &sh.zero, gu);
            xe = sh.u.g.dexp[0];
        }
        if (lane < 16) {
            sh.u.g.part[w][0][lane] = gu[0];
            sh.u.g.part[w][1][lane] = gu[1];
        }
        __syncthreads();
        if (tid < 16) {
            // SwiGLU of the 16 rows, then their digit form with one exponent
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
        // partials in combine order: [D/16 chunks][F/16][K+1 slots][16 rows]: 64-byte pieces, since 32-byte
        // write-through stores cost the weight stream about a fifth of its bandwidth
        const int NS = a.K + 1, KA = sk_early_slots(a);
        // row r = 256 i + t goes to combine chunk r / 16 = 16 i + t / 16, at row r % 16 of
        // piece (j, position of slot)
        const size_t ychunk = (size_t)NS * NPF * SK_CROWS;
        float *yp = ws_at<float>(a, li, a.o.ypart) + sk_piece(j, sk_pos(slot, a.K, KA), NPF, NS, KA + 1) +
                    (tid & (SK_CROWS - 1)) + (size_t)(tid / SK_CROWS) * ychunk;
        // every slice row and scale of this thread is read before the first product (rows
        // past D read shared memory that is never used), so the reads cost one latency
        u32x4 dqs[SK_PER_MAX];
        unsigned scs[SK_PER_MAX];
#pragma unroll
        for (int i = 0; i < SK_PER_MAX; i++) {
            dqs[i] = sh.dslice[i * SK_BLOCK + tid];
            scs[i] = sh.sc_d[i * SK_BLOCK + tid];
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
                const float f = digits_to_float(acc[0], acc[1], acc[2]);
                st_f(yp + (size_t)i * (SK_BLOCK / SK_CROWS) * ychunk,
                     f * ldexpf(__half2float(__ushort_as_half((unsigned short)scs[i])), hexp));
            }
        }
    }
    sk_stamp(sh, 5);
    // two-level count of the layer's (K+1) * F/16 items, then the layer's flag; group A's
    // items also count for the PARTA flag (on another wave, so the two run side by side)
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        const unsigned per_ctr = (unsigned)((a.K + 1) * NPF / SK_NPART);
        if (add_u(&a.ctr[SKC(SKC_PART + (slot * NPF + j) % SK_NPART)]) + 1u == (unsigned)(li + 1) * per_ctr &&
            add_u(&a.ctr[SKC(SKC_PART2)]) + 1u == (unsigned)(li + 1) * SK_NPART)
            st_u(&a.ctr[SKF(li, SKF_PART)], 1u);
    } else if (tid == 64) {
        const int KA = sk_early_slots(a), pos = sk_pos(slot, a.K, KA);
        const unsigned per_a = (unsigned)((KA + 1) * NPF / SK_NPART);
        if (pos <= KA && add_u(&a.ctr[SKC(SKC_PA + (pos * NPF + j) % SK_NPART)]) + 1u == (unsigned)(li + 1) * per_a &&
            add_u(&a.ctr[SKC(SKC_PA2)]) + 1u == (unsigned)(li + 1) * SK_NPART)
            st_u(&a.ctr[SKF(li, SKF_PARTA)], 1u);
    }
    return true;
}

// ---------------------------------------------------------------- combine
//
// Rows [16c, 16c+16) of x' = x + (shared + sum_k w_e * y_k) (infer.c:1192, 1212-1214),
// with y_k the sum of expert k's F/16 partials in a fixed order. Group A's partials
// (sk_early_slots) are summed first, while group B's items still run, then group B's.
// Each group's partials are one contiguous run ([j][position][16 rows]), copied to
// shared memory with wide loads.
//
// A group of np positions has P = 16 np (position, row) pairs and Q = min(8, 256 / P)
// groups of threads: thread q P + p adds the partials j = q, q + Q, ... of pair p in
// order, then P threads add the Q group sums in order. Shared-memory reads are issued
// eight at a time (clamped indices, masked values), so each batch costs one latency.
__device__ __attribute__((always_inline)) static void sk_combine_sums(const float *gb, int np, int p0, int NPF,
                                                                      SkShared &sh) {
    const int tid = phase_tid();
    const int P = np * SK_CROWS, Qm = SK_BLOCK / P, Q = Qm < 8 ? Qm : 8;
    if (tid < P * Q) {
        const int q = tid / P, pr = tid - q * P;
        float s = 0.0f;
        for (int j0 = q; j0 < NPF; j0 += 8 * Q) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int jq = j0 + u * Q;
                v[u] = gb[(jq < NPF ? jq : q) * P + pr];
            }
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (j0 + u * Q < NPF) s += v[u];
        }
        sh.u.c.acc[q][p0 + pr / SK_CROWS][pr % SK_CROWS] = s;
    }
    __syncthreads();
    if (tid < P) {  // each pair's Q group sums, in order
        float v[8];
#pragma unroll
        for (int q = 0; q < 8; q++) v[q] = sh.u.c.acc[q < Q ? q : 0][p0 + tid / SK_CROWS][tid % SK_CROWS];
        float y = v[0];
#pragma unroll
        for (int q = 1; q < 8; q++)
            if (q < Q) y += v[q];
        sh.u.c.y[p0 + tid / SK_CROWS][tid % SK_CROWS] = y;
    }
}

__device__ __attribute__((always_inline)) static bool sk_combine(const StackArgs &a, int li, int c, bool routed_on,
                                                                 SkShared &sh) {
    const int D = a.D, K = a.K, NS = K + 1, NPF = a.F >> 4, tid = phase_tid();
    const int KA = sk_early_slots(a), NA = KA + 1;
    // the residual rows, fetched while the expert items finish
    const int r = c * SK_CROWS + (tid & (SK_CROWS - 1));
    const float xr = tid < SK_CROWS ? (li == 0 ? a.x_in : ws_at<float>(a, li, a.o.x))[r] : 0.0f;
    // the chunk's partials: NPF * NS * 16 floats <= sizeof(sh.dslice) (the host checks it)
    const float *chunk = ws_at<float>(a, li, a.o.ypart) + (size_t)c * NPF * NS * SK_CROWS;
    for (int g = 0; g < 2; g++) {
        const int p0 = g == 0 ? 0 : NA, np = g == 0 ? NA : NS - NA;
        if (np == 0) break;  // block-uniform
        if (!wait_ge(&a.ctr[SKF(li, g == 0 ? SKF_PARTA : SKF_PART)], 1u, a.error, sh)) return false;
        const int off = p0 * NPF * SK_CROWS;  // group B follows group A's NPF * NA pieces
        dma_copy((float *)sh.dslice + off, chunk + off, np * NPF * SK_CROWS * (int)sizeof(float));
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        sk_combine_sums((const float *)sh.dslice + off, np, p0, NPF, sh);
    }
    __syncthreads();
    if (tid < SK_CROWS) {
        const int rl = tid;
        float y[GM_MAX_K];
#pragma unroll
        for (int k = 0; k < GM_MAX_K; k++) y[k] = sh.u.c.y[k < K ? sk_pos(k, K, KA) : 0][rl];
        float acc = 0.0f;
        if (routed_on) {
#pragma unroll
            for (int k = 0; k < GM_MAX_K; k++)
                if (k < K && sh.idx[k] >= 0) acc = __fadd_rn(acc, __fmul_rn(sh.ws[k], y[k]));
        }
        const float shv = sh.u.c.y[KA][rl];  // the shared expert's position
        st_f(a.routed_out + r, acc);
        st_f(a.shared_out + r, shv);
        float *xo = li == a.n_layers - 1 ? a.x_out : ws_at<float>(a, li + 1, a.o.x);
        st_f(xo + r, __fadd_rn(xr, __fadd_rn(shv, acc)));
    }
    sk_stamp(sh, 5);
    // two-level count of the layer's D/16 chunks, then the layer's flag
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        const unsigned per_ctr = (unsigned)(D / SK_CROWS / SK_NPART);
        if (add_u(&a.ctr[SKC(SKC_X + c % SK_NPART)]) + 1u == (unsigned)(li + 1) * per_ctr &&
            add_u(&a.ctr[SKC(SKC_X2)]) + 1u == (unsigned)(li + 1) * SK_NPART)
            st_u(&a.ctr[SKF(li, SKF_X)], 1u);
    }
    return true;
}

// Launch set-up, one block per layer plus one: block n_layers zeroes the counters; block
// li puts layer li's stage entries to SK_UNSET.
__global__ __launch_bounds__(SK_BLOCK) void k_stack_reset(unsigned *ctr, int n, int *error, StackArgs a) {
    const int li = blockIdx.x, tid = threadIdx.x;
    if (li == a.n_layers) {
        for (int i = tid; i < n; i += SK_BLOCK) ctr[i] = 0u;
        if (tid == 0) *error = 0;
        // relay.h: this launch writes the other parity into each of its workspace layers
        if (a.par_dev && tid < SK_MAX_LAYERS / 64) {
            const int lo = 64 * tid, cnt = a.n_layers - lo;
            if (cnt > 0) a.par_dev[tid] ^= cnt >= 64 ? ~0ull : (1ull << cnt) - 1ull;
        }
        return;
    }
    unsigned long long *stage = ws_at<unsigned long long>(a, li, a.o.stage);
    for (int i = tid; i < SK_STAGE_COPIES * SK_STAGE_COPY_WORDS; i += SK_BLOCK) stage[i] = SK_UNSET;
}

// Block roles: the first n_router blocks route, and router blocks 1.. then take the shared
// expert's items beyond the shared blocks' share; shared_blocks blocks from G/2 on run one
// shared item each, then wait until the layer's combine is done before taking the next
// layer's (so its 10 MB of weights stream during the next router phase, not during the
// routed burst or the combine's reads); the rest compute xn's digits themselves, wait for
// the routing, run the routed experts' items and then the combine chunks. Trace items of
// one layer are numbered: n_router router items, D/16 combine chunks, F/16 shared items,
// K*F/16 routed items (a routed block's top-k is stamped on its first expert item).
__device__ __attribute__((always_inline)) static bool sk_run(const StackArgs &a, SkShared &sh) {
    const int K = a.K, NS = K + 1;
    const int NPF = a.F >> 4, NCH = a.D / SK_CROWS;  // combine chunks
    const int NR = a.n_router, NSB = a.shared_blocks, G = (int)gridDim.x, NWB = G - NR - NSB;
    const int per_layer = NR + NCH + NS * NPF;
    const int b = blockIdx.x;
    // the shared blocks start at P = G/2, so that block b < NR shares its CU with shared
    // block b + G/2 (blocks b and b + G/2 of a two-per-CU grid are dispatched to one CU), not
    // with a routed block that computes its own digits meanwhile
    const int P = (G / 2 >= NR && G / 2 + NSB <= G) ? G / 2 : NR;
    for (int li = 0; li < a.n_layers; li++) {
        const StackLayer L = a.layers[li];
        const int layer = a.first_layer + li;
        const long base = (long)li * per_layer;
        const bool routed_on = !(a.flags & GMOE_FLAG_NO_ROUTED) && L.has_routed;
#define SK_ITEM(idx, call)                                                                    \
    do {                                                                                      \
        sh.trace_item = base + (idx);                                                         \
        if (a.trace && threadIdx.x == 0) trace_put(a.trace, SK_TRACE_STAMPS * sh.trace_item);   \
        if (!(call)) return false;                                                            \
        if (a.trace && threadIdx.x == 0) trace_put(a.trace, SK_TRACE_STAMPS * sh.trace_item + 2); \
        __syncthreads();                                                                      \
    } while (0)
        if (b < NR) {
            SK_ITEM(b, sk_router_item(a, L, layer, li, b, sh));
            // shared items past the shared blocks' share go to router blocks 1.. (block 0
            // also selects and writes the observables)
            if (b > 0)
                for (int j = NSB + b - 1; j < NPF; j += NR - 1) SK_ITEM(NR + NCH + j, sk_expert_item<false>(a, L, li, K, j, a.E, sh));
        } else if (b >= P && b < P + NSB) {
            const int sb = b - P;
            for (int j = sb; j < NPF; j += NSB) {
                if (j >= NSB && NR > 1) break;  // the router blocks' share
                SK_ITEM(NR + NCH + j, sk_expert_item<false>(a, L, li, K, j, a.E, sh));
            }
            sh.trace_item = base + NR + NCH + sb;
            if (!wait_ge(&a.ctr[SKF(li, SKF_X)], 1u, a.error, sh)) return false;
        } else {
            const int wb = b < P ? b - NR : b - NR - NSB;
            if (wb < K * NPF && routed_on) {
                sh.trace_item = base + NR + NCH + NPF + wb;  // stamps 1, 8 and 3 of its first item
                if (a.D == GM_MAX_COLS && !sk_local_digits(a, L, li, sh)) return false;
                if (!sk_stage_select(a, li, false, sh)) return false;
                if (!sh.sel_ok && !sk_read_topk(a, li, sh)) return false;
            }
            for (int i = wb; i < K * NPF; i += NWB) {
                const int slot = i / NPF;
                SK_ITEM(NR + NCH + NPF + i, sk_expert_item<true>(a, L, li, slot, i % NPF, routed_on ? sh.idx[slot] : -1, sh));
            }
            // combine chunks, by the blocks that hold this layer's routing
            const int ncb = NWB < K * NPF ? NWB : K * NPF;
            if (wb < ncb && wb < NCH) {
                if (routed_on && !sh.sel_ok && !sk_read_weights(a, li, sh)) return false;
                for (int c = wb; c < NCH; c += ncb) SK_ITEM(NR + c, sk_combine(a, li, c, routed_on, sh));
            }
        }
#undef SK_ITEM
    }
    return true;
}

__global__ __launch_bounds__(SK_BLOCK, 2) void k_moe_stack(StackArgs a) {
    __shared__ SkShared sh;
    if (threadIdx.x == 0) {
        sh.trace = a.trace;
        sh.ok = 1;
        sh.zero = 0u;
        sh.spin_limit = a.spin_limit;
    }
    __syncthreads();
    // a block whose wait gave up leaves the launch's failure where the host reads it
    // without synchronising (the next forward call reports it)
    if (!sk_run(a, sh) && threadIdx.x == 0)
        __hip_atomic_store(a.error_host, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
