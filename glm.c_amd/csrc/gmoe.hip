// gmoe.hip -- C ABI of the MI355X MoE FFN library (include/gmoe.h).
//
// A decode call (T=1) is one persistent launch, k_moe_stack (stack.h), that takes
// the token through any run of layers. A batch (T>1) runs per layer:
//   k_rt_norm       grid (T/4)             rmsnorm, a wave per token (router.h; E <= 64, else k_router_tok does all three)
//   k_rt_dots       grid (T/4, 4)          router logits' sums, a thread per (token, expert, quarter of D)
//   k_rt_select     grid (T)               bounds, certified top-k, exact replay when needed
//   k_act_split     grid (rows)            xn as fp16 hi+lo planes with a per-row exponent (grouped.h)
//   k_dispatch      grid (E)               exact per-expert token lists and GEMM tiles (dispatch.h)
//   k_group_gu      grid (F/64, tiles)     grouped gate/up GEMM + SwiGLU on fp16 MFMA (grouped.h)
//   k_act_split     grid (rows)            h as fp16 hi+lo planes
//   k_group_down    grid (D/64, tiles)     grouped down GEMM, one row per (token, slot) (grouped.h)
//   k_token_combine grid (D/1024, T)       weighted combine + shared expert + residual (grouped.h)
// With GMOE_GROUPED_MIN_T above T, batches take the per-token kernels k_gate_up and
// k_down_combine (experts.h) instead. Expert weights are uploaded once per layer
// into the tiled Q8_0 layout of common.h and stay resident.
#include "gmoe.h"

#include <gnu/libc-version.h>
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <mutex>
#include <deque>
#include <vector>
#include <stdlib.h>
#include <string.h>

#include "common.h"
#include "dispatch.h"
#include "experts.h"
#include "grouped.h"
#include "native.h"
#include "relay.h"
#include "repack.h"
#include "router.h"
#include "stack.h"

static_assert(SK_TRACE_STAMPS == GMOE_TRACE_STAMPS, "trace stamps per item: kernel and ABI disagree");

// Workspace of gmoe_forward_layers_noalloc: one fixed array per GPU, held until the
// process ends, so that the call allocates nothing. In host code `scratch` is only a
// host-side stand-in for the array, not a device address: gmoe_create looks up each
// device's own address once (scratch_lookup) and launches use that address.
static __device__ __align__(256) unsigned char scratch[GMOE_NOALLOC_SCRATCH_BYTES];
#define GM_MAX_DEVICES 64
static void *g_scratch_dev[GM_MAX_DEVICES];
static std::mutex g_scratch_mu;

// The k_moe_relay instance of a shape: D == 2048 or narrower; experts per lane in its
// selection; group size 32 with fp16 scales or 16 with fp32 scales.
typedef void (*relay_fn)(StackArgs);
template <bool G16>
static relay_fn relay_kernel_g(int D, int E) {
    const bool full = D == GM_MAX_COLS;
    if (E <= 64) return full ? k_moe_relay<true, 1, G16> : k_moe_relay<false, 1, G16>;
    if (E <= 128) return full ? k_moe_relay<true, 2, G16> : k_moe_relay<false, 2, G16>;
    return full ? k_moe_relay<true, 4, G16> : k_moe_relay<false, 4, G16>;
}
static relay_fn relay_kernel(int D, int E, bool g16) { return g16 ? relay_kernel_g<true>(D, E) : relay_kernel_g<false>(D, E); }

// Router blocks of the persistent kernel: the largest power of two <= min(E, 64), so
// that every block holds at most GM_MAX_E / 64 experts.
static int stack_routers(int E) {
    int nr = 1;
    while (nr * 2 <= E && nr * 2 <= SK_NR_MAX) nr *= 2;
    return nr;
}

static thread_local char g_err[512];

static void set_err(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

// The same message slot for the library's other translation units (model.hip).
__attribute__((visibility("hidden"))) void gm_set_err(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

#define HIP_OK(expr)                                                                     \
    do {                                                                                 \
        hipError_t err_ = (expr);                                                        \
        if (err_ != hipSuccess) {                                                        \
            set_err("%s failed: %s (%s:%d)", #expr, hipGetErrorString(err_), __FILE__, __LINE__); \
            return GMOE_ERR_HIP;                                                         \
        }                                                                                \
    } while (0)


struct LayerDev {
    uint8_t *experts = nullptr;  // (E+1) * stride bytes, tiled
    float *norm = nullptr;       // [D]
    float *gate_inp = nullptr;   // [E][D]
    float *bias = nullptr;       // [E]
    double *nu = nullptr;        // [E] sum_i |gate_inp[e][i]| (|ffn_norm[i]| + 1), for the router records' bound
    int has_routed = 0;
    int uploaded = 0;
    int last_T = 0;
};

struct ProfRecord {
    hipEvent_t start = nullptr, stop = nullptr;
    int kernel = 0;
};

struct gmoe_ctx {
    int device = 0;
    int prof_on = 0;
    size_t prof_used = 0;
    std::deque<ProfRecord> prof;  // a deque: records stay where they are while later ones are added
    gmoe_config cfg{};
    int D = 0, F = 0, E = 0, K = 0, S = 0, L = 0, Tmax = 0;
    size_t stride = 0, off_gq = 0, off_uq = 0, off_dq = 0, off_gs = 0, off_us = 0, off_ds = 0;
    LayerDev *layers = nullptr;

    float *xn = nullptr, *router_prob = nullptr, *topk_w = nullptr, *topk_ws = nullptr;
    double *rt_t = nullptr, *rt_sp = nullptr;  // the batch router's quarter sums [T][4][E] (E <= 64)
    float *rt_sa = nullptr;
    float *h = nullptr, *y = nullptr, *shared_out = nullptr, *routed_out = nullptr;
    double2 *stage = nullptr;
    int *topk_idx = nullptr;
    unsigned *tok_counter = nullptr, *panel_counter = nullptr;
    int *offsets = nullptr, *tokens = nullptr, *slots = nullptr;
    // prefill grouped GEMMs (grouped.h): list rows are [Tmax*K routed pairs][Tmax shared]
    __half *xspl = nullptr, *hspl = nullptr;
    int *xexp = nullptr, *hexp = nullptr, *pair_row = nullptr, *n_tiles = nullptr;
    float *hbuf = nullptr, *ybuf = nullptr;
    GpTile *tiles = nullptr;
    int max_tiles = 0;
    int *hist_idx = nullptr;
    float *hist_w = nullptr;
    unsigned long long *stats_dev = nullptr;
    float *x_host_io = nullptr;  // [T][D] device copy of gmoe_forward_host's activations

    // persistent decode kernel (stack.h)
    int grouped_min_t = 2;       // T from which batches take the grouped GEMMs (GMOE_GROUPED_MIN_T)
    int stack_ok = 0;            // shape fits k_moe_stack
    int stack_grid = 0;          // co-resident blocks
    int relay = 0;               // T=1 runs k_moe_relay (relay.h) rather than k_moe_stack
    int coop = 0;                // the persistent kernels go out as cooperative launches (GMOE_COOPERATIVE=1)
    unsigned long long *sk_par_dev = nullptr;  // k_moe_relay: its workspace layers' parities (StackArgs::par_dev)
    int native = 0;              // GMOE_Q8_NATIVE: checkpoint layout, fp32 scales, native.h kernels
    int g16 = 0;                 // GMOE_Q8_TILED16: tiled q planes, fp32 scales per 16 columns
    uint8_t *sk_ws = nullptr;    // per-layer workspace, L regions of sk_ws_layer bytes
    size_t sk_ws_layer = 0;
    StackWs sk_o{};
    unsigned *sk_ctr = nullptr;  // [GM_STACK_COUNTERS]
    int *sk_error = nullptr;
    int *sk_error_host = nullptr;      // pinned host word a failing launch sets (hipHostMalloc)
    // The host-visible outputs (x for the host-buffer forward, xn, shared_out, routed_out,
    // router_prob, topk_w, topk_idx: the pointers above are slices of it, in this order)
    // in one device block, and its pinned host image: gmoe_forward_host moves a layer's
    // input and all of its outputs with one copy each way.
    uint8_t *obs = nullptr, *obs_host = nullptr;
    size_t obs_bytes = 0;
    float *obs_pack = nullptr;  // a T-token call's parts of obs back to back, and the launch's error word
    int *sk_error_host_dev = nullptr;  // its device address
    unsigned sk_spin_limit = SK_SPIN_LIMIT;
    StackLayer *sk_layers = nullptr;  // [L], device
    unsigned long long *sk_trace = nullptr;  // per-item timestamps when tracing
    size_t sk_trace_items = 0;
    int sk_trace_on = 0;
    long long sk_trace_last = 0;  // items of the most recent traced launch

    uint8_t *staging = nullptr;
    size_t staging_bytes = 0;

    long long tokens_routed = 0;
    long long scale_inexact = 0;
    int expf_libc_match = 0;  // the running glibc is GM_EXPF_LIBC (expf_exact.h's table)
    int last_layer = -1, last_T = 0, last_flags = 0, last_dispatched = 0, stack_launched = 0;
    int stack_last = 0;  // the most recent forward was a persistent launch
    int *stack_error_dev = nullptr;  // the device error word that launch used
};

extern "C" const char *gmoe_last_error(void) { return g_err; }

// The device address of `scratch` on `device` (current), looked up once per device.
static int scratch_lookup(int device) {
    if (device < 0 || device >= GM_MAX_DEVICES) {
        set_err("device %d: at most %d devices are supported", device, GM_MAX_DEVICES);
        return GMOE_ERR_INVALID;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_dev[device]) return GMOE_OK;
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        set_err("hipGetSymbolAddress(scratch) on device %d failed: %s", device, hipGetErrorString(e));
        return GMOE_ERR_HIP;
    }
    g_scratch_dev[device] = p;
    return GMOE_OK;
}

template <typename T>
static int dev_alloc(T **p, size_t count) {
    *p = nullptr;
    if (count == 0) count = 1;
    hipError_t e = hipMalloc((void **)p, count * sizeof(T));
    if (e != hipSuccess) {
        set_err("hipMalloc of %zu bytes failed: %s", count * sizeof(T), hipGetErrorString(e));
        *p = nullptr;
        return GMOE_ERR_NOMEM;
    }
    return GMOE_OK;
}

static void dev_free(void *p) {
    if (p) (void)hipFree(p);
}

static void free_ctx(gmoe_ctx *c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    for (ProfRecord &r : c->prof) {
        if (r.start) (void)hipEventDestroy(r.start);
        if (r.stop) (void)hipEventDestroy(r.stop);
    }
    if (c->layers) {
        for (int l = 0; l < c->L; l++) {
            dev_free(c->layers[l].experts);
            dev_free(c->layers[l].norm);
            dev_free(c->layers[l].gate_inp);
            dev_free(c->layers[l].bias);
            dev_free(c->layers[l].nu);
        }
        delete[] c->layers;
    }
    void *bufs[] = {c->obs, c->obs_pack, c->topk_ws, c->h, c->y,
                    c->stage, c->tok_counter, c->panel_counter, c->offsets, c->tokens, c->slots, c->hist_idx, c->hist_w,
                    c->stats_dev, c->staging, c->sk_ws, c->sk_ctr, c->sk_error, c->sk_par_dev,
                    c->sk_layers, c->sk_trace, c->xspl, c->hspl, c->xexp, c->hexp, c->pair_row, c->n_tiles,
                    c->hbuf, c->ybuf, c->tiles, c->rt_t, c->rt_sp, c->rt_sa};
    for (void *b : bufs) dev_free(b);
    if (c->sk_error_host) (void)hipHostFree(c->sk_error_host);
    if (c->obs_host) (void)hipHostFree(c->obs_host);
    delete c;
}

extern "C" int gmoe_create(gmoe_ctx **out, int device, const gmoe_config *cfg) {
    if (!out || !cfg) {
        set_err("gmoe_create: null argument");
        return GMOE_ERR_INVALID;
    }
    *out = nullptr;
    const gmoe_config &g = *cfg;
    // Each of a block's 4 waves holds an equal share of a row's 64-column chunks in
    // registers (at most 8): dim and moe_ffn_dim are multiples of 256, at most 2048.
    if (g.dim <= 0 || g.dim % 256 || g.dim > GM_MAX_COLS || g.moe_ffn_dim <= 0 || g.moe_ffn_dim % 256 ||
        g.moe_ffn_dim > GM_MAX_COLS) {
        set_err("gmoe_create: dim and moe_ffn_dim must be positive multiples of 256 and <= %d (got %d, %d)",
                GM_MAX_COLS, g.dim, g.moe_ffn_dim);
        return GMOE_ERR_INVALID;
    }
    if (g.n_routed_experts < 1 || g.n_routed_experts > GM_MAX_E || g.n_experts_used < 1 ||
        g.n_experts_used > GM_MAX_K) {
        set_err("gmoe_create: need 1 <= n_routed_experts <= %d and 1 <= n_experts_used <= %d (got %d, %d)",
                GM_MAX_E, GM_MAX_K, g.n_routed_experts, g.n_experts_used);
        return GMOE_ERR_INVALID;
    }
    if (g.n_shared_experts != 1) {
        set_err("gmoe_create: glm.c always runs exactly one shared expert (infer.c:1197); got %d",
                g.n_shared_experts);
        return GMOE_ERR_INVALID;
    }
    if (g.q8_form != GMOE_Q8_AUTO && g.q8_form != GMOE_Q8_TILED && g.q8_form != GMOE_Q8_NATIVE &&
        g.q8_form != GMOE_Q8_TILED16) {
        set_err("gmoe_create: q8_form %d is not a GMOE_Q8_* value", g.q8_form);
        return GMOE_ERR_INVALID;
    }
    // group size 16 (the exporter's) goes to the tiled form with fp32 scales where the shape
    // runs on k_moe_relay (decided below), else to the native form
    bool g16 = g.q8_form == GMOE_Q8_TILED16 || (g.q8_form == GMOE_Q8_AUTO && g.group_size == 16);
    bool native = g.q8_form == GMOE_Q8_NATIVE || (g.q8_form == GMOE_Q8_AUTO && g.group_size != GM_QBLOCK && !g16);
    if (g.q8_form == GMOE_Q8_TILED16 && g.group_size != 16) {
        set_err("gmoe_create: GMOE_Q8_TILED16 needs group_size 16 (got %d)", g.group_size);
        return GMOE_ERR_INVALID;
    }
    if (!native && !g16 && g.group_size != GM_QBLOCK) {
        set_err("gmoe_create: the tiled form needs group_size %d (got %d); GMOE_Q8_NATIVE takes other sizes",
                GM_QBLOCK, g.group_size);
        return GMOE_ERR_INVALID;
    }
    if (native && (g.group_size < 16 || g.group_size % 16 || g.dim % g.group_size || g.moe_ffn_dim % g.group_size)) {
        set_err("gmoe_create: the native form needs a group_size that is a multiple of 16 and divides dim and "
                "moe_ffn_dim (got %d)", g.group_size);
        return GMOE_ERR_INVALID;
    }
    if (g.n_layers < 2 || g.max_tokens < 1 || g.max_tokens > 65535) {
        set_err("gmoe_create: need n_layers >= 2 and 1 <= max_tokens <= 65535 (got %d, %d)", g.n_layers,
                g.max_tokens);
        return GMOE_ERR_INVALID;
    }
    int ndev = 0;
    HIP_OK(hipGetDeviceCount(&ndev));
    if (device < 0 || device >= ndev) {
        set_err("gmoe_create: device %d out of range (%d devices)", device, ndev);
        return GMOE_ERR_INVALID;
    }
    HIP_OK(hipSetDevice(device));
    if (int src = scratch_lookup(device)) return src;

    gmoe_ctx *c = new gmoe_ctx();
    c->device = device;
    // the exact router replay reproduces the expf of the glibc its exception table was
    // measured against (expf_exact.h); glm.c on this host calls this process's glibc
    c->expf_libc_match = strcmp(gnu_get_libc_version(), GM_EXPF_LIBC) == 0;
    if (!c->expf_libc_match)
        fprintf(stderr,
                "[gmoe] warning: the GPU's expf table was measured against glibc %s but this process runs glibc %s; "
                "an exact router replay may order near-tied experts unlike this host's libm\n",
                GM_EXPF_LIBC, gnu_get_libc_version());
    c->cfg = g;
    c->D = g.dim;
    c->F = g.moe_ffn_dim;
    c->E = g.n_routed_experts;
    c->K = g.n_experts_used;
    c->S = g.n_shared_experts;
    c->L = g.n_layers;
    c->Tmax = g.max_tokens;
    const size_t qb = (size_t)c->F * c->D;  // bytes of one q plane
    const size_t sb = qb / GM_QBLOCK * 2;   // bytes of one fp16 s plane
    c->off_gq = 0;
    c->off_uq = qb;
    c->off_dq = 2 * qb;
    c->off_gs = 3 * qb;
    c->off_us = 3 * qb + sb;
    c->off_ds = 3 * qb + 2 * sb;
    c->stride = (3 * qb + 3 * sb + 255) & ~(size_t)255;
    if (native || g16) {
        // native: glm.c's layout per expert, gate, up, down int8 rows, then their fp32 scales;
        // group size 16 tiled: the tiled q planes, then fp32 scales per 16 columns
        // (gm_s16_offset, gm_ds16_offset), the same sizes
        const size_t sn = qb / (size_t)g.group_size * sizeof(float);
        c->native = native;
        c->g16 = g16;
        c->off_gs = 3 * qb;
        c->off_us = 3 * qb + sn;
        c->off_ds = 3 * qb + 2 * sn;
        c->stride = (3 * qb + 3 * sn + 255) & ~(size_t)255;
    }
    c->layers = new LayerDev[c->L];

    const size_t T = c->Tmax, D = c->D, F = c->F, E = c->E, K = c->K, NS = c->K + c->S;
    int rc = GMOE_OK;
    {
        // obs: x_host_io, xn, shared_out, routed_out [T][D]; router_prob [T][E]; topk_w,
        // topk_idx [T][K] -- 4-byte elements, in this order (obs_slice)
        c->obs_bytes = (4 * T * D + T * E + 2 * T * K + 1) * sizeof(float);
        rc |= dev_alloc(&c->obs, c->obs_bytes);
        rc |= dev_alloc(&c->obs_pack, c->obs_bytes / sizeof(float));
        if (!rc && hipHostMalloc((void **)&c->obs_host, c->obs_bytes, hipHostMallocDefault) != hipSuccess) {
            c->obs_host = nullptr;
            set_err("hipHostMalloc of %zu bytes failed", c->obs_bytes);
            rc |= GMOE_ERR_NOMEM;
        }
        if (!rc) {
            float *o = (float *)c->obs;
            c->x_host_io = o;
            c->xn = o + T * D;
            c->shared_out = o + 2 * T * D;
            c->routed_out = o + 3 * T * D;
            c->router_prob = o + 4 * T * D;
            c->topk_w = c->router_prob + T * E;
            c->topk_idx = (int *)(c->topk_w + T * K);
        }
    }
    if (E <= 64) {
        rc |= dev_alloc(&c->rt_t, T * 4 * E);
        rc |= dev_alloc(&c->rt_sp, T * 4 * E);
        rc |= dev_alloc(&c->rt_sa, T * 4 * E);
    }
    rc |= dev_alloc(&c->topk_ws, T * K);
    rc |= dev_alloc(&c->h, T * NS * F);
    rc |= dev_alloc(&c->y, T * NS * D);
    rc |= dev_alloc(&c->stage, T * E);
    rc |= dev_alloc(&c->tok_counter, T);
    rc |= dev_alloc(&c->panel_counter, T * (D / 16));
    rc |= dev_alloc(&c->offsets, E + 1);
    {
        const size_t rows = T * K + T;  // list rows: routed pairs, then the shared expert's
        c->max_tiles = (int)(E + (T * K + GP_TOK - 1) / GP_TOK + (T + GP_TOK - 1) / GP_TOK);
        rc |= dev_alloc(&c->xspl, T * 2 * D);
        rc |= dev_alloc(&c->xexp, T);
        rc |= dev_alloc(&c->hbuf, rows * F);
        rc |= dev_alloc(&c->hspl, rows * 2 * F);
        rc |= dev_alloc(&c->hexp, rows);
        rc |= dev_alloc(&c->ybuf, rows * D);
        rc |= dev_alloc(&c->pair_row, T * K);
        rc |= dev_alloc(&c->tiles, (size_t)c->max_tiles);
        rc |= dev_alloc(&c->n_tiles, 1);
    }
    rc |= dev_alloc(&c->tokens, T * K);
    rc |= dev_alloc(&c->slots, T * K);
    rc |= dev_alloc(&c->hist_idx, (size_t)c->L * T * K);
    rc |= dev_alloc(&c->hist_w, (size_t)c->L * T * K);
    rc |= dev_alloc(&c->stats_dev, GM_STAT_COUNT);
    // The persistent decode kernels hold one panel's chunks per wave in registers and xn in
    // shared memory: D, F <= 2048, D a multiple of 256, at most 8 routed slots. k_moe_stack
    // stages a combine chunk's partials, F/16 x (K+1) x 8 floats, in the slice buffer.
    c->stack_ok = !c->native && c->L <= SK_MAX_LAYERS &&
                  (size_t)(F / 16) * (K + 1) * SK_CROWS * sizeof(float) <= sizeof(SkShared::dslice);
    if (const char *g_env = getenv("GMOE_GROUPED_MIN_T")) c->grouped_min_t = atoi(g_env) > 1 ? atoi(g_env) : 2;
    const char *env = getenv("GMOE_STACK_KERNEL");
    if (env && env[0] == '0') c->stack_ok = 0;
    if (c->stack_ok) {
        int per_cu = 0, cus = 0;
        hipDeviceProp_t prop;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_moe_stack, SK_BLOCK, 0) != hipSuccess ||
            hipGetDeviceProperties(&prop, device) != hipSuccess || per_cu < 1) {
            c->stack_ok = 0;
        } else {
            cus = prop.multiProcessorCount;
            const int want = per_cu < 2 ? per_cu : 2;  // 2 blocks (8 waves) per CU
            c->stack_grid = want * cus;
            // roles: the router blocks, at least one shared-expert and one routed block
            if (c->stack_grid < stack_routers(c->E) + 2) c->stack_ok = 0;
            const char *dk_env = getenv("GMOE_DECODE_KERNEL");
            // k_moe_relay is the default where the shape fits it; GMOE_DECODE_KERNEL=0 asks for
            // k_moe_stack
            int per_cu_rl = 0;
            c->relay = c->stack_ok && !(dk_env && dk_env[0] == '0') &&
                       hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu_rl, relay_kernel(c->D, c->E, c->g16), SK_BLOCK, 0) ==
                           hipSuccess &&
                       per_cu_rl >= want && rl_fits(c->stack_grid, c->D, c->F, c->E, c->K);
            int coop_ok = 0;
            const char *co_env = getenv("GMOE_COOPERATIVE");
            // opt-in: a cooperative launch costs ~18 us per launch on MI355X (2 % of a 46-layer
            // decode step, far more on one-layer launches)
            c->coop = c->stack_ok && co_env && co_env[0] == '1' &&
                      hipDeviceGetAttribute(&coop_ok, hipDeviceAttributeCooperativeLaunch, device) == hipSuccess && coop_ok;
        }
    }
    if (c->g16) {
        // the group-size-16 tiled form runs on k_moe_relay at T=1 and on the grouped GEMMs
        // at T>1 only (k_moe_stack and the per-token kernels take fp16 scales per 32 columns)
        c->grouped_min_t = 2;
        if (!c->relay) {
            if (g.q8_form == GMOE_Q8_TILED16) {
                set_err("gmoe_create: GMOE_Q8_TILED16 runs on k_moe_relay, which this shape or GMOE_DECODE_KERNEL=0 / "
                        "GMOE_STACK_KERNEL=0 rules out; GMOE_Q8_NATIVE takes it");
                free_ctx(c);
                return GMOE_ERR_INVALID;
            }
            c->g16 = 0;  // same offsets and sizes as the native form at group size 16
            c->native = 1;
            c->stack_ok = 0;
            c->coop = 0;
        }
    }
    {
        // per-layer regions of the persistent kernel, each buffer on its own 256-byte lines
        size_t off = 0;
        auto take = [&](size_t bytes) {
            const size_t at = off;
            off += (bytes + 255) & ~(size_t)255;
            return at;
        };
        c->sk_o.x = take(D * sizeof(float));
        c->sk_o.xn = take(D * sizeof(float));
        c->sk_o.dig = take(3 * D);
        c->sk_o.dexp = take(D / 32 * sizeof(int));
        c->sk_o.stage = take(SK_STAGE_COPIES * SK_STAGE_COPY_WORDS * sizeof(unsigned long long));
        c->sk_o.ex_w = take(K * sizeof(float));
        // the expert items' partial sums
        c->sk_o.ypart = take(NS * (F / 16) * D * sizeof(float));
        // k_moe_relay's router records, one per chunk of RL_ROWS rows and expert
        const size_t rec_pieces = c->relay ? D / RL_ROWS : 0;
        c->sk_o.rec = take(rec_pieces * E * sizeof(RlRec));
        c->sk_o.xsq = take(rec_pieces * sizeof(double));
        c->sk_ws_layer = off;
        rc |= dev_alloc(&c->sk_ws, (size_t)c->L * off);
    }
    rc |= dev_alloc(&c->sk_par_dev, SK_MAX_LAYERS / 64);
    rc |= dev_alloc(&c->sk_ctr, GM_STACK_COUNTERS);
    rc |= dev_alloc(&c->sk_error, 1);
    rc |= dev_alloc(&c->sk_layers, (size_t)c->L);
    if (rc == GMOE_OK) {
        if (hipHostMalloc((void **)&c->sk_error_host, sizeof(int), hipHostMallocDefault) != hipSuccess ||
            hipHostGetDevicePointer((void **)&c->sk_error_host_dev, c->sk_error_host, 0) != hipSuccess) {
            set_err("gmoe_create: pinned host memory for the launch status failed");
            rc = GMOE_ERR_NOMEM;
        } else {
            *(volatile int *)c->sk_error_host = 0;
        }
    }
    if (rc != GMOE_OK) {
        free_ctx(c);
        return GMOE_ERR_NOMEM;
    }
    // Diagnostic: a lower poll limit for the persistent kernel's waits (tests force a
    // timed-out launch with it; every wait still ends, the kernel exits normally).
    if (const char *sl = getenv("GMOE_SPIN_LIMIT")) c->sk_spin_limit = (unsigned)strtoul(sl, nullptr, 10);
    // Counters start at zero; each kernel's last block puts its counter back to zero.
    hipError_t e0 = hipMemset(c->tok_counter, 0, T * sizeof(unsigned));
    hipError_t e1 = hipMemset(c->panel_counter, 0, T * (D / 16) * sizeof(unsigned));
    hipError_t e3 = hipMemset(c->stats_dev, 0, GM_STAT_COUNT * sizeof(unsigned long long));
    hipError_t e4 = hipMemset(c->hist_idx, 0xff, (size_t)c->L * T * K * sizeof(int));
    hipError_t e6 = hipMemset(c->sk_error, 0, sizeof(int));
    hipError_t e7 = hipMemset(c->sk_layers, 0, (size_t)c->L * sizeof(StackLayer));
    if (!e7) e7 = hipMemset(c->sk_ws, 0, (size_t)c->L * c->sk_ws_layer);
    if (!e7) e7 = hipMemset(c->sk_par_dev, 0, SK_MAX_LAYERS / 64 * sizeof(unsigned long long));
    hipError_t e5 = hipDeviceSynchronize();
    if (e0 || e1 || e3 || e4 || e5 || e6 || e7) {
        set_err("gmoe_create: initialising device buffers failed");
        free_ctx(c);
        return GMOE_ERR_HIP;
    }
    *out = c;
    return GMOE_OK;
}

extern "C" void gmoe_destroy(gmoe_ctx *ctx) { free_ctx(ctx); }

static int copy_in(void *dst, const void *src, size_t bytes) {
    HIP_OK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return GMOE_OK;
}

// Upload n_mat raw matrices (rows x cols int8 + fp32 scales) and repack them to
// dst + m*dst_stride (+off_q for q, +off_s for scales).
static void repack_staged(gmoe_ctx *c, int n_mat, int rows, int cols, uint8_t *dst, size_t dst_stride, size_t off_q,
                          size_t off_s, int layout, unsigned long long *inexact_dev) {
    const size_t qbytes = (size_t)n_mat * rows * cols;
    const size_t units = qbytes / 16;
    hipLaunchKernelGGL(k_repack_q, dim3((unsigned)((units + 255) / 256)), dim3(256), 0, 0,
                       (const int8_t *)c->staging, dst + off_q, dst_stride, rows, cols, n_mat, layout);
    if (c->g16) {
        const size_t ns = (size_t)n_mat * rows * (cols / 16);
        hipLaunchKernelGGL(k_repack_s16, dim3((unsigned)((ns + 255) / 256)), dim3(256), 0, 0,
                           (const float *)(c->staging + qbytes), dst + off_s, dst_stride, rows, cols, n_mat, layout);
        return;
    }
    const size_t ns = (size_t)n_mat * rows * (cols / GM_QBLOCK);
    hipLaunchKernelGGL(k_repack_s, dim3((unsigned)((ns + 255) / 256)), dim3(256), 0, 0,
                       (const float *)(c->staging + qbytes), dst + off_s, dst_stride, rows, cols, n_mat, layout,
                       inexact_dev);
}

// Copies n_mat matrices to the staging buffer and repacks them into `layout`; with
// layout2 >= 0 also into layout2 at off_q2 / off_s2 (scales counted once).
static int upload_matrices(gmoe_ctx *c, const int8_t *q, const float *s, int n_mat, int rows, int cols, uint8_t *dst,
                           size_t dst_stride, size_t off_q, size_t off_s, int layout, unsigned long long *inexact_dev) {
    const size_t qbytes = (size_t)n_mat * rows * cols;
    const size_t sbytes = (size_t)n_mat * rows * (cols / (c->g16 ? 16 : GM_QBLOCK)) * sizeof(float);
    if (qbytes + sbytes > c->staging_bytes) {
        dev_free(c->staging);
        c->staging = nullptr;
        c->staging_bytes = 0;
        if (dev_alloc(&c->staging, qbytes + sbytes) != GMOE_OK) return GMOE_ERR_NOMEM;
        c->staging_bytes = qbytes + sbytes;
    }
    int rc = copy_in(c->staging, q, qbytes);
    if (rc) return rc;
    rc = copy_in(c->staging + qbytes, s, sbytes);
    if (rc) return rc;
    repack_staged(c, n_mat, rows, cols, dst, dst_stride, off_q, off_s, layout, inexact_dev);
    HIP_OK(hipGetLastError());
    HIP_OK(hipDeviceSynchronize());
    return GMOE_OK;
}

extern "C" int gmoe_upload_layer(gmoe_ctx *c, int layer, const gmoe_layer_weights *w) {
    if (!c || !w) {
        set_err("gmoe_upload_layer: null argument");
        return GMOE_ERR_INVALID;
    }
    if (layer < 1 || layer >= c->L) {
        set_err("gmoe_upload_layer: layer %d outside the MoE layers 1..%d", layer, c->L - 1);
        return GMOE_ERR_INVALID;
    }
    if (!w->ffn_norm || !w->gate_inp || !w->exp_probs_b || !w->gate_sh_q || !w->gate_sh_s || !w->up_sh_q ||
        !w->up_sh_s || !w->down_sh_q || !w->down_sh_s) {
        set_err("gmoe_upload_layer: layer %d lacks its norm, router or shared expert", layer);
        return GMOE_ERR_INVALID;
    }
    const int has_routed = w->gate_q && w->gate_s && w->up_q && w->up_s && w->down_q && w->down_s;
    HIP_OK(hipSetDevice(c->device));
    LayerDev &L = c->layers[layer];
    L.uploaded = 0;
    const int D = c->D, F = c->F, E = c->E;
    if (!L.experts && dev_alloc(&L.experts, (size_t)(E + 1) * c->stride) != GMOE_OK) return GMOE_ERR_NOMEM;
    if (!L.norm && dev_alloc(&L.norm, (size_t)D) != GMOE_OK) return GMOE_ERR_NOMEM;
    if (!L.gate_inp && dev_alloc(&L.gate_inp, (size_t)E * D) != GMOE_OK) return GMOE_ERR_NOMEM;
    if (!L.bias && dev_alloc(&L.bias, (size_t)E) != GMOE_OK) return GMOE_ERR_NOMEM;
    if (!L.nu && dev_alloc(&L.nu, (size_t)E) != GMOE_OK) return GMOE_ERR_NOMEM;
    int rc;
    if ((rc = copy_in(L.norm, w->ffn_norm, (size_t)D * sizeof(float)))) return rc;
    if ((rc = copy_in(L.gate_inp, w->gate_inp, (size_t)E * D * sizeof(float)))) return rc;
    if ((rc = copy_in(L.bias, w->exp_probs_b, (size_t)E * sizeof(float)))) return rc;
    {
        // nu_e = sum_i |gate_inp[e][i]| (|ffn_norm[i]| + 1), rounded up: bounds what underflow in
        // xn's two fp32 roundings can add to expert e's router logit (relay.h)
        std::vector<double> nu((size_t)E);
        for (int e = 0; e < E; e++) {
            double s = 0.0;
            for (int i = 0; i < D; i++) s += fabs((double)w->gate_inp[(size_t)e * D + i]) * (fabs((double)w->ffn_norm[i]) + 1.0);
            nu[(size_t)e] = s * (1.0 + 0x1p-40);
        }
        if ((rc = copy_in(L.nu, nu.data(), (size_t)E * sizeof(double)))) return rc;
    }

    unsigned long long *inexact = nullptr;
    if (dev_alloc(&inexact, 1) != GMOE_OK) return GMOE_ERR_NOMEM;
    HIP_OK(hipMemset(inexact, 0, sizeof(unsigned long long)));
    uint8_t *sh = L.experts + (size_t)E * c->stride;
    if (c->native) {
        // the checkpoint's matrices and scales as they are, one expert per stride
        const int gs = c->cfg.group_size;
        const size_t qb = (size_t)F * D, sn = qb / gs * sizeof(float);
        struct {
            const void *src;
            size_t off, bytes;
            int n;
            uint8_t *dst;
        } parts[] = {{w->gate_sh_q, c->off_gq, qb, 1, sh},         {w->up_sh_q, c->off_uq, qb, 1, sh},
                     {w->down_sh_q, c->off_dq, qb, 1, sh},         {w->gate_sh_s, c->off_gs, sn, 1, sh},
                     {w->up_sh_s, c->off_us, sn, 1, sh},           {w->down_sh_s, c->off_ds, sn, 1, sh},
                     {w->gate_q, c->off_gq, qb, E, L.experts},     {w->up_q, c->off_uq, qb, E, L.experts},
                     {w->down_q, c->off_dq, qb, E, L.experts},     {w->gate_s, c->off_gs, sn, E, L.experts},
                     {w->up_s, c->off_us, sn, E, L.experts},       {w->down_s, c->off_ds, sn, E, L.experts}};
        for (auto &pt : parts) {
            if (pt.n == E && !has_routed) continue;
            if (hipMemcpy2D(pt.dst + pt.off, c->stride, pt.src, pt.bytes, pt.bytes, pt.n, hipMemcpyHostToDevice) != hipSuccess) {
                set_err("gmoe_upload_layer: copy of layer %d failed", layer);
                dev_free(inexact);
                return GMOE_ERR_HIP;
            }
        }
        dev_free(inexact);
        L.uploaded = 1;
        L.has_routed = has_routed;
        return GMOE_OK;
    }
    const int P = GM_LAYOUT_PANELS, S = GM_LAYOUT_SLICES;  // gate/up in row panels, down in column slices
    rc = upload_matrices(c, w->gate_sh_q, w->gate_sh_s, 1, F, D, sh, c->stride, c->off_gq, c->off_gs, P, inexact);
    if (!rc) rc = upload_matrices(c, w->up_sh_q, w->up_sh_s, 1, F, D, sh, c->stride, c->off_uq, c->off_us, P, inexact);
    if (!rc) rc = upload_matrices(c, w->down_sh_q, w->down_sh_s, 1, D, F, sh, c->stride, c->off_dq, c->off_ds, S, inexact);
    if (has_routed) {
        uint8_t *ex = L.experts;
        if (!rc) rc = upload_matrices(c, w->gate_q, w->gate_s, E, F, D, ex, c->stride, c->off_gq, c->off_gs, P, inexact);
        if (!rc) rc = upload_matrices(c, w->up_q, w->up_s, E, F, D, ex, c->stride, c->off_uq, c->off_us, P, inexact);
        if (!rc) rc = upload_matrices(c, w->down_q, w->down_s, E, D, F, ex, c->stride, c->off_dq, c->off_ds, S, inexact);
    }
    unsigned long long n_inexact = 0;
    if (!rc && hipMemcpy(&n_inexact, inexact, sizeof(n_inexact), hipMemcpyDeviceToHost) != hipSuccess) {
        set_err("gmoe_upload_layer: reading the scale check failed");
        rc = GMOE_ERR_HIP;
    }
    dev_free(inexact);
    if (rc) return rc;
    if (n_inexact) {
        c->scale_inexact += (long long)n_inexact;
        set_err("gmoe_upload_layer: layer %d has %llu scales that fp16 cannot hold exactly", layer, n_inexact);
        return GMOE_ERR_SCALE;
    }
    L.has_routed = has_routed;
    StackLayer sl;
    sl.experts = L.experts;
    sl.norm = L.norm;
    sl.gate_inp = L.gate_inp;
    sl.bias = L.bias;
    sl.nu = L.nu;
    sl.has_routed = has_routed;
    sl.pad = 0;
    if ((rc = copy_in(c->sk_layers + layer, &sl, sizeof(sl)))) return rc;
    L.uploaded = 1;
    return GMOE_OK;
}

// Event pair around one launch when profiling is on; returns the record or null.
static ProfRecord *prof_begin(gmoe_ctx *c, hipStream_t st, int kernel) {
    if (!c->prof_on) return nullptr;
    if (c->prof_used == c->prof.size()) {
        ProfRecord r;
        if (hipEventCreate(&r.start) != hipSuccess || hipEventCreate(&r.stop) != hipSuccess) return nullptr;
        c->prof.push_back(r);
    }
    ProfRecord *r = &c->prof[c->prof_used++];
    r->kernel = kernel;
    (void)hipEventRecord(r->start, st);
    return r;
}

static void prof_end(ProfRecord *r, hipStream_t st) {
    if (r) (void)hipEventRecord(r->stop, st);
}

extern "C" int gmoe_trace_items(gmoe_ctx *c, int enable) {
    if (!c) {
        set_err("gmoe_trace_items: null context");
        return GMOE_ERR_INVALID;
    }
    c->sk_trace_on = enable ? 1 : 0;
    return GMOE_OK;
}

extern "C" int64_t gmoe_trace_items_read(gmoe_ctx *c, uint64_t *out, int64_t max_items) {
    if (!c || !out || max_items < 0) {
        set_err("gmoe_trace_items_read: bad arguments");
        return GMOE_ERR_INVALID;
    }
    if (!c->sk_trace || c->sk_trace_last == 0) return 0;
    const int64_t n = c->sk_trace_last < max_items ? c->sk_trace_last : max_items;
    HIP_OK(hipDeviceSynchronize());
    HIP_OK(hipMemcpy(out, c->sk_trace, (size_t)n * SK_TRACE_STAMPS * sizeof(uint64_t), hipMemcpyDeviceToHost));
    return n;
}

extern "C" int gmoe_profile(gmoe_ctx *c, int enable) {
    if (!c) {
        set_err("gmoe_profile: null context");
        return GMOE_ERR_INVALID;
    }
    if (enable) c->prof_used = 0;
    c->prof_on = enable ? 1 : 0;
    return GMOE_OK;
}

extern "C" int gmoe_profile_read(gmoe_ctx *c, gmoe_kernel_times *o) {
    if (!c || !o) {
        set_err("gmoe_profile_read: null argument");
        return GMOE_ERR_INVALID;
    }
    memset(o, 0, sizeof(*o));
    HIP_OK(hipSetDevice(c->device));
    for (size_t i = 0; i < c->prof_used; i++) {
        ProfRecord &r = c->prof[i];
        HIP_OK(hipEventSynchronize(r.stop));
        float ms = 0.0f;
        HIP_OK(hipEventElapsedTime(&ms, r.start, r.stop));
        if (r.kernel >= 0 && r.kernel < GMOE_KERNEL_COUNT) {
            o->launches[r.kernel]++;
            o->ms[r.kernel] += ms;
        }
    }
    return GMOE_OK;
}

static int launch_dispatch(gmoe_ctx *c, int T, int routed_on, hipStream_t st) {
    DispatchArgs da;
    da.topk_idx = c->topk_idx;
    da.T = T;
    da.K = c->K;
    da.E = c->E;
    da.offsets = c->offsets;
    da.tokens = c->tokens;
    da.slots = c->slots;
    da.TK = c->Tmax * c->K;
    da.routed_on = routed_on;
    da.shared_on = c->S > 0;
    da.tiles = c->tiles;
    da.n_tiles = c->n_tiles;
    da.pair_row = c->pair_row;
    ProfRecord *pr = prof_begin(c, st, GMOE_KERNEL_DISPATCH);
    hipLaunchKernelGGL(k_dispatch, dim3(c->E), dim3(DP_BLOCK), 0, st, da);
    prof_end(pr, st);
    HIP_OK(hipGetLastError());
    c->last_dispatched = 1;
    return GMOE_OK;
}

// Where a persistent launch keeps its workspace: the context's buffers, or the fixed
// device array of gmoe_forward_layers_noalloc.
struct StackSpace {
    uint8_t *ws;   // n_layers regions of ws_layer bytes
    unsigned *ctr; // SK_CTR_WORDS(n_layers)
    int *error;
    unsigned long long *par;  // k_moe_relay's parities (SK_MAX_LAYERS / 64 words)
};

// What launch_stack launches: the reset kernel and then the persistent kernel over
// workspace layers 0..n-1 (SP_BOTH), the reset alone (SP_RESET), or k_moe_relay alone on
// workspace layers ws_base.. that an earlier SP_RESET of at least ws_base + n layers
// prepared (SP_KERNEL).
enum StackPart { SP_BOTH, SP_RESET, SP_KERNEL };

// T=1 through layers first..first+n-1 with the persistent kernel. With `space` the launch
// uses that workspace and records neither trace nor profile (both may allocate).
static int launch_stack(gmoe_ctx *c, int first, int n, const float *x_in, float *x_out, int flags, hipStream_t st,
                        const StackSpace *space = nullptr, StackPart part = SP_BOTH, int ws_base = 0) {
    const StackSpace own = {c->sk_ws, c->sk_ctr, c->sk_error, c->sk_par_dev};
    const StackSpace &sp = space ? *space : own;
    StackArgs a;
    a.layers = c->sk_layers + first;
    a.n_layers = n;
    a.first_layer = first;
    a.x_in = x_in;
    a.x_out = x_out;
    a.D = c->D;
    a.F = c->F;
    a.E = c->E;
    a.K = c->K;
    a.flags = flags;
    a.eps = c->cfg.norm_eps;
    a.routed_scale = c->cfg.routed_scale;
    a.stride = c->stride;
    a.off_gq = c->off_gq;
    a.off_uq = c->off_uq;
    a.off_dq = c->off_dq;
    a.off_gs = c->off_gs;
    a.off_us = c->off_us;
    a.off_ds = c->off_ds;
    a.ws = sp.ws;
    a.ws_layer_bytes = c->sk_ws_layer;
    a.o = c->sk_o;
    a.xn = c->xn;
    a.topk_idx = c->topk_idx;
    a.topk_w = c->topk_w;
    a.router_prob = c->router_prob;
    a.hist_idx = c->hist_idx;
    a.hist_w = c->hist_w;
    a.hist_stride = c->Tmax * c->K;
    a.shared_out = c->shared_out;
    a.routed_out = c->routed_out;
    a.ctr = sp.ctr;
    a.stats = c->stats_dev;
    a.error = sp.error;
    a.error_host = c->sk_error_host_dev;
    a.spin_limit = c->sk_spin_limit;
    a.trace = nullptr;
    {
        // One routed block per routed item when the grid allows, the rest of the non-router
        // blocks on the shared expert (at most one per item); otherwise split in proportion.
        const int nr = stack_routers(c->E), npf = c->F / 16;
        const int avail = c->stack_grid - nr;
        int nwb = c->K * npf, nsb = avail - nwb;
        if (nsb < 1) {
            nsb = avail / (c->K + 1) > 0 ? avail / (c->K + 1) : 1;
            nwb = avail - nsb;
        }
        if (nsb > npf) nsb = npf;
        a.n_router = nr;
        a.shared_blocks = nsb;
    }
    a.par_dev = c->relay ? sp.par : nullptr;
    a.par_base = 0;
    if (part == SP_KERNEL) {
        // workspace layer ws_base on: its region, its per-layer flags (k_moe_relay uses no
        // launch-wide counter) and its parity bit
        a.ws = sp.ws + (size_t)ws_base * c->sk_ws_layer;
        a.ctr = sp.ctr + (size_t)SKF_PER_LAYER * SKC_PAD * ws_base;
        a.par_base = ws_base;
    }
    a.rl_cb0 = 0;
    a.rl_poll = 0;
    if (const char *pm = getenv("GMOE_RELAY_POLL")) a.rl_poll = atoi(pm);
    if (c->relay) {
        a.rl_cb0 = rl_roles(c->stack_grid, c->D, c->F, c->E, c->K).cb0;
        // diagnostic: another first combine block (a routed block; its chunks must stay routed)
        if (const char *cb = getenv("GMOE_RELAY_CB0")) {
            const RlRoles rr = rl_roles(c->stack_grid, c->D, c->F, c->E, c->K);
            const int v = atoi(cb);
            if (v >= 0 && v + rr.nch <= rr.nri) a.rl_cb0 = v;
        }
    }
    if (c->sk_trace_on && !space && part == SP_BOTH) {
        // k_moe_stack: its work items; k_moe_relay: routed and shared items, combine chunks
        // and finisher blocks
        const RlRoles rr = rl_roles(c->stack_grid, c->D, c->F, c->E, c->K);
        const size_t items = c->relay ? (size_t)(rr.nri + rr.nsi + rr.nch + rr.nfb) * n
                                      : (size_t)(stack_routers(c->E) + c->D / SK_CROWS + (c->K + 1) * (c->F / 16)) * n;
        if (items > c->sk_trace_items) {
            dev_free(c->sk_trace);
            c->sk_trace = nullptr;
            c->sk_trace_items = 0;
            if (dev_alloc(&c->sk_trace, SK_TRACE_STAMPS * items) != GMOE_OK) return GMOE_ERR_NOMEM;
            c->sk_trace_items = items;
        }
        a.trace = c->sk_trace;
        c->sk_trace_last = (long long)items;
        HIP_OK(hipMemsetAsync(c->sk_trace, 0, SK_TRACE_STAMPS * items * sizeof(uint64_t), st));
    }
    const int n_ctr = SK_CTR_WORDS(n);
    if (c->relay && space) {
        // the fixed array's previous user may have been another context or kernel: its
        // workspace layers and their parities start from zeros
        const size_t n16 = (size_t)n * c->sk_ws_layer / 16;
        hipLaunchKernelGGL(k_relay_zero, dim3(1024), dim3(256), 0, st, (u32x4 *)sp.ws, n16);
        hipLaunchKernelGGL(k_relay_zero, dim3(1), dim3(256), 0, st, (u32x4 *)sp.par, (size_t)(SK_MAX_LAYERS / 64 * 8 / 16));
    }
    if (part != SP_KERNEL) hipLaunchKernelGGL(k_stack_reset, dim3(n + 1), dim3(SK_BLOCK), 0, st, sp.ctr, n_ctr, sp.error, a);
    if (part == SP_RESET) {
        HIP_OK(hipGetLastError());
        return GMOE_OK;
    }
    ProfRecord *pr = space ? nullptr
                           : prof_begin(c, st, c->relay ? GMOE_KERNEL_RELAY : GMOE_KERNEL_STACK);
    {
        const void *fn = c->relay ? (const void *)relay_kernel(c->D, c->E, c->g16) : (const void *)k_moe_stack;
        // Every block waits on others' results, so the grid must be resident at once: a
        // cooperative launch has the runtime guarantee it (or refuse the launch), where an
        // ordinary one relies on the GPU being otherwise idle and the bounded waits turn a
        // grid that does not fit into a timeout error. Graph capture takes the ordinary form.
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        if (c->coop) HIP_OK(hipStreamIsCapturing(st, &cap));
        if (c->coop && cap == hipStreamCaptureStatusNone) {
            void *args[] = {&a};
            HIP_OK(hipLaunchCooperativeKernel(fn, dim3(c->stack_grid), dim3(SK_BLOCK), args, 0, st));
        } else {
            if (c->relay)
                hipLaunchKernelGGL(relay_kernel(c->D, c->E, c->g16), dim3(c->stack_grid), dim3(SK_BLOCK), 0, st, a);
            else
                hipLaunchKernelGGL(k_moe_stack, dim3(c->stack_grid), dim3(SK_BLOCK), 0, st, a);
        }
    }
    prof_end(pr, st);
    HIP_OK(hipGetLastError());
    for (int l = first; l < first + n; l++) {
        LayerDev &L = c->layers[l];
        L.last_T = 1;
    }
    c->last_layer = first + n - 1;
    c->last_T = 1;
    c->last_flags = flags;
    c->last_dispatched = 0;
    c->tokens_routed += n;
    c->stack_launched = 1;
    c->stack_last = 1;
    c->stack_error_dev = sp.error;
    return GMOE_OK;
}

static const char k_timeout_msg[] =
    "persistent decode kernel: a dependency wait timed out (grid not co-resident?); its outputs are invalid";

// Without synchronising: GMOE_ERR_HIP if a persistent launch that has already ended gave up
// on a wait since the last report (the failing block sets the pinned host word). The
// report clears the word, so the next launch starts clean.
// After a launch of k_moe_relay that gave up: words of its workspace layers may hold the
// parity of an older launch, so the context's workspace goes back to zeros, and its
// parities with it (the fixed array of the no-alloc call is cleared before each use).
static void relay_reset(gmoe_ctx *c) {
    if (!c->relay) return;
    (void)hipDeviceSynchronize();
    (void)hipMemset(c->sk_ws, 0, (size_t)c->L * c->sk_ws_layer);
    (void)hipMemset(c->sk_par_dev, 0, SK_MAX_LAYERS / 64 * sizeof(unsigned long long));
    (void)hipDeviceSynchronize();
}

static int take_launch_error(gmoe_ctx *c) {
    volatile int *w = c->sk_error_host;
    if (!c->stack_launched || !w || *w == 0) return GMOE_OK;
    *w = 0;
    relay_reset(c);
    set_err("%s", k_timeout_msg);
    return GMOE_ERR_HIP;
}

// take_launch_error for the library's other translation units (model.hip), called after
// they have synchronised the stream of their launches.
__attribute__((visibility("hidden"))) int gm_take_launch_error(gmoe_ctx *c) { return c ? take_launch_error(c) : GMOE_OK; }

// One token's MoE layers through k_moe_relay, each in a launch of its own (model.hip puts
// attention between them), with one reset kernel for all of them: the token's w-th MoE
// layer runs on workspace layer w, so its launch needs no reset of its own.
// gm_decode_begin resets n workspace layers and sets *on when the context decodes with
// k_moe_relay (else the caller takes gmoe_forward per layer); gm_decode_layer then runs
// `layer` (uploaded, 1 <= layer < L) on workspace layer w < n, as gmoe_forward(layer, T=1).
__attribute__((visibility("hidden"))) int gm_decode_begin(gmoe_ctx *c, int n, hipStream_t st, int *on) {
    *on = 0;
    if (!c || !c->relay || !c->stack_ok || c->sk_trace_on || n < 1 || n >= c->L) return GMOE_OK;
    HIP_OK(hipSetDevice(c->device));
    if (int erc = take_launch_error(c)) return erc;
    if (int rc = launch_stack(c, 1, n, nullptr, nullptr, 0, st, nullptr, SP_RESET)) return rc;
    *on = 1;
    return GMOE_OK;
}
// The device rows of the last T=1 call's shared-expert output and routed combine
// (infer.c:1206, 1192), which each launch's last layer writes.
__attribute__((visibility("hidden"))) void gm_layer_outputs(const gmoe_ctx *c, const float **shared, const float **routed) {
    *shared = c ? c->shared_out : nullptr;
    *routed = c ? c->routed_out : nullptr;
}
// Whether `layer` is an uploaded MoE layer of c (what gmoe_forward accepts).
__attribute__((visibility("hidden"))) int gm_layer_ready(const gmoe_ctx *c, int layer) {
    return c && layer >= 1 && layer < c->L && c->layers[layer].uploaded;
}
// After gm_decode_begin, a token that fails before all n of its layers ran leaves some
// workspace layers with the reset's flipped parity but none of this token's data: the next
// token's flip would make their older words look current. Back to zeros, parities included.
__attribute__((visibility("hidden"))) void gm_decode_abort(gmoe_ctx *c) {
    if (c) relay_reset(c);
}
__attribute__((visibility("hidden"))) int gm_decode_layer(gmoe_ctx *c, int layer, int w, const float *x_in, float *x_out,
                                                          int flags, hipStream_t st) {
    if (layer < 1 || layer >= c->L || !c->layers[layer].uploaded || w < 0 || w >= c->L) {
        set_err("gmoe_model: MoE layer %d (workspace %d) cannot run", layer, w);
        return GMOE_ERR_INVALID;
    }
    return launch_stack(c, layer, 1, x_in, x_out, flags, st, nullptr, SP_KERNEL, w);
}

// 0, or GMOE_ERR_HIP if the most recent persistent launch timed out (synchronises).
static int check_stack_error(gmoe_ctx *c) {
    if (!c->stack_launched) return GMOE_OK;
    int err = 0;
    HIP_OK(hipDeviceSynchronize());
    if (c->stack_last) HIP_OK(hipMemcpy(&err, c->stack_error_dev, sizeof(int), hipMemcpyDeviceToHost));
    const int host_rc = take_launch_error(c);
    if (err || host_rc) {
        if (!host_rc) relay_reset(c);
        set_err("%s", k_timeout_msg);
        return GMOE_ERR_HIP;
    }
    return GMOE_OK;
}

extern "C" int gmoe_forward(gmoe_ctx *c, int layer, int T, const float *x_in, float *x_out, int flags,
                            void *stream) {
    if (!c || !x_in || !x_out) {
        set_err("gmoe_forward: null argument");
        return GMOE_ERR_INVALID;
    }
    if (layer < 1 || layer >= c->L || !c->layers[layer].uploaded) {
        set_err("gmoe_forward: layer %d is not an uploaded MoE layer", layer);
        return GMOE_ERR_INVALID;
    }
    if (T < 1 || T > c->Tmax) {
        set_err("gmoe_forward: n_tokens %d outside 1..%d", T, c->Tmax);
        return GMOE_ERR_INVALID;
    }
    HIP_OK(hipSetDevice(c->device));
    if (int erc = take_launch_error(c)) return erc;
    hipStream_t st = (hipStream_t)stream;
    LayerDev &L = c->layers[layer];
    if (T == 1 && c->stack_ok) return launch_stack(c, layer, 1, x_in, x_out, flags, st);
    const int fl = flags | (L.has_routed ? 0 : GMOE_FLAG_NO_ROUTED);
    const int D = c->D, F = c->F, E = c->E, K = c->K, NS = c->K + c->S;

    RouterArgs ra;
    ra.x = x_in;
    ra.norm_w = L.norm;
    ra.gate_inp = L.gate_inp;
    ra.bias = L.bias;
    ra.xn = c->xn;
    ra.router_prob = c->router_prob;
    ra.topk_idx = c->topk_idx;
    ra.topk_w = c->topk_w;
    ra.topk_ws = c->topk_ws;
    ra.hist_idx = c->hist_idx + (size_t)layer * c->Tmax * K;
    ra.hist_w = c->hist_w + (size_t)layer * c->Tmax * K;
    ra.stats = c->stats_dev;
    ra.D = D;
    ra.E = E;
    ra.K = K;
    ra.eps = c->cfg.norm_eps;
    ra.routed_scale = c->cfg.routed_scale;
    ra.force_exact = (flags & GMOE_FLAG_EXACT_ROUTER) != 0;
    ProfRecord *pr = prof_begin(c, st, GMOE_KERNEL_ROUTER);
    if (E <= 64) {
        RtParts rp;
        rp.t = c->rt_t;
        rp.sp = c->rt_sp;
        rp.sa = c->rt_sa;
        hipLaunchKernelGGL(k_rt_norm, dim3((T + 3) / 4), dim3(RT_BLOCK), 0, st, ra, T);
        hipLaunchKernelGGL(k_rt_dots, dim3((T + 3) / 4, 4), dim3(RT_BLOCK), 0, st, ra, rp, T);
        hipLaunchKernelGGL(k_rt_select, dim3(T), dim3(RT_BLOCK), 0, st, ra, rp);
    } else {
        hipLaunchKernelGGL(k_router_tok, dim3(T), dim3(RT_BLOCK), 0, st, ra);
    }
    prof_end(pr, st);
    const int routed_on = !(fl & GMOE_FLAG_NO_ROUTED);
    c->last_dispatched = 0;
    if (c->native) {
        // checkpoint-layout experts (native.h): gate/up + SwiGLU, down, combine; the
        // per-expert lists for T > 1 as on the other paths
        NativeArgs na;
        na.experts = L.experts;
        na.stride = c->stride;
        na.off_gq = c->off_gq;
        na.off_uq = c->off_uq;
        na.off_dq = c->off_dq;
        na.off_gs = c->off_gs;
        na.off_us = c->off_us;
        na.off_ds = c->off_ds;
        na.D = D;
        na.F = F;
        na.E = E;
        na.K = K;
        na.S = c->S;
        na.gs = c->cfg.group_size;
        na.flags = fl;
        pr = prof_begin(c, st, GMOE_KERNEL_GATE_UP);
        hipLaunchKernelGGL(k_native_gate_up, dim3(F / 16, NS, T), dim3(NV_BLOCK), 0, st, na, (const float *)c->xn,
                           (const int *)c->topk_idx, c->h);
        prof_end(pr, st);
        pr = prof_begin(c, st, GMOE_KERNEL_DOWN);
        hipLaunchKernelGGL(k_native_down, dim3(D / 4, NS, T), dim3(NV_BLOCK), 0, st, na, (const float *)c->h,
                           (const int *)c->topk_idx, c->y);
        prof_end(pr, st);
        pr = prof_begin(c, st, GMOE_KERNEL_COMBINE);
        hipLaunchKernelGGL(k_native_combine, dim3((D + NV_BLOCK - 1) / NV_BLOCK, T), dim3(NV_BLOCK), 0, st, na,
                           (const float *)c->y, (const int *)c->topk_idx, (const float *)c->topk_ws, x_in, x_out,
                           c->shared_out, c->routed_out);
        prof_end(pr, st);
        HIP_OK(hipGetLastError());
        if (T > 1) {
            int rc = launch_dispatch(c, T, routed_on, st);
            if (rc) return rc;
        }
    } else if (T >= c->grouped_min_t) {
        // prefill: digits of xn, the per-expert lists and tiles, grouped gate/up, digits
        // of h, grouped down, per-token combine (grouped.h)
        const int TK = c->Tmax * K;
        pr = prof_begin(c, st, GMOE_KERNEL_DIGITS);
        hipLaunchKernelGGL(k_act_split, dim3(T), dim3(GP_BLOCK), 0, st, (const float *)c->xn, D, T, (const int *)nullptr,
                           c->xspl, c->xexp);
        prof_end(pr, st);
        int rc = launch_dispatch(c, T, routed_on, st);
        if (rc) return rc;
        GroupArgs ga;
        ga.experts = L.experts;
        ga.stride = c->stride;
        ga.off_gq = c->off_gq;
        ga.off_uq = c->off_uq;
        ga.off_dq = c->off_dq;
        ga.off_gs = c->off_gs;
        ga.off_us = c->off_us;
        ga.off_ds = c->off_ds;
        ga.D = D;
        ga.F = F;
        ga.E = E;
        ga.T = T;
        ga.TK = TK;
        ga.tiles = c->tiles;
        ga.n_tiles = c->n_tiles;
        ga.tokens = c->tokens;
        ga.aspl = c->xspl;
        ga.aexp = c->xexp;
        ga.out = c->hbuf;
        const int max_tiles = (routed_on ? E + (T * K + GP_TOK - 1) / GP_TOK : 0) + (T + GP_TOK - 1) / GP_TOK;
        pr = prof_begin(c, st, GMOE_KERNEL_GATE_UP);
        if (c->g16) hipLaunchKernelGGL(k_group_gu<true>, dim3(F / 64, max_tiles), dim3(GP_BLOCK), 0, st, ga);
        else hipLaunchKernelGGL(k_group_gu<false>, dim3(F / 64, max_tiles), dim3(GP_BLOCK), 0, st, ga);
        prof_end(pr, st);
        // routed rows [0, offsets[E]) and the shared rows [TK, TK + T)
        pr = prof_begin(c, st, GMOE_KERNEL_DIGITS);
        if (routed_on)
            hipLaunchKernelGGL(k_act_split, dim3(T * K), dim3(GP_BLOCK), 0, st, (const float *)c->hbuf, F, T * K,
                               (const int *)(c->offsets + E), c->hspl, c->hexp);
        hipLaunchKernelGGL(k_act_split, dim3(T), dim3(GP_BLOCK), 0, st, (const float *)(c->hbuf + (size_t)TK * F), F, T,
                           (const int *)nullptr, c->hspl + (size_t)TK * 2 * F, c->hexp + TK);
        prof_end(pr, st);
        ga.aspl = c->hspl;
        ga.aexp = c->hexp;
        ga.out = c->ybuf;
        pr = prof_begin(c, st, GMOE_KERNEL_DOWN);
        if (c->g16) hipLaunchKernelGGL(k_group_down<true>, dim3(D / 64, max_tiles), dim3(GP_BLOCK), 0, st, ga);
        else hipLaunchKernelGGL(k_group_down<false>, dim3(D / 64, max_tiles), dim3(GP_BLOCK), 0, st, ga);
        prof_end(pr, st);
        TokenCombineArgs ta;
        ta.topk_idx = c->topk_idx;
        ta.topk_ws = c->topk_ws;
        ta.pair_row = c->pair_row;
        ta.y = c->ybuf;
        ta.x_in = x_in;
        ta.x_out = x_out;
        ta.shared_out = c->shared_out;
        ta.routed_out = c->routed_out;
        ta.D = D;
        ta.K = K;
        ta.TK = TK;
        ta.routed_on = routed_on;
        pr = prof_begin(c, st, GMOE_KERNEL_COMBINE);
        const bool vec = (((uintptr_t)ta.x_in | (uintptr_t)ta.x_out) & 15) == 0;
        if (vec)
            hipLaunchKernelGGL(k_token_combine<true>, dim3((D + 4 * GP_BLOCK - 1) / (4 * GP_BLOCK), T), dim3(GP_BLOCK), 0, st, ta);
        else
            hipLaunchKernelGGL(k_token_combine<false>, dim3((D + 4 * GP_BLOCK - 1) / (4 * GP_BLOCK), T), dim3(GP_BLOCK), 0, st, ta);
        prof_end(pr, st);
        HIP_OK(hipGetLastError());
    } else {
        // one token's experts at a time: gate/up (+SwiGLU), then down with the combine
        ExpertArgs ea;
        ea.experts = L.experts;
        ea.stride = c->stride;
        ea.off_gq = c->off_gq;
        ea.off_uq = c->off_uq;
        ea.off_dq = c->off_dq;
        ea.off_gs = c->off_gs;
        ea.off_us = c->off_us;
        ea.off_ds = c->off_ds;
        ea.D = D;
        ea.F = F;
        ea.E = E;
        ea.K = K;
        ea.S = c->S;
        ea.flags = fl;
        pr = prof_begin(c, st, GMOE_KERNEL_GATE_UP);
        hipLaunchKernelGGL(k_gate_up, dim3(F / 16, NS, T), dim3(EX_BLOCK), (size_t)3 * D + (size_t)(D / 32) * 4, st, ea,
                           (const float *)c->xn, (const int *)c->topk_idx, c->h);
        prof_end(pr, st);
        CombineArgs ca;
        ca.topk_idx = c->topk_idx;
        ca.topk_ws = c->topk_ws;
        ca.y = c->y;
        ca.panel_counter = c->panel_counter;
        ca.x_in = x_in;
        ca.x_out = x_out;
        ca.shared_out = c->shared_out;
        ca.routed_out = c->routed_out;
        pr = prof_begin(c, st, GMOE_KERNEL_DOWN);
        hipLaunchKernelGGL(k_down_combine, dim3(D / 16, NS, T), dim3(EX_BLOCK), (size_t)3 * F + (size_t)(F / 32) * 4,
                           st, ea, ca, (const float *)c->h);
        prof_end(pr, st);
        HIP_OK(hipGetLastError());
        if (T > 1) {
            int rc = launch_dispatch(c, T, routed_on, st);
            if (rc) return rc;
        }
    }
    c->last_layer = layer;
    c->last_T = T;
    c->last_flags = fl;
    c->stack_last = 0;
    L.last_T = T;
    c->tokens_routed += T;
    return GMOE_OK;
}

extern "C" int gmoe_forward_layers(gmoe_ctx *c, int first, int n, int T, const float *x_in, float *x_out, int flags,
                                   void *stream) {
    if (!c || n < 1 || !x_in || !x_out) {
        set_err("gmoe_forward_layers: bad arguments");
        return GMOE_ERR_INVALID;
    }
    if (first < 1 || first + n > c->L) {
        set_err("gmoe_forward_layers: layers %d..%d outside 1..%d", first, first + n - 1, c->L - 1);
        return GMOE_ERR_INVALID;
    }
    for (int l = first; l < first + n; l++) {
        if (!c->layers[l].uploaded) {
            set_err("gmoe_forward_layers: layer %d is not uploaded", l);
            return GMOE_ERR_INVALID;
        }
    }
    if (T == 1 && c->stack_ok) {
        HIP_OK(hipSetDevice(c->device));
        if (int erc = take_launch_error(c)) return erc;
        return launch_stack(c, first, n, x_in, x_out, flags, (hipStream_t)stream);
    }
    for (int i = 0; i < n; i++) {
        int rc = gmoe_forward(c, first + i, T, i == 0 ? x_in : x_out, x_out, flags, stream);
        if (rc) return rc;
    }
    return GMOE_OK;
}

// Workspace bytes of an n-layer launch inside `scratch`: the layers' regions, the counters
// (on 256-byte lines) and the error word.
static size_t noalloc_bytes(const gmoe_ctx *c, int n) {
    const size_t ctr = ((size_t)SK_CTR_WORDS(n) * sizeof(unsigned) + 255) & ~(size_t)255;
    return (size_t)n * c->sk_ws_layer + ctr + 256 + 256;  // + the error word's line + the parities' line
}

extern "C" int gmoe_forward_layers_noalloc(gmoe_ctx *c, int first, int n, const float *x_in, float *x_out, int flags,
                                           void *stream) {
    if (!c || n < 1 || !x_in || !x_out) {
        set_err("gmoe_forward_layers_noalloc: bad arguments");
        return GMOE_ERR_INVALID;
    }
    if (!c->stack_ok) {
        set_err("gmoe_forward_layers_noalloc: this shape does not run on the persistent decode kernel");
        return GMOE_ERR_INVALID;
    }
    if (noalloc_bytes(c, n) > GMOE_NOALLOC_SCRATCH_BYTES) {
        int most = 0;
        while (noalloc_bytes(c, most + 1) <= GMOE_NOALLOC_SCRATCH_BYTES) most++;
        set_err("gmoe_forward_layers_noalloc: %d layers need %zu bytes of workspace; the fixed array holds %u, "
                "at most %d layers of this shape per call",
                n, noalloc_bytes(c, n), (unsigned)GMOE_NOALLOC_SCRATCH_BYTES, most);
        return GMOE_ERR_INVALID;
    }
    if (first < 1 || first + n > c->L) {
        set_err("gmoe_forward_layers_noalloc: layers %d..%d outside 1..%d", first, first + n - 1, c->L - 1);
        return GMOE_ERR_INVALID;
    }
    for (int l = first; l < first + n; l++) {
        if (!c->layers[l].uploaded) {
            set_err("gmoe_forward_layers_noalloc: layer %d is not uploaded", l);
            return GMOE_ERR_INVALID;
        }
    }
    HIP_OK(hipSetDevice(c->device));
    if (int erc = take_launch_error(c)) return erc;
    uint8_t *base;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        base = (uint8_t *)g_scratch_dev[c->device];  // set by gmoe_create on this device
    }
    const size_t ws_bytes = (size_t)n * c->sk_ws_layer;
    const size_t ctr_bytes = noalloc_bytes(c, n) - ws_bytes - 512;
    StackSpace sp;
    sp.ws = base;
    sp.ctr = (unsigned *)(base + ws_bytes);
    sp.error = (int *)(base + ws_bytes + ctr_bytes);
    sp.par = (unsigned long long *)(base + ws_bytes + ctr_bytes + 256);
    return launch_stack(c, first, n, x_in, x_out, flags, (hipStream_t)stream, &sp);
}

static int copy_out(void *dst, const void *src, size_t bytes) {
    if (!dst || bytes == 0) return GMOE_OK;
    HIP_OK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return GMOE_OK;
}

extern "C" int gmoe_read_layer_state(gmoe_ctx *c, gmoe_layer_state *o, void *stream);

// The first T rows of obs's seven arrays (x, xn, shared_out, routed_out [T][D]; router_prob
// [T][E]; topk_w, topk_idx [T][K]) back to back into pack, then the persistent launch's error
// word (0 without one): a T-token call's observables leave the device in one copy.
__global__ __launch_bounds__(256) void k_obs_pack(const float *__restrict__ obs, float *__restrict__ pack, int T, int TM,
                                                  int D, int E, int K, const int *__restrict__ err) {
    const size_t TD = (size_t)T * D, n = 4 * TD + (size_t)T * E + 2 * (size_t)T * K;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i <= n; i += (size_t)gridDim.x * 256) {
        if (i == n) {
            pack[n] = __int_as_float(err ? *err : 0);
            continue;
        }
        size_t src;
        if (i < 4 * TD) {
            src = (i / TD) * (size_t)TM * D + i % TD;  // array i / TD, row-major [T][D] prefix
        } else {
            const size_t j = i - 4 * TD, TE = (size_t)T * E, TK = (size_t)T * K;
            const size_t base = 4 * (size_t)TM * D;
            src = j < TE ? base + j : j < TE + TK ? base + (size_t)TM * E + (j - TE)
                                                   : base + (size_t)TM * E + (size_t)TM * K + (j - TE - TK);
        }
        pack[i] = obs[src];
    }
}

extern "C" int gmoe_forward_host(gmoe_ctx *c, int layer, int T, const float *x_in, float *x_out, int flags,
                                 gmoe_layer_state *state) {
    if (!c || !x_in || !x_out) {
        set_err("gmoe_forward_host: null argument");
        return GMOE_ERR_INVALID;
    }
    if (T < 1 || T > c->Tmax) {
        set_err("gmoe_forward_host: n_tokens %d outside 1..%d", T, c->Tmax);
        return GMOE_ERR_INVALID;
    }
    HIP_OK(hipSetDevice(c->device));
    const size_t T_ = (size_t)T, TM = (size_t)c->Tmax, D = c->D, E = c->E, K = c->K;
    const size_t bytes = T_ * D * sizeof(float);
    // in: through the pinned image, one copy
    float *h = (float *)c->obs_host;
    memcpy(h, x_in, bytes);
    HIP_OK(hipMemcpyAsync(c->x_host_io, h, bytes, hipMemcpyHostToDevice, nullptr));
    int rc = gmoe_forward(c, layer, T, c->x_host_io, c->x_host_io, flags, nullptr);
    if (rc) return rc;
    // out: x, the observables and the launch's error word packed on the device, one copy, one
    // synchronisation
    const size_t TD = T_ * D, n = 4 * TD + T_ * E + 2 * T_ * K;
    const int *err_dev = c->stack_launched && c->stack_last ? c->stack_error_dev : nullptr;
    hipLaunchKernelGGL(k_obs_pack, dim3((unsigned)std::min<size_t>((n + 256) / 256, 1024)), dim3(256), 0, nullptr,
                       (const float *)c->obs, c->obs_pack, T, (int)TM, (int)D, (int)E, (int)K, err_dev);
    HIP_OK(hipGetLastError());
    HIP_OK(hipMemcpyAsync(c->obs_host, c->obs_pack, (n + 1) * sizeof(float), hipMemcpyDeviceToHost, nullptr));
    HIP_OK(hipStreamSynchronize(nullptr));
    const float *ho = (const float *)c->obs_host;
    // a timed-out launch leaves x_out untouched, so a caller may rerun the layer from it
    const int launch_rc = take_launch_error(c);
    int err_word = 0;
    memcpy(&err_word, ho + n, sizeof(int));
    if (launch_rc || err_word) {
        if (!launch_rc) relay_reset(c);
        set_err("%s", k_timeout_msg);
        return GMOE_ERR_HIP;
    }
    memcpy(x_out, ho, bytes);
    if (!state) return GMOE_OK;
    if (state->xn) memcpy(state->xn, ho + TD, bytes);
    if (state->shared_out) memcpy(state->shared_out, ho + 2 * TD, bytes);
    if (state->routed_out) memcpy(state->routed_out, ho + 3 * TD, bytes);
    if (state->router_prob) memcpy(state->router_prob, ho + 4 * TD, T_ * E * sizeof(float));
    if (state->topk_w) memcpy(state->topk_w, ho + 4 * TD + T_ * E, T_ * K * sizeof(float));
    if (state->topk_idx) memcpy(state->topk_idx, ho + 4 * TD + T_ * E + T_ * K, T_ * K * sizeof(int));
    if (state->expert_offsets || state->expert_tokens) {
        // the per-expert lists (dispatched on demand at T=1) take the general read-back
        gmoe_layer_state lists;
        memset(&lists, 0, sizeof(lists));
        lists.expert_offsets = state->expert_offsets;
        lists.expert_tokens = state->expert_tokens;
        return gmoe_read_layer_state(c, &lists, nullptr);
    }
    return GMOE_OK;
}

extern "C" int gmoe_read_layer_state(gmoe_ctx *c, gmoe_layer_state *o, void *stream) {
    if (!c || !o) {
        set_err("gmoe_read_layer_state: null argument");
        return GMOE_ERR_INVALID;
    }
    if (c->last_layer < 0) {
        set_err("gmoe_read_layer_state: no forward has run");
        return GMOE_ERR_INVALID;
    }
    HIP_OK(hipSetDevice(c->device));
    hipStream_t st = (hipStream_t)stream;
    const size_t T = c->last_T, D = c->D, E = c->E, K = c->K;
    if (int erc = check_stack_error(c)) return erc;
    if ((o->expert_offsets || o->expert_tokens) && !c->last_dispatched) {
        int rc = launch_dispatch(c, (int)T, !(c->last_flags & GMOE_FLAG_NO_ROUTED), st);
        if (rc) return rc;
    }
    HIP_OK(hipStreamSynchronize(st));
    int rc = GMOE_OK;
    rc |= copy_out(o->xn, c->xn, T * D * sizeof(float));
    rc |= copy_out(o->router_prob, c->router_prob, T * E * sizeof(float));
    rc |= copy_out(o->topk_idx, c->topk_idx, T * K * sizeof(int));
    rc |= copy_out(o->topk_w, c->topk_w, T * K * sizeof(float));
    rc |= copy_out(o->shared_out, c->shared_out, T * D * sizeof(float));
    rc |= copy_out(o->routed_out, c->routed_out, T * D * sizeof(float));
    rc |= copy_out(o->expert_offsets, c->offsets, (E + 1) * sizeof(int));
    if (o->expert_tokens) {
        int total = 0;
        if (hipMemcpy(&total, c->offsets + E, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess) return GMOE_ERR_HIP;
        // the caller's list holds T*K entries: a total outside that is device state gone
        // wrong, reported rather than copied past the end of the caller's buffer
        if (total < 0 || (size_t)total > T * K) {
            set_err("gmoe_read_layer_state: per-expert lists hold %d entries, more than n_tokens * K = %zu", total, T * K);
            return GMOE_ERR_HIP;
        }
        rc |= copy_out(o->expert_tokens, c->tokens, (size_t)total * sizeof(int));
    }
    return rc ? GMOE_ERR_HIP : GMOE_OK;
}

extern "C" int gmoe_read_topk(gmoe_ctx *c, int layer, int32_t *idx, float *w, void *stream) {
    if (!c || layer < 1 || layer >= c->L) {
        set_err("gmoe_read_topk: bad arguments");
        return GMOE_ERR_INVALID;
    }
    HIP_OK(hipSetDevice(c->device));
    HIP_OK(hipStreamSynchronize((hipStream_t)stream));
    if (int erc = check_stack_error(c)) return erc;
    const size_t n = (size_t)c->layers[layer].last_T * c->K;
    const size_t off = (size_t)layer * c->Tmax * c->K;
    int rc = copy_out(idx, c->hist_idx + off, n * sizeof(int));
    if (!rc) rc = copy_out(w, c->hist_w + off, n * sizeof(float));
    return rc;
}

extern "C" int gmoe_get_stats(gmoe_ctx *c, gmoe_stats *o) {
    if (!c || !o) {
        set_err("gmoe_get_stats: null argument");
        return GMOE_ERR_INVALID;
    }
    HIP_OK(hipSetDevice(c->device));
    unsigned long long s[GM_STAT_COUNT] = {0};
    HIP_OK(hipDeviceSynchronize());
    if (int erc = check_stack_error(c)) return erc;
    HIP_OK(hipMemcpy(s, c->stats_dev, sizeof(s), hipMemcpyDeviceToHost));
    o->tokens_routed = c->tokens_routed;
    o->routing_exact_path = (int64_t)s[GM_STAT_ROUTE_EXACT];
    o->routing_exact_subset = (int64_t)s[GM_STAT_ROUTE_SUBSET];
    o->norm_exact_path = (int64_t)s[GM_STAT_NORM_EXACT];
    o->scale_inexact = c->scale_inexact;
    o->expf_libc_match = c->expf_libc_match;
    o->q8_form = c->g16 ? GMOE_Q8_TILED16 : c->native ? GMOE_Q8_NATIVE : GMOE_Q8_TILED;
    return GMOE_OK;
}

__global__ void k_expf_eval(uint32_t first, int64_t count, int which, float *out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) return;
    const float x = __uint_as_float(first + (uint32_t)i);
    out[i] = which == 0 ? expf_libm(x) : expf(x);
}

extern "C" int gmoe_expf_eval(uint32_t first_bits, int64_t count, int which, float *out, void *stream) {
    if (!out || count < 0 || count > ((int64_t)1 << 32) || (which != 0 && which != 1)) {
        set_err("gmoe_expf_eval: bad arguments");
        return GMOE_ERR_INVALID;
    }
    if (count == 0) return GMOE_OK;
    const int64_t blocks = (count + 255) / 256;
    hipLaunchKernelGGL(k_expf_eval, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, first_bits, count, which, out);
    HIP_OK(hipGetLastError());
    return GMOE_OK;
}

extern "C" int64_t gmoe_expert_bytes_last(gmoe_ctx *c) {
    if (!c || c->last_layer < 0) return 0;
    const size_t n = (size_t)c->last_T * c->K;
    int *idx = (int *)malloc(n * sizeof(int));
    if (!idx) return 0;
    if (hipSetDevice(c->device) != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(idx, c->topk_idx, n * sizeof(int), hipMemcpyDeviceToHost) != hipSuccess) {
        free(idx);
        return 0;
    }
    unsigned char used[GM_MAX_E] = {0};
    int n_used = 0;
    if (!(c->last_flags & GMOE_FLAG_NO_ROUTED)) {
        for (size_t i = 0; i < n; i++) {
            if (idx[i] >= 0 && idx[i] < c->E && !used[idx[i]]) {
                used[idx[i]] = 1;
                n_used++;
            }
        }
    }
    free(idx);
    const int64_t per_expert = (int64_t)3 * c->F * c->D / GM_QBLOCK * (GM_QBLOCK + 2);
    return (int64_t)(n_used + c->S) * per_expert;
}
