/*
 * gmoe.h -- C ABI of the MI355X MoE FFN library (libgmoe.so, built by hipcc for gfx950).
 *
 * One call of gmoe_forward() replaces one call of glm.c's
 *   apply_moe_shared_ffn_layer(rt, st, gs, layer_idx, debug_mode, pos)   (infer.c:1087-1216)
 * for a batch of T tokens whose activations already sit in device memory:
 *   xn   = rmsnorm(x, ffn_norm)                                 infer.c:1098, 746-752
 *   p    = sigmoid(gate_inp . xn)                               infer.c:1103-1107, 927-938
 *   top-k of p + exp_probs_b, weights p / sum(p)                infer.c:1110-1145
 *   acc  = sum_k 1.8 * w_k * down_k(silu(gate_k xn) * up_k xn)  infer.c:1166-1195
 *   xb   = down_sh(silu(gate_sh xn) * up_sh xn)                 infer.c:1197-1206
 *   x   += xb + acc                                             infer.c:1212-1214
 * Router top-k indices, and for T > 1 the per-expert token lists, equal the CPU
 * path's exactly; the float outputs match it to fp32-accumulation accuracy.
 *
 * The ABI uses plain pointers and sizes only. Device pointers are HIP device
 * addresses; `stream` is a hipStream_t passed as void* (NULL = default stream).
 * Every function returns 0 on success and a negative GMOE_ERR_* code on failure,
 * with a message available from gmoe_last_error(). No function calls exit().
 * A context is single-threaded: calls on one context must not overlap.
 */
#ifndef GMOE_H
#define GMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GMOE_OK 0
#define GMOE_ERR_INVALID (-1)   /* bad argument, shape or state */
#define GMOE_ERR_HIP (-2)       /* a HIP runtime call failed */
#define GMOE_ERR_NOMEM (-3)     /* device or host allocation failed */
#define GMOE_ERR_SCALE (-4)     /* a weight scale is not representable in the device format */

/* forward() flags */
#define GMOE_FLAG_NO_ROUTED 1   /* skip routed experts, as GLM_DISABLE_MOE_ROUTED=1 does (infer.c:1161-1166) */
#define GMOE_FLAG_EXACT_ROUTER 2 /* always replay glm.c's fp32 router chain (infer.c:916-938) instead of
                                    certifying the fast fp64 result: same routing, slower; for validation */

typedef struct gmoe_ctx gmoe_ctx;

/* Model shape. Field meanings follow RuntimeConfig (model.h:7-45). */
typedef struct gmoe_config {
    int32_t dim;               /* hidden size D (model.h:9); multiple of 256, <= 2048 */
    int32_t moe_ffn_dim;       /* expert intermediate F (model.h:44); multiple of 256, <= 2048 */
    int32_t n_routed_experts;  /* E (model.h:21); 1..256 */
    int32_t n_experts_used;    /* K (model.h:22); 1..8 */
    int32_t n_shared_experts;  /* S (model.h:23); 0 or 1 */
    int32_t group_size;        /* quantisation group (model.h:26): 32 for the tiled form, 16 for the
                                * tiled form with fp32 scales, a multiple of 16 dividing dim and
                                * moe_ffn_dim for the native form */
    int32_t n_layers;          /* total layers; MoE layers are 1..n_layers-1 (infer.c:1844-1845) */
    int32_t max_tokens;        /* largest n_tokens passed to the forward calls */
    float routed_scale;        /* routed expert scale, hard-coded 1.8f at infer.c:1171 */
    float norm_eps;            /* rmsnorm epsilon, 1e-5f at infer.c:750 */
    int32_t q8_form;           /* GMOE_Q8_*: how the expert matrices are kept on the device */
} gmoe_config;

/* Device form of the Q8_0 expert matrices.
 * TILED: repacked into MFMA tiles with fp16 scales; needs group_size 32 and scales that
 *   fp16 holds exactly (gmoe_upload_layer returns GMOE_ERR_SCALE otherwise). The persistent
 *   decode kernels and the grouped prefill GEMMs run on this form.
 * NATIVE: glm.c's own layout, int8 rows and fp32 scales, for any group size that is a
 *   multiple of 16 and divides dim and moe_ffn_dim (the exporter writes group size 16 and
 *   scales max|w|/127, glm47_flash_export.py:36,157-169). Every T runs the native
 *   kernels: one wave per matrix row, each group's sum scaled by its own fp32 scale.
 * TILED16: the exporter's form on the fast path: group size 16, fp32 scales kept exactly
 *   as they are, q planes tiled as in TILED. T=1 runs the persistent relay decode kernel
 *   (k_moe_relay), T>1 the grouped prefill GEMMs; gmoe_create refuses it where the shape
 *   (or GMOE_DECODE_KERNEL=0, GMOE_STACK_KERNEL=0) rules the relay kernel out.
 * AUTO (0): TILED when group_size is 32; TILED16 when it is 16 and the relay kernel runs
 *   the shape, NATIVE otherwise. */
#define GMOE_Q8_AUTO 0
#define GMOE_Q8_TILED 1
#define GMOE_Q8_NATIVE 2
#define GMOE_Q8_TILED16 3

/* Host-side weights of one MoE layer in glm.c's checkpoint layout:
 * LayerMoeShared (model.h:65-75) followed by LayerMoeRouted (model.h:77-84).
 * Q8 matrices are int8 [rows][cols] with fp32 scales [rows][cols/group_size];
 * routed tensors hold all E experts back to back (infer.c:707-739, 1177-1182). */
typedef struct gmoe_layer_weights {
    const float *ffn_norm;     /* [D] */
    const float *gate_inp;     /* [E][D] fp32 router */
    const float *exp_probs_b;  /* [E] selection bias */
    const int8_t *gate_sh_q;   /* [F][D] */
    const float *gate_sh_s;    /* [F][D/gs] */
    const int8_t *up_sh_q;     /* [F][D] */
    const float *up_sh_s;      /* [F][D/gs] */
    const int8_t *down_sh_q;   /* [D][F] */
    const float *down_sh_s;    /* [D][F/gs] */
    const int8_t *gate_q;      /* [E][F][D] */
    const float *gate_s;       /* [E][F][D/gs] */
    const int8_t *up_q;        /* [E][F][D] */
    const float *up_s;         /* [E][F][D/gs] */
    const int8_t *down_q;      /* [E][D][F] */
    const float *down_s;       /* [E][D][F/gs] */
} gmoe_layer_weights;

/* Host copies of one layer's observable intermediates, the RunState MoE fields
 * of infer.c:855-862 widened to T tokens. Any pointer may be NULL. */
typedef struct gmoe_layer_state {
    float *xn;                 /* [T][D]   rmsnorm output (RunState.xn) */
    float *router_prob;        /* [T][E]   sigmoid router probabilities (RunState.moe_router) */
    int32_t *topk_idx;         /* [T][K]   selected experts, best first (RunState.moe_topk_idx) */
    float *topk_w;             /* [T][K]   normalised weights before routed_scale (RunState.moe_topk_w) */
    float *shared_out;         /* [T][D]   shared expert output (RunState.xb after the layer) */
    float *routed_out;         /* [T][D]   weighted routed sum (RunState.moe_out_acc) */
    int32_t *expert_offsets;   /* [E+1]    per-expert token list offsets */
    int32_t *expert_tokens;    /* [T*K]    token ids per expert, ascending within each expert */
} gmoe_layer_state;

/* Counters over the life of a context. */
typedef struct gmoe_stats {
    int64_t tokens_routed;       /* token-layer routings performed */
    int64_t routing_exact_path;  /* routings that needed the exact sequential-fp32 router replay */
    int64_t routing_exact_subset; /* of those, routings replayed on the few experts that could still be chosen */
    int64_t norm_exact_path;     /* rmsnorms that needed the exact sequential-fp64 sum replay */
    int64_t scale_inexact;       /* weight scales that were not fp16-exact at upload */
    int64_t expf_libc_match;     /* 1: this process runs the glibc release that the GPU's expf exception
                                    table was measured against, so an exact router replay reproduces
                                    its expf bit for bit; 0: near-tied experts may be ordered otherwise
                                    (gmoe_create warns on stderr) */
    int64_t q8_form;             /* the device form the context keeps its experts in (GMOE_Q8_TILED,
                                    GMOE_Q8_NATIVE or GMOE_Q8_TILED16; what GMOE_Q8_AUTO resolved to) */
} gmoe_stats;

/* Create a context on HIP device `device` and reserve device memory for
 * cfg->n_layers - 1 MoE layers and cfg->max_tokens tokens. */
int gmoe_create(gmoe_ctx **out, int device, const gmoe_config *cfg);

/* Upload and repack one MoE layer (1 <= layer < n_layers) from host memory into
 * the device form (q8_form). In the tiled form scales must be fp16-representable (checked;
 * GMOE_ERR_SCALE); the tiled form at group size 16 and the native form keep them as they are. */
int gmoe_upload_layer(gmoe_ctx *ctx, int layer, const gmoe_layer_weights *w);

/* One MoE layer for n_tokens tokens: x_out = x_in + shared + routed.
 * x_in and x_out are device pointers to [n_tokens][D] fp32 and may alias. */
int gmoe_forward(gmoe_ctx *ctx, int layer, int n_tokens, const float *x_in, float *x_out,
                 int flags, void *stream);

/* Layers first_layer .. first_layer+n_layers-1 in sequence, the MoE part of the
 * decode loop at infer.c:1818-1860. Device pointers; may alias. */
int gmoe_forward_layers(gmoe_ctx *ctx, int first_layer, int n_layers, int n_tokens,
                        const float *x_in, float *x_out, int flags, void *stream);

/* gmoe_forward_layers for one token (n_tokens = 1) that allocates nothing. It has no
 * counterpart in glm.c: it is for callers that cannot allocate device memory, such as code
 * under HIP graph capture or a tight serving loop. The persistent launch keeps its
 * workspace (every layer's activations, router entries and partial sums, the counters
 * and the error word) in one fixed device array of GMOE_NOALLOC_SCRATCH_BYTES per GPU,
 * which the library holds until the process ends, instead of the context's buffers.
 * At most as many layers per call as fit in that array (at GLM-4.7-Flash's shape 16):
 * a longer run is refused with GMOE_ERR_INVALID. Trace and profile recording are
 * skipped. Every call on one GPU shares the array, so calls that overlap on one GPU
 * (other streams, threads or contexts) race; calls in order on one stream do not. A
 * timed-out launch is reported by the context's next call. Results equal
 * gmoe_forward_layers' bit for bit. */
#define GMOE_NOALLOC_SCRATCH_BYTES (64u << 20)
int gmoe_forward_layers_noalloc(gmoe_ctx *ctx, int first_layer, int n_layers, const float *x_in, float *x_out,
                                int flags, void *stream);

/* Host-memory form of gmoe_forward for callers that make no HIP calls themselves,
 * such as glm.c's C host: copies x_in ([n_tokens][D] fp32, host) to the device, runs
 * the layer on the default stream, copies the result to x_out (host, may alias x_in)
 * and, when `state` is not NULL, the layer's intermediates. Synchronous. */
int gmoe_forward_host(gmoe_ctx *ctx, int layer, int n_tokens, const float *x_in, float *x_out, int flags,
                      gmoe_layer_state *state);

/* Copy the intermediates of the most recent gmoe_forward() call to host memory
 * (synchronises `stream`). expert_offsets/expert_tokens are filled for every T. */
int gmoe_read_layer_state(gmoe_ctx *ctx, gmoe_layer_state *out, void *stream);

/* Copy the top-k routing of `layer` from its most recent forward to host memory
 * ([n_tokens][K] each; either pointer may be NULL). Synchronises `stream`. */
int gmoe_read_topk(gmoe_ctx *ctx, int layer, int32_t *topk_idx, float *topk_w, void *stream);

int gmoe_get_stats(gmoe_ctx *ctx, gmoe_stats *out);

/* Per-kernel timing with HIP events recorded around every launch on the caller's
 * stream. gmoe_profile(ctx, 1) resets and starts recording, (ctx, 0) stops;
 * gmoe_profile_read synchronises and reports launches and summed milliseconds per
 * kernel of GMOE_KERNEL_*. Intended for measurement runs, not for serving. */
#define GMOE_KERNEL_ROUTER 0     /* rmsnorm + router + top-k */
#define GMOE_KERNEL_GATE_UP 1    /* gate/up products + SwiGLU */
#define GMOE_KERNEL_DOWN 2       /* down products + combine + residual */
#define GMOE_KERNEL_DISPATCH 3   /* per-expert token lists */
#define GMOE_KERNEL_STACK 4      /* persistent decode kernel (T=1, all requested layers) */
#define GMOE_KERNEL_DIGITS 5     /* prefill: activations to their int8 digit form */
#define GMOE_KERNEL_COMBINE 6    /* prefill: per-token combine + residual */
/* 7: unused (an earlier persistent decode kernel) */
#define GMOE_KERNEL_RELAY 8      /* persistent decode kernel whose phases poll each other's tagged results (T=1,
                                  * all requested layers) */
#define GMOE_KERNEL_COUNT 9
typedef struct gmoe_kernel_times {
    int64_t launches[GMOE_KERNEL_COUNT];
    double ms[GMOE_KERNEL_COUNT];
} gmoe_kernel_times;
int gmoe_profile(gmoe_ctx *ctx, int enable);
int gmoe_profile_read(gmoe_ctx *ctx, gmoe_kernel_times *out);

/* Diagnostic timeline of the persistent decode kernel. While enabled, every work
 * item of a T=1 launch records GMOE_TRACE_STAMPS 100 MHz wall-clock stamps (0 where a
 * stage does not apply): 0 picked up, 1 inputs ready (x, the expert items' completion,
 * or the combine's previous wait), 2 done, 3 top-k known, 4 h computed, 5 results
 * stored, 6 item weights and activations staged, 8 router results visible,
 * 11 norm reduced, 12 activation digits published, 13 logits done. Items of one
 * layer are numbered: n_router router items (min(E, 64) rounded down to a power of
 * two), D/16 combine chunks, F/16 shared-expert items, then K*F/16 routed items; layer
 * after layer. A routed block's per-layer top-k (stamps 8 and 3) is stamped on its
 * first item of the layer. gmoe_trace_items_read copies the most recent launch's
 * stamps ([n][GMOE_TRACE_STAMPS]) and returns n, or a negative error. Measurement
 * aid only: stamping slows the kernel slightly. */
#define GMOE_TRACE_STAMPS 32
int gmoe_trace_items(gmoe_ctx *ctx, int enable);
int64_t gmoe_trace_items_read(gmoe_ctx *ctx, uint64_t *out, int64_t max_items);

/* Self-check of the router's device expf: evaluates it on the `count` fp32 inputs whose
 * bit patterns are first_bits, first_bits + 1, ... (wrapping past 0xffffffff) into the
 * device buffer out[count]. which = 0: the libm-exact expf of the exact router replay,
 * equal to the C library's expf(x) bit for bit (infer.c:1105 calls it); which = 1: the
 * fast expf that evaluates the ends of a certified selection interval, where any result
 * within 2 ulp is sound. Asynchronous on `stream`. */
int gmoe_expf_eval(uint32_t first_bits, int64_t count, int which, float *out, void *stream);

/* Algorithmic Q8_0 bytes (34 per 32 weights) that one forward of n_tokens reads
 * for its experts, given the routing of its most recent call; used for GB/s. */
int64_t gmoe_expert_bytes_last(gmoe_ctx *ctx);

void gmoe_destroy(gmoe_ctx *ctx);

const char *gmoe_last_error(void);

#ifdef __cplusplus
}
#endif

#endif
