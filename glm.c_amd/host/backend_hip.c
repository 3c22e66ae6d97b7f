/*
 * backend_hip.c -- the --backend hip drop-in for glm.c's backend layer (backend.c).
 *
 * glm.c selects a backend once (glm_backend_init, infer.c:2174) and then runs every
 * token through glm_backend_forward_token (infer.c:2195). With BACKEND_HIP that is
 * glm_hip_forward_token (forward.c): glm.c's forward with every MoE FFN layer
 * (apply_moe_shared_ffn_layer, infer.c:1087-1216) on the GPU. A glm.c that keeps its
 * own forward can instead offload the MoE layers one at a time through
 * glm_backend_try_hip_moe, called from its layer loop (infer.c:1844-1845). Expert
 * weights are uploaded once, at init, into device memory by libgmoe.so.
 *
 * Messages use the "[glm-hip]" prefix, like backend.c's "[glm-metal]".
 * Environment:
 *   GLM_HIP_DEVICE          HIP device index (default 0)
 *   GLM_HIP_STRICT          exit(1) when a GPU layer fails instead of returning -1
 *   GLM_DISABLE_MOE_ROUTED  skip routed experts, as infer.c:1161-1166 does
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "glm_backend.h"
#include "glm_forward.h"
#include "gmoe.h"

_Static_assert(sizeof(int) == sizeof(int32_t), "RunState.moe_topk_idx is int; the ABI uses int32_t");

/* glm.c's CPU forward (infer.c:1903). Weak, so this library also loads on its own. */
int glm_cpu_forward_token(const Runtime *rt, RunState *st, int token, int pos, int debug_mode) __attribute__((weak));

static gmoe_ctx *g_ctx = NULL;
static int g_active = 0;
static gmoe_config g_cfg;  /* the context's config, kept to re-create it in the native form */
static int g_device = 0;

/* "0"/"false" (any case of the first letter, as backend.c:48-55 accepts) mean off. */
static int env_on(const char *name, int fallback) {
    const char *v = getenv(name);
    if (!v || !v[0]) return fallback;
    if (strcmp(v, "0") == 0 || strcmp(v, "false") == 0 || strcmp(v, "False") == 0 || strcmp(v, "FALSE") == 0)
        return 0;
    return 1;
}

/* infer.c:1161-1165 treats any value not starting with '0' as set. */
static int routed_disabled(void) {
    const char *v = getenv("GLM_DISABLE_MOE_ROUTED");
    return v && v[0] && v[0] != '0';
}

int glm_hip_init(const Runtime *rt, RunState *st) {
    (void)st;
    if (g_ctx) return 0;
    if (!rt) return -1;
    const RuntimeConfig *c = &rt->cfg;
    if (!rt->has_moe_shared || c->moe_ffn_dim <= 0 || c->n_layers < 2) {
        fprintf(stderr, "[glm-hip] checkpoint has no MoE layers\n");
        return -1;
    }
    gmoe_config cfg;
    memset(&cfg, 0, sizeof(cfg));
    cfg.dim = c->dim;
    cfg.moe_ffn_dim = c->moe_ffn_dim;
    cfg.n_routed_experts = c->n_routed_experts;
    cfg.n_experts_used = c->n_experts_used;
    cfg.n_shared_experts = 1; /* infer.c:1197-1206 always runs one shared expert */
    cfg.group_size = (int32_t)c->group_size;
    cfg.n_layers = c->n_layers;
    cfg.max_tokens = 1; /* the decode loop feeds one token at a time */
    cfg.routed_scale = 1.8f; /* infer.c:1171 */
    cfg.norm_eps = 1e-5f;    /* infer.c:750 */
    cfg.q8_form = GMOE_Q8_AUTO; /* tiled at group size 32, glm.c's own layout otherwise */
    const char *dev = getenv("GLM_HIP_DEVICE");
    int device = dev ? atoi(dev) : 0;
    if (gmoe_create(&g_ctx, device, &cfg) != GMOE_OK) {
        fprintf(stderr, "[glm-hip] %s\n", gmoe_last_error());
        g_ctx = NULL;
        return -1;
    }
    g_cfg = cfg;
    g_device = device;
    return 0;
}

int glm_hip_prepare(const Runtime *rt, RunState *st) {
    (void)st;
    if (!g_ctx || !rt) return -1;
    for (int l = 1; l < rt->cfg.n_layers; l++) {
        const LayerMoeShared *s = &rt->moe_layers[l];
        const LayerMoeRouted *r = (rt->has_moe_routed && rt->moe_routed_layers) ? &rt->moe_routed_layers[l] : NULL;
        if (!s->ffn_norm) continue;
        gmoe_layer_weights w;
        memset(&w, 0, sizeof(w));
        w.ffn_norm = s->ffn_norm;
        w.gate_inp = s->gate_inp;
        w.exp_probs_b = s->exp_probs_b;
        w.gate_sh_q = s->gate_sh_q;
        w.gate_sh_s = s->gate_sh_s;
        w.up_sh_q = s->up_sh_q;
        w.up_sh_s = s->up_sh_s;
        w.down_sh_q = s->down_sh_q;
        w.down_sh_s = s->down_sh_s;
        if (r) {
            w.gate_q = r->gate_q;
            w.gate_s = r->gate_s;
            w.up_q = r->up_q;
            w.up_s = r->up_s;
            w.down_q = r->down_q;
            w.down_s = r->down_s;
        }
        const int rc = gmoe_upload_layer(g_ctx, l, &w);
        if (rc == GMOE_ERR_SCALE && g_cfg.q8_form != GMOE_Q8_NATIVE) {
            /* fp32 scales that fp16 cannot hold (an exporter's max|w|/127): keep the
             * checkpoint's own layout instead, from the first layer again */
            fprintf(stderr, "[glm-hip] layer %d: %s; keeping glm.c's Q8_0 layout\n", l, gmoe_last_error());
            gmoe_destroy(g_ctx);
            g_ctx = NULL;
            g_cfg.q8_form = GMOE_Q8_NATIVE;
            if (gmoe_create(&g_ctx, g_device, &g_cfg) != GMOE_OK) {
                fprintf(stderr, "[glm-hip] %s\n", gmoe_last_error());
                g_ctx = NULL;
                return -1;
            }
            l = 0;
            continue;
        }
        if (rc != GMOE_OK) {
            fprintf(stderr, "[glm-hip] upload of layer %d failed: %s\n", l, gmoe_last_error());
            return -1;
        }
    }
    g_active = 1;
    return 0;
}

static float sum_of(const float *x, int n) {
    float s = 0.0f;
    for (int i = 0; i < n; i++) s += x[i];
    return s;
}

int glm_hip_moe_layer(const Runtime *rt, RunState *st, int layer_idx, int debug_mode) {
    if (!g_ctx || !rt || !st) return -1;
    /* the same no-op cases as infer.c:1088-1092 */
    if (!rt->has_moe_shared) return 0;
    if (layer_idx <= 0 || layer_idx >= rt->cfg.n_layers) return 0;
    if (rt->cfg.moe_ffn_dim <= 0) return 0;
    if (!rt->moe_layers[layer_idx].ffn_norm) return 0;

    gmoe_layer_state s;
    memset(&s, 0, sizeof(s));
    s.xn = st->xn;
    s.router_prob = st->moe_router;
    s.topk_idx = (int32_t *)st->moe_topk_idx;
    s.topk_w = st->moe_topk_w;
    s.shared_out = st->xb;
    s.routed_out = st->moe_out_acc;
    const int flags = routed_disabled() ? GMOE_FLAG_NO_ROUTED : 0;
    if (gmoe_forward_host(g_ctx, layer_idx, 1, st->x, st->x, flags, &s) != GMOE_OK) {
        fprintf(stderr, "[glm-hip] MoE layer %d failed: %s\n", layer_idx, gmoe_last_error());
        return -1;
    }
    if (debug_mode) {
        /* the per-layer sums that infer.c:1207-1210 prints */
        fprintf(stderr, "[glm-layer-sum] ffn_moe_out-%d sum=%.6f\n", layer_idx, sum_of(st->moe_out_acc, rt->cfg.dim));
        fprintf(stderr, "[glm-layer-sum] ffn_shexp-%d sum=%.6f\n", layer_idx, sum_of(st->xb, rt->cfg.dim));
    }
    return 0;
}

void glm_hip_free(void) {
    if (g_ctx) gmoe_destroy(g_ctx);
    g_ctx = NULL;
    g_active = 0;
}

int glm_backend_try_hip_moe(const Runtime *rt, RunState *st, int layer_idx, int debug_mode) {
    if (!g_active) return -1;
    if (glm_hip_moe_layer(rt, st, layer_idx, debug_mode) == 0) return 0;
    if (env_on("GLM_HIP_STRICT", 0)) {
        fprintf(stderr, "[glm-hip] strict mode: aborting after a failed GPU layer\n");
        exit(1);
    }
    return -1;
}

void glm_set_metal_matvec_mode(int enabled) { (void)enabled; }

int glm_backend_metal_matvec_enabled(void) { return 0; }

int glm_backend_try_metal_matvec(const int8_t *qmat, const float *smat, const float *x, float *y, int rows, int dim,
                                 int gs) {
    (void)qmat;
    (void)smat;
    (void)x;
    (void)y;
    (void)rows;
    (void)dim;
    (void)gs;
    return -1;
}

int glm_backend_init(BackendType backend, const Runtime *rt, RunState *st) {
    if (backend == BACKEND_METAL) {
        fprintf(stderr, "[glm-metal] unavailable on this platform\n");
        exit(1);
    }
    if (backend != BACKEND_HIP) return 0;
    if (glm_hip_init(rt, st) != 0) {
        fprintf(stderr, "[glm-hip] init failed\n");
        exit(1);
    }
    if (glm_hip_prepare(rt, st) != 0) {
        fprintf(stderr, "[glm-hip] prepare failed\n");
        exit(1);
    }
    return (int)BACKEND_HIP;
}

int glm_backend_forward_token(int use_gpu, const Runtime *rt, RunState *st, int token, int pos, int debug_mode) {
    if (use_gpu == (int)BACKEND_HIP) return glm_hip_forward_token(rt, st, token, pos, debug_mode);
    /* the CPU backend: glm.c's own forward (backend.c:88-91) */
    if (!glm_cpu_forward_token) {
        fprintf(stderr, "[glm-hip] glm_cpu_forward_token is not linked in\n");
        return -1;
    }
    return glm_cpu_forward_token(rt, st, token, pos, debug_mode);
}

void glm_backend_free(int use_gpu) {
    if (use_gpu == (int)BACKEND_HIP) glm_hip_free();
}
