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
 *   GLM_HIP_HOST_ATTN       keep embedding, attention, layer 0 and the LM head on the host
 *                           (glm.c's own arithmetic, forward.c) instead of the GPU model
 *   GLM_HIP_PREFILL_BATCH   most prompt tokens of one batched prefill step (glm_hip_prefill;
 *                           default 1024, 1 turns batching off)
 *   GLM_HIP_STRICT          exit(1) when a GPU layer fails instead of returning -1
 *   GLM_DISABLE_MOE_ROUTED  skip routed experts, as infer.c:1161-1166 does
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "glm_backend.h"
#include "glm_forward.h"
#include "gmoe.h"
#include "gmoe_model.h"

_Static_assert(sizeof(int) == sizeof(int32_t), "RunState.moe_topk_idx is int; the ABI uses int32_t");

/* glm.c's CPU forward (infer.c:1903). Weak, so this library also loads on its own. */
int glm_cpu_forward_token(const Runtime *rt, RunState *st, int token, int pos, int debug_mode) __attribute__((weak));

static gmoe_ctx *g_ctx = NULL;
static gmoe_model *g_model = NULL; /* the whole forward on the GPU (gmoe_model.h), when built */
static int g_active = 0;
static gmoe_config g_cfg;  /* the context's config, kept to re-create it in the native form */
static int g_device = 0;

static int prepare_model(const Runtime *rt, const RunState *st);
static int routed_disabled(void);

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
    /* the decode loop feeds one token at a time, glm_hip_prefill up to a batch of prompt tokens */
    const char *pb = getenv("GLM_HIP_PREFILL_BATCH");
    cfg.max_tokens = pb && atoi(pb) > 0 ? atoi(pb) : 1024;
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
    if (!env_on("GLM_HIP_HOST_ATTN", 0)) (void)prepare_model(rt, st);
    return 0;
}

/* The device model for rt with a cache of st->cache_cap positions: every tensor outside the
 * MoE layers uploaded, the MoE layers taken from g_ctx. 0, or -1 (and no model) when the
 * checkpoint's shape is one the model's kernels do not take or the GPU refuses it. */
static int prepare_model(const Runtime *rt, const RunState *st) {
    const RuntimeConfig *c = &rt->cfg;
    /* a Runtime that carries only MoE layers (the per-layer hook's callers) has no forward */
    if (!rt->tok_q || !rt->out_q || !rt->output_norm || c->vocab_size <= 0) return -1;
    gmoe_model_config mc;
    memset(&mc, 0, sizeof(mc));
    mc.dim = c->dim;
    mc.hidden_dim = c->hidden_dim;
    mc.n_layers = c->n_layers;
    mc.n_heads = c->n_heads;
    mc.vocab_size = c->vocab_size;
    mc.q_lora_rank = c->q_lora_rank;
    mc.kv_lora_rank = c->kv_lora_rank;
    mc.rope_dim = c->rope_dim;
    mc.qk_nope_dim = c->l0_qk_nope_dim;
    mc.head_k_dim = c->l0_head_k_dim;
    mc.v_head_dim = c->l0_v_head_dim;
    mc.group_size = (int32_t)c->group_size;
    mc.cache_cap = st ? st->cache_cap : 0;
    mc.attn_layers = rt->has_all_attn ? c->n_layers : (rt->has_l0_attn ? 1 : 0);
    mc.has_l0_ffn = rt->has_l0_ffn;
    mc.max_batch = g_cfg.max_tokens;
    gmoe_model *m = NULL;
    if (gmoe_model_create(&m, g_device, &mc) != GMOE_OK) {
        fprintf(stderr, "[glm-hip] %s; attention, layer 0 and the LM head stay on the host\n", gmoe_last_error());
        return -1;
    }
    gmoe_model_weights w;
    memset(&w, 0, sizeof(w));
    w.output_norm = rt->output_norm;
    w.tok_q = rt->tok_q;
    w.tok_s = rt->tok_s;
    w.out_q = rt->out_q;
    w.out_s = rt->out_s;
    w.l0_ffn_norm = rt->l0_ffn_norm;
    w.l0_ffn_gate_q = rt->l0_ffn_gate_q;
    w.l0_ffn_gate_s = rt->l0_ffn_gate_s;
    w.l0_ffn_up_q = rt->l0_ffn_up_q;
    w.l0_ffn_up_s = rt->l0_ffn_up_s;
    w.l0_ffn_down_q = rt->l0_ffn_down_q;
    w.l0_ffn_down_s = rt->l0_ffn_down_s;
    int rc = gmoe_model_upload(m, &w);
    for (int l = 0; l < mc.attn_layers && rc == GMOE_OK; l++) {
        /* LayerAttnWeights and gmoe_attn_weights list the same tensors in the same order */
        const LayerAttnWeights l0 = {rt->l0_attn_norm, rt->l0_q_a_norm, rt->l0_kv_a_norm, rt->l0_q_a_q, rt->l0_q_a_s,
                                     rt->l0_q_b_q,     rt->l0_q_b_s,    rt->l0_kv_a_q,    rt->l0_kv_a_s, rt->l0_k_b_q,
                                     rt->l0_k_b_s,     rt->l0_v_b_q,    rt->l0_v_b_s,     rt->l0_attn_out_q,
                                     rt->l0_attn_out_s};
        const LayerAttnWeights *a = rt->has_all_attn ? &rt->attn_layers[l] : &l0;
        const gmoe_attn_weights aw = {a->attn_norm, a->q_a_norm, a->kv_a_norm, a->q_a_q,  a->q_a_s,
                                      a->q_b_q,     a->q_b_s,    a->kv_a_q,    a->kv_a_s, a->k_b_q,
                                      a->k_b_s,     a->v_b_q,    a->v_b_s,     a->attn_out_q, a->attn_out_s};
        rc = gmoe_model_upload_attn(m, l, &aw);
    }
    if (rc == GMOE_OK) {
        uint8_t *on = (uint8_t *)calloc((size_t)c->n_layers, 1);
        if (!on) {
            rc = GMOE_ERR_NOMEM;
        } else {
            for (int l = 1; l < c->n_layers; l++)
                on[l] = (uint8_t)(rt->has_moe_shared && rt->moe_layers && rt->moe_layers[l].ffn_norm != NULL);
            rc = gmoe_model_set_moe(m, g_ctx, on, routed_disabled() ? GMOE_FLAG_NO_ROUTED : 0);
            free(on);
        }
    }
    if (rc != GMOE_OK) {
        fprintf(stderr, "[glm-hip] model upload failed: %s; attention, layer 0 and the LM head stay on the host\n",
                gmoe_last_error());
        gmoe_model_destroy(m);
        return -1;
    }
    g_model = m;
    return 0;
}

int glm_hip_model_active(void) { return g_model != NULL; }


/* The RunState whose decode history the GPU model's latent cache holds (positions
 * 0 .. g_model_len-1, in device memory: that state's own host cache is not written), and
 * its cache buffer, which tells the state from a copy of it. Every other RunState keeps its
 * history in its host cache, so the model runs a token only for this state, or to start
 * the first sequence at position 0; other states take glm.c's host steps. */
static const RunState *g_model_st = NULL;
static const float *g_model_cache = NULL;
static int g_model_len = 0;

int glm_hip_model_read_cache(int layer, int pos0, int n, float *comp_out, float *pe_out) {
    if (!g_model) return -1;
    if (gmoe_model_read_cache(g_model, layer, pos0, n, comp_out, pe_out, NULL) != GMOE_OK) {
        fprintf(stderr, "[glm-hip] %s\n", gmoe_last_error());
        return -1;
    }
    return 0;
}

int glm_hip_model_owns(const RunState *st, int pos) {
    if (!g_model || !st || pos < 0) return 0;
    if (!g_model_st) return pos == 0;
    return st == g_model_st && st->k_cache_comp == g_model_cache && pos <= g_model_len;
}

static void model_track(const RunState *st, int end) {
    if (g_model_st != st) g_model_len = 0;
    g_model_st = st;
    g_model_cache = st->k_cache_comp;
    if (end > g_model_len) g_model_len = end;
}

void glm_hip_model_forget(const RunState *st) {
    if (st && st == g_model_st) {
        g_model_st = NULL;
        g_model_cache = NULL;
        g_model_len = 0;
    }
}

int glm_hip_model_forward(const Runtime *rt, RunState *st, int token, int pos, int keep_state, float *logits,
                          float *attn_ckpt, float *layer_ckpt) {
    (void)rt;
    if (!g_model || !st) return -1;
    const int rc = gmoe_model_forward_token(g_model, token, pos, keep_state ? GMOE_MODEL_KEEP_CACHE : 0,
                                            logits ? logits : st->logits, keep_state ? NULL : st->x, attn_ckpt,
                                            layer_ckpt, NULL);
    if (rc != GMOE_OK) {
        fprintf(stderr, "[glm-hip] forward at position %d failed: %s\n", pos, gmoe_last_error());
        return -1;
    }
    if (!keep_state) model_track(st, pos + 1);
    return 0;
}

int glm_hip_model_forward_sums(RunState *st, int token, int pos, float *attn_ckpt, float *layer_ckpt, float *kv_out,
                               float *concat_out, float *shexp_out, float *moe_out) {
    if (!g_model || !st) return -1;
    if (gmoe_model_forward_token_debug(g_model, token, pos, 0, st->logits, st->x, attn_ckpt, layer_ckpt, kv_out,
                                       concat_out, shexp_out, moe_out, NULL) != GMOE_OK) {
        fprintf(stderr, "[glm-hip] forward at position %d failed: %s\n", pos, gmoe_last_error());
        return -1;
    }
    model_track(st, pos + 1);
    return 0;
}

int glm_hip_model_prefill(const Runtime *rt, RunState *st, const int *tokens, int n, int pos0) {
    (void)rt;
    if (!g_model || !st || !tokens || n < 1) return -1;
    const int B = g_cfg.max_tokens;
    for (int i = 0; i < n; i += B) {
        const int k = n - i < B ? n - i : B;
        if (gmoe_model_prefill(g_model, (const int32_t *)tokens + i, k, pos0 + i, st->logits, st->x, NULL) != GMOE_OK) {
            fprintf(stderr, "[glm-hip] prefill at positions %d..%d failed: %s\n", pos0 + i, pos0 + i + k - 1,
                    gmoe_last_error());
            return -1;
        }
        model_track(st, pos0 + i + k);
    }
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
    if (g_model) gmoe_model_destroy(g_model);
    g_model = NULL;
    g_model_st = NULL;
    g_model_cache = NULL;
    g_model_len = 0;
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
