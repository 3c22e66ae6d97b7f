/*
 * ORACLE (reference build) -- test infrastructure only (see oracle.h).
 *
 * Compiles glm.c's own infer.c into this translation unit, so that its static
 * apply_moe_shared_ffn_layer (infer.c:1087-1216) can be driven on synthetic
 * weights. The include path to the reference sources is supplied by
 * oracle/Makefile; nothing from the reference is copied into this repository.
 * The result, oracle/_ref/libref_moe.so, is built with the reference Makefile's
 * compiler flags (Makefile:1-2, 89) and serves as the bitwise check of the
 * restatement in moe_oracle.c and as the CPU baseline in bench.py.
 */
#include "infer.c"

#include "oracle.h"

/* A Runtime that holds only MoE layers 1..n_moe (layer 0 is the dense layer,
 * never touched here), shaped like runtime_open leaves it (infer.c:640-743). */
static void make_runtime(Runtime *rt, LayerMoeShared *sh, LayerMoeRouted *ro, const oracle_dims *d,
                         const oracle_layer *layers, int n_moe) {
    memset(rt, 0, sizeof(*rt));
    rt->cfg.dim = d->dim;
    rt->cfg.hidden_dim = d->group_size;
    rt->cfg.n_layers = n_moe + 1;
    rt->cfg.vocab_size = 1;
    rt->cfg.seq_len = 1;
    rt->cfg.n_routed_experts = d->n_routed_experts;
    rt->cfg.n_experts_used = d->n_experts_used;
    rt->cfg.n_shared_experts = 1;
    rt->cfg.group_size = (uint64_t)d->group_size;
    rt->cfg.moe_ffn_dim = d->moe_ffn_dim;
    memset(&sh[0], 0, sizeof(sh[0]));
    memset(&ro[0], 0, sizeof(ro[0]));
    int routed = 1;
    for (int l = 0; l < n_moe; l++) {
        const oracle_layer *w = &layers[l];
        LayerMoeShared *s = &sh[l + 1];
        LayerMoeRouted *r = &ro[l + 1];
        s->ffn_norm = w->ffn_norm;
        s->gate_inp = w->gate_inp;
        s->exp_probs_b = w->exp_probs_b;
        s->gate_sh_q = w->gate_sh_q;
        s->gate_sh_s = w->gate_sh_s;
        s->up_sh_q = w->up_sh_q;
        s->up_sh_s = w->up_sh_s;
        s->down_sh_q = w->down_sh_q;
        s->down_sh_s = w->down_sh_s;
        r->gate_q = w->gate_q;
        r->gate_s = w->gate_s;
        r->up_q = w->up_q;
        r->up_s = w->up_s;
        r->down_q = w->down_q;
        r->down_s = w->down_s;
        if (!w->gate_q) routed = 0;
    }
    rt->has_moe_shared = 1;
    rt->moe_layers = sh;
    rt->has_moe_routed = routed;
    rt->moe_routed_layers = ro;
}

int ref_moe_layer(const oracle_dims *d, const oracle_layer *w, int T, const float *x_in, const oracle_out *out,
                  int disable_routed) {
    if (!d || !w || !x_in || !out || T < 0) return -1;
    Runtime rt;
    LayerMoeShared sh[2];
    LayerMoeRouted ro[2];
    make_runtime(&rt, sh, ro, d, w, 1);
    RunState st;
    runstate_build(&st, &rt, 1);
    if (disable_routed) setenv("GLM_DISABLE_MOE_ROUTED", "1", 1);
    else unsetenv("GLM_DISABLE_MOE_ROUTED");
    const int D = d->dim, E = d->n_routed_experts, K = d->n_experts_used;
    const int gs = d->group_size;
    for (int t = 0; t < T; t++) {
        memcpy(st.x, x_in + (size_t)t * D, (size_t)D * sizeof(float));
        apply_moe_shared_ffn_layer(&rt, &st, gs, 1, 0, 0);
        if (out->x_out) memcpy(out->x_out + (size_t)t * D, st.x, (size_t)D * sizeof(float));
        if (out->xn) memcpy(out->xn + (size_t)t * D, st.xn, (size_t)D * sizeof(float));
        if (out->router_prob) memcpy(out->router_prob + (size_t)t * E, st.moe_router, (size_t)E * sizeof(float));
        if (out->topk_idx)
            for (int k = 0; k < K; k++) out->topk_idx[(size_t)t * K + k] = (int32_t)st.moe_topk_idx[k];
        if (out->topk_w) memcpy(out->topk_w + (size_t)t * K, st.moe_topk_w, (size_t)K * sizeof(float));
        if (out->shared_out) memcpy(out->shared_out + (size_t)t * D, st.xb, (size_t)D * sizeof(float));
        if (out->routed_out) memcpy(out->routed_out + (size_t)t * D, st.moe_out_acc, (size_t)D * sizeof(float));
    }
    unsetenv("GLM_DISABLE_MOE_ROUTED");
    runstate_free(&st);
    return 0;
}

int ref_moe_stack(const oracle_dims *d, const oracle_layer *layers, int n_layers, int T, float *x, int32_t *topk_idx) {
    if (!d || !layers || !x || n_layers < 0 || T < 0) return -1;
    Runtime rt;
    LayerMoeShared *sh = (LayerMoeShared *)calloc((size_t)n_layers + 1, sizeof(LayerMoeShared));
    LayerMoeRouted *ro = (LayerMoeRouted *)calloc((size_t)n_layers + 1, sizeof(LayerMoeRouted));
    if (!sh || !ro) {
        free(sh);
        free(ro);
        return -1;
    }
    make_runtime(&rt, sh, ro, d, layers, n_layers);
    RunState st;
    runstate_build(&st, &rt, 1);
    unsetenv("GLM_DISABLE_MOE_ROUTED");
    const int D = d->dim, K = d->n_experts_used, gs = d->group_size;
    for (int t = 0; t < T; t++) {
        memcpy(st.x, x + (size_t)t * D, (size_t)D * sizeof(float));
        for (int l = 1; l <= n_layers; l++) {
            apply_moe_shared_ffn_layer(&rt, &st, gs, l, 0, 0);
            if (topk_idx)
                for (int k = 0; k < K; k++) topk_idx[((size_t)(l - 1) * T + t) * K + k] = (int32_t)st.moe_topk_idx[k];
        }
        memcpy(x + (size_t)t * D, st.x, (size_t)D * sizeof(float));
    }
    runstate_free(&st);
    free(sh);
    free(ro);
    return 0;
}

/* CPU baseline timing (bench.py): n_tokens tokens through the stack from x (updated in
 * place), each layer call timed with glm.c's own monotonic_ms (infer.c:1426-1430) into
 * layer_ms[t * n_layers + l]. n_threads > 0 sets the OpenMP team (omp_set_num_threads). */
int ref_moe_stack_timed(const oracle_dims *d, const oracle_layer *layers, int n_layers, int n_tokens, float *x,
                        double *layer_ms, int n_threads) {
    if (!d || !layers || !x || !layer_ms || n_layers < 1 || n_tokens < 0) return -1;
    if (n_threads > 0) omp_set_num_threads(n_threads);
    Runtime rt;
    LayerMoeShared *sh = (LayerMoeShared *)calloc((size_t)n_layers + 1, sizeof(LayerMoeShared));
    LayerMoeRouted *ro = (LayerMoeRouted *)calloc((size_t)n_layers + 1, sizeof(LayerMoeRouted));
    if (!sh || !ro) {
        free(sh);
        free(ro);
        return -1;
    }
    make_runtime(&rt, sh, ro, d, layers, n_layers);
    RunState st;
    runstate_build(&st, &rt, 1);
    unsetenv("GLM_DISABLE_MOE_ROUTED");
    const int D = d->dim, gs = d->group_size;
    memcpy(st.x, x, (size_t)D * sizeof(float));
    for (int t = 0; t < n_tokens; t++) {
        for (int l = 1; l <= n_layers; l++) {
            const double t0 = monotonic_ms();
            apply_moe_shared_ffn_layer(&rt, &st, gs, l, 0, 0);
            layer_ms[(size_t)t * n_layers + (l - 1)] = monotonic_ms() - t0;
        }
    }
    memcpy(x, st.x, (size_t)D * sizeof(float));
    runstate_free(&st);
    free(sh);
    free(ro);
    return 0;
}

/* CPU baseline timing of a batch: glm.c routes prompt tokens one at a time
 * (infer.c:2190-2233), so each of the T tokens of x_in is one timed layer call
 * (token_ms[t]). */
int ref_moe_layer_timed(const oracle_dims *d, const oracle_layer *w, int T, const float *x_in, double *token_ms,
                        int n_threads) {
    if (!d || !w || !x_in || !token_ms || T < 0) return -1;
    if (n_threads > 0) omp_set_num_threads(n_threads);
    Runtime rt;
    LayerMoeShared sh[2];
    LayerMoeRouted ro[2];
    make_runtime(&rt, sh, ro, d, w, 1);
    RunState st;
    runstate_build(&st, &rt, 1);
    unsetenv("GLM_DISABLE_MOE_ROUTED");
    const int D = d->dim, gs = d->group_size;
    for (int t = 0; t < T; t++) {
        memcpy(st.x, x_in + (size_t)t * D, (size_t)D * sizeof(float));
        const double t0 = monotonic_ms();
        apply_moe_shared_ffn_layer(&rt, &st, gs, 1, 0, 0);
        token_ms[t] = monotonic_ms() - t0;
    }
    runstate_free(&st);
    return 0;
}

/* glm.c's own loader on a checkpoint file (runtime_open, infer.c:357-744; it exits the
 * process on a file it rejects, so callers run this in a child process): the header and
 * every tensor pointer as its file offset (0 for none), in the order of glm_ckpt_layout
 * (include/glm_ckpt.h). Returns the number of offsets. */
int ref_ckpt_layout(const char *path, uint64_t *out, int max, void *cfg_out) {
    Runtime rt;
    runtime_open(&rt, path);
    int n = 0;
#define PUT(p) do { if (n < max) out[n] = (p) ? (uint64_t)((const unsigned char *)(p) - rt.data) : 0u; n++; } while (0)
    PUT(rt.output_norm);
    PUT(rt.tok_q);
    PUT(rt.tok_s);
    PUT(rt.out_q);
    PUT(rt.out_s);
    const void *l0f[7] = {rt.l0_ffn_norm, rt.l0_ffn_gate_q, rt.l0_ffn_gate_s, rt.l0_ffn_up_q,
                          rt.l0_ffn_up_s, rt.l0_ffn_down_q, rt.l0_ffn_down_s};
    for (int i = 0; i < 7; i++) PUT(rt.has_l0_ffn ? l0f[i] : NULL);
    const void *l0a[15] = {rt.l0_attn_norm, rt.l0_q_a_norm, rt.l0_kv_a_norm, rt.l0_q_a_q, rt.l0_q_a_s,
                           rt.l0_q_b_q, rt.l0_q_b_s, rt.l0_kv_a_q, rt.l0_kv_a_s, rt.l0_k_b_q, rt.l0_k_b_s,
                           rt.l0_v_b_q, rt.l0_v_b_s, rt.l0_attn_out_q, rt.l0_attn_out_s};
    for (int i = 0; i < 15; i++) PUT(rt.has_l0_attn ? l0a[i] : NULL);
    for (int l = 0; l < rt.cfg.n_layers; l++) {
        const LayerAttnWeights *w = rt.has_all_attn ? &rt.attn_layers[l] : NULL;
        const void *a[15] = {0};
        if (w) {
            const void *t[15] = {w->attn_norm, w->q_a_norm, w->kv_a_norm, w->q_a_q, w->q_a_s, w->q_b_q, w->q_b_s,
                                 w->kv_a_q, w->kv_a_s, w->k_b_q, w->k_b_s, w->v_b_q, w->v_b_s, w->attn_out_q,
                                 w->attn_out_s};
            memcpy(a, t, sizeof(t));
        }
        for (int i = 0; i < 15; i++) PUT(a[i]);
    }
    for (int l = 1; l < rt.cfg.n_layers; l++) {
        const void *s[9] = {0}, *r[6] = {0};
        if (rt.has_moe_shared) {
            const LayerMoeShared *w = &rt.moe_layers[l];
            const void *t[9] = {w->ffn_norm, w->gate_inp, w->exp_probs_b, w->gate_sh_q, w->gate_sh_s,
                                w->up_sh_q, w->up_sh_s, w->down_sh_q, w->down_sh_s};
            memcpy(s, t, sizeof(t));
        }
        if (rt.has_moe_routed) {
            const LayerMoeRouted *w = &rt.moe_routed_layers[l];
            const void *t[6] = {w->gate_q, w->gate_s, w->up_q, w->up_s, w->down_q, w->down_s};
            memcpy(r, t, sizeof(t));
        }
        for (int i = 0; i < 9; i++) PUT(s[i]);
        for (int i = 0; i < 6; i++) PUT(r[i]);
    }
#undef PUT
    if (cfg_out) memcpy(cfg_out, &rt.cfg, sizeof(rt.cfg));
    runtime_close(&rt);
    return n;
}

/* glm.c's own token forward on the checkpoint at `path` (runtime_open, runstate_build,
 * infer.c:357-744, 827-860; a child process, as for ref_ckpt_layout): tokens[i] at
 * position i for i < n, teacher-forced. Per position, glm_cpu_forward_token_dual_checkpoints
 * (infer.c:1940-1983) gives x after each layer's attention and after its FFN, into
 * attn_out and layer_out ([n][n_layers][dim]), and glm_cpu_forward_token (infer.c:1903)
 * then advances the state, whose logits go to logits ([n][vocab]). 0, or -1. */
int ref_decode(const char *path, const int *tokens, int n, int cache_cap, float *attn_out, float *layer_out,
               float *logits) {
    Runtime rt;
    runtime_open(&rt, path);
    RunState st;
    runstate_build(&st, &rt, cache_cap);
    const int L = rt.cfg.n_layers, dim = rt.cfg.dim, V = rt.cfg.vocab_size;
    int rc = 0;
    for (int i = 0; i < n && !rc; i++) {
        int wa = 0, wl = 0;
        rc = glm_cpu_forward_token_dual_checkpoints(&rt, &st, tokens[i], i, 0, attn_out + (size_t)i * L * dim, dim, L,
                                                    &wa, layer_out + (size_t)i * L * dim, dim, L, &wl);
        if (!rc) rc = glm_cpu_forward_token(&rt, &st, tokens[i], i, 0);
        if (!rc) memcpy(logits + (size_t)i * V, st.logits, (size_t)V * sizeof(float));
    }
    runstate_free(&st);
    runtime_close(&rt);
    return rc;
}

/* CPU baseline timing of the whole forward (bench.py --e2e-cpu): glm.c's
 * glm_cpu_forward_token (infer.c:1903) on the checkpoint at `path` for n_tokens tokens at
 * positions pos, pos + 1, ... of a cache of cache_cap positions, each timed with glm.c's
 * monotonic_ms (infer.c:1426-1430) into token_ms. The cache below pos holds runstate_build's
 * zeros instead of a prompt's entries: the attention reads every position up to its own
 * either way (infer.c:1029-1051), so the work per token is that of a pos-token context.
 * n_threads > 0 sets the OpenMP team. A child process, as for ref_ckpt_layout. 0, or -1. */
int ref_forward_timed(const char *path, int token, int pos, int cache_cap, int n_tokens, int n_threads,
                      double *token_ms) {
    if (!path || !token_ms || pos < 0 || n_tokens < 1 || pos + n_tokens > cache_cap) return -1;
    if (n_threads > 0) omp_set_num_threads(n_threads);
    Runtime rt;
    runtime_open(&rt, path);
    RunState st;
    runstate_build(&st, &rt, cache_cap);
    int rc = 0;
    for (int i = 0; i < n_tokens && !rc; i++) {
        const double t0 = monotonic_ms();
        rc = glm_cpu_forward_token(&rt, &st, token, pos + i, 0);
        token_ms[i] = monotonic_ms() - t0;
    }
    runstate_free(&st);
    runtime_close(&rt);
    return rc;
}

/* glm.c's own steps of one token at position pos, each on inputs the caller gives (a child
 * process, as for ref_ckpt_layout), so that a device forward can be checked stage by stage
 * on its own intermediate values:
 *   stage 0  layer `layer`'s attention (apply_mla_attention_layer, infer.c:978-1065) on x_in,
 *            or for x_in == NULL on the token's embedding row (infer.c:1807-1810), over a
 *            cache whose positions 0..pos-1 are comp [pos][kv_lora] and pe [pos][rope];
 *            out = x after it [dim];
 *   stage 1  layer `layer`'s FFN (apply_l0_dense_ffn for layer 0, else
 *            apply_moe_shared_ffn_layer, infer.c:1067-1216) on x_in; out = x after it [dim];
 *   stage 2  the final rmsnorm and the LM head (infer.c:1886-1893) on x_in; out = logits.
 * 0, or -1. */
int ref_stage(const char *path, int stage, int layer, int token, int pos, const float *comp, const float *pe,
              const float *x_in, float *out) {
    Runtime rt;
    runtime_open(&rt, path);
    RunState st;
    runstate_build(&st, &rt, pos + 1);
    const RuntimeConfig *c = &rt.cfg;
    const int dim = c->dim, gs = (int)c->group_size;
    int rc = 0;
    if (x_in) {
        memcpy(st.x, x_in, (size_t)dim * sizeof(float));
    } else {
        if (token < 0 || token >= c->vocab_size) token = 0;
        dequant_row(rt.tok_q + (size_t)token * dim, rt.tok_s + (size_t)token * (dim / gs), st.x, dim, gs);
    }
    if (stage == 0) {
        if (!rt.has_all_attn || layer < 0 || layer >= c->n_layers) {
            rc = -1;
        } else {
            const size_t base = (size_t)layer * (size_t)st.cache_cap;
            if (pos > 0) {
                memcpy(st.k_cache_comp + base * c->kv_lora_rank, comp, (size_t)pos * c->kv_lora_rank * sizeof(float));
                memcpy(st.k_cache_pe + base * c->rope_dim, pe, (size_t)pos * c->rope_dim * sizeof(float));
            }
            apply_mla_attention_layer(&rt, &rt.attn_layers[layer], &st, gs, pos, layer, 0);
            memcpy(out, st.x, (size_t)dim * sizeof(float));
        }
    } else if (stage == 1) {
        if (layer == 0) apply_l0_dense_ffn(&rt, &st, gs, 0);
        else apply_moe_shared_ffn_layer(&rt, &st, gs, layer, 0, pos);
        memcpy(out, st.x, (size_t)dim * sizeof(float));
    } else if (stage == 2) {
        rmsnorm(st.xn, st.x, rt.output_norm, dim);
        matvec_rows(rt.out_q, rt.out_s, st.xn, out, c->vocab_size, dim, gs);
    } else {
        rc = -1;
    }
    runstate_free(&st);
    runtime_close(&rt);
    return rc;
}

/* glm.c's forward of `token` at position pos of a cache of pos + 1 positions as
 * runstate_build leaves it (zeros below pos; infer.c:827-860): the dual checkpoints
 * (infer.c:1940-1983) into attn_out and layer_out ([n_layers][dim]) and the logits. A child
 * process, as above. 0, or -1. */
int ref_forward_zero_cache(const char *path, int token, int pos, float *attn_out, float *layer_out, float *logits) {
    Runtime rt;
    runtime_open(&rt, path);
    RunState st;
    runstate_build(&st, &rt, pos + 1);
    const int L = rt.cfg.n_layers, dim = rt.cfg.dim;
    int wa = 0, wl = 0;
    int rc = glm_cpu_forward_token_dual_checkpoints(&rt, &st, token, pos, 0, attn_out, dim, L, &wa, layer_out, dim, L, &wl);
    if (!rc) rc = glm_cpu_forward_token(&rt, &st, token, pos, 0);
    if (!rc) memcpy(logits, st.logits, (size_t)rt.cfg.vocab_size * sizeof(float));
    runstate_free(&st);
    runtime_close(&rt);
    return rc;
}
