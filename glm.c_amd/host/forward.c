/*
 * forward.c -- glm.c's token forward (infer.c:1767-1901) for the --backend hip drop-in.
 *
 * One token at one position: embedding (infer.c:1807-1810), then per layer the MLA
 * attention (infer.c:978-1065) and the FFN -- layer 0's dense FFN (infer.c:1067-1085),
 * every MoE layer (infer.c:1087-1216) -- then the final rmsnorm and the LM head
 * (infer.c:1886-1893). When glm_hip_prepare built the GPU model (gmoe_model.h), all of it
 * runs there, with x and the latent cache in device memory. Otherwise (GLM_HIP_HOST_ATTN,
 * or a shape the model's kernels do not take) the steps below run on the host and each
 * MoE layer on the GPU through glm_hip_moe_layer.
 *
 * The host operations repeat glm.c's arithmetic operation for operation: the same
 * accumulation types and orders, the same parallel-rows / SIMD-reduction loop shape in
 * the Q8_0 matvec (compiled with the same flags, so the compiler forms the same
 * partial sums), the same libm calls. Before the first MoE layer the forward therefore
 * gives glm.c's bits; after it x carries the GPU layer's rounding (within max-abs 1e-2
 * and rel-L2 1e-3 of glm.c's FFN, ~1e-6 relative in practice).
 *
 * glm.c dies on a position past the cache and on allocation failure; these functions
 * print a "[glm-hip]" message and return -1 instead. With debug_mode both paths print
 * glm.c's "[glm-layer-sum]" lines: the MoE layers' two sums at every position
 * (infer.c:1207-1210) and the per-stage sums at position 0 (infer.c:1811-1895).
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "glm_backend.h"
#include "glm_forward.h"

/* ---- glm.c's host arithmetic ------------------------------------------------------ */

/* infer.c:746-752: fp64 sum of squares, fp32 mean and inverse root, x * inv * w. */
static void fw_rmsnorm(float *o, const float *x, const float *w, int n) {
    double ss = 0.0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * (double)x[i];
    const float mean = (float)(ss / (double)n);
    const float inv = 1.0f / sqrtf(mean + 1e-5f);
    for (int i = 0; i < n; i++) o[i] = x[i] * inv * w[i];
}

/* infer.c:754-763: one Q8_0 row to fp32. */
static void fw_dequant(const int8_t *q, const float *s, float *out, int n, int gs) {
    for (int g = 0; g < n / gs; g++) {
        const float sc = s[g];
        for (int k = 0; k < gs; k++) out[g * gs + k] = (float)q[g * gs + k] * sc;
    }
}

/* infer.c:765-786: y = Q8_0 matrix [rows][cols] . x. Each group's dot is a SIMD
 * reduction, scaled and added to the row's sum in group order; rows in parallel. */
static void fw_matvec(const int8_t *q, const float *s, const float *x, float *y, int rows, int cols, int gs) {
    const int ng = cols / gs;
#if defined(_OPENMP)
#pragma omp parallel for schedule(static) if (rows >= 64)
#endif
    for (int r = 0; r < rows; r++) {
        const int8_t *qr = q + (size_t)r * cols;
        const float *sr = s + (size_t)r * ng;
        float acc = 0.0f;
        for (int g = 0; g < ng; g++) {
            const float sc = sr[g];
            const int b = g * gs;
            float dot = 0.0f;
#if defined(_OPENMP)
#pragma omp simd reduction(+:dot)
#endif
            for (int k = 0; k < gs; k++) dot += (float)qr[b + k] * x[b + k];
            acc += sc * dot;
        }
        y[r] = acc;
    }
}

/* infer.c:916-925 (the build without BLAS): a sequential fp32 dot. */
static float fw_dot(const float *a, const float *b, int n) {
    float s = 0.0f;
    for (int i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

/* infer.c:940-949: the --debug sums, a sequential fp32 sum of a vector. */
static float fw_sum(const float *x, int n) {
    float s = 0.0f;
    for (int i = 0; i < n; i++) s += x[i];
    return s;
}
static void fw_print_sum(const char *name, int layer, float v) {
    if (layer >= 0)
        fprintf(stderr, "[glm-layer-sum] %s-%d sum=%.6f\n", name, layer, v);
    else
        fprintf(stderr, "[glm-layer-sum] %s sum=%.6f\n", name, v);
}

/* infer.c:912-914 */
static float fw_silu(float v) { return v / (1.0f + expf(-v)); }

/* infer.c:951-962 */
static void fw_softmax(float *v, int n) {
    float mx = v[0];
    for (int i = 1; i < n; i++)
        if (v[i] > mx) mx = v[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        v[i] = expf(v[i] - mx);
        sum += v[i];
    }
    if (sum <= 0.0f) return;
    const float inv = 1.0f / sum;
    for (int i = 0; i < n; i++) v[i] *= inv;
}

/* infer.c:964-976: rotary embedding of consecutive pairs, base 1e6. */
static void fw_rope(float *v, int n, int pos) {
    const float base = 1000000.0f;
    for (int i = 0; i + 1 < n; i += 2) {
        const float freq = powf(base, -((float)i / (float)n));
        const float ang = (float)pos * freq;
        const float c = cosf(ang), sn = sinf(ang);
        const float a = v[i], b = v[i + 1];
        v[i] = a * c - b * sn;
        v[i + 1] = a * sn + b * c;
    }
}

/* ---- layers ----------------------------------------------------------------------- */

/* infer.c:978-1065: MLA attention of layer `layer` at position pos, with the latent
 * cache (kv_lora values and rope_dim rotated values per position) in st. */
static int fw_attention(const Runtime *rt, const LayerAttnWeights *w, RunState *s, int gs, int pos, int layer) {
    if (!w) return 0;
    if (pos < 0 || pos >= s->cache_cap) {
        fprintf(stderr, "[glm-hip] position %d outside the attention cache (%d positions)\n", pos, s->cache_cap);
        return -1;
    }
    if (layer < 0 || layer >= s->n_attn_layers) {
        fprintf(stderr, "[glm-hip] attention layer %d outside the cache's %d layers\n", layer, s->n_attn_layers);
        return -1;
    }
    const RuntimeConfig *c = &rt->cfg;
    const int dim = c->dim, heads = c->n_heads, q_lora = c->q_lora_rank, kv_lora = c->kv_lora_rank;
    const int rope = c->rope_dim, nope = c->l0_qk_nope_dim, head_k = c->l0_head_k_dim, v_head = c->l0_v_head_dim;
    const float kq_scale = 1.0f / sqrtf((float)head_k);

    fw_rmsnorm(s->xn, s->x, w->attn_norm, dim);
    fw_matvec(w->q_a_q, w->q_a_s, s->xn, s->q_a, q_lora, dim, gs);
    fw_rmsnorm(s->q_a, s->q_a, w->q_a_norm, q_lora);
    fw_matvec(w->q_b_q, w->q_b_s, s->q_a, s->q_full, heads * head_k, q_lora, gs);
    fw_matvec(w->kv_a_q, w->kv_a_s, s->xn, s->kv_a, kv_lora + rope, dim, gs);
    fw_rmsnorm(s->kv_a, s->kv_a, w->kv_a_norm, kv_lora);

    const size_t first = (size_t)layer * (size_t)s->cache_cap;  // this layer's position 0
    float *comp = s->k_cache_comp + (first + (size_t)pos) * (size_t)kv_lora;
    float *pe = s->k_cache_pe + (first + (size_t)pos) * (size_t)rope;
    memcpy(comp, s->kv_a, (size_t)kv_lora * sizeof(float));
    memcpy(pe, s->kv_a + kv_lora, (size_t)rope * sizeof(float));
    fw_rope(pe, rope, pos);

    for (int h = 0; h < heads; h++) {
        const float *qh = s->q_full + (size_t)h * head_k;
        memcpy(s->q_nope, qh, (size_t)nope * sizeof(float));
        memcpy(s->q_pe, qh + nope, (size_t)rope * sizeof(float));
        fw_rope(s->q_pe, rope, pos);
        // the query absorbed into the latent space: k_b of head h [kv_lora][nope] . q_nope
        fw_matvec(w->k_b_q + (size_t)h * kv_lora * nope, w->k_b_s + (size_t)h * kv_lora * (nope / gs), s->q_nope,
                  s->q_abs, kv_lora, nope, gs);
        for (int t = 0; t <= pos; t++) {
            const float *kc = s->k_cache_comp + (first + (size_t)t) * (size_t)kv_lora;
            const float *kp = s->k_cache_pe + (first + (size_t)t) * (size_t)rope;
            const float score = fw_dot(s->q_abs, kc, kv_lora) + fw_dot(s->q_pe, kp, rope);
            s->att_scores[t] = score * kq_scale;
        }
        fw_softmax(s->att_scores, pos + 1);
        memset(s->att_ctx, 0, (size_t)kv_lora * sizeof(float));
        for (int t = 0; t <= pos; t++) {
            const float *kc = s->k_cache_comp + (first + (size_t)t) * (size_t)kv_lora;
            const float p = s->att_scores[t];
            for (int i = 0; i < kv_lora; i++) s->att_ctx[i] += p * kc[i];
        }
        // back out of the latent space: v_b of head h [v_head][kv_lora] . ctx
        fw_matvec(w->v_b_q + (size_t)h * v_head * kv_lora, w->v_b_s + (size_t)h * v_head * (kv_lora / gs), s->att_ctx,
                  s->att_concat + (size_t)h * v_head, v_head, kv_lora, gs);
    }
    fw_matvec(w->attn_out_q, w->attn_out_s, s->att_concat, s->xb, dim, heads * v_head, gs);
    for (int i = 0; i < dim; i++) s->x[i] += s->xb[i];
    return 0;
}

/* infer.c:1067-1085: layer 0's dense SwiGLU FFN and its residual. */
static void fw_dense_ffn(const Runtime *rt, RunState *s, int gs) {
    if (!rt->has_l0_ffn) return;
    const int dim = rt->cfg.dim, hid = rt->cfg.hidden_dim;
    fw_rmsnorm(s->xn, s->x, rt->l0_ffn_norm, dim);
    fw_matvec(rt->l0_ffn_gate_q, rt->l0_ffn_gate_s, s->xn, s->ff_gate, hid, dim, gs);
    fw_matvec(rt->l0_ffn_up_q, rt->l0_ffn_up_s, s->xn, s->ff_up, hid, dim, gs);
    for (int i = 0; i < hid; i++) s->ff_gate[i] = fw_silu(s->ff_gate[i]) * s->ff_up[i];
    fw_matvec(rt->l0_ffn_down_q, rt->l0_ffn_down_s, s->ff_gate, s->xb, dim, hid, gs);
    for (int i = 0; i < dim; i++) s->x[i] += s->xb[i];
}

/* MoE layer l on the GPU; the cases infer.c:1088-1092 treats as no layer do nothing. */
static int fw_moe(const Runtime *rt, RunState *s, int l, int debug_mode) {
    if (!rt->has_moe_shared || l <= 0 || l >= rt->cfg.n_layers || rt->cfg.moe_ffn_dim <= 0) return 0;
    if (!rt->moe_layers || !rt->moe_layers[l].ffn_norm) return 0;
    if (glm_hip_moe_layer(rt, s, l, debug_mode) != 0) {
        fprintf(stderr, "[glm-hip] MoE layer %d did not run on the GPU (is glm_backend_init(BACKEND_HIP) done?)\n", l);
        return -1;
    }
    return 0;
}

/* infer.c:1767-1901, with the optional per-layer copies of x after attention and
 * after the FFN. */
static int fw_forward(const Runtime *rt, RunState *s, int token, int pos, int debug_mode, float *attn_out,
                      int attn_stride, int max_attn, int *n_attn, float *layer_out, int layer_stride, int max_layers,
                      int *n_layers) {
    if (!rt || !s) return -1;
    const RuntimeConfig *c = &rt->cfg;
    const int dim = c->dim, gs = (int)c->group_size;
    if (token < 0 || token >= c->vocab_size) token = 0;
    if (n_attn) *n_attn = 0;
    if (n_layers) *n_layers = 0;
    const int keep_attn = attn_out && attn_stride >= dim && max_attn > 0;
    const int keep_layer = layer_out && layer_stride >= dim && max_layers > 0;

    fw_dequant(rt->tok_q + (size_t)token * dim, rt->tok_s + (size_t)token * (dim / gs), s->x, dim, gs);
    const int sums = debug_mode && pos == 0;  // infer.c:1811-1813, 1831-1859, 1885-1895
    if (sums) fw_print_sum("embd", -1, fw_sum(s->x, dim));

    // the three model forms of infer.c:1817-1881: attention in every layer (then the MoE
    // layers run), attention in layer 0 only, or layer 0's FFN alone
    const int n_run = rt->has_all_attn ? c->n_layers : 1;
    for (int l = 0; l < n_run; l++) {
        const float before_attn = sums && rt->has_all_attn ? fw_sum(s->x, dim) : 0.0f;
        float before_ffn = 0.0f;
        if (rt->has_all_attn || rt->has_l0_attn) {
            LayerAttnWeights l0 = {rt->l0_attn_norm, rt->l0_q_a_norm, rt->l0_kv_a_norm, rt->l0_q_a_q, rt->l0_q_a_s,
                                   rt->l0_q_b_q,     rt->l0_q_b_s,    rt->l0_kv_a_q,    rt->l0_kv_a_s, rt->l0_k_b_q,
                                   rt->l0_k_b_s,     rt->l0_v_b_q,    rt->l0_v_b_s,     rt->l0_attn_out_q,
                                   rt->l0_attn_out_s};
            const LayerAttnWeights *w = rt->has_all_attn ? &rt->attn_layers[l] : &l0;
            if (fw_attention(rt, w, s, gs, pos, l) != 0) return -1;
            if (keep_attn && l < max_attn) {
                memcpy(attn_out + (size_t)l * attn_stride, s->x, (size_t)dim * sizeof(float));
                if (n_attn) *n_attn = l + 1;
            }
        }
        if (sums && rt->has_all_attn) {
            fw_print_sum("Vcur", l, fw_sum(s->kv_a, c->kv_lora_rank));
            fw_print_sum("kqv_out", l, fw_sum(s->att_concat, c->n_heads * c->l0_v_head_dim));
            fw_print_sum("ffn_inp", l, fw_sum(s->x, dim));
            fw_print_sum("attn_out", l, fw_sum(s->x, dim) - before_attn);
            before_ffn = fw_sum(s->x, dim);
        }
        if (l == 0) {
            fw_dense_ffn(rt, s, gs);
        } else if (fw_moe(rt, s, l, debug_mode) != 0) {
            return -1;
        }
        if (keep_layer && l < max_layers) {
            memcpy(layer_out + (size_t)l * layer_stride, s->x, (size_t)dim * sizeof(float));
            if (n_layers) *n_layers = l + 1;
        }
        if (sums) {
            fw_print_sum("l_out", l, fw_sum(s->x, dim));
            if (rt->has_all_attn) fw_print_sum("ffn_out", l, fw_sum(s->x, dim) - before_ffn);
        }
    }
    fw_rmsnorm(s->xn, s->x, rt->output_norm, dim);
    if (sums) fw_print_sum("result_norm", -1, fw_sum(s->xn, dim));
    fw_matvec(rt->out_q, rt->out_s, s->xn, s->logits, c->vocab_size, dim, gs);
    if (sums) fw_print_sum("result_output", -1, fw_sum(s->logits, c->vocab_size));
    return 0;
}

/* The GPU model's forward with glm.c's --debug lines: at every position each MoE layer's
 * two sums (infer.c:1207-1210), and at position 0 the per-stage sums of infer.c:1811-1895,
 * from the intermediate vectors the model returns (gmoe_model_forward_token_debug), in
 * glm.c's order. Advances the model's state as glm_hip_forward_token does. */
static int fw_forward_device_debug(const Runtime *rt, RunState *s, int token, int pos) {
    const RuntimeConfig *c = &rt->cfg;
    const int L = c->n_layers, dim = c->dim, gs = (int)c->group_size, kv = c->kv_lora_rank;
    const int hv = c->n_heads * c->l0_v_head_dim;
    const int n_run = rt->has_all_attn ? L : 1;
    float *attn = (float *)calloc((size_t)L * dim, sizeof(float)), *lay = (float *)calloc((size_t)L * dim, sizeof(float));
    float *kvb = (float *)calloc((size_t)L * (kv > 0 ? kv : 1), sizeof(float));
    float *cat = (float *)calloc((size_t)L * (hv > 0 ? hv : 1), sizeof(float));
    float *sh = (float *)calloc((size_t)L * dim, sizeof(float)), *mo = (float *)calloc((size_t)L * dim, sizeof(float));
    float *x0 = (float *)calloc((size_t)dim, sizeof(float));
    int rc = -1;
    if (!attn || !lay || !kvb || !cat || !sh || !mo || !x0) {
        fprintf(stderr, "[glm-hip] out of memory for the debug sums\n");
    } else {
        if (token < 0 || token >= c->vocab_size) token = 0;
        rc = glm_hip_model_forward_sums(s, token, pos, attn, lay, kvb, cat, sh, mo);
    }
    if (rc == 0) {
        const int sums = pos == 0;
        fw_dequant(rt->tok_q + (size_t)token * dim, rt->tok_s + (size_t)token * (dim / gs), x0, dim, gs);
        if (sums) fw_print_sum("embd", -1, fw_sum(x0, dim));
        for (int l = 0; l < n_run; l++) {
            const float *xin = l == 0 ? x0 : lay + (size_t)(l - 1) * dim, *xa = attn + (size_t)l * dim;
            const float *xl = lay + (size_t)l * dim;
            float before_ffn = 0.0f;
            if (sums && rt->has_all_attn) {
                const float before_attn = fw_sum(xin, dim);
                fw_print_sum("Vcur", l, fw_sum(kvb + (size_t)l * kv, kv));
                fw_print_sum("kqv_out", l, fw_sum(cat + (size_t)l * hv, hv));
                fw_print_sum("ffn_inp", l, fw_sum(xa, dim));
                fw_print_sum("attn_out", l, fw_sum(xa, dim) - before_attn);
                before_ffn = fw_sum(xa, dim);
            }
            if (l > 0 && rt->has_moe_shared && rt->moe_layers && rt->moe_layers[l].ffn_norm) {
                fw_print_sum("ffn_moe_out", l, fw_sum(mo + (size_t)l * dim, dim));
                fw_print_sum("ffn_shexp", l, fw_sum(sh + (size_t)l * dim, dim));
            }
            if (sums) {
                fw_print_sum("l_out", l, fw_sum(xl, dim));
                if (rt->has_all_attn) fw_print_sum("ffn_out", l, fw_sum(xl, dim) - before_ffn);
            }
        }
        if (sums) {
            fw_rmsnorm(x0, s->x, rt->output_norm, dim);
            fw_print_sum("result_norm", -1, fw_sum(x0, dim));
            fw_print_sum("result_output", -1, fw_sum(s->logits, c->vocab_size));
        }
    }
    free(attn);
    free(lay);
    free(kvb);
    free(cat);
    free(sh);
    free(mo);
    free(x0);
    return rc;
}

/* The forward on the GPU model (glm_hip_model_forward), with the per-layer copies of x
 * placed at the caller's strides. keep: leave the model's cache and s as they were. */
static int fw_forward_device(const Runtime *rt, RunState *s, int token, int pos, int keep, float *attn_out,
                             int attn_stride, int max_attn, int *n_attn, float *layer_out, int layer_stride,
                             int max_layers, int *n_layers) {
    const RuntimeConfig *c = &rt->cfg;
    const int L = c->n_layers, dim = c->dim;
    const int n_run = rt->has_all_attn ? L : 1, n_att = (rt->has_all_attn || rt->has_l0_attn) ? n_run : 0;
    const int keep_attn = attn_out && attn_stride >= dim && max_attn > 0 && n_att > 0;
    const int keep_layer = layer_out && layer_stride >= dim && max_layers > 0;
    float *ab = keep_attn ? (float *)malloc((size_t)L * dim * sizeof(float)) : NULL;
    float *lb = keep_layer ? (float *)malloc((size_t)L * dim * sizeof(float)) : NULL;
    float *logits = keep ? (float *)malloc((size_t)c->vocab_size * sizeof(float)) : NULL;
    int rc = -1;
    if ((!keep_attn || ab) && (!keep_layer || lb) && (!keep || logits))
        rc = glm_hip_model_forward(rt, s, token, pos, keep, logits, ab, lb);
    else
        fprintf(stderr, "[glm-hip] out of memory for the forward's checkpoints\n");
    if (n_attn) *n_attn = 0;
    if (n_layers) *n_layers = 0;
    if (rc == 0) {
        const int na = keep_attn ? (n_att < max_attn ? n_att : max_attn) : 0;
        const int nl = keep_layer ? (n_run < max_layers ? n_run : max_layers) : 0;
        for (int l = 0; l < na; l++) memcpy(attn_out + (size_t)l * attn_stride, ab + (size_t)l * dim, (size_t)dim * sizeof(float));
        for (int l = 0; l < nl; l++) memcpy(layer_out + (size_t)l * layer_stride, lb + (size_t)l * dim, (size_t)dim * sizeof(float));
        if (n_attn) *n_attn = na;
        if (n_layers) *n_layers = nl;
    }
    free(ab);
    free(lb);
    free(logits);
    return rc;
}

/* ---- public ----------------------------------------------------------------------- */

int glm_hip_forward_token(const Runtime *rt, RunState *st, int token, int pos, int debug_mode) {
    if (rt && st && glm_hip_model_owns(st, pos)) {
        if (debug_mode) return fw_forward_device_debug(rt, st, token, pos);
        return fw_forward_device(rt, st, token, pos, 0, NULL, 0, 0, NULL, NULL, 0, 0, NULL);
    }
    return fw_forward(rt, st, token, pos, debug_mode, NULL, 0, 0, NULL, NULL, 0, 0, NULL);
}

int glm_hip_prefill(const Runtime *rt, RunState *st, const int *tokens, int n, int pos0, int debug_mode) {
    if (!rt || !st || !tokens || n < 1 || pos0 < 0) return -1;
    if (pos0 + n > st->cache_cap) {
        fprintf(stderr, "[glm-hip] prefill of positions %d..%d past the cache (%d positions)\n", pos0, pos0 + n - 1,
                st->cache_cap);
        return -1;
    }
    // with debug_mode, token by token: glm.c prints its per-token sums for prompt tokens too
    if (!debug_mode && glm_hip_model_owns(st, pos0)) return glm_hip_model_prefill(rt, st, tokens, n, pos0);
    for (int i = 0; i < n; i++) {
        int tok = tokens[i];
        if (tok < 0 || tok >= rt->cfg.vocab_size) tok = 0;  // infer.c:2220
        if (glm_hip_forward_token(rt, st, tok, pos0 + i, debug_mode) != 0) return -1;
    }
    return 0;
}

int glm_hip_forward_token_dual_checkpoints(const Runtime *rt, const RunState *src, int token, int pos, int debug_mode,
                                           float *attn_layer_out, int attn_layer_stride, int max_attn_layers,
                                           int *written_attn_layers, float *layer_out, int layer_stride, int max_layers,
                                           int *written_layers) {
    if (!rt || !src || src->cache_cap <= 0) return -1;
    if (attn_layer_out && (attn_layer_stride < rt->cfg.dim || max_attn_layers <= 0)) return -1;
    if (layer_out && (layer_stride < rt->cfg.dim || max_layers <= 0)) return -1;
    // src's history on the device (the GPU model restores what the token writes, so no copy
    // of src is needed); any other state's history is its host cache, on a copy
    if (glm_hip_model_owns(src, pos))
        return fw_forward_device(rt, (RunState *)src, token, pos, 1, attn_layer_out, attn_layer_stride, max_attn_layers,
                                 written_attn_layers, layer_out, layer_stride, max_layers, written_layers);
    RunState tmp;
    if (glm_runstate_build(&tmp, rt, src->cache_cap) != 0) return -1;
    glm_runstate_copy(rt, src, &tmp);
    int na = 0, nl = 0;
    const int rc = fw_forward(rt, &tmp, token, pos, debug_mode, attn_layer_out, attn_layer_stride, max_attn_layers, &na,
                              layer_out, layer_stride, max_layers, &nl);
    if (written_attn_layers) *written_attn_layers = na;
    if (written_layers) *written_layers = nl;
    glm_runstate_free(&tmp);
    return rc;
}

int glm_hip_forward_token_checkpoints(const Runtime *rt, const RunState *src, int token, int pos, int debug_mode,
                                      float *layer_out, int layer_stride, int max_layers, int *written_layers) {
    if (!layer_out || layer_stride < (rt ? rt->cfg.dim : 1) || max_layers <= 0) return -1;
    return glm_hip_forward_token_dual_checkpoints(rt, src, token, pos, debug_mode, NULL, 0, 0, NULL, layer_out,
                                                  layer_stride, max_layers, written_layers);
}

int glm_argmax(const float *x, int n) {
    int best = 0;
    for (int i = 1; i < n; i++)
        if (x[i] > x[best]) best = i;
    return best;
}

/* ---- RunState --------------------------------------------------------------------- */

void glm_runstate_free(RunState *s) {
    if (!s) return;
    glm_hip_model_forget(s);
    void *bufs[] = {s->x,       s->xn,          s->xb,         s->ff_gate,  s->ff_up,      s->logits,     s->k_cache_comp,
                    s->k_cache_pe, s->q_a,      s->q_full,     s->kv_a,     s->q_nope,     s->q_pe,       s->q_abs,
                    s->att_scores, s->att_ctx,  s->att_concat, s->moe_gate, s->moe_up,     s->moe_router, s->moe_out_acc,
                    s->moe_topk_idx, s->moe_topk_w};
    for (size_t i = 0; i < sizeof(bufs) / sizeof(bufs[0]); i++) free(bufs[i]);
    memset(s, 0, sizeof(*s));
}

static void *fw_zeros(size_t n, size_t size, int *ok) {
    void *p = calloc(n ? n : 1, size);
    if (!p) *ok = 0;
    return p;
}

int glm_runstate_build(RunState *s, const Runtime *rt, int cache_cap) {
    if (!s || !rt) return -1;
    memset(s, 0, sizeof(*s));
    const RuntimeConfig *c = &rt->cfg;
    int ok = 1;
    s->x = fw_zeros((size_t)c->dim, sizeof(float), &ok);
    s->xn = fw_zeros((size_t)c->dim, sizeof(float), &ok);
    s->xb = fw_zeros((size_t)c->dim, sizeof(float), &ok);
    s->ff_gate = fw_zeros((size_t)c->hidden_dim, sizeof(float), &ok);
    s->ff_up = fw_zeros((size_t)c->hidden_dim, sizeof(float), &ok);
    s->logits = fw_zeros((size_t)c->vocab_size, sizeof(float), &ok);
    s->cache_cap = cache_cap;
    s->n_attn_layers = rt->has_all_attn ? c->n_layers : (rt->has_l0_attn ? 1 : 0);
    if (s->n_attn_layers > 0) {
        const size_t slots = (size_t)s->n_attn_layers * (size_t)cache_cap;
        s->k_cache_comp = fw_zeros(slots * (size_t)c->kv_lora_rank, sizeof(float), &ok);
        s->k_cache_pe = fw_zeros(slots * (size_t)c->rope_dim, sizeof(float), &ok);
        s->q_a = fw_zeros((size_t)c->q_lora_rank, sizeof(float), &ok);
        s->q_full = fw_zeros((size_t)c->n_heads * (size_t)c->l0_head_k_dim, sizeof(float), &ok);
        s->kv_a = fw_zeros((size_t)(c->kv_lora_rank + c->rope_dim), sizeof(float), &ok);
        s->q_nope = fw_zeros((size_t)c->l0_qk_nope_dim, sizeof(float), &ok);
        s->q_pe = fw_zeros((size_t)c->rope_dim, sizeof(float), &ok);
        s->q_abs = fw_zeros((size_t)c->kv_lora_rank, sizeof(float), &ok);
        s->att_scores = fw_zeros((size_t)cache_cap, sizeof(float), &ok);
        s->att_ctx = fw_zeros((size_t)c->kv_lora_rank, sizeof(float), &ok);
        s->att_concat = fw_zeros((size_t)c->n_heads * (size_t)c->l0_v_head_dim, sizeof(float), &ok);
    }
    if (rt->has_moe_shared && c->moe_ffn_dim > 0) {
        s->moe_gate = fw_zeros((size_t)c->moe_ffn_dim, sizeof(float), &ok);
        s->moe_up = fw_zeros((size_t)c->moe_ffn_dim, sizeof(float), &ok);
        s->moe_router = fw_zeros((size_t)c->n_routed_experts, sizeof(float), &ok);
        s->moe_out_acc = fw_zeros((size_t)c->dim, sizeof(float), &ok);
        s->moe_topk_idx = fw_zeros((size_t)c->n_experts_used, sizeof(int), &ok);
        s->moe_topk_w = fw_zeros((size_t)c->n_experts_used, sizeof(float), &ok);
    }
    if (!ok) {
        fprintf(stderr, "[glm-hip] out of memory for the run state (cache of %d positions)\n", cache_cap);
        glm_runstate_free(s);
        return -1;
    }
    return 0;
}

void glm_runstate_copy(const Runtime *rt, const RunState *src, RunState *dst) {
    if (!rt || !src || !dst) return;
    const RuntimeConfig *c = &rt->cfg;
#define FW_COPY(f, n) \
    if (src->f && dst->f) memcpy(dst->f, src->f, (size_t)(n) * sizeof(*src->f))
    FW_COPY(x, c->dim);
    FW_COPY(xn, c->dim);
    FW_COPY(xb, c->dim);
    FW_COPY(ff_gate, c->hidden_dim);
    FW_COPY(ff_up, c->hidden_dim);
    FW_COPY(logits, c->vocab_size);
    if (src->n_attn_layers > 0) {
        const size_t slots = (size_t)src->n_attn_layers * (size_t)src->cache_cap;
        FW_COPY(k_cache_comp, slots * (size_t)c->kv_lora_rank);
        FW_COPY(k_cache_pe, slots * (size_t)c->rope_dim);
        FW_COPY(q_a, c->q_lora_rank);
        FW_COPY(q_full, (size_t)c->n_heads * (size_t)c->l0_head_k_dim);
        FW_COPY(kv_a, c->kv_lora_rank + c->rope_dim);
        FW_COPY(q_nope, c->l0_qk_nope_dim);
        FW_COPY(q_pe, c->rope_dim);
        FW_COPY(q_abs, c->kv_lora_rank);
        FW_COPY(att_scores, src->cache_cap);
        FW_COPY(att_ctx, c->kv_lora_rank);
        FW_COPY(att_concat, (size_t)c->n_heads * (size_t)c->l0_v_head_dim);
    }
    FW_COPY(moe_gate, c->moe_ffn_dim);
    FW_COPY(moe_up, c->moe_ffn_dim);
    FW_COPY(moe_router, c->n_routed_experts);
    FW_COPY(moe_out_acc, c->dim);
    FW_COPY(moe_topk_idx, c->n_experts_used);
    FW_COPY(moe_topk_w, c->n_experts_used);
#undef FW_COPY
}
