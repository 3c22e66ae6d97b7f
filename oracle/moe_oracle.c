/*
 * ORACLE -- test infrastructure only (see oracle.h). CPU restatement of glm.c's
 * MoE FFN hot path, arithmetic for arithmetic:
 *   oracle_rmsnorm        infer.c:746-752
 *   oracle_matvec_q8      infer.c:765-786   (same OpenMP row split and per-group simd dot)
 *   oracle_silu           infer.c:912-914
 *   oracle_router_logits  infer.c:916-938   (no-BLAS branch: one sequential fp32 chain per expert)
 *   oracle_sigmoid        infer.c:1104-1106
 *   oracle_topk           infer.c:1108-1145 (insertion top-k, ties to the lower index, normalise)
 *   oracle_moe_layer      infer.c:1087-1216
 *   oracle_dispatch       derived lists: the reference routes token by token and never builds them
 * Build flags follow the reference Makefile (Makefile:1-2: -O3, no -march, so no FMA
 * contraction on x86-64) plus -ffp-contract=off to keep that true on any host.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define ROUTED_SCALE 1.8f           /* infer.c:1171 */
#define NORM_EPS 1e-5f              /* infer.c:750 */
#define MIN_TOPK_DENOM 6.103515625e-5f /* infer.c:1141, smallest fp16 normal */

void oracle_rmsnorm(float *out, const float *x, const float *w, int n) {
    double sumsq = 0.0;
    for (int i = 0; i < n; i++) {
        double v = (double)x[i];
        sumsq += v * v;
    }
    const float mean_sq = (float)(sumsq / (double)n);
    const float scale = 1.0f / sqrtf(mean_sq + NORM_EPS);
    for (int i = 0; i < n; i++) out[i] = (x[i] * scale) * w[i];
}

void oracle_matvec_q8(const int8_t *q, const float *s, const float *x, float *y, int rows, int cols, int gs) {
    const int groups = cols / gs;
#if defined(_OPENMP)
#pragma omp parallel for schedule(static) if (rows >= 64)
#endif
    for (int r = 0; r < rows; r++) {
        const int8_t *qr = q + (size_t)r * cols;
        const float *sr = s + (size_t)r * groups;
        float acc = 0.0f;
        for (int g = 0; g < groups; g++) {
            const int8_t *qg = qr + (size_t)g * gs;
            const float *xg = x + (size_t)g * gs;
            float part = 0.0f;
#if defined(_OPENMP)
#pragma omp simd reduction(+ : part)
#endif
            for (int k = 0; k < gs; k++) part += (float)qg[k] * xg[k];
            acc += sr[g] * part;
        }
        y[r] = acc;
    }
}

float oracle_silu(float v) { return v / (1.0f + expf(-v)); }

float oracle_sigmoid(float logit) { return 1.0f / (1.0f + expf(-logit)); }

void oracle_router_logits(const float *gate_inp, const float *xn, float *logits, int E, int D) {
    for (int e = 0; e < E; e++) {
        const float *row = gate_inp + (size_t)e * D;
        float chain = 0.0f;
        for (int i = 0; i < D; i++) chain += row[i] * xn[i];
        logits[e] = chain;
    }
}

void oracle_topk(const float *prob, const float *bias, int E, int K, int32_t *idx, float *w) {
    for (int k = 0; k < K; k++) {
        idx[k] = -1;
        w[k] = -1e30f;
    }
    for (int e = 0; e < E; e++) {
        const float p = prob[e];
        const float score = p + bias[e];
        int at = -1;
        for (int k = 0; k < K && at < 0; k++) {
            const int j = idx[k];
            const float held = (j >= 0) ? prob[j] + bias[j] : -INFINITY;
            if (score > held) at = k;
        }
        if (at < 0) continue;
        for (int k = K - 1; k > at; k--) {
            idx[k] = idx[k - 1];
            w[k] = w[k - 1];
        }
        idx[at] = e;
        w[at] = p;
    }
    float total = 0.0f;
    for (int k = 0; k < K; k++)
        if (idx[k] >= 0) total += w[k];
    if (total > 0.0f) {
        const float denom = total < MIN_TOPK_DENOM ? MIN_TOPK_DENOM : total;
        const float inv = 1.0f / denom;
        for (int k = 0; k < K; k++) w[k] *= inv;
    }
}

typedef struct {
    float *xn, *router, *gate, *up, *xb, *acc;
    int32_t *idx;
    float *w;
} scratch_t;

static int scratch_alloc(scratch_t *s, const oracle_dims *d) {
    const int D = d->dim, F = d->moe_ffn_dim, E = d->n_routed_experts, K = d->n_experts_used;
    memset(s, 0, sizeof(*s));
    s->xn = (float *)calloc((size_t)D, sizeof(float));
    s->router = (float *)calloc((size_t)E, sizeof(float));
    s->gate = (float *)calloc((size_t)F, sizeof(float));
    s->up = (float *)calloc((size_t)F, sizeof(float));
    s->xb = (float *)calloc((size_t)D, sizeof(float));
    s->acc = (float *)calloc((size_t)D, sizeof(float));
    s->idx = (int32_t *)calloc((size_t)K, sizeof(int32_t));
    s->w = (float *)calloc((size_t)K, sizeof(float));
    return (s->xn && s->router && s->gate && s->up && s->xb && s->acc && s->idx && s->w) ? 0 : -1;
}

static void scratch_free(scratch_t *s) {
    free(s->xn);
    free(s->router);
    free(s->gate);
    free(s->up);
    free(s->xb);
    free(s->acc);
    free(s->idx);
    free(s->w);
}

/* Swiglu expert: xb = down(silu(gate xn) * up xn). */
static void expert_ffn(const oracle_dims *d, const int8_t *gq, const float *gsc, const int8_t *uq, const float *usc,
                       const int8_t *dq, const float *dsc, scratch_t *s) {
    const int D = d->dim, F = d->moe_ffn_dim, gs = d->group_size;
    oracle_matvec_q8(gq, gsc, s->xn, s->gate, F, D, gs);
    oracle_matvec_q8(uq, usc, s->xn, s->up, F, D, gs);
    for (int i = 0; i < F; i++) s->gate[i] = oracle_silu(s->gate[i]) * s->up[i];
    oracle_matvec_q8(dq, dsc, s->gate, s->xb, D, F, gs);
}

/* One token through one layer; x is updated in place. */
static void layer_token(const oracle_dims *d, const oracle_layer *w, float *x, scratch_t *s, int disable_routed) {
    const int D = d->dim, F = d->moe_ffn_dim, E = d->n_routed_experts, K = d->n_experts_used, gs = d->group_size;
    oracle_rmsnorm(s->xn, x, w->ffn_norm, D);
    oracle_router_logits(w->gate_inp, s->xn, s->router, E, D);
    for (int e = 0; e < E; e++) s->router[e] = oracle_sigmoid(s->router[e]);
    oracle_topk(s->router, w->exp_probs_b, E, K, s->idx, s->w);

    memset(s->acc, 0, (size_t)D * sizeof(float));
    if (!disable_routed && w->gate_q) {
        const size_t mq = (size_t)F * D;
        const size_t dsg = (size_t)F * (D / gs); /* scales per gate/up expert */
        const size_t usg = (size_t)D * (F / gs); /* scales per down expert */
        for (int k = 0; k < K; k++) {
            const int e = s->idx[k];
            if (e < 0) continue;
            const float we = s->w[k] * ROUTED_SCALE;
            expert_ffn(d, w->gate_q + e * mq, w->gate_s + e * dsg, w->up_q + e * mq, w->up_s + e * dsg, w->down_q + e * mq,
                       w->down_s + e * usg, s);
            for (int i = 0; i < D; i++) s->acc[i] += we * s->xb[i];
        }
    }
    expert_ffn(d, w->gate_sh_q, w->gate_sh_s, w->up_sh_q, w->up_sh_s, w->down_sh_q, w->down_sh_s, s);
    for (int i = 0; i < D; i++) x[i] += s->xb[i] + s->acc[i];
}

int oracle_moe_layer(const oracle_dims *d, const oracle_layer *w, int T, const float *x_in, const oracle_out *out,
                     int disable_routed) {
    if (!d || !w || !x_in || !out || T < 0) return -1;
    const int D = d->dim, E = d->n_routed_experts, K = d->n_experts_used;
    scratch_t s;
    if (scratch_alloc(&s, d) != 0) {
        scratch_free(&s);
        return -1;
    }
    float *x = (float *)malloc((size_t)D * sizeof(float));
    if (!x) {
        scratch_free(&s);
        return -1;
    }
    for (int t = 0; t < T; t++) {
        memcpy(x, x_in + (size_t)t * D, (size_t)D * sizeof(float));
        layer_token(d, w, x, &s, disable_routed);
        if (out->x_out) memcpy(out->x_out + (size_t)t * D, x, (size_t)D * sizeof(float));
        if (out->xn) memcpy(out->xn + (size_t)t * D, s.xn, (size_t)D * sizeof(float));
        if (out->router_prob) memcpy(out->router_prob + (size_t)t * E, s.router, (size_t)E * sizeof(float));
        if (out->topk_idx) memcpy(out->topk_idx + (size_t)t * K, s.idx, (size_t)K * sizeof(int32_t));
        if (out->topk_w) memcpy(out->topk_w + (size_t)t * K, s.w, (size_t)K * sizeof(float));
        if (out->shared_out) memcpy(out->shared_out + (size_t)t * D, s.xb, (size_t)D * sizeof(float));
        if (out->routed_out) memcpy(out->routed_out + (size_t)t * D, s.acc, (size_t)D * sizeof(float));
    }
    free(x);
    scratch_free(&s);
    return 0;
}

int oracle_moe_stack(const oracle_dims *d, const oracle_layer *layers, int n_layers, int T, float *x,
                     int32_t *topk_idx) {
    if (!d || !layers || !x || n_layers < 0 || T < 0) return -1;
    const int D = d->dim, K = d->n_experts_used;
    scratch_t s;
    if (scratch_alloc(&s, d) != 0) {
        scratch_free(&s);
        return -1;
    }
    for (int t = 0; t < T; t++) {
        for (int l = 0; l < n_layers; l++) {
            layer_token(d, &layers[l], x + (size_t)t * D, &s, 0);
            if (topk_idx) memcpy(topk_idx + ((size_t)l * T + t) * K, s.idx, (size_t)K * sizeof(int32_t));
        }
    }
    scratch_free(&s);
    return 0;
}

int oracle_dispatch(int T, int K, int E, const int32_t *topk_idx, int32_t *offsets, int32_t *tokens, int32_t *slots) {
    if (T < 0 || K <= 0 || E <= 0 || !topk_idx || !offsets) return -1;
    for (int e = 0; e <= E; e++) offsets[e] = 0;
    for (int t = 0; t < T; t++)
        for (int k = 0; k < K; k++) {
            int e = topk_idx[(size_t)t * K + k];
            if (e >= 0 && e < E) offsets[e + 1]++;
        }
    for (int e = 0; e < E; e++) offsets[e + 1] += offsets[e];
    int *fill = (int *)calloc((size_t)E, sizeof(int));
    if (!fill) return -1;
    for (int t = 0; t < T; t++)
        for (int k = 0; k < K; k++) {
            int e = topk_idx[(size_t)t * K + k];
            if (e < 0 || e >= E) continue;
            int at = offsets[e] + fill[e]++;
            if (tokens) tokens[at] = t;
            if (slots) slots[at] = k;
        }
    free(fill);
    return offsets[E];
}

/* glm.c's sigmoid calls the C library's expf (infer.c:1105). Compares `got` (a device
 * expf on the inputs with bit patterns first, first + 1, ...) against this libm's expf:
 * returns the number of inputs more than max_ulp apart (max_ulp 0: bitwise; NaN matches
 * NaN) and, in *first_bad, the bit pattern of the first such input (or -1). */
int64_t oracle_expf_compare(uint32_t first, int64_t count, const float *got, int max_ulp, int64_t *first_bad) {
    int64_t bad = 0, where = INT64_MAX;
#pragma omp parallel for schedule(static) reduction(+ : bad) reduction(min : where)
    for (int64_t i = 0; i < count; i++) {
        const uint32_t u = first + (uint32_t)i;
        float x;
        memcpy(&x, &u, 4);
        const float want = expf(x), g = got[i];
        int ok;
        if (want != want || g != g) {
            ok = (want != want) && (g != g);
        } else {
            uint32_t a, b;
            memcpy(&a, &want, 4);
            memcpy(&b, &g, 4);
            /* expf is never negative: bit patterns order as values */
            const int64_t dist = (int64_t)a - (int64_t)b;
            ok = (dist < 0 ? -dist : dist) <= max_ulp;
        }
        if (!ok) {
            bad++;
            if (i < where) where = i;
        }
    }
    if (first_bad) *first_bad = bad ? (int64_t)(uint32_t)(first + (uint32_t)where) : -1;
    return bad;
}
