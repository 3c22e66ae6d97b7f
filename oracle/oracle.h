/*
 * ORACLE -- test infrastructure only. Nothing in the product (libgmoe.so,
 * libglm_hip.so) may include, link or call this. Only tests/, the smoke() check
 * and bench.py's CPU-baseline leg use it, and only as the checker.
 *
 * Two implementations share this interface:
 *   oracle/moe_oracle.c  -> oracle/liboracle.so    CPU restatement of glm.c's MoE path
 *   oracle/ref_harness.c -> oracle/_ref/libref_moe.so   glm.c's own infer.c, compiled
 *                           from the reference sources by oracle/Makefile
 * `prefix` is oracle_ or ref_.
 */
#ifndef GLM_ORACLE_H
#define GLM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct oracle_dims {
    int32_t dim;               /* D */
    int32_t moe_ffn_dim;       /* F */
    int32_t n_routed_experts;  /* E */
    int32_t n_experts_used;    /* K */
    int32_t group_size;        /* gs */
} oracle_dims;

/* One MoE layer in checkpoint layout (LayerMoeShared then LayerMoeRouted, model.h:65-84). */
typedef struct oracle_layer {
    const float *ffn_norm, *gate_inp, *exp_probs_b;
    const int8_t *gate_sh_q; const float *gate_sh_s;
    const int8_t *up_sh_q; const float *up_sh_s;
    const int8_t *down_sh_q; const float *down_sh_s;
    const int8_t *gate_q; const float *gate_s;
    const int8_t *up_q; const float *up_s;
    const int8_t *down_q; const float *down_s;
} oracle_layer;

/* Outputs for T tokens; any pointer may be NULL. */
typedef struct oracle_out {
    float *x_out;        /* [T][D] */
    float *xn;           /* [T][D] */
    float *router_prob;  /* [T][E] */
    int32_t *topk_idx;   /* [T][K] */
    float *topk_w;       /* [T][K] */
    float *shared_out;   /* [T][D] */
    float *routed_out;   /* [T][D] */
} oracle_out;

/* Each of the T tokens runs one apply_moe_shared_ffn_layer (infer.c:1087-1216)
 * independently, as the reference's token loop does (infer.c:2190-2233). */
int oracle_moe_layer(const oracle_dims *d, const oracle_layer *w, int T, const float *x_in,
                     const oracle_out *out, int disable_routed);
int ref_moe_layer(const oracle_dims *d, const oracle_layer *w, int T, const float *x_in,
                  const oracle_out *out, int disable_routed);

/* n_layers MoE layers in sequence for T tokens (the FFN half of infer.c:1818-1860).
 * x is [T][D], updated in place; topk_idx, if not NULL, is [n_layers][T][K]. */
int oracle_moe_stack(const oracle_dims *d, const oracle_layer *layers, int n_layers, int T, float *x,
                     int32_t *topk_idx);
int ref_moe_stack(const oracle_dims *d, const oracle_layer *layers, int n_layers, int T, float *x,
                  int32_t *topk_idx);

/* CPU-baseline timing (reference build only): n_tokens decode tokens through the stack
 * from x, every layer call timed with glm.c's monotonic_ms (infer.c:1426-1430) into
 * layer_ms[n_tokens][n_layers]; and T tokens through one layer, one timed call each
 * (token_ms[T]). n_threads > 0 sets the OpenMP team size first. */
int ref_moe_stack_timed(const oracle_dims *d, const oracle_layer *layers, int n_layers, int n_tokens, float *x,
                        double *layer_ms, int n_threads);
int ref_moe_layer_timed(const oracle_dims *d, const oracle_layer *w, int T, const float *x_in, double *token_ms,
                        int n_threads);

/* Per-expert token lists derived from [T][K] top-k indices: expert e owns
 * tokens[offsets[e] .. offsets[e+1]) in ascending token order, and slots[]
 * holds the top-k slot each entry came from. Returns the number of entries. */
int oracle_dispatch(int T, int K, int E, const int32_t *topk_idx, int32_t *offsets, int32_t *tokens,
                    int32_t *slots);

/* Pieces of the layer, exposed so tests can pin each one on its own. */
void oracle_rmsnorm(float *out, const float *x, const float *w, int n);
void oracle_router_logits(const float *gate_inp, const float *xn, float *logits, int E, int D);
float oracle_sigmoid(float logit);
float oracle_silu(float x);
void oracle_topk(const float *prob, const float *bias, int E, int K, int32_t *idx, float *w);
void oracle_matvec_q8(const int8_t *q, const float *s, const float *x, float *y, int rows, int cols, int gs);

/* The C library's expf on the fp32 inputs first, first + 1, ... against `got`: the
 * number of inputs more than max_ulp apart, the first one's bit pattern in *first_bad. */
int64_t oracle_expf_compare(uint32_t first, int64_t count, const float *got, int max_ulp, int64_t *first_bad);

#ifdef __cplusplus
}
#endif

#endif
