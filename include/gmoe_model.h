/*
 * gmoe_model.h -- glm.c's whole decode forward (infer.c:1767-1901) on one GPU: the
 * embedding row, every layer's MLA attention over a latent cache kept in device memory
 * (infer.c:978-1065), layer 0's dense FFN (infer.c:1067-1085), the MoE layers through a
 * gmoe_ctx (gmoe.h), the final norm and the LM head. x, the cache and every weight stay
 * in device memory; a token's call moves its logits to the host and nothing else.
 *
 * No counterpart in the reference, whose forward is host code: this is the device side
 * of glm_hip_forward_token (glm_forward.h) when the HIP backend runs the whole model.
 * Return codes and gmoe_last_error() as in gmoe.h.
 */
#ifndef GMOE_MODEL_H
#define GMOE_MODEL_H

#include <stdint.h>

#include "gmoe.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gmoe_model gmoe_model;

/* The RuntimeConfig fields the forward reads (model.h:7-45, infer.c:983-991). */
typedef struct gmoe_model_config {
    int32_t dim, hidden_dim, n_layers, n_heads, vocab_size;
    int32_t q_lora_rank, kv_lora_rank, rope_dim, qk_nope_dim, head_k_dim, v_head_dim;
    int32_t group_size;     /* Q8_0 group: a multiple of 16 dividing every column count */
    int32_t cache_cap;      /* latent-cache positions per attention layer, <= 65536 */
    int32_t attn_layers;    /* layers with attention: n_layers (has_all_attn), 1 (layer 0 only) or 0 */
    int32_t has_l0_ffn;     /* layer 0's dense FFN is present */
    int32_t max_batch;      /* most tokens of one gmoe_model_prefill call (0 or 1: one) */
} gmoe_model_config;

/* One layer's attention tensors, in LayerAttnWeights order (model.h:47-63). */
typedef struct gmoe_attn_weights {
    const float *attn_norm, *q_a_norm, *kv_a_norm;
    const int8_t *q_a_q;
    const float *q_a_s;
    const int8_t *q_b_q;
    const float *q_b_s;
    const int8_t *kv_a_q;
    const float *kv_a_s;
    const int8_t *k_b_q;
    const float *k_b_s;
    const int8_t *v_b_q;
    const float *v_b_s;
    const int8_t *attn_out_q;
    const float *attn_out_s;
} gmoe_attn_weights;

/* The model-wide tensors (Runtime, model.h:86-118); the l0_* ones when has_l0_ffn. */
typedef struct gmoe_model_weights {
    const float *output_norm;
    const int8_t *tok_q;
    const float *tok_s;
    const int8_t *out_q;
    const float *out_s;
    const float *l0_ffn_norm;
    const int8_t *l0_ffn_gate_q;
    const float *l0_ffn_gate_s;
    const int8_t *l0_ffn_up_q;
    const float *l0_ffn_up_s;
    const int8_t *l0_ffn_down_q;
    const float *l0_ffn_down_s;
} gmoe_model_weights;

/* Device buffers for cfg on `device`; the weights come with the upload calls. */
int gmoe_model_create(gmoe_model **out, int device, const gmoe_model_config *cfg);
void gmoe_model_destroy(gmoe_model *m);

/* Copies the tensors to the device (each call replaces what an earlier one set). */
int gmoe_model_upload(gmoe_model *m, const gmoe_model_weights *w);
int gmoe_model_upload_attn(gmoe_model *m, int layer, const gmoe_attn_weights *w);

/* The MoE layers: layer l (1 <= l < n_layers) runs through `moe` (created for the same
 * dim and n_layers, its layer l uploaded) when layers[l] is nonzero. moe_flags as in
 * gmoe_forward. The context stays the caller's; the model's calls use its workspace (a
 * token's MoE layers on k_moe_relay share one reset, each on a workspace layer of its
 * own), so they must not overlap the caller's own calls on the context. */
int gmoe_model_set_moe(gmoe_model *m, gmoe_ctx *moe, const uint8_t *layers, int moe_flags);

/* One token at position pos (< cache_cap) through the model, on `stream`, then a
 * synchronisation: logits (vocab_size floats, host) and optionally x after the final
 * layer (x_out, dim floats, host). With attn_ckpt / layer_ckpt (host, [n_layers][dim]),
 * x after each layer's attention / FFN as glm.c's dual checkpoints record it
 * (infer.c:1940-1983). With GMOE_MODEL_KEEP_CACHE the cache entries the token writes are
 * restored afterwards, so the call leaves the model's state as it was. */
#define GMOE_MODEL_KEEP_CACHE 1
int gmoe_model_forward_token(gmoe_model *m, int token, int pos, int flags, float *logits, float *x_out,
                             float *attn_ckpt, float *layer_ckpt, void *stream);

/* gmoe_model_forward_token that also returns what glm.c's --debug sums at position 0
 * (infer.c:1832-1858, 1207-1210), per layer l, into host buffers (any may be NULL):
 * kv_out + l*kv_lora_rank the normalised kv entry of the position (glm.c's kv_a),
 * concat_out + l*n_heads*v_head_dim the heads' attention outputs (att_concat), and for MoE
 * layers shexp_out + l*dim the shared expert's output (xb) and moe_out + l*dim the routed
 * combine (moe_out_acc). */
int gmoe_model_forward_token_debug(gmoe_model *m, int token, int pos, int flags, float *logits, float *x_out,
                                   float *attn_ckpt, float *layer_ckpt, float *kv_out, float *concat_out,
                                   float *shexp_out, float *moe_out, void *stream);

/* n tokens at positions pos0 .. pos0+n-1 (n <= max_batch, pos0 + n <= cache_cap) through the
 * model at once, layer by layer, then a synchronisation: the same result as n calls of
 * gmoe_model_forward_token in order (the latent cache gains the n positions), but every
 * product over the batch in one launch, and each MoE layer one gmoe_forward over the n
 * tokens (the grouped expert GEMMs over per-expert token lists). glm.c prefills a prompt
 * token by token (infer.c:2190-2233); this is the batched form of that loop. logits (host,
 * vocab_size floats) are the last token's, and optionally x_out (host, dim floats) its x
 * after the final layer. The MoE context must take n tokens (gmoe_config.max_tokens >= n). */
int gmoe_model_prefill(gmoe_model *m, const int32_t *tokens, int n, int pos0, float *logits, float *x_out,
                       void *stream);

/* Positions pos0 .. pos0+n-1 of attention layer `layer`'s latent cache (host buffers, then
 * a synchronisation): comp_out [n][kv_lora_rank] and pe_out [n][rope_dim] (either may be
 * NULL), the entries glm.c keeps in RunState.k_cache_comp / k_cache_pe (infer.c:1012-1017,
 * the rope part rotated). For callers that check or hand over the decode state. */
int gmoe_model_read_cache(gmoe_model *m, int layer, int pos0, int n, float *comp_out, float *pe_out, void *stream);

#ifdef __cplusplus
}
#endif

#endif
