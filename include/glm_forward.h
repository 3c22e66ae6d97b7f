/*
 * glm_forward.h -- glm.c's token forward (infer.c:1767-1901) for the --backend hip
 * drop-in, and the RunState it runs on.
 *
 * glm_hip_forward_token takes one token at one position through the whole model:
 * embedding, each layer's MLA attention, layer 0's dense FFN, every MoE FFN layer,
 * the final norm and the LM head, leaving the logits in st->logits. The MoE layers
 * run on the GPU through libgmoe.so (glm_hip_moe_layer); the rest runs on the host
 * with glm.c's own arithmetic. glm_backend_init(BACKEND_HIP, ...) must have
 * succeeded first unless the checkpoint has no MoE layer.
 *
 * Each function keeps the signature, argument meaning and return convention of the
 * glm.c function named beside it (0 on success, -1 on failure); where glm.c calls
 * die() (a position past the cache, an allocation failure) these print a "[glm-hip]"
 * message and return -1.
 */
#ifndef GLM_FORWARD_H
#define GLM_FORWARD_H

#include "glm_model.h"

#ifdef __cplusplus
extern "C" {
#endif

/* runstate_build (infer.c:827-860): every buffer of st for rt, with a latent cache of
 * cache_cap positions per attention layer, zeroed. 0, or -1 with st left empty. */
int glm_runstate_build(RunState *st, const Runtime *rt, int cache_cap);
/* runstate_free (infer.c:803-826). */
void glm_runstate_free(RunState *st);
/* runstate_copy_from (infer.c:861-898): dst (built for the same rt and cache_cap) := src. */
void glm_runstate_copy(const Runtime *rt, const RunState *src, RunState *dst);

/* glm_cpu_forward_token (infer.c:1903-1905). */
int glm_hip_forward_token(const Runtime *rt, RunState *st, int token, int pos, int debug_mode);

/* The prompt loop of infer.c:2190-2219 for n prompt tokens at positions pos0 .. pos0+n-1:
 * the same state as n glm_hip_forward_token calls in order (the cache gains the n
 * positions, st->logits and st->x are the last token's; a token outside the vocabulary is
 * taken as 0, infer.c:2220). With the GPU model the tokens go through it in batches
 * (gmoe_model_prefill, GLM_HIP_PREFILL_BATCH tokens at a time), every layer's products and
 * MoE experts over the whole batch; otherwise token by token. 0, or -1. */
int glm_hip_prefill(const Runtime *rt, RunState *st, const int *tokens, int n, int pos0, int debug_mode);

/* glm_cpu_forward_token_checkpoints (infer.c:1907-1938): the forward on a copy of src
 * (src is left as it was), writing x after each layer's FFN to layer_out + l*layer_stride
 * for l < max_layers. */
int glm_hip_forward_token_checkpoints(const Runtime *rt, const RunState *src, int token, int pos, int debug_mode,
                                      float *layer_out, int layer_stride, int max_layers, int *written_layers);

/* glm_cpu_forward_token_dual_checkpoints (infer.c:1940-1983): as above, also writing x
 * after each layer's attention to attn_layer_out (either output may be NULL). */
int glm_hip_forward_token_dual_checkpoints(const Runtime *rt, const RunState *src, int token, int pos, int debug_mode,
                                           float *attn_layer_out, int attn_layer_stride, int max_attn_layers,
                                           int *written_attn_layers, float *layer_out, int layer_stride, int max_layers,
                                           int *written_layers);

/* argmax (infer.c:1218-1228): the first index of the largest value. */
int glm_argmax(const float *x, int n);

#ifdef __cplusplus
}
#endif

#endif
