/*
 * glm_backend.h -- glm.c's backend interface (backend.h:1-15) with a HIP backend.
 *
 * The first three functions keep the signatures and contracts of backend.h:7-9:
 *   glm_backend_init     returns the "use gpu" handle (0 = CPU, BACKEND_HIP = HIP) and
 *                        exits the process when the requested backend cannot start,
 *                        as backend.c:73-86 does for Metal;
 *   glm_backend_forward_token  0 on success, nonzero on failure (backend.c:88-91); with
 *                        BACKEND_HIP it runs glm_hip_forward_token (glm_forward.h), with
 *                        0 glm.c's own glm_cpu_forward_token when that is linked in;
 *   glm_backend_free.
 * glm_backend_try_hip_moe is the HIP counterpart of the per-op offload hook
 * glm_backend_try_metal_matvec (backend.h:13, called at infer.c:793): it runs one
 * whole MoE FFN layer (infer.c:1087-1216) on the GPU and returns 0, or returns -1 so
 * that the caller runs apply_moe_shared_ffn_layer on the CPU.
 * The glm_hip_* functions follow the backend-private pattern of backend.c:9-14.
 */
#ifndef GLM_BACKEND_H
#define GLM_BACKEND_H

#include <stdint.h>

#include "glm_model.h"

#ifdef __cplusplus
extern "C" {
#endif

int glm_backend_init(BackendType backend, const Runtime *rt, RunState *st);
int glm_backend_forward_token(int use_gpu, const Runtime *rt, RunState *st, int token, int pos, int debug_mode);
void glm_backend_free(int use_gpu);

/* backend.h:11-13. There is no Metal device here: matvec offload always declines (-1),
 * so infer.c:792-797 keeps its CPU matvec. Kept so this file can stand in for backend.c. */
void glm_set_metal_matvec_mode(int enabled);
int glm_backend_metal_matvec_enabled(void);
int glm_backend_try_metal_matvec(const int8_t *qmat, const float *smat, const float *x, float *y, int rows, int dim,
                                 int gs);

/* 0 if the HIP backend ran MoE layer `layer_idx` on `st` (filling x, xn, xb,
 * moe_router, moe_topk_idx, moe_topk_w, moe_out_acc as infer.c:1087-1216 does);
 * -1 if the HIP backend is not active or failed, so the CPU path must run it. */
int glm_backend_try_hip_moe(const Runtime *rt, RunState *st, int layer_idx, int debug_mode);

/* HIP backend private API (mirrors glm_metal_* in backend.c:9-14). */
int glm_hip_init(const Runtime *rt, RunState *st);      /* 0 ok, -1 failure; idempotent */
int glm_hip_prepare(const Runtime *rt, RunState *st);   /* uploads MoE layers 1..n_layers-1; 0 ok */
int glm_hip_moe_layer(const Runtime *rt, RunState *st, int layer_idx, int debug_mode); /* 0 ok, -1 error */
/* 1 when glm_hip_prepare built the whole forward on the GPU (gmoe_model.h; not with
 * GLM_HIP_HOST_ATTN set). glm_hip_model_forward then runs a token through it: logits into
 * `logits` (st->logits when NULL) and the final x into st->x; with keep_state the model's
 * cache and st are left as they were (the dual-checkpoint form); attn_ckpt / layer_ckpt,
 * when given, receive x after each layer's attention / FFN ([n_layers][dim]). 0 ok, -1 error. */
int glm_hip_model_active(void);
int glm_hip_model_forward(const Runtime *rt, RunState *st, int token, int pos, int keep_state, float *logits,
                          float *attn_ckpt, float *layer_ckpt);
/* glm_hip_model_forward (not keep_state, logits into st->logits) that also returns, per
 * layer, the vectors glm.c's --debug sums (gmoe_model_forward_token_debug): x after
 * attention and FFN, the kv entry, the heads' concat, and for MoE layers the shared and
 * routed outputs, each [n_layers][..] on the host. 0 ok, -1 error. */
int glm_hip_model_forward_sums(RunState *st, int token, int pos, float *attn_ckpt, float *layer_ckpt, float *kv_out,
                               float *concat_out, float *shexp_out, float *moe_out);
/* n prompt tokens at positions pos0.. through the GPU model in batches of GLM_HIP_PREFILL_BATCH
 * (gmoe_model_prefill): the last token's logits into st->logits and its final x into st->x.
 * 0 ok, -1 error (glm_hip_prefill in glm_forward.h is the form that also works without the model). */
int glm_hip_model_prefill(const Runtime *rt, RunState *st, const int *tokens, int n, int pos0);
/* The GPU model's latent cache holds one RunState's history (st->k_cache_* of that state
 * are not written). 1 when the model can take st's token at pos: st is that state and the
 * device holds every position below pos, or no state is held yet and pos is 0 (the
 * forward then takes st on). glm_hip_forward_token, glm_hip_prefill and the checkpoint
 * forwards run on the host steps otherwise, from st's own cache. */
int glm_hip_model_owns(const RunState *st, int pos);
/* Positions pos0.. of the GPU model's latent cache for attention layer `layer` (the held
 * state's k_cache_comp / k_cache_pe rows, gmoe_model_read_cache). 0 ok, -1 error. */
int glm_hip_model_read_cache(int layer, int pos0, int n, float *comp_out, float *pe_out);
/* st's buffers are about to be freed: the model holds no state's history any more. */
void glm_hip_model_forget(const RunState *st);
void glm_hip_free(void);

#ifdef __cplusplus
}
#endif

#endif
