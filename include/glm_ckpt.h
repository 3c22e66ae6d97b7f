/*
 * glm_ckpt.h -- glm.c's checkpoint file, version 4 (the .bin that infer.c:357-744 maps and
 * glm47_flash_export.py:681-819 writes): a synthetic writer and a reader.
 *
 * Layout (all little-endian, tensors back to back in this order):
 *   header, 256 bytes: RuntimeConfig (glm_model.h) then zeros;
 *   output_norm [dim] f32; tok_q [vocab][dim] i8, tok_s [vocab][dim/gs] f32;
 *   out_q, out_s likewise;
 *   layer 0's dense FFN: ffn_norm [dim]; gate, up [hidden][dim] + scales; down [dim][hidden] + scales;
 *   layer 0's MLA attention (l0_flags & 1), then every layer's, 15 tensors each
 *     (attn_norm [dim], q_a_norm [q_lora], kv_a_norm [kv_lora], q_a [q_lora][dim],
 *      q_b [heads*head_k][q_lora], kv_a [kv_lora+rope][dim], k_b [heads*kv_lora][qk_nope],
 *      v_b [heads*v_head][kv_lora], attn_out [dim][heads*v_head], each Q8 matrix then its scales);
 *   MoE layers 1..L-1, shared part: ffn_norm, gate_inp [E][dim] f32, exp_probs_b [E],
 *     gate_sh, up_sh [moe][dim] + scales, down_sh [dim][moe] + scales;
 *   MoE layers 1..L-1, routed part: gate, up [E*moe][dim] + scales, down [E*dim][moe] + scales.
 * Q8 scales are fp32, one per group_size columns of a row.
 */
#ifndef GLM_CKPT_H
#define GLM_CKPT_H

#include <stdint.h>

#include "glm_model.h"

#ifdef __cplusplus
extern "C" {
#endif

#define GLM_CKPT_MAGIC 0x67343763u /* infer.c:35 (the bytes "c74g" on disk) */
#define GLM_CKPT_VERSION 4u
#define GLM_CKPT_HEADER 256
#define GLM_CKPT_ALL_ATTN 1        /* l0_flags bit: every layer's attention block follows */

/* A synthetic checkpoint's shape and draws. The MoE layers are exactly synth_layer()'s
 * (synth.h) for this seed, norm_mode, bias_mode and scale_mode, so a test can regenerate
 * any layer without reading the file; every other tensor comes from the same counter
 * streams under its own tensor ids. */
typedef struct glm_ckpt_spec {
    int32_t dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len, rope_dim;
    int32_t q_lora_rank, kv_lora_rank, n_routed_experts, n_experts_used, bos_id, eos_id;
    int32_t qk_nope_dim, v_head_dim, moe_ffn_dim, group_size;
    uint64_t seed;
    int32_t norm_mode, bias_mode, scale_mode;
} glm_ckpt_spec;

/* Writes the checkpoint; 0, or -1 with glm_ckpt_error(). */
int glm_ckpt_write_synth(const char *path, const glm_ckpt_spec *spec);

/* Maps `path` read-only and fills rt the way infer.c's runtime_open does (the same checks,
 * the same optional blocks); 0, or -1 with glm_ckpt_error() and rt left empty. */
int glm_ckpt_open(const char *path, Runtime *rt);
void glm_ckpt_close(Runtime *rt);
const char *glm_ckpt_error(void);

/* Every tensor pointer of rt as its offset in the file (0 for none), in a fixed order: the
 * global tensors, layer 0's FFN and attention, each layer's attention, each MoE layer's
 * shared then routed tensors. Writes at most max entries; returns the count it needs. */
int glm_ckpt_layout(const Runtime *rt, uint64_t *out, int max);

#ifdef __cplusplus
}
#endif

#endif
