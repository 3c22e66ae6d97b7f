/*
 * synth.h -- deterministic synthetic inputs for GLM-4.7-Flash-shaped MoE layers.
 *
 * Every value is a pure function of (seed, layer, tensor, expert, element index):
 * a splitmix64-style counter stream, so any expert of any layer can be regenerated
 * on its own, in any order, on any machine with the same libm. Draws:
 *   Q8 weights   uniform integers in [-127, 127]
 *   Q8 scales    fp16(|N(0,1)| * 0.002), RNE incl. subnormals, stored as fp32
 *   gate_inp     N(0, 0.02)        exp_probs_b   N(0, 0.01) or Zipf-shaped
 *   ffn_norm     1.0 or 1 + N(0, 0.1)            x             N(0, 1)
 * Tensors are written in glm.c's checkpoint layout (model.h:65-84).
 */
#ifndef GLM_SYNTH_H
#define GLM_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    SYNTH_NORM_ONES = 0,      /* ffn_norm = 1 */
    SYNTH_NORM_RANDOM = 1,    /* ffn_norm = 1 + N(0, 0.1) */
};

enum {
    SYNTH_BIAS_NORMAL = 0,    /* exp_probs_b ~ N(0, 0.01) */
    SYNTH_BIAS_ZIPF = 1,      /* beta * (-s * ln rank_e) + N(0, 0.01), ranks a random permutation */
};

enum {
    SYNTH_SCALES_FP16 = 0,    /* |N(0,1)| * 0.002 rounded to fp16 (the tiled device form holds them exactly) */
    SYNTH_SCALES_FP32 = 1,    /* |N(0,1)| * 0.002 in fp32, as an exporter's max|w|/127 scales are */
};

typedef struct synth_spec {
    uint64_t seed;
    int32_t dim, moe_ffn_dim, n_routed_experts, group_size;
    int32_t norm_mode;
    int32_t bias_mode;
    double zipf_s;            /* Zipf exponent for SYNTH_BIAS_ZIPF */
    double zipf_beta;         /* bias gain for SYNTH_BIAS_ZIPF */
    int32_t scale_mode;       /* SYNTH_SCALES_* */
} synth_spec;

/* Pointers to caller-owned host buffers in checkpoint layout; NULL entries are skipped. */
typedef struct synth_layer_buffers {
    float *ffn_norm, *gate_inp, *exp_probs_b;
    int8_t *gate_sh_q; float *gate_sh_s;
    int8_t *up_sh_q; float *up_sh_s;
    int8_t *down_sh_q; float *down_sh_s;
    int8_t *gate_q; float *gate_s;
    int8_t *up_q; float *up_s;
    int8_t *down_q; float *down_s;
} synth_layer_buffers;

/* Fill one MoE layer. Routed tensors are generated for experts [e_begin, e_end)
 * only, at their checkpoint offsets (the rest of the buffer is left untouched). */
int synth_layer(const synth_spec *spec, int layer, int e_begin, int e_end, const synth_layer_buffers *b);

/* x[t][i] ~ N(0,1) for t in [0, n_tokens), stream chosen by (seed, stream). */
void synth_activations(uint64_t seed, int stream, int n_tokens, int dim, float *x);

/* Nearest fp16 value of f (round to nearest even, subnormals kept), as a float. */
float synth_round_fp16(float f);

/* x[i] = mean + sd * N(0,1) from stream `key` (synth_key), n values. */
void synth_normal_fill(uint64_t key, size_t n, double mean, double sd, float *out);

/* A Q8 matrix drawn as the experts' are: int8 [rows][cols] from stream kq, scales
 * [rows][cols/gs] from ks in the form scale_mode (SYNTH_SCALES_*); NULL q or s is skipped. */
void synth_q8_matrix(uint64_t kq, uint64_t ks, int rows, int cols, int gs, int scale_mode, int8_t *q, float *s);

/* Raw stream access, for tests of the generator itself. */
uint64_t synth_key(uint64_t seed, int layer, int tensor, int expert);
uint64_t synth_draw(uint64_t key, uint64_t n);
int synth_q8_at(uint64_t key, uint64_t n);
double synth_normal_at(uint64_t key, uint64_t n);

#ifdef __cplusplus
}
#endif

#endif
