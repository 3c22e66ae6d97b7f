/*
 * synth.c -- deterministic synthetic GLM-4.7-Flash-shaped MoE layers (see synth.h).
 */
#include "synth.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define SYNTH_GOLDEN 0x9E3779B97F4A7C15ULL

enum {
    T_NORM = 1,
    T_GATE_INP = 2,
    T_PROBS_B = 3,
    T_GATE_Q = 4,
    T_GATE_S = 5,
    T_UP_Q = 6,
    T_UP_S = 7,
    T_DOWN_Q = 8,
    T_DOWN_S = 9,
    T_RANK = 10,
    T_X = 11,
};
#define SHARED_EXPERT_ID 0xFFFF

/* splitmix64 output function (Steele, Lea, Flood, OOPSLA 2014). */
static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

uint64_t synth_key(uint64_t seed, int layer, int tensor, int expert) {
    uint64_t k = mix64(seed + SYNTH_GOLDEN);
    k = mix64(k ^ ((uint64_t)(uint32_t)layer * 0xD1B54A32D192ED03ULL));
    k = mix64(k ^ (((uint64_t)(uint32_t)tensor << 32) | (uint64_t)(uint32_t)expert));
    return k;
}

uint64_t synth_draw(uint64_t key, uint64_t n) { return mix64(key + (n + 1) * SYNTH_GOLDEN); }

/* Weight n takes one 32-bit half of draw n/2; Lemire's multiply-shift maps it to 0..254. */
static inline int q8_at(uint64_t key, uint64_t n) {
    uint64_t r = synth_draw(key, n >> 1);
    uint32_t h = (n & 1) ? (uint32_t)(r >> 32) : (uint32_t)r;
    return (int)(((uint64_t)h * 255u) >> 32) - 127;
}

int synth_q8_at(uint64_t key, uint64_t n) { return q8_at(key, n); }

/* Box-Muller on draws 2n and 2n+1 (cosine branch only). */
double synth_normal_at(uint64_t key, uint64_t n) {
    uint64_t a = synth_draw(key, 2 * n);
    uint64_t b = synth_draw(key, 2 * n + 1);
    double u1 = (double)((a >> 11) + 1) * 0x1p-53; /* (0, 1] */
    double u2 = (double)(b >> 11) * 0x1p-53;       /* [0, 1) */
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925 * u2);
}

float synth_round_fp16(float f) {
    if (!isfinite(f)) return f;
    double a = fabs((double)f);
    double r;
    if (a >= 65520.0) {
        r = INFINITY; /* at or beyond the rounding midpoint above 65504 */
    } else if (a < 0x1p-14) {
        r = rint(a * 0x1p24) * 0x1p-24; /* subnormal quantum 2^-24 */
    } else {
        int e;
        frexp(a, &e); /* a = m * 2^e, m in [0.5, 1) */
        double q = ldexp(1.0, e - 11); /* 10 fraction bits */
        r = rint(a / q) * q;
    }
    return (float)copysign(r, (double)f);
}

static void fill_q8_matrix(uint64_t kq, uint64_t ks, int rows, int cols, int gs, int fp32_scales, int8_t *q, float *s) {
    const int groups = cols / gs;
    if (q) {
#pragma omp parallel for schedule(static)
        for (int r = 0; r < rows; r++) {
            int8_t *row = q + (size_t)r * cols;
            uint64_t base = (uint64_t)r * (uint64_t)cols;
            for (int c = 0; c < cols; c++) row[c] = (int8_t)q8_at(kq, base + (uint64_t)c);
        }
    }
    if (s) {
#pragma omp parallel for schedule(static)
        for (int r = 0; r < rows; r++) {
            float *row = s + (size_t)r * groups;
            uint64_t base = (uint64_t)r * (uint64_t)groups;
            for (int g = 0; g < groups; g++) {
                double z = fabs(synth_normal_at(ks, base + (uint64_t)g));
                row[g] = fp32_scales ? (float)(z * 0.002) : synth_round_fp16((float)(z * 0.002));
            }
        }
    }
}

static void fill_normal(uint64_t key, size_t n, double mean, double sd, float *out) {
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; i++) out[i] = (float)(mean + sd * synth_normal_at(key, (uint64_t)i));
}

void synth_normal_fill(uint64_t key, size_t n, double mean, double sd, float *out) { fill_normal(key, n, mean, sd, out); }

void synth_q8_matrix(uint64_t kq, uint64_t ks, int rows, int cols, int gs, int scale_mode, int8_t *q, float *s) {
    fill_q8_matrix(kq, ks, rows, cols, gs, scale_mode == SYNTH_SCALES_FP32, q, s);
}

int synth_layer(const synth_spec *sp, int layer, int e_begin, int e_end, const synth_layer_buffers *b) {
    if (!sp || !b) return -1;
    const int D = sp->dim, F = sp->moe_ffn_dim, E = sp->n_routed_experts, gs = sp->group_size;
    if (D <= 0 || F <= 0 || E <= 0 || gs <= 0 || D % gs || F % gs) return -1;
    if (e_begin < 0) e_begin = 0;
    if (e_end > E) e_end = E;
    const uint64_t seed = sp->seed;

    if (b->ffn_norm) {
        if (sp->norm_mode == SYNTH_NORM_RANDOM) {
            fill_normal(synth_key(seed, layer, T_NORM, 0), (size_t)D, 1.0, 0.1, b->ffn_norm);
        } else {
            for (int i = 0; i < D; i++) b->ffn_norm[i] = 1.0f;
        }
    }
    if (b->gate_inp) fill_normal(synth_key(seed, layer, T_GATE_INP, 0), (size_t)E * D, 0.0, 0.02, b->gate_inp);
    if (b->exp_probs_b) {
        fill_normal(synth_key(seed, layer, T_PROBS_B, 0), (size_t)E, 0.0, 0.01, b->exp_probs_b);
        if (sp->bias_mode == SYNTH_BIAS_ZIPF) {
            /* Fisher-Yates permutation of ranks 1..E from the rank stream. */
            int *rank = (int *)malloc((size_t)E * sizeof(int));
            if (!rank) return -1;
            for (int e = 0; e < E; e++) rank[e] = e + 1;
            uint64_t kr = synth_key(seed, layer, T_RANK, 0);
            for (int i = E - 1; i > 0; i--) {
                int j = (int)(synth_draw(kr, (uint64_t)i) % (uint64_t)(i + 1));
                int t = rank[i];
                rank[i] = rank[j];
                rank[j] = t;
            }
            for (int e = 0; e < E; e++) {
                double zb = sp->zipf_beta * (-sp->zipf_s * log((double)rank[e]));
                b->exp_probs_b[e] = (float)((double)b->exp_probs_b[e] + zb);
            }
            free(rank);
        }
    }

    const int dg = D / gs, fg = F / gs, f32 = sp->scale_mode == SYNTH_SCALES_FP32;
    const size_t mq = (size_t)F * D; /* weights per expert matrix */
    fill_q8_matrix(synth_key(seed, layer, T_GATE_Q, SHARED_EXPERT_ID), synth_key(seed, layer, T_GATE_S, SHARED_EXPERT_ID),
                   F, D, gs, f32, b->gate_sh_q, b->gate_sh_s);
    fill_q8_matrix(synth_key(seed, layer, T_UP_Q, SHARED_EXPERT_ID), synth_key(seed, layer, T_UP_S, SHARED_EXPERT_ID),
                   F, D, gs, f32, b->up_sh_q, b->up_sh_s);
    fill_q8_matrix(synth_key(seed, layer, T_DOWN_Q, SHARED_EXPERT_ID), synth_key(seed, layer, T_DOWN_S, SHARED_EXPERT_ID),
                   D, F, gs, f32, b->down_sh_q, b->down_sh_s);
    for (int e = e_begin; e < e_end; e++) {
        fill_q8_matrix(synth_key(seed, layer, T_GATE_Q, e), synth_key(seed, layer, T_GATE_S, e), F, D, gs, f32,
                       b->gate_q ? b->gate_q + (size_t)e * mq : NULL, b->gate_s ? b->gate_s + (size_t)e * F * dg : NULL);
        fill_q8_matrix(synth_key(seed, layer, T_UP_Q, e), synth_key(seed, layer, T_UP_S, e), F, D, gs, f32,
                       b->up_q ? b->up_q + (size_t)e * mq : NULL, b->up_s ? b->up_s + (size_t)e * F * dg : NULL);
        fill_q8_matrix(synth_key(seed, layer, T_DOWN_Q, e), synth_key(seed, layer, T_DOWN_S, e), D, F, gs, f32,
                       b->down_q ? b->down_q + (size_t)e * mq : NULL, b->down_s ? b->down_s + (size_t)e * D * fg : NULL);
    }
    return 0;
}

void synth_activations(uint64_t seed, int stream, int n_tokens, int dim, float *x) {
    fill_normal(synth_key(seed, stream, T_X, 0), (size_t)n_tokens * (size_t)dim, 0.0, 1.0, x);
}
