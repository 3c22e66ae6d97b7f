/*
 * expf_table.c -- the exception table that lets the GPU reproduce the host libm's
 * expf bit for bit.
 *
 * glm.c's router probability is p = 1.0f / (1.0f + expf(-logit)) with the C
 * library's expf (infer.c:1104-1107), and its top-k compares p + bias with strict
 * `>` (infer.c:1110-1135). Two experts whose scores differ only in expf's last bit
 * are ordered by that bit, so an exact GPU replay of the router needs the same
 * expf results, not merely close ones.
 *
 * The GPU evaluates r = RN_f32(exp(x)) from a double-precision exp (error < 2^-50
 * relative). glibc's expf (a double-precision polynomial with relative error below
 * 2^-33, then one rounding to fp32) returns that correctly rounded value except
 * where exp(x) lies within its polynomial error of a midpoint between two floats.
 * Whether those few inputs round up or down is a property of glibc's evaluation,
 * not of the mathematics, so it is measured here: this program evaluates expf and
 * exp for every finite fp32 input and records
 *   (1) every x whose expf(x) is not RN_f32(exp((double)x)), and
 *   (2) every x whose exp(x) lies within 2^-20 fp32 ulp of a midpoint, where the
 *       GPU's and the host's double results could round to different floats,
 * each with one bit: whether expf(x) is the float just above exp(x) or just below.
 * It also proves the premise of the GPU's shortcut: every input of kind (1) lies
 * within GM_EXPF_NEAR of a midpoint, so an input further away needs no lookup.
 *
 *   expf_table sweep OUT.bin     measure the table with this host's libm
 *   expf_table inc IN.bin OUT    write it as C initialisers for the device code
 *
 * Table file (little-endian): "GMEXPF02", u32 n, u32 near_log2 (the lookup
 * threshold, as -log2 of fp32 ulps), char libc[16] (gnu_get_libc_version() of the
 * measuring host, NUL-padded), u32 keys[n] (fp32 bit patterns of x, ascending),
 * u32 up[(n + 31) / 32] (bit i of word i / 32: entry i rounds to the float above).
 * The generated initialisers carry the version as GM_EXPF_LIBC, which gmoe_create
 * compares with the running process's C library.
 */
#include <gnu/libc-version.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define NEAR_LOG2 7          /* the GPU looks up x when exp(x) is within 2^-7 ulp of a midpoint */
#define HARD_LOG2 20         /* kind (2): within 2^-20 ulp */
#define MISROUND_MAX_LOG2 9  /* kind (1) must lie within 2^-9 ulp, well inside the lookup zone */
#define LIBC_LEN 16          /* bytes of the libc version field */

static float u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static uint32_t f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

/* exp value d placed on the fp32 grid: d = (fl + frac) * 2^ue, fl an integer, frac in [0, 1). */
static void grid_of(double d, int *ue, double *fl, double *frac) {
    int ex;
    (void)frexp(d, &ex); /* d = m 2^ex, m in [0.5, 1): fp32 spacing there is 2^(ex - 24) */
    int e = ex - 24;
    if (e < -149) e = -149; /* subnormal fp32 spacing */
    const double q = ldexp(d, -e);
    *ue = e;
    *fl = floor(q);
    *frac = q - *fl;
}

typedef struct {
    uint32_t *keys;
    uint8_t *up;
    size_t n, cap;
} Chunk;

static void push(Chunk *c, uint32_t key, int up) {
    if (c->n == c->cap) {
        c->cap = c->cap ? 2 * c->cap : 64;
        c->keys = realloc(c->keys, c->cap * sizeof *c->keys);
        c->up = realloc(c->up, c->cap);
        if (!c->keys || !c->up) {
            fprintf(stderr, "expf_table: out of memory\n");
            exit(1);
        }
    }
    c->keys[c->n] = key;
    c->up[c->n] = (uint8_t)up;
    c->n++;
}

static int sweep(const char *out_path) {
    enum { NCH = 65536 };
    Chunk *ch = calloc(NCH, sizeof *ch);
    long long bad = 0, misround = 0, hard = 0;
    double worst = 0.0; /* largest midpoint distance of a misrounded input, in fp32 ulps */
#pragma omp parallel for schedule(dynamic, 16) reduction(+ : bad, misround, hard) reduction(max : worst)
    for (int hi = 0; hi < NCH; hi++) {
        for (uint32_t lo = 0; lo < 65536u; lo++) {
            const uint32_t key = ((uint32_t)hi << 16) | lo;
            const float x = u2f(key);
            if (!isfinite(x)) continue;
            const float g = expf(x);
            /* the GPU answers these without the table: +inf from 89 up, 0 below -104 */
            if (!(x < 89.0f) || x < -104.0f) {
                if (f2u(g) != f2u(x > 0.0f ? INFINITY : 0.0f)) bad++;
                continue;
            }
            const double d = exp((double)x);
            int ue;
            double fl, frac;
            grid_of(d, &ue, &fl, &frac);
            const float rn = (float)d;
            const double dist = fabs(frac - 0.5);
            const int mis = f2u(g) != f2u(rn);
            const int is_hard = dist < ldexp(1.0, -HARD_LOG2);
            if (!mis && !is_hard) continue;
            const float below = (float)ldexp(fl, ue), above = (float)ldexp(fl + 1.0, ue);
            int up;
            if (f2u(g) == f2u(above))
                up = 1;
            else if (f2u(g) == f2u(below))
                up = 0;
            else {
                bad++; /* expf is not one of the two neighbours of exp(x) */
                continue;
            }
            if (mis) {
                misround++;
                if (dist > worst) worst = dist;
            }
            if (is_hard) hard++;
            push(&ch[hi], key, up);
        }
    }
    size_t n = 0;
    for (int i = 0; i < NCH; i++) n += ch[i].n;
    printf("expf_table: %zu entries (%lld misrounded by libm, %lld within 2^-%d ulp of a midpoint), "
           "worst misround at %.3g ulp from a midpoint, %lld inputs outside the model\n",
           n, misround, hard, HARD_LOG2, worst, bad);
    if (bad || worst >= ldexp(1.0, -MISROUND_MAX_LOG2)) {
        fprintf(stderr, "expf_table: this libm's expf is not within the table's model\n");
        return 1;
    }
    FILE *f = fopen(out_path, "wb");
    if (!f) {
        perror(out_path);
        return 1;
    }
    const uint32_t n32 = (uint32_t)n, near = NEAR_LOG2;
    char libc[LIBC_LEN] = {0};
    strncpy(libc, gnu_get_libc_version(), LIBC_LEN - 1);
    fwrite("GMEXPF02", 1, 8, f);
    fwrite(&n32, 4, 1, f);
    fwrite(&near, 4, 1, f);
    fwrite(libc, 1, LIBC_LEN, f);
    for (int i = 0; i < NCH; i++) fwrite(ch[i].keys, 4, ch[i].n, f);
    const size_t nw = (n + 31) / 32;
    uint32_t *bits = calloc(nw ? nw : 1, 4);
    size_t k = 0;
    for (int i = 0; i < NCH; i++)
        for (size_t j = 0; j < ch[i].n; j++, k++)
            if (ch[i].up[j]) bits[k / 32] |= 1u << (k % 32);
    fwrite(bits, 4, nw, f);
    free(bits);
    for (int i = 0; i < NCH; i++) {
        free(ch[i].keys);
        free(ch[i].up);
    }
    free(ch);
    return fclose(f) == 0 ? 0 : 1;
}

/* separator before element i of an initialiser printed `per` to a line */
static const char *sep(size_t i, size_t per) { return i == 0 ? "\n" : i % per ? "," : ",\n"; }

static int to_inc(const char *in_path, const char *out_path) {
    FILE *f = fopen(in_path, "rb");
    if (!f) {
        perror(in_path);
        return 1;
    }
    char magic[8], libc[LIBC_LEN];
    uint32_t n, near;
    if (fread(magic, 1, 8, f) != 8 || memcmp(magic, "GMEXPF02", 8) != 0 || fread(&n, 4, 1, f) != 1 ||
        fread(&near, 4, 1, f) != 1 || fread(libc, 1, LIBC_LEN, f) != LIBC_LEN || libc[LIBC_LEN - 1] != 0) {
        fprintf(stderr, "%s: not an expf table\n", in_path);
        return 1;
    }
    for (const char *c = libc; *c; c++)
        if (!((*c >= '0' && *c <= '9') || *c == '.')) {
            fprintf(stderr, "%s: bad libc version field\n", in_path);
            return 1;
        }
    const size_t nw = (n + 31) / 32;
    uint32_t *keys = malloc((size_t)n * 4 + 4), *bits = malloc(nw * 4 + 4);
    if (fread(keys, 4, n, f) != n || fread(bits, 4, nw, f) != nw) {
        fprintf(stderr, "%s: truncated\n", in_path);
        return 1;
    }
    fclose(f);
    for (uint32_t i = 1; i < n; i++)
        if (keys[i] <= keys[i - 1]) {
            fprintf(stderr, "%s: keys not ascending at %u\n", in_path, i);
            return 1;
        }
    FILE *o = fopen(out_path, "w");
    if (!o) {
        perror(out_path);
        return 1;
    }
    fprintf(o, "// generated from %s by expf_table inc; do not edit\n", in_path);
    fprintf(o, "#define GM_EXPF_N %uu\n#define GM_EXPF_NEAR_LOG2 %u\n#define GM_EXPF_LIBC \"%s\"\n", n, near, libc);
    fprintf(o, "__device__ const unsigned gm_expf_keys[GM_EXPF_N] = {");
    for (uint32_t i = 0; i < n; i++) fprintf(o, "%s0x%08x", sep(i, 8), keys[i]);
    fprintf(o, "};\n__device__ const unsigned gm_expf_up[%zu] = {", nw);
    for (size_t i = 0; i < nw; i++) fprintf(o, "%s0x%08x", sep(i, 8), bits[i]);
    /* index[h] = first entry whose key has high half >= h */
    fprintf(o, "};\n__device__ const unsigned gm_expf_index[65537] = {");
    uint32_t k = 0;
    for (uint32_t h = 0; h <= 65536u; h++) {
        while (k < n && (keys[k] >> 16) < h) k++;
        fprintf(o, "%s%u", sep(h, 16), h == 65536u ? n : k);
    }
    fprintf(o, "};\n");
    free(keys);
    free(bits);
    return fclose(o) == 0 ? 0 : 1;
}

int main(int argc, char **argv) {
    if (argc == 3 && strcmp(argv[1], "sweep") == 0) return sweep(argv[2]);
    if (argc == 4 && strcmp(argv[1], "inc") == 0) return to_inc(argv[2], argv[3]);
    fprintf(stderr, "usage: expf_table sweep OUT.bin | expf_table inc IN.bin OUT.inc\n");
    return 2;
}
