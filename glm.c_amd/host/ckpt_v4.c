/*
 * ckpt_v4.c -- glm.c's version-4 checkpoint file (glm_ckpt.h): a writer of synthetic
 * checkpoints and a reader into glm_model.h's Runtime.
 *
 * The file is a header and a run of blocks (global tensors, layer 0's FFN, attention
 * blocks, MoE blocks). Each block is described once, as a list of tensors (a norm of n
 * floats, an fp32 matrix, or a Q8 matrix = int8 rows then fp32 scales), and both the
 * writer and the reader walk those lists; the Runtime holds each block's tensor pointers
 * as consecutive fields in file order (model.h:47-84, 103-145), which the reader fills in
 * turn. The reader keeps the reference loader's rules (infer.c:357-744): which version
 * holds which block, which sizes must divide by the group size, and that an optional block
 * is present exactly when bytes remain after the previous one.
 */
#include "glm_ckpt.h"

#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "synth.h"

static char g_err[256];

static int fail(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return -1;
}

const char *glm_ckpt_error(void) { return g_err; }

/* ---------------------------------------------------------------- block descriptions */

enum { K_NORM, K_F32, K_Q8 };
typedef struct {
    int kind;
    size_t rows, cols; /* K_NORM, K_F32: rows x cols floats; K_Q8: rows x cols int8 + scales */
} tensor_t;

#define BLOCK_MAX 9
typedef struct {
    int n;
    tensor_t t[BLOCK_MAX];
    int fields; /* pointer fields of the Runtime block (a Q8 tensor fills two) */
} block_t;

typedef struct {
    size_t dim, hidden, vocab, gs, q_lora, kv_lora, rope, heads, qk_nope, head_k, v_head, moe, E;
} dims_t;

static void add(block_t *b, int kind, size_t rows, size_t cols) {
    b->t[b->n++] = (tensor_t){kind, rows, cols};
    b->fields += kind == K_Q8 ? 2 : 1;
}

static block_t block_global(const dims_t *d) {
    block_t b = {0};
    add(&b, K_NORM, 1, d->dim);          /* output_norm */
    add(&b, K_Q8, d->vocab, d->dim);     /* token embedding */
    add(&b, K_Q8, d->vocab, d->dim);     /* LM head */
    return b;
}
static block_t block_l0_ffn(const dims_t *d) {
    block_t b = {0};
    add(&b, K_NORM, 1, d->dim);
    add(&b, K_Q8, d->hidden, d->dim);    /* gate */
    add(&b, K_Q8, d->hidden, d->dim);    /* up */
    add(&b, K_Q8, d->dim, d->hidden);    /* down */
    return b;
}
static block_t block_attn(const dims_t *d) {
    block_t b = {0};
    add(&b, K_NORM, 1, d->dim);                          /* attn_norm */
    add(&b, K_NORM, 1, d->q_lora);                       /* q_a_norm */
    add(&b, K_NORM, 1, d->kv_lora);                      /* kv_a_norm */
    add(&b, K_Q8, d->q_lora, d->dim);                    /* q_a */
    add(&b, K_Q8, d->heads * d->head_k, d->q_lora);      /* q_b */
    add(&b, K_Q8, d->kv_lora + d->rope, d->dim);         /* kv_a (with the rope part) */
    add(&b, K_Q8, d->heads * d->kv_lora, d->qk_nope);    /* k_b */
    add(&b, K_Q8, d->heads * d->v_head, d->kv_lora);     /* v_b */
    add(&b, K_Q8, d->dim, d->heads * d->v_head);         /* attn_out */
    return b;
}
static block_t block_moe_shared(const dims_t *d) {
    block_t b = {0};
    add(&b, K_NORM, 1, d->dim);          /* ffn_norm */
    add(&b, K_F32, d->E, d->dim);        /* gate_inp (router) */
    add(&b, K_F32, 1, d->E);             /* exp_probs_b */
    add(&b, K_Q8, d->moe, d->dim);       /* gate_sh */
    add(&b, K_Q8, d->moe, d->dim);       /* up_sh */
    add(&b, K_Q8, d->dim, d->moe);       /* down_sh */
    return b;
}
static block_t block_moe_routed(const dims_t *d) {
    block_t b = {0};
    add(&b, K_Q8, d->E * d->moe, d->dim);
    add(&b, K_Q8, d->E * d->moe, d->dim);
    add(&b, K_Q8, d->E * d->dim, d->moe);
    return b;
}

static size_t tensor_bytes(const tensor_t *t, size_t gs, size_t *q, size_t *s) {
    if (t->kind != K_Q8) {
        *q = t->rows * t->cols * sizeof(float);
        *s = 0;
    } else {
        *q = t->rows * t->cols;
        *s = t->rows * (t->cols / gs) * sizeof(float);
    }
    return *q + *s;
}
static size_t block_bytes(const block_t *b, size_t gs) {
    size_t n = 0, q, s;
    for (int i = 0; i < b->n; i++) n += tensor_bytes(&b->t[i], gs, &q, &s);
    return n;
}

static dims_t dims_of(const RuntimeConfig *c) {
    dims_t d;
    d.dim = (size_t)c->dim;
    d.hidden = (size_t)c->hidden_dim;
    d.vocab = (size_t)c->vocab_size;
    d.gs = (size_t)c->group_size;
    d.q_lora = (size_t)c->q_lora_rank;
    d.kv_lora = (size_t)c->kv_lora_rank;
    d.rope = (size_t)c->rope_dim;
    d.heads = (size_t)c->n_heads;
    d.qk_nope = (size_t)(c->l0_qk_nope_dim > 0 ? c->l0_qk_nope_dim : 0);
    d.head_k = (size_t)(c->l0_head_k_dim > 0 ? c->l0_head_k_dim : 0);
    d.v_head = (size_t)(c->l0_v_head_dim > 0 ? c->l0_v_head_dim : 0);
    d.moe = (size_t)(c->moe_ffn_dim > 0 ? c->moe_ffn_dim : 0);
    d.E = (size_t)(c->n_routed_experts > 0 ? c->n_routed_experts : 0);
    return d;
}

/* ---------------------------------------------------------------- writer */

/* tensor ids of the non-MoE draws (synth.h's MoE ids stay below 32) */
enum { ID_GLOBAL = 32, ID_L0_FFN = 40, ID_ATTN = 48 };

static int write_all(FILE *f, const void *p, size_t n) { return fwrite(p, 1, n, f) == n ? 0 : -1; }

/* one generated tensor: norms 1 + N(0, 0.1), fp32 matrices N(0, 0.02), Q8 matrices as the
 * MoE experts' (uniform int8, |N(0,1)| * 0.002 scales in the spec's form) */
static int write_tensor(FILE *f, const glm_ckpt_spec *sp, int layer, int id, const tensor_t *t) {
    size_t q, s;
    tensor_bytes(t, (size_t)sp->group_size, &q, &s);
    void *buf = malloc(q + s + 1);
    if (!buf) return fail("out of memory for a %zu-byte tensor", q + s);
    const uint64_t kq = synth_key(sp->seed, layer, id, 0), ks = synth_key(sp->seed, layer, id, 1);
    if (t->kind == K_NORM)
        synth_normal_fill(kq, t->rows * t->cols, 1.0, 0.1, (float *)buf);
    else if (t->kind == K_F32)
        synth_normal_fill(kq, t->rows * t->cols, 0.0, 0.02, (float *)buf);
    else
        synth_q8_matrix(kq, ks, (int)t->rows, (int)t->cols, sp->group_size, sp->scale_mode, (int8_t *)buf,
                        (float *)((char *)buf + q));
    const int rc = write_all(f, buf, q + s);
    free(buf);
    return rc ? fail("write failed") : 0;
}

static int write_block(FILE *f, const glm_ckpt_spec *sp, int layer, int id0, const block_t *b) {
    for (int i = 0; i < b->n; i++)
        if (write_tensor(f, sp, layer, id0 + i, &b->t[i])) return -1;
    return 0;
}

/* MoE layer l's shared (routed = 0) or routed (1) tensors, as synth_layer draws them */
static int write_moe(FILE *f, const glm_ckpt_spec *sp, const dims_t *d, int layer, int routed) {
    synth_spec ss;
    memset(&ss, 0, sizeof(ss));
    ss.seed = sp->seed;
    ss.dim = (int32_t)d->dim;
    ss.moe_ffn_dim = (int32_t)d->moe;
    ss.n_routed_experts = (int32_t)d->E;
    ss.group_size = sp->group_size;
    ss.norm_mode = sp->norm_mode;
    ss.bias_mode = sp->bias_mode;
    ss.scale_mode = sp->scale_mode;
    ss.zipf_s = 1.2;
    ss.zipf_beta = 0.095;
    const block_t b = routed ? block_moe_routed(d) : block_moe_shared(d);
    void *ptr[2 * BLOCK_MAX];
    size_t len[2 * BLOCK_MAX];
    int nf = 0, rc = 0;
    for (int i = 0; i < b.n; i++) {
        size_t q, s;
        tensor_bytes(&b.t[i], d->gs, &q, &s);
        ptr[nf] = calloc(1, q);
        len[nf++] = q;
        if (s) {
            ptr[nf] = calloc(1, s);
            len[nf++] = s;
        }
    }
    for (int i = 0; i < nf; i++)
        if (!ptr[i]) rc = fail("out of memory for MoE layer %d", layer);
    if (!rc) {
        synth_layer_buffers lb;
        memset(&lb, 0, sizeof(lb));
        /* synth_layer_buffers lists the shared fields, then the routed ones, in file order */
        void **slot = (void **)&lb + (routed ? 9 : 0);
        for (int i = 0; i < nf; i++) slot[i] = ptr[i];
        if (synth_layer(&ss, layer, 0, routed ? (int)d->E : 0, &lb)) rc = fail("synth_layer failed for layer %d", layer);
    }
    for (int i = 0; i < nf && !rc; i++)
        if (write_all(f, ptr[i], len[i])) rc = fail("write failed");
    for (int i = 0; i < nf; i++) free(ptr[i]);
    return rc;
}

int glm_ckpt_write_synth(const char *path, const glm_ckpt_spec *sp) {
    if (!path || !sp) return fail("glm_ckpt_write_synth: null argument");
    const int gs = sp->group_size;
    if (gs <= 0 || sp->dim <= 0 || sp->hidden_dim <= 0 || sp->vocab_size <= 0 || sp->n_layers < 1 ||
        sp->dim % gs || sp->hidden_dim % gs || sp->q_lora_rank % gs || sp->kv_lora_rank % gs || sp->qk_nope_dim % gs ||
        (sp->n_heads * sp->v_head_dim) % gs || (sp->moe_ffn_dim > 0 && sp->moe_ffn_dim % gs) || sp->n_heads <= 0 ||
        sp->qk_nope_dim <= 0 || sp->v_head_dim <= 0)
        return fail("glm_ckpt_write_synth: shape does not divide by the group size %d, or a size is not positive", gs);
    RuntimeConfig c;
    memset(&c, 0, sizeof(c));
    c.magic = GLM_CKPT_MAGIC;
    c.version = GLM_CKPT_VERSION;
    c.dim = sp->dim;
    c.hidden_dim = sp->hidden_dim;
    c.n_layers = sp->n_layers;
    c.n_heads = sp->n_heads;
    c.n_kv_heads = sp->n_kv_heads;
    c.vocab_size = sp->vocab_size;
    c.seq_len = sp->seq_len;
    c.rope_dim = sp->rope_dim;
    c.q_lora_rank = sp->q_lora_rank;
    c.kv_lora_rank = sp->kv_lora_rank;
    c.kv_mqa_width = sp->kv_lora_rank + sp->rope_dim;
    c.n_routed_experts = sp->n_routed_experts;
    c.n_experts_used = sp->n_experts_used;
    c.n_shared_experts = 1;
    c.bos_id = sp->bos_id;
    c.eos_id = sp->eos_id;
    c.group_size = (uint64_t)gs;
    c.l0_qk_nope_dim = sp->qk_nope_dim;
    c.l0_head_k_dim = sp->qk_nope_dim + sp->rope_dim;
    c.l0_v_head_dim = sp->v_head_dim;
    c.l0_flags = GLM_CKPT_ALL_ATTN;
    c.moe_ffn_dim = sp->moe_ffn_dim;
    const dims_t d = dims_of(&c);

    /* offsets: the global and layer-0 FFN tensors are addressed from the header */
    uint64_t *goff[] = {&c.off_norm, &c.off_tok_q, &c.off_tok_s, &c.off_out_q, &c.off_out_s,
                        &c.off_l0_ffn_norm, &c.off_l0_ffn_gate_q, &c.off_l0_ffn_gate_s, &c.off_l0_ffn_up_q,
                        &c.off_l0_ffn_up_s, &c.off_l0_ffn_down_q, &c.off_l0_ffn_down_s};
    size_t off = GLM_CKPT_HEADER;
    int k = 0;
    const block_t head[2] = {block_global(&d), block_l0_ffn(&d)};
    for (int bi = 0; bi < 2; bi++)
        for (int i = 0; i < head[bi].n; i++) {
            size_t q, s;
            tensor_bytes(&head[bi].t[i], d.gs, &q, &s);
            *goff[k++] = off;
            off += q;
            if (s) {
                *goff[k++] = off;
                off += s;
            }
        }
    const block_t attn = block_attn(&d), msh = block_moe_shared(&d), mro = block_moe_routed(&d);
    const size_t L = (size_t)sp->n_layers, nmoe = d.moe > 0 && L > 1 ? L - 1 : 0;
    off += block_bytes(&attn, d.gs) * (1 + L) + (block_bytes(&msh, d.gs) + block_bytes(&mro, d.gs)) * nmoe;
    c.total_bytes = off;

    FILE *f = fopen(path, "wb");
    if (!f) return fail("cannot create %s", path);
    unsigned char header[GLM_CKPT_HEADER];
    memset(header, 0, sizeof(header));
    memcpy(header, &c, sizeof(c));
    int rc = write_all(f, header, sizeof(header)) ? fail("write failed") : 0;
    if (!rc) rc = write_block(f, sp, -1, ID_GLOBAL, &head[0]);
    if (!rc) rc = write_block(f, sp, 0, ID_L0_FFN, &head[1]);
    /* layer 0's attention (the v4 extension), then every layer's: layer 0's twice, the same draws */
    if (!rc) rc = write_block(f, sp, 0, ID_ATTN, &attn);
    for (size_t l = 0; l < L && !rc; l++) rc = write_block(f, sp, (int)l, ID_ATTN, &attn);
    for (size_t l = 1; l <= nmoe && !rc; l++) rc = write_moe(f, sp, &d, (int)l, 0);
    for (size_t l = 1; l <= nmoe && !rc; l++) rc = write_moe(f, sp, &d, (int)l, 1);
    if (fclose(f) && !rc) rc = fail("closing %s failed", path);
    return rc;
}

/* ---------------------------------------------------------------- reader */

typedef struct {
    const unsigned char *data;
    size_t size, off;
    const char *what;
} cursor_t;

static int in_file(size_t size, uint64_t off, size_t bytes) { return off <= size && bytes <= size - off; }

/* the block's tensors from the cursor on, into its consecutive pointer fields */
static int take_block(cursor_t *c, const block_t *b, size_t gs, const void **fields) {
    int k = 0;
    for (int i = 0; i < b->n; i++) {
        size_t q, s;
        tensor_bytes(&b->t[i], gs, &q, &s);
        if (!in_file(c->size, c->off, q + s)) return fail("%s: tensor %d out of bounds", c->what, i);
        fields[k++] = c->data + c->off;
        c->off += q;
        if (b->t[i].kind == K_Q8) {
            fields[k++] = c->data + c->off;
            c->off += s;
        }
    }
    return 0;
}

static int check_config(const RuntimeConfig *c, size_t size) {
    if (c->magic != GLM_CKPT_MAGIC) return fail("invalid checkpoint magic");
    if (c->version != 2u && c->version != 3u && c->version != GLM_CKPT_VERSION) return fail("unsupported version %u", c->version);
    if ((size_t)c->total_bytes != size) return fail("checkpoint size mismatch");
    if (c->group_size == 0) return fail("invalid group size");
    if (c->dim <= 0 || c->hidden_dim <= 0 || c->vocab_size <= 0) return fail("invalid dimensions");
    const int gs = (int)c->group_size;
    if (c->dim % gs || c->hidden_dim % gs || c->q_lora_rank % gs || c->kv_lora_rank % gs)
        return fail("dim, hidden_dim, q_lora_rank and kv_lora_rank must divide by the group size");
    return 0;
}

int glm_ckpt_open(const char *path, Runtime *rt) {
    if (!path || !rt) return fail("glm_ckpt_open: null argument");
    memset(rt, 0, sizeof(*rt));
    struct stat st;
    if (stat(path, &st) != 0 || st.st_size <= 0) return fail("cannot stat %s", path);
    const size_t size = (size_t)st.st_size;
    if (size < GLM_CKPT_HEADER) return fail("checkpoint too small");
    const int fd = open(path, O_RDONLY);
    if (fd < 0) return fail("cannot open %s", path);
    void *map = mmap(NULL, size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return fail("mmap of %s failed", path);
    rt->data = (unsigned char *)map;
    rt->file_size = size;
    memcpy(&rt->cfg, rt->data, sizeof(RuntimeConfig));
    const RuntimeConfig *c = &rt->cfg;
    int rc = check_config(c, size);
    const dims_t d = dims_of(c);
    cursor_t cur = {rt->data, size, 0, "base tensors"};
    /* global and layer-0 FFN tensors sit where the header says */
    const uint64_t goff[5] = {c->off_norm, c->off_tok_q, c->off_tok_s, c->off_out_q, c->off_out_s};
    const size_t gbytes[5] = {d.dim * 4, d.vocab * d.dim, d.vocab * (d.dim / (d.gs ? d.gs : 1)) * 4, d.vocab * d.dim,
                              d.vocab * (d.dim / (d.gs ? d.gs : 1)) * 4};
    const void **gfield = (const void **)&rt->output_norm;
    for (int i = 0; i < 5 && !rc; i++) {
        if (!in_file(size, goff[i], gbytes[i])) rc = fail("base tensor offsets out of bounds");
        else gfield[i] = rt->data + goff[i];
    }
    if (!rc && c->version >= 3u && c->off_l0_ffn_norm != 0) {
        const uint64_t loff[7] = {c->off_l0_ffn_norm, c->off_l0_ffn_gate_q, c->off_l0_ffn_gate_s, c->off_l0_ffn_up_q,
                                  c->off_l0_ffn_up_s, c->off_l0_ffn_down_q, c->off_l0_ffn_down_s};
        const size_t dg = d.dim / d.gs, hg = d.hidden / d.gs;
        const size_t lbytes[7] = {d.dim * 4, d.hidden * d.dim, d.hidden * dg * 4, d.hidden * d.dim, d.hidden * dg * 4,
                                  d.dim * d.hidden, d.dim * hg * 4};
        const void **lfield = (const void **)&rt->l0_ffn_norm;
        for (int i = 0; i < 7 && !rc; i++) {
            if (!in_file(size, loff[i], lbytes[i])) rc = fail("layer-0 FFN offsets out of bounds");
            else lfield[i] = rt->data + loff[i];
        }
        if (!rc) rt->has_l0_ffn = 1;
    }
    /* the blocks after layer 0's FFN follow one another */
    if (!rc) cur.off = (size_t)c->off_l0_ffn_down_s + d.dim * (d.hidden / d.gs) * sizeof(float);
    const block_t attn = block_attn(&d);
    if (!rc && c->version >= 4u && (c->l0_flags & GLM_CKPT_ALL_ATTN)) {
        const int gs = (int)c->group_size;
        if (c->l0_qk_nope_dim <= 0 || c->l0_head_k_dim <= 0 || c->l0_v_head_dim <= 0) rc = fail("invalid v4 MLA dims");
        else if (c->l0_head_k_dim != c->l0_qk_nope_dim + c->rope_dim) rc = fail("invalid v4 MLA shape relation");
        else if (c->l0_qk_nope_dim % gs || (c->n_heads * c->l0_v_head_dim) % gs)
            rc = fail("MLA widths must divide by the group size");
        cur.what = "layer-0 attention";
        if (!rc) rc = take_block(&cur, &attn, d.gs, (const void **)&rt->l0_attn_norm);
        if (!rc) rt->has_l0_attn = 1;
    }
    const size_t L = c->n_layers > 0 ? (size_t)c->n_layers : 0;
    if (!rc && rt->has_l0_attn && cur.off < size) {
        if (block_bytes(&attn, d.gs) * L > size - cur.off) rc = fail("incomplete all-layer attention block");
        else if (!(rt->attn_layers = (LayerAttnWeights *)calloc(L, sizeof(LayerAttnWeights)))) rc = fail("out of memory");
        cur.what = "attention layers";
        for (size_t l = 0; l < L && !rc; l++) rc = take_block(&cur, &attn, d.gs, (const void **)&rt->attn_layers[l]);
        if (!rc) rt->has_all_attn = 1;
    }
    if (!rc && c->moe_ffn_dim > 0 && L > 1 && cur.off < size) {
        if (d.moe % d.gs) rc = fail("moe_ffn_dim must divide by the group size");
        const block_t msh = block_moe_shared(&d), mro = block_moe_routed(&d);
        if (!rc && block_bytes(&msh, d.gs) * (L - 1) > size - cur.off) rc = fail("incomplete MoE shared block");
        else if (!rc && !(rt->moe_layers = (LayerMoeShared *)calloc(L, sizeof(LayerMoeShared)))) rc = fail("out of memory");
        cur.what = "MoE shared layers";
        for (size_t l = 1; l < L && !rc; l++) rc = take_block(&cur, &msh, d.gs, (const void **)&rt->moe_layers[l]);
        if (!rc) rt->has_moe_shared = 1;
        if (!rc && cur.off < size) {
            if (block_bytes(&mro, d.gs) * (L - 1) > size - cur.off) rc = fail("incomplete MoE routed block");
            else if (!(rt->moe_routed_layers = (LayerMoeRouted *)calloc(L, sizeof(LayerMoeRouted)))) rc = fail("out of memory");
            cur.what = "MoE routed layers";
            for (size_t l = 1; l < L && !rc; l++) rc = take_block(&cur, &mro, d.gs, (const void **)&rt->moe_routed_layers[l]);
            if (!rc) rt->has_moe_routed = 1;
        }
    }
    if (rc) glm_ckpt_close(rt);
    return rc;
}

void glm_ckpt_close(Runtime *rt) {
    if (!rt) return;
    free(rt->attn_layers);
    free(rt->moe_layers);
    free(rt->moe_routed_layers);
    if (rt->data && rt->file_size) munmap(rt->data, rt->file_size);
    memset(rt, 0, sizeof(*rt));
}

int glm_ckpt_layout(const Runtime *rt, uint64_t *out, int max) {
    int n = 0;
#define PUT(p) do { if (n < max) out[n] = (p) ? (uint64_t)((const unsigned char *)(p) - rt->data) : 0u; n++; } while (0)
    const void *const *g = (const void *const *)&rt->output_norm;
    for (int i = 0; i < 5; i++) PUT(g[i]);
    const void *const *f = (const void *const *)&rt->l0_ffn_norm;
    for (int i = 0; i < 7; i++) PUT(rt->has_l0_ffn ? f[i] : NULL);
    const void *const *a = (const void *const *)&rt->l0_attn_norm;
    for (int i = 0; i < 15; i++) PUT(rt->has_l0_attn ? a[i] : NULL);
    const int L = rt->cfg.n_layers;
    for (int l = 0; l < L; l++) {
        const void *const *w = rt->has_all_attn ? (const void *const *)&rt->attn_layers[l] : NULL;
        for (int i = 0; i < 15; i++) PUT(w ? w[i] : NULL);
    }
    for (int l = 1; l < L; l++) {
        const void *const *s = rt->has_moe_shared ? (const void *const *)&rt->moe_layers[l] : NULL;
        for (int i = 0; i < 9; i++) PUT(s ? s[i] : NULL);
        const void *const *r = rt->has_moe_routed ? (const void *const *)&rt->moe_routed_layers[l] : NULL;
        for (int i = 0; i < 6; i++) PUT(r ? r[i] : NULL);
    }
#undef PUT
    return n;
}
