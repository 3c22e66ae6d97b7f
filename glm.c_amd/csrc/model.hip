// model.hip -- gmoe_model (include/gmoe_model.h): glm.c's decode forward (infer.c:1767-1901)
// with every weight, the latent cache and x in device memory. A prefill runs the same steps
// over a batch of tokens, each product launched once for the batch (grid y = token), the
// attention over the cache once per token, and each MoE layer as one grouped call.
// Per token, on one stream:
//
//   k_embed                      x = the token's embedding row
//   per attention layer (infer.c:978-1065):
//     k_gemv                     q_a = q_a . rmsnorm(x), kv_a = kv_a . rmsnorm(x)
//     k_gemv                     q = q_b . rmsnorm(q_a)
//     k_attn_query               q_abs = k_b_h . q_nope_h per head, and on one more block the
//                                position's cache entry (normalised kv, rotated rope part)
//                                and every head's rotated query part
//     k_attn_chunk, k_attn_merge   softmax over the cache, weighted sum of entries
//     k_gemv (per head)          concat_h = v_b_h . ctx_h
//     k_gemv (residual)          x += attn_out . concat
//   layer 0: k_gemv (SwiGLU pair), k_gemv (residual): the dense FFN (infer.c:1067-1085)
//   layers 1..: gmoe_forward of the MoE context, in place on x
//   k_gemv                       logits = out . rmsnorm(x)
//
// The rope angles' cosines and sines are computed once on the host with libm, as glm.c
// computes them (infer.c:964-976), so the rotations are glm.c's to the bit.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <vector>

#include "gmoe_model.h"
#include "common.h"
#include "dense.h"
#include "attn.h"
#include "attn16.h"
#include "gemm.h"

// gmoe.hip
void gm_set_err(const char *fmt, ...);
int gm_take_launch_error(gmoe_ctx *c);
int gm_decode_begin(gmoe_ctx *c, int n, hipStream_t st, int *on);
int gm_decode_layer(gmoe_ctx *c, int layer, int w, const float *x_in, float *x_out, int flags, hipStream_t st);
int gm_layer_ready(const gmoe_ctx *c, int layer);
void gm_layer_outputs(const gmoe_ctx *c, const float **shared, const float **routed);
void gm_decode_abort(gmoe_ctx *c);

#define MH_OK(expr)                                                                                  \
    do {                                                                                             \
        hipError_t e_ = (expr);                                                                      \
        if (e_ != hipSuccess) {                                                                      \
            gm_set_err("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, __LINE__); \
            return GMOE_ERR_HIP;                                                                     \
        }                                                                                            \
    } while (0)

// MH_OK's check without the return: the error into rc (for loops that must clean up)
#define MH_RC(rc, expr)                                                                              \
    do {                                                                                             \
        hipError_t e_ = (expr);                                                                      \
        if (e_ != hipSuccess) {                                                                      \
            gm_set_err("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, __LINE__); \
            rc = GMOE_ERR_HIP;                                                                       \
        }                                                                                            \
    } while (0)

namespace {

struct AttnDev {
    float *attn_norm = nullptr, *q_a_norm = nullptr, *kv_a_norm = nullptr;
    int8_t *q_a_q = nullptr, *q_b_q = nullptr, *kv_a_q = nullptr, *k_b_q = nullptr, *v_b_q = nullptr, *out_q = nullptr;
    float *q_a_s = nullptr, *q_b_s = nullptr, *kv_a_s = nullptr, *k_b_s = nullptr, *v_b_s = nullptr, *out_s = nullptr;
    bool set = false;
};

}  // namespace

struct gmoe_model {
    int device = 0;
    int n_cu = 256;  // compute units of the device: k_attn_chunk fills them once per head group
    gmoe_model_config c{};
    gmoe_ctx *moe = nullptr;
    std::vector<uint8_t> moe_on;
    int moe_flags = 0;
    // model-wide tensors
    float *output_norm = nullptr, *tok_s = nullptr, *out_s = nullptr;
    int8_t *tok_q = nullptr, *out_q = nullptr;
    float *l0_norm = nullptr, *l0_gate_s = nullptr, *l0_up_s = nullptr, *l0_down_s = nullptr;
    int8_t *l0_gate_q = nullptr, *l0_up_q = nullptr, *l0_down_q = nullptr;
    bool globals = false;
    std::vector<AttnDev> attn;
    // the latent cache [attn_layers][cap][kv], [..][rope] and the rope table [cap][rope/2][2]
    float *comp = nullptr, *pe = nullptr, *rope_cs = nullptr;
    // activations, each [max_batch][..] (a single token uses the first row)
    float *x = nullptr, *q_a = nullptr, *q_full = nullptr, *kv_a = nullptr, *q_pe = nullptr, *q_abs = nullptr,
          *ctx = nullptr, *concat = nullptr, *ffh = nullptr, *logits = nullptr, *part_ctx = nullptr,
          *part_ml = nullptr, *saved = nullptr;
    // the caches' split fp16 form for the batch attention (dense.h: ksp rows, vsp blocks; null
    // where the shape does not take it), cap rounded up to 16 positions
    _Float16 *ksp = nullptr, *vsp = nullptr;
    size_t cap16 = 0;
    // positions stale_lo .. stale_hi - 1 hold fp32 entries a decode step wrote without their
    // split form (decode reads only the fp32 cache); a prefill converts them first
    int stale_lo = 0, stale_hi = 0;
    int32_t *tokens = nullptr;  // [max_batch] a prefill's token ids
    // a prefill's GEMM inputs (gemm.h): [max_batch][2][widest input] fp16, their exponents,
    // and 64 bytes of zeros
    __half *xs = nullptr;
    int *xe = nullptr;
    __half *zeros = nullptr;
    std::vector<void *> allocs;  // every device allocation, freed by gmoe_model_destroy
};

namespace {

template <typename T>
int mdalloc(gmoe_model *m, T **p, size_t n) {
    *p = nullptr;
    if (n == 0) n = 1;
    const hipError_t e = hipMalloc((void **)p, n * sizeof(T));
    if (e != hipSuccess) {
        gm_set_err("gmoe_model: hipMalloc of %zu bytes failed: %s", n * sizeof(T), hipGetErrorString(e));
        *p = nullptr;
        return GMOE_ERR_NOMEM;
    }
    m->allocs.push_back(*p);
    return GMOE_OK;
}

// Device copy of n elements from host src into *dst (allocated on first use).
template <typename T>
int upload(gmoe_model *m, T **dst, const T *src, size_t n, const char *what) {
    if (!src) {
        gm_set_err("gmoe_model: %s is missing", what);
        return GMOE_ERR_INVALID;
    }
    if (!*dst) {
        if (int rc = mdalloc(m, dst, n)) return rc;
    }
    MH_OK(hipMemcpy(*dst, src, n * sizeof(T), hipMemcpyHostToDevice));
    return GMOE_OK;
}

// The k_gemv instance for cols columns: 16 lanes per row up to 64 units of 16 columns,
// a whole wave per row beyond (at most 640 units).
template <int MODE>
int launch_gemv_mode(const GemvArgs &a, hipStream_t st, int nb) {
    const int units = a.cols >> 4;
    const int lpr = units <= 64 ? 16 : 64;
    const int rpw = 64 / lpr, nrg = (a.rows + a.rows_b + rpw - 1) / rpw;
    const dim3 grid((unsigned)std::min((nrg + 3) / 4, 2048), (unsigned)nb), block(DM_BLOCK);
    if (lpr == 16) {
        switch ((units + 15) / 16) {
        case 1: hipLaunchKernelGGL((k_gemv<16, 1, MODE>), grid, block, 0, st, a); break;
        case 2: hipLaunchKernelGGL((k_gemv<16, 2, MODE>), grid, block, 0, st, a); break;
        case 3: hipLaunchKernelGGL((k_gemv<16, 3, MODE>), grid, block, 0, st, a); break;
        default: hipLaunchKernelGGL((k_gemv<16, 4, MODE>), grid, block, 0, st, a); break;
        }
    } else {
        switch ((units + 63) / 64) {
        case 2: hipLaunchKernelGGL((k_gemv<64, 2, MODE>), grid, block, 0, st, a); break;
        case 3: hipLaunchKernelGGL((k_gemv<64, 3, MODE>), grid, block, 0, st, a); break;
        case 4: hipLaunchKernelGGL((k_gemv<64, 4, MODE>), grid, block, 0, st, a); break;
        case 5: hipLaunchKernelGGL((k_gemv<64, 5, MODE>), grid, block, 0, st, a); break;
        case 6: hipLaunchKernelGGL((k_gemv<64, 6, MODE>), grid, block, 0, st, a); break;
        case 7:
        case 8: hipLaunchKernelGGL((k_gemv<64, 8, MODE>), grid, block, 0, st, a); break;
        default: hipLaunchKernelGGL((k_gemv<64, 10, MODE>), grid, block, 0, st, a); break;
        }
    }
    return GMOE_OK;
}

// k_attn_query for nb tokens: kb (the k_b product, batched) and one prep block per token.
template <int LPR, int U>
void launch_query_lu(const GemvArgs &kb, const AttnArgs &aa, dim3 grid, hipStream_t st) {
    hipLaunchKernelGGL((k_attn_query<LPR, U>), grid, dim3(DM_BLOCK), 0, st, kb, aa);
}

// k_attn_query's prep blocks alone (the cache entries and rotated queries of nb tokens).
void launch_prep(const GemvArgs &kb, const AttnArgs &aa, hipStream_t st, int nb) {
    launch_query_lu<16, 1>(kb, aa, dim3(1, (unsigned)nb), st);
}

int launch_query(const GemvArgs &kb, const AttnArgs &aa, hipStream_t st, int nb) {
    const int units = kb.cols >> 4;
    const int lpr = units <= 64 ? 16 : 64;
    const int rpw = 64 / lpr, nrg = (kb.rows + rpw - 1) / rpw;
    const dim3 grid((unsigned)std::min((nrg + 3) / 4, 2048) + 1, (unsigned)nb);
    if (lpr == 16) {
        switch ((units + 15) / 16) {
        case 1: launch_query_lu<16, 1>(kb, aa, grid, st); break;
        case 2: launch_query_lu<16, 2>(kb, aa, grid, st); break;
        case 3: launch_query_lu<16, 3>(kb, aa, grid, st); break;
        default: launch_query_lu<16, 4>(kb, aa, grid, st); break;
        }
    } else {
        switch ((units + 63) / 64) {
        case 2: launch_query_lu<64, 2>(kb, aa, grid, st); break;
        case 3: launch_query_lu<64, 3>(kb, aa, grid, st); break;
        case 4: launch_query_lu<64, 4>(kb, aa, grid, st); break;
        case 5: launch_query_lu<64, 5>(kb, aa, grid, st); break;
        case 6: launch_query_lu<64, 6>(kb, aa, grid, st); break;
        case 7:
        case 8: launch_query_lu<64, 8>(kb, aa, grid, st); break;
        default: launch_query_lu<64, 10>(kb, aa, grid, st); break;
        }
    }
    return GMOE_OK;
}

// The rows per wave of k_gemv for cols columns (a second matrix's rows start on a multiple).
int gemv_rows_per_wave(int cols) { return (cols >> 4) <= 64 ? 4 : 1; }

// One launch for nb tokens (a.bx, a.by, a.br apart).
int launch_gemv(const GemvArgs &a, int mode, hipStream_t st, int nb = 1) {
    if (mode == GV_RESID) return launch_gemv_mode<GV_RESID>(a, st, nb);
    if (mode == GV_PAIR) return launch_gemv_mode<GV_PAIR>(a, st, nb);
    return launch_gemv_mode<GV_PLAIN>(a, st, nb);
}

// gemv() over a batch: token t's input x + t bx, output y + t by.
GemvArgs batched(GemvArgs a, int bx, int by) {
    a.bx = bx;
    a.by = by;
    return a;
}

// y = q . x for one shared input (normalised by norm when given).
GemvArgs gemv(const int8_t *q, const float *s, const float *x, const float *norm, float *y, int rows, int cols, int gs) {
    GemvArgs a{};
    a.q = q;
    a.s = s;
    a.x = x;
    a.norm = norm;
    a.y = y;
    a.rows = rows;
    a.cols = cols;
    a.gs = gs;
    a.x_rows = 1 << 30;
    a.x_stride = 0;
    a.bx = a.by = a.br = 0;
    a.qb = nullptr;
    a.sb = nullptr;
    a.yb = nullptr;
    a.rows_b = a.by_b = 0;
    return a;
}

// a (GV_PLAIN) and b, two products of the same input and norm, in one launch when a's rows
// end on a row group of the kernel (else b is left for its own launch: returns false).
bool fuse_second(GemvArgs &a, const GemvArgs &b) {
    if (a.rows % gemv_rows_per_wave(a.cols) || b.cols != a.cols) return false;
    a.qb = b.q;
    a.sb = b.s;
    a.yb = b.y;
    a.rows_b = b.rows;
    a.by_b = b.by;
    return true;
}

constexpr int kMaxCols = 16 * 64 * 10;  // the widest k_gemv instance
static_assert(kMaxCols <= QG_SPLIT_MAX * QG_BLOCK, "k_norm_split holds a whole row");

int check_config(const gmoe_model_config &c) {
    const int gs = c.group_size;
    auto cols_ok = [&](int n) { return n > 0 && n % 16 == 0 && n % gs == 0 && n <= kMaxCols; };
    if (gs < 16 || gs % 16 || c.dim <= 0 || c.n_layers < 1 || c.vocab_size < 1) {
        gm_set_err("gmoe_model_create: need group_size a multiple of 16 and positive dim, n_layers, vocab_size");
        return GMOE_ERR_INVALID;
    }
    if (!cols_ok(c.dim)) {
        gm_set_err("gmoe_model_create: dim %d must be a multiple of 16 and of group_size, at most %d", c.dim, kMaxCols);
        return GMOE_ERR_INVALID;
    }
    if (c.has_l0_ffn && !cols_ok(c.hidden_dim)) {
        gm_set_err("gmoe_model_create: hidden_dim %d must be a multiple of 16 and of group_size, at most %d", c.hidden_dim,
                   kMaxCols);
        return GMOE_ERR_INVALID;
    }
    if (c.attn_layers != 0 && c.attn_layers != 1 && c.attn_layers != c.n_layers) {
        gm_set_err("gmoe_model_create: attn_layers must be 0, 1 or n_layers (got %d)", c.attn_layers);
        return GMOE_ERR_INVALID;
    }
    if (c.max_batch < 0 || c.max_batch > 65536) {
        gm_set_err("gmoe_model_create: max_batch %d outside 0..65536", c.max_batch);
        return GMOE_ERR_INVALID;
    }
    if (c.cache_cap < 1 || c.cache_cap > 65536) {
        gm_set_err("gmoe_model_create: cache_cap %d outside 1..65536", c.cache_cap);
        return GMOE_ERR_INVALID;
    }
    if (c.attn_layers > 0) {
        const int H = c.n_heads, kv = c.kv_lora_rank, rope = c.rope_dim;
        if (H < 1 || kv < 64 || kv % 64 || kv > AT_KV_MAX || rope < 2 || rope % 2 || rope > AT_ROPE_MAX ||
            c.head_k_dim != c.qk_nope_dim + rope || c.head_k_dim % 4 || c.v_head_dim < 4 || c.v_head_dim % 4 ||
            !cols_ok(c.q_lora_rank) || !cols_ok(c.qk_nope_dim) || !cols_ok(kv) || !cols_ok(H * c.v_head_dim)) {
            gm_set_err("gmoe_model_create: attention shape not supported (heads %d, q_lora %d, kv_lora %d, rope %d, "
                       "nope %d, head_k %d, v_head %d, group %d): kv_lora a multiple of 64 up to %d, rope even up to %d, "
                       "head_k = nope + rope, every product's columns multiples of 16 and of the group",
                       H, c.q_lora_rank, kv, rope, c.qk_nope_dim, c.head_k_dim, c.v_head_dim, gs, AT_KV_MAX, AT_ROPE_MAX);
            return GMOE_ERR_INVALID;
        }
    }
    return GMOE_OK;
}

// The arguments of layer l's attention kernels for a token at position pos.
AttnArgs attn_args(gmoe_model *m, int l, int pos) {
    const gmoe_model_config &c = m->c;
    const int H = c.n_heads, kv = c.kv_lora_rank, rope = c.rope_dim;
    AttnArgs aa{};
    aa.kv_a = m->kv_a;
    aa.kv_norm = m->attn[l].kv_a_norm;
    aa.q_full = m->q_full;
    aa.rope_cs = m->rope_cs;
    aa.comp = m->comp + (size_t)l * c.cache_cap * kv;
    aa.pe = m->pe + (size_t)l * c.cache_cap * rope;
    aa.q_pe = m->q_pe;
    aa.q_abs = m->q_abs;
    aa.part_ctx = m->part_ctx;
    aa.part_ml = m->part_ml;
    aa.ctx = m->ctx;
    aa.ksp = m->ksp ? m->ksp + (size_t)l * m->cap16 * SPL_KROW : nullptr;
    aa.vsp = m->vsp ? m->vsp + (size_t)l * m->cap16 * 2 * kv : nullptr;
    aa.H = H;
    aa.kv = kv;
    aa.rope = rope;
    aa.head_k = c.head_k_dim;
    aa.nope = c.qk_nope_dim;
    aa.pos = pos;
    const int groups = (H + AT_HG - 1) / AT_HG;  // blocks per chunk, heads spread evenly over them
    aa.hg = (H + groups - 1) / groups;
    aa.kq_scale = 1.0f / sqrtf((float)c.head_k_dim);  // infer.c:992
    return aa;
}

// Position ranges of the attention over pos + 1 positions: about 32 positions each (a tile's
// worth), at most one block per CU over all head groups.
int attn_ranges(int n_cu, int groups, int positions) {
    const int by_len = (positions + 31) / 32, by_cu = std::max(1, n_cu / groups);
    return std::min(std::min(by_len, by_cu), AT_MAX_PARTS);
}

// The attention over the cache for one token (q_abs, q_pe of aa.pos into ctx): the ranges,
// then their merge.
void launch_attn_cache(gmoe_model *m, AttnArgs aa, hipStream_t st) {
    const int groups = (aa.H + aa.hg - 1) / aa.hg;
    aa.nblk = attn_ranges(m->n_cu, groups, aa.pos + 1);
    hipLaunchKernelGGL(k_attn_chunk, dim3(aa.nblk, groups), dim3(AT_BLOCK), 0, st, aa);
    hipLaunchKernelGGL(k_attn_merge, dim3(aa.H, aa.kv / 64), dim3(DM_BLOCK), 0, st, aa);
}

// The attention over the cache for n tokens at positions aa.pos .. aa.pos + n - 1 (their
// cache entries already written): one launch of ranges for the whole batch (grid z = token,
// up to AT_PREFILL_RANGES ranges each, so that the tokens' blocks share the CUs), then one
// merge.
// The merge of n tokens' ranges: a wave per (token, head) where at most AM_SMALL ranges
// were written (GMOE_ATTN_MERGE_WIDE=1 forces k_attn_merge's block per 64 columns, a
// diagnostic: the two give the same bits).
void launch_attn_merge(const AttnArgs &aa, int n, hipStream_t st) {
    const char *env = getenv("GMOE_ATTN_MERGE_WIDE");
    const bool wide = env && env[0] == '1';
    if (aa.nblk <= AM_SMALL && !wide)
        hipLaunchKernelGGL(k_attn_merge_small, dim3((unsigned)((n * aa.H + DM_BLOCK / 64 - 1) / (DM_BLOCK / 64))),
                           dim3(DM_BLOCK), 0, st, aa, n);
    else
        hipLaunchKernelGGL(k_attn_merge, dim3(aa.H, aa.kv / 64, (unsigned)n), dim3(DM_BLOCK), 0, st, aa);
}

void launch_attn_cache_batch(gmoe_model *m, AttnArgs aa, int n, hipStream_t st) {
    const int groups = (aa.H + aa.hg - 1) / aa.hg;
    aa.nblk = std::min(AT_PREFILL_RANGES, std::max(1, m->n_cu / groups));
    hipLaunchKernelGGL(k_attn_chunk, dim3(aa.nblk, groups, (unsigned)n), dim3(AT_BLOCK), 0, st, aa);
    launch_attn_merge(aa, n, st);
}

// Whether k_attn_tile takes this model's attention: 16-column groups of the entry and of
// each part, and an entry that the staging holds.
bool attn_tile_ok(const gmoe_model_config &c) {
    return c.kv_lora_rank % 64 == 0 && c.rope_dim % 16 == 0 && c.kv_lora_rank + c.rope_dim <= AQ_KQ_MAX;
}

// The attention of n tokens at positions aa.pos .. (their cache entries already written) by
// query tiles: each token's positions in as few chunks (at most its AT_PREFILL_RANGES
// partial-result slots) as keep the CUs busy, since every chunk's partial results are
// written and merged; then k_attn_merge over each token's chunks.
void launch_attn_tile(gmoe_model *m, AttnArgs aa, int n, hipStream_t st) {
    const int P = aa.pos + n;  // positions any token of the batch attends
    // chunks per token: about AQ_BLOCKS_PER_CU blocks per CU over the tiles and heads
    const int tiles = (n + AQ_T - 1) / AQ_T;
    const int want = (AQ_BLOCKS_PER_CU * m->n_cu + tiles * aa.H - 1) / (tiles * aa.H);
    const int nch = std::min(AT_PREFILL_RANGES, std::max(1, want));
    const int per = (P + nch - 1) / nch;
    AttnTileArgs g;
    g.n = n;
    g.chunk = std::max(AQ_P, (per + AQ_P - 1) / AQ_P * AQ_P);
    aa.nblk = (P + g.chunk - 1) / g.chunk;
    g.a = aa;
    const dim3 grid((unsigned)aa.nblk, (unsigned)tiles, (unsigned)aa.H);
    // fp16 matrix cores on the cache's split form (attn16.h; the model keeps it where the shape
    // fits); GMOE_ATTN_TILE_FP32=1 keeps the fp32 MFMA kernel (a diagnostic and the tests'
    // reference for the split form)
    const char *env = getenv("GMOE_ATTN_TILE_FP32");
    if (!(env && env[0] == '1') && aa.ksp) {
        hipLaunchKernelGGL(k_attn_tile16, grid, dim3(AQ_BLOCK), 0, st, g);
    } else {
        switch (aq_rounds(aa.kv + aa.rope)) {
        case 1: hipLaunchKernelGGL(k_attn_tile<1>, grid, dim3(AQ_BLOCK), 0, st, g); break;
        case 2: hipLaunchKernelGGL(k_attn_tile<2>, grid, dim3(AQ_BLOCK), 0, st, g); break;
        default: hipLaunchKernelGGL(k_attn_tile<3>, grid, dim3(AQ_BLOCK), 0, st, g); break;
        }
    }
    launch_attn_merge(aa, n, st);
}
static_assert(aq_rounds(AQ_KQ_MAX) <= 3, "k_attn_tile instances cover the widest entry");

int attention(gmoe_model *m, int l, int pos, hipStream_t st) {
    const gmoe_model_config &c = m->c;
    const AttnDev &A = m->attn[l];
    const int gs = c.group_size, H = c.n_heads, kv = c.kv_lora_rank, rope = c.rope_dim;
    {
        GemvArgs qa = gemv(A.q_a_q, A.q_a_s, m->x, A.attn_norm, m->q_a, c.q_lora_rank, c.dim, gs);
        const GemvArgs kva = gemv(A.kv_a_q, A.kv_a_s, m->x, A.attn_norm, m->kv_a, kv + rope, c.dim, gs);
        if (!fuse_second(qa, kva)) launch_gemv(kva, GV_PLAIN, st);
        launch_gemv(qa, GV_PLAIN, st);
    }
    launch_gemv(gemv(A.q_b_q, A.q_b_s, m->q_a, A.q_a_norm, m->q_full, H * c.head_k_dim, c.q_lora_rank, gs), GV_PLAIN, st);
    AttnArgs aa = attn_args(m, l, pos);
    aa.ksp = aa.vsp = nullptr;  // the split form waits for the next prefill (k_spl_fill)
    // the query absorbed into the latent space, per head: k_b_h [kv][nope] . q_nope_h, with
    // the cache entry and the rotated queries in the same launch
    GemvArgs kb = gemv(A.k_b_q, A.k_b_s, m->q_full, nullptr, m->q_abs, H * kv, c.qk_nope_dim, gs);
    kb.x_rows = kv;
    kb.x_stride = c.head_k_dim;
    launch_query(kb, aa, st, 1);
    launch_attn_cache(m, aa, st);
    // back out of the latent space, per head: v_b_h [v_head][kv] . ctx_h
    GemvArgs vb = gemv(A.v_b_q, A.v_b_s, m->ctx, nullptr, m->concat, H * c.v_head_dim, kv, gs);
    vb.x_rows = c.v_head_dim;
    vb.x_stride = kv;
    launch_gemv(vb, GV_PLAIN, st);
    GemvArgs ao = gemv(A.out_q, A.out_s, m->concat, nullptr, m->x, c.dim, H * c.v_head_dim, gs);
    ao.resid = m->x;
    launch_gemv(ao, GV_RESID, st);
    return GMOE_OK;
}

int dense_ffn(gmoe_model *m, hipStream_t st) {
    const gmoe_model_config &c = m->c;
    GemvArgs gu = gemv(m->l0_gate_q, m->l0_gate_s, m->x, m->l0_norm, m->ffh, c.hidden_dim, c.dim, c.group_size);
    gu.q2 = m->l0_up_q;
    gu.s2 = m->l0_up_s;
    launch_gemv(gu, GV_PAIR, st);
    GemvArgs dn = gemv(m->l0_down_q, m->l0_down_s, m->ffh, nullptr, m->x, c.dim, c.hidden_dim, c.group_size);
    dn.resid = m->x;
    launch_gemv(dn, GV_RESID, st);
    return GMOE_OK;
}

// attention() over a batch: n tokens of x at positions pos0 .. pos0+n-1. Every product is one
// launch for the batch; every token's cache entry is written before any token's scores
// (token t reads positions up to pos0 + t only), then the attention over the cache runs
// per token, since its length differs.
// Whether a batch of n tokens takes the GEMMs of gemm.h for its dense products (a weight
// panel read once per QG_TT tokens) rather than k_gemv per token: a batch of a few tokens
// gains nothing from tiles. Group sizes 16 (glm.c's exporter) and 32 take it.
bool gemm_batch(const gmoe_model *m, int n) {
    const int gs = m->c.group_size;
    return m->xs && n >= QG_GEMM_MIN_TOKENS && (gs == 16 || gs == 32);
}

// The n tokens' inputs x (ldx apart, cols columns), normalised by norm when given, into
// the GEMM's split buffer.
void gemm_inputs(gmoe_model *m, const float *x, int ldx, int cols, const float *norm, int n, hipStream_t st) {
    const dim3 grid((unsigned)n), block(QG_BLOCK);
    if (cols <= 2 * QG_BLOCK) hipLaunchKernelGGL(k_norm_split<2>, grid, block, 0, st, x, ldx, cols, norm, m->xs, m->xe);
    else if (cols <= 8 * QG_BLOCK) hipLaunchKernelGGL(k_norm_split<8>, grid, block, 0, st, x, ldx, cols, norm, m->xs, m->xe);
    else if (cols <= 20 * QG_BLOCK) hipLaunchKernelGGL(k_norm_split<20>, grid, block, 0, st, x, ldx, cols, norm, m->xs, m->xe);
    else hipLaunchKernelGGL(k_norm_split<QG_SPLIT_MAX>, grid, block, 0, st, x, ldx, cols, norm, m->xs, m->xe);
}

// y = q . v for the n tokens' split inputs (gemm_inputs, cols columns): rows of group g
// (x_rows each) read input columns g * x_stride .. (x_rows = rows: one group); mode
// QG_PLAIN, QG_RESID (y = resid + dot) or QG_PAIR (y = silu(q . v) * (q2 . v)).
void gemm_launch(gmoe_model *m, const int8_t *q, const float *s, const int8_t *q2, const float *s2, int rows, int cols,
                 int x_rows, int x_stride, int xcols, float *y, int ldy, const float *resid, int ldr, int mode, int n,
                 hipStream_t st) {
    QgArgs a{};
    a.q = q;
    a.s = s;
    a.q2 = q2;
    a.s2 = s2;
    a.xs = m->xs;
    a.xe = m->xe;
    a.zeros = m->zeros;
    a.y = y;
    a.resid = resid;
    a.rows = rows;
    a.cols = cols;
    a.gs = m->c.group_size;
    a.n = n;
    a.xcols = xcols;
    a.ldy = ldy;
    a.ldr = ldr;
    a.x_rows = x_rows;
    a.x_stride = x_stride;
    a.bpg = (x_rows + 63) / 64;
    a.groups = (rows + x_rows - 1) / x_rows;
    a.tiles = (n + QG_TT - 1) / QG_TT;
    const int panels = a.bpg * a.groups;
    const dim3 grid((unsigned)(QG_XCD * ((panels + QG_XCD - 1) / QG_XCD) * a.tiles));
    const bool k32 = a.gs % 32 == 0 && cols % 32 == 0;
    if (k32) {
        if (mode == QG_PAIR) hipLaunchKernelGGL((k_gemm_q8<32, QG_PAIR>), grid, dim3(QG_BLOCK), 0, st, a);
        else if (mode == QG_RESID) hipLaunchKernelGGL((k_gemm_q8<32, QG_RESID>), grid, dim3(QG_BLOCK), 0, st, a);
        else hipLaunchKernelGGL((k_gemm_q8<32, QG_PLAIN>), grid, dim3(QG_BLOCK), 0, st, a);
    } else {
        if (mode == QG_PAIR) hipLaunchKernelGGL((k_gemm_q8<16, QG_PAIR>), grid, dim3(QG_BLOCK), 0, st, a);
        else if (mode == QG_RESID) hipLaunchKernelGGL((k_gemm_q8<16, QG_RESID>), grid, dim3(QG_BLOCK), 0, st, a);
        else hipLaunchKernelGGL((k_gemm_q8<16, QG_PLAIN>), grid, dim3(QG_BLOCK), 0, st, a);
    }
}

int attention_batch(gmoe_model *m, int l, int pos0, int n, hipStream_t st) {
    const gmoe_model_config &c = m->c;
    const AttnDev &A = m->attn[l];
    const int gs = c.group_size, H = c.n_heads, kv = c.kv_lora_rank, rope = c.rope_dim, D = c.dim;
    const int ql = c.q_lora_rank, hk = c.head_k_dim, vh = c.v_head_dim;
    if (gemm_batch(m, n)) {
        gemm_inputs(m, m->x, D, D, A.attn_norm, n, st);
        gemm_launch(m, A.q_a_q, A.q_a_s, nullptr, nullptr, ql, D, ql, 0, D, m->q_a, ql, nullptr, 0, QG_PLAIN, n, st);
        gemm_launch(m, A.kv_a_q, A.kv_a_s, nullptr, nullptr, kv + rope, D, kv + rope, 0, D, m->kv_a, kv + rope, nullptr,
                    0, QG_PLAIN, n, st);
        gemm_inputs(m, m->q_a, ql, ql, A.q_a_norm, n, st);
        gemm_launch(m, A.q_b_q, A.q_b_s, nullptr, nullptr, H * hk, ql, H * hk, 0, ql, m->q_full, H * hk, nullptr, 0,
                    QG_PLAIN, n, st);
    } else {
        GemvArgs qa = batched(gemv(A.q_a_q, A.q_a_s, m->x, A.attn_norm, m->q_a, ql, D, gs), D, ql);
        const GemvArgs kva = batched(gemv(A.kv_a_q, A.kv_a_s, m->x, A.attn_norm, m->kv_a, kv + rope, D, gs), D, kv + rope);
        if (!fuse_second(qa, kva)) launch_gemv(kva, GV_PLAIN, st, n);
        launch_gemv(qa, GV_PLAIN, st, n);
        launch_gemv(batched(gemv(A.q_b_q, A.q_b_s, m->q_a, A.q_a_norm, m->q_full, H * hk, ql, gs), ql, H * hk), GV_PLAIN, st, n);
    }
    const AttnArgs aa = attn_args(m, l, pos0);
    GemvArgs kb = batched(gemv(A.k_b_q, A.k_b_s, m->q_full, nullptr, m->q_abs, H * kv, c.qk_nope_dim, gs), H * hk, H * kv);
    kb.x_rows = kv;
    kb.x_stride = hk;
    if (gemm_batch(m, n)) {
        // the absorbed queries as one GEMM (group h: k_b_h . q_nope_h), then the cache entries
        // and rotated queries (k_attn_query's last block alone)
        gemm_inputs(m, m->q_full, H * hk, H * hk, nullptr, n, st);
        gemm_launch(m, A.k_b_q, A.k_b_s, nullptr, nullptr, H * kv, c.qk_nope_dim, kv, hk, H * hk, m->q_abs, H * kv,
                    nullptr, 0, QG_PLAIN, n, st);
        launch_prep(kb, aa, st, n);
    } else {
        launch_query(kb, aa, st, n);  // every token's cache entry before any token's attention
    }
    if (attn_tile_ok(c))
        launch_attn_tile(m, aa, n, st);
    else
        launch_attn_cache_batch(m, aa, n, st);
    if (gemm_batch(m, n)) {
        // per head: concat_h = v_b_h . ctx_h, then x += attn_out . concat
        gemm_inputs(m, m->ctx, H * kv, H * kv, nullptr, n, st);
        gemm_launch(m, A.v_b_q, A.v_b_s, nullptr, nullptr, H * vh, kv, vh, kv, H * kv, m->concat, H * vh, nullptr, 0,
                    QG_PLAIN, n, st);
        gemm_inputs(m, m->concat, H * vh, H * vh, nullptr, n, st);
        gemm_launch(m, A.out_q, A.out_s, nullptr, nullptr, D, H * vh, D, 0, H * vh, m->x, D, m->x, D, QG_RESID, n, st);
        return GMOE_OK;
    }
    GemvArgs vb = batched(gemv(A.v_b_q, A.v_b_s, m->ctx, nullptr, m->concat, H * vh, kv, gs), H * kv, H * vh);
    vb.x_rows = vh;
    vb.x_stride = kv;
    launch_gemv(vb, GV_PLAIN, st, n);
    GemvArgs ao = batched(gemv(A.out_q, A.out_s, m->concat, nullptr, m->x, D, H * vh, gs), H * vh, D);
    ao.resid = m->x;
    ao.br = D;
    launch_gemv(ao, GV_RESID, st, n);
    return GMOE_OK;
}

// dense_ffn() over a batch of n tokens of x.
int dense_ffn_batch(gmoe_model *m, int n, hipStream_t st) {
    const gmoe_model_config &c = m->c;
    const int D = c.dim, F = c.hidden_dim;
    if (gemm_batch(m, n)) {
        gemm_inputs(m, m->x, D, D, m->l0_norm, n, st);
        gemm_launch(m, m->l0_gate_q, m->l0_gate_s, m->l0_up_q, m->l0_up_s, F, D, F, 0, D, m->ffh, F, nullptr, 0, QG_PAIR, n,
                    st);
        gemm_inputs(m, m->ffh, F, F, nullptr, n, st);
        gemm_launch(m, m->l0_down_q, m->l0_down_s, nullptr, nullptr, D, F, D, 0, F, m->x, D, m->x, D, QG_RESID, n, st);
        return GMOE_OK;
    }
    GemvArgs gu = batched(gemv(m->l0_gate_q, m->l0_gate_s, m->x, m->l0_norm, m->ffh, F, D, c.group_size), D, F);
    gu.q2 = m->l0_up_q;
    gu.s2 = m->l0_up_s;
    launch_gemv(gu, GV_PAIR, st, n);
    GemvArgs dn = batched(gemv(m->l0_down_q, m->l0_down_s, m->ffh, nullptr, m->x, D, F, c.group_size), F, D);
    dn.resid = m->x;
    dn.br = D;
    launch_gemv(dn, GV_RESID, st, n);
    return GMOE_OK;
}

}  // namespace

extern "C" int gmoe_model_create(gmoe_model **out, int device, const gmoe_model_config *cfg) {
    if (!out || !cfg) {
        gm_set_err("gmoe_model_create: null argument");
        return GMOE_ERR_INVALID;
    }
    *out = nullptr;
    if (int rc = check_config(*cfg)) return rc;
    MH_OK(hipSetDevice(device));
    int n_cu = 0;
    MH_OK(hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, device));
    gmoe_model *m = new gmoe_model();
    m->device = device;
    m->n_cu = std::max(1, n_cu);
    m->c = *cfg;
    const gmoe_model_config &c = m->c;
    const size_t L = (size_t)c.n_layers, A = (size_t)c.attn_layers, cap = (size_t)c.cache_cap;
    const size_t H = (size_t)c.n_heads, kv = (size_t)c.kv_lora_rank, rope = (size_t)c.rope_dim;
    m->attn.resize(A);
    m->moe_on.assign(L, 0);
    int rc = GMOE_OK;
    const size_t B = (size_t)(c.max_batch > 1 ? c.max_batch : 1);
    // partial results: the most a token's launch uses, or AT_PREFILL_RANGES per token of a batch
    const size_t ranges = std::max((size_t)attn_ranges(m->n_cu, 1, (int)cap), B * AT_PREFILL_RANGES);
    rc |= mdalloc(m, &m->x, B * c.dim);
    rc |= mdalloc(m, &m->tokens, B);
    if (B >= QG_GEMM_MIN_TOKENS) {
        size_t w = (size_t)c.dim;
        if (c.has_l0_ffn) w = std::max(w, (size_t)c.hidden_dim);
        if (A > 0) w = std::max({w, (size_t)c.q_lora_rank, H * kv, H * (size_t)c.v_head_dim, H * (size_t)c.head_k_dim});
        rc |= mdalloc(m, &m->xs, B * 2 * w);
        rc |= mdalloc(m, &m->xe, B);
        rc |= mdalloc(m, &m->zeros, 64);
    }
    rc |= mdalloc(m, &m->logits, (size_t)c.vocab_size);
    if (c.has_l0_ffn) rc |= mdalloc(m, &m->ffh, B * c.hidden_dim);
    if (A > 0) {
        rc |= mdalloc(m, &m->comp, A * cap * kv);
        rc |= mdalloc(m, &m->pe, A * cap * rope);
        rc |= mdalloc(m, &m->rope_cs, cap * rope);
        rc |= mdalloc(m, &m->q_a, B * c.q_lora_rank);
        rc |= mdalloc(m, &m->q_full, B * H * c.head_k_dim);
        rc |= mdalloc(m, &m->kv_a, B * (kv + rope));
        rc |= mdalloc(m, &m->q_pe, B * H * rope);
        rc |= mdalloc(m, &m->q_abs, B * H * kv);
        rc |= mdalloc(m, &m->ctx, B * H * kv);
        rc |= mdalloc(m, &m->concat, B * H * c.v_head_dim);
        rc |= mdalloc(m, &m->part_ctx, ranges * H * kv);
        rc |= mdalloc(m, &m->part_ml, ranges * H * 2);
        rc |= mdalloc(m, &m->saved, A * (kv + rope));
        if (attn_tile_ok(c) && kv <= AT_KV_MAX) {
            m->cap16 = (cap + 15) / 16 * 16;
            rc |= mdalloc(m, &m->ksp, A * m->cap16 * SPL_KROW);
            rc |= mdalloc(m, &m->vsp, A * m->cap16 * 2 * kv);
        }
    }
    if (!rc && A > 0) {
        // glm.c's angles (infer.c:964-976): pair i of position p turns by p * 1e6^(-2i / rope)
        std::vector<float> cs(cap * rope);
        for (size_t p = 0; p < cap; p++)
            for (size_t i = 0; i + 1 < rope; i += 2) {
                const float freq = powf(1000000.0f, -((float)i / (float)rope));
                const float ang = (float)p * freq;
                cs[p * rope + i] = cosf(ang);
                cs[p * rope + i + 1] = sinf(ang);
            }
        if (hipMemcpy(m->rope_cs, cs.data(), cs.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
            gm_set_err("gmoe_model_create: copy of the rope table failed");
            rc = GMOE_ERR_HIP;
        }
        if (!rc && (hipMemset(m->comp, 0, A * cap * kv * sizeof(float)) != hipSuccess ||
                    hipMemset(m->pe, 0, A * cap * rope * sizeof(float)) != hipSuccess ||
                    (m->ksp && hipMemset(m->ksp, 0, A * m->cap16 * SPL_KROW * sizeof(_Float16)) != hipSuccess) ||
                    (m->vsp && hipMemset(m->vsp, 0, A * m->cap16 * 2 * kv * sizeof(_Float16)) != hipSuccess))) {
            gm_set_err("gmoe_model_create: clearing the cache failed");
            rc = GMOE_ERR_HIP;
        }
    }
    if (!rc && m->zeros && hipMemset(m->zeros, 0, 64) != hipSuccess) {
        gm_set_err("gmoe_model_create: clearing the GEMM's zero row failed");
        rc = GMOE_ERR_HIP;
    }
    if (rc) {
        gmoe_model_destroy(m);
        return rc;
    }
    *out = m;
    return GMOE_OK;
}

extern "C" void gmoe_model_destroy(gmoe_model *m) {
    if (!m) return;
    (void)hipSetDevice(m->device);
    for (void *p : m->allocs) (void)hipFree(p);
    delete m;
}

extern "C" int gmoe_model_upload(gmoe_model *m, const gmoe_model_weights *w) {
    if (!m || !w) {
        gm_set_err("gmoe_model_upload: null argument");
        return GMOE_ERR_INVALID;
    }
    MH_OK(hipSetDevice(m->device));
    const gmoe_model_config &c = m->c;
    const size_t D = (size_t)c.dim, V = (size_t)c.vocab_size, gs = (size_t)c.group_size, F = (size_t)c.hidden_dim;
    int rc = GMOE_OK;
    if (!rc) rc = upload(m, &m->output_norm, w->output_norm, D, "output_norm");
    if (!rc) rc = upload(m, &m->tok_q, w->tok_q, V * D, "tok_q");
    if (!rc) rc = upload(m, &m->tok_s, w->tok_s, V * D / gs, "tok_s");
    if (!rc) rc = upload(m, &m->out_q, w->out_q, V * D, "out_q");
    if (!rc) rc = upload(m, &m->out_s, w->out_s, V * D / gs, "out_s");
    if (c.has_l0_ffn) {
        if (!rc) rc = upload(m, &m->l0_norm, w->l0_ffn_norm, D, "l0_ffn_norm");
        if (!rc) rc = upload(m, &m->l0_gate_q, w->l0_ffn_gate_q, F * D, "l0_ffn_gate_q");
        if (!rc) rc = upload(m, &m->l0_gate_s, w->l0_ffn_gate_s, F * D / gs, "l0_ffn_gate_s");
        if (!rc) rc = upload(m, &m->l0_up_q, w->l0_ffn_up_q, F * D, "l0_ffn_up_q");
        if (!rc) rc = upload(m, &m->l0_up_s, w->l0_ffn_up_s, F * D / gs, "l0_ffn_up_s");
        if (!rc) rc = upload(m, &m->l0_down_q, w->l0_ffn_down_q, D * F, "l0_ffn_down_q");
        if (!rc) rc = upload(m, &m->l0_down_s, w->l0_ffn_down_s, D * F / gs, "l0_ffn_down_s");
    }
    m->globals = rc == GMOE_OK;
    return rc;
}

extern "C" int gmoe_model_upload_attn(gmoe_model *m, int layer, const gmoe_attn_weights *w) {
    if (!m || !w || layer < 0 || layer >= m->c.attn_layers) {
        gm_set_err("gmoe_model_upload_attn: bad arguments (layer %d of %d attention layers)", layer, m ? m->c.attn_layers : 0);
        return GMOE_ERR_INVALID;
    }
    MH_OK(hipSetDevice(m->device));
    const gmoe_model_config &c = m->c;
    const size_t D = (size_t)c.dim, gs = (size_t)c.group_size, H = (size_t)c.n_heads, ql = (size_t)c.q_lora_rank;
    const size_t kv = (size_t)c.kv_lora_rank, rope = (size_t)c.rope_dim, hk = (size_t)c.head_k_dim;
    const size_t nope = (size_t)c.qk_nope_dim, vh = (size_t)c.v_head_dim;
    AttnDev &A = m->attn[layer];
    int rc = GMOE_OK;
    if (!rc) rc = upload(m, &A.attn_norm, w->attn_norm, D, "attn_norm");
    if (!rc) rc = upload(m, &A.q_a_norm, w->q_a_norm, ql, "q_a_norm");
    if (!rc) rc = upload(m, &A.kv_a_norm, w->kv_a_norm, kv, "kv_a_norm");
    if (!rc) rc = upload(m, &A.q_a_q, w->q_a_q, ql * D, "q_a_q");
    if (!rc) rc = upload(m, &A.q_a_s, w->q_a_s, ql * D / gs, "q_a_s");
    if (!rc) rc = upload(m, &A.q_b_q, w->q_b_q, H * hk * ql, "q_b_q");
    if (!rc) rc = upload(m, &A.q_b_s, w->q_b_s, H * hk * ql / gs, "q_b_s");
    if (!rc) rc = upload(m, &A.kv_a_q, w->kv_a_q, (kv + rope) * D, "kv_a_q");
    if (!rc) rc = upload(m, &A.kv_a_s, w->kv_a_s, (kv + rope) * D / gs, "kv_a_s");
    if (!rc) rc = upload(m, &A.k_b_q, w->k_b_q, H * kv * nope, "k_b_q");
    if (!rc) rc = upload(m, &A.k_b_s, w->k_b_s, H * kv * nope / gs, "k_b_s");
    if (!rc) rc = upload(m, &A.v_b_q, w->v_b_q, H * vh * kv, "v_b_q");
    if (!rc) rc = upload(m, &A.v_b_s, w->v_b_s, H * vh * kv / gs, "v_b_s");
    if (!rc) rc = upload(m, &A.out_q, w->attn_out_q, D * H * vh, "attn_out_q");
    if (!rc) rc = upload(m, &A.out_s, w->attn_out_s, D * H * vh / gs, "attn_out_s");
    A.set = rc == GMOE_OK;
    return rc;
}

extern "C" int gmoe_model_set_moe(gmoe_model *m, gmoe_ctx *moe, const uint8_t *layers, int moe_flags) {
    if (!m) {
        gm_set_err("gmoe_model_set_moe: null model");
        return GMOE_ERR_INVALID;
    }
    m->moe = moe;
    m->moe_flags = moe_flags;
    for (int l = 0; l < m->c.n_layers; l++) m->moe_on[l] = moe && layers && l > 0 ? layers[l] : 0;
    return GMOE_OK;
}

namespace {
// Host buffers of the debug form ([n_layers][..] each; any may be null).
struct DebugOut {
    float *kv = nullptr, *concat = nullptr, *shexp = nullptr, *moe = nullptr;
};

int forward_token(gmoe_model *m, int token, int pos, int flags, float *logits, float *x_out, float *attn_ckpt,
                  float *layer_ckpt, const DebugOut *dbg, void *stream);
}  // namespace

extern "C" int gmoe_model_forward_token(gmoe_model *m, int token, int pos, int flags, float *logits, float *x_out,
                                        float *attn_ckpt, float *layer_ckpt, void *stream) {
    return forward_token(m, token, pos, flags, logits, x_out, attn_ckpt, layer_ckpt, nullptr, stream);
}

extern "C" int gmoe_model_forward_token_debug(gmoe_model *m, int token, int pos, int flags, float *logits,
                                              float *x_out, float *attn_ckpt, float *layer_ckpt, float *kv_out,
                                              float *concat_out, float *shexp_out, float *moe_out, void *stream) {
    DebugOut d;
    d.kv = kv_out;
    d.concat = concat_out;
    d.shexp = shexp_out;
    d.moe = moe_out;
    return forward_token(m, token, pos, flags, logits, x_out, attn_ckpt, layer_ckpt, &d, stream);
}

namespace {
int forward_token(gmoe_model *m, int token, int pos, int flags, float *logits, float *x_out, float *attn_ckpt,
                  float *layer_ckpt, const DebugOut *dbg, void *stream) {
    if (!m || !logits) {
        gm_set_err("gmoe_model_forward_token: null argument");
        return GMOE_ERR_INVALID;
    }
    const gmoe_model_config &c = m->c;
    if (!m->globals) {
        gm_set_err("gmoe_model_forward_token: gmoe_model_upload has not succeeded");
        return GMOE_ERR_INVALID;
    }
    for (int l = 0; l < c.attn_layers; l++)
        if (!m->attn[l].set) {
            gm_set_err("gmoe_model_forward_token: attention layer %d is not uploaded", l);
            return GMOE_ERR_INVALID;
        }
    if (c.attn_layers > 0 && (pos < 0 || pos >= c.cache_cap)) {
        gm_set_err("gmoe_model_forward_token: position %d outside the cache (%d positions)", pos, c.cache_cap);
        return GMOE_ERR_INVALID;
    }
    if (token < 0 || token >= c.vocab_size) token = 0;  // infer.c:1781
    MH_OK(hipSetDevice(m->device));
    hipStream_t st = (hipStream_t)stream;
    const size_t D = (size_t)c.dim, kv = (size_t)c.kv_lora_rank, rope = (size_t)c.rope_dim, cap = (size_t)c.cache_cap;
    const size_t A = (size_t)c.attn_layers;
    const bool keep = (flags & GMOE_MODEL_KEEP_CACHE) && A > 0;
    if (m->ksp && !keep) {
        m->stale_lo = m->stale_hi > m->stale_lo ? std::min(m->stale_lo, pos) : pos;
        m->stale_hi = std::max(m->stale_hi, pos + 1);
    }
    if (keep) {
        // the entries this position is about to overwrite, one per attention layer
        MH_OK(hipMemcpy2DAsync(m->saved, kv * sizeof(float), m->comp + pos * kv, cap * kv * sizeof(float),
                               kv * sizeof(float), A, hipMemcpyDeviceToDevice, st));
        MH_OK(hipMemcpy2DAsync(m->saved + A * kv, rope * sizeof(float), m->pe + pos * rope, cap * rope * sizeof(float),
                               rope * sizeof(float), A, hipMemcpyDeviceToDevice, st));
    }
    hipLaunchKernelGGL(k_embed, dim3((unsigned)((D + DM_BLOCK - 1) / DM_BLOCK)), dim3(DM_BLOCK), 0, st, m->tok_q, m->tok_s,
                       token, c.dim, c.group_size, m->x);
    // the three model forms of infer.c:1817-1881
    const int n_run = c.attn_layers == c.n_layers ? c.n_layers : 1;
    int rc = GMOE_OK;
    // the token's MoE layers on k_moe_relay share one reset launch (workspace layer w for
    // the w-th of them); other decode kernels take gmoe_forward per layer
    int n_moe = 0, relay = 0, w = 0;
    for (int l = 1; l < n_run; l++) {
        if (!m->moe_on[l]) continue;
        // every MoE layer must be able to run before the reset below: a token that stops
        // after it would leave workspace layers flipped but unwritten
        if (!gm_layer_ready(m->moe, l)) {
            gm_set_err("gmoe_model_forward_token: MoE layer %d is not uploaded to the model's context", l);
            return GMOE_ERR_INVALID;
        }
        n_moe++;
    }
    if (n_moe > 0) rc = gm_decode_begin(m->moe, n_moe, st, &relay);
    const size_t HV = (size_t)c.n_heads * c.v_head_dim;
    for (int l = 0; l < n_run && !rc; l++) {
        if (A > 0) rc = attention(m, l, pos, st);
        if (!rc && attn_ckpt) MH_RC(rc, hipMemcpyAsync(attn_ckpt + l * D, m->x, D * sizeof(float), hipMemcpyDeviceToHost, st));
        if (!rc && dbg && A > 0) {
            // the position's normalised kv entry (glm.c's kv_a, infer.c:1001-1003) and the heads' concat
            if (dbg->kv)
                MH_RC(rc, hipMemcpyAsync(dbg->kv + l * kv, m->comp + ((size_t)l * cap + pos) * kv, kv * sizeof(float),
                                         hipMemcpyDeviceToHost, st));
            if (!rc && dbg->concat)
                MH_RC(rc, hipMemcpyAsync(dbg->concat + l * HV, m->concat, HV * sizeof(float), hipMemcpyDeviceToHost, st));
        }
        if (!rc && l == 0 && c.has_l0_ffn) rc = dense_ffn(m, st);
        if (!rc && l > 0 && m->moe_on[l]) {
            rc = relay ? gm_decode_layer(m->moe, l, w++, m->x, m->x, m->moe_flags, st)
                       : gmoe_forward(m->moe, l, 1, m->x, m->x, m->moe_flags, st);
            if (!rc && dbg && (dbg->shexp || dbg->moe)) {
                const float *sh = nullptr, *ro = nullptr;
                gm_layer_outputs(m->moe, &sh, &ro);
                if (dbg->shexp && sh)
                    MH_RC(rc, hipMemcpyAsync(dbg->shexp + l * D, sh, D * sizeof(float), hipMemcpyDeviceToHost, st));
                if (!rc && dbg->moe && ro)
                    MH_RC(rc, hipMemcpyAsync(dbg->moe + l * D, ro, D * sizeof(float), hipMemcpyDeviceToHost, st));
            }
        }
        if (!rc && layer_ckpt) MH_RC(rc, hipMemcpyAsync(layer_ckpt + l * D, m->x, D * sizeof(float), hipMemcpyDeviceToHost, st));
    }
    if (rc) {
        if (relay) gm_decode_abort(m->moe);
        return rc;
    }
    launch_gemv(gemv(m->out_q, m->out_s, m->x, m->output_norm, m->logits, c.vocab_size, c.dim, c.group_size), GV_PLAIN, st);
    MH_OK(hipGetLastError());
    MH_OK(hipMemcpyAsync(logits, m->logits, (size_t)c.vocab_size * sizeof(float), hipMemcpyDeviceToHost, st));
    if (x_out) MH_OK(hipMemcpyAsync(x_out, m->x, D * sizeof(float), hipMemcpyDeviceToHost, st));
    if (keep) {
        MH_OK(hipMemcpy2DAsync(m->comp + pos * kv, cap * kv * sizeof(float), m->saved, kv * sizeof(float),
                               kv * sizeof(float), A, hipMemcpyDeviceToDevice, st));
        MH_OK(hipMemcpy2DAsync(m->pe + pos * rope, cap * rope * sizeof(float), m->saved + A * kv, rope * sizeof(float),
                               rope * sizeof(float), A, hipMemcpyDeviceToDevice, st));
    }
    MH_OK(hipStreamSynchronize(st));
    if (m->moe && gm_take_launch_error(m->moe)) return GMOE_ERR_HIP;
    return GMOE_OK;
}
}  // namespace

extern "C" int gmoe_model_prefill(gmoe_model *m, const int32_t *tokens, int n, int pos0, float *logits, float *x_out,
                                  void *stream) {
    if (!m || !tokens || !logits) {
        gm_set_err("gmoe_model_prefill: null argument");
        return GMOE_ERR_INVALID;
    }
    const gmoe_model_config &c = m->c;
    const int B = c.max_batch > 1 ? c.max_batch : 1;
    if (n < 1 || n > B) {
        gm_set_err("gmoe_model_prefill: %d tokens outside 1..%d (the model's max_batch)", n, B);
        return GMOE_ERR_INVALID;
    }
    if (!m->globals) {
        gm_set_err("gmoe_model_prefill: gmoe_model_upload has not succeeded");
        return GMOE_ERR_INVALID;
    }
    for (int l = 0; l < c.attn_layers; l++)
        if (!m->attn[l].set) {
            gm_set_err("gmoe_model_prefill: attention layer %d is not uploaded", l);
            return GMOE_ERR_INVALID;
        }
    if (c.attn_layers > 0 && (pos0 < 0 || pos0 + n > c.cache_cap)) {
        gm_set_err("gmoe_model_prefill: positions %d..%d outside the cache (%d positions)", pos0, pos0 + n - 1, c.cache_cap);
        return GMOE_ERR_INVALID;
    }
    MH_OK(hipSetDevice(m->device));
    hipStream_t st = (hipStream_t)stream;
    const size_t D = (size_t)c.dim;
    if (m->ksp && m->stale_hi > m->stale_lo) {
        // the entries decode steps wrote without their split form, before any attention of
        // this batch reads them
        hipLaunchKernelGGL(k_spl_fill, dim3((unsigned)(m->stale_hi - m->stale_lo), (unsigned)c.attn_layers), dim3(DM_BLOCK),
                           0, st, m->comp, m->pe, m->ksp, m->vsp, (size_t)c.cache_cap, m->cap16, c.kv_lora_rank, c.rope_dim,
                           m->stale_lo);
        m->stale_lo = m->stale_hi = 0;
    }
    MH_OK(hipMemcpyAsync(m->tokens, tokens, (size_t)n * sizeof(int32_t), hipMemcpyHostToDevice, st));
    hipLaunchKernelGGL(k_embed_batch, dim3((unsigned)((D + DM_BLOCK - 1) / DM_BLOCK), (unsigned)n), dim3(DM_BLOCK), 0, st,
                       m->tok_q, m->tok_s, m->tokens, c.vocab_size, c.dim, c.group_size, m->x);
    // the three model forms of infer.c:1817-1881, layer by layer over the batch
    const int n_run = c.attn_layers == c.n_layers ? c.n_layers : 1;
    int rc = GMOE_OK;
    for (int l = 0; l < n_run && !rc; l++) {
        if (c.attn_layers > 0) rc = attention_batch(m, l, pos0, n, st);
        if (!rc && l == 0 && c.has_l0_ffn) rc = dense_ffn_batch(m, n, st);
        if (!rc && l > 0 && m->moe_on[l]) rc = gmoe_forward(m->moe, l, n, m->x, m->x, m->moe_flags, st);
    }
    if (rc) return rc;
    const float *xl = m->x + (size_t)(n - 1) * D;  // the last token
    launch_gemv(gemv(m->out_q, m->out_s, xl, m->output_norm, m->logits, c.vocab_size, c.dim, c.group_size), GV_PLAIN, st);
    MH_OK(hipGetLastError());
    MH_OK(hipMemcpyAsync(logits, m->logits, (size_t)c.vocab_size * sizeof(float), hipMemcpyDeviceToHost, st));
    if (x_out) MH_OK(hipMemcpyAsync(x_out, xl, D * sizeof(float), hipMemcpyDeviceToHost, st));
    MH_OK(hipStreamSynchronize(st));
    if (m->moe && gm_take_launch_error(m->moe)) return GMOE_ERR_HIP;
    return GMOE_OK;
}

extern "C" int gmoe_model_read_cache(gmoe_model *m, int layer, int pos0, int n, float *comp_out, float *pe_out,
                                     void *stream) {
    if (!m || (!comp_out && !pe_out)) {
        gm_set_err("gmoe_model_read_cache: null argument");
        return GMOE_ERR_INVALID;
    }
    const gmoe_model_config &c = m->c;
    if (layer < 0 || layer >= c.attn_layers || pos0 < 0 || n < 1 || pos0 + n > c.cache_cap) {
        gm_set_err("gmoe_model_read_cache: layer %d, positions %d..%d outside %d attention layers x %d positions", layer,
                   pos0, pos0 + n - 1, c.attn_layers, c.cache_cap);
        return GMOE_ERR_INVALID;
    }
    MH_OK(hipSetDevice(m->device));
    hipStream_t st = (hipStream_t)stream;
    const size_t kv = (size_t)c.kv_lora_rank, rope = (size_t)c.rope_dim, row0 = (size_t)layer * c.cache_cap + pos0;
    if (comp_out)
        MH_OK(hipMemcpyAsync(comp_out, m->comp + row0 * kv, (size_t)n * kv * sizeof(float), hipMemcpyDeviceToHost, st));
    if (pe_out)
        MH_OK(hipMemcpyAsync(pe_out, m->pe + row0 * rope, (size_t)n * rope * sizeof(float), hipMemcpyDeviceToHost, st));
    MH_OK(hipStreamSynchronize(st));
    return GMOE_OK;
}
