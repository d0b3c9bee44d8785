/*
 * detref decoder forward — TEST INFRASTRUCTURE ONLY (the oracle).
 *
 * Restates crates/det-model/src/lib.rs of mii443/detllm:
 *   LlamaConfig::from_gguf / validate          lib.rs:1498-1616
 *   F32Llama::from_gguf + tensor readers       lib.rs:1035-1140, 1674-1953
 *   RopeTables::llama                          lib.rs:813-847
 *   KvCache                                    lib.rs:850-960
 *   forward_one_with_workspace                 lib.rs:1249-1400
 *   gemv dispatch (Q8A shared / Q8_K per call) lib.rs:445-655
 *   rmsnorm, apply_rope, attention, swiglu     lib.rs:2011-2434
 *   logits_hash_for_tokens_chunked             lib.rs:1406-1465
 * The row-partitioned thread pool restates gemv_rows_parallel
 * (lib.rs:291-321) and the per-head attention split (lib.rs:2198-2297):
 * both split only independent outputs, so results do not depend on the
 * thread count.
 */
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "detref.h"
#include "detref_gguf.h"
#include "detref_internal.h"

#define MIN_PARALLEL_ATTENTION_WORK 32768

enum { T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q8_0 = 8, T_Q4K = 12, T_Q6K = 14 };

typedef struct {
    int type; /* T_F32 (F16 tensors are widened to F32), T_Q8_0, T_Q4_0, T_Q4K, T_Q6K */
    size_t rows, cols, bpr;
    void *data;
    int owned;
} wmat;

typedef struct {
    float *attn_norm, *ffn_norm;
    float *bq, *bk, *bv;
    wmat wq, wk, wv, wo, gate, up, down;
} layer_w;

typedef struct {
    size_t block_count, d, ff, heads, kv_heads, context_length, rope_dim;
    float eps, attention_scale, rope_base;
    int split_half;
} cfg_t;

struct ref_model {
    cfg_t c;
    size_t head_dim, vocab;
    wmat emb, out;
    float *out_norm;
    layer_w *layers;
};

struct ref_session {
    const ref_model *m;
    size_t max_ctx;
    float *rope_cos, *rope_sin; /* [max_ctx][rope_dim/2] */
    float *kc, *vc;             /* [L][KV][ctx][hd] */
    float *x, *h, *q, *k, *v, *attn, *scores, *probs, *tmp, *gate, *up, *ffo;
    ref_q8a_block *q8a;
    ref_q8k_block *q8k;
};

/* ---------------------------------------------------------------------- */
/* thread pool                                                             */
/* ---------------------------------------------------------------------- */
static size_t g_threads_override = 0;
static int g_simd = 0;
void ref_set_threads(size_t threads) { g_threads_override = threads; }
/* Selects the AVX2 integer block dot for Q8_0 rows (the reference's simd
 * feature); its results are bit-identical to the scalar block dot. */
void ref_set_simd(int on) { g_simd = on; }
static size_t requested_threads(void) {
    if (g_threads_override) return g_threads_override;
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (size_t)n : 1;
}

typedef int (*item_fn)(void *ctx, size_t begin, size_t end);
typedef struct {
    pthread_t tid;
    item_fn fn;
    void *ctx;
    size_t begin, end;
    int status;
} job_t;

static void *job_main(void *p) {
    job_t *j = p;
    j->status = j->fn(j->ctx, j->begin, j->end);
    return NULL;
}

/* Split [0, n) into ceil(n/threads)-sized contiguous chunks, one thread
 * each (gemv_rows_parallel, lib.rs:291-321).  Returns the first error. */
static int run_partitioned(item_fn fn, void *ctx, size_t n, size_t threads) {
    if (threads > n) threads = n ? n : 1;
    if (threads <= 1 || n < 2) return fn(ctx, 0, n);
    size_t chunk = (n + threads - 1) / threads;
    size_t jobs = (n + chunk - 1) / chunk;
    job_t *js = calloc(jobs, sizeof(job_t));
    for (size_t i = 0; i < jobs; i++) {
        js[i].fn = fn;
        js[i].ctx = ctx;
        js[i].begin = i * chunk;
        js[i].end = (i + 1) * chunk < n ? (i + 1) * chunk : n;
        if (i) pthread_create(&js[i].tid, NULL, job_main, &js[i]);
    }
    job_main(&js[0]);
    int st = js[0].status;
    for (size_t i = 1; i < jobs; i++) {
        pthread_join(js[i].tid, NULL);
        if (!st && js[i].status) st = js[i].status;
    }
    free(js);
    return st;
}

/* ---------------------------------------------------------------------- */
/* helpers                                                                 */
/* ---------------------------------------------------------------------- */
static int finite_slice(const float *x, size_t n) {
    for (size_t i = 0; i < n; i++)
        if (!isfinite(x[i])) return 0;
    return 1;
}

static int map_quant(int q) {
    switch (q) {
    case QERR_OK: return REF_OK;
    case QERR_NON_FINITE_INPUT: case QERR_NON_FINITE_SCALE: case QERR_NON_FINITE_OUTPUT:
        return REF_ERR_NON_FINITE;
    default: return REF_ERR_SHAPE;
    }
}

static int map_meta(int g) { return g == G_METADATA_NOT_FOUND ? REF_ERR_MISSING_METADATA : REF_ERR_GGUF; }

/* rmsnorm: lib.rs:2053-2073 */
int ref_rmsnorm(const float *x, const float *w, float eps, size_t n, float *out) {
    if (n == 0) return REF_ERR_SHAPE;
    if (!finite_slice(x, n) || !finite_slice(w, n) || !isfinite(eps)) return REF_ERR_NON_FINITE;
    float ss = ref_sum_squares_f32(x, n);
    float m = ss / (float)n;
    float r = 1.0f / sqrtf(m + eps);
    if (!isfinite(r)) return REF_ERR_NON_FINITE;
    for (size_t i = 0; i < n; i++) {
        out[i] = (x[i] * r) * w[i];
        if (!isfinite(out[i])) return REF_ERR_NON_FINITE;
    }
    return REF_OK;
}

/* ---------------------------------------------------------------------- */
/* GEMV                                                                    */
/* ---------------------------------------------------------------------- */
typedef struct {
    const wmat *w;
    const float *x;
    const ref_q8a_block *qa;
    const ref_q8k_block *qk;
    float *out;
    int avx2;
} gemv_ctx;

static int gemv_rows_fn(void *p, size_t begin, size_t end) {
    gemv_ctx *g = p;
    const wmat *w = g->w;
    for (size_t r = begin; r < end; r++) {
        float v = 0.0f;
        int q = QERR_OK;
        switch (w->type) {
        case T_F32:
            v = ref_dot_f32((const float *)w->data + r * w->cols, g->x, w->cols);
            break;
        case T_Q8_0: {
            const ref_q8_0_block *b = (const ref_q8_0_block *)w->data + r * w->bpr;
            if (g->avx2) {
                float sum = 0.0f;
                for (size_t k = 0; k < w->bpr && !q; k++) {
                    if (!isfinite(b[k].d) || !isfinite(g->qa[k].d)) { q = QERR_NON_FINITE_SCALE; break; }
                    float blk = ref_dot_q8_0_q8a_block_avx2(&b[k], &g->qa[k]);
                    if (!isfinite(blk)) { q = QERR_NON_FINITE_OUTPUT; break; }
                    sum += blk;
                    if (!isfinite(sum)) q = QERR_NON_FINITE_OUTPUT;
                }
                v = sum;
            } else {
                q = ref_dot_q8_0_q8a(b, g->qa, w->bpr, &v);
            }
            break;
        }
        case T_Q4_0:
            q = ref_dot_q4_0_q8a((const ref_q4_0_block *)w->data + r * w->bpr, g->qa, w->bpr, &v);
            break;
        case T_Q4K:
            q = ref_dot_q4_k_q8a((const ref_q4k_block *)w->data + r * w->bpr, g->qa, w->bpr, &v);
            break;
        case T_Q6K:
            q = ref_dot_q6_k_q8k((const ref_q6k_block *)w->data + r * w->bpr, g->qk, w->bpr, &v);
            break;
        default: return REF_ERR_UNSUPPORTED_TENSOR_TYPE;
        }
        if (q) return map_quant(q);
        if (!isfinite(v)) return REF_ERR_NON_FINITE;
        g->out[r] = v;
    }
    return REF_OK;
}

static int needs_q8a(const wmat *w) { return w->type == T_Q8_0 || w->type == T_Q4_0 || w->type == T_Q4K; }

static int quantize_q8a_vec(const float *x, size_t n, ref_q8a_block *out) {
    if (n == 0 || n % QK) return REF_ERR_SHAPE;
    for (size_t b = 0; b < n / QK; b++) {
        int q = ref_q8a_block_quantize(x + b * QK, &out[b]);
        if (q) return map_quant(q);
    }
    return REF_OK;
}

static int quantize_q8k_vec(const float *x, size_t n, ref_q8k_block *out) {
    if (n == 0 || n % QKK) return REF_ERR_SHAPE;
    for (size_t b = 0; b < n / QKK; b++) {
        int q = ref_q8k_block_quantize(x + b * QKK, &out[b]);
        if (q) return map_quant(q);
    }
    return REF_OK;
}

/* gemv_with_optional_q8a_and_q8k_scratch (lib.rs:550-606) when qa is given;
 * gemv_with_quant_scratch (lib.rs:608-655) when quantize_own is set. */
static int gemv(const wmat *w, const float *x, const ref_q8a_block *qa, int quantize_own,
                ref_q8a_block *q8a_scratch, ref_q8k_block *q8k_scratch, float *out) {
    if (!finite_slice(x, w->cols)) return REF_ERR_NON_FINITE;
    gemv_ctx g = {w, x, qa, NULL, out, 0};
    int st;
    if (w->type == T_Q6K) {
        if ((st = quantize_q8k_vec(x, w->cols, q8k_scratch))) return st;
        g.qk = q8k_scratch;
    } else if (needs_q8a(w)) {
        if (quantize_own) {
            if ((st = quantize_q8a_vec(x, w->cols, q8a_scratch))) return st;
            g.qa = q8a_scratch;
        } else if (!qa) {
            return REF_ERR_SHAPE;
        }
    }
    g.avx2 = w->type == T_Q8_0 && g_simd && ref_cpu_has_avx2();
    return run_partitioned(gemv_rows_fn, &g, w->rows, requested_threads());
}

/* ---------------------------------------------------------------------- */
/* embedding rows (write_row_validated, lib.rs:667-746)                     */
/* ---------------------------------------------------------------------- */
static int write_row(const wmat *w, size_t row, float *out) {
    size_t dst = 0;
    switch (w->type) {
    case T_F32:
        memcpy(out, (const float *)w->data + row * w->cols, w->cols * 4);
        return REF_OK;
    case T_Q8_0: {
        const ref_q8_0_block *b = (const ref_q8_0_block *)w->data + row * w->bpr;
        for (size_t k = 0; k < w->bpr; k++)
            for (int i = 0; i < QK; i++) {
                float v = b[k].d * (float)b[k].q[i];
                if (!isfinite(v)) return REF_ERR_NON_FINITE;
                out[dst++] = v;
            }
        return REF_OK;
    }
    case T_Q4_0: {
        const ref_q4_0_block *b = (const ref_q4_0_block *)w->data + row * w->bpr;
        for (size_t k = 0; k < w->bpr; k++)
            for (int i = 0; i < QK; i++) {
                uint8_t nib = i < 16 ? (b[k].qs[i] & 0x0f) : (b[k].qs[i - 16] >> 4);
                float v = b[k].d * (float)((int)nib - 8);
                if (!isfinite(v)) return REF_ERR_NON_FINITE;
                out[dst++] = v;
            }
        return REF_OK;
    }
    case T_Q4K: {
        const ref_q4k_block *b = (const ref_q4k_block *)w->data + row * w->bpr;
        for (size_t k = 0; k < w->bpr; k++)
            for (int i = 0; i < QKK; i++) {
                float v = ref_q4_k_value(&b[k], i);
                if (!isfinite(v)) return REF_ERR_NON_FINITE;
                out[dst++] = v;
            }
        return REF_OK;
    }
    case T_Q6K: {
        const ref_q6k_block *b = (const ref_q6k_block *)w->data + row * w->bpr;
        for (size_t k = 0; k < w->bpr; k++)
            for (int i = 0; i < QKK; i++) {
                float v = ref_q6_k_value(&b[k], i);
                if (!isfinite(v)) return REF_ERR_NON_FINITE;
                out[dst++] = v;
            }
        return REF_OK;
    }
    default: return REF_ERR_UNSUPPORTED_TENSOR_TYPE;
    }
}

/* ---------------------------------------------------------------------- */
/* loading                                                                 */
/* ---------------------------------------------------------------------- */
static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

static int read_dense_f32(const g_file *g, const g_tensor *t, size_t n, float **out) {
    const uint8_t *data;
    size_t len;
    if (g_tensor_data(g, t, &data, &len)) return REF_ERR_GGUF;
    float *v = malloc(n * 4 + 4);
    if (t->type == T_F32) {
        if (len != n * 4) { free(v); return REF_ERR_SHAPE; }
        memcpy(v, data, n * 4);
        for (size_t i = 0; i < n; i++)
            if (!isfinite(v[i])) { free(v); return REF_ERR_NON_FINITE; }
    } else if (t->type == T_F16) {
        if (len != n * 2) { free(v); return REF_ERR_SHAPE; }
        for (size_t i = 0; i < n; i++) {
            uint16_t b = rd16(data + 2 * i);
            if (!ref_f16_is_finite(b)) { free(v); return REF_ERR_NON_FINITE; }
            v[i] = ref_f16_to_f32(b);
        }
    } else {
        free(v);
        return REF_ERR_UNSUPPORTED_TENSOR_TYPE;
    }
    *out = v;
    return REF_OK;
}

/* read_f32_vector (lib.rs:1674-1685) */
static int read_vec(const g_file *g, const char *name, size_t n, float **out) {
    const g_tensor *t;
    if (g_find_tensor(g, name, &t)) return REF_ERR_GGUF;
    if (t->ndim != 1 || t->dims[0] != n) return REF_ERR_SHAPE;
    uint64_t el;
    if (g_tensor_elements(t, &el)) return REF_ERR_SHAPE;
    return read_dense_f32(g, t, n, out);
}

static int read_opt_vec(const g_file *g, const char *name, size_t n, float **out) {
    const g_tensor *t;
    int e = g_find_tensor(g, name, &t);
    if (e == G_TENSOR_NOT_FOUND) { *out = NULL; return REF_OK; }
    if (e) return REF_ERR_GGUF;
    return read_vec(g, name, n, out);
}

/* read_weight_matrix (lib.rs:1778-1810) and the block readers (1812-1953) */
static int read_matrix(const g_file *g, const char *name, size_t rows, size_t cols, wmat *w) {
    const g_tensor *t;
    memset(w, 0, sizeof *w);
    if (g_find_tensor(g, name, &t)) return REF_ERR_GGUF;
    if (t->ndim != 2 || t->dims[0] != cols || t->dims[1] != rows) return REF_ERR_SHAPE;
    const uint8_t *data;
    size_t len;
    w->rows = rows;
    w->cols = cols;
    w->owned = 1;
    if (t->type == T_F32 || t->type == T_F16) {
        if (rows == 0 || cols == 0) return REF_ERR_SHAPE;
        w->type = T_F32;
        return read_dense_f32(g, t, rows * cols, (float **)&w->data);
    }
    if (t->type != T_Q8_0 && t->type != T_Q4_0 && t->type != T_Q4K && t->type != T_Q6K)
        return REF_ERR_UNSUPPORTED_TENSOR_TYPE;
    size_t bs = (t->type == T_Q4K || t->type == T_Q6K) ? QKK : QK;
    if (cols % bs) return REF_ERR_SHAPE;
    if (g_tensor_data(g, t, &data, &len)) return REF_ERR_GGUF;
    w->type = t->type;
    w->bpr = cols / bs;
    size_t nb = rows * w->bpr;
    switch (t->type) {
    case T_Q8_0: {
        if (len != nb * 34) return REF_ERR_SHAPE;
        ref_q8_0_block *b = malloc(nb * sizeof *b);
        for (size_t i = 0; i < nb; i++) {
            const uint8_t *p = data + i * 34;
            if (!ref_f16_is_finite(rd16(p))) { free(b); return REF_ERR_NON_FINITE; }
            b[i].d = ref_f16_to_f32(rd16(p));
            memcpy(b[i].q, p + 2, 32);
        }
        w->data = b;
        break;
    }
    case T_Q4_0: {
        if (len != nb * 18) return REF_ERR_SHAPE;
        ref_q4_0_block *b = malloc(nb * sizeof *b);
        for (size_t i = 0; i < nb; i++) {
            const uint8_t *p = data + i * 18;
            if (!ref_f16_is_finite(rd16(p))) { free(b); return REF_ERR_NON_FINITE; }
            b[i].d = ref_f16_to_f32(rd16(p));
            memcpy(b[i].qs, p + 2, 16);
        }
        w->data = b;
        break;
    }
    case T_Q4K: {
        if (len != nb * 144) return REF_ERR_SHAPE;
        ref_q4k_block *b = malloc(nb * sizeof *b);
        for (size_t i = 0; i < nb; i++) {
            const uint8_t *p = data + i * 144;
            if (!ref_f16_is_finite(rd16(p)) || !ref_f16_is_finite(rd16(p + 2))) {
                free(b);
                return REF_ERR_NON_FINITE;
            }
            b[i].d = ref_f16_to_f32(rd16(p));
            b[i].dmin = ref_f16_to_f32(rd16(p + 2));
            memcpy(b[i].scales, p + 4, 12);
            memcpy(b[i].qs, p + 16, 128);
        }
        w->data = b;
        break;
    }
    case T_Q6K: {
        if (len != nb * 210) return REF_ERR_SHAPE;
        ref_q6k_block *b = malloc(nb * sizeof *b);
        for (size_t i = 0; i < nb; i++) {
            const uint8_t *p = data + i * 210;
            memcpy(b[i].ql, p, 128);
            memcpy(b[i].qh, p + 128, 64);
            memcpy(b[i].scales, p + 192, 16);
            if (!ref_f16_is_finite(rd16(p + 208))) { free(b); return REF_ERR_NON_FINITE; }
            b[i].d = ref_f16_to_f32(rd16(p + 208));
        }
        w->data = b;
        break;
    }
    }
    return REF_OK;
}

static void free_mat(wmat *w) {
    if (w->owned) free(w->data);
    w->data = NULL;
}

static int opt_u32(const g_file *g, const char *key, uint32_t *v, int *present) {
    int e = g_meta_u32(g, key, v);
    if (e == G_METADATA_NOT_FOUND) { *present = 0; return REF_OK; }
    if (e) return map_meta(e);
    *present = 1;
    return REF_OK;
}

static int opt_f32(const g_file *g, const char *key, float *v, int *present) {
    int e = g_meta_f32(g, key, v);
    if (e == G_METADATA_NOT_FOUND) { *present = 0; return REF_OK; }
    if (e) return map_meta(e);
    *present = 1;
    return REF_OK;
}

static int opt_bool(const g_file *g, const char *key, int *v, int *present) {
    const g_kv *kv = g_find_kv(g, key);
    if (!kv) { *present = 0; return REF_OK; }
    if (kv->type != GV_BOOL) return REF_ERR_GGUF;
    *present = 1;
    *v = kv->v.b;
    return REF_OK;
}

static int reject_nonzero_f32(const g_file *g, const char *key) {
    const g_kv *kv = g_find_kv(g, key);
    if (!kv) return REF_OK;
    if (kv->type != GV_F32 && kv->type != GV_F64) return REF_ERR_GGUF;
    if (!isfinite(kv->v.f)) return REF_ERR_SHAPE;
    if (kv->v.f != 0.0) return REF_ERR_UNSUPPORTED_MODEL_FEATURE;
    return REF_OK;
}

/* LlamaConfig::validate (lib.rs:1581-1616) */
static int cfg_validate(const cfg_t *c) {
    if (c->block_count == 0 || c->d == 0 || c->ff == 0 || c->heads == 0 || c->kv_heads == 0 ||
        c->context_length == 0 || c->heads % c->kv_heads != 0 || c->rope_dim == 0 ||
        c->rope_dim % 2 != 0 || !isfinite(c->eps) || c->eps <= 0.0f ||
        !isfinite(c->attention_scale) || c->attention_scale <= 0.0f || !isfinite(c->rope_base) ||
        c->rope_base <= 0.0f)
        return REF_ERR_SHAPE;
    if (c->d % c->heads != 0) return REF_ERR_SHAPE;
    if (c->rope_dim > c->d / c->heads) return REF_ERR_SHAPE;
    return REF_OK;
}

/* LlamaConfig::from_gguf (lib.rs:1498-1565) */
static int cfg_from_gguf(const g_file *g, cfg_t *c) {
    const char *arch;
    size_t al;
    int e = g_meta_str(g, "general.architecture", &arch, &al);
    if (e) return map_meta(e);
    int is_llama = al == 5 && !memcmp(arch, "llama", 5);
    int is_qwen2 = al == 5 && !memcmp(arch, "qwen2", 5);
    if (!is_llama && !is_qwen2) return REF_ERR_UNSUPPORTED_ARCHITECTURE;
    memset(c, 0, sizeof *c);
    c->split_half = is_qwen2;
    char key[256];
#define K(s) (snprintf(key, sizeof key, "%.*s.%s", (int)al, arch, s), key)
    uint32_t v;
    int present;
    if ((e = g_meta_u32(g, K("attention.head_count"), &v))) return map_meta(e);
    c->heads = v;
    if ((e = opt_u32(g, K("attention.head_count_kv"), &v, &present))) return e;
    c->kv_heads = present ? v : c->heads;
    if ((e = g_meta_u32(g, K("embedding_length"), &v))) return map_meta(e);
    c->d = v;
    if (c->heads == 0 || c->d % c->heads != 0) return REF_ERR_SHAPE;
    if ((e = opt_u32(g, K("embedding_length_out"), &v, &present))) return e;
    if (present && v != c->d) return REF_ERR_UNSUPPORTED_MODEL_FEATURE;
    int b;
    if ((e = opt_bool(g, K("attention.causal"), &b, &present))) return e;
    if (present && !b) return REF_ERR_UNSUPPORTED_MODEL_FEATURE;
    {
        const char *s;
        size_t sl;
        e = g_meta_str(g, K("rope.scaling.type"), &s, &sl);
        if (e && e != G_METADATA_NOT_FOUND) return map_meta(e);
        if (!e && !(sl == 4 && !memcmp(s, "none", 4))) return REF_ERR_UNSUPPORTED_ROPE_SCALING;
    }
    if ((e = opt_bool(g, K("use_parallel_residual"), &b, &present))) return e;
    if (present && b) return REF_ERR_UNSUPPORTED_MODEL_FEATURE;
    if ((e = opt_u32(g, K("attention.sliding_window"), &v, &present))) return e;
    if (present && v != 0) return REF_ERR_UNSUPPORTED_MODEL_FEATURE;
    static const char *f32keys[] = {"attention.max_alibi_bias", "attention.clamp_kqv",
                                    "attention.value_scale",    "attn_logit_softcapping",
                                    "final_logit_softcapping",  "logit_scale",
                                    "embedding_scale",          "residual_scale"};
    for (size_t i = 0; i < sizeof f32keys / sizeof *f32keys; i++)
        if ((e = reject_nonzero_f32(g, K(f32keys[i])))) return e;
    size_t head_dim = c->d / c->heads;
    if ((e = opt_u32(g, K("attention.key_length"), &v, &present))) return e;
    if (present && v != head_dim) return REF_ERR_UNSUPPORTED_ATTENTION_HEAD_LENGTH;
    if ((e = opt_u32(g, K("attention.value_length"), &v, &present))) return e;
    if (present && v != head_dim) return REF_ERR_UNSUPPORTED_ATTENTION_HEAD_LENGTH;
    float f;
    if ((e = opt_f32(g, K("attention.scale"), &f, &present))) return e;
    c->attention_scale = present ? f : 1.0f / sqrtf((float)head_dim);
    if ((e = g_meta_u32(g, K("block_count"), &v))) return map_meta(e);
    c->block_count = v;
    if ((e = g_meta_u32(g, K("feed_forward_length"), &v))) return map_meta(e);
    c->ff = v;
    if ((e = g_meta_f32(g, K("attention.layer_norm_rms_epsilon"), &f))) return map_meta(e);
    c->eps = f;
    if ((e = opt_f32(g, K("rope.freq_base"), &f, &present))) return e;
    c->rope_base = present ? f : 10000.0f;
    if ((e = opt_u32(g, K("rope.dimension_count"), &v, &present))) return e;
    c->rope_dim = present ? v : head_dim;
    if ((e = g_meta_u32(g, K("context_length"), &v))) return map_meta(e);
    c->context_length = v;
#undef K
    return cfg_validate(c);
}

/* vocab_size (lib.rs:1648-1672) */
static int vocab_size(const g_file *g, size_t *out) {
    const char *arch;
    size_t al;
    int e = g_meta_str(g, "general.architecture", &arch, &al);
    if (e) return map_meta(e);
    char key[256];
    snprintf(key, sizeof key, "%.*s.vocab_size", (int)al, arch);
    const char *keys[2] = {key, "llama.vocab_size"};
    for (int i = 0; i < 2; i++) {
        uint32_t v;
        e = g_meta_u32(g, keys[i], &v);
        if (!e) { *out = v; return REF_OK; }
        if (e != G_METADATA_NOT_FOUND) return map_meta(e);
    }
    const g_kv *kv = g_find_kv(g, "tokenizer.ggml.tokens");
    if (kv) {
        if (kv->type != GV_ARRAY || kv->arr_type != GV_STRING) return REF_ERR_GGUF;
        *out = (size_t)kv->arr_count;
        return REF_OK;
    }
    const g_tensor *t;
    if (g_find_tensor(g, "token_embd.weight", &t)) return REF_ERR_GGUF;
    if (t->ndim == 2) { *out = (size_t)t->dims[1]; return REF_OK; }
    return REF_ERR_MISSING_METADATA;
}

void ref_model_free(ref_model *m) {
    if (!m) return;
    if (m->layers) {
        for (size_t l = 0; l < m->c.block_count; l++) {
            layer_w *L = &m->layers[l];
            free(L->attn_norm); free(L->ffn_norm); free(L->bq); free(L->bk); free(L->bv);
            free_mat(&L->wq); free_mat(&L->wk); free_mat(&L->wv); free_mat(&L->wo);
            free_mat(&L->gate); free_mat(&L->up); free_mat(&L->down);
        }
        free(m->layers);
    }
    free_mat(&m->emb);
    free_mat(&m->out);
    free(m->out_norm);
    free(m);
}

/* F32Llama::from_gguf (lib.rs:1035-1140) */
ref_model *ref_model_load(const uint8_t *bytes, size_t len, int *status) {
    g_file g;
    int e = g_parse(bytes, len, &g);
    if (e) { *status = REF_ERR_GGUF; return NULL; }
    ref_model *m = calloc(1, sizeof *m);
    if ((e = cfg_from_gguf(&g, &m->c))) goto fail;
    m->head_dim = m->c.d / m->c.heads;
    size_t d = m->c.d, ff = m->c.ff, hd = m->head_dim;
    if ((e = vocab_size(&g, &m->vocab))) goto fail;
    if ((e = read_matrix(&g, "token_embd.weight", m->vocab, d, &m->emb))) goto fail;
    m->layers = calloc(m->c.block_count, sizeof(layer_w));
    for (size_t l = 0; l < m->c.block_count; l++) {
        layer_w *L = &m->layers[l];
        char name[128];
#define NM(s) (snprintf(name, sizeof name, "blk.%zu.%s", l, s), name)
        if ((e = read_vec(&g, NM("attn_norm.weight"), d, &L->attn_norm))) goto fail;
        if ((e = read_matrix(&g, NM("attn_q.weight"), m->c.heads * hd, d, &L->wq))) goto fail;
        if ((e = read_opt_vec(&g, NM("attn_q.bias"), m->c.heads * hd, &L->bq))) goto fail;
        if ((e = read_matrix(&g, NM("attn_k.weight"), m->c.kv_heads * hd, d, &L->wk))) goto fail;
        if ((e = read_opt_vec(&g, NM("attn_k.bias"), m->c.kv_heads * hd, &L->bk))) goto fail;
        if ((e = read_matrix(&g, NM("attn_v.weight"), m->c.kv_heads * hd, d, &L->wv))) goto fail;
        if ((e = read_opt_vec(&g, NM("attn_v.bias"), m->c.kv_heads * hd, &L->bv))) goto fail;
        if ((e = read_matrix(&g, NM("attn_output.weight"), d, m->c.heads * hd, &L->wo))) goto fail;
        if ((e = read_vec(&g, NM("ffn_norm.weight"), d, &L->ffn_norm))) goto fail;
        if ((e = read_matrix(&g, NM("ffn_gate.weight"), ff, d, &L->gate))) goto fail;
        if ((e = read_matrix(&g, NM("ffn_up.weight"), ff, d, &L->up))) goto fail;
        if ((e = read_matrix(&g, NM("ffn_down.weight"), d, ff, &L->down))) goto fail;
#undef NM
    }
    if ((e = read_vec(&g, "output_norm.weight", d, &m->out_norm))) goto fail;
    {
        const g_tensor *t;
        int fe = g_find_tensor(&g, "output.weight", &t);
        if (fe == G_OK) {
            if ((e = read_matrix(&g, "output.weight", m->emb.rows, d, &m->out))) goto fail;
        } else if (fe == G_TENSOR_NOT_FOUND) {
            m->out = m->emb;
            m->out.owned = 0;
        } else {
            e = REF_ERR_GGUF;
            goto fail;
        }
    }
    g_free(&g);
    *status = REF_OK;
    return m;
fail:
    g_free(&g);
    ref_model_free(m);
    *status = e;
    return NULL;
}

void ref_model_config(const ref_model *m, int64_t out[16]) {
    float f[3] = {m->c.eps, m->c.attention_scale, m->c.rope_base};
    uint32_t b[3];
    memcpy(b, f, sizeof b);
    int has_bias = m->layers[0].bq || m->layers[0].bk || m->layers[0].bv;
    int64_t v[16] = {(int64_t)m->c.block_count, (int64_t)m->c.d, (int64_t)m->c.ff,
                     (int64_t)m->c.heads, (int64_t)m->c.kv_heads, (int64_t)m->head_dim,
                     (int64_t)m->c.rope_dim, m->c.split_half, (int64_t)m->c.context_length,
                     (int64_t)m->vocab, b[0], b[1], b[2], m->emb.type, m->out.type, has_bias};
    memcpy(out, v, sizeof v);
}

/* The q (which 0), k (1) or v (2) bias vector of one layer, as loaded by
 * F32Llama::from_gguf (lib.rs:1060-1092): copies min(len, cap) values and
 * returns len, or 0 when the layer has no such bias. */
size_t ref_model_bias(const ref_model *m, size_t layer, int which, float *out, size_t cap) {
    if (layer >= m->c.block_count || which < 0 || which > 2) return 0;
    const layer_w *L = &m->layers[layer];
    const float *b = which == 0 ? L->bq : which == 1 ? L->bk : L->bv;
    if (!b) return 0;
    size_t n = (which == 0 ? m->c.heads : m->c.kv_heads) * m->head_dim;
    memcpy(out, b, (n < cap ? n : cap) * sizeof(float));
    return n;
}

/* ---------------------------------------------------------------------- */
/* RoPE tables (lib.rs:813-847)                                             */
/* ---------------------------------------------------------------------- */
static int rope_table(const cfg_t *c, size_t positions, float *cs, float *sn) {
    size_t half = c->rope_dim / 2;
    double ln_base = ref_ln_f64((double)c->rope_base);
    for (size_t pos = 0; pos < positions; pos++)
        for (size_t j = 0; j < half; j++) {
            double exponent = -((double)(2 * j)) / (double)c->rope_dim;
            double omega = ref_exp_f64(exponent * ln_base);
            double phi = (double)pos * omega;
            float cv = (float)ref_cos_f64(phi);
            float sv = (float)ref_sin_f64(phi);
            if (!isfinite(cv) || !isfinite(sv)) return REF_ERR_NON_FINITE;
            cs[pos * half + j] = cv;
            sn[pos * half + j] = sv;
        }
    return REF_OK;
}

int ref_rope_table(const ref_model *m, size_t positions, float *cs, float *sn) {
    return rope_table(&m->c, positions, cs, sn);
}

/* ---------------------------------------------------------------------- */
/* sessions                                                                */
/* ---------------------------------------------------------------------- */
void ref_session_free(ref_session *s) {
    if (!s) return;
    free(s->rope_cos); free(s->rope_sin); free(s->kc); free(s->vc);
    free(s->x); free(s->h); free(s->q); free(s->k); free(s->v); free(s->attn);
    free(s->scores); free(s->probs); free(s->tmp); free(s->gate); free(s->up); free(s->ffo);
    free(s->q8a); free(s->q8k);
    free(s);
}

ref_session *ref_session_new(const ref_model *m, size_t max_ctx, int *status) {
    if (max_ctx == 0 || max_ctx > m->c.context_length) { *status = REF_ERR_SHAPE; return NULL; }
    ref_session *s = calloc(1, sizeof *s);
    const cfg_t *c = &m->c;
    size_t hd = m->head_dim, half = c->rope_dim / 2;
    size_t maxdim = c->d > c->ff ? c->d : c->ff;
    if (c->heads * hd > maxdim) maxdim = c->heads * hd;
    s->m = m;
    s->max_ctx = max_ctx;
    s->rope_cos = malloc(max_ctx * half * 4);
    s->rope_sin = malloc(max_ctx * half * 4);
    int e = rope_table(c, max_ctx, s->rope_cos, s->rope_sin);
    if (e) { ref_session_free(s); *status = e; return NULL; }
    size_t kv = c->block_count * c->kv_heads * c->context_length * hd;
    s->kc = calloc(kv, 4);
    s->vc = calloc(kv, 4);
    s->x = calloc(c->d, 4); s->h = calloc(c->d, 4); s->tmp = calloc(c->d, 4);
    s->q = calloc(c->heads * hd, 4); s->attn = calloc(c->heads * hd, 4);
    s->k = calloc(c->kv_heads * hd, 4); s->v = calloc(c->kv_heads * hd, 4);
    s->scores = calloc(c->heads * max_ctx, 4); s->probs = calloc(c->heads * max_ctx, 4);
    s->gate = calloc(c->ff, 4); s->up = calloc(c->ff, 4); s->ffo = calloc(c->ff, 4);
    s->q8a = calloc(maxdim / QK + 1, sizeof(ref_q8a_block));
    s->q8k = calloc(maxdim / QKK + 1, sizeof(ref_q8k_block));
    *status = REF_OK;
    return s;
}

int ref_session_reset(ref_session *s) {
    const cfg_t *c = &s->m->c;
    size_t kv = c->block_count * c->kv_heads * c->context_length * s->m->head_dim;
    memset(s->kc, 0, kv * 4);
    memset(s->vc, 0, kv * 4);
    return REF_OK;
}

/* apply_rope (lib.rs:2011-2051) */
/* apply_rope (lib.rs:2011-2051) with one position's table row: pairs
 * (2j, 2j+1) (Adjacent) or (j, j+half) (SplitHalf) of each head's first
 * rope_dim dims rotate by (cos_row[j], sin_row[j]); the rest are untouched. */
int ref_apply_rope(float *x, size_t heads, size_t head_dim, size_t rope_dim, int split_half,
                   const float *cos_row, const float *sin_row) {
    size_t half = rope_dim / 2;
    if (rope_dim % 2 != 0 || rope_dim > head_dim) return REF_ERR_SHAPE;
    if (!finite_slice(x, heads * head_dim)) return REF_ERR_NON_FINITE;
    for (size_t h = 0; h < heads; h++) {
        size_t base = h * head_dim;
        for (size_t j = 0; j < half; j++) {
            size_t a, b;
            if (split_half) { a = base + j; b = base + j + half; }
            else { a = base + 2 * j; b = a + 1; }
            float x0 = x[a], x1 = x[b];
            float cv = cos_row[j], sv = sin_row[j];
            x[a] = x0 * cv - x1 * sv;
            x[b] = x0 * sv + x1 * cv;
            if (!isfinite(x[a]) || !isfinite(x[b])) return REF_ERR_NON_FINITE;
        }
    }
    return REF_OK;
}

static int apply_rope(const ref_session *s, float *x, size_t heads, size_t pos) {
    const ref_model *m = s->m;
    size_t half = m->c.rope_dim / 2;
    return ref_apply_rope(x, heads, m->head_dim, m->c.rope_dim, m->c.split_half,
                          s->rope_cos + pos * half, s->rope_sin + pos * half);
}

/* softmax_in_place (lib.rs:2361-2388) */
static int softmax(float *x, size_t n) {
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++) {
        if (!isfinite(x[i])) return REF_ERR_NON_FINITE;
        if (x[i] > max) max = x[i];
    }
    for (size_t i = 0; i < n; i++) {
        float t = x[i] - max;
        x[i] = ref_exp_f32(t < -88.0f ? -88.0f : t);
    }
    float z = ref_sum_f32(x, n);
    if (!isfinite(z) || z == 0.0f) return REF_ERR_NON_FINITE;
    for (size_t i = 0; i < n; i++) {
        x[i] /= z;
        if (!isfinite(x[i])) return REF_ERR_NON_FINITE;
    }
    return REF_OK;
}

typedef struct {
    ref_session *s;
    size_t layer, pos;
} attn_ctx;

/* attention_one_head (lib.rs:2300-2333) with the scores (2335-2359) and
 * P.V chain (2390-2418). */
static int attention_heads_fn(void *p, size_t begin, size_t end) {
    attn_ctx *a = p;
    ref_session *s = a->s;
    const ref_model *m = s->m;
    size_t hd = m->head_dim, ctx = m->c.context_length, len = a->pos + 1;
    size_t group = m->c.heads / m->c.kv_heads;
    for (size_t h = begin; h < end; h++) {
        size_t kvh = h / group;
        size_t base = (a->layer * m->c.kv_heads + kvh) * ctx * hd;
        const float *keys = s->kc + base, *vals = s->vc + base;
        float *out = s->attn + h * hd;
        if (len == 1) {
            memcpy(out, vals, hd * 4);
            continue;
        }
        const float *qh = s->q + h * hd;
        float *sc = s->scores + h * s->max_ctx;
        float *pr = s->probs + h * s->max_ctx;
        if (!finite_slice(qh, hd) || !finite_slice(keys, len * hd)) return REF_ERR_NON_FINITE;
        for (size_t j = 0; j < len; j++) {
            sc[j] = ref_dot_f32(qh, keys + j * hd, hd) * m->c.attention_scale;
            if (!isfinite(sc[j])) return REF_ERR_NON_FINITE;
        }
        memcpy(pr, sc, len * 4);
        int e = softmax(pr, len);
        if (e) return e;
        if (!finite_slice(vals, len * hd)) return REF_ERR_NON_FINITE;
        for (size_t dd = 0; dd < hd; dd++) out[dd] = 0.0f;
        for (size_t j = 0; j < len; j++) {
            float pj = pr[j];
            for (size_t dd = 0; dd < hd; dd++) {
                out[dd] += pj * vals[j * hd + dd];
                if (!isfinite(out[dd])) return REF_ERR_NON_FINITE;
            }
        }
    }
    return REF_OK;
}

static int add_vec(float *x, const float *b, size_t n) {
    if (!b) return REF_OK;
    if (!finite_slice(x, n) || !finite_slice(b, n)) return REF_ERR_NON_FINITE;
    for (size_t i = 0; i < n; i++) {
        x[i] += b[i];
        if (!isfinite(x[i])) return REF_ERR_NON_FINITE;
    }
    return REF_OK;
}

/* forward_one_with_workspace (lib.rs:1249-1400) */
int ref_forward_one(ref_session *s, size_t token, size_t pos, float *logits) {
    const ref_model *m = s->m;
    const cfg_t *c = &m->c;
    size_t d = c->d, hd = m->head_dim, ctx = c->context_length;
    if (pos >= ctx || token >= m->emb.rows || pos >= s->max_ctx) return REF_ERR_SHAPE;
    int e;
    if ((e = write_row(&m->emb, token, s->x))) return e;
    for (size_t l = 0; l < c->block_count; l++) {
        const layer_w *L = &m->layers[l];
        if ((e = ref_rmsnorm(s->x, L->attn_norm, c->eps, d, s->h))) return e;
        const ref_q8a_block *qa = NULL;
        if (needs_q8a(&L->wq) || needs_q8a(&L->wk) || needs_q8a(&L->wv)) {
            if ((e = quantize_q8a_vec(s->h, d, s->q8a))) return e;
            qa = s->q8a;
        }
        if ((e = gemv(&L->wq, s->h, qa, 0, s->q8a, s->q8k, s->q))) return e;
        if ((e = add_vec(s->q, L->bq, c->heads * hd))) return e;
        if ((e = gemv(&L->wk, s->h, qa, 0, s->q8a, s->q8k, s->k))) return e;
        if ((e = add_vec(s->k, L->bk, c->kv_heads * hd))) return e;
        if ((e = gemv(&L->wv, s->h, qa, 0, s->q8a, s->q8k, s->v))) return e;
        if ((e = add_vec(s->v, L->bv, c->kv_heads * hd))) return e;
        if ((e = apply_rope(s, s->q, c->heads, pos))) return e;
        if ((e = apply_rope(s, s->k, c->kv_heads, pos))) return e;
        if (!finite_slice(s->k, c->kv_heads * hd) || !finite_slice(s->v, c->kv_heads * hd))
            return REF_ERR_NON_FINITE;
        for (size_t kvh = 0; kvh < c->kv_heads; kvh++) {
            size_t off = ((l * c->kv_heads + kvh) * ctx + pos) * hd;
            memcpy(s->kc + off, s->k + kvh * hd, hd * 4);
            memcpy(s->vc + off, s->v + kvh * hd, hd * 4);
        }
        attn_ctx ac = {s, l, pos};
        size_t threads = requested_threads();
        if (threads > c->heads) threads = c->heads;
        size_t work = c->heads * (pos + 1) * hd;
        if (threads > 1 && c->heads > 1 && work >= MIN_PARALLEL_ATTENTION_WORK)
            e = run_partitioned(attention_heads_fn, &ac, c->heads, threads);
        else
            e = attention_heads_fn(&ac, 0, c->heads);
        if (e) return e;
        if ((e = gemv(&L->wo, s->attn, NULL, 1, s->q8a, s->q8k, s->tmp))) return e;
        if ((e = add_vec(s->x, s->tmp, d))) return e;
        if ((e = ref_rmsnorm(s->x, L->ffn_norm, c->eps, d, s->h))) return e;
        qa = NULL;
        if (needs_q8a(&L->gate) || needs_q8a(&L->up)) {
            if ((e = quantize_q8a_vec(s->h, d, s->q8a))) return e;
            qa = s->q8a;
        }
        if ((e = gemv(&L->gate, s->h, qa, 0, s->q8a, s->q8k, s->gate))) return e;
        if ((e = gemv(&L->up, s->h, qa, 0, s->q8a, s->q8k, s->up))) return e;
        if (!finite_slice(s->gate, c->ff) || !finite_slice(s->up, c->ff)) return REF_ERR_NON_FINITE;
        for (size_t i = 0; i < c->ff; i++) {
            s->ffo[i] = ref_silu_f32(s->gate[i]) * s->up[i];
            if (!isfinite(s->ffo[i])) return REF_ERR_NON_FINITE;
        }
        if ((e = gemv(&L->down, s->ffo, NULL, 1, s->q8a, s->q8k, s->tmp))) return e;
        if ((e = add_vec(s->x, s->tmp, d))) return e;
    }
    if ((e = ref_rmsnorm(s->x, m->out_norm, c->eps, d, s->h))) return e;
    return gemv(&m->out, s->h, NULL, 1, s->q8a, s->q8k, logits);
}

/* logits_hash_for_tokens_chunked (lib.rs:1406-1465): the chunk size only
 * groups iterations and has no numeric effect. */
int ref_logits_hash(const ref_model *m, const uint32_t *tokens, size_t n, size_t chunk,
                    uint8_t out[32]) {
    if (n == 0 || chunk == 0 || n > m->c.context_length) return REF_ERR_SHAPE;
    for (size_t i = 0; i < n; i++)
        if (tokens[i] >= m->emb.rows) return REF_ERR_SHAPE;
    int e;
    ref_session *s = ref_session_new(m, n, &e);
    if (!s) return e;
    float *logits = malloc(m->out.rows * 4);
    ref_sha256_ctx c;
    ref_sha256_init(&c);
    for (size_t i = 0; i < n; i++) {
        if ((e = ref_forward_one(s, tokens[i], i, logits))) break;
        ref_sha256_update(&c, logits, m->out.rows * 4); /* little-endian host */
    }
    free(logits);
    ref_session_free(s);
    if (e) return e;
    ref_sha256_final(&c, out);
    return REF_OK;
}

int ref_logits(const ref_model *m, const uint32_t *tokens, size_t n, float *out) {
    if (n == 0 || n > m->c.context_length) return REF_ERR_SHAPE;
    int e;
    ref_session *s = ref_session_new(m, n, &e);
    if (!s) return e;
    for (size_t i = 0; i < n; i++)
        if ((e = ref_forward_one(s, tokens[i], i, out + i * m->out.rows))) break;
    ref_session_free(s);
    return e;
}

/* Dot of one GGUF-encoded row against x, quantising x as the reference
 * does for the row type (lib.rs:445-490). */
int ref_dot_row(int ggml_type, const uint8_t *row, size_t cols, const float *x, float *out) {
    int e;
    switch (ggml_type) {
    case T_F32: {
        float *w = malloc(cols * 4);
        memcpy(w, row, cols * 4);
        *out = ref_dot_f32(w, x, cols);
        free(w);
        return REF_OK;
    }
    case T_Q8_0: case T_Q4_0: case T_Q4K: {
        size_t bs = ggml_type == T_Q4K ? QKK : QK, nb = cols / bs;
        if (cols % bs) return REF_ERR_SHAPE;
        ref_q8a_block *qa = malloc((cols / QK) * sizeof *qa);
        if ((e = quantize_q8a_vec(x, cols, qa))) { free(qa); return e; }
        int q;
        if (ggml_type == T_Q8_0) {
            ref_q8_0_block *b = malloc(nb * sizeof *b);
            for (size_t i = 0; i < nb; i++) {
                b[i].d = ref_f16_to_f32(rd16(row + 34 * i));
                memcpy(b[i].q, row + 34 * i + 2, 32);
            }
            q = ref_dot_q8_0_q8a(b, qa, nb, out);
            free(b);
        } else if (ggml_type == T_Q4_0) {
            ref_q4_0_block *b = malloc(nb * sizeof *b);
            for (size_t i = 0; i < nb; i++) {
                b[i].d = ref_f16_to_f32(rd16(row + 18 * i));
                memcpy(b[i].qs, row + 18 * i + 2, 16);
            }
            q = ref_dot_q4_0_q8a(b, qa, nb, out);
            free(b);
        } else {
            ref_q4k_block *b = malloc(nb * sizeof *b);
            for (size_t i = 0; i < nb; i++) {
                const uint8_t *p = row + 144 * i;
                b[i].d = ref_f16_to_f32(rd16(p));
                b[i].dmin = ref_f16_to_f32(rd16(p + 2));
                memcpy(b[i].scales, p + 4, 12);
                memcpy(b[i].qs, p + 16, 128);
            }
            q = ref_dot_q4_k_q8a(b, qa, nb, out);
            free(b);
        }
        free(qa);
        return map_quant(q);
    }
    case T_Q6K: {
        if (cols % QKK) return REF_ERR_SHAPE;
        size_t nb = cols / QKK;
        ref_q8k_block *qk = malloc(nb * sizeof *qk);
        if ((e = quantize_q8k_vec(x, cols, qk))) { free(qk); return e; }
        ref_q6k_block *b = malloc(nb * sizeof *b);
        for (size_t i = 0; i < nb; i++) {
            const uint8_t *p = row + 210 * i;
            memcpy(b[i].ql, p, 128);
            memcpy(b[i].qh, p + 128, 64);
            memcpy(b[i].scales, p + 192, 16);
            b[i].d = ref_f16_to_f32(rd16(p + 208));
        }
        int q = ref_dot_q6_k_q8k(b, qk, nb, out);
        free(b);
        free(qk);
        return map_quant(q);
    }
    default: return REF_ERR_UNSUPPORTED_TENSOR_TYPE;
    }
}
