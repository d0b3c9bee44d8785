/*
 * Minimal GGUF v2/v3 reader for the oracle (TEST INFRASTRUCTURE ONLY).
 * Restates crates/det-gguf/src/lib.rs of mii443/detllm: header, metadata
 * value types (lib.rs:374-486), tensor infos, 32-byte data alignment
 * (lib.rs:199-216) and the tensor-range overlap validation (lib.rs:218-245).
 */
#include <stdlib.h>
#include <string.h>

#include "detref_gguf.h"

typedef struct {
    const uint8_t *b;
    size_t len, pos;
} rd;

static int rd_exact(rd *r, size_t n, const uint8_t **p) {
    if (n > r->len - r->pos) return G_TRUNCATED;
    *p = r->b + r->pos;
    r->pos += n;
    return G_OK;
}
static int rd_u8(rd *r, uint8_t *v) {
    const uint8_t *p;
    int e = rd_exact(r, 1, &p);
    if (!e) *v = p[0];
    return e;
}
static int rd_u16(rd *r, uint16_t *v) {
    const uint8_t *p;
    int e = rd_exact(r, 2, &p);
    if (!e) *v = (uint16_t)(p[0] | (p[1] << 8));
    return e;
}
static int rd_u32(rd *r, uint32_t *v) {
    const uint8_t *p;
    int e = rd_exact(r, 4, &p);
    if (!e) *v = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
    return e;
}
static int rd_u64(rd *r, uint64_t *v) {
    uint32_t lo, hi;
    int e = rd_u32(r, &lo);
    if (!e) e = rd_u32(r, &hi);
    if (!e) *v = ((uint64_t)hi << 32) | lo;
    return e;
}

/* Strict UTF-8 validation (the reference builds Rust Strings). */
static int utf8_ok(const uint8_t *s, size_t n) {
    size_t i = 0;
    while (i < n) {
        uint8_t c = s[i];
        if (c < 0x80) { i++; continue; }
        size_t need;
        uint32_t cp, min;
        if ((c & 0xe0) == 0xc0) { need = 1; cp = c & 0x1f; min = 0x80; }
        else if ((c & 0xf0) == 0xe0) { need = 2; cp = c & 0x0f; min = 0x800; }
        else if ((c & 0xf8) == 0xf0) { need = 3; cp = c & 0x07; min = 0x10000; }
        else return 0;
        if (i + need >= n) return 0;
        for (size_t k = 1; k <= need; k++) {
            if ((s[i + k] & 0xc0) != 0x80) return 0;
            cp = (cp << 6) | (s[i + k] & 0x3f);
        }
        if (cp < min || cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff)) return 0;
        i += need + 1;
    }
    return 1;
}

static int rd_string(rd *r, const char **s, size_t *n) {
    uint64_t len;
    int e = rd_u64(r, &len);
    if (e) return e;
    if (len > r->len - r->pos) return G_TRUNCATED;
    const uint8_t *p;
    e = rd_exact(r, (size_t)len, &p);
    if (e) return e;
    if (!utf8_ok(p, (size_t)len)) return G_INVALID_UTF8;
    *s = (const char *)p;
    *n = (size_t)len;
    return G_OK;
}

static int ensure_count(rd *r, uint64_t n, uint64_t min_bytes) {
    uint64_t rem = r->len - r->pos;
    if (min_bytes && n > rem / min_bytes) return G_TRUNCATED;
    return G_OK;
}

static int read_value(rd *r, g_kv *kv) {
    uint32_t ty;
    int e = rd_u32(r, &ty);
    if (e) return e;
    kv->type = ty;
    switch (ty) {
    case GV_U8: case GV_I8: { uint8_t v = 0; e = rd_u8(r, &v); kv->v.u = v; kv->v.i = ty == GV_I8 ? (int8_t)v : v; return e; }
    case GV_U16: case GV_I16: { uint16_t v = 0; e = rd_u16(r, &v); kv->v.u = v; kv->v.i = ty == GV_I16 ? (int16_t)v : v; return e; }
    case GV_U32: case GV_I32: { uint32_t v = 0; e = rd_u32(r, &v); kv->v.u = v; kv->v.i = ty == GV_I32 ? (int32_t)v : (int64_t)v; return e; }
    case GV_F32: { uint32_t v = 0; e = rd_u32(r, &v); float f; memcpy(&f, &v, 4); kv->v.f = f; return e; }
    case GV_BOOL: { uint8_t v = 0; e = rd_u8(r, &v); if (e) return e; if (v > 1) return G_INVALID_BOOL; kv->v.b = v; return G_OK; }
    case GV_STRING: return rd_string(r, &kv->str, &kv->str_len);
    case GV_U64: case GV_I64: { uint64_t v = 0; e = rd_u64(r, &v); kv->v.u = v; kv->v.i = (int64_t)v; return e; }
    case GV_F64: { uint64_t v = 0; e = rd_u64(r, &v); double f; memcpy(&f, &v, 8); kv->v.f = f; return e; }
    case GV_ARRAY: {
        uint32_t et;
        uint64_t n;
        if ((e = rd_u32(r, &et))) return e;
        if ((e = rd_u64(r, &n))) return e;
        uint64_t min;
        switch (et) {
        case 0: case 1: case 7: min = 1; break;
        case 2: case 3: min = 2; break;
        case 4: case 5: case 6: min = 4; break;
        case 8: case 10: case 11: case 12: min = 8; break;
        default: return G_UNSUPPORTED_VALUE_TYPE;
        }
        if ((e = ensure_count(r, n, min))) return e;
        kv->arr_type = et;
        kv->arr_count = n;
        kv->arr_offset = r->pos;
        for (uint64_t k = 0; k < n; k++) {
            if (et == 8) {
                const char *s;
                size_t sl;
                if ((e = rd_string(r, &s, &sl))) return e;
            } else if (et == 7) {
                uint8_t v;
                if ((e = rd_u8(r, &v))) return e;
                if (v > 1) return G_INVALID_BOOL;
            } else {
                const uint8_t *p;
                if ((e = rd_exact(r, (size_t)min, &p))) return e;
            }
        }
        return G_OK;
    }
    default: return G_UNSUPPORTED_VALUE_TYPE;
    }
}

int g_type_size(uint32_t type, uint64_t *ts, uint64_t *bs) {
    switch (type) {
    case 0: *ts = 4; *bs = 1; return G_OK;
    case 1: *ts = 2; *bs = 1; return G_OK;
    case 2: *ts = 18; *bs = 32; return G_OK;
    case 3: *ts = 20; *bs = 32; return G_OK;
    case 6: *ts = 22; *bs = 32; return G_OK;
    case 7: *ts = 24; *bs = 32; return G_OK;
    case 8: *ts = 34; *bs = 32; return G_OK;
    case 9: *ts = 40; *bs = 32; return G_OK;
    case 10: *ts = 84; *bs = 256; return G_OK;
    case 11: *ts = 110; *bs = 256; return G_OK;
    case 12: *ts = 144; *bs = 256; return G_OK;
    case 13: *ts = 176; *bs = 256; return G_OK;
    case 14: *ts = 210; *bs = 256; return G_OK;
    case 15: *ts = 292; *bs = 256; return G_OK;
    default: return G_UNSUPPORTED_TENSOR_TYPE;
    }
}

int g_tensor_elements(const g_tensor *t, uint64_t *n) {
    if (t->ndim == 0) return G_INVALID_TENSOR_SHAPE;
    uint64_t acc = 1;
    for (uint32_t i = 0; i < t->ndim; i++) {
        if (t->dims[i] == 0) return G_INVALID_TENSOR_SHAPE;
        if (acc > UINT64_MAX / t->dims[i]) return G_INVALID_TENSOR_SHAPE;
        acc *= t->dims[i];
    }
    *n = acc;
    return G_OK;
}

static int encoded_len(const g_tensor *t, uint64_t *len) {
    uint64_t n, ts, bs;
    int e = g_tensor_elements(t, &n);
    if (e) return e;
    if ((e = g_type_size(t->type, &ts, &bs))) return e;
    if (n % bs) return G_INVALID_TENSOR_SHAPE;
    if (n / bs > UINT64_MAX / ts) return G_INVALID_TENSOR_SHAPE;
    *len = (n / bs) * ts;
    return G_OK;
}

typedef struct { uint64_t s, e; } rng;
static int rng_cmp(const void *a, const void *b) {
    const rng *x = a, *y = b;
    return x->s < y->s ? -1 : x->s > y->s;
}

int g_parse(const uint8_t *bytes, size_t len, g_file *out) {
    memset(out, 0, sizeof *out);
    rd r = {bytes, len, 0};
    const uint8_t *magic;
    int e;
    if ((e = rd_exact(&r, 4, &magic))) return e;
    if (memcmp(magic, "GGUF", 4)) return G_BAD_MAGIC;
    uint32_t version;
    if ((e = rd_u32(&r, &version))) return e;
    if (version != 2 && version != 3) return G_UNSUPPORTED_VERSION;
    uint64_t n_t, n_kv;
    if ((e = rd_u64(&r, &n_t))) return e;
    if ((e = rd_u64(&r, &n_kv))) return e;
    out->bytes = bytes;
    out->len = len;
    out->version = version;
    /* Each metadata entry takes at least 12 bytes, each tensor info 24. */
    if (n_kv > len / 12 + 1) return G_TRUNCATED;
    out->kv = calloc(n_kv ? n_kv : 1, sizeof(g_kv));
    for (uint64_t i = 0; i < n_kv; i++) {
        g_kv *kv = &out->kv[i];
        if ((e = rd_string(&r, &kv->key, &kv->key_len))) goto fail;
        for (size_t j = 0; j < i; j++)
            if (out->kv[j].key_len == kv->key_len && !memcmp(out->kv[j].key, kv->key, kv->key_len)) {
                e = G_DUPLICATE_METADATA_KEY;
                goto fail;
            }
        if ((e = read_value(&r, kv))) goto fail;
        out->n_kv = i + 1;
    }
    if ((e = ensure_count(&r, n_t, 24))) goto fail;
    out->tensors = calloc(n_t ? n_t : 1, sizeof(g_tensor));
    for (uint64_t i = 0; i < n_t; i++) {
        g_tensor *t = &out->tensors[i];
        if ((e = rd_string(&r, &t->name, &t->name_len))) goto fail;
        if ((e = rd_u32(&r, &t->ndim))) goto fail;
        if (t->ndim > 4) { e = G_INVALID_TENSOR_SHAPE; goto fail; }
        for (uint32_t k = 0; k < t->ndim; k++)
            if ((e = rd_u64(&r, &t->dims[k]))) goto fail;
        if ((e = rd_u32(&r, &t->type))) goto fail;
        if ((e = rd_u64(&r, &t->offset))) goto fail;
        for (uint64_t j = 0; j < i; j++)
            if (out->tensors[j].name_len == t->name_len &&
                !memcmp(out->tensors[j].name, t->name, t->name_len)) {
                e = G_DUPLICATE_TENSOR_NAME;
                goto fail;
            }
        out->n_tensors = i + 1;
    }
    out->data_offset = (r.pos + 31) & ~(size_t)31;
    if (out->data_offset > len) { e = G_TRUNCATED; goto fail; }
    {
        rng *rs = calloc(out->n_tensors ? out->n_tensors : 1, sizeof(rng));
        for (size_t i = 0; i < out->n_tensors; i++) {
            uint64_t el;
            if ((e = encoded_len(&out->tensors[i], &el))) { free(rs); goto fail; }
            uint64_t s = out->data_offset + out->tensors[i].offset;
            if (s < out->tensors[i].offset || s + el < s) { free(rs); e = G_INVALID_TENSOR_OFFSET; goto fail; }
            if (s + el > len) { free(rs); e = G_TRUNCATED; goto fail; }
            rs[i].s = s;
            rs[i].e = s + el;
        }
        qsort(rs, out->n_tensors, sizeof(rng), rng_cmp);
        for (size_t i = 1; i < out->n_tensors; i++)
            if (rs[i - 1].e > rs[i].s) { free(rs); e = G_INVALID_TENSOR_OFFSET; goto fail; }
        free(rs);
    }
    return G_OK;
fail:
    g_free(out);
    return e;
}

void g_free(g_file *f) {
    free(f->kv);
    free(f->tensors);
    f->kv = NULL;
    f->tensors = NULL;
}

const g_kv *g_find_kv(const g_file *f, const char *key) {
    size_t n = strlen(key);
    for (size_t i = 0; i < f->n_kv; i++)
        if (f->kv[i].key_len == n && !memcmp(f->kv[i].key, key, n)) return &f->kv[i];
    return NULL;
}

int g_find_tensor(const g_file *f, const char *name, const g_tensor **out) {
    size_t n = strlen(name);
    const g_tensor *hit = NULL;
    for (size_t i = 0; i < f->n_tensors; i++)
        if (f->tensors[i].name_len == n && !memcmp(f->tensors[i].name, name, n)) {
            if (hit) return G_DUPLICATE_TENSOR_NAME;
            hit = &f->tensors[i];
        }
    if (!hit) return G_TENSOR_NOT_FOUND;
    *out = hit;
    return G_OK;
}

/* lib.rs:286-300 */
int g_meta_u32(const g_file *f, const char *key, uint32_t *out) {
    const g_kv *kv = g_find_kv(f, key);
    if (!kv) return G_METADATA_NOT_FOUND;
    if (kv->type == GV_U32) { *out = (uint32_t)kv->v.u; return G_OK; }
    if (kv->type == GV_U64) {
        if (kv->v.u > 0xffffffffull) return G_METADATA_TYPE_MISMATCH;
        *out = (uint32_t)kv->v.u;
        return G_OK;
    }
    return G_METADATA_TYPE_MISMATCH;
}

int g_meta_f32(const g_file *f, const char *key, float *out) {
    const g_kv *kv = g_find_kv(f, key);
    if (!kv) return G_METADATA_NOT_FOUND;
    if (kv->type == GV_F32 || kv->type == GV_F64) { *out = (float)kv->v.f; return G_OK; }
    return G_METADATA_TYPE_MISMATCH;
}

int g_meta_str(const g_file *f, const char *key, const char **s, size_t *len) {
    const g_kv *kv = g_find_kv(f, key);
    if (!kv) return G_METADATA_NOT_FOUND;
    if (kv->type != GV_STRING) return G_METADATA_TYPE_MISMATCH;
    *s = kv->str;
    *len = kv->str_len;
    return G_OK;
}

int g_tensor_data(const g_file *f, const g_tensor *t, const uint8_t **data, size_t *len) {
    uint64_t el;
    int e = encoded_len(t, &el);
    if (e) return e;
    uint64_t s = f->data_offset + t->offset;
    if (s + el > f->len) return G_TRUNCATED;
    *data = f->bytes + s;
    *len = (size_t)el;
    return G_OK;
}
