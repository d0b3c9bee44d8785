/*
 * detref logits->CDF and range coder — TEST INFRASTRUCTURE ONLY (the oracle).
 *
 * Restates crates/det-coder of mii443/detllm:
 *   logits_to_cdf_with_scratch (+ byte-escape tail)  src/cdf.rs:52-106, 255-300
 *   logits_to_symbol_range_impl                      src/cdf.rs:138-199
 *   logits_to_decoder_distribution_impl + lookup     src/cdf.rs:201-245, 392-425
 *   uniform_symbol_range                              src/cdf.rs:322-341
 *   RangeEncoder / RangeDecoder                       src/range.rs:1-178
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "detref.h"
#include "detref_internal.h"

#define CDF_M 16777216.0f
#define MAX_SYMBOLS (1u << 18)
#define TOTAL_LIMIT (1ull << 31)

/* Shared front half: max, clamped exp, 8-lane Z (cdf.rs:63-76). */
static int cdf_prepare(const float *logits, size_t n, size_t tail, float **exp_out, float *z_out) {
    if (n == 0) return REF_ERR_CDF_EMPTY;
    if (n + tail > MAX_SYMBOLS) return REF_ERR_CDF_TOO_MANY_SYMBOLS;
    float max = -INFINITY;
    for (size_t i = 0; i < n; i++) {
        if (!isfinite(logits[i])) return REF_ERR_CDF_NON_FINITE_LOGIT;
        if (logits[i] > max) max = logits[i];
    }
    float *e = malloc(n * sizeof(float));
    for (size_t i = 0; i < n; i++) {
        float t = logits[i] - max;
        e[i] = ref_exp_f32(t < -88.0f ? -88.0f : t);
    }
    *z_out = ref_sum_f32(e, n);
    *exp_out = e;
    return REF_OK;
}

static inline uint32_t freq_of(float ei, float z) {
    float p = ei / z;
    float g = p * CDF_M;
    /* Rust `as u32`: truncation, saturating; p*M lies in [0, 2^24]. */
    uint32_t gi = g <= 0.0f ? 0u : (g >= 4294967296.0f ? 0xffffffffu : (uint32_t)g);
    return gi + 1;
}

int ref_logits_to_cdf(const float *logits, size_t n, size_t tail, uint32_t *freq, uint64_t *cum,
                      uint64_t *total) {
    float *e, z;
    int st = cdf_prepare(logits, n, tail, &e, &z);
    if (st) return st;
    uint64_t t = 0;
    for (size_t i = 0; i < n; i++) {
        uint32_t f = freq_of(e[i], z);
        cum[i] = t;
        freq[i] = f;
        t += f;
    }
    free(e);
    if (t >= TOTAL_LIMIT) return REF_ERR_CDF_TOTAL_TOO_LARGE;
    if (tail) {
        if (t + tail >= TOTAL_LIMIT) return REF_ERR_CDF_TOTAL_TOO_LARGE;
        for (size_t i = 0; i < tail; i++) {
            cum[n + i] = t;
            freq[n + i] = 1;
            t += 1;
        }
    }
    *total = t;
    return REF_OK;
}

int ref_symbol_range(const float *logits, size_t n, size_t symbol, size_t tail, uint64_t *cum,
                     uint32_t *freq, uint64_t *total) {
    if (n == 0) return REF_ERR_CDF_EMPTY;
    if (n + tail > MAX_SYMBOLS) return REF_ERR_CDF_TOO_MANY_SYMBOLS;
    if (symbol >= n + tail) return REF_ERR_CDF_SYMBOL_OUT_OF_RANGE;
    float *e, z;
    int st = cdf_prepare(logits, n, tail, &e, &z);
    if (st) return st;
    uint64_t t = 0, c = 0;
    uint32_t fs = 0;
    for (size_t i = 0; i < n; i++) {
        uint32_t f = freq_of(e[i], z);
        if (i == symbol) { c = t; fs = f; }
        t += f;
    }
    free(e);
    if (symbol >= n) { c = t + (symbol - n); fs = 1; }
    t += tail;
    if (t >= TOTAL_LIMIT) return REF_ERR_CDF_TOTAL_TOO_LARGE;
    *cum = c;
    *freq = fs;
    *total = t;
    return REF_OK;
}

static int decoder_freqs(const float *logits, size_t n, size_t tail, uint32_t **fo, uint64_t *total) {
    float *e, z;
    int st = cdf_prepare(logits, n, tail, &e, &z);
    if (st) return st;
    uint32_t *f = malloc(n * sizeof(uint32_t));
    uint64_t t = 0;
    for (size_t i = 0; i < n; i++) {
        f[i] = freq_of(e[i], z);
        t += f[i];
    }
    free(e);
    t += tail;
    if (t >= TOTAL_LIMIT) { free(f); return REF_ERR_CDF_TOTAL_TOO_LARGE; }
    *fo = f;
    *total = t;
    return REF_OK;
}

int ref_decoder_total(const float *logits, size_t n, size_t tail, uint64_t *total) {
    uint32_t *f;
    int st = decoder_freqs(logits, n, tail, &f, total);
    if (!st) free(f);
    return st;
}

/* DecoderDistribution::symbol_range (cdf.rs:392-425): linear scan. */
int ref_decoder_lookup(const float *logits, size_t n, size_t tail, uint64_t value, uint64_t *symbol,
                       uint64_t *cum, uint32_t *freq, uint64_t *total) {
    uint32_t *f;
    uint64_t t;
    int st = decoder_freqs(logits, n, tail, &f, &t);
    if (st) return st;
    *total = t;
    if (value >= t) { free(f); return REF_ERR_CDF_SYMBOL_OUT_OF_RANGE; }
    uint64_t c = 0;
    for (size_t i = 0; i < n; i++) {
        uint64_t next = c + f[i];
        if (value < next) {
            *symbol = i;
            *cum = c;
            *freq = f[i];
            free(f);
            return REF_OK;
        }
        c = next;
    }
    free(f);
    uint64_t off = value - c;
    if (off < tail) {
        *symbol = n + off;
        *cum = value;
        *freq = 1;
        return REF_OK;
    }
    return REF_ERR_CDF_SYMBOL_OUT_OF_RANGE;
}

int ref_uniform_symbol_range(size_t symbol, size_t symbols, uint64_t *cum, uint32_t *freq,
                             uint64_t *total) {
    if (symbols == 0) return REF_ERR_CDF_EMPTY;
    if (symbols > MAX_SYMBOLS) return REF_ERR_CDF_TOO_MANY_SYMBOLS;
    if (symbol >= symbols) return REF_ERR_CDF_SYMBOL_OUT_OF_RANGE;
    *cum = symbol;
    *freq = 1;
    *total = symbols;
    return REF_OK;
}

/* ---- range coder: crates/det-coder/src/range.rs ------------------------- */
#define RC_TOP (1ull << 56)
#define RC_BOTTOM (1ull << 48)

struct ref_range_encoder {
    uint64_t low, range;
    uint8_t *out;
    size_t len, cap;
};

static void push_byte(ref_range_encoder *e, uint8_t b) {
    if (e->len == e->cap) {
        e->cap = e->cap ? e->cap * 2 : 256;
        e->out = realloc(e->out, e->cap);
    }
    e->out[e->len++] = b;
}

static int rc_validate(uint64_t cum, uint64_t freq, uint64_t total) {
    uint64_t end = cum + freq;
    if (end < cum) return REF_ERR_RANGE_INVALID_FREQUENCY;
    if (freq == 0 || total == 0 || total >= TOTAL_LIMIT || end > total)
        return REF_ERR_RANGE_INVALID_FREQUENCY;
    return REF_OK;
}

/* normalize_step (range.rs:168-178) */
static int normalize_step(uint64_t low, uint64_t *range) {
    if ((low ^ (low + *range)) < RC_TOP) return 1;
    if (*range < RC_BOTTOM) {
        *range = (0 - low) & (RC_BOTTOM - 1);
        return 1;
    }
    return 0;
}

ref_range_encoder *ref_range_encoder_new(void) {
    ref_range_encoder *e = calloc(1, sizeof *e);
    e->range = UINT64_MAX;
    return e;
}

int ref_range_encode(ref_range_encoder *e, uint64_t cum, uint64_t freq, uint64_t total) {
    int st = rc_validate(cum, freq, total);
    if (st) return st;
    e->range /= total;
    e->low += e->range * cum;
    e->range *= freq;
    while (normalize_step(e->low, &e->range)) {
        push_byte(e, (uint8_t)(e->low >> 56));
        e->low <<= 8;
        e->range <<= 8;
    }
    return REF_OK;
}

size_t ref_range_encoder_finish(ref_range_encoder *e, uint8_t *out, size_t cap) {
    uint64_t low = e->low;
    size_t base = e->len;
    for (int i = 0; i < 8; i++) {
        push_byte(e, (uint8_t)(low >> 56));
        low <<= 8;
    }
    size_t n = e->len;
    if (out && cap) memcpy(out, e->out, n < cap ? n : cap);
    e->len = base;
    return n;
}

void ref_range_encoder_free(ref_range_encoder *e) {
    if (!e) return;
    free(e->out);
    free(e);
}

struct ref_range_decoder {
    uint64_t low, code, range;
    int pending;
    uint64_t pending_range, pending_total;
    const uint8_t *in;
    size_t len, pos;
};

static int read_byte(ref_range_decoder *d, uint8_t *b) {
    if (d->pos >= d->len) return REF_ERR_RANGE_UNEXPECTED_EOF;
    *b = d->in[d->pos++];
    return REF_OK;
}

ref_range_decoder *ref_range_decoder_new(const uint8_t *data, size_t len, int *status) {
    ref_range_decoder *d = calloc(1, sizeof *d);
    d->range = UINT64_MAX;
    d->in = data;
    d->len = len;
    for (int i = 0; i < 8; i++) {
        uint8_t b;
        if ((*status = read_byte(d, &b))) { free(d); return NULL; }
        d->code = (d->code << 8) | b;
    }
    *status = REF_OK;
    return d;
}

int ref_range_decode_freq(ref_range_decoder *d, uint64_t total, uint64_t *value) {
    if (d->pending) return REF_ERR_RANGE_INVALID_FREQUENCY;
    if (total == 0 || total >= TOTAL_LIMIT) return REF_ERR_RANGE_INVALID_FREQUENCY;
    uint64_t r = d->range / total;
    if (r == 0) return REF_ERR_RANGE_INVALID_FREQUENCY;
    uint64_t v = (d->code - d->low) / r;
    if (v >= total) return REF_ERR_RANGE_INVALID_FREQUENCY;
    d->pending = 1;
    d->pending_range = r;
    d->pending_total = total;
    *value = v;
    return REF_OK;
}

int ref_range_decode_advance(ref_range_decoder *d, uint64_t cum, uint64_t freq, uint64_t total) {
    int st = rc_validate(cum, freq, total);
    if (st) return st;
    if (!d->pending || d->pending_total != total) return REF_ERR_RANGE_INVALID_FREQUENCY;
    d->pending = 0;
    d->range = d->pending_range;
    d->low += d->range * cum;
    d->range *= freq;
    while (normalize_step(d->low, &d->range)) {
        uint8_t b;
        if ((st = read_byte(d, &b))) return st;
        d->code = (d->code << 8) | b;
        d->low <<= 8;
        d->range <<= 8;
    }
    return REF_OK;
}

void ref_range_decoder_free(ref_range_decoder *d) { free(d); }
