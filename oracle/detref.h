/*
 * detref — CPU oracle for the detllm hot path (TEST INFRASTRUCTURE ONLY).
 *
 * This library is a plain-C restatement of the reference CPU arithmetic of
 * mii443/detllm (crates det-num, det-quant, det-gguf, det-model, det-coder).
 * It exists to check the HIP implementation: only tests/, the smoke check
 * and the CPU-baseline leg of bench.py may load it.  Nothing in the product
 * library links or calls it.
 *
 * Every function cites the reference file:line it follows.  Status codes
 * restate the reference error enums (ModelError, CdfError, RangeError)
 * with the numeric values used across this repository's C ABI.
 */
#ifndef DETREF_H
#define DETREF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    REF_OK = 0,
    /* det-model ModelError (crates/det-model/src/lib.rs:48-59) */
    REF_ERR_SHAPE = 1,
    REF_ERR_NON_FINITE = 2,
    REF_ERR_UNSUPPORTED_ARCHITECTURE = 3,
    REF_ERR_UNSUPPORTED_ATTENTION_HEAD_LENGTH = 4,
    REF_ERR_UNSUPPORTED_MODEL_FEATURE = 5,
    REF_ERR_UNSUPPORTED_ROPE_SCALING = 6,
    REF_ERR_MISSING_METADATA = 7,
    REF_ERR_GGUF = 8,
    REF_ERR_UNSUPPORTED_TENSOR_TYPE = 9,
    REF_ERR_THREAD_PANICKED = 10,
    /* det-coder CdfError (crates/det-coder/src/cdf.rs:9-17) */
    REF_ERR_CDF_EMPTY = 20,
    REF_ERR_CDF_MALFORMED = 21,
    REF_ERR_CDF_NON_FINITE_LOGIT = 22,
    REF_ERR_CDF_SYMBOL_OUT_OF_RANGE = 23,
    REF_ERR_CDF_TOO_MANY_SYMBOLS = 24,
    REF_ERR_CDF_TOTAL_TOO_LARGE = 25,
    /* det-coder RangeError (crates/det-coder/src/range.rs:4-8) */
    REF_ERR_RANGE_INVALID_FREQUENCY = 30,
    REF_ERR_RANGE_UNEXPECTED_EOF = 31,
    /* det-quant QuantError surfaced directly by the block-level entry points */
    REF_ERR_QUANT = 50
};

/* ---- det-num ---------------------------------------------------------- */
float ref_exp_f32(float x);
void ref_exp_f32_array(const float *x, float *out, size_t n, int clamp);
double ref_exp_f64(double x);
double ref_ln_f64(double x);
double ref_sin_f64(double x);
double ref_cos_f64(double x);
float ref_silu_f32(float x);
float ref_f16_to_f32(uint16_t bits);
int32_t ref_round_ties_even_i32(float x);
int64_t ref_round_ties_even_i64(double x);
float ref_dot_f32(const float *x, const float *y, size_t n);
float ref_sum_f32(const float *x, size_t n);
float ref_sum_squares_f32(const float *x, size_t n);
void ref_sha256(const void *data, size_t len, uint8_t out[32]);
void ref_numeric_canary(uint8_t out[32]);
int ref_runtime_canary(uint8_t out[32]);
int ref_quant_kernel_hash(uint8_t out[32]);

/* ---- det-quant -------------------------------------------------------- */
/* Quantise n floats (n % 32 == 0) into Q8A: d[n/32], q[n]. */
int ref_quantize_q8a(const float *x, size_t n, float *d, int8_t *q);
/* Quantise n floats (n % 256 == 0) into Q8_K: d[n/256], q[n]. */
int ref_quantize_q8k(const float *x, size_t n, float *d, int8_t *q);
/* One GEMV row in GGUF encoding (type 0 F32, 2 Q4_0, 8 Q8_0, 12 Q4_K,
 * 14 Q6_K) against activations x[cols], quantising x as the reference
 * does for that type. */
int ref_dot_row(int ggml_type, const uint8_t *row, size_t cols, const float *x, float *out);

/* ---- det-model -------------------------------------------------------- */
typedef struct ref_model ref_model;
typedef struct ref_session ref_session;

ref_model *ref_model_load(const uint8_t *gguf, size_t len, int *status);
void ref_model_free(ref_model *m);
/* out[0..15]: block_count, d, ff, heads, kv_heads, head_dim, rope_dim,
 * pairing (0 adjacent, 1 split-half), context_length, vocab,
 * rms_eps bits, attention_scale bits, rope_base bits, emb type, out type, has_bias */
void ref_model_config(const ref_model *m, int64_t out[16]);
/* One layer's q (which 0), k (1) or v (2) bias: copies min(len, cap)
 * values into out and returns len, 0 when absent. */
size_t ref_model_bias(const ref_model *m, size_t layer, int which, float *out, size_t cap);
ref_session *ref_session_new(const ref_model *m, size_t max_ctx, int *status);
void ref_session_free(ref_session *s);
int ref_session_reset(ref_session *s);
int ref_forward_one(ref_session *s, size_t token, size_t pos, float *logits);
int ref_logits_hash(const ref_model *m, const uint32_t *tokens, size_t n, size_t chunk, uint8_t out[32]);
int ref_logits(const ref_model *m, const uint32_t *tokens, size_t n, float *out);
int ref_rope_table(const ref_model *m, size_t positions, float *cos_out, float *sin_out);
/* apply_rope (det-model lib.rs:2011-2051) on heads x head_dim values with
 * one position's cos/sin row (rope_dim/2 entries). */
int ref_apply_rope(float *x, size_t heads, size_t head_dim, size_t rope_dim, int split_half,
                   const float *cos_row, const float *sin_row);
void ref_set_threads(size_t threads);
void ref_set_simd(int on);

/* ---- det-coder -------------------------------------------------------- */
int ref_logits_to_cdf(const float *logits, size_t n, size_t tail, uint32_t *freq, uint64_t *cum,
                      uint64_t *total);
int ref_symbol_range(const float *logits, size_t n, size_t symbol, size_t tail, uint64_t *cum,
                     uint32_t *freq, uint64_t *total);
int ref_decoder_lookup(const float *logits, size_t n, size_t tail, uint64_t value, uint64_t *symbol,
                       uint64_t *cum, uint32_t *freq, uint64_t *total);
int ref_decoder_total(const float *logits, size_t n, size_t tail, uint64_t *total);
int ref_uniform_symbol_range(size_t symbol, size_t symbols, uint64_t *cum, uint32_t *freq,
                             uint64_t *total);

typedef struct ref_range_encoder ref_range_encoder;
ref_range_encoder *ref_range_encoder_new(void);
int ref_range_encode(ref_range_encoder *e, uint64_t cum, uint64_t freq, uint64_t total);
/* Finishes the stream; copies min(len, cap) bytes into out; returns len. */
size_t ref_range_encoder_finish(ref_range_encoder *e, uint8_t *out, size_t cap);
void ref_range_encoder_free(ref_range_encoder *e);

typedef struct ref_range_decoder ref_range_decoder;
ref_range_decoder *ref_range_decoder_new(const uint8_t *data, size_t len, int *status);
int ref_range_decode_freq(ref_range_decoder *d, uint64_t total, uint64_t *value);
int ref_range_decode_advance(ref_range_decoder *d, uint64_t cum, uint64_t freq, uint64_t total);
void ref_range_decoder_free(ref_range_decoder *d);

/* ---- det-token byte fallback + det-cli windowed codec ----------------- */
int ref_canonical_byte_token(const char *tok, size_t len);
int ref_byte_fallback_tables(const char *text, const size_t *off, size_t n, const uint8_t *emit,
                             int32_t byte_to_token[256], int16_t *token_to_byte);
void ref_codec_symbols(const int32_t byte_to_token[256], const uint8_t *in, size_t n,
                       size_t vocab_len, uint32_t *out);
size_t ref_next_window_start(size_t pos, size_t window_start, size_t n_ctx, size_t overlap);
int ref_codec_encode(const ref_model *m, const uint32_t *symbols, size_t n, size_t n_ctx,
                     size_t overlap, int escapes, uint8_t *out, size_t cap, size_t *len);
int ref_codec_decode(const ref_model *m, const int16_t *token_to_byte, const uint8_t *payload,
                     size_t plen, size_t byte_len, size_t n_ctx, size_t overlap, int escapes,
                     uint32_t *symbols, uint8_t *bytes, size_t *n_out);

#ifdef __cplusplus
}
#endif
#endif
