/*
 * detllm_amd — MI355X (gfx950) implementation of detllm's per-token decoder
 * forward pass and logits -> integer-CDF step, behind a C ABI.
 *
 * Every entry point replaces one item of the reference Rust API of
 * mii443/detllm (crates/det-model, crates/det-coder); the comment above each
 * declaration names it (file:line).  Results are bit-identical to the
 * reference CPU arithmetic: logits, CDF frequencies and range-coder bytes.
 *
 * Conventions
 *   - Every function returns a dtl_status (0 = OK).  No exceptions or
 *     unwinding cross this boundary.
 *   - Host pointers only; the library owns all device memory.
 *   - A dtl_model is immutable after load and may be shared by sessions on
 *     any host thread.  A dtl_session is single-threaded: it owns one HIP
 *     stream, a KV cache, RoPE tables and a workspace for up to max_chunk
 *     positions (the reference's KvCache + ForwardWorkspace + RopeTables).
 */
#ifndef DETLLM_H
#define DETLLM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  1-10 mirror det-model ModelError (lib.rs:48-59),
 * 20-25 det-coder CdfError (cdf.rs:9-17), 30-31 RangeError (range.rs:4-8). */
typedef enum {
    DTL_OK = 0,
    DTL_ERR_SHAPE = 1,
    DTL_ERR_NON_FINITE = 2,
    DTL_ERR_UNSUPPORTED_ARCHITECTURE = 3,
    DTL_ERR_UNSUPPORTED_ATTENTION_HEAD_LENGTH = 4,
    DTL_ERR_UNSUPPORTED_MODEL_FEATURE = 5,
    DTL_ERR_UNSUPPORTED_ROPE_SCALING = 6,
    DTL_ERR_MISSING_METADATA = 7,
    DTL_ERR_GGUF = 8,
    DTL_ERR_UNSUPPORTED_TENSOR_TYPE = 9,
    DTL_ERR_THREAD_PANICKED = 10,
    DTL_ERR_CDF_EMPTY = 20,
    DTL_ERR_CDF_MALFORMED = 21,
    DTL_ERR_CDF_NON_FINITE_LOGIT = 22,
    DTL_ERR_CDF_SYMBOL_OUT_OF_RANGE = 23,
    DTL_ERR_CDF_TOO_MANY_SYMBOLS = 24,
    DTL_ERR_CDF_TOTAL_TOO_LARGE = 25,
    DTL_ERR_RANGE_INVALID_FREQUENCY = 30,
    DTL_ERR_RANGE_UNEXPECTED_EOF = 31,
    /* No reference counterpart: device / argument failures of this library. */
    DTL_ERR_DEVICE = 40,
    DTL_ERR_OUT_OF_MEMORY = 41,
    DTL_ERR_INVALID_ARGUMENT = 42,
    DTL_ERR_NO_DEVICE = 43,
    DTL_ERR_BUFFER_TOO_SMALL = 44, /* output capacity below the size in *len */
    DTL_ERR_STATIC_SCRATCH_LIMIT = 45, /* a call larger than dtl_symbol_ranges_static's scratch */
    /* 60-77: det-token TokenError (crates/det-token/src/lib.rs:6-25), in order;
     * 77 also reports a BPE / SentencePiece vocabulary, which this library
     * does not tokenize. */
    DTL_ERR_TOKEN_MISSING_BYTE_FALLBACK = 60,
    DTL_ERR_TOKEN_INVALID_TOKEN = 61,
    DTL_ERR_TOKEN_MISSING_VOCABULARY = 62,
    DTL_ERR_TOKEN_MISSING_TOKEN_BYTES = 63,
    DTL_ERR_TOKEN_MISSING_MERGE_TOKEN = 64,
    DTL_ERR_TOKEN_INCOMPLETE_BYTE_FALLBACK = 65,
    DTL_ERR_TOKEN_METADATA_TYPE = 66,
    DTL_ERR_TOKEN_TYPE_LENGTH = 67,
    DTL_ERR_TOKEN_INVALID_TOKEN_TYPE = 68,
    DTL_ERR_TOKEN_SCORES_LENGTH = 69,
    DTL_ERR_TOKEN_NON_FINITE_SCORE = 70,
    DTL_ERR_TOKEN_INDEX_OVERFLOW = 71,
    DTL_ERR_TOKEN_DUPLICATE_BYTE_FALLBACK = 72,
    DTL_ERR_TOKEN_DUPLICATE_TOKEN_ID = 73,
    DTL_ERR_TOKEN_DUPLICATE_TOKEN_BYTES = 74,
    DTL_ERR_TOKEN_INVALID_MERGE = 75,
    DTL_ERR_TOKEN_DUPLICATE_MERGE = 76,
    DTL_ERR_TOKEN_UNSUPPORTED_MODEL = 77,
    /* 80-85: det-coder FileError (crates/det-coder/src/file.rs:18-25). */
    DTL_ERR_FILE_TOO_SHORT = 80,
    DTL_ERR_FILE_BAD_MAGIC = 81,
    DTL_ERR_FILE_UNSUPPORTED_VERSION = 82,
    DTL_ERR_FILE_UNSUPPORTED_FLAGS = 83,
    DTL_ERR_FILE_INVALID_CONTEXT = 84,
    DTL_ERR_FILE_INVALID_OVERLAP = 85,
    /* 90-92: the codec failures det-cli reports as messages
     * (crates/det-cli/src/main.rs:478-480, 503-507, 571-573). */
    DTL_ERR_CODEC_MODEL_MISMATCH = 90,
    DTL_ERR_CODEC_NOT_CANONICAL = 91,
    DTL_ERR_CODEC_ESCAPE_IN_TOKEN_STREAM = 92,
    DTL_ERR_CODEC_VOCAB_MISMATCH = 93 /* tokenizer vocabulary != model vocabulary */
} dtl_status;

typedef struct dtl_model dtl_model;
typedef struct dtl_session dtl_session;

/* LlamaConfig (crates/det-model/src/lib.rs:27-39) plus the output vocab. */
typedef struct {
    uint64_t block_count;
    uint64_t embedding_length;
    uint64_t feed_forward_length;
    uint64_t head_count;
    uint64_t head_count_kv;
    uint64_t head_dim;
    uint64_t rope_dimension_count;
    uint64_t context_length;
    uint64_t vocab;               /* output.rows() */
    float rms_epsilon;
    float attention_scale;
    float rope_freq_base;
    int32_t rope_split_half;      /* RopePairing: 0 Adjacent (llama), 1 SplitHalf (qwen2) */
    int32_t embedding_type;       /* ggml type id of token_embd */
    int32_t output_type;          /* ggml type id of output (or tied embedding) */
    int32_t has_qkv_bias;
    uint64_t device_bytes;        /* device memory held by the weights */
} dtl_model_config;

/* Human-readable name of a status code (static storage). */
const char *dtl_status_string(int status);

/* ---- det-model --------------------------------------------------------- */

/* F32Llama::from_gguf (det-model lib.rs:1035-1140) with det_gguf::parse
 * (det-gguf lib.rs:156-216).  The caller keeps ownership of the bytes; the
 * weights are validated, repacked and copied to the current HIP device. */
int dtl_model_load(const uint8_t *gguf, size_t len, dtl_model **out);
void dtl_model_free(dtl_model *model);
/* F32Llama::config + output.rows() (det-model lib.rs:27-39, 1178-1187). */
int dtl_model_get_config(const dtl_model *model, dtl_model_config *out);

/* F32Llama::forward_workspace + KvCache::new + RopeTables::llama
 * (det-model lib.rs:1244, 850, 813).  n_ctx <= context_length positions of
 * RoPE table and KV cache; max_chunk = most positions one dtl_forward_chunk
 * call may carry (1 for pure decode). */
int dtl_session_new(const dtl_model *model, size_t n_ctx, size_t max_chunk, dtl_session **out);
void dtl_session_free(dtl_session *session);
/* A fresh KvCache for window replay (det-cli main.rs:691-701). */
int dtl_session_reset(dtl_session *session);

/* F32Llama::forward_one_with_workspace (det-model lib.rs:1249-1400).
 * logits: vocab floats on the host, or NULL to keep them on the device
 * (they then feed dtl_symbol_ranges / dtl_decoder_lookup). */
int dtl_forward_one(dtl_session *session, uint32_t token, size_t pos, float *logits);

/* n consecutive forward_one_with_workspace calls at positions pos0..pos0+n-1
 * as one batched device pass (teacher-forced encode).  Bit-identical to n
 * single-token calls.  logits: n*vocab host floats or NULL. */
int dtl_forward_chunk(dtl_session *session, const uint32_t *tokens, size_t n, size_t pos0,
                      float *logits);

/* Copies rows [first, first+n) of the last forward's logits to the host. */
int dtl_session_logits(dtl_session *session, size_t first, size_t n, float *out);

/* The session's window (n_ctx), chunk capacity and the model's output vocab
 * (no reference counterpart: lets host drivers size their work). */
int dtl_session_get_info(const dtl_session *session, size_t *n_ctx, size_t *max_chunk,
                         size_t *vocab);

/* F32Llama::logits_hash_for_tokens_chunked (det-model lib.rs:1406-1465):
 * SHA-256 of every position's f32 logits (little-endian bits), positions
 * ascending.  chunk sets how many positions share one device pass. */
int dtl_logits_hash(const dtl_model *model, const uint32_t *tokens, size_t n, size_t chunk,
                    uint8_t out[32]);

/* ---- device timing (no reference counterpart: measurement support) ------ */

/* Per kernel class: launches, summed device time of those launches (HIP
 * events bound to the kernels on the session stream, first kernel's start
 * to last kernel's end of each timed launch), and the algorithmic HBM bytes /
 * multiply-accumulates they imply. */
typedef struct {
    char name[32];
    uint64_t launches;
    double total_ms;
    double bytes;
    double macs;
} dtl_kernel_stat;

/* Enables (1) or disables (0) event timing of every launch; enabling
 * clears the accumulated statistics. */
int dtl_session_set_profiling(dtl_session *session, int enable);
/* While profiling is enabled, time only launches of this kernel class
 * (NULL or "": every class); the others run untimed. */
int dtl_session_profile_only(dtl_session *session, const char *kernel_class);
/* Copies up to cap entries; *n receives the number of kernel classes. */
int dtl_session_profile(dtl_session *session, dtl_kernel_stat *out, size_t cap, size_t *n);

/* ---- det-coder on device-resident logits -------------------------------- */

/* logits_to_symbol_range_with_scratch / _with_byte_escapes
 * (det-coder cdf.rs:123-199) for rows [first, first+n) of the session's
 * last logits: symbols[i] is coded against row first+i.  tail_symbols is 0
 * or 256 (BYTE_ESCAPE_SYMBOLS). */
int dtl_symbol_ranges(dtl_session *session, size_t first, size_t n, const uint32_t *symbols,
                      size_t tail_symbols, uint64_t *cum, uint32_t *freq, uint64_t *total);

/* The same for an arbitrary row of the last forward per symbol: symbols[i]
 * is coded against row rows[i] (several symbols may share a row, as byte
 * escapes share the logits of the last token in det-cli's codec loop). */
int dtl_symbol_ranges_rows(dtl_session *session, size_t n, const uint32_t *rows,
                           const uint32_t *symbols, size_t tail_symbols, uint64_t *cum,
                           uint32_t *freq, uint64_t *total);

/* The forwards and symbol ranges of one codec window in one call: the
 * per-token loop of encode_symbols_with_model (det-cli main.rs:521-551:
 * state.sync / symbol_range / advance), batched.  Forwards tokens[0..n) at
 * positions pos0.. in chunks of the session's max_chunk and codes
 * symbols[i] against the logits of token rows[i] (rows relative to pos0,
 * non-decreasing, < n).  The same results as dtl_forward_chunk followed by
 * dtl_symbol_ranges_rows per chunk; four chunks are in flight on four
 * streams.  Afterwards no logits rows are valid (dtl_session_logits and
 * dtl_cdf need a new forward). */
int dtl_forward_ranges(dtl_session *session, const uint32_t *tokens, size_t n, size_t pos0,
                       size_t n_sym, const uint32_t *rows, const uint32_t *symbols,
                       size_t tail_symbols, uint64_t *cum, uint32_t *freq, uint64_t *total);

/* logits_to_cdf_with_scratch / _with_byte_escapes (cdf.rs:52-106): the
 * full table for one row; freq and cum hold vocab + tail_symbols entries. */
int dtl_cdf(dtl_session *session, size_t row, size_t tail_symbols, uint32_t *freq, uint64_t *cum,
            uint64_t *total);

/* logits_to_decoder_distribution_* + DecoderDistribution::total
 * (cdf.rs:108-121, 201-245, 387-390). */
int dtl_decoder_total(dtl_session *session, size_t row, size_t tail_symbols, uint64_t *total);

/* DecoderDistribution::symbol_range (cdf.rs:392-425), run on the device. */
int dtl_decoder_lookup(dtl_session *session, size_t row, size_t tail_symbols, uint64_t value,
                       uint32_t *symbol, uint64_t *cum, uint32_t *freq, uint64_t *total);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory: code under HIP graph capture, serving loops and harnesses that
 * forbid hipMalloc.  The symbol ranges of dtl_symbol_ranges /
 * dtl_logits_to_symbol_range (logits_to_symbol_range_*, det-coder
 * cdf.rs:122-199) of symbols[i] against row i of logits[rows][vocab], with
 * every pointer in device memory and the work enqueued on `stream` (a
 * hipStream_t; NULL is the default stream) without waiting for it.  The
 * CDF scratch is a static device array of 8,399,360 bytes per GPU (the
 * scratch of 8 rows at vocab 2^18), held until the
 * process ends: rows <= 8 and vocab + tail_symbols <= 2^18, else
 * DTL_ERR_STATIC_SCRATCH_LIMIT.  The call allocates nothing.  *status_bits
 * (device memory) is overwritten with the call's error bits once the stream
 * reaches it; dtl_status_from_bits maps them to a dtl_status.  Calls that
 * overlap on one GPU share the scratch and race. */
int dtl_symbol_ranges_static(const float *logits, size_t rows, size_t vocab, const uint32_t *symbols,
                             size_t tail_symbols, uint64_t *cum, uint32_t *freq, uint64_t *total,
                             int *status_bits, void *stream);
/* The dtl_status a device status word of dtl_symbol_ranges_static reports. */
int dtl_status_from_bits(int bits);

/* logits_to_cdf / logits_to_symbol_range on caller logits (host memory):
 * uploads them and runs the same device kernels (cdf.rs:47-199). */
int dtl_logits_to_cdf(const float *logits, size_t n, size_t tail_symbols, uint32_t *freq,
                      uint64_t *cum, uint64_t *total);
int dtl_logits_to_symbol_range(const float *logits, size_t n, size_t symbol, size_t tail_symbols,
                               uint64_t *cum, uint32_t *freq, uint64_t *total);

/* uniform_cdf (cdf.rs:302-320): freq[i] = 1, cum[i] = i over `symbols`
 * entries, total = symbols (the CDF of a window's first position, context
 * length 0, with vocab + 256 symbols when byte escapes are on). */
int dtl_uniform_cdf(size_t symbols, uint32_t *freq, uint64_t *cum, uint64_t *total);
/* uniform_symbol_range (cdf.rs:322-341). */
int dtl_uniform_symbol_range(size_t symbol, size_t symbols, uint64_t *cum, uint32_t *freq,
                             uint64_t *total);

/* ---- det-coder range coder (host) --------------------------------------- */
typedef struct dtl_range_encoder dtl_range_encoder;
typedef struct dtl_range_decoder dtl_range_decoder;

/* RangeEncoder::{new, encode, finish} (det-coder range.rs:30-92). */
int dtl_range_encoder_new(dtl_range_encoder **out);
int dtl_range_encode(dtl_range_encoder *enc, uint64_t cum, uint64_t freq, uint64_t total);
/* Appends the 8 flush bytes and copies min(len, cap) bytes; *len = full size.
 * The encoder stays usable (finish does not consume it). */
int dtl_range_encoder_finish(dtl_range_encoder *enc, uint8_t *out, size_t cap, size_t *len);
/* RangeEncoder::snapshot (det-coder range.rs:48-54): low, range and the
 * bytes emitted so far (out NULL: only their count in *len;
 * DTL_ERR_BUFFER_TOO_SMALL when cap < *len).  The encoder is unchanged. */
int dtl_range_encoder_snapshot(const dtl_range_encoder *enc, uint64_t *low, uint64_t *range,
                               uint8_t *out, size_t cap, size_t *len);
/* RangeEncoder::from_snapshot (range.rs:37-46): a new encoder resuming from
 * (low, range, bytes); range 0 is DTL_ERR_RANGE_INVALID_FREQUENCY. */
int dtl_range_encoder_from_snapshot(uint64_t low, uint64_t range, const uint8_t *bytes, size_t len,
                                    dtl_range_encoder **out);
void dtl_range_encoder_free(dtl_range_encoder *enc);

/* RangeDecoder::{new, decode_freq, advance} (det-coder range.rs:94-159). */
int dtl_range_decoder_new(const uint8_t *data, size_t len, dtl_range_decoder **out);
int dtl_range_decode_freq(dtl_range_decoder *dec, uint64_t total, uint64_t *value);
int dtl_range_decode_advance(dtl_range_decoder *dec, uint64_t cum, uint64_t freq, uint64_t total);
void dtl_range_decoder_free(dtl_range_decoder *dec);
/* A range decoder's state between two symbols: the RangeDecoder fields low,
 * range and code (det-coder range.rs:85-92) and the input bytes consumed.
 * No counterpart in the reference, whose decoder runs in one call: for a
 * long payload decoded across several calls (dtl_decompress_part). */
typedef struct dtl_range_decoder_state {
    uint64_t low, range, code, pos;
} dtl_range_decoder_state;
/* Copies the state (DTL_ERR_RANGE_INVALID_FREQUENCY between decode_freq and
 * advance). */
int dtl_range_decoder_snapshot(const dtl_range_decoder *dec, dtl_range_decoder_state *state);
/* A decoder over data[0, len) resuming from `state` (pos in [8, len]). */
int dtl_range_decoder_from_snapshot(const uint8_t *data, size_t len, const dtl_range_decoder_state *state,
                                    dtl_range_decoder **out);

/* The model branch of decode_symbol (det-cli main.rs:724-750) for logits
 * row `row`: logits_to_decoder_distribution_* (cdf.rs:108-121, 201-245),
 * RangeDecoder::decode_freq of its total (range.rs:110-126),
 * DecoderDistribution::symbol_range (cdf.rs:392-425) and
 * RangeDecoder::advance, with one wait for the device: the device forms
 * decode_freq's value from the decoder's state for the lookup, the host
 * forms it again and advances `dec`.  The same symbol, decoder state and
 * errors as dtl_decoder_total, dtl_range_decode_freq, dtl_decoder_lookup
 * and dtl_range_decode_advance in turn (DTL_ERR_DEVICE if the two values
 * differ). */
int dtl_decoder_decode(dtl_session *session, size_t row, size_t tail_symbols, dtl_range_decoder *dec,
                       uint32_t *symbol);

/* One step of the decode loop (det-cli main.rs:570-575, 604-626): advance
 * (main.rs:753-771, forward_one_with_workspace of `token` at `pos`) and
 * then decode_symbol of its logits, as dtl_decoder_decode of row 0, with
 * one wait for the device for both.  The forward's errors come first, as
 * from dtl_forward_one. */
int dtl_forward_decode(dtl_session *session, uint32_t token, size_t pos, size_t tail_symbols,
                       dtl_range_decoder *dec, uint32_t *symbol);

/* ---- det-token byte-fallback tokenizer (host) ---------------------------- */
typedef struct dtl_tokenizer dtl_tokenizer;

/* Tokenizer::from_gguf (det-token lib.rs:86-131) for the byte-fallback kind
 * (ByteFallbackTokenizer::from_tokens_and_emit_mask, lib.rs:262-317): the
 * "<0xHH>" vocabulary tokens and the token-type emit mask of the GGUF. */
int dtl_tokenizer_from_gguf(const uint8_t *gguf, size_t len, dtl_tokenizer **out);
void dtl_tokenizer_free(dtl_tokenizer *tok);
/* Number of vocabulary tokens the tokenizer was built from. */
size_t dtl_tokenizer_vocab_len(const dtl_tokenizer *tok);
/* Tokenizer::codec_symbols (lib.rs:150-159): one symbol per input byte, the
 * byte's token or the escape vocab_len + byte.  *n_out receives the count;
 * out may be NULL to query it. */
int dtl_tokenizer_codec_symbols(const dtl_tokenizer *tok, const uint8_t *input, size_t n,
                                size_t vocab_len, uint32_t *out, size_t cap, size_t *n_out);
/* Tokenizer::decode_codec_symbol (lib.rs:182-196): the bytes of one symbol. */
int dtl_tokenizer_decode_symbol(const dtl_tokenizer *tok, uint32_t symbol, size_t vocab_len,
                                uint8_t *out, size_t cap, size_t *n_out);

/* ---- det-cli windowed codec + DTLZ file (host driver over the device) ---- */

#define DTL_DTLZ_FLAG_BYTE_ESCAPES 1u
#define DTL_DTLZ_HEADER_LEN 56u

/* next_window_start (det-cli main.rs:801-808): the start of the codec
 * window for position pos (a rollover starts it overlap tokens back once
 * the window holds n_ctx tokens). */
size_t dtl_codec_next_window_start(size_t pos, size_t window_start, size_t n_ctx, size_t overlap);
/* encode_symbols_with_model (det-cli main.rs:521-551): codec symbols coded
 * window by window (window = the session's n_ctx, overlap tokens replayed
 * at each rollover), each against the logits of the window's last token or
 * uniformly when the window is empty.  *len = payload size; out NULL is a
 * size query (it runs the whole encode), cap < *len returns
 * DTL_ERR_BUFFER_TOO_SMALL.  The session's cache is overwritten. */
int dtl_codec_encode(dtl_session *session, const uint32_t *symbols, size_t n, size_t overlap,
                     int byte_escapes, uint8_t *out, size_t cap, size_t *len);
/* decode_bytes_with_model / decode_tokens_with_model (main.rs:553-632):
 * decodes symbols until piece_len (bytes per symbol, vocab + 256 entries, 0
 * for a symbol that decodes to nothing) sums to byte_len, or max_symbols
 * symbols when piece_len is NULL. */
int dtl_codec_decode(dtl_session *session, const uint8_t *payload, size_t len, size_t overlap,
                     int byte_escapes, const uint8_t *piece_len, size_t byte_len,
                     size_t max_symbols, uint32_t *symbols, size_t *n_out);
/* DtlzHeader::{encode_checked, decode} (det-coder file.rs:1-89): 56 bytes. */
int dtl_dtlz_header_encode(uint16_t flags, const uint8_t model_sha256[32], uint32_t n_ctx,
                           uint32_t overlap, uint64_t orig_len, uint8_t out[56]);
int dtl_dtlz_header_decode(const uint8_t *bytes, size_t len, uint16_t *flags,
                           uint8_t model_sha256[32], uint32_t *n_ctx, uint32_t *overlap,
                           uint64_t *orig_len);
/* compress (det-cli main.rs:431-462): header (model SHA-256, n_ctx, overlap
 * n_ctx/4, byte escapes on, original length) + payload.  n_ctx 0 = the
 * model's context length; max_chunk (0 = 64) positions per device pass.
 * The tokenizer must be the model's (LoadedModel::load, main.rs:932-1000).
 * *out is allocated by the library: release it with dtl_bytes_free. */
int dtl_compress(const dtl_model *model, const dtl_tokenizer *tok, const uint8_t model_sha256[32],
                 const uint8_t *input, size_t n, size_t n_ctx, size_t max_chunk, uint8_t **out,
                 size_t *len);
/* decompress (main.rs:464-512): validates the header before touching the
 * model (model and tok may be NULL for a header that fails), checks the
 * model hash, decodes up to the header's original length, and requires the
 * payload to be the canonical encoding of what it decoded.  *out as for
 * dtl_compress. */
int dtl_decompress(const dtl_model *model, const dtl_tokenizer *tok,
                   const uint8_t model_sha256[32], const uint8_t *file, size_t len,
                   size_t max_chunk, uint8_t **out, size_t *out_len);
/* dtl_decompress in several calls, for a payload too long to decode in one
 * (no counterpart in the reference, whose decompress runs in one call: for
 * callers that bound the time of a call).  The first call passes
 * n_prior = 0 and state_in = NULL; each call decodes up to max_new further
 * symbols after `prior` (every symbol the earlier calls returned, in order)
 * into `symbols` (cap >= max_new), and returns their count and the range
 * decoder's state after them.  The window schedule is replayed from `prior`
 * and the current window's tokens are forwarded again, so the symbols are
 * those of one uninterrupted decode.  When they cover the header's original
 * length, *done = 1 and, after the canonical check over all symbols, *out
 * holds the bytes (as for dtl_decompress). */
int dtl_decompress_part(const dtl_model *model, const dtl_tokenizer *tok,
                        const uint8_t model_sha256[32], const uint8_t *file, size_t len,
                        size_t max_chunk, const uint32_t *prior, size_t n_prior,
                        const dtl_range_decoder_state *state_in, size_t max_new, uint32_t *symbols,
                        size_t cap, size_t *n_new, dtl_range_decoder_state *state_out, int *done,
                        uint8_t **out, size_t *out_len);
/* Releases a buffer returned by dtl_compress / dtl_decompress. */
void dtl_bytes_free(uint8_t *p);

/* ---- det-num / det-quant kernels, exposed for parity checks ------------- */

/* exp_f32 (det-num math.rs:5-7) over n values on the device. */
int dtl_kernel_exp_f32(const float *in, float *out, size_t n);
/* silu_f32 (math.rs:30-34). */
int dtl_kernel_silu_f32(const float *in, float *out, size_t n);
/* exp_f32(max(t, -88)) as softmax_in_place (det-model lib.rs:2361-2388) and
 * the CDF (det-coder cdf.rs:255-300) use it, for t <= 0 (every caller passes
 * t = x - max): the device's restatement for that domain.  A t > 0 is
 * DTL_ERR_INVALID_ARGUMENT. */
int dtl_kernel_exp_clamped_f32(const float *in, float *out, size_t n);
/* No counterpart in the reference: measurement support for the roofline of
 * the f32 chain kernels.  Runs 16 f32 VALU instructions per iteration (eight
 * separately rounded multiplies, eight adds, independent chains, operands in
 * per-lane registers) on eight waves of every SIMD and returns the lanes'
 * operations per second, the issue ceiling of the reference's
 * multiply-then-add arithmetic without fused or packed instructions. */
int dtl_valu_probe(double *lane_ops_per_s);
/* No counterpart in the reference: measurement support for the roofline of
 * the Q4_K chunk GEMMs.  Runs their inner pattern (four f32 16x16x1 MFMA
 * outer products, then 64 ordered adds per lane) on four waves of every SIMD
 * and returns multiply-adds per second: the SIMD runs the MFMAs and the adds
 * one after the other, so this bounds those kernels. */
int dtl_mfp_probe(double *macs_per_s);
/* f16 -> f32 (det-num f16.rs:6-34) on the device. */
int dtl_kernel_f16_to_f32(const uint16_t *in, float *out, size_t n);
/* sqrt and division as used by rmsnorm / softmax / quantisers. */
int dtl_kernel_div_sqrt(const float *a, const float *b, float *quot, float *root, size_t n);
/* quantize_q8a_into / quantize_q8k_into (det-quant lib.rs:67-105) over rows
 * of length n: d[rows*n/32] q[rows*n] (Q8A), d[rows*n/256] q[rows*n] (Q8_K). */
int dtl_kernel_quantize(const float *x, size_t rows, size_t n, float *q8a_d, int8_t *q8a_q,
                        float *q8k_d, int8_t *q8k_q);
/* rmsnorm (det-model lib.rs:2053-2073) of rows x[rows][n]. */
int dtl_kernel_rmsnorm(const float *x, const float *w, float eps, size_t rows, size_t n, float *out);
/* One weight matrix in GGUF encoding (ggml type 0/1/2/8/12/14, rows x cols)
 * against x[T][cols]: out[T][rows] exactly as WeightMatrix::gemv
 * (det-model lib.rs:445-490) computes each token's row dots. */
int dtl_kernel_gemv(int ggml_type, const uint8_t *weights, size_t rows, size_t cols,
                    const float *x, size_t T, float *out);
/* No counterpart in the reference: test support for the Q4_K chunk GEMMs of
 * the encode, every output a dot_q4_k_q8a chain (det-quant lib.rs:281-315)
 * of the Q8A form of x ([T][cols] f32, quantised first as the forward does).
 * mode 0: out0[T][rows0] = W0 x; mode 1: W0 gate and W1 up of the same shape,
 * out0[T][rows0] = silu(W0 x) * (W1 x) (det-model lib.rs:2420-2434); mode 2:
 * W0 and W1 (wq, wk) in one launch, out0[T][rows0] and out1[T][rows1].
 * overlapped != 0 runs the kernels the pipelined encode runs with other
 * chunks in flight, 0 those of a launch alone.  Needs T >= 16 and cols a
 * multiple of 256 (DTL_ERR_SHAPE otherwise). */
int dtl_kernel_q4k_chunk(int mode, int overlapped, const uint8_t *w0, size_t rows0, const uint8_t *w1,
                         size_t rows1, size_t cols, const float *x, size_t T, float *out0, float *out1);
/* RopeTables::llama (det-model lib.rs:813-847) computed on the device. */
int dtl_kernel_rope_table(float rope_freq_base, size_t rope_dim, size_t positions, float *cos_out,
                          float *sin_out);

#ifdef __cplusplus
}
#endif
#endif
