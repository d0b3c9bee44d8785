/*
 * detref windowed model codec and byte-fallback symbols — TEST
 * INFRASTRUCTURE ONLY (the oracle).
 *
 * Restates, token by token as the reference runs it:
 *   canonical_byte_fallback_token            det-token lib.rs:841-847
 *   ByteFallbackTokenizer::from_tokens_and_emit_mask + from_pairs
 *                                            det-token lib.rs:258-298
 *   Tokenizer::codec_symbols (byte fallback) det-token lib.rs:150-180, 306-312
 *   Tokenizer::decode_codec_symbol           det-token lib.rs:182-196, 314-325
 *   encode_symbols_with_model                det-cli main.rs:521-551
 *   decode_bytes_with_model                  det-cli main.rs:573-632
 *   WindowedModelState (sync/replay/symbol_range/decode_symbol/advance)
 *                                            det-cli main.rs:634-799
 *   next_window_start                        det-cli main.rs:801-808
 *   validate_window                          det-cli main.rs:810-825
 */
#include <stdlib.h>
#include <string.h>

#include "detref.h"

#define ESCAPES 256u

/* canonical_byte_fallback_token: "<0x" + two bytes + ">", parsed by
 * u8::from_str_radix(_, 16), which takes an optional leading '+'. */
static int hexval(char c) {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
}

int ref_canonical_byte_token(const char *tok, size_t len) {
    if (len != 6 || memcmp(tok, "<0x", 3) != 0 || tok[5] != '>') return -1;
    if (tok[3] == '+') return hexval(tok[4]);
    int a = hexval(tok[3]), b = hexval(tok[4]);
    return a < 0 || b < 0 ? -1 : a * 16 + b;
}

/* from_tokens_and_emit_mask: tokens given as a concatenation with offsets
 * (off[i]..off[i+1]); emit may be NULL (every token emittable).
 * byte_to_token[b]: emittable token of byte b or -1; token_to_byte[i]: byte
 * of token i or -1.  Returns 72 duplicate byte, 65 incomplete coverage. */
int ref_byte_fallback_tables(const char *text, const size_t *off, size_t n, const uint8_t *emit,
                             int32_t byte_to_token[256], int16_t *token_to_byte) {
    int seen[256] = {0};
    for (int b = 0; b < 256; b++) byte_to_token[b] = -1;
    for (size_t i = 0; i < n; i++) {
        token_to_byte[i] = -1;
        int b = ref_canonical_byte_token(text + off[i], off[i + 1] - off[i]);
        if (b < 0) continue;
        if (seen[b]) return 72;
        seen[b] = 1;
        token_to_byte[i] = (int16_t)b;
        if (!emit || emit[i]) byte_to_token[b] = (int32_t)i;
    }
    for (int b = 0; b < 256; b++)
        if (!seen[b]) return 65;
    return REF_OK;
}

/* codec_symbols for the byte-fallback kind: the byte's token, else the
 * escape vocab_len + byte. */
void ref_codec_symbols(const int32_t byte_to_token[256], const uint8_t *in, size_t n,
                       size_t vocab_len, uint32_t *out) {
    for (size_t i = 0; i < n; i++) {
        int32_t t = byte_to_token[in[i]];
        out[i] = t >= 0 ? (uint32_t)t : (uint32_t)(vocab_len + in[i]);
    }
}

size_t ref_next_window_start(size_t pos, size_t window_start, size_t n_ctx, size_t overlap) {
    size_t used = pos > window_start ? pos - window_start : 0;
    if (used >= n_ctx) return pos > overlap ? pos - overlap : 0;
    return window_start;
}

/* WindowedModelState over one oracle session. */
typedef struct {
    const ref_model *m;
    ref_session *s;
    size_t n_ctx, window_start, context_len, vocab, tail;
    float *logits;
} win_state;

static int state_init(win_state *w, const ref_model *m, size_t n_ctx, int escapes) {
    int64_t cfg[16];
    ref_model_config(m, cfg);
    memset(w, 0, sizeof *w);
    w->m = m;
    w->n_ctx = n_ctx;
    w->vocab = (size_t)cfg[9];
    w->tail = escapes ? ESCAPES : 0;
    int st = REF_OK;
    w->s = ref_session_new(m, n_ctx, &st);
    if (!w->s) return st;
    w->logits = calloc(w->vocab, sizeof(float));
    return REF_OK;
}

static void state_free(win_state *w) {
    ref_session_free(w->s);
    free(w->logits);
}

static int state_advance(win_state *w, uint32_t token) {
    if (w->context_len >= w->n_ctx) return REF_ERR_SHAPE;
    int st = ref_forward_one(w->s, token, w->context_len, w->logits);
    if (st) return st;
    w->context_len++;
    return REF_OK;
}

static int state_sync(win_state *w, const uint32_t *tokens, size_t pos, size_t overlap) {
    size_t next = ref_next_window_start(pos, w->window_start, w->n_ctx, overlap);
    if (next == w->window_start) return REF_OK;
    /* replay: fresh cache, zero logits, the window's tokens re-forwarded */
    ref_session_reset(w->s);
    memset(w->logits, 0, w->vocab * sizeof(float));
    w->window_start = next;
    w->context_len = 0;
    for (size_t p = next; p < pos; p++) {
        int st = state_advance(w, tokens[p]);
        if (st) return st;
    }
    return REF_OK;
}

static int validate_window(const ref_model *m, size_t n_ctx, size_t overlap) {
    int64_t cfg[16];
    ref_model_config(m, cfg);
    if (n_ctx == 0 || n_ctx > (size_t)cfg[8] || overlap >= n_ctx) return REF_ERR_SHAPE;
    return REF_OK;
}

/* encode_symbols_with_model: returns the payload length through *len (the
 * bytes go to out when cap allows). */
int ref_codec_encode(const ref_model *m, const uint32_t *symbols, size_t n, size_t n_ctx,
                     size_t overlap, int escapes, uint8_t *out, size_t cap, size_t *len) {
    int st = validate_window(m, n_ctx, overlap);
    if (st) return st;
    win_state w;
    if ((st = state_init(&w, m, n_ctx, escapes))) return st;
    uint32_t *context = malloc((n + 1) * sizeof(uint32_t));
    size_t ctx_n = 0;
    ref_range_encoder *enc = ref_range_encoder_new();
    for (size_t k = 0; k < n && st == REF_OK; k++) {
        const uint32_t sym = symbols[k];
        if ((st = state_sync(&w, context, ctx_n, overlap))) break;
        uint64_t cum, total;
        uint32_t freq;
        if (w.context_len == 0)
            st = ref_uniform_symbol_range(sym, w.vocab + w.tail, &cum, &freq, &total);
        else
            st = ref_symbol_range(w.logits, w.vocab, sym, w.tail, &cum, &freq, &total);
        if (st) break;
        if ((st = ref_range_encode(enc, cum, freq, total))) break;
        if (escapes && sym >= w.vocab) continue;
        if (sym >= w.vocab) { st = REF_ERR_CDF_SYMBOL_OUT_OF_RANGE; break; }
        context[ctx_n++] = sym;
        st = state_advance(&w, sym);
    }
    if (st == REF_OK) *len = ref_range_encoder_finish(enc, out, cap);
    ref_range_encoder_free(enc);
    free(context);
    state_free(&w);
    return st;
}

/* decode_bytes_with_model with byte-fallback pieces (token_to_byte; escapes
 * decode to their byte): decodes until byte_len bytes; symbols[] needs
 * byte_len entries.  *n_out = symbols decoded. */
int ref_codec_decode(const ref_model *m, const int16_t *token_to_byte, const uint8_t *payload,
                     size_t plen, size_t byte_len, size_t n_ctx, size_t overlap, int escapes,
                     uint32_t *symbols, uint8_t *bytes, size_t *n_out) {
    *n_out = 0;
    int st = validate_window(m, n_ctx, overlap);
    if (st) return st;
    win_state w;
    if ((st = state_init(&w, m, n_ctx, escapes))) return st;
    ref_range_decoder *dec = ref_range_decoder_new(payload, plen, &st);
    if (!dec) { state_free(&w); return st; }
    uint32_t *context = malloc((byte_len + 1) * sizeof(uint32_t));
    size_t ctx_n = 0, nb = 0, ns = 0;
    while (nb < byte_len && st == REF_OK) {
        if ((st = state_sync(&w, context, ctx_n, overlap))) break;
        uint64_t value, cum, total, sym;
        uint32_t freq;
        if (w.context_len == 0) {
            total = w.vocab + w.tail;
            if ((st = ref_range_decode_freq(dec, total, &value))) break;
            sym = value; /* uniform: symbol v covers [v, v + 1) */
            if ((st = ref_range_decode_advance(dec, value, 1, total))) break;
        } else {
            if ((st = ref_decoder_total(w.logits, w.vocab, w.tail, &total))) break;
            if ((st = ref_range_decode_freq(dec, total, &value))) break;
            if ((st = ref_decoder_lookup(w.logits, w.vocab, w.tail, value, &sym, &cum, &freq,
                                         &total)))
                break;
            if ((st = ref_range_decode_advance(dec, cum, freq, total))) break;
        }
        int byte;
        if (sym < w.vocab) byte = token_to_byte[sym];
        else byte = sym < w.vocab + ESCAPES ? (int)(sym - w.vocab) : -1;
        if (byte < 0) { st = 61; break; } /* TokenError::InvalidToken */
        bytes[nb++] = (uint8_t)byte;
        symbols[ns++] = (uint32_t)sym;
        if (escapes && sym >= w.vocab) continue;
        context[ctx_n++] = (uint32_t)sym;
        st = state_advance(&w, (uint32_t)sym);
    }
    *n_out = ns;
    free(context);
    ref_range_decoder_free(dec);
    state_free(&w);
    return st;
}
