// Windowed model codec and the DTLZ file (crates/det-cli/src/main.rs:431-808
// and crates/det-coder/src/file.rs of mii443/detllm), on top of this
// library's session, CDF and range-coder entry points.
//
// The reference advances the model one token at a time.  Encoding knows
// every token in advance, so here each window's forwards run as chunks of
// positions on the device and the symbol ranges of all symbols coded against
// a chunk's rows are computed in one call; the (cum, freq, total) triplets
// are then range-coded in symbol order.  Decoding is sequential as in the
// reference: one forward per decoded token.
#include <algorithm>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <new>
#include <vector>

#include "../../include/detllm.h"

namespace {

constexpr size_t kEscapes = 256;  // BYTE_ESCAPE_SYMBOLS

struct Info {
  size_t n_ctx, max_chunk, vocab;
};

int session_info(dtl_session* s, Info* in) {
  return dtl_session_get_info(s, &in->n_ctx, &in->max_chunk, &in->vocab);
}

// validate_window (main.rs:810-825) against the session's window.
int validate_window(size_t n_ctx, size_t overlap) {
  if (n_ctx == 0) return DTL_ERR_FILE_INVALID_CONTEXT;
  if (overlap >= n_ctx) return DTL_ERR_FILE_INVALID_OVERLAP;
  return DTL_OK;
}


struct Range3 {
  uint64_t cum, total;
  uint32_t freq;
};

// encode_symbols_with_model (main.rs:521-551).
int encode_payload(dtl_session* s, const uint32_t* symbols, size_t n, size_t overlap,
                   int byte_escapes, std::vector<uint8_t>* payload) {
  Info in;
  int st = session_info(s, &in);
  if (st) return st;
  if ((st = validate_window(in.n_ctx, overlap))) return st;
  const size_t V = in.vocab, tail = byte_escapes ? kEscapes : 0;
  // Plan: the window each symbol falls in and the window position of the
  // forward whose logits code it (SIZE_MAX: uniform, the window is empty).
  struct Window {
    size_t start;                // first context token of the window
    std::vector<uint32_t> toks;  // the window's forwards, in order
  };
  std::vector<Window> windows;
  std::vector<size_t> sym_window(n), sym_row(n);
  std::vector<uint32_t> context;
  size_t window_start = 0;
  windows.push_back({0, {}});
  for (size_t k = 0; k < n; k++) {
    const uint32_t sym = symbols[k];
    if (sym >= V + tail) return DTL_ERR_CDF_SYMBOL_OUT_OF_RANGE;
    const size_t pos = context.size();
    const size_t next = dtl_codec_next_window_start(pos, window_start, in.n_ctx, overlap);
    if (next != window_start) {
      window_start = next;
      windows.push_back({next, std::vector<uint32_t>(context.begin() + next, context.end())});
    }
    Window& w = windows.back();
    sym_window[k] = windows.size() - 1;
    sym_row[k] = w.toks.empty() ? SIZE_MAX : w.toks.size() - 1;
    if (sym < V) {
      context.push_back(sym);
      w.toks.push_back(sym);
    }
  }
  // Device work: each window from a fresh cache; its forwards and the
  // ranges of the symbols coded against them come from one pipelined call.
  std::vector<Range3> ranges(n);
  std::vector<size_t> by_window_start(windows.size() + 1, 0);
  {
    // symbols are ordered by window already: find each window's first symbol
    size_t k = 0;
    for (size_t w = 0; w < windows.size(); w++) {
      by_window_start[w] = k;
      while (k < n && sym_window[k] == w) k++;
    }
    by_window_start[windows.size()] = n;
  }
  std::vector<uint32_t> rows, syms;
  std::vector<uint64_t> cum, total;
  std::vector<uint32_t> freq;
  for (size_t w = 0; w < windows.size(); w++) {
    const Window& win = windows[w];
    const size_t k0 = by_window_start[w], k1 = by_window_start[w + 1];
    // uniform symbols (empty window)
    for (size_t k = k0; k < k1; k++) {
      if (sym_row[k] != SIZE_MAX) continue;
      uint64_t c, t;
      uint32_t f;
      if ((st = dtl_uniform_symbol_range(symbols[k], V + tail, &c, &f, &t))) return st;
      ranges[k] = {c, t, f};
    }
    rows.clear();
    syms.clear();
    for (size_t k = k0; k < k1; k++) {
      if (sym_row[k] == SIZE_MAX) continue;
      rows.push_back((uint32_t)sym_row[k]);
      syms.push_back(symbols[k]);
    }
    if (rows.empty()) continue;
    if ((st = dtl_session_reset(s))) return st;
    // Tokens after the last coded row only advance a state the next window
    // discards, so the forwards stop there.
    cum.resize(rows.size());
    freq.resize(rows.size());
    total.resize(rows.size());
    if ((st = dtl_forward_ranges(s, win.toks.data(), (size_t)rows.back() + 1, 0, rows.size(),
                                 rows.data(), syms.data(), tail, cum.data(), freq.data(),
                                 total.data())))
      return st;
    size_t j = 0;
    for (size_t k = k0; k < k1; k++) {
      if (sym_row[k] == SIZE_MAX) continue;
      ranges[k] = {cum[j], total[j], freq[j]};
      j++;
    }
  }
  dtl_range_encoder* enc = nullptr;
  if ((st = dtl_range_encoder_new(&enc))) return st;
  for (size_t k = 0; k < n && st == DTL_OK; k++)
    st = dtl_range_encode(enc, ranges[k].cum, ranges[k].freq, ranges[k].total);
  size_t len = 0;
  if (st == DTL_OK) st = dtl_range_encoder_finish(enc, nullptr, 0, &len);
  if (st == DTL_OK) {
    payload->resize(len);
    st = dtl_range_encoder_finish(enc, payload->data(), len, &len);
  }
  dtl_range_encoder_free(enc);
  return st;
}

// decode_bytes_with_model (main.rs:573-632) over WindowedModelState
// (main.rs:634-799), symbols appended to *out.
//
// A decode may continue an earlier one (dtl_decompress_part): `prior` holds
// the symbols decoded so far and `resume` the range decoder's state after
// them.  The window schedule and the context are replayed from `prior`, and
// the current window's tokens are forwarded again, as at a window rollover,
// so the session then holds the same rows as the uninterrupted decode would.
// With `final_state` the decoder's state after the last symbol is returned.
int decode_symbols(dtl_session* s, const uint8_t* payload, size_t plen, size_t overlap,
                   int byte_escapes, const uint8_t* piece_len, size_t byte_len, size_t max_symbols,
                   std::vector<uint32_t>* out, const uint32_t* prior = nullptr, size_t n_prior = 0,
                   const dtl_range_decoder_state* resume = nullptr,
                   dtl_range_decoder_state* final_state = nullptr) {
  Info in;
  int st = session_info(s, &in);
  if (st) return st;
  if ((st = validate_window(in.n_ctx, overlap))) return st;
  const size_t V = in.vocab, tail = byte_escapes ? kEscapes : 0;
  if ((n_prior != 0) != (resume != nullptr)) return DTL_ERR_INVALID_ARGUMENT;
  dtl_range_decoder* dec = nullptr;
  st = resume ? dtl_range_decoder_from_snapshot(payload, plen, resume, &dec)
              : dtl_range_decoder_new(payload, plen, &dec);
  if (st) return st;
  std::vector<uint32_t> context;
  size_t window_start = 0, context_len = 0, last_row = 0, bytes = 0;
  // A decoded token whose forward (advance) is enqueued with the next
  // symbol's decode, one wait for both; a window replay forwards it instead.
  bool pend = false;
  uint32_t pend_tok = 0;
  size_t pend_pos = 0;
  if ((st = dtl_session_reset(s))) goto done;
  for (size_t k = 0; k < n_prior; k++) {
    const uint32_t sym = prior[k];
    if (sym >= V + tail) {
      st = DTL_ERR_INVALID_ARGUMENT;
      goto done;
    }
    const size_t pos = context.size();
    window_start = dtl_codec_next_window_start(pos, window_start, in.n_ctx, overlap);
    if (piece_len) bytes += piece_len[sym];
    if (sym < V) context.push_back(sym);
  }
  if (n_prior) {
    // the rows of the current window, as a rollover replays them
    const size_t pos = context.size();
    window_start = dtl_codec_next_window_start(pos, window_start, in.n_ctx, overlap);
    for (size_t p0 = window_start; p0 < pos; p0 += in.max_chunk) {
      const size_t T = std::min(in.max_chunk, pos - p0);
      if ((st = dtl_forward_chunk(s, context.data() + p0, T, p0 - window_start, nullptr))) goto done;
      context_len += T;
      last_row = T - 1;
    }
  }
  while (out->size() < max_symbols && (piece_len ? bytes < byte_len : true)) {
    const size_t pos = context.size();
    const size_t next = dtl_codec_next_window_start(pos, window_start, in.n_ctx, overlap);
    if (next != window_start) {
      // replay (main.rs:690-701): fresh cache, the window's tokens re-forwarded
      window_start = next;
      context_len = 0;
      pend = false;
      if ((st = dtl_session_reset(s))) goto done;
      for (size_t p0 = next; p0 < pos; p0 += in.max_chunk) {
        const size_t T = std::min(in.max_chunk, pos - p0);
        if ((st = dtl_forward_chunk(s, context.data() + p0, T, p0 - next, nullptr))) goto done;
        context_len += T;
        last_row = T - 1;
      }
    }
    uint32_t sym;
    uint64_t value;
    if (context_len == 0) {
      // uniform_cdf[_with_byte_escapes]: symbol v covers [v, v + 1)
      const uint64_t total = V + tail;
      if ((st = dtl_range_decode_freq(dec, total, &value))) goto done;
      sym = (uint32_t)value;
      if ((st = dtl_range_decode_advance(dec, value, 1, total))) goto done;
    } else if (pend) {
      // advance(token) + decode_symbol (main.rs:570-575)
      pend = false;
      if ((st = dtl_forward_decode(s, pend_tok, pend_pos, tail, dec, &sym))) goto done;
      last_row = 0;
    } else {
      // decode_symbol after a window replay or a byte escape
      if ((st = dtl_decoder_decode(s, last_row, tail, dec, &sym))) goto done;
    }
    if (!byte_escapes && sym >= V) {
      st = DTL_ERR_CODEC_ESCAPE_IN_TOKEN_STREAM;
      goto done;
    }
    if (piece_len) {
      if (piece_len[sym] == 0) {  // "decoded symbol produced no bytes"
        st = DTL_ERR_TOKEN_INVALID_TOKEN;
        goto done;
      }
      bytes += piece_len[sym];
    }
    out->push_back(sym);
    if (sym < V) {
      if (context_len >= in.n_ctx) {  // "context window invariant violated"
        st = DTL_ERR_SHAPE;
        goto done;
      }
      pend = true;
      pend_tok = sym;
      pend_pos = context_len;
      context.push_back(sym);
      context_len++;
    }
  }
  // the last token's advance, whose decode never comes
  if (pend) st = dtl_forward_one(s, pend_tok, pend_pos, nullptr);
done:
  if (st == DTL_OK && final_state) st = dtl_range_decoder_snapshot(dec, final_state);
  dtl_range_decoder_free(dec);
  return st;
}

}  // namespace

extern "C" {

// next_window_start (main.rs:801-808): a new window starts overlap tokens
// back once the current one holds n_ctx tokens.
size_t dtl_codec_next_window_start(size_t pos, size_t window_start, size_t n_ctx, size_t overlap) {
  return pos - std::min(pos, window_start) >= n_ctx ? pos - std::min(pos, overlap) : window_start;
}

int dtl_codec_encode(dtl_session* s, const uint32_t* symbols, size_t n, size_t overlap,
                     int byte_escapes, uint8_t* out, size_t cap, size_t* len) {
  if (!s || (!symbols && n) || !len) return DTL_ERR_INVALID_ARGUMENT;
  try {
    std::vector<uint8_t> payload;
    const int st = encode_payload(s, symbols, n, overlap, byte_escapes, &payload);
    if (st) return st;
    *len = payload.size();
    if (!out) return DTL_OK;
    if (cap < payload.size()) return DTL_ERR_BUFFER_TOO_SMALL;
    if (!payload.empty()) std::memcpy(out, payload.data(), payload.size());
    return DTL_OK;
  } catch (const std::bad_alloc&) {
    return DTL_ERR_OUT_OF_MEMORY;
  }
}

// decode_bytes_with_model / decode_tokens_with_model (main.rs:553-632) and
// WindowedModelState (main.rs:634-799): one forward per decoded token.
// Stops after max_symbols symbols, or once piece_len (when given) sums to
// byte_len.
int dtl_codec_decode(dtl_session* s, const uint8_t* payload, size_t plen, size_t overlap,
                     int byte_escapes, const uint8_t* piece_len, size_t byte_len,
                     size_t max_symbols, uint32_t* symbols, size_t* n_out) {
  if (!s || (!payload && plen) || (!symbols && max_symbols) || !n_out)
    return DTL_ERR_INVALID_ARGUMENT;
  *n_out = 0;
  try {
    std::vector<uint32_t> out;
    out.reserve(std::min<size_t>(max_symbols, 1 << 16));
    const int st = decode_symbols(s, payload, plen, overlap, byte_escapes, piece_len, byte_len,
                                  max_symbols, &out);
    if (!out.empty()) std::memcpy(symbols, out.data(), out.size() * 4);
    *n_out = out.size();
    return st;
  } catch (const std::bad_alloc&) {
    return DTL_ERR_OUT_OF_MEMORY;
  }
}

// DtlzHeader::{encode, decode, validate} (det-coder file.rs:1-89).
int dtl_dtlz_header_encode(uint16_t flags, const uint8_t model_sha256[32], uint32_t n_ctx,
                           uint32_t overlap, uint64_t orig_len, uint8_t out[56]) {
  if (!model_sha256 || !out) return DTL_ERR_INVALID_ARGUMENT;
  if (flags & ~(uint16_t)DTL_DTLZ_FLAG_BYTE_ESCAPES) return DTL_ERR_FILE_UNSUPPORTED_FLAGS;
  if (n_ctx == 0) return DTL_ERR_FILE_INVALID_CONTEXT;
  if (overlap >= n_ctx) return DTL_ERR_FILE_INVALID_OVERLAP;
  const uint16_t version = 1;
  std::memcpy(out, "DTLZ", 4);
  std::memcpy(out + 4, &version, 2);
  std::memcpy(out + 6, &flags, 2);
  std::memcpy(out + 8, model_sha256, 32);
  std::memcpy(out + 40, &n_ctx, 4);
  std::memcpy(out + 44, &overlap, 4);
  std::memcpy(out + 48, &orig_len, 8);
  return DTL_OK;
}

int dtl_dtlz_header_decode(const uint8_t* bytes, size_t len, uint16_t* flags,
                           uint8_t model_sha256[32], uint32_t* n_ctx, uint32_t* overlap,
                           uint64_t* orig_len) {
  if (!bytes && len) return DTL_ERR_INVALID_ARGUMENT;
  if (len < 56) return DTL_ERR_FILE_TOO_SHORT;
  if (std::memcmp(bytes, "DTLZ", 4) != 0) return DTL_ERR_FILE_BAD_MAGIC;
  uint16_t version, f;
  std::memcpy(&version, bytes + 4, 2);
  if (version != 1) return DTL_ERR_FILE_UNSUPPORTED_VERSION;
  std::memcpy(&f, bytes + 6, 2);
  if (f & ~(uint16_t)DTL_DTLZ_FLAG_BYTE_ESCAPES) return DTL_ERR_FILE_UNSUPPORTED_FLAGS;
  uint32_t nc, ov;
  uint64_t ol;
  std::memcpy(&nc, bytes + 40, 4);
  std::memcpy(&ov, bytes + 44, 4);
  std::memcpy(&ol, bytes + 48, 8);
  if (nc == 0) return DTL_ERR_FILE_INVALID_CONTEXT;
  if (ov >= nc) return DTL_ERR_FILE_INVALID_OVERLAP;
  if (flags) *flags = f;
  if (model_sha256) std::memcpy(model_sha256, bytes + 8, 32);
  if (n_ctx) *n_ctx = nc;
  if (overlap) *overlap = ov;
  if (orig_len) *orig_len = ol;
  return DTL_OK;
}

// Library-owned result buffer of dtl_compress / dtl_decompress.
static int hand_out(const std::vector<uint8_t>& v, uint8_t** out, size_t* len) {
  uint8_t* p = static_cast<uint8_t*>(std::malloc(v.empty() ? 1 : v.size()));
  if (!p) return DTL_ERR_OUT_OF_MEMORY;
  if (!v.empty()) std::memcpy(p, v.data(), v.size());
  *out = p;
  *len = v.size();
  return DTL_OK;
}

void dtl_bytes_free(uint8_t* p) { std::free(p); }

// LoadedModel::load checks (main.rs:932-1000): the tokenizer's vocabulary is
// the model's, and vocab + 256 escapes fit the CDF symbol limit.
static int check_codec_model(const dtl_model_config& cfg, const dtl_tokenizer* tok) {
  if (dtl_tokenizer_vocab_len(tok) != cfg.vocab) return DTL_ERR_CODEC_VOCAB_MISMATCH;
  if (cfg.vocab + kEscapes > (1u << 18)) return DTL_ERR_CDF_TOO_MANY_SYMBOLS;
  return DTL_OK;
}

// compress (main.rs:431-462): byte-fallback codec symbols, window n_ctx,
// overlap n_ctx / 4, byte escapes on; header + payload.
int dtl_compress(const dtl_model* model, const dtl_tokenizer* tok, const uint8_t model_sha256[32],
                 const uint8_t* input, size_t n, size_t n_ctx, size_t max_chunk, uint8_t** out,
                 size_t* len) {
  if (!model || !tok || !model_sha256 || (!input && n) || !out || !len)
    return DTL_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  *len = 0;
  try {
    dtl_model_config cfg;
    int st = dtl_model_get_config(model, &cfg);
    if (st) return st;
    if ((st = check_codec_model(cfg, tok))) return st;
    if (n_ctx == 0) n_ctx = cfg.context_length;
    // validate_window (main.rs:810-825) with overlap n_ctx / 4
    if (n_ctx == 0 || n_ctx > cfg.context_length || n_ctx > 0xffffffffull)
      return DTL_ERR_FILE_INVALID_CONTEXT;
    const size_t overlap = n_ctx / 4;
    std::vector<uint32_t> symbols(n);
    size_t ns = 0;
    if ((st = dtl_tokenizer_codec_symbols(tok, input, n, cfg.vocab, symbols.data(), n, &ns)))
      return st;
    dtl_session* s = nullptr;
    if ((st = dtl_session_new(model, n_ctx, max_chunk ? max_chunk : 64, &s))) return st;
    std::vector<uint8_t> file(DTL_DTLZ_HEADER_LEN);
    std::vector<uint8_t> payload;
    st = encode_payload(s, symbols.data(), ns, overlap, 1, &payload);
    dtl_session_free(s);
    if (st) return st;
    if ((st = dtl_dtlz_header_encode(DTL_DTLZ_FLAG_BYTE_ESCAPES, model_sha256, (uint32_t)n_ctx,
                                     (uint32_t)overlap, (uint64_t)n, file.data())))
      return st;
    file.insert(file.end(), payload.begin(), payload.end());
    return hand_out(file, out, len);
  } catch (const std::bad_alloc&) {
    return DTL_ERR_OUT_OF_MEMORY;
  }
}

// decompress (main.rs:464-512): header first (before any model work), model
// hash check, window check, decode to the original length, then the
// canonical re-encode check.
namespace {
// The header checks and symbol tables shared by dtl_decompress and
// dtl_decompress_part.
struct DecompressPlan {
  uint32_t n_ctx = 0, overlap = 0;
  uint64_t orig_len = 0;
  int escapes = 0;
  std::vector<uint8_t> piece, one;
};

int plan_decompress(const dtl_model* model, const dtl_tokenizer* tok, const uint8_t model_sha256[32],
                    const uint8_t* file, size_t len, DecompressPlan* P) {
  uint16_t flags;
  uint8_t sha[32];
  int st = dtl_dtlz_header_decode(file, len, &flags, sha, &P->n_ctx, &P->overlap, &P->orig_len);
  if (st) return st;
  if (!model || !tok || !model_sha256) return DTL_ERR_INVALID_ARGUMENT;
  dtl_model_config cfg;
  if ((st = dtl_model_get_config(model, &cfg))) return st;
  if ((st = check_codec_model(cfg, tok))) return st;
  if (std::memcmp(sha, model_sha256, 32) != 0) return DTL_ERR_CODEC_MODEL_MISMATCH;
  if (P->n_ctx > cfg.context_length) return DTL_ERR_FILE_INVALID_CONTEXT;
  P->escapes = (flags & DTL_DTLZ_FLAG_BYTE_ESCAPES) ? 1 : 0;
  const size_t V = cfg.vocab;
  // bytes of each symbol (0: decodes to nothing) and, for the byte-fallback
  // kind, the one byte itself
  P->piece.assign(V + kEscapes, 0);
  P->one.assign(V + kEscapes, 0);
  for (size_t sym = 0; sym < V + kEscapes; sym++) {
    size_t nb = 0;
    uint8_t b;
    if (dtl_tokenizer_decode_symbol(tok, (uint32_t)sym, V, &b, 1, &nb) == DTL_OK && nb == 1) {
      P->piece[sym] = 1;
      P->one[sym] = b;
    }
  }
  return DTL_OK;
}

// The canonical check (the payload re-encoded from the symbols must equal
// the file's) and the decompressed bytes.
int finish_decompress(dtl_session* s, const DecompressPlan& P, const uint8_t* file, size_t len,
                      const std::vector<uint32_t>& symbols, uint8_t** out, size_t* out_len) {
  std::vector<uint8_t> again;
  int st = encode_payload(s, symbols.data(), symbols.size(), P.overlap, P.escapes, &again);
  if (st) return st;
  if (again.size() != len - DTL_DTLZ_HEADER_LEN ||
      std::memcmp(again.data(), file + DTL_DTLZ_HEADER_LEN, again.size()) != 0)
    return DTL_ERR_CODEC_NOT_CANONICAL;
  std::vector<uint8_t> bytes;
  bytes.reserve(symbols.size());
  for (uint32_t sym : symbols) bytes.push_back(P.one[sym]);
  bytes.resize((size_t)P.orig_len);
  return hand_out(bytes, out, out_len);
}
}  // namespace

int dtl_decompress(const dtl_model* model, const dtl_tokenizer* tok,
                   const uint8_t model_sha256[32], const uint8_t* file, size_t len,
                   size_t max_chunk, uint8_t** out, size_t* out_len) {
  if ((!file && len) || !out || !out_len) return DTL_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  *out_len = 0;
  try {
    DecompressPlan P;
    int st = plan_decompress(model, tok, model_sha256, file, len, &P);
    if (st) return st;
    dtl_session* s = nullptr;
    if ((st = dtl_session_new(model, P.n_ctx, max_chunk ? max_chunk : 64, &s))) return st;
    std::vector<uint32_t> symbols;
    symbols.reserve((size_t)std::min<uint64_t>(P.orig_len, 8192));
    // orig_len beyond what the payload codes ends in a range-coder error
    // (UnexpectedEof), as in the reference
    st = decode_symbols(s, file + DTL_DTLZ_HEADER_LEN, len - DTL_DTLZ_HEADER_LEN, P.overlap, P.escapes,
                        P.piece.data(), P.orig_len > SIZE_MAX ? SIZE_MAX : (size_t)P.orig_len, SIZE_MAX,
                        &symbols);
    if (st == DTL_OK) st = finish_decompress(s, P, file, len, symbols, out, out_len);
    dtl_session_free(s);
    return st;
  } catch (const std::bad_alloc&) {
    return DTL_ERR_OUT_OF_MEMORY;
  }
}

int dtl_decompress_part(const dtl_model* model, const dtl_tokenizer* tok,
                        const uint8_t model_sha256[32], const uint8_t* file, size_t len,
                        size_t max_chunk, const uint32_t* prior, size_t n_prior,
                        const dtl_range_decoder_state* state_in, size_t max_new, uint32_t* symbols,
                        size_t cap, size_t* n_new, dtl_range_decoder_state* state_out, int* done,
                        uint8_t** out, size_t* out_len) {
  if ((!file && len) || (!prior && n_prior) || (!symbols && cap) || !n_new || !state_out || !done ||
      !out || !out_len || cap < max_new || (n_prior != 0) != (state_in != nullptr))
    return DTL_ERR_INVALID_ARGUMENT;
  *n_new = 0;
  *done = 0;
  *out = nullptr;
  *out_len = 0;
  try {
    DecompressPlan P;
    int st = plan_decompress(model, tok, model_sha256, file, len, &P);
    if (st) return st;
    dtl_session* s = nullptr;
    if ((st = dtl_session_new(model, P.n_ctx, max_chunk ? max_chunk : 64, &s))) return st;
    std::vector<uint32_t> fresh;
    fresh.reserve(std::min<size_t>(max_new, 1 << 16));
    const size_t byte_len = P.orig_len > SIZE_MAX ? SIZE_MAX : (size_t)P.orig_len;
    st = decode_symbols(s, file + DTL_DTLZ_HEADER_LEN, len - DTL_DTLZ_HEADER_LEN, P.overlap, P.escapes,
                        P.piece.data(), byte_len, max_new, &fresh, prior, n_prior, state_in, state_out);
    if (st == DTL_OK) {
      if (!fresh.empty()) std::memcpy(symbols, fresh.data(), fresh.size() * 4);
      *n_new = fresh.size();
      size_t bytes = 0;
      for (size_t k = 0; k < n_prior; k++) bytes += P.piece[prior[k]];
      for (uint32_t sym : fresh) bytes += P.piece[sym];
      if (bytes >= byte_len) {
        std::vector<uint32_t> all(prior, prior + n_prior);
        all.insert(all.end(), fresh.begin(), fresh.end());
        st = finish_decompress(s, P, file, len, all, out, out_len);
        if (st == DTL_OK) *done = 1;
      }
    }
    dtl_session_free(s);
    return st;
  } catch (const std::bad_alloc&) {
    return DTL_ERR_OUT_OF_MEMORY;
  }
}

}  // extern "C"
