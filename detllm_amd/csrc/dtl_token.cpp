// Byte-fallback tokenizer and codec symbol stream (crates/det-token of
// mii443/detllm, lib.rs:85-132, 150-209, 228-326, 619-710, 841-847): every
// byte with an emittable "<0xHH>" vocabulary token becomes that token, every
// other byte the escape symbol vocab + byte.  The GGUF vocabulary chooses
// the tokenizer kind as Tokenizer::from_gguf does; only the byte-fallback
// kind (no tokenizer model, merges or scores) is implemented here.
#include <cstring>
#include <memory>
#include <string_view>
#include <vector>

#include "../../include/detllm.h"
#include "dtl_gguf.h"

using namespace dtl;

struct dtl_tokenizer {
  int32_t byte_to_token[256];          // emittable token of each byte, or -1
  std::vector<int16_t> token_to_byte;  // byte of each byte-fallback token, or -1
};

namespace {

// canonical_byte_fallback_token (lib.rs:841-847): "<0x" + exactly two
// characters + ">", parsed as an unsigned base-16 integer (a leading '+' is
// accepted, as u8::from_str_radix accepts it).
int canonical_byte(std::string_view t) {
  if (t.size() != 6 || t.substr(0, 3) != "<0x" || t[5] != '>') return -1;
  auto hexval = [](char c) -> int {
    if (c >= '0' && c <= '9') return c - '0';
    if (c >= 'a' && c <= 'f') return c - 'a' + 10;
    if (c >= 'A' && c <= 'F') return c - 'A' + 10;
    return -1;
  };
  const char a = t[3], b = t[4];
  if (a == '+') return hexval(b);
  const int hi = hexval(a), lo = hexval(b);
  if (hi < 0 || lo < 0) return -1;
  return hi * 16 + lo;
}

// token_type_is_emittable (lib.rs:704-710).
int emittable(int64_t type) {
  if (type == 1 || type == 4 || type == 6) return 1;
  if (type == 2 || type == 3 || type == 5) return 0;
  return -1;
}

}  // namespace

extern "C" {

int dtl_tokenizer_from_gguf(const uint8_t* gguf, size_t len, dtl_tokenizer** out) {
  if (!gguf || !out) return DTL_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  Gguf g;
  if (g.parse(gguf, len) != GgufError::None) return DTL_ERR_GGUF;
  std::vector<std::string_view> tokens;
  GgufError e = g.array_strings("tokenizer.ggml.tokens", &tokens);
  if (e == GgufError::MetadataNotFound) return DTL_ERR_TOKEN_MISSING_VOCABULARY;
  if (e != GgufError::None) return DTL_ERR_TOKEN_METADATA_TYPE;
  // optional_gguf_emit_mask (lib.rs:666-695): i32 or u32 token types.
  std::vector<int8_t> emit(tokens.size(), 1);
  if (const GgufValue* tv = g.find("tokenizer.ggml.token_type")) {
    if (tv->type != GV_ARRAY || (tv->array_type != GV_I32 && tv->array_type != GV_U32))
      return DTL_ERR_TOKEN_METADATA_TYPE;
    std::vector<int64_t> types;
    if (g.array_ints("tokenizer.ggml.token_type", &types) != GgufError::None)
      return DTL_ERR_TOKEN_METADATA_TYPE;
    if (types.size() != tokens.size()) return DTL_ERR_TOKEN_TYPE_LENGTH;
    for (size_t i = 0; i < types.size(); i++) {
      const int em = emittable(types[i]);
      if (em < 0) return DTL_ERR_TOKEN_INVALID_TOKEN_TYPE;
      emit[i] = (int8_t)em;
    }
  }
  // Tokenizer kind (lib.rs:86-131): a named model, merges or scores select a
  // BPE / SentencePiece tokenizer, which this library does not provide.
  if (const GgufValue* mv = g.find("tokenizer.ggml.model")) {
    if (mv->type != GV_STRING) return DTL_ERR_TOKEN_METADATA_TYPE;
    return DTL_ERR_TOKEN_UNSUPPORTED_MODEL;
  }
  if (const GgufValue* mg = g.find("tokenizer.ggml.merges")) {
    if (mg->type != GV_ARRAY || mg->array_type != GV_STRING) return DTL_ERR_TOKEN_METADATA_TYPE;
    if (mg->array_len > 0) return DTL_ERR_TOKEN_UNSUPPORTED_MODEL;
  }
  if (g.find("tokenizer.ggml.scores")) return DTL_ERR_TOKEN_UNSUPPORTED_MODEL;
  // ByteFallbackTokenizer::from_tokens_and_emit_mask (lib.rs:262-317).
  auto t = std::make_unique<dtl_tokenizer>();
  for (int b = 0; b < 256; b++) t->byte_to_token[b] = -1;
  t->token_to_byte.assign(tokens.size(), -1);
  bool seen[256] = {};
  for (size_t i = 0; i < tokens.size(); i++) {
    const int b = canonical_byte(tokens[i]);
    if (b < 0) continue;
    if (i > 0xffffffffull) return DTL_ERR_TOKEN_INDEX_OVERFLOW;
    if (seen[b]) return DTL_ERR_TOKEN_DUPLICATE_BYTE_FALLBACK;
    seen[b] = true;
    t->token_to_byte[i] = (int16_t)b;
    if (emit[i]) t->byte_to_token[b] = (int32_t)i;
  }
  for (int b = 0; b < 256; b++)
    if (!seen[b]) return DTL_ERR_TOKEN_INCOMPLETE_BYTE_FALLBACK;
  *out = t.release();
  return DTL_OK;
}

void dtl_tokenizer_free(dtl_tokenizer* t) { delete t; }

size_t dtl_tokenizer_vocab_len(const dtl_tokenizer* t) { return t ? t->token_to_byte.size() : 0; }

int dtl_tokenizer_codec_symbols(const dtl_tokenizer* t, const uint8_t* input, size_t n,
                                size_t vocab_len, uint32_t* out, size_t cap, size_t* n_out) {
  if (!t || (!input && n) || !n_out) return DTL_ERR_INVALID_ARGUMENT;
  if (vocab_len + 256 > 0xffffffffull) return DTL_ERR_TOKEN_INDEX_OVERFLOW;
  *n_out = n;  // one symbol per byte for the byte-fallback kind
  if (!out || cap < n) return out ? DTL_ERR_INVALID_ARGUMENT : DTL_OK;
  for (size_t i = 0; i < n; i++) {
    const int32_t tok = t->byte_to_token[input[i]];
    out[i] = tok >= 0 ? (uint32_t)tok : (uint32_t)(vocab_len + input[i]);
  }
  return DTL_OK;
}

int dtl_tokenizer_decode_symbol(const dtl_tokenizer* t, uint32_t symbol, size_t vocab_len,
                                uint8_t* out, size_t cap, size_t* n_out) {
  if (!t || !n_out) return DTL_ERR_INVALID_ARGUMENT;
  uint8_t b;
  if (symbol < vocab_len) {
    if (symbol >= t->token_to_byte.size() || t->token_to_byte[symbol] < 0)
      return DTL_ERR_TOKEN_INVALID_TOKEN;
    b = (uint8_t)t->token_to_byte[symbol];
  } else if (symbol < vocab_len + 256) {
    b = (uint8_t)(symbol - vocab_len);
  } else {
    return DTL_ERR_TOKEN_INVALID_TOKEN;
  }
  *n_out = 1;
  if (!out || cap < 1) return out ? DTL_ERR_INVALID_ARGUMENT : DTL_OK;
  out[0] = b;
  return DTL_OK;
}

}  // extern "C"
