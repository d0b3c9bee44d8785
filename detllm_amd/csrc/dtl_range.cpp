// 64-bit carry-less range coder on the host: RangeEncoder / RangeDecoder of
// crates/det-coder/src/range.rs (mii443/detllm).  The GPU produces the
// (cum, freq, total) triples and decoder tables; the coder itself is a
// strictly sequential byte stream and stays on the CPU.
#include <cstdint>
#include <cstring>
#include <new>
#include <vector>

#include "../../include/detllm.h"

namespace {

constexpr uint64_t kTop = 1ull << 56;
constexpr uint64_t kBottom = 1ull << 48;
constexpr uint64_t kTotalLimit = 1ull << 31;

// validate (range.rs:160-166)
bool valid_triple(uint64_t cum, uint64_t freq, uint64_t total) {
  uint64_t end = cum + freq;
  if (end < cum) return false;
  return freq != 0 && total != 0 && total < kTotalLimit && end <= total;
}

// normalize_step (range.rs:168-178): shift out a byte when the top byte of
// low is settled, or force a settle when the range underflows.
bool normalize_step(uint64_t low, uint64_t* range) {
  if ((low ^ (low + *range)) < kTop) return true;
  if (*range < kBottom) {
    *range = (0 - low) & (kBottom - 1);
    return true;
  }
  return false;
}

}  // namespace

struct dtl_range_encoder {
  uint64_t low = 0;
  uint64_t range = ~0ull;
  std::vector<uint8_t> out;
};

struct dtl_range_decoder {
  uint64_t low = 0, code = 0, range = ~0ull;
  bool pending = false;
  uint64_t pending_range = 0, pending_total = 0;
  const uint8_t* in = nullptr;
  size_t len = 0, pos = 0;

  bool next(uint8_t* b) {
    if (pos >= len) return false;
    *b = in[pos++];
    return true;
  }
};

extern "C" {

int dtl_range_encoder_new(dtl_range_encoder** out) {
  if (!out) return DTL_ERR_INVALID_ARGUMENT;
  *out = new (std::nothrow) dtl_range_encoder();
  return *out ? DTL_OK : DTL_ERR_OUT_OF_MEMORY;
}

int dtl_range_encode(dtl_range_encoder* e, uint64_t cum, uint64_t freq, uint64_t total) {
  if (!e) return DTL_ERR_INVALID_ARGUMENT;
  if (!valid_triple(cum, freq, total)) return DTL_ERR_RANGE_INVALID_FREQUENCY;
  e->range /= total;
  e->low += e->range * cum;
  e->range *= freq;
  while (normalize_step(e->low, &e->range)) {
    e->out.push_back((uint8_t)(e->low >> 56));
    e->low <<= 8;
    e->range <<= 8;
  }
  return DTL_OK;
}

// RangeEncoder::snapshot (range.rs:48-54): the coder state (low, range) and
// the bytes emitted so far; out may be null to ask for their count in *len.
int dtl_range_encoder_snapshot(const dtl_range_encoder* e, uint64_t* low, uint64_t* range, uint8_t* out,
                               size_t cap, size_t* len) {
  if (!e || !low || !range || !len) return DTL_ERR_INVALID_ARGUMENT;
  *low = e->low;
  *range = e->range;
  *len = e->out.size();
  if (!out) return DTL_OK;
  if (cap < e->out.size()) return DTL_ERR_BUFFER_TOO_SMALL;
  if (!e->out.empty()) std::memcpy(out, e->out.data(), e->out.size());
  return DTL_OK;
}

// RangeEncoder::from_snapshot (range.rs:37-46): a zero range is rejected as
// RangeError::InvalidFrequency.
int dtl_range_encoder_from_snapshot(uint64_t low, uint64_t range, const uint8_t* bytes, size_t len,
                                    dtl_range_encoder** out) {
  if (!out || (len && !bytes)) return DTL_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  if (range == 0) return DTL_ERR_RANGE_INVALID_FREQUENCY;
  dtl_range_encoder* e = new (std::nothrow) dtl_range_encoder();
  if (!e) return DTL_ERR_OUT_OF_MEMORY;
  e->low = low;
  e->range = range;
  e->out.assign(bytes, bytes + len);
  *out = e;
  return DTL_OK;
}

int dtl_range_encoder_finish(dtl_range_encoder* e, uint8_t* out, size_t cap, size_t* len) {
  if (!e || !len) return DTL_ERR_INVALID_ARGUMENT;
  size_t n = e->out.size() + 8;
  *len = n;
  if (out) {
    size_t body = e->out.size() < cap ? e->out.size() : cap;
    if (body) std::memcpy(out, e->out.data(), body);
    uint64_t low = e->low;
    for (size_t i = 0; i < 8; i++) {
      if (e->out.size() + i < cap) out[e->out.size() + i] = (uint8_t)(low >> 56);
      low <<= 8;
    }
  }
  return DTL_OK;
}

void dtl_range_encoder_free(dtl_range_encoder* e) { delete e; }

int dtl_range_decoder_new(const uint8_t* data, size_t len, dtl_range_decoder** out) {
  if (!out || (!data && len)) return DTL_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  dtl_range_decoder* d = new (std::nothrow) dtl_range_decoder();
  if (!d) return DTL_ERR_OUT_OF_MEMORY;
  d->in = data;
  d->len = len;
  for (int i = 0; i < 8; i++) {
    uint8_t b;
    if (!d->next(&b)) {
      delete d;
      return DTL_ERR_RANGE_UNEXPECTED_EOF;
    }
    d->code = (d->code << 8) | b;
  }
  *out = d;
  return DTL_OK;
}

// The decoder's state between symbols (no pending decode_freq), for a
// decode that continues in a later call.
int dtl_range_decoder_snapshot(const dtl_range_decoder* d, dtl_range_decoder_state* st) {
  if (!d || !st) return DTL_ERR_INVALID_ARGUMENT;
  if (d->pending) return DTL_ERR_RANGE_INVALID_FREQUENCY;
  st->low = d->low;
  st->range = d->range;
  st->code = d->code;
  st->pos = d->pos;
  return DTL_OK;
}

int dtl_range_decoder_from_snapshot(const uint8_t* data, size_t len, const dtl_range_decoder_state* st,
                                    dtl_range_decoder** out) {
  if (!out || !st || (!data && len)) return DTL_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  if (st->pos > len || st->pos < 8 || st->range == 0) return DTL_ERR_INVALID_ARGUMENT;
  dtl_range_decoder* d = new (std::nothrow) dtl_range_decoder();
  if (!d) return DTL_ERR_OUT_OF_MEMORY;
  d->in = data;
  d->len = len;
  d->pos = (size_t)st->pos;
  d->low = st->low;
  d->range = st->range;
  d->code = st->code;
  *out = d;
  return DTL_OK;
}

int dtl_range_decode_freq(dtl_range_decoder* d, uint64_t total, uint64_t* value) {
  if (!d || !value) return DTL_ERR_INVALID_ARGUMENT;
  if (d->pending || total == 0 || total >= kTotalLimit) return DTL_ERR_RANGE_INVALID_FREQUENCY;
  uint64_t r = d->range / total;
  if (r == 0) return DTL_ERR_RANGE_INVALID_FREQUENCY;
  uint64_t v = (d->code - d->low) / r;
  if (v >= total) return DTL_ERR_RANGE_INVALID_FREQUENCY;
  d->pending = true;
  d->pending_range = r;
  d->pending_total = total;
  *value = v;
  return DTL_OK;
}

int dtl_range_decode_advance(dtl_range_decoder* d, uint64_t cum, uint64_t freq, uint64_t total) {
  if (!d) return DTL_ERR_INVALID_ARGUMENT;
  if (!valid_triple(cum, freq, total)) return DTL_ERR_RANGE_INVALID_FREQUENCY;
  if (!d->pending || d->pending_total != total) return DTL_ERR_RANGE_INVALID_FREQUENCY;
  d->pending = false;
  d->range = d->pending_range;
  d->low += d->range * cum;
  d->range *= freq;
  while (normalize_step(d->low, &d->range)) {
    uint8_t b;
    if (!d->next(&b)) return DTL_ERR_RANGE_UNEXPECTED_EOF;
    d->code = (d->code << 8) | b;
    d->low <<= 8;
    d->range <<= 8;
  }
  return DTL_OK;
}

void dtl_range_decoder_free(dtl_range_decoder* d) { delete d; }

}  // extern "C"
