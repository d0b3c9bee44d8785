// GGUF v2/v3 container reader; see dtl_gguf.h.
#include "dtl_gguf.h"

#include <algorithm>
#include <cstring>

namespace dtl {

namespace {

class Cursor {
 public:
  Cursor(const uint8_t* b, size_t n) : b_(b), n_(n) {}
  size_t pos() const { return pos_; }
  size_t remaining() const { return n_ - pos_; }

  GgufError take(size_t k, const uint8_t** p) {
    if (k > remaining()) return GgufError::Truncated;
    *p = b_ + pos_;
    pos_ += k;
    return GgufError::None;
  }
  template <typename T>
  GgufError le(T* v) {
    const uint8_t* p;
    GgufError e = take(sizeof(T), &p);
    if (e != GgufError::None) return e;
    uint64_t acc = 0;
    for (size_t i = 0; i < sizeof(T); i++) acc |= (uint64_t)p[i] << (8 * i);
    *v = (T)acc;
    return GgufError::None;
  }
  GgufError string(std::string_view* s) {
    uint64_t len;
    GgufError e = le(&len);
    if (e != GgufError::None) return e;
    if (len > remaining()) return GgufError::Truncated;
    const uint8_t* p;
    take((size_t)len, &p);
    if (!valid_utf8(p, (size_t)len)) return GgufError::InvalidUtf8;
    *s = std::string_view((const char*)p, (size_t)len);
    return GgufError::None;
  }
  // Rejects counts whose minimum encoding cannot fit in the rest of the file.
  GgufError ensure_count(uint64_t count, uint64_t min_bytes) const {
    if (min_bytes != 0 && count > remaining() / min_bytes) return GgufError::Truncated;
    return GgufError::None;
  }

 private:
  static bool valid_utf8(const uint8_t* s, size_t n) {
    size_t i = 0;
    while (i < n) {
      uint8_t c = s[i];
      if (c < 0x80) {
        i++;
        continue;
      }
      size_t extra;
      uint32_t cp, lowest;
      if ((c & 0xe0) == 0xc0) {
        extra = 1; cp = c & 0x1f; lowest = 0x80;
      } else if ((c & 0xf0) == 0xe0) {
        extra = 2; cp = c & 0x0f; lowest = 0x800;
      } else if ((c & 0xf8) == 0xf0) {
        extra = 3; cp = c & 0x07; lowest = 0x10000;
      } else {
        return false;
      }
      if (i + extra >= n) return false;
      for (size_t k = 1; k <= extra; k++) {
        if ((s[i + k] & 0xc0) != 0x80) return false;
        cp = (cp << 6) | (s[i + k] & 0x3f);
      }
      if (cp < lowest || cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff)) return false;
      i += extra + 1;
    }
    return true;
  }

  const uint8_t* b_;
  size_t n_;
  size_t pos_ = 0;
};

GgufError read_value(Cursor& c, GgufValue* v) {
  GgufError e = c.le(&v->type);
  if (e != GgufError::None) return e;
  switch (v->type) {
    case GV_U8: { uint8_t x = 0; e = c.le(&x); v->u = x; v->i = x; return e; }
    case GV_I8: { uint8_t x = 0; e = c.le(&x); v->u = x; v->i = (int8_t)x; return e; }
    case GV_U16: { uint16_t x = 0; e = c.le(&x); v->u = x; v->i = x; return e; }
    case GV_I16: { uint16_t x = 0; e = c.le(&x); v->u = x; v->i = (int16_t)x; return e; }
    case GV_U32: { uint32_t x = 0; e = c.le(&x); v->u = x; v->i = x; return e; }
    case GV_I32: { uint32_t x = 0; e = c.le(&x); v->u = x; v->i = (int32_t)x; return e; }
    case GV_F32: {
      uint32_t x = 0;
      e = c.le(&x);
      float f;
      std::memcpy(&f, &x, 4);
      v->f = f;
      return e;
    }
    case GV_BOOL: {
      uint8_t x = 0;
      if ((e = c.le(&x)) != GgufError::None) return e;
      if (x > 1) return GgufError::InvalidBool;
      v->u = x;
      return GgufError::None;
    }
    case GV_STRING: return c.string(&v->str);
    case GV_U64: { uint64_t x = 0; e = c.le(&x); v->u = x; v->i = (int64_t)x; return e; }
    case GV_I64: { uint64_t x = 0; e = c.le(&x); v->u = x; v->i = (int64_t)x; return e; }
    case GV_F64: {
      uint64_t x = 0;
      e = c.le(&x);
      std::memcpy(&v->f, &x, 8);
      return e;
    }
    case GV_ARRAY: {
      if ((e = c.le(&v->array_type)) != GgufError::None) return e;
      if ((e = c.le(&v->array_len)) != GgufError::None) return e;
      uint64_t width;
      switch (v->array_type) {
        case GV_U8: case GV_I8: case GV_BOOL: width = 1; break;
        case GV_U16: case GV_I16: width = 2; break;
        case GV_U32: case GV_I32: case GV_F32: width = 4; break;
        case GV_STRING: case GV_U64: case GV_I64: case GV_F64: width = 8; break;
        default: return GgufError::UnsupportedValueType;
      }
      if ((e = c.ensure_count(v->array_len, width)) != GgufError::None) return e;
      v->array_offset = c.pos();
      for (uint64_t k = 0; k < v->array_len; k++) {
        if (v->array_type == GV_STRING) {
          std::string_view s;
          if ((e = c.string(&s)) != GgufError::None) return e;
        } else {
          const uint8_t* p;
          if ((e = c.take((size_t)width, &p)) != GgufError::None) return e;
          if (v->array_type == GV_BOOL && *p > 1) return GgufError::InvalidBool;
        }
      }
      return GgufError::None;
    }
    default: return GgufError::UnsupportedValueType;
  }
}

}  // namespace

bool ggml_type_size(uint32_t type, uint64_t* bytes, uint64_t* block) {
  static const struct { uint32_t t; uint64_t b, n; } table[] = {
      {0, 4, 1},     {1, 2, 1},     {2, 18, 32},   {3, 20, 32},   {6, 22, 32},
      {7, 24, 32},   {8, 34, 32},   {9, 40, 32},   {10, 84, 256}, {11, 110, 256},
      {12, 144, 256}, {13, 176, 256}, {14, 210, 256}, {15, 292, 256}};
  for (const auto& r : table)
    if (r.t == type) {
      *bytes = r.b;
      *block = r.n;
      return true;
    }
  return false;
}

GgufError Gguf::element_count(const GgufTensor& t, uint64_t* n) {
  if (t.dims.empty()) return GgufError::InvalidTensorShape;
  uint64_t acc = 1;
  for (uint64_t d : t.dims) {
    if (d == 0 || acc > UINT64_MAX / d) return GgufError::InvalidTensorShape;
    acc *= d;
  }
  *n = acc;
  return GgufError::None;
}

GgufError Gguf::encoded_len(const GgufTensor& t, uint64_t* n) {
  uint64_t count;
  GgufError e = element_count(t, &count);
  if (e != GgufError::None) return e;
  uint64_t bytes, block;
  if (!ggml_type_size(t.type, &bytes, &block)) return GgufError::UnsupportedTensorType;
  if (count % block != 0 || count / block > UINT64_MAX / bytes) return GgufError::InvalidTensorShape;
  *n = count / block * bytes;
  return GgufError::None;
}

GgufError Gguf::parse(const uint8_t* data, size_t len) {
  bytes_ = data;
  len_ = len;
  meta_.clear();
  tensors_.clear();
  Cursor c(data, len);
  const uint8_t* magic;
  GgufError e = c.take(4, &magic);
  if (e != GgufError::None) return e;
  if (std::memcmp(magic, "GGUF", 4) != 0) return GgufError::BadMagic;
  if ((e = c.le(&version_)) != GgufError::None) return e;
  if (version_ != 2 && version_ != 3) return GgufError::UnsupportedVersion;
  uint64_t n_tensors, n_meta;
  if ((e = c.le(&n_tensors)) != GgufError::None) return e;
  if ((e = c.le(&n_meta)) != GgufError::None) return e;
  for (uint64_t k = 0; k < n_meta; k++) {
    std::string_view key;
    if ((e = c.string(&key)) != GgufError::None) return e;
    GgufValue v;
    if ((e = read_value(c, &v)) != GgufError::None) return e;
    if (!meta_.emplace(key, v).second) return GgufError::DuplicateMetadataKey;
  }
  if ((e = c.ensure_count(n_tensors, 24)) != GgufError::None) return e;
  tensors_.reserve((size_t)n_tensors);
  for (uint64_t k = 0; k < n_tensors; k++) {
    GgufTensor t;
    if ((e = c.string(&t.name)) != GgufError::None) return e;
    uint32_t ndim;
    if ((e = c.le(&ndim)) != GgufError::None) return e;
    if ((e = c.ensure_count(ndim, 8)) != GgufError::None) return e;
    t.dims.resize(ndim);
    for (uint32_t d = 0; d < ndim; d++)
      if ((e = c.le(&t.dims[d])) != GgufError::None) return e;
    if ((e = c.le(&t.type)) != GgufError::None) return e;
    if ((e = c.le(&t.offset)) != GgufError::None) return e;
    for (const auto& o : tensors_)
      if (o.name == t.name) return GgufError::DuplicateTensorName;
    tensors_.push_back(std::move(t));
  }
  data_offset_ = (c.pos() + 31) & ~(size_t)31;
  if (data_offset_ > len) return GgufError::Truncated;
  std::vector<std::pair<uint64_t, uint64_t>> ranges;
  for (const auto& t : tensors_) {
    uint64_t n;
    if ((e = encoded_len(t, &n)) != GgufError::None) return e;
    uint64_t start = (uint64_t)data_offset_ + t.offset;
    if (start < t.offset || start + n < start) return GgufError::InvalidTensorOffset;
    if (start + n > len) return GgufError::Truncated;
    ranges.emplace_back(start, start + n);
  }
  std::sort(ranges.begin(), ranges.end());
  for (size_t k = 1; k < ranges.size(); k++)
    if (ranges[k - 1].second > ranges[k].first) return GgufError::InvalidTensorOffset;
  return GgufError::None;
}

const GgufValue* Gguf::find(std::string_view key) const {
  auto it = meta_.find(key);
  return it == meta_.end() ? nullptr : &it->second;
}

GgufError Gguf::tensor(std::string_view name, const GgufTensor** out) const {
  const GgufTensor* hit = nullptr;
  for (const auto& t : tensors_)
    if (t.name == name) {
      if (hit) return GgufError::DuplicateTensorName;
      hit = &t;
    }
  if (!hit) return GgufError::TensorNotFound;
  *out = hit;
  return GgufError::None;
}

GgufError Gguf::meta_u32(std::string_view key, uint32_t* out) const {
  const GgufValue* v = find(key);
  if (!v) return GgufError::MetadataNotFound;
  if (v->type == GV_U32) {
    *out = (uint32_t)v->u;
    return GgufError::None;
  }
  if (v->type == GV_U64) {
    if (v->u > 0xffffffffull) return GgufError::MetadataTypeMismatch;
    *out = (uint32_t)v->u;
    return GgufError::None;
  }
  return GgufError::MetadataTypeMismatch;
}

GgufError Gguf::meta_f32(std::string_view key, float* out) const {
  const GgufValue* v = find(key);
  if (!v) return GgufError::MetadataNotFound;
  if (v->type != GV_F32 && v->type != GV_F64) return GgufError::MetadataTypeMismatch;
  *out = (float)v->f;
  return GgufError::None;
}

GgufError Gguf::array_strings(std::string_view key, std::vector<std::string_view>* out) const {
  const GgufValue* v = find(key);
  if (!v) return GgufError::MetadataNotFound;
  if (v->type != GV_ARRAY || v->array_type != GV_STRING) return GgufError::MetadataTypeMismatch;
  out->clear();
  out->reserve((size_t)v->array_len);
  size_t pos = v->array_offset;
  for (uint64_t k = 0; k < v->array_len; k++) {
    uint64_t n;
    std::memcpy(&n, bytes_ + pos, 8);  // validated by parse()
    out->emplace_back((const char*)bytes_ + pos + 8, (size_t)n);
    pos += 8 + (size_t)n;
  }
  return GgufError::None;
}

GgufError Gguf::array_ints(std::string_view key, std::vector<int64_t>* out) const {
  const GgufValue* v = find(key);
  if (!v) return GgufError::MetadataNotFound;
  if (v->type != GV_ARRAY) return GgufError::MetadataTypeMismatch;
  size_t width;
  switch (v->array_type) {
    case GV_U8: case GV_I8: width = 1; break;
    case GV_U16: case GV_I16: width = 2; break;
    case GV_U32: case GV_I32: width = 4; break;
    case GV_U64: case GV_I64: width = 8; break;
    default: return GgufError::MetadataTypeMismatch;
  }
  out->clear();
  out->reserve((size_t)v->array_len);
  const uint8_t* p = bytes_ + v->array_offset;
  for (uint64_t k = 0; k < v->array_len; k++, p += width) {
    int64_t x = 0;
    switch (v->array_type) {
      case GV_U8: x = p[0]; break;
      case GV_I8: x = (int8_t)p[0]; break;
      case GV_U16: { uint16_t t; std::memcpy(&t, p, 2); x = t; break; }
      case GV_I16: { int16_t t; std::memcpy(&t, p, 2); x = t; break; }
      case GV_U32: { uint32_t t; std::memcpy(&t, p, 4); x = t; break; }
      case GV_I32: { int32_t t; std::memcpy(&t, p, 4); x = t; break; }
      default: std::memcpy(&x, p, 8); break;
    }
    out->push_back(x);
  }
  return GgufError::None;
}

GgufError Gguf::meta_str(std::string_view key, std::string_view* out) const {
  const GgufValue* v = find(key);
  if (!v) return GgufError::MetadataNotFound;
  if (v->type != GV_STRING) return GgufError::MetadataTypeMismatch;
  *out = v->str;
  return GgufError::None;
}

GgufError Gguf::tensor_data(const GgufTensor& t, const uint8_t** data, size_t* len) const {
  uint64_t n;
  GgufError e = encoded_len(t, &n);
  if (e != GgufError::None) return e;
  uint64_t start = (uint64_t)data_offset_ + t.offset;
  if (start + n > len_) return GgufError::Truncated;
  *data = bytes_ + start;
  *len = (size_t)n;
  return GgufError::None;
}

}  // namespace dtl
