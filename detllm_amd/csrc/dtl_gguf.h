// GGUF v2/v3 container reader (host side of the library).
// Follows crates/det-gguf/src/lib.rs of mii443/detllm: little-endian
// header, metadata key/value table (lib.rs:374-486), tensor infos with
// ggml type ids, 32-byte aligned data section (lib.rs:199-216) and
// non-overlapping tensor ranges (lib.rs:218-245).  Zero copy: views point
// into the caller's buffer.
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <string_view>
#include <vector>

namespace dtl {

enum class GgufError {
  None, BadMagic, UnsupportedVersion, Truncated, UnsupportedValueType, InvalidUtf8,
  InvalidTensorOffset, InvalidTensorShape, TensorNotFound, MetadataNotFound,
  DuplicateMetadataKey, DuplicateTensorName, InvalidBool, MetadataTypeMismatch,
  UnsupportedTensorType
};

enum GgufValueType : uint32_t {
  GV_U8 = 0, GV_I8 = 1, GV_U16 = 2, GV_I16 = 3, GV_U32 = 4, GV_I32 = 5, GV_F32 = 6,
  GV_BOOL = 7, GV_STRING = 8, GV_ARRAY = 9, GV_U64 = 10, GV_I64 = 11, GV_F64 = 12
};

enum GgmlType : uint32_t {
  GGML_F32 = 0, GGML_F16 = 1, GGML_Q4_0 = 2, GGML_Q8_0 = 8, GGML_Q4_K = 12, GGML_Q6_K = 14
};

struct GgufValue {
  uint32_t type = 0;
  uint64_t u = 0;     // unsigned / bool payload
  int64_t i = 0;      // signed payload
  double f = 0.0;     // float payload
  std::string_view str;
  uint32_t array_type = 0;
  uint64_t array_len = 0;
  size_t array_offset = 0;  // byte offset of the first element in the file
};

struct GgufTensor {
  std::string_view name;
  std::vector<uint64_t> dims;
  uint32_t type = 0;
  uint64_t offset = 0;
};

// Type size in bytes per block and elements per block (det-gguf lib.rs:110-141).
bool ggml_type_size(uint32_t type, uint64_t* bytes, uint64_t* block);

class Gguf {
 public:
  GgufError parse(const uint8_t* data, size_t len);

  const GgufValue* find(std::string_view key) const;
  GgufError tensor(std::string_view name, const GgufTensor** out) const;
  GgufError meta_u32(std::string_view key, uint32_t* out) const;
  GgufError meta_f32(std::string_view key, float* out) const;
  GgufError meta_str(std::string_view key, std::string_view* out) const;
  // Elements of an array-of-strings / array-of-integers metadata value
  // (MetadataTypeMismatch for another element type).
  GgufError array_strings(std::string_view key, std::vector<std::string_view>* out) const;
  GgufError array_ints(std::string_view key, std::vector<int64_t>* out) const;
  GgufError tensor_data(const GgufTensor& t, const uint8_t** data, size_t* len) const;
  static GgufError element_count(const GgufTensor& t, uint64_t* n);
  static GgufError encoded_len(const GgufTensor& t, uint64_t* n);

  const uint8_t* bytes() const { return bytes_; }

 private:
  const uint8_t* bytes_ = nullptr;
  size_t len_ = 0;
  uint32_t version_ = 0;
  size_t data_offset_ = 0;
  std::map<std::string_view, GgufValue> meta_;
  std::vector<GgufTensor> tensors_;
};

}  // namespace dtl
