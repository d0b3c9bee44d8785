// Host side of libdetllm_amd: GGUF model loading and device repacking,
// sessions (KV cache, RoPE tables, workspace, stream), the per-layer launch
// sequence of the decoder forward and the C ABI declared in detllm.h.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../../include/detllm.h"
#include "dtl_device.h"
#include "dtl_gguf.h"
#include "dtl_sha256.h"

using namespace dtl;

namespace {

// ---------------------------------------------------------------------------
// device memory helpers

struct DevBuf {
  void* p = nullptr;
  size_t n = 0;
};

int hip_status(hipError_t e) {
  if (e == hipSuccess) return DTL_OK;
  if (e == hipErrorOutOfMemory) return DTL_ERR_OUT_OF_MEMORY;
  if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) return DTL_ERR_NO_DEVICE;
  return DTL_ERR_DEVICE;
}

// DETLLM_TRACE_ERRORS=1 names the failing runtime call on stderr.
int hip_fail(hipError_t e, const char* expr, int line) {
  static const bool trace = [] {
    const char* v = getenv("DETLLM_TRACE_ERRORS");
    return v && *v && *v != '0';
  }();
  if (trace) std::fprintf(stderr, "detllm: %s (dtl_api.hip:%d): %s\n", expr, line, hipGetErrorString(e));
  return hip_status(e);
}

#define HIP_TRY(expr)                                              \
  do {                                                             \
    hipError_t e_ = (expr);                                        \
    if (e_ != hipSuccess) return hip_fail(e_, #expr, __LINE__);    \
  } while (0)

// Owner of a set of device allocations, freed together.
class Arena {
 public:
  ~Arena() { release(); }
  template <typename T>
  int alloc(T** out, size_t count) {
    void* p = nullptr;
    size_t bytes = count * sizeof(T);
    if (bytes == 0) bytes = 16;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return hip_status(e);
    ptrs_.push_back(p);
    bytes_ += bytes;
    *out = static_cast<T*>(p);
    return DTL_OK;
  }
  template <typename T>
  int upload(T** out, const void* host, size_t count) {
    int st = alloc(out, count);
    if (st) return st;
    return hip_status(hipMemcpy(*out, host, count * sizeof(T), hipMemcpyHostToDevice));
  }
  void release() {
    for (void* p : ptrs_) (void)hipFree(p);
    ptrs_.clear();
    bytes_ = 0;
  }
  size_t bytes() const { return bytes_; }

 private:
  std::vector<void*> ptrs_;
  size_t bytes_ = 0;
};

uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

bool f16_finite(uint16_t b) { return (b & 0x7c00) != 0x7c00; }

// Bit-exact f16 -> f32 on the host (det-num f16.rs:6-34), used when F16
// tensors are widened to F32 at load (det-model lib.rs:1753-1768).
float f16_to_f32_host(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16, exp = (h >> 10) & 0x1f, frac = h & 0x3ff, out;
  if (exp == 0) {
    if (frac == 0) {
      out = sign;
    } else {
      int e = -14;
      while ((frac & 0x400) == 0) {
        frac <<= 1;
        e--;
      }
      out = sign | ((uint32_t)(e + 127) << 23) | ((frac & 0x3ff) << 13);
    }
  } else if (exp == 0x1f) {
    out = sign | 0x7f800000u | (frac << 13);
  } else {
    out = sign | ((exp + 112) << 23) | (frac << 13);
  }
  float f;
  std::memcpy(&f, &out, 4);
  return f;
}

// ---------------------------------------------------------------------------
// model

struct HostConfig {
  size_t block_count = 0, d = 0, ff = 0, heads = 0, kv_heads = 0, ctx = 0, rope_dim = 0;
  float eps = 0, attention_scale = 0, rope_base = 0;
  int split_half = 0;
};

struct Layer {
  float* attn_norm = nullptr;
  float* ffn_norm = nullptr;
  float* bq = nullptr;
  float* bk = nullptr;
  float* bv = nullptr;
  DevMat wq{}, wk{}, wv{}, wo{}, gate{}, up{}, down{};
};

}  // namespace

struct dtl_model {
  HostConfig c;
  size_t head_dim = 0, vocab = 0;
  DevMat emb{}, out{};
  float* out_norm = nullptr;
  std::vector<Layer> layers;
  int device = 0;
  Arena arena;
};

namespace {

int map_meta(GgufError e) {
  return e == GgufError::MetadataNotFound ? DTL_ERR_MISSING_METADATA : DTL_ERR_GGUF;
}

// Repacks one GGUF tensor into the device layout of DevMat (values unchanged).
int upload_matrix(const Gguf& g, const GgufTensor& t, size_t rows, size_t cols, Arena& arena,
                  DevMat* out) {
  const uint8_t* data;
  size_t len;
  if (g.tensor_data(t, &data, &len) != GgufError::None) return DTL_ERR_GGUF;
  DevMat m{};
  m.rows = (int32_t)rows;
  m.cols = (int32_t)cols;
  int st;
  if (t.type == GGML_F32 || t.type == GGML_F16) {
    std::vector<float> v(rows * cols);
    if (t.type == GGML_F32) {
      if (len != rows * cols * 4) return DTL_ERR_SHAPE;
      std::memcpy(v.data(), data, len);
      for (float f : v)
        if (!std::isfinite(f)) return DTL_ERR_NON_FINITE;
    } else {
      if (len != rows * cols * 2) return DTL_ERR_SHAPE;
      for (size_t i = 0; i < rows * cols; i++) {
        uint16_t b = rd16(data + 2 * i);
        if (!f16_finite(b)) return DTL_ERR_NON_FINITE;
        v[i] = f16_to_f32_host(b);
      }
    }
    m.type = GGML_F32;
    m.nb = (int32_t)cols;
    float* w;
    if ((st = arena.upload(&w, v.data(), v.size()))) return st;
    m.w = w;
    *out = m;
    return DTL_OK;
  }
  if (t.type != GGML_Q8_0 && t.type != GGML_Q4_0 && t.type != GGML_Q4_K && t.type != GGML_Q6_K)
    return DTL_ERR_UNSUPPORTED_TENSOR_TYPE;
  size_t bs = (t.type == GGML_Q4_K || t.type == GGML_Q6_K) ? 256 : 32;
  if (cols % bs) return DTL_ERR_SHAPE;
  size_t nb = cols / bs, nblk = rows * nb;
  m.type = (int32_t)t.type;
  m.nb = (int32_t)nb;
  switch (t.type) {
    case GGML_Q8_0: {
      if (len != nblk * 34) return DTL_ERR_SHAPE;
      std::vector<int8_t> q(nblk * 32);
      std::vector<uint16_t> d(nblk);
      for (size_t b = 0; b < nblk; b++) {
        const uint8_t* p = data + b * 34;
        d[b] = rd16(p);
        if (!f16_finite(d[b])) return DTL_ERR_NON_FINITE;
        std::memcpy(&q[b * 32], p + 2, 32);
      }
      int8_t* wq;
      uint16_t* wd;
      if ((st = arena.upload(&wq, q.data(), q.size()))) return st;
      if ((st = arena.upload(&wd, d.data(), d.size()))) return st;
      m.w = wq;
      m.d16 = wd;
      break;
    }
    case GGML_Q4_0: {
      if (len != nblk * 18) return DTL_ERR_SHAPE;
      std::vector<uint8_t> q(nblk * 16);
      std::vector<uint16_t> d(nblk);
      for (size_t b = 0; b < nblk; b++) {
        const uint8_t* p = data + b * 18;
        d[b] = rd16(p);
        if (!f16_finite(d[b])) return DTL_ERR_NON_FINITE;
        std::memcpy(&q[b * 16], p + 2, 16);
      }
      uint8_t* wq;
      uint16_t* wd;
      if ((st = arena.upload(&wq, q.data(), q.size()))) return st;
      if ((st = arena.upload(&wd, d.data(), d.size()))) return st;
      m.w = wq;
      m.d16 = wd;
      break;
    }
    case GGML_Q4_K: {
      if (len != nblk * 144) return DTL_ERR_SHAPE;
      std::vector<uint8_t> q(nblk * 128), h(nblk * 16);
      for (size_t b = 0; b < nblk; b++) {
        const uint8_t* p = data + b * 144;
        if (!f16_finite(rd16(p)) || !f16_finite(rd16(p + 2))) return DTL_ERR_NON_FINITE;
        std::memcpy(&h[b * 16], p, 16);
        std::memcpy(&q[b * 128], p + 16, 128);
      }
      uint8_t *wq, *wh;
      if ((st = arena.upload(&wq, q.data(), q.size()))) return st;
      if ((st = arena.upload(&wh, h.data(), h.size()))) return st;
      m.w = wq;
      m.hdr = wh;
      break;
    }
    case GGML_Q6_K: {
      if (len != nblk * 210) return DTL_ERR_SHAPE;
      std::vector<uint8_t> body(nblk * 208);
      std::vector<uint16_t> d(nblk);
      for (size_t b = 0; b < nblk; b++) {
        const uint8_t* p = data + b * 210;
        d[b] = rd16(p + 208);
        if (!f16_finite(d[b])) return DTL_ERR_NON_FINITE;
        std::memcpy(&body[b * 208], p, 208);
      }
      uint8_t* wb;
      uint16_t* wd;
      if ((st = arena.upload(&wb, body.data(), body.size()))) return st;
      if ((st = arena.upload(&wd, d.data(), d.size()))) return st;
      m.w = wb;
      m.d16 = wd;
      break;
    }
  }
  *out = m;
  return DTL_OK;
}

// read_weight_matrix (det-model lib.rs:1778-1810)
int read_matrix(const Gguf& g, const std::string& name, size_t rows, size_t cols, Arena& arena,
                DevMat* out) {
  const GgufTensor* t;
  if (g.tensor(name, &t) != GgufError::None) return DTL_ERR_GGUF;
  if (t->dims.size() != 2 || t->dims[0] != cols || t->dims[1] != rows) return DTL_ERR_SHAPE;
  return upload_matrix(g, *t, rows, cols, arena, out);
}

// read_f32_vector / read_dense_tensor_as_f32 (det-model lib.rs:1674-1776)
int read_vector(const Gguf& g, const std::string& name, size_t n, Arena& arena, float** out,
                bool optional) {
  const GgufTensor* t;
  GgufError e = g.tensor(name, &t);
  if (e == GgufError::TensorNotFound && optional) {
    *out = nullptr;
    return DTL_OK;
  }
  if (e != GgufError::None) return DTL_ERR_GGUF;
  if (t->dims.size() != 1 || t->dims[0] != n) return DTL_ERR_SHAPE;
  const uint8_t* data;
  size_t len;
  if (g.tensor_data(*t, &data, &len) != GgufError::None) return DTL_ERR_GGUF;
  std::vector<float> v(n);
  if (t->type == GGML_F32) {
    if (len != n * 4) return DTL_ERR_SHAPE;
    std::memcpy(v.data(), data, len);
    for (float f : v)
      if (!std::isfinite(f)) return DTL_ERR_NON_FINITE;
  } else if (t->type == GGML_F16) {
    if (len != n * 2) return DTL_ERR_SHAPE;
    for (size_t i = 0; i < n; i++) {
      uint16_t b = rd16(data + 2 * i);
      if (!f16_finite(b)) return DTL_ERR_NON_FINITE;
      v[i] = f16_to_f32_host(b);
    }
  } else {
    return DTL_ERR_UNSUPPORTED_TENSOR_TYPE;
  }
  return arena.upload(out, v.data(), n);
}

int opt_u32(const Gguf& g, const std::string& key, uint32_t* v, bool* present) {
  GgufError e = g.meta_u32(key, v);
  *present = e == GgufError::None;
  if (e == GgufError::None || e == GgufError::MetadataNotFound) return DTL_OK;
  return map_meta(e);
}

int opt_f32(const Gguf& g, const std::string& key, float* v, bool* present) {
  GgufError e = g.meta_f32(key, v);
  *present = e == GgufError::None;
  if (e == GgufError::None || e == GgufError::MetadataNotFound) return DTL_OK;
  return map_meta(e);
}

int opt_bool(const Gguf& g, const std::string& key, bool* v, bool* present) {
  const GgufValue* kv = g.find(key);
  *present = kv != nullptr;
  if (!kv) return DTL_OK;
  if (kv->type != GV_BOOL) return DTL_ERR_GGUF;
  *v = kv->u != 0;
  return DTL_OK;
}

int reject_nonzero_f32(const Gguf& g, const std::string& key) {
  const GgufValue* kv = g.find(key);
  if (!kv) return DTL_OK;
  if (kv->type != GV_F32 && kv->type != GV_F64) return DTL_ERR_GGUF;
  if (!std::isfinite(kv->f)) return DTL_ERR_SHAPE;
  return kv->f != 0.0 ? DTL_ERR_UNSUPPORTED_MODEL_FEATURE : DTL_OK;
}

// LlamaConfig::validate (det-model lib.rs:1581-1616)
int validate_config(const HostConfig& c) {
  if (c.block_count == 0 || c.d == 0 || c.ff == 0 || c.heads == 0 || c.kv_heads == 0 ||
      c.ctx == 0 || c.heads % c.kv_heads != 0 || c.rope_dim == 0 || c.rope_dim % 2 != 0 ||
      !std::isfinite(c.eps) || c.eps <= 0.0f || !std::isfinite(c.attention_scale) ||
      c.attention_scale <= 0.0f || !std::isfinite(c.rope_base) || c.rope_base <= 0.0f)
    return DTL_ERR_SHAPE;
  if (c.d % c.heads != 0 || c.rope_dim > c.d / c.heads) return DTL_ERR_SHAPE;
  return DTL_OK;
}

// LlamaConfig::from_gguf (det-model lib.rs:1498-1565), including the
// metadata policy that rejects unsupported model features.
int config_from_gguf(const Gguf& g, HostConfig* c) {
  std::string_view arch;
  GgufError ge = g.meta_str("general.architecture", &arch);
  if (ge != GgufError::None) return map_meta(ge);
  if (arch != "llama" && arch != "qwen2") return DTL_ERR_UNSUPPORTED_ARCHITECTURE;
  c->split_half = arch == "qwen2";
  std::string p = std::string(arch) + ".";
  uint32_t v;
  float f;
  bool present, b;
  int st;
  if ((ge = g.meta_u32(p + "attention.head_count", &v)) != GgufError::None) return map_meta(ge);
  c->heads = v;
  if ((st = opt_u32(g, p + "attention.head_count_kv", &v, &present))) return st;
  c->kv_heads = present ? v : c->heads;
  if ((ge = g.meta_u32(p + "embedding_length", &v)) != GgufError::None) return map_meta(ge);
  c->d = v;
  if (c->heads == 0 || c->d % c->heads != 0) return DTL_ERR_SHAPE;
  if ((st = opt_u32(g, p + "embedding_length_out", &v, &present))) return st;
  if (present && v != c->d) return DTL_ERR_UNSUPPORTED_MODEL_FEATURE;
  if ((st = opt_bool(g, p + "attention.causal", &b, &present))) return st;
  if (present && !b) return DTL_ERR_UNSUPPORTED_MODEL_FEATURE;
  {
    std::string_view s;
    ge = g.meta_str(p + "rope.scaling.type", &s);
    if (ge != GgufError::None && ge != GgufError::MetadataNotFound) return map_meta(ge);
    if (ge == GgufError::None && s != "none") return DTL_ERR_UNSUPPORTED_ROPE_SCALING;
  }
  if ((st = opt_bool(g, p + "use_parallel_residual", &b, &present))) return st;
  if (present && b) return DTL_ERR_UNSUPPORTED_MODEL_FEATURE;
  if ((st = opt_u32(g, p + "attention.sliding_window", &v, &present))) return st;
  if (present && v != 0) return DTL_ERR_UNSUPPORTED_MODEL_FEATURE;
  for (const char* k : {"attention.max_alibi_bias", "attention.clamp_kqv", "attention.value_scale",
                        "attn_logit_softcapping", "final_logit_softcapping", "logit_scale",
                        "embedding_scale", "residual_scale"})
    if ((st = reject_nonzero_f32(g, p + k))) return st;
  size_t hd = c->d / c->heads;
  for (const char* k : {"attention.key_length", "attention.value_length"}) {
    if ((st = opt_u32(g, p + k, &v, &present))) return st;
    if (present && v != hd) return DTL_ERR_UNSUPPORTED_ATTENTION_HEAD_LENGTH;
  }
  if ((st = opt_f32(g, p + "attention.scale", &f, &present))) return st;
  c->attention_scale = present ? f : 1.0f / std::sqrt((float)hd);
  if ((ge = g.meta_u32(p + "block_count", &v)) != GgufError::None) return map_meta(ge);
  c->block_count = v;
  if ((ge = g.meta_u32(p + "feed_forward_length", &v)) != GgufError::None) return map_meta(ge);
  c->ff = v;
  if ((ge = g.meta_f32(p + "attention.layer_norm_rms_epsilon", &f)) != GgufError::None)
    return map_meta(ge);
  c->eps = f;
  if ((st = opt_f32(g, p + "rope.freq_base", &f, &present))) return st;
  c->rope_base = present ? f : 10000.0f;
  if ((st = opt_u32(g, p + "rope.dimension_count", &v, &present))) return st;
  c->rope_dim = present ? v : hd;
  if ((ge = g.meta_u32(p + "context_length", &v)) != GgufError::None) return map_meta(ge);
  c->ctx = v;
  return validate_config(*c);
}

// vocab_size (det-model lib.rs:1648-1672)
int vocab_size(const Gguf& g, size_t* out) {
  std::string_view arch;
  GgufError ge = g.meta_str("general.architecture", &arch);
  if (ge != GgufError::None) return map_meta(ge);
  for (std::string key : {std::string(arch) + ".vocab_size", std::string("llama.vocab_size")}) {
    uint32_t v;
    ge = g.meta_u32(key, &v);
    if (ge == GgufError::None) {
      *out = v;
      return DTL_OK;
    }
    if (ge != GgufError::MetadataNotFound) return map_meta(ge);
  }
  if (const GgufValue* kv = g.find("tokenizer.ggml.tokens")) {
    if (kv->type != GV_ARRAY || kv->array_type != GV_STRING) return DTL_ERR_GGUF;
    *out = (size_t)kv->array_len;
    return DTL_OK;
  }
  const GgufTensor* t;
  if (g.tensor("token_embd.weight", &t) != GgufError::None) return DTL_ERR_GGUF;
  if (t->dims.size() == 2) {
    *out = (size_t)t->dims[1];
    return DTL_OK;
  }
  return DTL_ERR_MISSING_METADATA;
}

bool needs_q8a(const DevMat& m) {
  return m.type == GGML_Q8_0 || m.type == GGML_Q4_0 || m.type == GGML_Q4_K;
}

}  // namespace

namespace {

// Exact f32 copies of the Q4_K matrices the forward multiplies (the values
// q4_k_value computes), used by the chunked-encode GEMM.  Skipped when the
// device lacks room for them or DETLLM_NO_F32_MIRROR is set; the packed
// kernels then serve every chunk size.
// Copies the chunked-encode GEMMs read instead of the GGUF blocks: the
// exact f32 value of every Q4_K weight, the int8 matrix-core planes of
// every Q6_K matrix and the int8 values of every Q4_0 matrix; and the
// decode GEMV's layout of tall Q6_K matrices (the output projection).  DETLLM_NO_F32_MIRROR=1 keeps Q4_K packed only and
// DETLLM_NO_Q6K_PLANES=1 keeps Q6_K packed only (the GEMMs then decode the
// superblocks themselves; results are identical either way).
bool env_flag(const char* name) {
  const char* v = getenv(name);
  return v && *v && *v != '0';
}
bool f32_mirror_enabled() { return !env_flag("DETLLM_NO_F32_MIRROR"); }
bool q6k_planes_enabled() { return !env_flag("DETLLM_NO_Q6K_PLANES"); }

int build_encode_copies(dtl_model* m) {
  std::vector<DevMat*> q4k, q6k, q40, q6d;
  auto add = [&](DevMat* M) {
    if (M->type == GGML_Q4_K && f32_mirror_enabled()) q4k.push_back(M);
    if (M->type == GGML_Q6_K && q6k_planes_enabled()) q6k.push_back(M);
    if (M->type == GGML_Q4_0) q40.push_back(M);
    if (M->type == GGML_Q6_K && q6k_decode_layout_applies(*M)) q6d.push_back(M);
  };
  for (Layer& L : m->layers)
    for (DevMat* M : {&L.wq, &L.wk, &L.wv, &L.wo, &L.gate, &L.up, &L.down}) add(M);
  add(&m->out);
  size_t need = 0;
  for (DevMat* M : q4k) need += (size_t)M->rows * M->cols * sizeof(float);
  for (DevMat* M : q6k) need += q6k_planes_bytes(*M);
  for (DevMat* M : q40) need += (size_t)M->rows * M->cols;
  // the decode layouts are not optional copies: always built
  for (DevMat* M : q6d) {
    uint4* p;
    int st = m->arena.alloc(&p, q6k_decode_layout_bytes(*M) / sizeof(uint4));
    if (st) return st;
    launch_q6k_decode_layout(*M, p, nullptr);
    M->q6d = p;
  }
  if (q4k.empty() && q6k.empty() && q40.empty()) {
    HIP_TRY(hipGetLastError());
    HIP_TRY(hipDeviceSynchronize());
    return DTL_OK;
  }
  size_t free_b = 0, total_b = 0;
  HIP_TRY(hipMemGetInfo(&free_b, &total_b));
  if (need + (size_t(4) << 30) > free_b) return DTL_OK;
  for (DevMat* M : q4k) {
    float* w;
    int st = m->arena.alloc(&w, (size_t)M->rows * M->cols);
    if (st) return st;
    launch_dequant_q4k(*M, w, nullptr);
    M->w32 = w;
  }
  for (DevMat* M : q6k) {
    int8_t* p;
    int st = m->arena.alloc(&p, q6k_planes_bytes(*M));
    if (st) return st;
    launch_q6k_planes(*M, p, nullptr);
    M->planes = p;
  }
  for (DevMat* M : q40) {
    int8_t* p;
    int st = m->arena.alloc(&p, (size_t)M->rows * M->cols);
    if (st) return st;
    launch_q4_0_i8(*M, p, nullptr);
    M->i8 = p;
  }
  HIP_TRY(hipGetLastError());
  HIP_TRY(hipDeviceSynchronize());
  return DTL_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// session

namespace {

}  // namespace

thread_local dtl::LaunchTiming* dtl::tl_timing = nullptr;

namespace {

// Timing of every launch on the session stream, grouped by kernel class:
// the events are bound to the kernels themselves (first start .. last end).
class Profiler {
 public:
  bool on = false;

  ~Profiler() {
    for (hipEvent_t e : pool_) (void)hipEventDestroy(e);
  }
  void enable(bool v) {
    on = v;
    only_.clear();
    stats_.clear();
    pending_.clear();
    next_ = 0;
  }
  // Time only launches of this class (empty: every class).
  void only(const char* name) { only_ = name ? name : ""; }
  // Records one launch: `launch` is called between two events.
  template <typename F>
  void timed(hipStream_t s, const char* name, double bytes, double macs, F&& launch) {
    if (!on || (!only_.empty() && only_ != name)) {
      launch();
      return;
    }
    (void)s;
    LaunchTiming lt{take(), take(), false};
    tl_timing = &lt;
    launch();
    tl_timing = nullptr;
    if (lt.launched) pending_.push_back({name, lt.start, lt.stop, bytes, macs});
  }
  // Called after the stream has been synchronised.
  void collect() {
    for (const Pending& p : pending_) {
      float ms = 0.0f;
      (void)hipEventElapsedTime(&ms, p.a, p.b);
      dtl_kernel_stat* st = find(p.name);
      st->launches += 1;
      st->total_ms += ms;
      st->bytes += p.bytes;
      st->macs += p.macs;
    }
    pending_.clear();
    next_ = 0;
  }
  const std::vector<dtl_kernel_stat>& stats() const { return stats_; }

 private:
  struct Pending {
    const char* name;
    hipEvent_t a, b;
    double bytes, macs;
  };
  hipEvent_t take() {
    if (next_ == pool_.size()) {
      hipEvent_t e;
      (void)hipEventCreate(&e);
      pool_.push_back(e);
    }
    return pool_[next_++];
  }
  dtl_kernel_stat* find(const char* name) {
    for (auto& s : stats_)
      if (std::strcmp(s.name, name) == 0) return &s;
    dtl_kernel_stat s{};
    std::snprintf(s.name, sizeof s.name, "%s", name);
    stats_.push_back(s);
    return &stats_.back();
  }
  std::string only_;
  std::vector<hipEvent_t> pool_;
  size_t next_ = 0;
  std::vector<Pending> pending_;
  std::vector<dtl_kernel_stat> stats_;
};

// Algorithmic bytes per weight element, as stored in GGUF.
double weight_bytes_per_elem(int type) {
  switch (type) {
    case GGML_F32: return 4.0;
    case GGML_Q8_0: return 34.0 / 32.0;
    case GGML_Q4_0: return 18.0 / 32.0;
    case GGML_Q4_K: return 144.0 / 256.0;
    case GGML_Q6_K: return 210.0 / 256.0;
  }
  return 0.0;
}

const char* gemm_class(int type) {
  switch (type) {
    case GGML_F32: return "gemm_f32";
    case GGML_Q8_0: return "gemm_q8_0";
    case GGML_Q4_0: return "gemm_q4_0";
    case GGML_Q4_K: return "gemm_q4_k";
    case GGML_Q6_K: return "gemm_q6_k";
  }
  return "gemm";
}

// The output projection (lm_head) is timed as its own class: it is the one
// large matrix of a decode step.
const char* lm_head_class(int type) {
  switch (type) {
    case GGML_F32: return "lm_head_f32";
    case GGML_Q8_0: return "lm_head_q8_0";
    case GGML_Q4_0: return "lm_head_q4_0";
    case GGML_Q4_K: return "lm_head_q4_k";
    case GGML_Q6_K: return "lm_head_q6_k";
  }
  return "lm_head";
}

}  // namespace

// The buffers of one chunk in flight: activations, logits, the CDF staging,
// the error flag and the stream its launches go to.  A session has 3 or 4 of
// them, so the pipelined encode (dtl_forward_ranges) runs the next chunks
// beside chunk c; every other entry point works on lane 0.
// Measured on MI355X for the 64-position encode: with HIP's default of four
// hardware queues per process three lanes (14.6k tokens/s; four lanes make
// two streams share a queue: 13.0k); with GPU_MAX_HW_QUEUES=8 four lanes
// (15.2k; five: 14.1k).  A session takes four lanes when the process has at
// least five queues, else three; DETLLM_LANES (1-4) overrides.
constexpr int kMaxLanes = 4;

static int lane_count() {
  if (const char* l = getenv("DETLLM_LANES")) {
    const int n = atoi(l);
    if (n >= 1 && n <= kMaxLanes) return n;
  }
  const char* e = getenv("GPU_MAX_HW_QUEUES");
  const int queues = e && *e ? atoi(e) : 4;
  return queues >= 5 ? 4 : 3;
}

struct Lane {
  hipStream_t stream = nullptr;
  float *x = nullptr, *h = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *attn = nullptr;
  float *g = nullptr, *u = nullptr, *ffo = nullptr, *logits = nullptr, *scores = nullptr;
  int8_t *qa = nullptr, *qk = nullptr;
  float *da = nullptr, *af = nullptr, *dk = nullptr;
  uint32_t* tokens = nullptr;
  int* err = nullptr;
  // CDF staging
  uint32_t *c_sym = nullptr, *c_freq = nullptr, *c_freq_tab = nullptr;
  uint64_t *c_cum = nullptr, *c_total = nullptr, *c_values = nullptr, *c_cum_tab = nullptr;
  uint64_t* c_pack = nullptr;  // a decoder call's results and error bits, for one copy out
  uint8_t* c_scratch = nullptr;  // multi-workgroup CDF scratch for max_chunk rows
  uint32_t* c_rows = nullptr;    // row index per symbol (dtl_symbol_ranges_rows)
  // Row / tail whose decoder-total block results the scratch still holds.
  size_t cdf_ready_row = SIZE_MAX, cdf_ready_tail = SIZE_MAX;
  size_t rows_valid = 0;  // rows of `logits` written by the last forward
  // Per layer: recorded once this lane's chunk has stored its K/V rows
  // (pipelined encode only).
  std::vector<hipEvent_t> kv_ready;
  // Pinned host staging of the pipelined encode: token ids, symbol rows and
  // symbols in; ranges and the error flag out.
  uint32_t *h_tokens = nullptr, *h_rows = nullptr, *h_sym = nullptr, *h_freq = nullptr;
  uint64_t *h_cum = nullptr, *h_total = nullptr;
  int* h_err = nullptr;
  size_t h_cap = 0;  // symbols the h_rows .. h_total staging holds
  // Pinned staging of the decoder entry points (value in, results out), so
  // that their copies are plain DMA rather than staged pageable copies.
  uint64_t* h_io = nullptr;
};

// Grows a lane's pinned symbol staging to n symbols (the lane must be idle).
static int lane_reserve(Lane& L, size_t n) {
  if (n <= L.h_cap) return DTL_OK;
  for (void* p : {(void*)L.h_rows, (void*)L.h_sym, (void*)L.h_freq, (void*)L.h_cum, (void*)L.h_total})
    if (p) (void)hipHostFree(p);
  L.h_rows = L.h_sym = L.h_freq = nullptr;
  L.h_cum = L.h_total = nullptr;
  L.h_cap = 0;
  HIP_TRY(hipHostMalloc((void**)&L.h_rows, n * 4, hipHostMallocDefault));
  HIP_TRY(hipHostMalloc((void**)&L.h_sym, n * 4, hipHostMallocDefault));
  HIP_TRY(hipHostMalloc((void**)&L.h_freq, n * 4, hipHostMallocDefault));
  HIP_TRY(hipHostMalloc((void**)&L.h_cum, n * 8, hipHostMallocDefault));
  HIP_TRY(hipHostMalloc((void**)&L.h_total, n * 8, hipHostMallocDefault));
  L.h_cap = n;
  return DTL_OK;
}

struct dtl_session {
  const dtl_model* m = nullptr;
  size_t n_ctx = 0, max_chunk = 0, max_in = 0;
  Arena arena;
  float *rope_cos = nullptr, *rope_sin = nullptr, *kc = nullptr, *vc = nullptr;
  Lane lanes[kMaxLanes];
  int nlanes = 1;        // lanes set up (the rest stay empty)
  Lane* ln = &lanes[0];  // the lane the launches below go to
  // Captured single-position forwards (see forward_device), on lane 0:
  // [0] for rows up to attention_fused_max_len() keys, [1] for the whole
  // window.  graph_maxlen: the row bound of the graph being captured.
  hipGraphExec_t graph[2] = {nullptr, nullptr};
  int graph_maxlen = 0;
  bool graph_failed = false;
  bool overlapped = false;  // dtl_forward_ranges has chunks in flight on several lanes
  int* pos_dev = nullptr;   // device copy of the position for the graph
  int* pos_host = nullptr;  // pinned staging for it
  Profiler prof;
  ~dtl_session() {
    for (Lane& L : lanes) {
      if (L.stream) {
        (void)hipStreamSynchronize(L.stream);
        (void)hipStreamDestroy(L.stream);
      }
      for (hipEvent_t e : L.kv_ready)
        if (e) (void)hipEventDestroy(e);
      for (void* p : {(void*)L.h_tokens, (void*)L.h_rows, (void*)L.h_sym, (void*)L.h_freq,
                      (void*)L.h_cum, (void*)L.h_total, (void*)L.h_err, (void*)L.h_io})
        if (p) (void)hipHostFree(p);
    }
    for (hipGraphExec_t g : graph)
      if (g) (void)hipGraphExecDestroy(g);
    if (pos_host) (void)hipHostFree(pos_host);
  }
};

namespace {

size_t max_input_width(const dtl_model* m) {
  size_t w = m->c.d;
  if (m->c.ff > w) w = m->c.ff;
  if (m->c.heads * m->head_dim > w) w = m->c.heads * m->head_dim;
  return w;
}

int read_err(dtl_session* s, int* bits) {
  HIP_TRY(hipMemcpyAsync(s->ln->h_err, s->ln->err, sizeof(int), hipMemcpyDeviceToHost, s->ln->stream));
  HIP_TRY(hipStreamSynchronize(s->ln->stream));
  *bits = *s->ln->h_err;
  return DTL_OK;
}

__global__ void k_clear_flag(int* p) { *p = 0; }

// The decoder entry points' results in one buffer: symbol, cum, freq, total
// (absent ones 0) and the error bits.
__global__ void k_pack_decoder(const uint32_t* sym, const uint64_t* cum, const uint32_t* freq,
                               const uint64_t* total, const int* err, uint64_t* out) {
  out[0] = sym ? sym[0] : 0;
  out[1] = cum ? cum[0] : 0;
  out[2] = freq ? freq[0] : 0;
  out[3] = total[0];
  out[4] = (uint64_t)(uint32_t)err[0];
}

// Packs, copies to the lane's pinned staging (h_io[2..6]) and waits.
int read_decoder(dtl_session* s, const uint32_t* sym, const uint64_t* cum, const uint32_t* freq,
                 int* bits) {
  Lane& L = *s->ln;
  launch_kernel(k_pack_decoder, dim3(1), dim3(1), 0, L.stream, sym, cum, freq, L.c_total, L.err, L.c_pack);
  HIP_TRY(hipMemcpyAsync(L.h_io + 2, L.c_pack, 5 * sizeof(uint64_t), hipMemcpyDeviceToHost, L.stream));
  HIP_TRY(hipStreamSynchronize(L.stream));
  *bits = (int)(uint32_t)L.h_io[6];
  return DTL_OK;
}

void clear_err(dtl_session* s) { launch_kernel(k_clear_flag, dim3(1), dim3(1), 0, s->ln->stream, s->ln->err); }

// Which activation forms the given consumers need.
void needed_forms(std::initializer_list<const DevMat*> consumers, bool* q8a, bool* q8k) {
  *q8a = *q8k = false;
  for (const DevMat* m : consumers) {
    if (needs_q8a(*m)) *q8a = true;
    if (m->type == GGML_Q6_K) *q8k = true;
  }
}

// Bytes the quantisation writes per element (Q8A: quant, dequantised f32
// and a scale per 32; Q8_K: quant and a scale per 256).
double quant_bytes(bool q8a, bool q8k) {
  return (q8a ? 1.0 + 4.0 / 32 + 4.0 : 0.0) + (q8k ? 1.0 + 4.0 / 256 : 0.0);
}

DevAct session_act(dtl_session* s, const float* x) {
  DevAct a{};
  a.x = x;
  a.qa = s->ln->qa;
  a.da = s->ln->da;
  a.af = s->ln->af;
  a.qk = s->ln->qk;
  a.dk = s->ln->dk;
  a.overlapped = s->overlapped;
  return a;
}

// Produces the activation forms the given consumers need from x[T][n].
DevAct prepare_input(dtl_session* s, const float* x, int T, int n,
                     std::initializer_list<const DevMat*> consumers) {
  bool q8a, q8k;
  needed_forms(consumers, &q8a, &q8k);
  if (q8a || q8k) {
    double bytes = (double)T * n * (4.0 + quant_bytes(q8a, q8k));
    s->prof.timed(s->ln->stream, "quantize", bytes, 0.0, [&] {
      launch_quantize(x, T, n, q8a, q8k, s->ln->qa, s->ln->da, s->ln->af, s->ln->qk, s->ln->dk, s->ln->err, s->ln->stream);
    });
  }
  return session_act(s, x);
}

// forward_one_with_workspace (det-model lib.rs:1249-1400) for the T
// positions whose token ids are in the current lane's tokens: enqueues
// every launch on the lane's stream (no host synchronisation).  pos_dev:
// when set, the position-dependent kernels read pos0 from that device int.
// after: a lane whose chunk (the positions just before these) is still in
// flight; each layer's attention waits for that lane's kv_ready event of the
// layer.  record_kv: record this lane's kv_ready event of each layer once
// its rows are stored and the wait above has passed, so the event covers
// the rows of every earlier chunk too (the chain of lanes is transitive).
int enqueue_forward(dtl_session* s, int T, size_t pos0, const int* pos_dev,
                    const Lane* after = nullptr, bool record_kv = false) {
  const dtl_model* m = s->m;
  const HostConfig& c = m->c;
  hipStream_t st = s->ln->stream;
  clear_err(s);
  int d = (int)c.d, ff = (int)c.ff, H = (int)c.heads, KV = (int)c.kv_heads;
  int hd = (int)m->head_dim;
  Profiler& P = s->prof;
  // Algorithmic traffic of one GEMM: weights once, quantised activations
  // and f32 outputs per position (the residual epilogue also reads x).
  // Q4_K decode GEMV from the raw f32 input, residual epilogue.
  auto q4k_gemv_bytes = [&](const DevMat& W, int Tn, bool residual) {
    return (double)W.rows * W.cols * weight_bytes_per_elem(GGML_Q4_K) + (double)Tn * W.cols * 4.0 +
           (double)Tn * W.rows * (residual ? 8.0 : 4.0);
  };
  auto gemm = [&](const DevMat& W, const DevAct& a, float* out, const float* bias, int epi,
                  const char* cls) {
    double act = W.type == GGML_F32 ? 4.0 : (W.type == GGML_Q6_K ? 1.0 + 4.0 / 256 : 1.0 + 4.0 / 32);
    double bytes = (double)W.rows * W.cols * weight_bytes_per_elem(W.type) +
                   (double)T * W.cols * act + (double)T * W.rows * (epi == EPI_RESIDUAL ? 8.0 : 4.0);
    P.timed(st, cls ? cls : gemm_class(W.type), bytes, (double)W.rows * W.cols * T,
            [&] { launch_gemm(W, a, T, out, bias, epi, s->ln->err, st); });
  };
  // rmsnorm of the residual stream into h, fused with the quantisation the
  // consumers of h need.
  auto rms = [&](const float* w, std::initializer_list<const DevMat*> consumers) {
    bool q8a, q8k;
    needed_forms(consumers, &q8a, &q8k);
    P.timed(st, "rmsnorm_quantize", (double)T * d * (8.0 + quant_bytes(q8a, q8k)) + d * 4.0, 0.0,
            [&] {
              launch_rmsnorm_quant(s->ln->x, w, c.eps, T, d, s->ln->h, q8a, q8k, s->ln->qa, s->ln->da, s->ln->af,
                                   s->ln->qk, s->ln->dk, s->ln->err, st);
            });
    return session_act(s, s->ln->h);
  };
  P.timed(st, "embed", (double)T * d * (4.0 + weight_bytes_per_elem(m->emb.type)), 0.0,
          [&] { launch_embed(m->emb, s->ln->tokens, T, s->ln->x, s->ln->err, st); });
  // K and V rows read by one layer's attention over the chunk (GQA heads
  // of one group share them), and its multiply-accumulates.
  double kv_rows = 0.0;
  for (int t = 0; t < T; t++) kv_rows += (double)(pos0 + t + 1);
  // Decode shapes with Q8_0 / Q4_0 weights fold the rmsnorm and the
  // activation quantisation into the GEMV launches (each workgroup forms
  // the Q8A activations it needs), q/k/v share one launch, and gate/up
  // finish as swiglu in theirs.
  const bool fuse = T <= kGemvMaxT && !env_flag("DETLLM_NO_FUSED_DECODE");
  auto fused = [&](std::initializer_list<const DevMat*> ms, bool pair, std::initializer_list<float*> outs,
                   std::initializer_list<const float*> biases, std::initializer_list<int> epis,
                   const float* x, const float* norm_w, const char* cls, int8_t* out_qa = nullptr,
                   float* out_da = nullptr) {
    const DevMat* mv[3];
    float* ov[3];
    const float* bv[3];
    int ev[3];
    int nm = 0;
    double bytes = 0.0, macs = 0.0;
    for (const DevMat* mm : ms) {
      mv[nm++] = mm;
      bytes += (double)mm->rows * mm->cols * weight_bytes_per_elem(mm->type);
      macs += (double)mm->rows * mm->cols * T;
    }
    int i = 0;
    for (float* o : outs) ov[i++] = o;
    i = 0;
    for (const float* b : biases) bv[i++] = b;
    i = 0;
    for (int e : epis) ev[i++] = e;
    const int rows_out = pair ? mv[0]->rows : (int)(macs / T / mv[0]->cols);
    bytes += (double)T * mv[0]->cols * 4.0 + (double)T * rows_out * 4.0;
    FusedIn in{x, norm_w, c.eps, out_qa, out_da};
    P.timed(st, cls, bytes, macs,
            [&] { (void)launch_gemv_fused(mv, nm, pair, ov, bv, ev, in, T, s->ln->err, st); });
  };
  auto fits = [&](std::initializer_list<const DevMat*> ms, bool pair, bool norm) {
    const DevMat* mv[3];
    int nm = 0;
    for (const DevMat* mm : ms) mv[nm++] = mm;
    return fuse && gemv_fused_fits(mv, nm, pair, norm, T);
  };
  for (size_t l = 0; l < c.block_count; l++) {
    const Layer& L = m->layers[l];
    const int e_q = L.bq ? EPI_BIAS : EPI_STORE, e_k = L.bk ? EPI_BIAS : EPI_STORE;
    const int e_v = L.bv ? EPI_BIAS : EPI_STORE;
    DevAct a{};
    bool attn_quantized = false;
    if (fits({&L.wq, &L.wk, &L.wv}, false, true)) {
      fused({&L.wq, &L.wk, &L.wv}, false, {s->ln->q, s->ln->k, s->ln->v}, {L.bq, L.bk, L.bv}, {e_q, e_k, e_v},
            s->ln->x, L.attn_norm, "gemv_fused_qkv");
    } else if (fits({&L.wq}, false, true) && fits({&L.wk}, false, true) &&
               fits({&L.wv}, false, true)) {
      fused({&L.wq}, false, {s->ln->q}, {L.bq}, {e_q}, s->ln->x, L.attn_norm, "gemv_fused_qkv");
      fused({&L.wk}, false, {s->ln->k}, {L.bk}, {e_k}, s->ln->x, L.attn_norm, "gemv_fused_qkv");
      fused({&L.wv}, false, {s->ln->v}, {L.bv}, {e_v}, s->ln->x, L.attn_norm, "gemv_fused_qkv");
    } else if (gemv_q4k_fit(L.wq, &L.wk, false, true, T, &L.wv)) {
      // decode: the attention rmsnorm, its Q8A and Q8_K forms, wq+wk and
      // wv (Q6_K, its rows on the workgroups' spare waves) in one launch
      double bytes = (double)(L.wq.rows + L.wk.rows) * L.wq.cols * weight_bytes_per_elem(GGML_Q4_K) +
                     (double)L.wv.rows * L.wv.cols * weight_bytes_per_elem(L.wv.type) +
                     (double)T * d * 4.0 + (double)d * 4.0 +
                     (double)T * (L.wq.rows + L.wk.rows + L.wv.rows) * 4.0;
      Q4kIn in{nullptr, s->ln->x, L.attn_norm, c.eps};
      in.v6 = &L.wv;
      in.v6out = s->ln->v;
      in.v6bias = L.bv;
      in.v6epi = e_v;
      P.timed(st, "gemv_q4_k_qkv", bytes, (double)(L.wq.rows + L.wk.rows + L.wv.rows) * L.wq.cols * T, [&] {
        launch_gemv_q4k(L.wq, &L.wk, false, in, T, s->ln->q, s->ln->k, L.bq, L.bk, e_q, e_k, s->ln->err, st);
      });
    } else if (L.wv.type == GGML_Q6_K && gemv_q4k_fit(L.wq, &L.wk, false, true, T)) {
      // decode: the attention rmsnorm and its quantisation inside the
      // wq+wk launch, whose first workgroup also writes the Q8_K form wv reads
      double bytes = (double)(L.wq.rows + L.wk.rows) * L.wq.cols * weight_bytes_per_elem(GGML_Q4_K) +
                     (double)T * d * 4.0 + (double)d * 4.0 + (double)T * (L.wq.rows + L.wk.rows) * 4.0;
      P.timed(st, "gemv_q4_k_qk", bytes, (double)(L.wq.rows + L.wk.rows) * L.wq.cols * T, [&] {
        launch_gemv_q4k(L.wq, &L.wk, false, Q4kIn{nullptr, s->ln->x, L.attn_norm, c.eps, s->ln->qk, s->ln->dk},
                        T, s->ln->q, s->ln->k, L.bq, L.bk, e_q, e_k, s->ln->err, st);
      });
      gemm(L.wv, session_act(s, s->ln->h), s->ln->v, L.bv, e_v, nullptr);
    } else {
      a = rms(L.attn_norm, {&L.wq, &L.wk, &L.wv});
      if (L.wq.type == GGML_Q4_K && L.wk.type == GGML_Q4_K && L.wq.w32 && L.wk.w32 && T >= 16 &&
          (L.bq != nullptr) == (L.bk != nullptr)) {
        // wq and wk share the input: one launch over their concatenated rows.
        double bytes = (double)(L.wq.rows + L.wk.rows) * L.wq.cols * weight_bytes_per_elem(GGML_Q4_K) +
                       (double)T * L.wq.cols * (1.0 + 4.0 / 32) + (double)T * (L.wq.rows + L.wk.rows) * 4.0;
        P.timed(st, "gemm_q4_k_qk", bytes, (double)(L.wq.rows + L.wk.rows) * L.wq.cols * T, [&] {
          launch_gemm_cat_q4k(L.wq, L.wk, a, T, s->ln->q, s->ln->k, L.bq, L.bk, L.bq ? EPI_BIAS : EPI_STORE,
                              s->ln->err, st);
        });
      } else if (gemv_q4k_fit(L.wq, &L.wk, false, false, T)) {
        // decode: the same pair in one GEMV launch
        double bytes = (double)(L.wq.rows + L.wk.rows) * L.wq.cols * weight_bytes_per_elem(GGML_Q4_K) +
                       (double)T * L.wq.cols * 4.0 + (double)T * (L.wq.rows + L.wk.rows) * 4.0;
        P.timed(st, "gemv_q4_k_qk", bytes, (double)(L.wq.rows + L.wk.rows) * L.wq.cols * T, [&] {
          launch_gemv_q4k(L.wq, &L.wk, false, Q4kIn{a.af, nullptr, nullptr, 0.0f}, T, s->ln->q, s->ln->k,
                          L.bq, L.bk, e_q, e_k, s->ln->err, st);
        });
      } else {
        gemm(L.wq, a, s->ln->q, L.bq, L.bq ? EPI_BIAS : EPI_STORE, nullptr);
        gemm(L.wk, a, s->ln->k, L.bk, L.bk ? EPI_BIAS : EPI_STORE, nullptr);
      }
      gemm(L.wv, a, s->ln->v, L.bv, L.bv ? EPI_BIAS : EPI_STORE, nullptr);
    }
    if (attention_dec_applies(hd, T, (int)pos0, (int)s->n_ctx, pos_dev != nullptr)) {
      // RoPE and the cache store happen inside the decode attention.
      if (after) HIP_TRY(hipStreamWaitEvent(st, after->kv_ready[l], 0));
      const RopeIn R{s->ln->k, s->ln->v, s->rope_cos, s->rope_sin, (int)c.rope_dim, c.split_half ? 1 : 0,
                     s->kc, s->vc};
      P.timed(st, "attention_dec", 2.0 * kv_rows * KV * hd * 4.0 + (double)T * (2 * H + 3 * KV) * hd * 4.0,
              2.0 * kv_rows * H * hd, [&] {
                launch_attention_dec(s->ln->q, R, (int)l, T, (int)pos0, H, KV, (int)s->n_ctx,
                                     s->graph_maxlen, c.attention_scale, s->ln->scores, s->ln->attn,
                                     pos_dev, s->ln->err, st);
              });
      if (record_kv) HIP_TRY(hipEventRecord(s->ln->kv_ready[l], st));
    } else {
      P.timed(st, "rope_store", (double)T * (H + 3 * KV) * hd * 8.0, 0.0, [&] {
        launch_rope_store(s->ln->q, s->ln->k, s->ln->v, s->rope_cos, s->rope_sin, T, (int)pos0, H, KV, hd,
                          (int)c.rope_dim, c.split_half, s->kc, s->vc, (int)l, (int)s->n_ctx,
                          pos_dev, s->ln->err, st);
      });
      // The store above writes only this chunk's rows; the attention below
      // also reads the earlier chunks'.  The event is recorded after the
      // wait, so it marks every chunk's rows up to this one as stored.
      if (after) HIP_TRY(hipStreamWaitEvent(st, after->kv_ready[l], 0));
      if (record_kv) HIP_TRY(hipEventRecord(s->ln->kv_ready[l], st));
      // The chunked attention also writes the Q8A form wo reads, when that
      // is the only form wo needs.
      bool q8a, q8k;
      needed_forms({&L.wo}, &q8a, &q8k);
      attn_quantized = q8a && !q8k && !fits({&L.wo}, false, false) &&
                       attention_quantizes_q8a(hd, H, KV, T, (int)pos0, (int)s->n_ctx);
      P.timed(st, "attention", kv_rows * KV * hd * 8.0 + (double)T * H * hd * 8.0,
              kv_rows * H * hd * 2.0, [&] {
                launch_attention(s->ln->q, s->kc, s->vc, (int)l, T, (int)pos0, H, KV, hd,
                                 (int)s->n_ctx, c.attention_scale, s->ln->scores, s->ln->attn, s->ln->err, st,
                                 attn_quantized ? s->ln->qa : nullptr,
                                 attn_quantized ? s->ln->da : nullptr,
                                 attn_quantized ? s->ln->af : nullptr);
              });
    }
    if (fits({&L.wo}, false, false)) {
      fused({&L.wo}, false, {s->ln->x}, {nullptr}, {EPI_RESIDUAL}, s->ln->attn, nullptr, "gemv_fused_o");
    } else if (!attn_quantized && gemv_q4k_fit(L.wo, nullptr, false, true, T)) {
      // decode: the attention output's quantisation inside the wo launch
      P.timed(st, "gemv_q4_k_o", q4k_gemv_bytes(L.wo, T, true), (double)L.wo.rows * L.wo.cols * T, [&] {
        launch_gemv_q4k(L.wo, nullptr, false, Q4kIn{nullptr, s->ln->attn, nullptr, 0.0f}, T, s->ln->x,
                        nullptr, nullptr, nullptr, EPI_RESIDUAL, 0, s->ln->err, st);
      });
    } else {
      a = attn_quantized ? session_act(s, s->ln->attn) : prepare_input(s, s->ln->attn, T, H * hd, {&L.wo});
      gemm(L.wo, a, s->ln->x, nullptr, EPI_RESIDUAL, nullptr);
    }
    // When down is a fused-shape Q8_0 / Q4_0 GEMV too, the gate/up launch
    // also writes the Q8A form of its output, so down reads it directly.
    bool down_input_quantized = false;
    if (fits({&L.gate, &L.up}, true, true)) {
      down_input_quantized = fits({&L.down}, false, false) && needs_q8a(L.down) &&
                             gemv_fused_pair_quantizes(L.gate, L.up, true, T);
      fused({&L.gate, &L.up}, true, {s->ln->ffo}, {nullptr, nullptr}, {EPI_STORE, EPI_STORE}, s->ln->x,
            L.ffn_norm, "gemv_fused_gate_up", down_input_quantized ? s->ln->qa : nullptr,
            down_input_quantized ? s->ln->da : nullptr);
    } else if (fits({&L.gate}, false, true) && fits({&L.up}, false, true)) {
      fused({&L.gate}, false, {s->ln->g}, {nullptr}, {EPI_STORE}, s->ln->x, L.ffn_norm, "gemv_fused_gate_up");
      fused({&L.up}, false, {s->ln->u}, {nullptr}, {EPI_STORE}, s->ln->x, L.ffn_norm, "gemv_fused_gate_up");
      P.timed(st, "swiglu", (double)T * ff * 12.0, 0.0,
              [&] { launch_swiglu(s->ln->g, s->ln->u, T * ff, s->ln->ffo, s->ln->err, st); });
    } else if (gemv_q4k_fit(L.gate, &L.up, true, true, T)) {
      // decode: the FFN rmsnorm, its quantisation, gate, up and swiglu in one launch
      double bytes = 2.0 * L.gate.rows * L.gate.cols * weight_bytes_per_elem(GGML_Q4_K) +
                     (double)T * d * 4.0 + (double)d * 4.0 + (double)T * ff * 4.0;
      P.timed(st, "gemv_q4_k_gate_up", bytes, 2.0 * L.gate.rows * L.gate.cols * T, [&] {
        launch_gemv_q4k(L.gate, &L.up, true, Q4kIn{nullptr, s->ln->x, L.ffn_norm, c.eps}, T, s->ln->ffo,
                        nullptr, nullptr, nullptr, EPI_STORE, EPI_STORE, s->ln->err, st);
      });
    } else {
      a = rms(L.ffn_norm, {&L.gate, &L.up});
      if (T >= 16 && L.gate.type == GGML_Q4_K && L.up.type == GGML_Q4_K &&
          L.gate.rows == L.up.rows && L.gate.cols == L.up.cols) {
        // gate, up and swiglu in one pass: both chains of a row share one wave.
        double bytes = 2.0 * L.gate.rows * L.gate.cols * weight_bytes_per_elem(GGML_Q4_K) +
                       (double)T * d * (1.0 + 4.0 / 32) + (double)T * ff * 4.0;
        P.timed(st, "gemm_q4_k_gate_up", bytes, 2.0 * L.gate.rows * L.gate.cols * T, [&] {
          launch_gemm_pair_swiglu_q4k(L.gate, L.up, a, T, nullptr, nullptr, s->ln->ffo, s->ln->err, st);
        });
      } else {
        gemm(L.gate, a, s->ln->g, nullptr, EPI_STORE, nullptr);
        gemm(L.up, a, s->ln->u, nullptr, EPI_STORE, nullptr);
        P.timed(st, "swiglu", (double)T * ff * 12.0, 0.0,
                [&] { launch_swiglu(s->ln->g, s->ln->u, T * ff, s->ln->ffo, s->ln->err, st); });
      }
    }
    if (down_input_quantized) {
      gemm(L.down, session_act(s, s->ln->ffo), s->ln->x, nullptr, EPI_RESIDUAL, "gemv_down");
    } else if (fits({&L.down}, false, false)) {
      fused({&L.down}, false, {s->ln->x}, {nullptr}, {EPI_RESIDUAL}, s->ln->ffo, nullptr, "gemv_fused_down");
    } else if (gemv_q4k_fit(L.down, nullptr, false, true, T)) {
      // decode: the FFN product's quantisation inside the down launch
      P.timed(st, "gemv_q4_k_down", q4k_gemv_bytes(L.down, T, true), (double)L.down.rows * L.down.cols * T, [&] {
        launch_gemv_q4k(L.down, nullptr, false, Q4kIn{nullptr, s->ln->ffo, nullptr, 0.0f}, T, s->ln->x,
                        nullptr, nullptr, nullptr, EPI_RESIDUAL, 0, s->ln->err, st);
      });
    } else {
      a = prepare_input(s, s->ln->ffo, T, ff, {&L.down});
      gemm(L.down, a, s->ln->x, nullptr, EPI_RESIDUAL, nullptr);
    }
  }
  DevAct a = rms(m->out_norm, {&m->out});
  gemm(m->out, a, s->ln->logits, nullptr, EPI_STORE, lm_head_class(m->out.type));
  HIP_TRY(hipGetLastError());
  return DTL_OK;
}

// Single-position forwards replay a captured graph of the whole pass, one
// for positions whose rows fit the one-launch decode attention and one for
// the rest of the window: the position reaches the kernels through
// s->pos_dev, copied in before each replay.  DETLLM_NO_GRAPH=1 keeps the
// eager launches.
bool graph_eligible(const dtl_session* s) {
  return !s->prof.on && !s->graph_failed && !env_flag("DETLLM_NO_GRAPH") &&
         attention_pos_dev_supported((int)s->m->head_dim, 1, (int)s->n_ctx);
}

// The replayed forward of regime k serves positions below decode_graph_bound(k).
int decode_graph_bound(const dtl_session* s, int k) {
  const int fused = attention_fused_max_len();
  return k == 0 && (size_t)fused < s->n_ctx ? fused : (int)s->n_ctx;
}

int capture_decode_graph(dtl_session* s, int k) {
  hipStream_t st = s->ln->stream;
  s->graph_maxlen = decode_graph_bound(s, k);
  HIP_TRY(hipStreamBeginCapture(st, hipStreamCaptureModeRelaxed));
  int rc = enqueue_forward(s, 1, 0, s->pos_dev);
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(st, &g);
  if (rc == DTL_OK && e == hipSuccess && g)
    e = hipGraphInstantiate(&s->graph[k], g, nullptr, nullptr, 0);
  if (g) (void)hipGraphDestroy(g);
  if (rc != DTL_OK || e != hipSuccess) {
    (void)hipGetLastError();
    s->graph[k] = nullptr;
    s->graph_failed = true;
    return DTL_ERR_DEVICE;
  }
  return DTL_OK;
}

// check: wait for the forward and report its non-finite check here; without
// it the caller's next wait reads the error bits (the forward's launches
// clear them first) and sets rows_valid.
int forward_device(dtl_session* s, const uint32_t* tokens_host, int T, size_t pos0, bool check = true) {
  const dtl_model* m = s->m;
  if (T <= 0 || (size_t)T > s->max_chunk || pos0 + (size_t)T > s->n_ctx) return DTL_ERR_SHAPE;
  for (int t = 0; t < T; t++)
    if (tokens_host[t] >= (uint32_t)m->emb.rows) return DTL_ERR_SHAPE;
  hipStream_t st = s->ln->stream;
  HIP_TRY(hipSetDevice(m->device));
  s->ln->rows_valid = 0;
  s->ln->cdf_ready_row = SIZE_MAX;
  HIP_TRY(hipMemcpyAsync(s->ln->tokens, tokens_host, T * sizeof(uint32_t), hipMemcpyHostToDevice, st));
  bool replayed = false;
  if (T == 1 && graph_eligible(s)) {
    const int k = pos0 < (size_t)decode_graph_bound(s, 0) ? 0 : 1;
    if (!s->graph[k]) (void)capture_decode_graph(s, k);
    if (s->graph[k]) {
      *s->pos_host = (int)pos0;
      HIP_TRY(hipMemcpyAsync(s->pos_dev, s->pos_host, sizeof(int), hipMemcpyHostToDevice, st));
      HIP_TRY(hipGraphLaunch(s->graph[k], st));
      replayed = true;
    }
  }
  if (!replayed) {
    int rc = enqueue_forward(s, T, pos0, nullptr);
    if (rc) return rc;
  }
  if (!check) return DTL_OK;
  int bits = 0;
  int rc = read_err(s, &bits);
  if (rc) return rc;
  s->prof.collect();
  if (bits & ERRBIT_NON_FINITE) return DTL_ERR_NON_FINITE;
  s->ln->rows_valid = (size_t)T;
  return DTL_OK;
}

int cdf_status(int bits) {
  if (bits & ERRBIT_CDF_NON_FINITE) return DTL_ERR_CDF_NON_FINITE_LOGIT;
  if (bits & ERRBIT_CDF_TOTAL) return DTL_ERR_CDF_TOTAL_TOO_LARGE;
  if (bits & ERRBIT_CDF_LOOKUP) return DTL_ERR_CDF_SYMBOL_OUT_OF_RANGE;
  return DTL_OK;
}

constexpr size_t kMaxSymbols = 1u << 18;

// The decode step's device round trip (dtl_decoder_decode, dtl_forward_decode):
// the CDF of logits row `row` and, on the device, decode_freq's value from
// the decoder's window and its lookup; one copy out, one wait.  Then the
// host's own decode_freq, which must give the device's value, and advance.
// after_forward: the forward of that row was enqueued unchecked just before.
int decode_step(dtl_session* s, size_t row, size_t tail, dtl_range_decoder* dec,
                const dtl_range_decoder_state& ds, uint32_t* symbol, bool after_forward) {
  Lane& L = *s->ln;
  const size_t V = s->m->vocab;
  if (!after_forward) clear_err(s);
  launch_cdf_decode(L.logits + row * V, (int)V, (int)tail, ds.code - ds.low, ds.range, L.c_scratch, L.c_pack,
                    L.err, L.stream);
  uint64_t* io = L.h_io;  // [1] symbol, [2] cum, [3] freq, [4] total, [5] error bits, [6] value, [7] valid
  HIP_TRY(hipMemcpyAsync(io + 1, L.c_pack, 7 * sizeof(uint64_t), hipMemcpyDeviceToHost, L.stream));
  HIP_TRY(hipStreamSynchronize(L.stream));
  s->prof.collect();
  const int bits = (int)(uint32_t)io[5];
  if (after_forward) {
    if (bits & ERRBIT_NON_FINITE) return DTL_ERR_NON_FINITE;
    L.rows_valid = 1;
  }
  // the distribution's own errors, as dtl_decoder_total reports them
  int st = cdf_status(bits & ~ERRBIT_CDF_LOOKUP);
  if (st) return st;
  // the scratch holds this row's block results, as after dtl_decoder_total
  L.cdf_ready_row = row;
  L.cdf_ready_tail = tail;
  const uint64_t total = io[4];
  uint64_t value = 0;
  if ((st = dtl_range_decode_freq(dec, total, &value))) return st;
  if (io[7] != 1 || io[6] != value) return DTL_ERR_DEVICE;  // the device formed another value
  if ((st = cdf_status(bits))) return st;                     // no symbol covers the value
  if ((st = dtl_range_decode_advance(dec, io[2], io[3], total))) return st;
  *symbol = (uint32_t)io[1];
  return DTL_OK;
}

}  // namespace

extern "C" {

const char* dtl_status_string(int status) {
  switch (status) {
    case DTL_OK: return "ok";
    case DTL_ERR_SHAPE: return "shape";
    case DTL_ERR_NON_FINITE: return "non-finite";
    case DTL_ERR_UNSUPPORTED_ARCHITECTURE: return "unsupported architecture";
    case DTL_ERR_UNSUPPORTED_ATTENTION_HEAD_LENGTH: return "unsupported attention head length";
    case DTL_ERR_UNSUPPORTED_MODEL_FEATURE: return "unsupported model feature";
    case DTL_ERR_UNSUPPORTED_ROPE_SCALING: return "unsupported rope scaling";
    case DTL_ERR_MISSING_METADATA: return "missing metadata";
    case DTL_ERR_GGUF: return "gguf";
    case DTL_ERR_UNSUPPORTED_TENSOR_TYPE: return "unsupported tensor type";
    case DTL_ERR_THREAD_PANICKED: return "thread panicked";
    case DTL_ERR_CDF_EMPTY: return "cdf: empty";
    case DTL_ERR_CDF_MALFORMED: return "cdf: malformed";
    case DTL_ERR_CDF_NON_FINITE_LOGIT: return "cdf: non-finite logit";
    case DTL_ERR_CDF_SYMBOL_OUT_OF_RANGE: return "cdf: symbol out of range";
    case DTL_ERR_CDF_TOO_MANY_SYMBOLS: return "cdf: too many symbols";
    case DTL_ERR_CDF_TOTAL_TOO_LARGE: return "cdf: total too large";
    case DTL_ERR_RANGE_INVALID_FREQUENCY: return "range: invalid frequency";
    case DTL_ERR_RANGE_UNEXPECTED_EOF: return "range: unexpected eof";
    case DTL_ERR_DEVICE: return "device error";
    case DTL_ERR_OUT_OF_MEMORY: return "device out of memory";
    case DTL_ERR_INVALID_ARGUMENT: return "invalid argument";
    case DTL_ERR_NO_DEVICE: return "no HIP device";
    case DTL_ERR_BUFFER_TOO_SMALL: return "output buffer too small";
    case DTL_ERR_STATIC_SCRATCH_LIMIT: return "call exceeds the static scratch (rows <= 8, vocab + tail <= 2^18)";
    case DTL_ERR_TOKEN_MISSING_BYTE_FALLBACK: return "token: missing byte fallback";
    case DTL_ERR_TOKEN_INVALID_TOKEN: return "token: invalid token";
    case DTL_ERR_TOKEN_MISSING_VOCABULARY: return "token: missing vocabulary";
    case DTL_ERR_TOKEN_MISSING_TOKEN_BYTES: return "token: missing token bytes";
    case DTL_ERR_TOKEN_MISSING_MERGE_TOKEN: return "token: missing merge token";
    case DTL_ERR_TOKEN_INCOMPLETE_BYTE_FALLBACK: return "token: incomplete byte fallback";
    case DTL_ERR_TOKEN_METADATA_TYPE: return "token: metadata type";
    case DTL_ERR_TOKEN_TYPE_LENGTH: return "token: token type length";
    case DTL_ERR_TOKEN_INVALID_TOKEN_TYPE: return "token: invalid token type";
    case DTL_ERR_TOKEN_SCORES_LENGTH: return "token: scores length";
    case DTL_ERR_TOKEN_NON_FINITE_SCORE: return "token: non-finite score";
    case DTL_ERR_TOKEN_INDEX_OVERFLOW: return "token: index overflow";
    case DTL_ERR_TOKEN_DUPLICATE_BYTE_FALLBACK: return "token: duplicate byte fallback";
    case DTL_ERR_TOKEN_DUPLICATE_TOKEN_ID: return "token: duplicate token id";
    case DTL_ERR_TOKEN_DUPLICATE_TOKEN_BYTES: return "token: duplicate token bytes";
    case DTL_ERR_TOKEN_INVALID_MERGE: return "token: invalid merge";
    case DTL_ERR_TOKEN_DUPLICATE_MERGE: return "token: duplicate merge";
    case DTL_ERR_TOKEN_UNSUPPORTED_MODEL: return "token: unsupported tokenizer model";
    case DTL_ERR_FILE_TOO_SHORT: return "dtlz: too short";
    case DTL_ERR_FILE_BAD_MAGIC: return "dtlz: bad magic";
    case DTL_ERR_FILE_UNSUPPORTED_VERSION: return "dtlz: unsupported version";
    case DTL_ERR_FILE_UNSUPPORTED_FLAGS: return "dtlz: unsupported flags";
    case DTL_ERR_FILE_INVALID_CONTEXT: return "dtlz: invalid context";
    case DTL_ERR_FILE_INVALID_OVERLAP: return "dtlz: invalid overlap";
    case DTL_ERR_CODEC_MODEL_MISMATCH: return "codec: model SHA-256 does not match the header";
    case DTL_ERR_CODEC_NOT_CANONICAL: return "codec: payload is not the canonical encoding";
    case DTL_ERR_CODEC_ESCAPE_IN_TOKEN_STREAM: return "codec: byte escape in a token-only stream";
    case DTL_ERR_CODEC_VOCAB_MISMATCH: return "codec: tokenizer vocabulary does not match the model";
    default: return "unknown status";
  }
}

int dtl_model_load(const uint8_t* bytes, size_t len, dtl_model** out) {
  if (!bytes || !out) return DTL_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev == 0) return DTL_ERR_NO_DEVICE;
  Gguf g;
  if (g.parse(bytes, len) != GgufError::None) return DTL_ERR_GGUF;
  std::unique_ptr<dtl_model> m(new dtl_model());
  HIP_TRY(hipGetDevice(&m->device));
  int st;
  if ((st = config_from_gguf(g, &m->c))) return st;
  const HostConfig& c = m->c;
  m->head_dim = c.d / c.heads;
  size_t d = c.d, ff = c.ff, hd = m->head_dim;
  size_t vocab;
  if ((st = vocab_size(g, &vocab))) return st;
  if ((st = read_matrix(g, "token_embd.weight", vocab, d, m->arena, &m->emb))) return st;
  m->layers.resize(c.block_count);
  for (size_t l = 0; l < c.block_count; l++) {
    Layer& L = m->layers[l];
    std::string p = "blk." + std::to_string(l) + ".";
    if ((st = read_vector(g, p + "attn_norm.weight", d, m->arena, &L.attn_norm, false))) return st;
    if ((st = read_matrix(g, p + "attn_q.weight", c.heads * hd, d, m->arena, &L.wq))) return st;
    if ((st = read_vector(g, p + "attn_q.bias", c.heads * hd, m->arena, &L.bq, true))) return st;
    if ((st = read_matrix(g, p + "attn_k.weight", c.kv_heads * hd, d, m->arena, &L.wk))) return st;
    if ((st = read_vector(g, p + "attn_k.bias", c.kv_heads * hd, m->arena, &L.bk, true))) return st;
    if ((st = read_matrix(g, p + "attn_v.weight", c.kv_heads * hd, d, m->arena, &L.wv))) return st;
    if ((st = read_vector(g, p + "attn_v.bias", c.kv_heads * hd, m->arena, &L.bv, true))) return st;
    if ((st = read_matrix(g, p + "attn_output.weight", d, c.heads * hd, m->arena, &L.wo))) return st;
    if ((st = read_vector(g, p + "ffn_norm.weight", d, m->arena, &L.ffn_norm, false))) return st;
    if ((st = read_matrix(g, p + "ffn_gate.weight", ff, d, m->arena, &L.gate))) return st;
    if ((st = read_matrix(g, p + "ffn_up.weight", ff, d, m->arena, &L.up))) return st;
    if ((st = read_matrix(g, p + "ffn_down.weight", d, ff, m->arena, &L.down))) return st;
  }
  if ((st = read_vector(g, "output_norm.weight", d, m->arena, &m->out_norm, false))) return st;
  const GgufTensor* t;
  GgufError ge = g.tensor("output.weight", &t);
  if (ge == GgufError::None) {
    if ((st = read_matrix(g, "output.weight", (size_t)m->emb.rows, d, m->arena, &m->out))) return st;
  } else if (ge == GgufError::TensorNotFound) {
    m->out = m->emb;  // tied embeddings share the device copy
  } else {
    return DTL_ERR_GGUF;
  }
  m->vocab = (size_t)m->out.rows;
  if ((st = build_encode_copies(m.get()))) return st;
  *out = m.release();
  return DTL_OK;
}

void dtl_model_free(dtl_model* model) { delete model; }

int dtl_model_get_config(const dtl_model* m, dtl_model_config* out) {
  if (!m || !out) return DTL_ERR_INVALID_ARGUMENT;
  std::memset(out, 0, sizeof *out);
  out->block_count = m->c.block_count;
  out->embedding_length = m->c.d;
  out->feed_forward_length = m->c.ff;
  out->head_count = m->c.heads;
  out->head_count_kv = m->c.kv_heads;
  out->head_dim = m->head_dim;
  out->rope_dimension_count = m->c.rope_dim;
  out->context_length = m->c.ctx;
  out->vocab = m->vocab;
  out->rms_epsilon = m->c.eps;
  out->attention_scale = m->c.attention_scale;
  out->rope_freq_base = m->c.rope_base;
  out->rope_split_half = m->c.split_half;
  out->embedding_type = m->emb.type;
  out->output_type = m->out.type;
  out->has_qkv_bias = !m->layers.empty() &&
                      (m->layers[0].bq || m->layers[0].bk || m->layers[0].bv);
  out->device_bytes = m->arena.bytes();
  return DTL_OK;
}

int dtl_session_new(const dtl_model* m, size_t n_ctx, size_t max_chunk, dtl_session** out) {
  if (!m || !out) return DTL_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  if (n_ctx == 0 || n_ctx > m->c.ctx || max_chunk == 0) return DTL_ERR_SHAPE;
  if (max_chunk > n_ctx) max_chunk = n_ctx;
  HIP_TRY(hipSetDevice(m->device));
  std::unique_ptr<dtl_session> s(new dtl_session());
  s->m = m;
  s->n_ctx = n_ctx;
  s->max_chunk = max_chunk;
  s->max_in = max_input_width(m);
  const HostConfig& c = m->c;
  size_t hd = m->head_dim, C = max_chunk, half = c.rope_dim / 2;
  Arena& A = s->arena;
  int st;
  size_t kv = c.block_count * c.kv_heads * n_ctx * hd;
#define ALLOC(ptr, n) \
  if ((st = A.alloc(&s->ptr, (n)))) return st;
  ALLOC(rope_cos, n_ctx * half);
  ALLOC(rope_sin, n_ctx * half);
  ALLOC(kc, kv);
  ALLOC(vc, kv);
  ALLOC(pos_dev, 1);
#undef ALLOC
  s->nlanes = lane_count();
  for (int li = 0; li < s->nlanes; li++) {
    Lane& L = s->lanes[li];
    HIP_TRY(hipStreamCreateWithFlags(&L.stream, hipStreamNonBlocking));
#define ALLOC(ptr, n) \
  if ((st = A.alloc(&L.ptr, (n)))) return st;
    ALLOC(x, C * c.d);
    ALLOC(h, C * c.d);
    ALLOC(q, C * c.heads * hd);
    ALLOC(k, C * c.kv_heads * hd);
    ALLOC(v, C * c.kv_heads * hd);
    ALLOC(attn, C * c.heads * hd);
    ALLOC(g, C * c.ff);
    ALLOC(u, C * c.ff);
    ALLOC(ffo, C * c.ff);
    ALLOC(logits, C * m->vocab);
    ALLOC(scores, C * c.heads * n_ctx);
    ALLOC(qa, C * s->max_in);
    ALLOC(qk, C * s->max_in);
    ALLOC(af, C * s->max_in);
    ALLOC(da, C * (s->max_in / 32 + 1));
    ALLOC(dk, C * (s->max_in / 256 + 1));
    ALLOC(tokens, C);
    ALLOC(err, 1);
    ALLOC(c_sym, C);
    ALLOC(c_freq, C);
    ALLOC(c_cum, C);
    ALLOC(c_total, C);
    ALLOC(c_values, C);
    ALLOC(c_pack, 8);
    ALLOC(c_freq_tab, m->vocab + 256);
    ALLOC(c_cum_tab, m->vocab + 256);
    ALLOC(c_scratch, cdf_scratch_bytes((int)C, (int)m->vocab));
    ALLOC(c_rows, C);
#undef ALLOC
    L.kv_ready.assign(c.block_count, nullptr);
    for (hipEvent_t& e : L.kv_ready) HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    HIP_TRY(hipHostMalloc((void**)&L.h_tokens, C * 4, hipHostMallocDefault));
    HIP_TRY(hipHostMalloc((void**)&L.h_err, sizeof(int), hipHostMallocDefault));
    HIP_TRY(hipHostMalloc((void**)&L.h_io, 8 * sizeof(uint64_t), hipHostMallocDefault));
    if ((st = lane_reserve(L, C))) return st;
  }
  HIP_TRY(hipHostMalloc((void**)&s->pos_host, sizeof(int), hipHostMallocDefault));
  HIP_TRY(hipMemsetAsync(s->kc, 0, kv * 4, s->ln->stream));
  HIP_TRY(hipMemsetAsync(s->vc, 0, kv * 4, s->ln->stream));
  clear_err(s.get());
  launch_rope_table(c.rope_base, (int)c.rope_dim, (int)n_ctx, s->rope_cos, s->rope_sin, s->ln->err,
                    s->ln->stream);
  int bits = 0;
  if ((st = read_err(s.get(), &bits))) return st;
  if (bits) return DTL_ERR_NON_FINITE;
  *out = s.release();
  return DTL_OK;
}

void dtl_session_free(dtl_session* s) {
  if (!s) return;
  (void)hipSetDevice(s->m->device);
  delete s;  // ~dtl_session drains the lanes' streams before releasing them
}

int dtl_session_reset(dtl_session* s) {
  if (!s) return DTL_ERR_INVALID_ARGUMENT;
  HIP_TRY(hipSetDevice(s->m->device));
  size_t kv = s->m->c.block_count * s->m->c.kv_heads * s->n_ctx * s->m->head_dim;
  HIP_TRY(hipMemsetAsync(s->kc, 0, kv * 4, s->ln->stream));
  HIP_TRY(hipMemsetAsync(s->vc, 0, kv * 4, s->ln->stream));
  HIP_TRY(hipStreamSynchronize(s->ln->stream));
  s->ln->rows_valid = 0;
  return DTL_OK;
}

int dtl_forward_chunk(dtl_session* s, const uint32_t* tokens, size_t n, size_t pos0, float* logits) {
  if (!s || !tokens) return DTL_ERR_INVALID_ARGUMENT;
  if (n == 0 || n > s->max_chunk) return DTL_ERR_SHAPE;
  int st = forward_device(s, tokens, (int)n, pos0);
  if (st) return st;
  if (logits) {
    HIP_TRY(hipMemcpyAsync(logits, s->ln->logits, n * s->m->vocab * sizeof(float),
                           hipMemcpyDeviceToHost, s->ln->stream));
    HIP_TRY(hipStreamSynchronize(s->ln->stream));
  }
  return DTL_OK;
}

int dtl_forward_one(dtl_session* s, uint32_t token, size_t pos, float* logits) {
  return dtl_forward_chunk(s, &token, 1, pos, logits);
}

int dtl_session_logits(dtl_session* s, size_t first, size_t n, float* out) {
  if (!s || !out) return DTL_ERR_INVALID_ARGUMENT;
  if (first + n > s->ln->rows_valid) return DTL_ERR_SHAPE;
  HIP_TRY(hipSetDevice(s->m->device));
  HIP_TRY(hipMemcpyAsync(out, s->ln->logits + first * s->m->vocab, n * s->m->vocab * sizeof(float),
                         hipMemcpyDeviceToHost, s->ln->stream));
  HIP_TRY(hipStreamSynchronize(s->ln->stream));
  return DTL_OK;
}

int dtl_logits_hash(const dtl_model* m, const uint32_t* tokens, size_t n, size_t chunk,
                    uint8_t out[32]) {
  if (!m || !tokens || !out) return DTL_ERR_INVALID_ARGUMENT;
  if (n == 0 || chunk == 0 || n > m->c.ctx) return DTL_ERR_SHAPE;
  for (size_t i = 0; i < n; i++)
    if (tokens[i] >= (uint32_t)m->emb.rows) return DTL_ERR_SHAPE;
  dtl_session* s;
  size_t c = chunk < n ? chunk : n;
  int st = dtl_session_new(m, n, c, &s);
  if (st) return st;
  std::vector<float> buf(c * m->vocab);
  Sha256 sha;
  for (size_t p = 0; p < n && !st; p += c) {
    size_t len = n - p < c ? n - p : c;
    st = dtl_forward_chunk(s, tokens + p, len, p, buf.data());
    if (!st) sha.update(buf.data(), len * m->vocab * sizeof(float));
  }
  dtl_session_free(s);
  if (st) return st;
  sha.digest(out);
  return DTL_OK;
}

// ---- det-coder on device logits -------------------------------------------

int dtl_symbol_ranges(dtl_session* s, size_t first, size_t n, const uint32_t* symbols,
                      size_t tail, uint64_t* cum, uint32_t* freq, uint64_t* total) {
  if (!s || !symbols || !cum || !freq || !total) return DTL_ERR_INVALID_ARGUMENT;
  size_t V = s->m->vocab;
  if (n == 0 || first + n > s->ln->rows_valid) return DTL_ERR_SHAPE;
  if (V + tail > kMaxSymbols) return DTL_ERR_CDF_TOO_MANY_SYMBOLS;
  for (size_t i = 0; i < n; i++)
    if (symbols[i] >= V + tail) return DTL_ERR_CDF_SYMBOL_OUT_OF_RANGE;
  HIP_TRY(hipSetDevice(s->m->device));
  clear_err(s);
  Lane& L = *s->ln;
  L.cdf_ready_row = SIZE_MAX;
  // through the lane's pinned staging (n <= max_chunk symbols fit it)
  std::memcpy(L.h_sym, symbols, n * 4);
  HIP_TRY(hipMemcpyAsync(L.c_sym, L.h_sym, n * 4, hipMemcpyHostToDevice, L.stream));
  s->prof.timed(L.stream, "cdf_symbol_range", (double)n * V * 4.0, 0.0, [&] {
    launch_cdf_blocks(L.logits + first * V, nullptr, (int)n, (int)V, (int)tail, 0, L.c_sym, nullptr,
                      L.c_cum, L.c_freq, L.c_total, nullptr, L.c_scratch, false, L.err, L.stream);
  });
  HIP_TRY(hipMemcpyAsync(L.h_cum, L.c_cum, n * 8, hipMemcpyDeviceToHost, L.stream));
  HIP_TRY(hipMemcpyAsync(L.h_freq, L.c_freq, n * 4, hipMemcpyDeviceToHost, L.stream));
  HIP_TRY(hipMemcpyAsync(L.h_total, L.c_total, n * 8, hipMemcpyDeviceToHost, L.stream));
  int bits = 0, st = read_err(s, &bits);
  s->prof.collect();
  if (st) return st;
  std::memcpy(cum, L.h_cum, n * 8);
  std::memcpy(freq, L.h_freq, n * 4);
  std::memcpy(total, L.h_total, n * 8);
  return cdf_status(bits);
}

int dtl_symbol_ranges_rows(dtl_session* s, size_t n, const uint32_t* rows, const uint32_t* symbols,
                           size_t tail, uint64_t* cum, uint32_t* freq, uint64_t* total) {
  if (!s || !rows || !symbols || !cum || !freq || !total) return DTL_ERR_INVALID_ARGUMENT;
  size_t V = s->m->vocab;
  if (n == 0) return DTL_ERR_SHAPE;
  if (V + tail > kMaxSymbols) return DTL_ERR_CDF_TOO_MANY_SYMBOLS;
  for (size_t i = 0; i < n; i++) {
    if (rows[i] >= s->ln->rows_valid) return DTL_ERR_SHAPE;
    if (symbols[i] >= V + tail) return DTL_ERR_CDF_SYMBOL_OUT_OF_RANGE;
  }
  HIP_TRY(hipSetDevice(s->m->device));
  s->ln->cdf_ready_row = SIZE_MAX;
  // batches of at most max_chunk symbols (the size of the staging buffers
  // and of the CDF scratch)
  for (size_t b0 = 0; b0 < n; b0 += s->max_chunk) {
    const size_t m = std::min(s->max_chunk, n - b0);
    clear_err(s);
    HIP_TRY(hipMemcpyAsync(s->ln->c_sym, symbols + b0, m * 4, hipMemcpyHostToDevice, s->ln->stream));
    HIP_TRY(hipMemcpyAsync(s->ln->c_rows, rows + b0, m * 4, hipMemcpyHostToDevice, s->ln->stream));
    s->prof.timed(s->ln->stream, "cdf_symbol_range", (double)m * V * 4.0, 0.0, [&] {
      launch_cdf_blocks(s->ln->logits, s->ln->c_rows, (int)m, (int)V, (int)tail, 0, s->ln->c_sym, nullptr,
                        s->ln->c_cum, s->ln->c_freq, s->ln->c_total, nullptr, s->ln->c_scratch, false, s->ln->err,
                        s->ln->stream);
    });
    HIP_TRY(hipMemcpyAsync(cum + b0, s->ln->c_cum, m * 8, hipMemcpyDeviceToHost, s->ln->stream));
    HIP_TRY(hipMemcpyAsync(freq + b0, s->ln->c_freq, m * 4, hipMemcpyDeviceToHost, s->ln->stream));
    HIP_TRY(hipMemcpyAsync(total + b0, s->ln->c_total, m * 8, hipMemcpyDeviceToHost, s->ln->stream));
    int bits = 0, st = read_err(s, &bits);
    s->prof.collect();
    if (st) return st;
    if ((st = cdf_status(bits))) return st;
  }
  return DTL_OK;
}

// The forwards and symbol ranges of encode_symbols_with_model (det-cli
// main.rs:521-551) for one window, with one chunk in flight per lane: chunk
// c runs on lane c % nlanes and starts while the chunks before it are still
// running (its attention at each layer waits for chunk c - 1's K/V rows of
// that layer; every other launch is independent).  The host collects a
// lane's ranges before reusing it.  Results equal dtl_forward_chunk +
// dtl_symbol_ranges_rows per chunk.
int dtl_forward_ranges(dtl_session* s, const uint32_t* tokens, size_t n, size_t pos0, size_t n_sym,
                       const uint32_t* rows, const uint32_t* symbols, size_t tail, uint64_t* cum,
                       uint32_t* freq, uint64_t* total) {
  if (!s || !tokens || (n_sym && (!rows || !symbols || !cum || !freq || !total)))
    return DTL_ERR_INVALID_ARGUMENT;
  const dtl_model* m = s->m;
  const size_t V = m->vocab, C = s->max_chunk;
  if (n == 0 || pos0 + n > s->n_ctx) return DTL_ERR_SHAPE;
  if (V + tail > kMaxSymbols) return DTL_ERR_CDF_TOO_MANY_SYMBOLS;
  for (size_t i = 0; i < n; i++)
    if (tokens[i] >= (uint32_t)m->emb.rows) return DTL_ERR_SHAPE;
  for (size_t i = 0; i < n_sym; i++) {
    if (rows[i] >= n || (i && rows[i] < rows[i - 1])) return DTL_ERR_SHAPE;
    if (symbols[i] >= V + tail) return DTL_ERR_CDF_SYMBOL_OUT_OF_RANGE;
  }
  HIP_TRY(hipSetDevice(m->device));
  // Back on lane 0 with both lanes drained however this returns.
  struct Restore {
    dtl_session* s;
    ~Restore() {
      for (int li = 0; li < s->nlanes; li++) (void)hipStreamSynchronize(s->lanes[li].stream);
      s->ln = &s->lanes[0];
      s->overlapped = false;
    }
  } restore{s};
  s->overlapped = s->nlanes > 1;
  for (Lane& L : s->lanes) {
    L.rows_valid = 0;
    L.cdf_ready_row = SIZE_MAX;
  }
  const int nl = s->nlanes;
  size_t first[kMaxLanes] = {}, count[kMaxLanes] = {};  // symbols of each lane's chunk
  auto collect = [&](int li) -> int {
    Lane& L = s->lanes[li];
    HIP_TRY(hipStreamSynchronize(L.stream));
    if (*L.h_err & ERRBIT_NON_FINITE) return DTL_ERR_NON_FINITE;
    if (int st = cdf_status(*L.h_err)) return st;
    for (size_t i = 0; i < count[li]; i++) {
      cum[first[li] + i] = L.h_cum[i];
      freq[first[li] + i] = L.h_freq[i];
      total[first[li] + i] = L.h_total[i];
    }
    count[li] = 0;
    return DTL_OK;
  };
  const size_t nchunks = (n + C - 1) / C;
  size_t k = 0;
  for (size_t c = 0; c < nchunks; c++) {
    const int li = (int)(c % nl);
    if (c >= (size_t)nl)
      if (int st = collect(li)) return st;
    Lane& L = s->lanes[li];
    s->ln = &L;
    const size_t p0 = c * C, T = std::min(C, n - p0);
    std::memcpy(L.h_tokens, tokens + p0, T * sizeof(uint32_t));
    HIP_TRY(hipMemcpyAsync(L.tokens, L.h_tokens, T * 4, hipMemcpyHostToDevice, L.stream));
    const Lane* prev = c ? &s->lanes[(c - 1) % nl] : nullptr;
    int rc = enqueue_forward(s, (int)T, pos0 + p0, nullptr, prev, true);
    if (rc) return rc;
    const size_t k0 = k;
    while (k < n_sym && rows[k] < p0 + T) k++;
    // Several symbols may share a row (byte escapes), so a chunk can code
    // more symbols than it has rows: the host staging grows to fit, the
    // device staging and CDF scratch take max_chunk symbols per launch.
    const size_t ms = k - k0;
    if (int st = lane_reserve(L, ms)) return st;
    for (size_t i = 0; i < ms; i++) {
      L.h_rows[i] = (uint32_t)(rows[k0 + i] - p0);
      L.h_sym[i] = symbols[k0 + i];
    }
    for (size_t b0 = 0; b0 < ms; b0 += C) {
      const size_t mb = std::min(C, ms - b0);
      HIP_TRY(hipMemcpyAsync(L.c_rows, L.h_rows + b0, mb * 4, hipMemcpyHostToDevice, L.stream));
      HIP_TRY(hipMemcpyAsync(L.c_sym, L.h_sym + b0, mb * 4, hipMemcpyHostToDevice, L.stream));
      s->prof.timed(L.stream, "cdf_symbol_range", (double)mb * V * 4.0, 0.0, [&] {
        launch_cdf_blocks(L.logits, L.c_rows, (int)mb, (int)V, (int)tail, 0, L.c_sym, nullptr,
                          L.c_cum, L.c_freq, L.c_total, nullptr, L.c_scratch, false, L.err,
                          L.stream);
      });
      HIP_TRY(hipMemcpyAsync(L.h_cum + b0, L.c_cum, mb * 8, hipMemcpyDeviceToHost, L.stream));
      HIP_TRY(hipMemcpyAsync(L.h_freq + b0, L.c_freq, mb * 4, hipMemcpyDeviceToHost, L.stream));
      HIP_TRY(hipMemcpyAsync(L.h_total + b0, L.c_total, mb * 8, hipMemcpyDeviceToHost, L.stream));
    }
    HIP_TRY(hipMemcpyAsync(L.h_err, L.err, sizeof(int), hipMemcpyDeviceToHost, L.stream));
    first[li] = k0;
    count[li] = ms;
  }
  // the chunks still in flight, oldest first
  for (size_t c = nchunks > (size_t)nl ? nchunks - nl : 0; c < nchunks; c++)
    if (int st = collect((int)(c % nl))) return st;
  s->prof.collect();
  return DTL_OK;
}

int dtl_session_get_info(const dtl_session* s, size_t* n_ctx, size_t* max_chunk, size_t* vocab) {
  if (!s) return DTL_ERR_INVALID_ARGUMENT;
  if (n_ctx) *n_ctx = s->n_ctx;
  if (max_chunk) *max_chunk = s->max_chunk;
  if (vocab) *vocab = s->m->vocab;
  return DTL_OK;
}

int dtl_session_set_profiling(dtl_session* s, int enable) {
  if (!s) return DTL_ERR_INVALID_ARGUMENT;
  HIP_TRY(hipStreamSynchronize(s->ln->stream));
  s->prof.enable(enable != 0);
  return DTL_OK;
}

int dtl_session_profile_only(dtl_session* s, const char* kernel_class) {
  if (!s) return DTL_ERR_INVALID_ARGUMENT;
  HIP_TRY(hipStreamSynchronize(s->ln->stream));
  s->prof.only(kernel_class);
  return DTL_OK;
}

int dtl_session_profile(dtl_session* s, dtl_kernel_stat* out, size_t cap, size_t* n) {
  if (!s || !n) return DTL_ERR_INVALID_ARGUMENT;
  const auto& st = s->prof.stats();
  *n = st.size();
  for (size_t i = 0; i < st.size() && i < cap && out; i++) out[i] = st[i];
  return DTL_OK;
}

int dtl_cdf(dtl_session* s, size_t row, size_t tail, uint32_t* freq, uint64_t* cum,
            uint64_t* total) {
  if (!s || !freq || !cum || !total) return DTL_ERR_INVALID_ARGUMENT;
  size_t V = s->m->vocab;
  if (row >= s->ln->rows_valid) return DTL_ERR_SHAPE;
  if (V + tail > kMaxSymbols) return DTL_ERR_CDF_TOO_MANY_SYMBOLS;
  if (tail > 256) return DTL_ERR_INVALID_ARGUMENT;  // table staging holds vocab + 256 entries
  HIP_TRY(hipSetDevice(s->m->device));
  clear_err(s);
  launch_cdf(s->ln->logits + row * V, 1, (int)V, (int)tail, 1, nullptr, nullptr, nullptr, nullptr,
             s->ln->c_total, nullptr, s->ln->c_freq_tab, s->ln->c_cum_tab, s->ln->err, s->ln->stream);
  HIP_TRY(hipMemcpyAsync(freq, s->ln->c_freq_tab, (V + tail) * 4, hipMemcpyDeviceToHost, s->ln->stream));
  HIP_TRY(hipMemcpyAsync(cum, s->ln->c_cum_tab, (V + tail) * 8, hipMemcpyDeviceToHost, s->ln->stream));
  HIP_TRY(hipMemcpyAsync(total, s->ln->c_total, 8, hipMemcpyDeviceToHost, s->ln->stream));
  int bits = 0, st = read_err(s, &bits);
  return st ? st : cdf_status(bits);
}

int dtl_decoder_total(dtl_session* s, size_t row, size_t tail, uint64_t* total) {
  if (!s || !total) return DTL_ERR_INVALID_ARGUMENT;
  size_t V = s->m->vocab;
  if (row >= s->ln->rows_valid) return DTL_ERR_SHAPE;
  if (V + tail > kMaxSymbols) return DTL_ERR_CDF_TOO_MANY_SYMBOLS;
  HIP_TRY(hipSetDevice(s->m->device));
  clear_err(s);
  launch_cdf_blocks(s->ln->logits + row * V, nullptr, 1, (int)V, (int)tail, 3, nullptr, nullptr,
                    nullptr, nullptr, s->ln->c_total, nullptr, s->ln->c_scratch, false, s->ln->err, s->ln->stream);
  int bits = 0, st = read_decoder(s, nullptr, nullptr, nullptr, &bits);
  if (st) return st;
  *total = s->ln->h_io[5];
  st = cdf_status(bits);
  if (st == DTL_OK) {
    // The block results of this row stay in the scratch for a lookup.
    s->ln->cdf_ready_row = row;
    s->ln->cdf_ready_tail = tail;
  }
  return st;
}

int dtl_decoder_decode(dtl_session* s, size_t row, size_t tail, dtl_range_decoder* dec, uint32_t* symbol) {
  if (!s || !dec || !symbol) return DTL_ERR_INVALID_ARGUMENT;
  const size_t V = s->m->vocab;
  if (row >= s->ln->rows_valid) return DTL_ERR_SHAPE;
  if (V + tail > kMaxSymbols) return DTL_ERR_CDF_TOO_MANY_SYMBOLS;
  dtl_range_decoder_state ds;
  if (int st = dtl_range_decoder_snapshot(dec, &ds)) return st;  // between decode_freq and advance
  HIP_TRY(hipSetDevice(s->m->device));
  return decode_step(s, row, tail, dec, ds, symbol, false);
}

int dtl_forward_decode(dtl_session* s, uint32_t token, size_t pos, size_t tail, dtl_range_decoder* dec,
                       uint32_t* symbol) {
  if (!s || !dec || !symbol) return DTL_ERR_INVALID_ARGUMENT;
  if (s->m->vocab + tail > kMaxSymbols) return DTL_ERR_CDF_TOO_MANY_SYMBOLS;
  dtl_range_decoder_state ds;
  if (int st = dtl_range_decoder_snapshot(dec, &ds)) return st;
  int st = forward_device(s, &token, 1, pos, false);
  if (st) return st;
  return decode_step(s, 0, tail, dec, ds, symbol, true);
}

int dtl_decoder_lookup(dtl_session* s, size_t row, size_t tail, uint64_t value, uint32_t* symbol,
                       uint64_t* cum, uint32_t* freq, uint64_t* total) {
  if (!s || !symbol || !cum || !freq || !total) return DTL_ERR_INVALID_ARGUMENT;
  size_t V = s->m->vocab;
  if (row >= s->ln->rows_valid) return DTL_ERR_SHAPE;
  if (V + tail > kMaxSymbols) return DTL_ERR_CDF_TOO_MANY_SYMBOLS;
  HIP_TRY(hipSetDevice(s->m->device));
  clear_err(s);
  uint64_t* io = s->ln->h_io;  // [1] value in; [2] symbol, [3] cum, [4] freq, [5] total, [6] error bits out
  io[1] = value;
  HIP_TRY(hipMemcpyAsync(s->ln->c_values, io + 1, 8, hipMemcpyHostToDevice, s->ln->stream));
  const bool reuse = s->ln->cdf_ready_row == row && s->ln->cdf_ready_tail == tail;
  launch_cdf_blocks(s->ln->logits + row * V, nullptr, 1, (int)V, (int)tail, 2, nullptr, s->ln->c_values,
                    s->ln->c_cum, s->ln->c_freq, s->ln->c_total, s->ln->c_sym, s->ln->c_scratch, reuse, s->ln->err,
                    s->ln->stream);
  int bits = 0, st = read_decoder(s, s->ln->c_sym, s->ln->c_cum, s->ln->c_freq, &bits);
  if (st) return st;
  *symbol = (uint32_t)io[2];
  *cum = io[3];
  *freq = (uint32_t)io[4];
  *total = io[5];
  if (value >= *total) return DTL_ERR_CDF_SYMBOL_OUT_OF_RANGE;
  return cdf_status(bits);
}

}  // extern "C"

// ---- standalone kernels on host data -----------------------------------------

namespace {

// RAII scratch for the one-shot entry points.
struct Scratch {
  Arena arena;
  hipStream_t stream = nullptr;
  int* err = nullptr;
  ~Scratch() {
    if (stream) {
      (void)hipStreamSynchronize(stream);
      (void)hipStreamDestroy(stream);
    }
  }
  int init() {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) return DTL_ERR_NO_DEVICE;
    HIP_TRY(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
    int st = arena.alloc(&err, 1);
    if (st) return st;
    HIP_TRY(hipMemsetAsync(err, 0, sizeof(int), stream));
    return DTL_OK;
  }
  int finish(int* bits) {
    HIP_TRY(hipGetLastError());
    HIP_TRY(hipMemcpyAsync(bits, err, sizeof(int), hipMemcpyDeviceToHost, stream));
    HIP_TRY(hipStreamSynchronize(stream));
    return DTL_OK;
  }
};

int run_cdf_host(const float* logits, size_t n, size_t tail, int mode, uint32_t symbol,
                 uint64_t* cum, uint32_t* freq, uint64_t* total, uint32_t* freq_tab,
                 uint64_t* cum_tab) {
  if (n == 0) return DTL_ERR_CDF_EMPTY;
  if (n + tail > kMaxSymbols) return DTL_ERR_CDF_TOO_MANY_SYMBOLS;
  Scratch sc;
  int st = sc.init();
  if (st) return st;
  float* dl;
  uint32_t *dsym, *dfreq, *dft = nullptr;
  uint64_t *dcum, *dtot, *dct = nullptr;
  if ((st = sc.arena.upload(&dl, logits, n))) return st;
  if ((st = sc.arena.upload(&dsym, &symbol, 1))) return st;
  if ((st = sc.arena.alloc(&dfreq, 1))) return st;
  if ((st = sc.arena.alloc(&dcum, 1))) return st;
  if ((st = sc.arena.alloc(&dtot, 1))) return st;
  if (mode == 1) {
    if ((st = sc.arena.alloc(&dft, n + tail))) return st;
    if ((st = sc.arena.alloc(&dct, n + tail))) return st;
  }
  if (mode == 1) {
    launch_cdf(dl, 1, (int)n, (int)tail, mode, dsym, nullptr, dcum, dfreq, dtot, nullptr, dft, dct,
               sc.err, sc.stream);
  } else {
    uint8_t* scratch;
    if ((st = sc.arena.alloc(&scratch, cdf_scratch_bytes(1, (int)n)))) return st;
    launch_cdf_blocks(dl, nullptr, 1, (int)n, (int)tail, mode, dsym, nullptr, dcum, dfreq, dtot,
                      nullptr, scratch, false, sc.err, sc.stream);
  }
  if (mode == 1) {
    HIP_TRY(hipMemcpyAsync(freq_tab, dft, (n + tail) * 4, hipMemcpyDeviceToHost, sc.stream));
    HIP_TRY(hipMemcpyAsync(cum_tab, dct, (n + tail) * 8, hipMemcpyDeviceToHost, sc.stream));
  } else {
    HIP_TRY(hipMemcpyAsync(cum, dcum, 8, hipMemcpyDeviceToHost, sc.stream));
    HIP_TRY(hipMemcpyAsync(freq, dfreq, 4, hipMemcpyDeviceToHost, sc.stream));
  }
  HIP_TRY(hipMemcpyAsync(total, dtot, 8, hipMemcpyDeviceToHost, sc.stream));
  int bits = 0;
  if ((st = sc.finish(&bits))) return st;
  return cdf_status(bits);
}

}  // namespace

extern "C" {

int dtl_logits_to_cdf(const float* logits, size_t n, size_t tail, uint32_t* freq, uint64_t* cum,
                      uint64_t* total) {
  if (!logits || !freq || !cum || !total) return DTL_ERR_INVALID_ARGUMENT;
  return run_cdf_host(logits, n, tail, 1, 0, nullptr, nullptr, total, freq, cum);
}

int dtl_logits_to_symbol_range(const float* logits, size_t n, size_t symbol, size_t tail,
                               uint64_t* cum, uint32_t* freq, uint64_t* total) {
  if (!logits || !cum || !freq || !total) return DTL_ERR_INVALID_ARGUMENT;
  if (n == 0) return DTL_ERR_CDF_EMPTY;
  if (n + tail > kMaxSymbols) return DTL_ERR_CDF_TOO_MANY_SYMBOLS;
  if (symbol >= n + tail) return DTL_ERR_CDF_SYMBOL_OUT_OF_RANGE;
  return run_cdf_host(logits, n, tail, 0, (uint32_t)symbol, cum, freq, total, nullptr, nullptr);
}

int dtl_uniform_cdf(size_t symbols, uint32_t* freq, uint64_t* cum, uint64_t* total) {
  if (!freq || !cum || !total) return DTL_ERR_INVALID_ARGUMENT;
  if (symbols == 0) return DTL_ERR_CDF_EMPTY;
  if (symbols > kMaxSymbols) return DTL_ERR_CDF_TOO_MANY_SYMBOLS;
  for (size_t i = 0; i < symbols; i++) {
    freq[i] = 1;
    cum[i] = i;
  }
  *total = symbols;
  return DTL_OK;
}

int dtl_uniform_symbol_range(size_t symbol, size_t symbols, uint64_t* cum, uint32_t* freq,
                             uint64_t* total) {
  if (!cum || !freq || !total) return DTL_ERR_INVALID_ARGUMENT;
  if (symbols == 0) return DTL_ERR_CDF_EMPTY;
  if (symbols > kMaxSymbols) return DTL_ERR_CDF_TOO_MANY_SYMBOLS;
  if (symbol >= symbols) return DTL_ERR_CDF_SYMBOL_OUT_OF_RANGE;
  *cum = symbol;
  *freq = 1;
  *total = symbols;
  return DTL_OK;
}

// ---- symbol ranges without allocation ----------------------------------------
// Callers that cannot allocate (code under HIP graph capture, serving loops
// that forbid hipMalloc) get the multi-workgroup CDF's scratch from one
// file-scope device array per GPU instead of a per-call or per-session
// buffer.  Its device address comes from hipGetSymbolAddress on the
// entry point's first call on each device; host code never passes the
// array's name to a kernel.  Calls on one GPU share the array, so calls
// that overlap on one GPU race.  No field of the scratch has to start at
// zero (every kernel writes what the next one reads); the caller's status
// word is cleared by the first launch of each call, with a kernel rather
// than a memset so that the call can be captured into a graph.
}  // extern "C"

namespace {
constexpr size_t kStaticCdfRows = 8;
// The largest call: kStaticCdfRows rows of vocab 2^18 (the scratch depends
// on the vocabulary, not on the tail), rounded up to 256 bytes: 8,399,360.
constexpr size_t kStaticCdfScratchBytes = (cdf_scratch_bytes_for(kStaticCdfRows, kMaxSymbols) + 255) & ~(size_t)255;
static_assert(kStaticCdfScratchBytes >= cdf_scratch_bytes_for(kStaticCdfRows, kMaxSymbols), "static scratch");
static_assert(kStaticCdfScratchBytes == 8399360, "static scratch size as documented");
static __device__ __align__(256) uint8_t scratch[kStaticCdfScratchBytes];
constexpr int kStaticMaxDevices = 64;
std::atomic<void*> g_static_scratch[kStaticMaxDevices];

// The device address of this device's scratch array (null on failure).
void* static_scratch_ptr(int dev) {
  if (dev < 0 || dev >= kStaticMaxDevices) return nullptr;
  void* p = g_static_scratch[dev].load(std::memory_order_acquire);
  if (p) return p;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
    (void)hipGetLastError();
    return nullptr;
  }
  g_static_scratch[dev].store(p, std::memory_order_release);
  return p;
}

// Clears the status word and flags symbols outside [0, limit): the range
// kernels themselves never index with the symbol past the table, so a bad
// symbol only has to be reported.
__global__ void k_static_prepare(int* bits, const uint32_t* symbols, int R, uint32_t limit) {
  __shared__ int bad;
  if (threadIdx.x == 0) bad = 0;
  __syncthreads();
  for (int r = threadIdx.x; r < R; r += blockDim.x)
    if (symbols[r] >= limit) bad = 1;
  __syncthreads();
  if (threadIdx.x == 0) *bits = bad ? ERRBIT_CDF_SYMBOL : 0;
}
}  // namespace

extern "C" {

int dtl_symbol_ranges_static(const float* logits, size_t rows, size_t vocab, const uint32_t* symbols,
                             size_t tail, uint64_t* cum, uint32_t* freq, uint64_t* total,
                             int* status_bits, void* stream) {
  if (!logits || !symbols || !cum || !freq || !total || !status_bits) return DTL_ERR_INVALID_ARGUMENT;
  if (rows == 0 || vocab == 0) return DTL_ERR_CDF_EMPTY;
  if (vocab + tail > kMaxSymbols) return DTL_ERR_CDF_TOO_MANY_SYMBOLS;
  if (rows > kStaticCdfRows) return DTL_ERR_STATIC_SCRATCH_LIMIT;
  if (cdf_scratch_bytes((int)rows, (int)vocab) > kStaticCdfScratchBytes) return DTL_ERR_STATIC_SCRATCH_LIMIT;
  int dev = 0;
  HIP_TRY(hipGetDevice(&dev));
  void* ptr = static_scratch_ptr(dev);
  if (!ptr) return DTL_ERR_DEVICE;
  hipStream_t st = static_cast<hipStream_t>(stream);
  launch_kernel(k_static_prepare, dim3(1), dim3(64), 0, st, status_bits, symbols, (int)rows,
                (uint32_t)(vocab + tail));
  launch_cdf_blocks(logits, nullptr, (int)rows, (int)vocab, (int)tail, 0, symbols, nullptr, cum, freq,
                    total, nullptr, ptr, false, status_bits, st);
  HIP_TRY(hipGetLastError());
  return DTL_OK;
}

int dtl_status_from_bits(int bits) {
  if (bits & ERRBIT_NON_FINITE) return DTL_ERR_NON_FINITE;
  if (bits & ERRBIT_CDF_SYMBOL) return DTL_ERR_CDF_SYMBOL_OUT_OF_RANGE;
  return cdf_status(bits);
}

int dtl_kernel_exp_f32(const float* in, float* out, size_t n) {
  if (!in || !out) return DTL_ERR_INVALID_ARGUMENT;
  Scratch sc;
  int st = sc.init();
  if (st) return st;
  float *di, *dout;
  if ((st = sc.arena.upload(&di, in, n))) return st;
  if ((st = sc.arena.alloc(&dout, n))) return st;
  launch_exp_f32(di, dout, (int)n, 0, sc.stream);
  HIP_TRY(hipMemcpyAsync(out, dout, n * 4, hipMemcpyDeviceToHost, sc.stream));
  int bits;
  return sc.finish(&bits);
}

int dtl_kernel_silu_f32(const float* in, float* out, size_t n) {
  if (!in || !out) return DTL_ERR_INVALID_ARGUMENT;
  Scratch sc;
  int st = sc.init();
  if (st) return st;
  float *di, *dout;
  if ((st = sc.arena.upload(&di, in, n))) return st;
  if ((st = sc.arena.alloc(&dout, n))) return st;
  launch_exp_f32(di, dout, (int)n, 1, sc.stream);
  HIP_TRY(hipMemcpyAsync(out, dout, n * 4, hipMemcpyDeviceToHost, sc.stream));
  int bits;
  return sc.finish(&bits);
}

int dtl_kernel_exp_clamped_f32(const float* in, float* out, size_t n) {
  if (!in || !out) return DTL_ERR_INVALID_ARGUMENT;
  for (size_t i = 0; i < n; i++)
    if (in[i] > 0.0f) return DTL_ERR_INVALID_ARGUMENT;  // outside exp_clamped's domain
  Scratch sc;
  int st = sc.init();
  if (st) return st;
  float *di, *dout;
  if ((st = sc.arena.upload(&di, in, n))) return st;
  if ((st = sc.arena.alloc(&dout, n))) return st;
  launch_exp_f32(di, dout, (int)n, 2, sc.stream);
  HIP_TRY(hipMemcpyAsync(out, dout, n * 4, hipMemcpyDeviceToHost, sc.stream));
  int bits;
  return sc.finish(&bits);
}

int dtl_valu_probe(double* lane_ops_per_s) {
  if (!lane_ops_per_s) return DTL_ERR_INVALID_ARGUMENT;
  Scratch sc;
  int st = sc.init();
  if (st) return st;
  int dev = 0, cus = 0;
  HIP_TRY(hipGetDevice(&dev));
  HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  float* out;
  if ((st = sc.arena.alloc(&out, 1024))) return st;
  // two 1024-thread workgroups per CU: eight waves on every SIMD
  const int wgs = 2 * cus, iters = 20000;
  hipEvent_t e0, e1;
  HIP_TRY(hipEventCreate(&e0));
  HIP_TRY(hipEventCreate(&e1));
  launch_valu_probe(out, wgs, 64, sc.stream);
  HIP_TRY(hipEventRecord(e0, sc.stream));
  launch_valu_probe(out, wgs, iters, sc.stream);
  HIP_TRY(hipEventRecord(e1, sc.stream));
  HIP_TRY(hipEventSynchronize(e1));
  float ms = 0.0f;
  HIP_TRY(hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  *lane_ops_per_s = (double)wgs * 1024.0 * iters * 16.0 / (ms * 1e-3);
  int bits;
  return sc.finish(&bits);
}

int dtl_mfp_probe(double* macs_per_s) {
  if (!macs_per_s) return DTL_ERR_INVALID_ARGUMENT;
  Scratch sc;
  int st = sc.init();
  if (st) return st;
  int dev = 0, cus = 0;
  HIP_TRY(hipGetDevice(&dev));
  HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  float* out;
  if ((st = sc.arena.alloc(&out, 256))) return st;
  // four 256-thread workgroups per CU: four waves on every SIMD
  const int wgs = 4 * cus, iters = 20000;
  hipEvent_t e0, e1;
  HIP_TRY(hipEventCreate(&e0));
  HIP_TRY(hipEventCreate(&e1));
  launch_mfp_probe(out, wgs, 64, sc.stream);
  HIP_TRY(hipEventRecord(e0, sc.stream));
  launch_mfp_probe(out, wgs, iters, sc.stream);
  HIP_TRY(hipEventRecord(e1, sc.stream));
  HIP_TRY(hipEventSynchronize(e1));
  float ms = 0.0f;
  HIP_TRY(hipEventElapsedTime(&ms, e0, e1));
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  // 4096 products (and adds) per wave per iteration, four waves per workgroup
  *macs_per_s = (double)wgs * 4.0 * iters * 4096.0 / (ms * 1e-3);
  int bits;
  return sc.finish(&bits);
}

int dtl_kernel_f16_to_f32(const uint16_t* in, float* out, size_t n) {
  if (!in || !out) return DTL_ERR_INVALID_ARGUMENT;
  Scratch sc;
  int st = sc.init();
  if (st) return st;
  uint16_t* di;
  float* dout;
  if ((st = sc.arena.upload(&di, in, n))) return st;
  if ((st = sc.arena.alloc(&dout, n))) return st;
  launch_f16_to_f32(di, dout, (int)n, sc.stream);
  HIP_TRY(hipMemcpyAsync(out, dout, n * 4, hipMemcpyDeviceToHost, sc.stream));
  int bits;
  return sc.finish(&bits);
}

int dtl_kernel_div_sqrt(const float* a, const float* b, float* quot, float* root, size_t n) {
  if (!a || !b || !quot || !root) return DTL_ERR_INVALID_ARGUMENT;
  Scratch sc;
  int st = sc.init();
  if (st) return st;
  float *da, *db, *dq, *dr;
  if ((st = sc.arena.upload(&da, a, n))) return st;
  if ((st = sc.arena.upload(&db, b, n))) return st;
  if ((st = sc.arena.alloc(&dq, n))) return st;
  if ((st = sc.arena.alloc(&dr, n))) return st;
  launch_div_sqrt(da, db, dq, dr, (int)n, sc.stream);
  HIP_TRY(hipMemcpyAsync(quot, dq, n * 4, hipMemcpyDeviceToHost, sc.stream));
  HIP_TRY(hipMemcpyAsync(root, dr, n * 4, hipMemcpyDeviceToHost, sc.stream));
  int bits;
  return sc.finish(&bits);
}

int dtl_kernel_quantize(const float* x, size_t rows, size_t n, float* q8a_d, int8_t* q8a_q,
                        float* q8k_d, int8_t* q8k_q) {
  if (!x || rows == 0 || n == 0) return DTL_ERR_INVALID_ARGUMENT;
  bool want_a = q8a_d && q8a_q, want_k = q8k_d && q8k_q;
  if ((want_a && n % 32) || (want_k && n % 256)) return DTL_ERR_SHAPE;
  Scratch sc;
  int st = sc.init();
  if (st) return st;
  float *dx, *da, *af, *dk;
  int8_t *qa, *qk;
  size_t tot = rows * n;
  if ((st = sc.arena.upload(&dx, x, tot))) return st;
  if ((st = sc.arena.alloc(&qa, tot))) return st;
  if ((st = sc.arena.alloc(&qk, tot))) return st;
  if ((st = sc.arena.alloc(&af, tot))) return st;
  if ((st = sc.arena.alloc(&da, tot / 32 + 1))) return st;
  if ((st = sc.arena.alloc(&dk, tot / 256 + 1))) return st;
  launch_quantize(dx, (int)rows, (int)n, want_a, want_k, qa, da, af, qk, dk, sc.err, sc.stream);
  if (want_a) {
    HIP_TRY(hipMemcpyAsync(q8a_q, qa, tot, hipMemcpyDeviceToHost, sc.stream));
    HIP_TRY(hipMemcpyAsync(q8a_d, da, tot / 32 * 4, hipMemcpyDeviceToHost, sc.stream));
  }
  std::vector<int8_t> perm;
  if (want_k) {
    perm.resize(tot);
    HIP_TRY(hipMemcpyAsync(perm.data(), qk, tot, hipMemcpyDeviceToHost, sc.stream));
    HIP_TRY(hipMemcpyAsync(q8k_d, dk, tot / 256 * 4, hipMemcpyDeviceToHost, sc.stream));
  }
  int bits = 0;
  if ((st = sc.finish(&bits))) return st;
  // Device Q8_K blocks are class-major; return them in element order.
  for (size_t b = 0; b < perm.size() / 256; b++)
    for (size_t e = 0; e < 256; e++) q8k_q[b * 256 + e] = perm[b * 256 + (e % 8) * 32 + e / 8];
  return bits ? DTL_ERR_NON_FINITE : DTL_OK;
}

int dtl_kernel_rmsnorm(const float* x, const float* w, float eps, size_t rows, size_t n,
                       float* out) {
  if (!x || !w || !out || rows == 0 || n == 0) return DTL_ERR_INVALID_ARGUMENT;
  Scratch sc;
  int st = sc.init();
  if (st) return st;
  float *dx, *dw, *dout;
  if ((st = sc.arena.upload(&dx, x, rows * n))) return st;
  if ((st = sc.arena.upload(&dw, w, n))) return st;
  if ((st = sc.arena.alloc(&dout, rows * n))) return st;
  launch_rmsnorm(dx, dw, eps, (int)rows, (int)n, dout, sc.err, sc.stream);
  HIP_TRY(hipMemcpyAsync(out, dout, rows * n * 4, hipMemcpyDeviceToHost, sc.stream));
  int bits = 0;
  if ((st = sc.finish(&bits))) return st;
  return bits ? DTL_ERR_NON_FINITE : DTL_OK;
}

namespace {
// A matrix of raw GGUF blocks on the device as a loaded model holds it: the
// bytes are wrapped in a one-tensor GGUF container so that the load-time
// repack path (upload_matrix) is the one under test, then the encode-GEMM
// and decode-layout copies a loaded model keeps are built.
int upload_raw_matrix(Scratch& sc, int ggml_type, const uint8_t* weights, size_t rows, size_t cols,
                      DevMat* out) {
  uint64_t tb, bs;
  if (!ggml_type_size((uint32_t)ggml_type, &tb, &bs)) return DTL_ERR_UNSUPPORTED_TENSOR_TYPE;
  if (cols % bs) return DTL_ERR_SHAPE;
  size_t row_bytes = cols / bs * tb;
  std::vector<uint8_t> file;
  auto put = [&](const void* p, size_t k) {
    const uint8_t* b = (const uint8_t*)p;
    file.insert(file.end(), b, b + k);
  };
  uint32_t u32;
  uint64_t u64;
  put("GGUF", 4);
  u32 = 3; put(&u32, 4);
  u64 = 1; put(&u64, 8);
  u64 = 0; put(&u64, 8);
  u64 = 1; put(&u64, 8);
  put("w", 1);
  u32 = 2; put(&u32, 4);
  u64 = cols; put(&u64, 8);
  u64 = rows; put(&u64, 8);
  u32 = (uint32_t)ggml_type; put(&u32, 4);
  u64 = 0; put(&u64, 8);
  while (file.size() % 32) file.push_back(0);
  put(weights, rows * row_bytes);
  Gguf g;
  if (g.parse(file.data(), file.size()) != GgufError::None) return DTL_ERR_GGUF;
  const GgufTensor* gt;
  if (g.tensor("w", &gt) != GgufError::None) return DTL_ERR_GGUF;
  DevMat W{};
  int st;
  if ((st = upload_matrix(g, *gt, rows, cols, sc.arena, &W))) return st;
  if (W.type == GGML_Q4_K && f32_mirror_enabled()) {
    float* w32;
    if ((st = sc.arena.alloc(&w32, rows * cols))) return st;
    launch_dequant_q4k(W, w32, sc.stream);
    W.w32 = w32;
  }
  if (W.type == GGML_Q6_K && q6k_planes_enabled()) {
    int8_t* planes;
    if ((st = sc.arena.alloc(&planes, q6k_planes_bytes(W)))) return st;
    launch_q6k_planes(W, planes, sc.stream);
    W.planes = planes;
  }
  if (W.type == GGML_Q4_0) {
    int8_t* i8;
    if ((st = sc.arena.alloc(&i8, rows * cols))) return st;
    launch_q4_0_i8(W, i8, sc.stream);
    W.i8 = i8;
  }
  if (W.type == GGML_Q6_K && q6k_decode_layout_applies(W)) {
    uint4* q6d;
    if ((st = sc.arena.alloc(&q6d, q6k_decode_layout_bytes(W) / sizeof(uint4)))) return st;
    launch_q6k_decode_layout(W, q6d, sc.stream);
    W.q6d = q6d;
  }
  *out = W;
  return DTL_OK;
}
}  // namespace

int dtl_kernel_gemv(int ggml_type, const uint8_t* weights, size_t rows, size_t cols,
                    const float* x, size_t T, float* out) {
  if (!weights || !x || !out || rows == 0 || cols == 0 || T == 0) return DTL_ERR_INVALID_ARGUMENT;
  Scratch sc;
  int st = sc.init();
  if (st) return st;
  DevMat W{};
  if ((st = upload_raw_matrix(sc, ggml_type, weights, rows, cols, &W))) return st;
  float *dx, *dout, *af, *da, *dk;
  int8_t *qa, *qk;
  if ((st = sc.arena.upload(&dx, x, T * cols))) return st;
  if ((st = sc.arena.alloc(&dout, T * rows))) return st;
  if ((st = sc.arena.alloc(&qa, T * cols))) return st;
  if ((st = sc.arena.alloc(&qk, T * cols))) return st;
  if ((st = sc.arena.alloc(&af, T * cols))) return st;
  if ((st = sc.arena.alloc(&da, T * cols / 32 + 1))) return st;
  if ((st = sc.arena.alloc(&dk, T * cols / 256 + 1))) return st;
  bool q8a = needs_q8a(W), q8k = W.type == GGML_Q6_K;
  if (q8a || q8k)
    launch_quantize(dx, (int)T, (int)cols, q8a, q8k, qa, da, af, qk, dk, sc.err, sc.stream);
  DevAct a{dx, qa, da, af, qk, dk};
  launch_gemm(W, a, (int)T, dout, nullptr, EPI_STORE, sc.err, sc.stream);
  HIP_TRY(hipMemcpyAsync(out, dout, T * rows * 4, hipMemcpyDeviceToHost, sc.stream));
  int bits = 0;
  if ((st = sc.finish(&bits))) return st;
  return bits ? DTL_ERR_NON_FINITE : DTL_OK;
}

int dtl_kernel_q4k_chunk(int mode, int overlapped, const uint8_t* w0, size_t rows0, const uint8_t* w1,
                         size_t rows1, size_t cols, const float* x, size_t T, float* out0, float* out1) {
  if (mode < 0 || mode > 2 || !w0 || !x || !out0 || rows0 == 0 || cols == 0 || T == 0)
    return DTL_ERR_INVALID_ARGUMENT;
  if (mode != 0 && !w1) return DTL_ERR_INVALID_ARGUMENT;
  if (mode == 2 && (!out1 || rows1 == 0)) return DTL_ERR_INVALID_ARGUMENT;
  if (mode == 1) rows1 = rows0;  // gate and up have the same shape
  if (T < 16 || cols % 256) return DTL_ERR_SHAPE;
  if (!f32_mirror_enabled()) return DTL_ERR_UNSUPPORTED_TENSOR_TYPE;
  Scratch sc;
  int st = sc.init();
  if (st) return st;
  DevMat W0{}, W1{};
  if ((st = upload_raw_matrix(sc, GGML_Q4_K, w0, rows0, cols, &W0))) return st;
  if (mode != 0 && (st = upload_raw_matrix(sc, GGML_Q4_K, w1, rows1, cols, &W1))) return st;
  float *dx, *d0, *d1 = nullptr, *af, *da;
  int8_t* qa;
  if ((st = sc.arena.upload(&dx, x, T * cols))) return st;
  if ((st = sc.arena.alloc(&d0, T * rows0))) return st;
  if (mode == 2 && (st = sc.arena.alloc(&d1, T * rows1))) return st;
  if ((st = sc.arena.alloc(&qa, T * cols))) return st;
  if ((st = sc.arena.alloc(&af, T * cols))) return st;
  if ((st = sc.arena.alloc(&da, T * cols / 32 + 1))) return st;
  launch_quantize(dx, (int)T, (int)cols, true, false, qa, da, af, nullptr, nullptr, sc.err, sc.stream);
  DevAct a{dx, qa, da, af, nullptr, nullptr};
  a.overlapped = overlapped != 0;
  if (mode == 0) {
    launch_gemm_tok(W0, a, (int)T, d0, nullptr, EPI_STORE, sc.err, sc.stream);
  } else if (mode == 1) {
    launch_gemm_pair_swiglu_q4k(W0, W1, a, (int)T, nullptr, nullptr, d0, sc.err, sc.stream);
  } else if (!launch_gemm_cat_q4k(W0, W1, a, (int)T, d0, d1, nullptr, nullptr, EPI_STORE, sc.err,
                                  sc.stream)) {
    return DTL_ERR_SHAPE;
  }
  HIP_TRY(hipMemcpyAsync(out0, d0, T * rows0 * 4, hipMemcpyDeviceToHost, sc.stream));
  if (mode == 2) HIP_TRY(hipMemcpyAsync(out1, d1, T * rows1 * 4, hipMemcpyDeviceToHost, sc.stream));
  int bits = 0;
  if ((st = sc.finish(&bits))) return st;
  return bits ? DTL_ERR_NON_FINITE : DTL_OK;
}

int dtl_kernel_rope_table(float base, size_t rope_dim, size_t positions, float* cos_out,
                          float* sin_out) {
  if (!cos_out || !sin_out || rope_dim == 0 || rope_dim % 2 || positions == 0)
    return DTL_ERR_INVALID_ARGUMENT;
  Scratch sc;
  int st = sc.init();
  if (st) return st;
  size_t n = positions * rope_dim / 2;
  float *dc, *ds;
  if ((st = sc.arena.alloc(&dc, n))) return st;
  if ((st = sc.arena.alloc(&ds, n))) return st;
  launch_rope_table(base, (int)rope_dim, (int)positions, dc, ds, sc.err, sc.stream);
  HIP_TRY(hipMemcpyAsync(cos_out, dc, n * 4, hipMemcpyDeviceToHost, sc.stream));
  HIP_TRY(hipMemcpyAsync(sin_out, ds, n * 4, hipMemcpyDeviceToHost, sc.stream));
  int bits = 0;
  if ((st = sc.finish(&bits))) return st;
  return bits ? DTL_ERR_NON_FINITE : DTL_OK;
}

}  // extern "C"
