// gfx950 kernels for the detllm decoder forward and logits->CDF step.
//
// Every floating-point reduction follows the reference's fixed order:
// one lane owns one dependent chain (a GEMV row for one position, one of
// the 8 interleaved lanes of det-num's reductions, one P.V output element)
// and walks it in ascending index order, while independent chains run in
// parallel across lanes, waves and workgroups.  Integer stages (Q8_0/Q4_0
// block sums, Q6_K lane sums, CDF prefix sums) are exact and use any order.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dtl_device.h"
#include "dtl_blocks.h"
#include "dtl_numerics.h"
#include "dtl_quant.h"

namespace dtl {

namespace {

constexpr int kGgmlF32 = 0, kGgmlQ4_0 = 2, kGgmlQ8_0 = 8, kGgmlQ4K = 12, kGgmlQ6K = 14;

__device__ __forceinline__ void flag(int* err, int bit) { atomicOr(err, bit); }

__device__ __forceinline__ uint16_t ld_u16(const uint8_t* p) {
  return (uint16_t)(p[0] | ((uint16_t)p[1] << 8));
}

// det-quant lib.rs:519-529: 6-bit scale and min of Q4_K sub-block `j`.
__device__ __forceinline__ void q4k_scale_min(const uint8_t* sc, int j, int* scale, int* mn) {
  if (j < 4) {
    *scale = sc[j] & 0x3f;
    *mn = sc[j + 4] & 0x3f;
  } else {
    *scale = (sc[j + 4] & 0x0f) | ((sc[j - 4] >> 6) << 4);
    *mn = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
  }
}

// One weight value, as write_row_validated dequantises it (det-model lib.rs:667-746).
__device__ float mat_value(const DevMat& M, int row, int i) {
  switch (M.type) {
    case kGgmlF32:
      return ((const float*)M.w)[(size_t)row * M.cols + i];
    case kGgmlQ8_0: {
      float d = f16_to_f32(M.d16[(size_t)row * M.nb + i / 32]);
      return d * (float)((const int8_t*)M.w)[(size_t)row * M.cols + i];
    }
    case kGgmlQ4_0: {
      int b = i / 32, j = i % 32;
      const uint8_t* qs = (const uint8_t*)M.w + ((size_t)row * M.nb + b) * 16;
      int nib = j < 16 ? (qs[j] & 0x0f) : (qs[j - 16] >> 4);
      float d = f16_to_f32(M.d16[(size_t)row * M.nb + b]);
      return d * (float)(nib - 8);
    }
    case kGgmlQ4K: {
      int sb = i / 256, idx = i % 256, sub = idx / 32, within = idx % 32;
      size_t blk = (size_t)row * M.nb + sb;
      const uint8_t* h = M.hdr + blk * 16;
      float d = f16_to_f32(ld_u16(h)), dmin = f16_to_f32(ld_u16(h + 2));
      int sc, mn;
      q4k_scale_min(h + 4, sub, &sc, &mn);
      uint8_t byte = ((const uint8_t*)M.w)[blk * 128 + (sub / 2) * 32 + within];
      int q = (sub & 1) ? (byte >> 4) : (byte & 0x0f);
      return (d * (float)sc) * (float)q - (dmin * (float)mn);
    }
    case kGgmlQ6K: {
      int sb = i / 256, e = i % 256;
      size_t blk = (size_t)row * M.nb + sb;
      const uint8_t* body = (const uint8_t*)M.w + blk * 208;
      float d = f16_to_f32(M.d16[blk]);
      return (d * (float)q6k_scale(body, e)) * (float)q6k_quant(body, e);
    }
  }
  return 0.0f;
}

// ---- row dots: one lane computes one (row, position) chain ---------------

// dot_f32_ref (det-num reduce.rs:2-11)
__device__ float row_dot_f32(const float* w, const float* x, int n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int i = 0; i < n; i++) acc[i & 7] += w[i] * x[i];
  return finish_8lane(acc);
}

// dot_q8_0_q8a (det-quant lib.rs:237-257): exact i32 per block, then
// (dw*da)*isum added in block order.
__device__ float row_dot_q8_0(const int8_t* wq, const uint16_t* wd, const int8_t* aq,
                              const float* ad, int nb) {
  float sum = 0.0f;
  const int* w4 = (const int*)wq;
  const int* a4 = (const int*)aq;
  for (int b = 0; b < nb; b++) {
    int isum = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) isum = __builtin_amdgcn_sdot4(w4[b * 8 + k], a4[b * 8 + k], isum, false);
    float scale = f16_to_f32(wd[b]) * ad[b];
    sum += scale * (float)isum;
  }
  return sum;
}

// dot_q4_0_q8a (lib.rs:259-279, 492-504)
__device__ float row_dot_q4_0(const uint8_t* wq, const uint16_t* wd, const int8_t* aq,
                              const float* ad, int nb) {
  float sum = 0.0f;
  for (int b = 0; b < nb; b++) {
    const uint8_t* qs = wq + b * 16;
    const int8_t* a = aq + b * 32;
    int isum = 0;
    for (int i = 0; i < 16; i++) {
      int lo = (qs[i] & 0x0f) - 8, hi = (qs[i] >> 4) - 8;
      isum += lo * (int)a[i];
      isum += hi * (int)a[i + 16];
    }
    float scale = f16_to_f32(wd[b]) * ad[b];
    sum += scale * (float)isum;
  }
  return sum;
}

// dot_q4_k_q8a (lib.rs:281-315): one sequential chain over the whole row,
// weight = (d*sc)*q - dmin*m, activation = da*qa, sum += weight*activation.
__device__ float row_dot_q4k(const uint8_t* qs, const uint8_t* hdr, const float* af, int nsb) {
  float sum = 0.0f;
  for (int sb = 0; sb < nsb; sb++) {
    const uint8_t* h = hdr + sb * 16;
    float d = f16_to_f32(ld_u16(h)), dmin = f16_to_f32(ld_u16(h + 2));
    for (int sub = 0; sub < 8; sub++) {
      int sc, mn;
      q4k_scale_min(h + 4, sub, &sc, &mn);
      float dsc = d * (float)sc, dm = dmin * (float)mn;
      const uint8_t* q = qs + sb * 128 + (sub / 2) * 32;
      const float* a = af + sb * 256 + sub * 32;
      int shift = (sub & 1) * 4;
      for (int w = 0; w < 32; w++) {
        float weight = dsc * (float)((q[w] >> shift) & 0x0f) - dm;
        sum += weight * a[w];
      }
    }
  }
  return sum;
}

// dot_q6_k_q8k (lib.rs:353-397): exact i32 lane sums (lane = index mod 8)
// per superblock, f32 lane accumulators, sequential lane combine from 0.0.
__device__ float row_dot_q6k(const uint8_t* body, const uint16_t* wd, const int8_t* qk,
                             const float* dk, int nsb) {
  float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int sb = 0; sb < nsb; sb++) {
    const uint8_t* b = body + (size_t)sb * 208;
    const int8_t* a = qk + sb * 256;
    int aux[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    // Q8_K quants are stored class-major: element e sits at (e % 8) * 32 + e / 8.
    for (int e = 0; e < 256; e++)
      aux[e & 7] += q6k_scale(b, e) * (int)a[(e & 7) * 32 + (e >> 3)] * q6k_quant(b, e);
    float d = f16_to_f32(wd[sb]) * dk[sb];
#pragma unroll
    for (int l = 0; l < 8; l++) sums[l] += d * (float)aux[l];
  }
  float sum = 0.0f;
#pragma unroll
  for (int l = 0; l < 8; l++) sum += sums[l];
  return sum;
}

}  // namespace

// ---------------------------------------------------------------------------
// embedding: write_row_validated (det-model lib.rs:667-746)
__global__ void k_embed(DevMat E, const uint32_t* tokens, int T, float* x, int* err) {
  int t = blockIdx.y;
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= T || i >= E.cols) return;
  float v = mat_value(E, (int)tokens[t], i);
  if (!finite(v)) flag(err, ERRBIT_NON_FINITE);
  x[(size_t)t * E.cols + i] = v;
}

void launch_embed(const DevMat& E, const uint32_t* tokens, int T, float* x, int* err,
                  hipStream_t s) {
  dim3 grid((E.cols + 255) / 256, T);
  launch_kernel(k_embed, grid, dim3(256), 0, s, E, tokens, T, x, err);
}

// ---------------------------------------------------------------------------
// Activation quantisation: Q8A (det-quant lib.rs:111-137) per 32-element
// block and Q8_K (lib.rs:139-172) per 256-element block.  One wave
// quantises one 256-element span: lane l holds elements 4l..4l+3, so a Q8A
// block is 8 lanes and a Q8_K block the whole wave; every reduction is a
// wave shuffle.  Spans are whole Q8A blocks (n % 32 == 0) and, when Q8_K is
// wanted, whole Q8_K blocks (n % 256 == 0).

// Four waves per workgroup, one 256-element span each.
__global__ void __launch_bounds__(256) k_quantize(const float* x, int n, int want_q8a,
                                                  int want_q8k, QuantOut q, int* err) {
  const int t = blockIdx.y;
  const int span = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int e = span * 256 + 4 * (threadIdx.x & 63);
  const bool in = e < n;
  float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (in) {
    float4 f = *reinterpret_cast<const float4*>(x + (size_t)t * n + e);
    v[0] = f.x;
    v[1] = f.y;
    v[2] = f.z;
    v[3] = f.w;
    if (!finite(v[0]) || !finite(v[1]) || !finite(v[2]) || !finite(v[3]))
      flag(err, ERRBIT_NON_FINITE);
  }
  if (span * 256 < n)
    quantize_span(v, in, (size_t)t * n + (size_t)span * 256, want_q8a, want_q8k, q);
}

void launch_quantize(const float* x, int T, int n, bool want_q8a, bool want_q8k, int8_t* qa,
                     float* da, float* af, int8_t* qk, float* dk, int* err, hipStream_t s) {
  dim3 grid((n + 1023) / 1024, T);
  QuantOut q{qa, da, af, qk, dk};
  launch_kernel(k_quantize, grid, dim3(256), 0, s, x, n, (int)want_q8a, (int)want_q8k, q, err);
}

// ---------------------------------------------------------------------------
// rmsnorm (det-model lib.rs:2053-2073): ss by 8 interleaved chains, r =
// 1/sqrt(ss/n + eps), out = (x*r)*w.  One workgroup per position.  The
// squares are formed in parallel and stored chain-major in LDS (chain c
// holds x[c]^2, x[c+8]^2, ... contiguously), so each of the eight serial
// chains streams float4 reads.  Optionally quantises the normalised row
// (Q8A / Q8_K) in the same pass, one wave per 256-element span.
namespace {
// Output pass of one 256-element span: (x*r)*w, then the quantised forms.
// w4 holds the span's weights for this lane when have_w4 (else read from w).
// Returns true when a value was non-finite.
__device__ __forceinline__ bool rms_span(const float* xs, const float* w, float4 w4, bool have_w4,
                                         float r, int n, int t, int span, float* o, int want_q8a,
                                         int want_q8k, const QuantOut& q) {
  const int lane = threadIdx.x & 63;
  const int e0 = span * 256 + 4 * lane;
  const bool in = e0 < n;
  const float wl[4] = {w4.x, w4.y, w4.z, w4.w};
  float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  bool bad = false;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    int i = e0 + c;
    if (i < n) {
      float wi = have_w4 ? wl[c] : w[i];
      v[c] = (xs[i] * r) * wi;
      if (!finite(v[c])) bad = true;
      o[i] = v[c];
    }
  }
  if (want_q8a || want_q8k)
    quantize_span(v, in, (size_t)t * n + (size_t)span * 256, want_q8a, want_q8k, q);
  return bad;
}
}  // namespace

__global__ void __launch_bounds__(256) k_rmsnorm(const float* x, const float* w, float eps, int n,
                                                 float* out, int want_q8a, int want_q8k,
                                                 QuantOut q, int* err) {
  extern __shared__ __align__(16) float xs[];  // [n] row, then [8][cs] squares
  __shared__ float lane_sum[8];
  constexpr int kMaxSpansPerWave = 4;  // n <= 4096 keeps w in registers
  const int t = blockIdx.x;
  const int cs = (((n + 7) / 8) + 3) & ~3;    // per-chain stride, float4 aligned
  float* sq = xs + ((n + 3) & ~3);
  const float* xr = x + (size_t)t * n;
  float* o = out + (size_t)t * n;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  bool bad = false;
  // The norm weights this thread scales in the output pass are loaded now,
  // alongside x, so their latency overlaps the sum of squares.
  float wv[kMaxSpansPerWave][4];
  const bool w_in_regs = n <= 4 * 256 * kMaxSpansPerWave;
  if (w_in_regs) {
#pragma unroll
    for (int k = 0; k < kMaxSpansPerWave; k++)
#pragma unroll
      for (int c = 0; c < 4; c++) {
        int i = (wave + 4 * k) * 256 + 4 * lane + c;
        wv[k][c] = i < n ? w[i] : 0.0f;
      }
  }
  // x (and the finiteness of x and w) in float4 batches: every load of a
  // batch is issued before any is used, so the row costs one round trip.
  constexpr int kRowBatch = 4;  // float4 per thread per batch: 4096 elements
  if (n % 4 != 0) {  // rows not float4-aligned (only the kernel-level entry point)
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      const float v = xr[i];
      bad |= any_nonfinite(v, w[i]);
      xs[i] = v;
      sq[(i & 7) * cs + (i >> 3)] = v * v;
    }
  }
  for (int base = 0; n % 4 == 0 && base < n; base += 1024 * kRowBatch) {
    float4 xv[kRowBatch], wq[kRowBatch];
#pragma unroll
    for (int k = 0; k < kRowBatch; k++) {
      const int i = base + 1024 * k + 4 * threadIdx.x;
      xv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
      wq[k] = xv[k];
      if (i < n) {
        xv[k] = *reinterpret_cast<const float4*>(xr + i);
        wq[k] = *reinterpret_cast<const float4*>(w + i);
      }
    }
#pragma unroll
    for (int k = 0; k < kRowBatch; k++) {
      const int i = base + 1024 * k + 4 * threadIdx.x;
      if (i < n) {
        const float xe[4] = {xv[k].x, xv[k].y, xv[k].z, xv[k].w};
        const float we[4] = {wq[k].x, wq[k].y, wq[k].z, wq[k].w};
        *reinterpret_cast<float4*>(xs + i) = xv[k];
#pragma unroll
        for (int c = 0; c < 4; c++) {
          bad |= any_nonfinite(xe[c], we[c]);
          sq[((i & 7) + c) * cs + (i >> 3)] = xe[c] * xe[c];
        }
      }
    }
  }
  __syncthreads();
  if (n % 8 == 0) {
    // the eight chains on the DPP rows of waves 0 and 1
    if (wave < 2) {
      const int c = 4 * wave + (lane >> 4);
      const float sum = chain_group_lds<16>(0.0f, sq + c * cs, n / 8);
      if ((lane & 15) == 0) lane_sum[c] = sum;
    }
  } else if (threadIdx.x < 8) {
    const int c = threadIdx.x;  // elements c, c+8, ... below n
    lane_sum[c] = chain_sum_lds(0.0f, sq + c * cs, (n - c + 7) / 8);
  }
  __syncthreads();
  // every thread forms r from the eight sums (no thread-0 pass and barrier)
  const float ss = finish_8lane(lane_sum);
  const float m = ss / (float)n;
  const float r = 1.0f / sqrtf(m + eps);
  if (!finite(r)) bad = true;
#pragma unroll
  for (int k = 0; k < kMaxSpansPerWave; k++) {
    const int span = wave + 4 * k;
    if (span * 256 >= n) break;
    float4 w4 = w_in_regs ? make_float4(wv[k][0], wv[k][1], wv[k][2], wv[k][3])
                          : make_float4(0.f, 0.f, 0.f, 0.f);
    bad |= rms_span(xs, w, w4, w_in_regs, r, n, t, span, o, want_q8a, want_q8k, q);
  }
  for (int span = wave + 4 * kMaxSpansPerWave; span * 256 < n; span += 4)
    bad |= rms_span(xs, w, make_float4(0.f, 0.f, 0.f, 0.f), false, r, n, t, span, o, want_q8a,
                    want_q8k, q);
  if (bad) flag(err, ERRBIT_NON_FINITE);
}

size_t rmsnorm_smem(int n) {
  return ((size_t)((n + 3) & ~3) + 8 * (size_t)((((n + 7) / 8) + 3) & ~3)) * sizeof(float);
}

void launch_rmsnorm_quant(const float* x, const float* w, float eps, int T, int n, float* out,
                          bool want_q8a, bool want_q8k, int8_t* qa, float* da, float* af,
                          int8_t* qk, float* dk, int* err, hipStream_t s) {
  QuantOut q{qa, da, af, qk, dk};
  static bool attr_set = false;
  if (!attr_set) {
    (void)hipFuncSetAttribute((const void*)k_rmsnorm, hipFuncAttributeMaxDynamicSharedMemorySize,
                              150 * 1024);
    attr_set = true;
  }
  launch_kernel(k_rmsnorm, dim3(T), dim3(256), rmsnorm_smem(n), s, x, w, eps, n, out,
                     (int)want_q8a, (int)want_q8k, q, err);
}

void launch_rmsnorm(const float* x, const float* w, float eps, int T, int n, float* out, int* err,
                    hipStream_t s) {
  launch_rmsnorm_quant(x, w, eps, T, n, out, false, false, nullptr, nullptr, nullptr, nullptr,
                       nullptr, err, s);
}

// ---------------------------------------------------------------------------
// GEMM: out[t][r] = row r . activation t, one lane per (r, t), with the
// bias add (add_optional_bias, lib.rs:1982-1998) or residual add
// (residual_add, lib.rs:1967-1980) applied to the finished dot.
__global__ void __launch_bounds__(256) k_gemm_rowlane(DevMat W, DevAct A, int T, float* out,
                                                      const float* bias, int epi, int* err) {
  int r = blockIdx.x * blockDim.x + threadIdx.x;
  int t = blockIdx.y;
  if (r >= W.rows || t >= T) return;
  float v;
  switch (W.type) {
    case kGgmlF32:
      v = row_dot_f32((const float*)W.w + (size_t)r * W.cols, A.x + (size_t)t * W.cols, W.cols);
      break;
    case kGgmlQ8_0:
      v = row_dot_q8_0((const int8_t*)W.w + (size_t)r * W.cols, W.d16 + (size_t)r * W.nb,
                       A.qa + (size_t)t * W.cols, A.da + (size_t)t * (W.cols / 32), W.nb);
      break;
    case kGgmlQ4_0:
      v = row_dot_q4_0((const uint8_t*)W.w + (size_t)r * W.nb * 16, W.d16 + (size_t)r * W.nb,
                       A.qa + (size_t)t * W.cols, A.da + (size_t)t * (W.cols / 32), W.nb);
      break;
    case kGgmlQ4K:
      v = row_dot_q4k((const uint8_t*)W.w + (size_t)r * W.nb * 128, W.hdr + (size_t)r * W.nb * 16,
                      A.af + (size_t)t * W.cols, W.nb);
      break;
    default:
      v = row_dot_q6k((const uint8_t*)W.w + (size_t)r * W.nb * 208, W.d16 + (size_t)r * W.nb,
                      A.qk + (size_t)t * W.cols, A.dk + (size_t)t * (W.cols / 256), W.nb);
      break;
  }
  bool bad = !finite(v);
  size_t o = (size_t)t * W.rows + r;
  if (epi == EPI_BIAS) {
    v = v + bias[r];
  } else if (epi == EPI_RESIDUAL) {
    v = out[o] + v;
  }
  if (bad || !finite(v)) flag(err, ERRBIT_NON_FINITE);
  out[o] = v;
}

void launch_gemm(const DevMat& W, const DevAct& A, int T, float* out, const float* bias, int epi,
                 int* err, hipStream_t s) {
  // Chunks of positions take the token-parallel kernels (weights decoded once
  // per wave and shared by up to 64 positions); short batches keep one lane
  // per (row, position).
  if (gemm_tok_supported(W) && (T >= 16 || (W.type == kGgmlQ6K && T >= 2))) {
    launch_gemm_tok(W, A, T, out, bias, epi, err, s);
    return;
  }
  if (T <= kGemvMaxT && launch_gemv(W, A, T, out, bias, epi, err, s)) return;
  dim3 grid((W.rows + 255) / 256, T);
  launch_kernel(k_gemm_rowlane, grid, dim3(256), 0, s, W, A, T, out, bias, epi, err);
}

// ---------------------------------------------------------------------------
// apply_rope on q and k (det-model lib.rs:2011-2051) and KvCache::store
// (lib.rs:883-920).  One workgroup per position.
__global__ void __launch_bounds__(256) k_rope_store(float* q, float* k, const float* v,
                                                    const float* rc, const float* rs, int pos0,
                                                    int H, int KV, int hd, int rope_dim,
                                                    int split_half, float* kc, float* vc,
                                                    int layer, int n_ctx, const int* pos_dev,
                                                    int* err) {
  // One pass without barriers: every rotation pair is read, checked,
  // rotated and written by one thread (a key pair also into the cache), and
  // every element outside the pairs and every value is copied by one thread.
  int t = blockIdx.x;
  int pos = (pos_dev ? *pos_dev : pos0) + t;
  int half = rope_dim / 2;
  bool bad = false;
  float* qt = q + (size_t)t * H * hd;
  float* kt = k + (size_t)t * KV * hd;
  const float* vt = v + (size_t)t * KV * hd;
  const float* ct = rc + (size_t)pos * half;
  const float* st = rs + (size_t)pos * half;
  auto cache = [&](int kvh, int dd) { return (((size_t)layer * KV + kvh) * n_ctx + pos) * hd + dd; };
  for (int p = threadIdx.x; p < (H + KV) * half; p += blockDim.x) {
    int head = p / half, j = p % half;
    float* base = head < H ? qt + head * hd : kt + (head - H) * hd;
    int a = split_half ? j : 2 * j;
    int b = split_half ? j + half : 2 * j + 1;
    float x0 = base[a], x1 = base[b];
    float c = ct[j], s = st[j];
    float y0 = x0 * c - x1 * s;
    float y1 = x0 * s + x1 * c;
    if (!finite(x0) || !finite(x1) || !finite(y0) || !finite(y1)) bad = true;
    base[a] = y0;
    base[b] = y1;
    if (head >= H) {
      kc[cache(head - H, a)] = y0;
      kc[cache(head - H, b)] = y1;
    }
  }
  // dimensions past the rotated pairs (rope_dim < hd), unchanged
  const int r0 = 2 * half, rest = hd - r0;
  for (int i = threadIdx.x; i < (H + KV) * rest; i += blockDim.x) {
    int head = i / rest, dd = r0 + i % rest;
    float x = head < H ? qt[head * hd + dd] : kt[(head - H) * hd + dd];
    if (!finite(x)) bad = true;
    if (head >= H) kc[cache(head - H, dd)] = x;
  }
  for (int i = threadIdx.x; i < KV * hd; i += blockDim.x) {
    float vv = vt[i];
    if (!finite(vv)) bad = true;
    vc[cache(i / hd, i % hd)] = vv;
  }
  if (bad) flag(err, ERRBIT_NON_FINITE);
}

void launch_rope_store(float* q, float* k, const float* v, const float* rope_cos,
                       const float* rope_sin, int T, int pos0, int H, int KV, int hd, int rope_dim,
                       int split_half, float* kc, float* vc, int layer, int n_ctx,
                       const int* pos_dev, int* err, hipStream_t s) {
  launch_kernel(k_rope_store, dim3(T), dim3(256), 0, s, q, k, v, rope_cos, rope_sin, pos0, H,
                     KV, hd, rope_dim, split_half, kc, vc, layer, n_ctx, pos_dev, err);
}

// ---------------------------------------------------------------------------
// attention_one_head (det-model lib.rs:2300-2418) for every (head, position)
// of the chunk: causal over cache positions 0..pos.  One wave per pair.
__global__ void __launch_bounds__(64) k_attention(const float* q, const float* kc, const float* vc,
                                                  int layer, int pos0, int H, int KV, int hd,
                                                  int n_ctx, float scale, float* scores,
                                                  float* out, int* err) {
  int h = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
  int pos = pos0 + t, len = pos + 1;
  int kvh = h / (H / KV);
  const float* keys = kc + ((size_t)layer * KV + kvh) * n_ctx * hd;
  const float* vals = vc + ((size_t)layer * KV + kvh) * n_ctx * hd;
  float* o = out + (size_t)t * H * hd + (size_t)h * hd;
  if (len == 1) {  // a single score copies V exactly (lib.rs:2319-2321)
    for (int dd = lane; dd < hd; dd += 64) o[dd] = vals[dd];
    return;
  }
  const float* qh = q + (size_t)t * H * hd + (size_t)h * hd;
  float* sc = scores + ((size_t)t * H + h) * n_ctx;
  bool bad = false;
  // scores: dot_f32_ref(q, k_j) * scale
  float mx = -__builtin_huge_valf();
  for (int j = lane; j < len; j += 64) {
    const float* kj = keys + (size_t)j * hd;
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = 0; i < hd; i++) acc[i & 7] += qh[i] * kj[i];
    float s = finish_8lane(acc) * scale;
    if (!finite(s)) bad = true;
    sc[j] = s;
    mx = fmaxf(mx, s);
  }
  mx = wave_fmax(mx);
  for (int j = lane; j < len; j += 64) sc[j] = exp_clamped(sc[j] - mx);
  __syncthreads();
  // Z = sum_f32_ref(e): lane c < 8 walks chain c in ascending order.
  float acc = 0.0f;
  if (lane < 8)
    for (int j = lane; j < len; j += 8) acc += sc[j];
  float part[8];
#pragma unroll
  for (int c = 0; c < 8; c++) part[c] = __shfl(acc, c);
  float z = finish_8lane(part);
  if (!finite(z) || z == 0.0f) bad = true;
  __syncthreads();
  for (int j = lane; j < len; j += 64) {
    float p = sc[j] / z;
    if (!finite(p)) bad = true;
    sc[j] = p;
  }
  __syncthreads();
  // P.V: out[d] = 0.0; out[d] += p_j * v_j[d] for j ascending.
  for (int dd = lane; dd < hd; dd += 64) {
    float a = 0.0f;
    for (int j = 0; j < len; j++) a += sc[j] * vals[(size_t)j * hd + dd];
    if (!finite(a)) bad = true;
    o[dd] = a;
  }
  if (bad) flag(err, ERRBIT_NON_FINITE);
}

// The same computation with the heads of one KV group in one workgroup
// (one wave per head): K and V tiles of 64 positions are staged once in LDS
// for the whole group, K transposed so lane j reads key j conflict-free.
// Scores and probabilities of every head stay in LDS.
constexpr int kAttnTile = 64;

__global__ void __launch_bounds__(1024) k_attention_grp(const float* q, const float* kc,
                                                        const float* vc, int layer, int pos0,
                                                        int H, int KV, int hd, int n_ctx,
                                                        float scale, float* out, int* err) {
  extern __shared__ __align__(16) float smem[];
  const int G = H / KV;
  const int g = blockIdx.x, t = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int h = g * G + wave;
  const int pos = pos0 + t, len = pos + 1;
  const int nthreads = G * 64;
  const float* keys = kc + ((size_t)layer * KV + g) * n_ctx * hd;
  const float* vals = vc + ((size_t)layer * KV + g) * n_ctx * hd;
  float* o = out + (size_t)t * H * hd + (size_t)h * hd;
  if (len == 1) {  // a single score copies V exactly (lib.rs:2319-2321)
    for (int dd = lane; dd < hd; dd += 64) o[dd] = vals[dd];
    return;
  }
  float* sc = smem;                          // [G][n_ctx]
  float* tile = sc + (size_t)G * n_ctx;      // K^T [hd][kAttnTile + 1] or V [kAttnTile][hd]
  float* qs = tile + (kAttnTile + 1) * hd;   // [G][hd]
  float* my = sc + (size_t)wave * n_ctx;
  bool bad = false;
  const float* qh = q + (size_t)t * H * hd + (size_t)h * hd;
  for (int i = lane; i < hd; i += 64) qs[wave * hd + i] = qh[i];
  // scores: dot_f32_ref(q, k_j) * scale
  for (int j0 = 0; j0 < len; j0 += kAttnTile) {
    int n = len - j0 < kAttnTile ? len - j0 : kAttnTile;
    __syncthreads();
    for (int x = threadIdx.x; x < n * hd; x += nthreads) {
      int j = x / hd, i = x % hd;
      tile[i * (kAttnTile + 1) + j] = keys[(size_t)(j0 + j) * hd + i];
    }
    __syncthreads();
    if (lane < n) {
      float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      const float* qw = qs + wave * hd;
      for (int i = 0; i < hd; i++) acc[i & 7] += qw[i] * tile[i * (kAttnTile + 1) + lane];
      float s = finish_8lane(acc) * scale;
      if (!finite(s)) bad = true;
      my[j0 + lane] = s;
    }
  }
  __syncthreads();
  // softmax_in_place (lib.rs:2361-2388), per wave
  float mx = -__builtin_huge_valf();
  for (int j = lane; j < len; j += 64) mx = fmaxf(mx, my[j]);
  mx = wave_fmax(mx);
  for (int j = lane; j < len; j += 64) my[j] = exp_clamped(my[j] - mx);
  __syncthreads();
  float acc = 0.0f;
  if (lane < 8)
    for (int j = lane; j < len; j += 8) acc += my[j];
  float part[8];
#pragma unroll
  for (int c = 0; c < 8; c++) part[c] = __shfl(acc, c);
  float z = finish_8lane(part);
  if (!finite(z) || z == 0.0f) bad = true;
  for (int j = lane; j < len; j += 64) {
    float p = my[j] / z;
    if (!finite(p)) bad = true;
    my[j] = p;
  }
  // P.V: out[d] = 0.0; out[d] += p_j * v_j[d] for j ascending
  float av[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int j0 = 0; j0 < len; j0 += kAttnTile) {
    int n = len - j0 < kAttnTile ? len - j0 : kAttnTile;
    __syncthreads();
    for (int x = threadIdx.x; x < n * hd; x += nthreads) tile[x] = vals[(size_t)j0 * hd + x];
    __syncthreads();
#pragma unroll
    for (int c = 0; c < 4; c++) {
      int dd = lane + 64 * c;
      if (dd < hd) {
        float a = av[c];
        for (int j = 0; j < n; j++) a += my[j0 + j] * tile[j * hd + dd];
        av[c] = a;
      }
    }
  }
#pragma unroll
  for (int c = 0; c < 4; c++) {
    int dd = lane + 64 * c;
    if (dd < hd) {
      if (!finite(av[c])) bad = true;
      o[dd] = av[c];
    }
  }
  if (bad) flag(err, ERRBIT_NON_FINITE);
}

// Head dimension 64 (every Llama/Qwen shape served here): the same
// arithmetic as k_attention_grp.  One workgroup per (KV group, position),
// one wave per head of the group.  K and V stream through LDS in 64-row
// tiles (K transposed); each thread holds PER float4 of a tile, and a ring of
// D tiles is in flight in registers, so a tile's global loads have D tiles
// of compute to land (one tile of compute is far shorter than one HBM/L2
// round trip).  The serial chains (the softmax Z and P.V, one per lane) read
// sixteen operands from LDS ahead of their adds.
constexpr int kA64Tile = 64;           // K/V rows per tile
constexpr int kA64KStride = 65;        // K^T row stride (conflict-free column reads)
constexpr int kA64Buf = 64 * kA64KStride;

template <int PER, int D, int NT>
__global__ void __launch_bounds__(NT) k_attention_hd64(const float* q, const float* kc,
                                                         const float* vc, int layer, int pos0,
                                                         int H, int KV, int n_ctx, int sc_stride,
                                                         float scale, float* out, QuantOut oq,
                                                         int* err) {
  extern __shared__ __align__(16) float smem[];
  constexpr int hd = 64;
  const int G = H / KV;
  const int g = blockIdx.x, t = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int h = g * G + wave;
  const int pos = pos0 + t, len = pos + 1;
  const int nthreads = G * 64;
  const float* keys = kc + ((size_t)layer * KV + g) * n_ctx * hd;
  const float* vals = vc + ((size_t)layer * KV + g) * n_ctx * hd;
  float* o = out + (size_t)t * H * hd + (size_t)h * hd;
  // With oq.qa set, the wave also writes the Q8A form of its head's output
  // (the input of wo): two 32-element blocks per head.
  const size_t qbase = (size_t)t * H * hd + (size_t)h * hd;
  if (len == 1) {  // a single score copies V exactly (lib.rs:2319-2321)
    const float v0 = vals[lane];
    o[lane] = v0;
    if (oq.qa) quantize_q8a_lanes(v0, qbase, oq);
    return;
  }
  float* sc = smem;                                // [G][sc_stride]
  float* tiles = sc + (size_t)G * sc_stride;       // [2][kA64Buf]
  float* qs = tiles + 2 * kA64Buf;                 // [G][64]
  float* my = sc + (size_t)wave * sc_stride;
  bool bad = false;
  qs[wave * hd + lane] = q[(size_t)t * H * hd + (size_t)h * hd + lane];
  // With up to 512 threads there are registers for the whole query row in
  // every lane (read once from memory, the same address for the wave), so
  // the score loop reads only keys from LDS.
  constexpr bool kQReg = NT <= 512;
  float qr[kQReg ? 64 : 1];
  if constexpr (kQReg) {
    const float4* qg = reinterpret_cast<const float4*>(q + (size_t)t * H * hd + (size_t)h * hd);
#pragma unroll
    for (int i4 = 0; i4 < 16; i4++) {
      const float4 v = qg[i4];
      qr[4 * i4 + 0] = v.x;
      qr[4 * i4 + 1] = v.y;
      qr[4 * i4 + 2] = v.z;
      qr[4 * i4 + 3] = v.w;
    }
  }
  const int ntiles = (len + kA64Tile - 1) / kA64Tile;
  // Tile loads: float4 index x = threadIdx.x + c * nthreads covers row
  // x / 16, columns 4 * (x % 16); rows at or past len are not read.
  float4 ring[D][PER];
  // Loads are unconditional (slots past the tile or the row range read row
  // 0, which commit never stores), so the compiler counts the loads in
  // flight instead of draining them at every tile.
  auto issue = [&](float4 (&dst)[PER], const float* base, int j0) {
    // At 1024 threads (128 registers) the lane's thread index goes through
    // an empty asm, so the V phase's per-lane addresses are formed where they
    // are used rather than held from the kernel's start (they went to scratch)
    int tx = threadIdx.x;
    if constexpr (NT > 512) asm volatile("" : "+v"(tx));
#pragma unroll
    for (int c = 0; c < PER; c++) {
      const int x = tx + c * nthreads;
      const int j = x >> 4;
      const bool ok = x < 1024 && j0 + j < len;
      dst[c] = *reinterpret_cast<const float4*>(base + (size_t)(ok ? j0 + j : 0) * hd + (x & 15) * 4);
    }
  };
  auto commit_k = [&](const float4 (&src)[PER], float* buf, int j0) {
#pragma unroll
    for (int c = 0; c < PER; c++) {
      const int x = threadIdx.x + c * nthreads;
      const int j = x >> 4, i = (x & 15) * 4;
      if (x < 1024 && j0 + j < len) {
        buf[(i + 0) * kA64KStride + j] = src[c].x;
        buf[(i + 1) * kA64KStride + j] = src[c].y;
        buf[(i + 2) * kA64KStride + j] = src[c].z;
        buf[(i + 3) * kA64KStride + j] = src[c].w;
      }
    }
  };
  auto commit_v = [&](const float4 (&src)[PER], float* buf, int j0) {
#pragma unroll
    for (int c = 0; c < PER; c++) {
      const int x = threadIdx.x + c * nthreads;
      if (x < 1024 && j0 + (x >> 4) < len) reinterpret_cast<float4*>(buf)[x] = src[c];
    }
  };
  // scores: dot_f32_ref(q, k_j) * scale.  Tile k sits in ring slot k % D.
#pragma unroll
  for (int u = 0; u < D; u++) issue(ring[u], keys, u * kA64Tile);
  commit_k(ring[0], tiles, 0);
  issue(ring[0], keys, D * kA64Tile);
  __syncthreads();
  for (int k0 = 0; k0 < ntiles; k0 += D) {
#pragma unroll
    for (int u = 0; u < D; u++) {
      const int k = k0 + u;
      if (k < ntiles) {
        const int j0 = k * kA64Tile;
        const float* cur = tiles + (k & 1) * kA64Buf;
        if (j0 + lane < len) {
          float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
          if constexpr (kQReg) {
            // the key column read in one batch, then 64 multiply-adds
            float kv[64];
#pragma unroll
            for (int i = 0; i < 64; i++) kv[i] = cur[i * kA64KStride + lane];
#pragma unroll
            for (int i = 0; i < 64; i++) acc[i & 7] += qr[i] * kv[i];
          } else {
            const float4* qw = reinterpret_cast<const float4*>(qs + wave * hd);
#pragma unroll
            for (int i4 = 0; i4 < 16; i4++) {
              const float4 qv = qw[i4];
              const int i = i4 * 4;
              acc[(i + 0) & 7] += qv.x * cur[(i + 0) * kA64KStride + lane];
              acc[(i + 1) & 7] += qv.y * cur[(i + 1) * kA64KStride + lane];
              acc[(i + 2) & 7] += qv.z * cur[(i + 2) * kA64KStride + lane];
              acc[(i + 3) & 7] += qv.w * cur[(i + 3) * kA64KStride + lane];
            }
          }
          const float sv = finish_8lane(acc) * scale;
          if (!finite(sv)) bad = true;
          my[j0 + lane] = sv;
        }
        // tile k + 1 into the other buffer (its last reader, tile k - 1,
        // finished before the previous barrier); its slot then takes
        // tile k + 1 + D
        if (k + 1 < ntiles) commit_k(ring[(u + 1) % D], tiles + ((k + 1) & 1) * kA64Buf, j0 + kA64Tile);
      }
      issue(ring[(u + 1) % D], keys, (k0 + u + 1 + D) * kA64Tile);
      __syncthreads();
    }
  }
  // The first V tiles' loads overlap the softmax.
#pragma unroll
  for (int u = 0; u < D; u++) issue(ring[u], vals, u * kA64Tile);
  // softmax_in_place (lib.rs:2361-2388), per wave
  float mx = -__builtin_huge_valf();
  for (int j = lane; j < len; j += 64) mx = fmaxf(mx, my[j]);
  mx = wave_fmax(mx);
  for (int j = lane; j < len; j += 64) my[j] = exp_clamped(my[j] - mx);
  __syncthreads();
  float zacc = 0.0f;
  if (lane < 8) {
    int j = lane;
    for (; j + 8 * 15 < len; j += 8 * 16) {
      float e[16];
#pragma unroll
      for (int k = 0; k < 16; k++) e[k] = my[j + 8 * k];
#pragma unroll
      for (int k = 0; k < 16; k++) zacc += e[k];
    }
    for (; j < len; j += 8) zacc += my[j];
  }
  float part[8];
#pragma unroll
  for (int c = 0; c < 8; c++) part[c] = __shfl(zacc, c);
  const float z = finish_8lane(part);
  if (!finite(z) || z == 0.0f) bad = true;
  for (int j = lane; j < len; j += 64) {
    const float p = my[j] / z;
    if (!finite(p)) bad = true;
    my[j] = p;
  }
  commit_v(ring[0], tiles, 0);
  issue(ring[0], vals, D * kA64Tile);
  __syncthreads();
  // P.V: out[d] = 0.0; out[d] += p_j * v_j[d] for j ascending
  float a = 0.0f;
  for (int k0 = 0; k0 < ntiles; k0 += D) {
#pragma unroll
    for (int u = 0; u < D; u++) {
      const int k = k0 + u;
      if (k < ntiles) {
        const int j0 = k * kA64Tile;
        const int n = len - j0 < kA64Tile ? len - j0 : kA64Tile;
        const float* cur = tiles + (k & 1) * kA64Buf;
        if (n == kA64Tile) {
#pragma unroll
          for (int jb = 0; jb < kA64Tile; jb += 16) {
            float v[16];
            float4 pv[4];
#pragma unroll
            for (int kk = 0; kk < 16; kk++) v[kk] = cur[(jb + kk) * hd + lane];
#pragma unroll
            for (int kk = 0; kk < 4; kk++) pv[kk] = reinterpret_cast<const float4*>(my + j0 + jb)[kk];
#pragma unroll
            for (int kk = 0; kk < 4; kk++) {
              a += pv[kk].x * v[4 * kk + 0];
              a += pv[kk].y * v[4 * kk + 1];
              a += pv[kk].z * v[4 * kk + 2];
              a += pv[kk].w * v[4 * kk + 3];
            }
          }
        } else {
          for (int j = 0; j < n; j++) a += my[j0 + j] * cur[j * hd + lane];
        }
        if (k + 1 < ntiles) commit_v(ring[(u + 1) % D], tiles + ((k + 1) & 1) * kA64Buf, j0 + kA64Tile);
      }
      issue(ring[(u + 1) % D], vals, (k0 + u + 1 + D) * kA64Tile);
      __syncthreads();
    }
  }
  if (!finite(a)) bad = true;
  o[lane] = a;
  if (oq.qa) quantize_q8a_lanes(a, qbase, oq);
  if (bad) flag(err, ERRBIT_NON_FINITE);
}

// Head dimension 64 and at most eight heads per KV group: the arithmetic of
// k_attention_hd64 with the lanes split over keys and heads.  Eight waves
// per (KV group, position), each staging its own share of every 64-key tile
// in a private LDS area, so the scores and P.V phases run without
// workgroup barriers (one between the phases); each wave keeps D tiles of
// its global loads in flight in registers.
//   scores  wave w takes keys 8w..8w+7 of each tile, lane = (key lane % 8,
//           head lane / 8); a lane holds its head's query row in registers
//           and reads its key's row (row-major in the wave's area) as float4.
//   softmax wave h < G over head h's scores (max, exp_f32, the 8-lane sum,
//           the divisions), eight elements per lane in flight.
//   P.V     lane = (head lane / 8, dimension 8w + lane % 8); the wave stores
//           its eight dimensions of the tile's values transposed, so a lane
//           reads four keys' values of its dimension and its head's four
//           probabilities as two float4, in key order.
constexpr int kS64Stride = 68;  // key rows and value columns (floats) of a wave's area
constexpr int kS64Buf = 64 * kS64Stride;

__host__ __device__ constexpr int attn_split_lane_stride(int len_max) {
  return ((len_max + 63) & ~63) + 4;  // 8 probability rows x float4 on 32 banks
}

namespace {
// Orders one wave's LDS stores before its lanes' later loads of them.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
}  // namespace

template <int D>
__global__ void __launch_bounds__(512) k_attention_hd64s(const float* q, const float* kc,
                                                       const float* vc, int layer, int pos0,
                                                       int H, int KV, int n_ctx, int scs,
                                                       float scale, float* out, QuantOut oq,
                                                       int* err) {
  extern __shared__ __align__(16) float smem[];
  constexpr int hd = 64;
  const int G = H / KV;
  const int g = blockIdx.x, t = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int pos = pos0 + t, len = pos + 1;
  const float* keys = kc + ((size_t)layer * KV + g) * n_ctx * hd;
  const float* vals = vc + ((size_t)layer * KV + g) * n_ctx * hd;
  if (len == 1) {  // a single score copies V exactly (lib.rs:2319-2321)
    if (wave < G) {
      const int h = g * G + wave;
      const float v0 = vals[lane];
      out[(size_t)t * H * hd + (size_t)h * hd + lane] = v0;
      if (oq.qa) quantize_q8a_lanes(v0, (size_t)t * H * hd + (size_t)h * hd, oq);
    }
    return;
  }
  float* sc = smem;                                  // [G][scs] scores -> probabilities
  float* pb = sc + (size_t)G * scs + (size_t)wave * 8 * kS64Stride;  // this wave's [8][68]
  bool bad = false;
  const int kk = lane & 7, hh = lane >> 3;  // scores: key and head of the lane
  const int hq = hh < G ? hh : 0;
  float qr[64];
  {
    const float4* qg = reinterpret_cast<const float4*>(q + (size_t)t * H * hd + (size_t)(g * G + hq) * hd);
#pragma unroll
    for (int i4 = 0; i4 < 16; i4++) {
      const float4 v = qg[i4];
      qr[4 * i4 + 0] = v.x;
      qr[4 * i4 + 1] = v.y;
      qr[4 * i4 + 2] = v.z;
      qr[4 * i4 + 3] = v.w;
    }
  }
  const int ntiles = (len + 63) / 64;
  float4 ring[D][2];
  // Key rows 64 k + 8 wave + f / 16 (float4 f % 16) for f = lane, lane + 64;
  // rows past len read row 0 and are not used.
  auto issue_k = [&](float4 (&dst)[2], int k) {
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const int f = lane + 64 * c;
      const int j = 64 * k + 8 * wave + (f >> 4);
      dst[c] = *reinterpret_cast<const float4*>(keys + (size_t)(j < len ? j : 0) * hd + (f & 15) * 4);
    }
  };
  // Value row 64 k + lane, dimensions 8 wave .. 8 wave + 7.
  auto issue_v = [&](float4 (&dst)[2], int k) {
    const int j = 64 * k + lane;
#pragma unroll
    for (int c = 0; c < 2; c++)
      dst[c] = *reinterpret_cast<const float4*>(vals + (size_t)(j < len ? j : 0) * hd + 8 * wave + 4 * c);
  };
  // scores: dot_f32_ref(q, k_j) * scale (8-lane order).  Tile k sits in ring
  // slot k % D.  Every pass stores and refills its slot, past the last tile
  // too: with the refill under a branch the compiler waits for every load
  // in flight there, and the ring would hold one tile.  Each lane also keeps
  // the maximum of its scores (fmax is exact in any order).
  float lmax = -__builtin_huge_valf();
  // issued in slot order (the scheduler would otherwise reorder them, and the
  // loop's first wait would then cover every slot)
#pragma unroll
  for (int u = 0; u < D; u++) {
    issue_k(ring[u], u);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int k0 = 0; k0 < ntiles; k0 += D) {
#pragma unroll
    for (int u = 0; u < D; u++) {
      const int k = k0 + u;
#pragma unroll
      for (int c = 0; c < 2; c++) {
        const int f = lane + 64 * c;
        *reinterpret_cast<float4*>(pb + (f >> 4) * kS64Stride + (f & 15) * 4) = ring[u][c];
      }
      wave_lds_sync();
      issue_k(ring[u], k + D);
      const int j = 64 * k + 8 * wave + kk;
      if (j < len && hh < G) {
        const float* kr = pb + kk * kS64Stride;
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int i4 = 0; i4 < 16; i4++) {
          const float4 kv = *reinterpret_cast<const float4*>(kr + 4 * i4);
          const int i = 4 * i4;
          acc[(i + 0) & 7] += qr[i + 0] * kv.x;
          acc[(i + 1) & 7] += qr[i + 1] * kv.y;
          acc[(i + 2) & 7] += qr[i + 2] * kv.z;
          acc[(i + 3) & 7] += qr[i + 3] * kv.w;
        }
        const float sv = finish_8lane(acc) * scale;
        if (!finite(sv)) bad = true;
        lmax = fmaxf(lmax, sv);
        sc[(size_t)hh * scs + j] = sv;
      }
      wave_lds_sync();
    }
  }
  // the head's maximum over the wave's eight key lanes, then (below) over the waves
  lmax = fmaxf(lmax, dpp_f32<kDppXor1>(lmax));
  lmax = fmaxf(lmax, dpp_f32<kDppXor2>(lmax));
  lmax = fmaxf(lmax, dpp_f32<kDppMirror8>(lmax));
  if (kk == 0) pb[hh] = lmax;  // the wave's own area, free until P.V
  // The first V tiles' loads overlap the softmax.
#pragma unroll
  for (int u = 0; u < D; u++) issue_v(ring[u], u);
  __syncthreads();
  // softmax_in_place (lib.rs:2361-2388), wave h for head h.  Loads are
  // clamped to the row, stores past it skipped, so no load sits under a
  // per-element branch.
  if (wave < G) {
    constexpr int U = 8;  // elements per lane in flight
    float* my = sc + (size_t)wave * scs;
    float mx = -__builtin_huge_valf();
#pragma unroll
    for (int w = 0; w < 8; w++) mx = fmaxf(mx, sc[(size_t)G * scs + (size_t)w * 8 * kS64Stride + wave]);
    for (int j0 = lane; j0 < len; j0 += 64 * U) {
      float e[U];
#pragma unroll
      for (int c = 0; c < U; c++) {
        const int j = j0 + 64 * c;
        e[c] = my[j < len ? j : len - 1];
      }
#pragma unroll
      for (int c = 0; c < U; c++) e[c] = exp_clamped(e[c] - mx);
#pragma unroll
      for (int c = 0; c < U; c++)
        if (j0 + 64 * c < len) my[j0 + 64 * c] = e[c];
    }
    wave_lds_sync();
    float zacc = 0.0f;
    if (lane < 8) {
      int j = lane;
      for (; j + 8 * 15 < len; j += 8 * 16) {
        float e[16];
#pragma unroll
        for (int c = 0; c < 16; c++) e[c] = my[j + 8 * c];
#pragma unroll
        for (int c = 0; c < 16; c++) zacc += e[c];
      }
      for (; j < len; j += 8) zacc += my[j];
    }
    float part[8];
#pragma unroll
    for (int c = 0; c < 8; c++) part[c] = __shfl(zacc, c);
    const float z = finish_8lane(part);
    if (!finite(z) || z == 0.0f) bad = true;
    for (int j0 = lane; j0 < len; j0 += 64 * U) {
      float e[U];
#pragma unroll
      for (int c = 0; c < U; c++) {
        const int j = j0 + 64 * c;
        e[c] = my[j < len ? j : len - 1];
      }
#pragma unroll
      for (int c = 0; c < U; c++) e[c] = e[c] / z;
#pragma unroll
      for (int c = 0; c < U; c++)
        if (j0 + 64 * c < len) {
          if (!finite(e[c])) bad = true;
          my[j0 + 64 * c] = e[c];
        }
    }
  }
  __syncthreads();
  // P.V: out[d] = 0.0; out[d] += p_j * v_j[d] for j ascending.  As in the
  // scores, every pass stores and refills its ring slot.
  const int ph = lane >> 3, pd = lane & 7;  // head, dimension 8 wave + pd
  const float* prow = sc + (size_t)(ph < G ? ph : 0) * scs;
  const float* vr = pb + pd * kS64Stride;
  float a = 0.0f;
  for (int k0 = 0; k0 < ntiles; k0 += D) {
#pragma unroll
    for (int u = 0; u < D; u++) {
      const int k = k0 + u;
      // the wave's eight dimensions of value rows 64 k .. 64 k + 63, transposed
#pragma unroll
      for (int c = 0; c < 2; c++) {
        pb[(4 * c + 0) * kS64Stride + lane] = ring[u][c].x;
        pb[(4 * c + 1) * kS64Stride + lane] = ring[u][c].y;
        pb[(4 * c + 2) * kS64Stride + lane] = ring[u][c].z;
        pb[(4 * c + 3) * kS64Stride + lane] = ring[u][c].w;
      }
      wave_lds_sync();
      issue_v(ring[u], k + D);
      if (k < ntiles) {
        const int j0 = k * 64;
        const int n = len - j0 < 64 ? len - j0 : 64;
        const float* pr = prow + j0;
        if (n == 64) {
#pragma unroll
          for (int jb = 0; jb < 64; jb += 4) {
            const float4 v4 = *reinterpret_cast<const float4*>(vr + jb);
            const float4 p4 = *reinterpret_cast<const float4*>(pr + jb);
            a += p4.x * v4.x;
            a += p4.y * v4.y;
            a += p4.z * v4.z;
            a += p4.w * v4.w;
          }
        } else {
          for (int j = 0; j < n; j++) a += pr[j] * vr[j];
        }
      }
      wave_lds_sync();
    }
  }
  // out through LDS so that each head's 64 values sit in one wave (its Q8A
  // form is two 32-element blocks)
  __syncthreads();
  float* ob = sc + (size_t)G * scs;  // [8][64] over the waves' areas
  if (ph < G) ob[ph * 64 + 8 * wave + pd] = a;
  __syncthreads();
  if (wave < G) {
    const float v = ob[wave * 64 + lane];
    if (!finite(v)) bad = true;
    const size_t base = (size_t)t * H * hd + (size_t)(g * G + wave) * hd;
    out[base + lane] = v;
    if (oq.qa) quantize_q8a_lanes(v, base, oq);
  }
  if (bad) flag(err, ERRBIT_NON_FINITE);
}

// Tiles in flight per wave.  One: in an A/B of the pipelined TinyLlama
// encode on one box (ms per 2048-token step) 97.1-97.3 against 97.4-97.5 for
// two, 97.8-97.9 for four, 99.0 for six and 99.4 for eight; the fewer
// registers leave room for the other chunks' waves.
constexpr int kHd64sRing = 1;

size_t attention_hd64s_smem(int G, int scs) {
  // the score rows, then each wave's [8][68] area (the output's [8][64] reuses it)
  return ((size_t)G * scs + 8 * 8 * kS64Stride) * sizeof(float);
}

// Decode shape (a few positions): one workgroup of 1024 threads per (head,
// position), with the RoPE and cache store of the chunk folded in.  The
// workgroup applies RoPE (lib.rs:2011-2051) to its query head and to the
// chunk's new keys of its KV group in LDS, and the first head of each group
// stores its position's key and value; cache rows before the chunk come from
// memory, the chunk's own rows from LDS, so no workgroup reads a row another
// one writes.  Then: scores (8-lane dot order), a block max, the clamped
// exps in parallel, the 8-lane Z chains (lanes 0-7), p = e / Z in parallel.
// P.V (lib.rs:2390-2420: out[d] = 0; out[d] += p_j * v_j[d] for j
// ascending) splits into the products, which every thread forms for one
// float4 of a 64-position V tile and stores dimension-major in LDS, and the
// 64 serial sums, which wave 0 runs over the stored products (lane =
// dimension, four products per LDS read).  V tiles stream through a ring of
// kDecDepth registers per thread, so kDecDepth tiles of loads are in flight
// while wave 0 sums.
constexpr int kDecThreads = 1024, kDecTile = 64, kDecStride = 68, kDecDepth = 8, kDecMaxT = 4;

__global__ void __launch_bounds__(kDecThreads) k_attention_dec(const float* q, RopeIn R, int layer,
                                                               int pos0, int H, int KV, int n_ctx,
                                                               float scale, float* out,
                                                               const int* pos_dev, int* err) {
  extern __shared__ __align__(16) float sc[];  // [len] scores -> exps -> probabilities
  __shared__ __align__(16) float prod[2][64 * kDecStride];  // [dim][position in tile]
  __shared__ __align__(16) float qs[64];
  __shared__ __align__(16) float kn[kDecMaxT][64];  // the chunk's keys (after RoPE)
  __shared__ __align__(16) float vn[kDecMaxT][64];  // the chunk's values
  __shared__ float red[kDecThreads / 64];
  __shared__ float zc[8];
  constexpr int hd = 64;
  const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int G = H / KV, g = h / G;
  const int pb = pos_dev ? *pos_dev : pos0;  // first position of the chunk
  const int pos = pb + t, len = pos + 1;
  const int half = R.rope_dim / 2;
  const float* keys = R.kc + ((size_t)layer * KV + g) * n_ctx * hd;
  const float* vals = R.vc + ((size_t)layer * KV + g) * n_ctx * hd;
  float* o = out + (size_t)t * H * hd + (size_t)h * hd;
  bool bad = false;
  // Raw rows: the query head, then the group's keys and values of chunk
  // positions 0..t.
  for (int i = tid; i < (t + 2) * hd; i += kDecThreads) {
    const int r = i >> 6, d = i & 63;
    const float v = r == 0 ? q[((size_t)t * H + h) * hd + d] : R.k[((size_t)(r - 1) * KV + g) * hd + d];
    bad |= !finite(v);
    if (r == 0) qs[d] = v;
    else kn[r - 1][d] = v;
  }
  for (int i = tid; i < (t + 1) * hd; i += kDecThreads)
    vn[i >> 6][i & 63] = R.v[((size_t)(i >> 6) * KV + g) * hd + (i & 63)];
  __syncthreads();
  // RoPE: x0*c - x1*s, x0*s + x1*c on pairs (2j, 2j+1) or (j, j + half).
  for (int p = tid; p < (t + 2) * half; p += kDecThreads) {
    const int r = p / half, j = p - r * half;
    float* base = r == 0 ? qs : kn[r - 1];
    const int ppos = r == 0 ? pos : pb + r - 1;
    const int ia = R.split_half ? j : 2 * j;
    const int ib = R.split_half ? j + half : 2 * j + 1;
    const float x0 = base[ia], x1 = base[ib];
    const float c = R.rc[(size_t)ppos * half + j], sn = R.rs[(size_t)ppos * half + j];
    const float y0 = x0 * c - x1 * sn;
    const float y1 = x0 * sn + x1 * c;
    bad |= any_nonfinite(y0, y1);
    base[ia] = y0;
    base[ib] = y1;
  }
  __syncthreads();
  if (h % G == 0 && tid < hd) {
    const size_t off = (((size_t)layer * KV + g) * n_ctx + pos) * hd + tid;
    const float kv = kn[t][tid], vv = vn[t][tid];
    bad |= any_nonfinite(kv, vv);
    R.kc[off] = kv;
    R.vc[off] = vv;
  }
  if (len == 1) {  // a single score copies V exactly (lib.rs:2319-2321)
    if (tid < hd) o[tid] = vn[0][tid];
    if (bad) flag(err, ERRBIT_NON_FINITE);
    return;
  }
  // scores: dot_f32_ref(q, k_j) * scale.  Eight lanes per key: lane r forms
  // the 8-lane accumulator r (dims r, r + 8, ..., r + 56 in order), three
  // shuffle levels then give ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)).  A round
  // covers 128 keys; the key rows of kScoreDepth rounds are in flight.
  {
    constexpr int kKeysPerRound = kDecThreads / 8, kScoreDepth = 4;
    const int r = tid & 7, kq = tid >> 3;
    float qr[8];
#pragma unroll
    for (int u = 0; u < 8; u++) qr[u] = qs[r + 8 * u];
    const int nrounds = (len + kKeysPerRound - 1) / kKeysPerRound;
    // Key rows are loaded unconditionally (rows outside the cached part read
    // row 0 and are replaced from LDS at use), so the loads in flight are
    // counted rather than drained.
    float kb[kScoreDepth][8];
    auto load_keys = [&](float (&dst)[8], int round) {
      const int j = kq + kKeysPerRound * round;
      const float* kr = keys + (size_t)(j < pb ? j : 0) * hd + r;
#pragma unroll
      for (int u = 0; u < 8; u++) dst[u] = kr[8 * u];
    };
#pragma unroll
    for (int d = 0; d < kScoreDepth; d++) load_keys(kb[d], d);
    for (int r0 = 0; r0 < nrounds; r0 += kScoreDepth) {
#pragma unroll
      for (int d = 0; d < kScoreDepth; d++) {
        const int round = r0 + d;
        const int j = kq + kKeysPerRound * round;
        const int jv = j - pb < 0 ? 0 : (j - pb < kDecMaxT ? j - pb : kDecMaxT - 1);
        float acc = 0.0f;
#pragma unroll
        for (int u = 0; u < 8; u++) acc += qr[u] * (j < pb ? kb[d][u] : kn[jv][r + 8 * u]);
        const float s3 = finish_8lane_dpp(acc);
        if (r == 0 && j < len) {
          const float sv = s3 * scale;
          if (!finite(sv)) bad = true;
          sc[j] = sv;
        }
        load_keys(kb[d], round + kScoreDepth);
      }
    }
  }
  __syncthreads();
  // softmax_in_place (lib.rs:2361-2388)
  float mx = -__builtin_huge_valf();
  for (int j = tid; j < len; j += kDecThreads) mx = fmaxf(mx, sc[j]);
  mx = wave_fmax(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int w = 1; w < kDecThreads / 64; w++) mx = fmaxf(mx, red[w]);
  for (int j = tid; j < len; j += kDecThreads) sc[j] = exp_clamped(sc[j] - mx);
  __syncthreads();
  if (tid < 8) {
    float acc = 0.0f;
    int j = tid;
    for (; j + 56 < len; j += 64) {
      const float e0 = sc[j], e1 = sc[j + 8], e2 = sc[j + 16], e3 = sc[j + 24];
      const float e4 = sc[j + 32], e5 = sc[j + 40], e6 = sc[j + 48], e7 = sc[j + 56];
      acc += e0; acc += e1; acc += e2; acc += e3;
      acc += e4; acc += e5; acc += e6; acc += e7;
    }
    for (; j < len; j += 8) acc += sc[j];
    zc[tid] = acc;
  }
  __syncthreads();
  const float z = finish_8lane(zc);
  if (!finite(z) || z == 0.0f) bad = true;
  for (int j = tid; j < len; j += kDecThreads) {
    const float p = sc[j] / z;
    if (!finite(p)) bad = true;
    sc[j] = p;
  }
  __syncthreads();
  // P.V.  Thread tid owns row jr of each tile and dimensions c4 .. c4 + 3:
  // a wave covers 16 rows x 16 dimensions, so its product stores (dimension-
  // major) spread over all LDS banks while each row's 64 bytes stay one
  // coalesced global segment.
  const int ntiles = (len + kDecTile - 1) / kDecTile;
  const int jr = 16 * (wave & 3) + (lane & 15), c4 = 16 * (wave >> 2) + 4 * (lane >> 4);
  // Every ring load is issued unconditionally (rows past the cached part
  // read row 0 and are replaced at use), so the compiler can count the
  // loads in flight instead of draining them all at each tile.
  float4 ring[kDecDepth];
#pragma unroll
  for (int u = 0; u < kDecDepth; u++) {
    const int j = u * kDecTile + jr;
    ring[u] = *reinterpret_cast<const float4*>(vals + (size_t)(j < pb ? j : 0) * hd + c4);
  }
  float a = 0.0f;
  for (int k0 = 0; k0 < ntiles; k0 += kDecDepth) {
#pragma unroll
    for (int u = 0; u < kDecDepth; u++) {
      const int k = k0 + u;
      const int j = k * kDecTile + jr;
      // chunk rows come from LDS; rows past len contribute nothing
      const int jv = j - pb < 0 ? 0 : (j - pb < kDecMaxT ? j - pb : kDecMaxT - 1);
      const float4 vl = *reinterpret_cast<const float4*>(&vn[jv][c4]);
      const float4 v = j < pb ? ring[u] : (j < len ? vl : make_float4(0.f, 0.f, 0.f, 0.f));
      const float p = j < len ? sc[j < len ? j : 0] : 0.0f;
      if (k < ntiles) {
        float* pr = prod[k & 1];
        pr[(c4 + 0) * kDecStride + jr] = p * v.x;
        pr[(c4 + 1) * kDecStride + jr] = p * v.y;
        pr[(c4 + 2) * kDecStride + jr] = p * v.z;
        pr[(c4 + 3) * kDecStride + jr] = p * v.w;
      }
      // issued on every step (rows outside the cached part read row 0)
      const int jn = j + kDecDepth * kDecTile;
      ring[u] = *reinterpret_cast<const float4*>(vals + (size_t)(jn < pb ? jn : 0) * hd + c4);
      __syncthreads();
      if (k < ntiles && wave == 0) {
        const float* pr = prod[k & 1] + lane * kDecStride;
        const int n = min(kDecTile, len - k * kDecTile);
        if (n == kDecTile) {
          // all sixteen reads first, then the 64 adds in order
          float4 p4[kDecTile / 4];
#pragma unroll
          for (int q4 = 0; q4 < kDecTile / 4; q4++)
            p4[q4] = *reinterpret_cast<const float4*>(pr + 4 * q4);
#pragma unroll
          for (int q4 = 0; q4 < kDecTile / 4; q4++) {
            a += p4[q4].x;
            a += p4[q4].y;
            a += p4[q4].z;
            a += p4[q4].w;
          }
        } else {
          for (int jj = 0; jj < n; jj++) a += pr[jj];
        }
      }
    }
  }
  if (wave == 0) {
    if (!finite(a)) bad = true;
    o[lane] = a;
  }
  if (bad) flag(err, ERRBIT_NON_FINITE);
}

// Decode shape split over many workgroups.  One workgroup per (head,
// position) streams the whole K and V prefix through a single CU, whose
// load bandwidth then bounds the launch (about 800 KB at position 1560 for a
// Qwen2.5-0.5B-shaped head).  Here k_attn_split_scores gives every 128-key
// block its own workgroup, and k_attn_split_pv gives every 16 dimensions of
// a head its own, so the K and V streams spread over the chip.  Values and
// order are those of k_attention_dec: the same 8-lane dot per score (the
// scores cross the launch boundary through memory as f32), the same max,
// clamped exps, 8-lane Z chains and divisions, and per dimension the same
// ascending chain of products p_j * v_j[d].
constexpr int kSplitKeys = 128;   // keys per score workgroup
constexpr int kSplitDims = 16;    // dimensions per P.V workgroup

// RoPE (lib.rs:2011-2051) of the query head and of the chunk's keys of its
// group into LDS, from the raw projections; returns whether any input or
// output is non-finite.  Each thread takes at most one rotated pair (the
// launch has at least (kDecMaxT + 1) * 32 threads), whose table entries it
// loads together with the raw rows, before the first barrier.
__device__ bool split_rope_rows(const float* q, const RopeIn& R, int h, int g, int t, int KV, int H,
                                int pb, float* qs, float (*kn)[64]) {
  constexpr int hd = 64;
  const int tid = threadIdx.x, nt = blockDim.x, half = R.rope_dim / 2;
  const int np = (t + 2) * half;
  const int p = tid < np ? tid : 0;
  const int pr = half > 0 ? p / half : 0, pj = p - pr * half;
  const int ppos = pr == 0 ? pb + t : pb + pr - 1;
  const float c = R.rc[(size_t)ppos * half + pj], sn = R.rs[(size_t)ppos * half + pj];
  bool bad = false;
  for (int i = tid; i < (t + 2) * hd; i += nt) {
    const int r = i >> 6, d = i & 63;
    const float v = r == 0 ? q[((size_t)t * H + h) * hd + d] : R.k[((size_t)(r - 1) * KV + g) * hd + d];
    bad |= !finite(v);
    if (r == 0) qs[d] = v;
    else kn[r - 1][d] = v;
  }
  __syncthreads();
  if (tid < np) {
    float* base = pr == 0 ? qs : kn[pr - 1];
    const int ia = R.split_half ? pj : 2 * pj;
    const int ib = R.split_half ? pj + half : 2 * pj + 1;
    const float x0 = base[ia], x1 = base[ib];
    const float y0 = x0 * c - x1 * sn;
    const float y1 = x0 * sn + x1 * c;
    bad |= any_nonfinite(y0, y1);
    base[ia] = y0;
    base[ib] = y1;
  }
  __syncthreads();
  return bad;
}

// Scores of keys [128 b, 128 b + 128) for (head h, chunk position t); the
// workgroup holding key `pos` of the group's first head also stores the
// position's key and value rows into the cache.  scores: [T][H][n_ctx].
__global__ void __launch_bounds__(256) k_attn_split_scores(const float* q, RopeIn R, int layer,
                                                           int pos0, int H, int KV, int n_ctx,
                                                           float scale, float* scores,
                                                           const int* pos_dev, int* err) {
  __shared__ __align__(16) float qs[64];
  __shared__ __align__(16) float kn[kDecMaxT][64];
  constexpr int hd = 64;
  const int b = blockIdx.x, h = blockIdx.y, t = blockIdx.z, tid = threadIdx.x;
  const int G = H / KV, g = h / G;
  const int pb = pos_dev ? *pos_dev : pos0;
  const int pos = pb + t, len = pos + 1;
  const int j0 = b * kSplitKeys;
  if (j0 >= len) return;  // the grid covers the longest row the launch can see
  // Eight lanes per key: lane r forms the 8-lane accumulator r (dims r,
  // r + 8, ..., r + 56 in order); three shuffle levels give
  // ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)).  All four rounds' cached key rows
  // are loaded before the RoPE phase, whose loads and barriers they then
  // overlap (rows outside the cached part read row 0 and are replaced from
  // LDS at use; a barrier waits for LDS only, not for these loads).
  constexpr int kRounds = kSplitKeys / 32;
  const float* keys = R.kc + ((size_t)layer * KV + g) * n_ctx * hd;
  const int r = tid & 7, kq = tid >> 3;
  float kb[kRounds][8];
#pragma unroll
  for (int d = 0; d < kRounds; d++) {
    const int j = j0 + kq + 32 * d;
    const float* kr = keys + (size_t)(j < pb ? j : 0) * hd + r;
#pragma unroll
    for (int u = 0; u < 8; u++) kb[d][u] = kr[8 * u];
  }
  bool bad = split_rope_rows(q, R, h, g, t, KV, H, pb, qs, kn);
  if (h % G == 0 && pos / kSplitKeys == b && tid < hd) {
    const size_t off = (((size_t)layer * KV + g) * n_ctx + pos) * hd + tid;
    const float kv = kn[t][tid], vv = R.v[((size_t)t * KV + g) * hd + tid];
    bad |= any_nonfinite(kv, vv);
    R.kc[off] = kv;
    R.vc[off] = vv;
  }
  if (len > 1) {  // a single score is never formed (the output copies V)
    float* srow = scores + ((size_t)t * H + h) * n_ctx;
    float qr[8];
#pragma unroll
    for (int u = 0; u < 8; u++) qr[u] = qs[r + 8 * u];
#pragma unroll
    for (int d = 0; d < kRounds; d++) {
      const int j = j0 + kq + 32 * d;
      const int jv = j - pb < 0 ? 0 : (j - pb < kDecMaxT ? j - pb : kDecMaxT - 1);
      float acc = 0.0f;
#pragma unroll
      for (int u = 0; u < 8; u++) acc += qr[u] * (j < pb ? kb[d][u] : kn[jv][r + 8 * u]);
      const float s3 = finish_8lane_dpp(acc);
      if (r == 0 && j < len) {
        const float sv = s3 * scale;
        bad |= !finite(sv);
        srow[j] = sv;
      }
    }
  }
  if (bad) flag(err, ERRBIT_NON_FINITE);
}

// softmax_in_place (lib.rs:2361-2388) of the score row, then
// out[d] = 0; out[d] += p_j * v_j[d] (j ascending, lib.rs:2390-2420) for
// dimensions [16 blockIdx.x, +16).  1024 threads, so that the latency-bound
// phases (the clamped exps, the divides) have four waves per SIMD.  Each
// thread issues its loads first: the score row, then V as 4 x 4 blocks (four
// rows of four dimensions), which arrive while the max runs and are stored
// dimension-major (one float4 per row block and dimension).  The exps are
// also stored chain-major (element j at chain j % 8, slot j / 8) for the
// eight Z chains.  After p_j = e_j / Z the sixteen serial P.V chains run
// over p and the dimension-major V, each product p_j * v_j[d] formed just
// before its add (a separate pass writing the products back into LDS was
// bound by LDS bandwidth: 2.4k cycles at 1500 keys).  The Z and P.V chains
// are DPP chains (chain_group_lds / chain_group_dot_lds: one chain per
// 16-lane row, each add's operand broadcast from the lane holding it, about
// 5 cycles per dependent add).
namespace {
// Raw buffer loads with a byte bound: a read past num_records returns zeros
// and generates no memory request.  Descriptor word 3 as for gfx9 targets.
typedef int BufRsrc __attribute__((ext_vector_type(4)));
typedef float F32x4 __attribute__((ext_vector_type(4)));
__device__ F32x4 raw_buffer_load_f32x4(BufRsrc rsrc, int voffset, int soffset, int aux) __asm(
    "llvm.amdgcn.raw.buffer.load.v4f32");
__device__ float raw_buffer_load_f32(BufRsrc rsrc, int voffset, int soffset, int aux) __asm(
    "llvm.amdgcn.raw.buffer.load.f32");
__device__ __forceinline__ BufRsrc buf_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  BufRsrc r;
  r.x = (int)(uint32_t)a;
  r.y = (int)((uint32_t)(a >> 32) & 0xffffu);  // stride 0
  r.z = (int)bytes;
  r.w = 0x00020000;
  return r;
}
__device__ __forceinline__ float4 buf_load_f32x4(const BufRsrc& r, int byte_off) {
  const F32x4 v = raw_buffer_load_f32x4(r, byte_off, 0, 0);
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float buf_load_f32(const BufRsrc& r, int byte_off) {
  return raw_buffer_load_f32(r, byte_off, 0, 0);
}
}  // namespace

constexpr int kSplitMaxRows = 2048;  // positions the register staging covers
constexpr int kPvThreads = 1024;
constexpr int kSplitVBlocks = kSplitMaxRows / kPvThreads;  // 4-row blocks per thread
static_assert(kPvThreads / 64 == 16 && 4 * (kPvThreads / 4) == kPvThreads, "one wave per dimension, 256 row quads");

struct SplitLayout {  // LDS of k_attn_split_pv, in floats
  int len4, zs, ld, zoff, voff, total;
};

__host__ __device__ inline SplitLayout split_layout(int maxlen) {
  SplitLayout L;
  L.len4 = (maxlen + 3) & ~3;
  L.zs = (((maxlen + 7) / 8 + 3) & ~3) + 4;  // chain-major row (a multiple of 4)
  L.ld = L.len4 + 4;                           // V row of one dimension
  L.zoff = L.len4;
  L.voff = L.zoff + 8 * L.zs;
  L.total = L.voff + kSplitDims * L.ld;
  return L;
}

size_t split_pv_smem(int maxlen) { return (size_t)split_layout(maxlen).total * sizeof(float); }

__global__ void __launch_bounds__(kPvThreads) k_attn_split_pv(const float* scores, RopeIn R, int layer,
                                                              int pos0, int H, int KV, int n_ctx,
                                                              int maxlen, float* out,
                                                              const int* pos_dev, int* err) {
  // [len4] scores -> probabilities, [8][zs] exps chain-major, [16][ld] V (then
  // the products) by dimension
  extern __shared__ __align__(16) float pr[];
  constexpr int NW = kPvThreads / 64;
  __shared__ float red[NW];
  __shared__ float zc[8];
  constexpr int hd = 64;
  const int dg = blockIdx.x, h = blockIdx.y, t = blockIdx.z, tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int G = H / KV, g = h / G;
  const int pb = pos_dev ? *pos_dev : pos0;
  const int pos = pb + t, len = pos + 1;
  const int d0 = dg * kSplitDims;
  const SplitLayout L = split_layout(maxlen);
  float* zcm = pr + L.zoff;
  float* vt = pr + L.voff;
  const float* vals = R.vc + ((size_t)layer * KV + g) * n_ctx * hd;
  // chunk rows (j >= pb) come from the raw projection, never from the cache
  auto vrow = [&](int j) -> const float* {
    return j < pb ? vals + (size_t)j * hd : R.v + ((size_t)(j - pb) * KV + g) * hd;
  };
  float* o = out + ((size_t)t * H + h) * hd + d0;
  bool bad = false;
  if (len == 1) {  // a single score copies V exactly (lib.rs:2319-2321)
    if (tid < kSplitDims) o[tid] = vrow(0)[d0 + tid];
    return;
  }
  // The score row and the V rows are read with buffer loads bounded by len:
  // past it they return zeros without touching memory, so every load stays
  // unconditional (the wait before the max counts the V loads still in
  // flight) and a short row costs only its own bytes.  The current
  // positions' K and V rows are in the cache: the scores launch stores them.
  const float* srow = scores + ((size_t)t * H + h) * n_ctx;
  const BufRsrc srs = buf_rsrc(srow, (uint32_t)len * 4u);
  const BufRsrc vrs = buf_rsrc(vals, (uint32_t)len * hd * 4u);
  float sv[kSplitMaxRows / kPvThreads];
#pragma unroll
  for (int k = 0; k < kSplitMaxRows / kPvThreads; k++) sv[k] = buf_load_f32(srs, 4 * (kPvThreads * k + tid));
  // V block i of this thread: rows 4 (256 i + jq) .. +3, dimensions d0 + c .. +3
  const int jq = tid >> 2, c = 4 * (tid & 3);
  float4 vb[kSplitVBlocks][4];
#pragma unroll
  for (int i = 0; i < kSplitVBlocks; i++)
#pragma unroll
    for (int r = 0; r < 4; r++)
      vb[i][r] = buf_load_f32x4(vrs, (4 * (256 * i + jq) + r) * hd * 4 + (d0 + c) * 4);
  float mx = -__builtin_huge_valf();
#pragma unroll
  for (int k = 0; k < kSplitMaxRows / kPvThreads; k++) {
    const int j = kPvThreads * k + tid;
    if (j < len) {
      pr[j] = sv[k];
      mx = fmaxf(mx, sv[k]);
    }
  }
  mx = wave_fmax(mx);
  if (lane == 0) red[wave] = mx;
  // V, dimension-major: each 4 x 4 block transposed in registers, one float4
  // per dimension (rows past len are stored too; no chain reads them)
#pragma unroll
  for (int i = 0; i < kSplitVBlocks; i++) {
    const int j4 = 4 * (256 * i + jq);
    if (j4 < len) {
      *reinterpret_cast<float4*>(vt + (c + 0) * L.ld + j4) =
          make_float4(vb[i][0].x, vb[i][1].x, vb[i][2].x, vb[i][3].x);
      *reinterpret_cast<float4*>(vt + (c + 1) * L.ld + j4) =
          make_float4(vb[i][0].y, vb[i][1].y, vb[i][2].y, vb[i][3].y);
      *reinterpret_cast<float4*>(vt + (c + 2) * L.ld + j4) =
          make_float4(vb[i][0].z, vb[i][1].z, vb[i][2].z, vb[i][3].z);
      *reinterpret_cast<float4*>(vt + (c + 3) * L.ld + j4) =
          make_float4(vb[i][0].w, vb[i][1].w, vb[i][2].w, vb[i][3].w);
    }
  }
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int w = 1; w < NW; w++) mx = fmaxf(mx, red[w]);
  {
    float e[kSplitMaxRows / kPvThreads];
#pragma unroll
    for (int k = 0; k < kSplitMaxRows / kPvThreads; k++) {
      const int j = tid + kPvThreads * k;
      e[k] = j < len ? exp_clamped(pr[j < len ? j : 0] - mx) : 0.0f;
    }
    // The chain-major rows are padded to the longest chain's length with
    // +0.0 (e is zero past len), which no sum of exps changes.
#pragma unroll
    for (int k = 0; k < kSplitMaxRows / kPvThreads; k++) {
      const int j = tid + kPvThreads * k;
      if (j < len) pr[j] = e[k];
      if (j < ((len + 7) & ~7)) zcm[(j & 7) * L.zs + (j >> 3)] = e[k];
    }
  }
  __syncthreads();
  // The eight Z chains as DPP chains: chain c on the 16-lane row c % 4 of
  // wave c / 4.
  if (tid < 128) {
    const int c = tid >> 4;
    const float zs = chain_group_lds<16>(0.0f, zcm + c * L.zs, (len + 7) / 8);
    if ((tid & 15) == 0) zc[c] = zs;
  }
  __syncthreads();
  const float z = finish_8lane(zc);
  bad |= !finite(z) || z == 0.0f;
  for (int j = tid; j < len; j += kPvThreads) {
    const float p = pr[j] / z;
    bad |= !finite(p);
    pr[j] = p;
  }
  __syncthreads();
  // The sixteen P.V chains as DPP chains, each product formed just before
  // its add: dimension d on the 16-lane row d % 4 of wave d / 4.
  if (tid < 64 * (kSplitDims / 4)) {
    const int d = tid >> 4;
    const float a = chain_group_dot_lds<16>(0.0f, pr, vt + d * L.ld, len);
    if ((tid & 15) == 0) {
      bad |= !finite(a);
      o[d] = a;
    }
  }
  if (bad) flag(err, ERRBIT_NON_FINITE);
}

// Decode attention in one launch for rows of at most kFusedMaxLen keys: the
// work of k_attn_split_scores and k_attn_split_pv for (16 dimensions, head,
// position) in one workgroup.  Each of a head's four workgroups forms the
// whole score row itself (the scores never leave LDS), which costs a read of
// the head's cached keys per workgroup: cheap for short rows, where the
// second launch would cost more than the repeated scores (on Qwen2.5-0.5B
// and TinyLlama-1.1B shapes the one launch is faster up to about 512 keys,
// the pair beyond).  Values and order
// are those of the split pair: the same 8-lane dots and scaling, max,
// clamped exps, Z chains, divisions and P.V chains.  The cache store of the
// positions' key and value rows is done by the first workgroup of each group
// (dimension block 0 of the group's first head); no workgroup reads a cache
// row at or past the launch's first position, which come from the raw
// projections instead (keys after RoPE in LDS).
constexpr int kFusedMaxLen = 512;
constexpr int kFusedVBlocks = (kFusedMaxLen + kPvThreads - 1) / kPvThreads;  // 4-row V blocks per thread
constexpr int kFusedKeyBatch = 4;                         // rounds of 128 keys per batch of loads
static_assert(kFusedMaxLen % (128 * kFusedKeyBatch) == 0 && kFusedVBlocks >= 1, "whole batches");

__global__ void __launch_bounds__(kPvThreads) k_attn_fused(const float* q, RopeIn R, int layer,
                                                           int pos0, int H, int KV, int n_ctx,
                                                           int maxlen, float scale, float* out,
                                                           const int* pos_dev, int* err) {
  // [len4] scores -> probabilities, [8][zs] exps chain-major, [16][ld] V (then
  // the products) by dimension
  extern __shared__ __align__(16) float pr[];
  constexpr int NW = kPvThreads / 64;
  constexpr int hd = 64;
  __shared__ __align__(16) float qs[64];
  __shared__ __align__(16) float kn[kDecMaxT][64];
  __shared__ float red[NW];
  __shared__ float zc[8];
  const int dg = blockIdx.x, h = blockIdx.y, t = blockIdx.z, tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int G = H / KV, g = h / G;
  const int pb = pos_dev ? *pos_dev : pos0;
  const int pos = pb + t, len = pos + 1;
  const int d0 = dg * kSplitDims;
  const SplitLayout L = split_layout(maxlen);
  float* zcm = pr + L.zoff;
  float* vt = pr + L.voff;
  const float* keys = R.kc + ((size_t)layer * KV + g) * n_ctx * hd;
  const float* vals = R.vc + ((size_t)layer * KV + g) * n_ctx * hd;
  float* o = out + ((size_t)t * H + h) * hd + d0;
  bool bad = false;
  // Loads first.  V rows of the cached part through buffer loads bounded by
  // pb rows (past it they return zeros without a memory request); the raw V
  // rows of the chunk positions this row sees (row pb + tid / 16, dimension
  // d0 + tid % 16); the first batch of cached key rows (eight lanes per key,
  // rows outside the cached part read row 0 and are replaced from LDS).
  const BufRsrc vrs = buf_rsrc(vals, (uint32_t)pb * hd * 4u);
  const int jq = tid >> 2, c = 4 * (tid & 3);
  float4 vb[kFusedVBlocks][4];
#pragma unroll
  for (int i = 0; i < kFusedVBlocks; i++)
#pragma unroll
    for (int r = 0; r < 4; r++)
      vb[i][r] = buf_load_f32x4(vrs, (4 * (256 * i + jq) + r) * hd * 4 + (d0 + c) * 4);
  const int nv = len - pb;  // t + 1 chunk rows
  const int vj = (tid >> 4) < nv ? (tid >> 4) : 0;
  const float vraw = R.v[((size_t)vj * KV + g) * hd + d0 + (tid & 15)];
  const int r8 = tid & 7, kq = tid >> 3;
  float kb[kFusedKeyBatch][8];
#pragma unroll
  for (int d = 0; d < kFusedKeyBatch; d++) {
    const int j = kq + 128 * d;
    const float* kr = keys + (size_t)(j < pb ? j : 0) * hd + r8;
#pragma unroll
    for (int u = 0; u < 8; u++) kb[d][u] = kr[8 * u];
  }
  bad |= split_rope_rows(q, R, h, g, t, KV, H, pb, qs, kn);
  if (dg == 0 && h % G == 0 && tid < hd) {
    const size_t off = (((size_t)layer * KV + g) * n_ctx + pos) * hd + tid;
    const float kv = kn[t][tid], vv = R.v[((size_t)t * KV + g) * hd + tid];
    bad |= any_nonfinite(kv, vv);
    R.kc[off] = kv;
    R.vc[off] = vv;
  }
  if (len == 1) {  // a single score copies V exactly (lib.rs:2319-2321)
    if (tid < kSplitDims) o[tid] = vraw;
    if (bad) flag(err, ERRBIT_NON_FINITE);
    return;
  }
  // Scores, 128 keys per round, straight into the probability row.
  float qr[8];
#pragma unroll
  for (int u = 0; u < 8; u++) qr[u] = qs[r8 + 8 * u];
  float mx = -__builtin_huge_valf();
  for (int jb = 0; jb < len; jb += 128 * kFusedKeyBatch) {
    if (jb > 0) {
#pragma unroll
      for (int d = 0; d < kFusedKeyBatch; d++) {
        const int j = jb + kq + 128 * d;
        const float* kr = keys + (size_t)(j < pb ? j : 0) * hd + r8;
#pragma unroll
        for (int u = 0; u < 8; u++) kb[d][u] = kr[8 * u];
      }
    }
#pragma unroll
    for (int d = 0; d < kFusedKeyBatch; d++) {
      const int j = jb + kq + 128 * d;
      const int jv = j - pb < 0 ? 0 : (j - pb < kDecMaxT ? j - pb : kDecMaxT - 1);
      float acc = 0.0f;
#pragma unroll
      for (int u = 0; u < 8; u++) acc += qr[u] * (j < pb ? kb[d][u] : kn[jv][r8 + 8 * u]);
      const float s3 = finish_8lane_dpp(acc);
      if (r8 == 0 && j < len) {
        const float sv = s3 * scale;
        bad |= !finite(sv);
        pr[j] = sv;
        mx = fmaxf(mx, sv);
      }
    }
  }
  mx = wave_fmax(mx);
  if (lane == 0) red[wave] = mx;
  // V, dimension-major: each 4 x 4 block transposed in registers, one float4
  // per dimension (rows past len are stored too; no chain reads them)
#pragma unroll
  for (int i = 0; i < kFusedVBlocks; i++) {
    const int j4 = 4 * (256 * i + jq);
    if (j4 < len) {
      *reinterpret_cast<float4*>(vt + (c + 0) * L.ld + j4) =
          make_float4(vb[i][0].x, vb[i][1].x, vb[i][2].x, vb[i][3].x);
      *reinterpret_cast<float4*>(vt + (c + 1) * L.ld + j4) =
          make_float4(vb[i][0].y, vb[i][1].y, vb[i][2].y, vb[i][3].y);
      *reinterpret_cast<float4*>(vt + (c + 2) * L.ld + j4) =
          make_float4(vb[i][0].z, vb[i][1].z, vb[i][2].z, vb[i][3].z);
      *reinterpret_cast<float4*>(vt + (c + 3) * L.ld + j4) =
          make_float4(vb[i][0].w, vb[i][1].w, vb[i][2].w, vb[i][3].w);
    }
  }
  __syncthreads();
  // the chunk rows, which the bounded loads above returned as zeros
  if (tid < nv * kSplitDims) vt[(tid & 15) * L.ld + pb + (tid >> 4)] = vraw;
  mx = red[0];
#pragma unroll
  for (int w = 1; w < NW; w++) mx = fmaxf(mx, red[w]);
  {
    float e[kFusedVBlocks];
#pragma unroll
    for (int k = 0; k < kFusedVBlocks; k++) {
      const int j = tid + kPvThreads * k;
      e[k] = j < len ? exp_clamped(pr[j < len ? j : 0] - mx) : 0.0f;
    }
    // The chain-major rows are padded to the longest chain's length with
    // +0.0 (e is zero past len), which no sum of exps changes.
#pragma unroll
    for (int k = 0; k < kFusedVBlocks; k++) {
      const int j = tid + kPvThreads * k;
      if (j < len) pr[j] = e[k];
      if (j < ((len + 7) & ~7)) zcm[(j & 7) * L.zs + (j >> 3)] = e[k];
    }
  }
  __syncthreads();
  if (tid < 128) {
    const int cz = tid >> 4;
    const float zsum = chain_group_lds<16>(0.0f, zcm + cz * L.zs, (len + 7) / 8);
    if ((tid & 15) == 0) zc[cz] = zsum;
  }
  __syncthreads();
  const float z = finish_8lane(zc);
  bad |= !finite(z) || z == 0.0f;
  for (int j = tid; j < len; j += kPvThreads) {
    const float p = pr[j] / z;
    bad |= !finite(p);
    pr[j] = p;
  }
  __syncthreads();
  if (tid < 64 * (kSplitDims / 4)) {
    const int d = tid >> 4;
    const float a = chain_group_dot_lds<16>(0.0f, pr, vt + d * L.ld, len);
    if ((tid & 15) == 0) {
      bad |= !finite(a);
      o[d] = a;
    }
  }
  if (bad) flag(err, ERRBIT_NON_FINITE);
}

size_t attention_hd64_smem(int G, int sc_stride) {
  return ((size_t)G * sc_stride + 2 * kA64Buf + (size_t)G * 64) * sizeof(float);
}

size_t attention_grp_smem(int H, int KV, int hd, int n_ctx) {
  int G = H / KV;
  return ((size_t)G * n_ctx + (size_t)(kAttnTile + 1) * hd + (size_t)G * hd) * sizeof(float);
}

// Dynamic LDS of k_attention_dec (the score row); its static LDS holds the
// product tiles.
constexpr size_t kDecMaxScoreBytes = 112 * 1024;

bool attention_pos_dev_supported(int hd, int T, int n_ctx) {
  return hd == 64 && T <= kDecMaxT && (size_t)n_ctx * sizeof(float) <= kDecMaxScoreBytes;
}

bool attention_dec_applies(int hd, int T, int pos0, int n_ctx, bool pos_in_device) {
  const size_t smem = (size_t)(pos_in_device ? n_ctx : pos0 + T) * sizeof(float);
  return hd == 64 && T <= kDecMaxT && smem <= kDecMaxScoreBytes;
}

int attention_fused_max_len() { return kFusedMaxLen; }

void launch_attention_dec(const float* q, const RopeIn& R, int layer, int T, int pos0, int H,
                          int KV, int n_ctx, int maxlen_dev, float scale, float* scores, float* out,
                          const int* pos_dev, int* err, hipStream_t s) {
  // With the position in device memory the grids and LDS are sized for the
  // longest row the replays may see.
  const int maxlen = pos_dev ? maxlen_dev : pos0 + T;
  const size_t smem = (size_t)maxlen * sizeof(float);
  const size_t pv_smem = split_pv_smem(maxlen);
  if (maxlen <= kFusedMaxLen) {
    static bool attr_fused_set = false;
    if (!attr_fused_set) {
      (void)hipFuncSetAttribute((const void*)k_attn_fused, hipFuncAttributeMaxDynamicSharedMemorySize,
                                158 * 1024);
      attr_fused_set = true;
    }
    launch_kernel(k_attn_fused, dim3(64 / kSplitDims, H, T), dim3(kPvThreads), pv_smem, s, q, R, layer,
                  pos0, H, KV, n_ctx, maxlen, scale, out, pos_dev, err);
    return;
  }
  if (maxlen <= kSplitMaxRows && pv_smem <= 158 * 1024) {
    static bool attr_pv_set = false;
    if (!attr_pv_set) {
      (void)hipFuncSetAttribute((const void*)k_attn_split_pv,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 158 * 1024);
      attr_pv_set = true;
    }
    launch_kernel(k_attn_split_scores, dim3((maxlen + kSplitKeys - 1) / kSplitKeys, H, T), dim3(256), 0,
                  s, q, R, layer, pos0, H, KV, n_ctx, scale, scores, pos_dev, err);
    launch_kernel(k_attn_split_pv, dim3(64 / kSplitDims, H, T), dim3(kPvThreads), pv_smem, s, scores, R,
                  layer, pos0, H, KV, n_ctx, maxlen, out, pos_dev, err);
    return;
  }
  // Longer windows: one workgroup per (head, position).
  static bool attr_dec_set = false;
  if (!attr_dec_set) {
    (void)hipFuncSetAttribute((const void*)k_attention_dec,
                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)kDecMaxScoreBytes);
    attr_dec_set = true;
  }
  launch_kernel(k_attention_dec, dim3(H, T), dim3(kDecThreads), smem, s, q, R, layer, pos0, H, KV,
                n_ctx, scale, out, pos_dev, err);
}

bool attention_quantizes_q8a(int hd, int H, int KV, int T, int pos0, int n_ctx) {
  const int G = H / KV;
  if (attention_dec_applies(hd, T, pos0, n_ctx, false)) return false;
  return hd == 64 && G >= 2 && G <= 16 &&
         attention_hd64_smem(G, ((pos0 + T) + 3) & ~3) <= 150 * 1024;
}

void launch_attention(const float* q, const float* kc, const float* vc, int layer, int T, int pos0,
                      int H, int KV, int hd, int n_ctx, float scale, float* scores, float* out,
                      int* err, hipStream_t s, int8_t* qa, float* da, float* af) {
  int G = H / KV;
  if (hd == 64 && G >= 1 && G <= 8) {
    const int scs = attn_split_lane_stride(pos0 + T);
    const size_t smem = attention_hd64s_smem(G, scs);
    if (smem <= 150 * 1024) {
      static const bool attr = hipFuncSetAttribute((const void*)k_attention_hd64s<kHd64sRing>,
                                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   150 * 1024) == hipSuccess;
      (void)attr;
      const QuantOut oq{qa, da, af, nullptr, nullptr};
      launch_kernel(k_attention_hd64s<kHd64sRing>, dim3(KV, T), dim3(512), smem, s, q, kc, vc, layer, pos0, H,
                    KV, n_ctx, scs, scale, out, oq, err);
      return;
    }
  }
  if (hd == 64 && G >= 2 && G <= 16) {
    // Scores only need the longest row of this chunk (rounded to float4).
    int sc_stride = ((pos0 + T) + 3) & ~3;
    size_t smem64 = attention_hd64_smem(G, sc_stride);
    if (smem64 <= 150 * 1024) {
      // float4 per thread per tile (64 rows x 16) and tiles in flight
      const int per = (1024 + G * 64 - 1) / (G * 64);
      auto go = [&](auto kern) {
        static bool attr64_set = false;
        if (!attr64_set) {
          (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    150 * 1024);
          attr64_set = true;
        }
        const QuantOut oq{qa, da, af, nullptr, nullptr};
        launch_kernel(kern, dim3(KV, T), dim3(G * 64), smem64, s, q, kc, vc, layer, pos0, H, KV,
                      n_ctx, sc_stride, scale, out, oq, err);
      };
      if (G * 64 > 512) go(k_attention_hd64<2, 8, 1024>);
      else if (per <= 2) go(k_attention_hd64<2, 8, 512>);
      else if (per <= 4) go(k_attention_hd64<4, 4, 512>);
      else go(k_attention_hd64<8, 2, 256>);
      return;
    }
  }
  size_t smem = attention_grp_smem(H, KV, hd, n_ctx);
  if (G <= 16 && hd <= 256 && smem <= 150 * 1024) {
    static bool attr_set = false;
    if (!attr_set) {
      (void)hipFuncSetAttribute((const void*)k_attention_grp,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024);
      attr_set = true;
    }
    launch_kernel(k_attention_grp, dim3(KV, T), dim3(G * 64), smem, s, q, kc, vc, layer, pos0,
                       H, KV, hd, n_ctx, scale, out, err);
    return;
  }
  launch_kernel(k_attention, dim3(H, T), dim3(64), 0, s, q, kc, vc, layer, pos0, H, KV, hd,
                     n_ctx, scale, scores, out, err);
}

// ---------------------------------------------------------------------------
// swiglu (det-model lib.rs:2420-2434)
__global__ void k_swiglu(const float* g, const float* u, int count, float* out, int* err) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  float gv = g[i], uv = u[i];
  float v = silu_det(gv) * uv;
  if (!finite(gv) || !finite(uv) || !finite(v)) flag(err, ERRBIT_NON_FINITE);
  out[i] = v;
}

void launch_swiglu(const float* g, const float* u, int count, float* out, int* err, hipStream_t s) {
  launch_kernel(k_swiglu, dim3((count + 255) / 256), dim3(256), 0, s, g, u, count, out, err);
}

// ---------------------------------------------------------------------------
// RopeTables::llama (det-model lib.rs:813-847) in f64 on the device.
__global__ void k_rope_table(float base, int rope_dim, int positions, float* co, float* so,
                             int* err) {
  int half = rope_dim / 2;
  int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= positions * half) return;
  int pos = idx / half, j = idx % half;
  double ln_base = log64((double)base);
  double exponent = -((double)(2 * j)) / (double)rope_dim;
  double omega = exp64(exponent * ln_base);
  double phi = (double)pos * omega;
  float c = (float)cos64(phi);
  float s = (float)sin64(phi);
  if (!finite(c) || !finite(s)) flag(err, ERRBIT_NON_FINITE);
  co[idx] = c;
  so[idx] = s;
}

void launch_rope_table(float base, int rope_dim, int positions, float* cos_out, float* sin_out,
                       int* err, hipStream_t s) {
  int n = positions * (rope_dim / 2);
  launch_kernel(k_rope_table, dim3((n + 255) / 256), dim3(256), 0, s, base, rope_dim,
                     positions, cos_out, sin_out, err);
}

// ---------------------------------------------------------------------------
// logits -> integer CDF (det-coder cdf.rs).  One workgroup of 256 threads
// per row.  max -> e_i = exp_f32(max(l_i - m, -88)) -> Z by the 8-lane sum
// (8 chains over LDS tiles) -> f_i = (u32)(e_i/Z * 2^24) + 1 -> exact
// integer sums / scans.
namespace {
constexpr int kCdfThreads = 256;
constexpr int kCdfTile = kCdfThreads * 8;

__device__ __forceinline__ uint32_t cdf_freq(float e, float z) {
  float p = e / z;
  float g = p * 16777216.0f;
  uint32_t gi = g <= 0.0f ? 0u : (g >= 4294967296.0f ? 0xffffffffu : (uint32_t)g);
  return gi + 1u;
}

// Block-wide inclusive scan of one u64 per thread (256 threads).
__device__ uint64_t block_scan_u64(uint64_t v, uint64_t* sh, uint64_t* total) {
  int tid = threadIdx.x;
  sh[tid] = v;
  __syncthreads();
  for (int off = 1; off < kCdfThreads; off <<= 1) {
    uint64_t add = tid >= off ? sh[tid - off] : 0;
    __syncthreads();
    sh[tid] += add;
    __syncthreads();
  }
  uint64_t incl = sh[tid];
  *total = sh[kCdfThreads - 1];
  __syncthreads();
  return incl;
}
}  // namespace

__global__ void __launch_bounds__(256) k_cdf(const float* logits, int V, int tail, int mode,
                                             const uint32_t* symbols, const uint64_t* values,
                                             uint64_t* cum, uint32_t* freq, uint64_t* total,
                                             uint32_t* sym, uint32_t* freq_tab, uint64_t* cum_tab,
                                             int* err) {
  // Z tiles, chain-major: element idx of a tile sits at [idx % 8][idx / 8],
  // double-buffered (wave 0 sums one while waves 1-3 fill the other).
  constexpr int kChainLen = kCdfTile / 8;
  constexpr int kChainStride = kChainLen + 4;
  __shared__ __align__(16) float ztile[2][8][kChainStride];
  __shared__ float chain[8];
  __shared__ float red[kCdfThreads / 64];
  __shared__ uint64_t scan[kCdfThreads];
  int r = blockIdx.x, tid = threadIdx.x;
  const float* l = logits + (size_t)r * V;
  // max (order independent) + finiteness
  // Strided passes over the row load 8 values ahead of their use.
  constexpr int kBatch = 8;
  float mx = -__builtin_huge_valf();
  bool bad = false;
  for (int i0 = tid; i0 < V; i0 += kBatch * kCdfThreads) {
    float v[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; k++) {
      int i = i0 + k * kCdfThreads;
      v[k] = i < V ? l[i] : -__builtin_huge_valf();
    }
#pragma unroll
    for (int k = 0; k < kBatch; k++) {
      if (i0 + k * kCdfThreads < V && !finite(v[k])) bad = true;
      mx = fmaxf(mx, v[k]);
    }
  }
  mx = wave_fmax(mx);
  if ((tid & 63) == 0) red[tid / 64] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  if (bad) flag(err, ERRBIT_CDF_NON_FINITE);
  // Z: chain c adds e_i for i = c mod 8 ascending (tiles start at multiples
  // of 8, so tile index idx keeps i's class).  Waves 1-3 produce tile k+1
  // while lanes 0-7 of wave 0 consume tile k.
  const int ntiles = (V + kCdfTile - 1) / kCdfTile;
  constexpr int kProducers = kCdfThreads - 64;
  constexpr int kPerProducer = (kCdfTile + kProducers - 1) / kProducers;
  auto produce = [&](int k) {
    const int base = k * kCdfTile;
    float(*dst)[kChainStride] = ztile[k & 1];
    float v[kPerProducer];
#pragma unroll
    for (int j = 0; j < kPerProducer; j++) {
      int idx = tid - 64 + j * kProducers;
      int i = base + idx;
      v[j] = idx < kCdfTile && i < V ? l[i] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < kPerProducer; j++) {
      int idx = tid - 64 + j * kProducers;
      int i = base + idx;
      if (idx < kCdfTile) dst[idx & 7][idx >> 3] = i < V ? exp_clamped(v[j] - mx) : 0.0f;
    }
  };
  float acc = 0.0f;
  if (tid >= 64) produce(0);
  __syncthreads();
  for (int k = 0; k < ntiles; k++) {
    if (tid >= 64) {
      if (k + 1 < ntiles) produce(k + 1);
    } else if (tid < 8) {
      const int base = k * kCdfTile;
      const int lim = V - base < kCdfTile ? V - base : kCdfTile;
      const int cnt = (lim - tid + 7) / 8;  // elements tid, tid+8, ... below lim
      const float* my = ztile[k & 1][tid];
      int j = 0;
      for (; j + 16 <= cnt; j += 16) {
        float4 f0 = *reinterpret_cast<const float4*>(my + j);
        float4 f1 = *reinterpret_cast<const float4*>(my + j + 4);
        float4 f2 = *reinterpret_cast<const float4*>(my + j + 8);
        float4 f3 = *reinterpret_cast<const float4*>(my + j + 12);
        acc += f0.x; acc += f0.y; acc += f0.z; acc += f0.w;
        acc += f1.x; acc += f1.y; acc += f1.z; acc += f1.w;
        acc += f2.x; acc += f2.y; acc += f2.z; acc += f2.w;
        acc += f3.x; acc += f3.y; acc += f3.z; acc += f3.w;
      }
      for (; j < cnt; j++) acc += my[j];
    }
    __syncthreads();
  }
  if (tid < 8) chain[tid] = acc;
  __syncthreads();
  float z = finish_8lane(chain);
  if (mode == 0) {
    // Symbol range: three plain sums (every f_i, the f_i below the symbol)
    // and the symbol's own f; integer sums are exact in any order.
    const uint32_t want_sym = symbols[r];
    uint64_t run_part = 0, below_part = 0;
    uint32_t found_freq = 0;
    bool found = false;
    for (int i0 = tid; i0 < V; i0 += kBatch * kCdfThreads) {
      float v[kBatch];
#pragma unroll
      for (int k = 0; k < kBatch; k++) {
        int i = i0 + k * kCdfThreads;
        v[k] = i < V ? l[i] : 0.0f;
      }
#pragma unroll
      for (int k = 0; k < kBatch; k++) {
        int i = i0 + k * kCdfThreads;
        if (i < V) {
          uint32_t f = cdf_freq(exp_clamped(v[k] - mx), z);
          run_part += f;
          if ((uint32_t)i < want_sym) below_part += f;
          if ((uint32_t)i == want_sym) {
            found = true;
            found_freq = f;
          }
        }
      }
    }
    uint64_t run, below;
    block_scan_u64(run_part, scan, &run);
    block_scan_u64(below_part, scan, &below);
    uint64_t tot_all = run + (uint64_t)tail;
    if (tid == 0 && (run >= (1ull << 31) || tot_all >= (1ull << 31))) flag(err, ERRBIT_CDF_TOTAL);
    if (found) {
      cum[r] = below;
      freq[r] = found_freq;
    }
    if (tid == 0) {
      if (want_sym >= (uint32_t)V) {
        cum[r] = run + (want_sym - (uint32_t)V);
        freq[r] = 1;
      }
      total[r] = tot_all;
    }
    return;
  }
  // Table / lookup / total: each thread owns 8 consecutive entries of a
  // tile; an exact block scan gives each entry's cumulative frequency.
  uint64_t target = 0, run = 0;
  if (mode == 2) target = values[r];
  uint64_t found_cum = 0;
  uint32_t found_freq = 0, found_sym = 0;
  bool found = false;
  for (int base = 0; base < V; base += kCdfTile) {
    uint32_t f[8];
    uint64_t local = 0;
    int i0 = base + tid * 8;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      int i = i0 + k;
      f[k] = i < V ? cdf_freq(exp_clamped(l[i] - mx), z) : 0u;
      local += f[k];
    }
    uint64_t tot;
    uint64_t incl = block_scan_u64(local, scan, &tot);
    uint64_t c = run + incl - local;
#pragma unroll
    for (int k = 0; k < 8; k++) {
      int i = i0 + k;
      if (i < V) {
        if (mode == 1) {
          freq_tab[i] = f[k];
          cum_tab[i] = c;
        } else if (mode == 2 && !found && target >= c && target < c + f[k]) {
          found = true;
          found_sym = (uint32_t)i;
          found_cum = c;
          found_freq = f[k];
        }
        c += f[k];
      }
    }
    run += tot;
  }
  // run = sum of all f_i over the vocabulary
  uint64_t tot_all = run + (uint64_t)tail;
  if (run >= (1ull << 31) || tot_all >= (1ull << 31)) {
    if (tid == 0) flag(err, ERRBIT_CDF_TOTAL);
  }
  if (mode == 1) {
    for (int k = tid; k < tail; k += kCdfThreads) {
      freq_tab[V + k] = 1;
      cum_tab[V + k] = run + (uint64_t)k;
    }
    if (tid == 0) total[0] = tot_all;
  } else if (mode == 2) {
    if (found) {
      sym[r] = found_sym;
      cum[r] = found_cum;
      freq[r] = found_freq;
    }
    if (tid == 0) {
      total[r] = tot_all;
      if (target >= run) {
        uint64_t off = target - run;
        if (off < (uint64_t)tail) {
          sym[r] = (uint32_t)(V + off);
          cum[r] = target;
          freq[r] = 1;
        } else {
          flag(err, ERRBIT_CDF_LOOKUP);
        }
      }
    }
  } else {
    if (tid == 0) total[r] = tot_all;
  }
}

// ---------------------------------------------------------------------------
// The same CDF split over many workgroups per row (modes 0, 2, 3): block
// maxima, block exps written chain-major, one wave per row for the eight
// serial Z chains, block frequency sums, and a per-row finish with the exact
// integer sums / search.  Every f32 operation is the one k_cdf performs.
namespace {
constexpr int kCdfBlk = (int)kCdfBlockElems;  // elements per workgroup (256 threads x 16)

__host__ __device__ inline int cdf_nblk(int V) { return (V + kCdfBlk - 1) / kCdfBlk; }
__host__ __device__ inline int cdf_v8(int V) { return (((V + 7) / 8) + 3) & ~3; }
}  // namespace

size_t cdf_scratch_bytes(int R, int V) { return cdf_scratch_bytes_for((size_t)R, (size_t)V); }

namespace {
struct CdfScratch {
  float* pmax;       // [R][nblk]
  float* ebuf;       // [R][8][v8]
  float* z;          // [R]
  uint64_t* bsum;    // [R][nblk]
  uint64_t* bbelow;  // [R][nblk]
  uint32_t* symf;    // [R]
};

CdfScratch cdf_scratch(void* base, int R, int V) {
  const size_t nb = (size_t)cdf_nblk(V);
  char* p = (char*)base;
  auto take = [&](size_t bytes) {
    char* q = p;
    p += (bytes + 15) & ~(size_t)15;
    return q;
  };
  CdfScratch c;
  c.bsum = (uint64_t*)take((size_t)R * nb * 8);
  c.bbelow = (uint64_t*)take((size_t)R * nb * 8);
  c.pmax = (float*)take((size_t)R * nb * 4);
  c.ebuf = (float*)take((size_t)R * 8 * cdf_v8(V) * 4);
  c.z = (float*)take((size_t)R * 4);
  c.symf = (uint32_t*)take((size_t)R * 4);
  return c;
}

__device__ float block_max_256(float v, float* red) {
  v = wave_fmax(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

__device__ uint64_t block_sum_u64_256(uint64_t v, uint64_t* red) {
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  uint64_t s = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return s;
}
}  // namespace

// Block maxima (order independent) and finiteness.
__global__ void __launch_bounds__(256) k_cdf_bmax(const float* logits, const uint32_t* rows, int V,
                                                  CdfScratch cs, int* err) {
  __shared__ float red[4];
  const int r = blockIdx.y, b = blockIdx.x, nb = gridDim.x;
  const float* l = logits + (size_t)(rows ? rows[r] : r) * V;
  float v[16];
#pragma unroll
  for (int k = 0; k < 16; k++) {
    int i = b * kCdfBlk + k * 256 + threadIdx.x;
    v[k] = i < V ? l[i] : -__builtin_huge_valf();
  }
  float mx = -__builtin_huge_valf();
  bool bad = false;
#pragma unroll
  for (int k = 0; k < 16; k++) {
    int i = b * kCdfBlk + k * 256 + threadIdx.x;
    if (i < V && !finite(v[k])) bad = true;
    mx = fmaxf(mx, v[k]);
  }
  if (bad) flag(err, ERRBIT_CDF_NON_FINITE);
  mx = block_max_256(mx, red);
  if (threadIdx.x == 0) cs.pmax[(size_t)r * nb + b] = mx;
}

// e_i = exp_f32(max(l_i - m, -88)) for the block, stored chain-major:
// element i at [i % 8][i / 8] of the row's buffer.
__global__ void __launch_bounds__(256) k_cdf_bexp(const float* logits, const uint32_t* rows, int V,
                                                  CdfScratch cs) {
  const int r = blockIdx.y, b = blockIdx.x, nb = gridDim.x;
  const float* l = logits + (size_t)(rows ? rows[r] : r) * V;
  float mx = -__builtin_huge_valf();
  for (int k = 0; k < nb; k++) mx = fmaxf(mx, cs.pmax[(size_t)r * nb + k]);
  const int v8 = cdf_v8(V);
  float* e = cs.ebuf + (size_t)r * 8 * v8;
  float v[16];
#pragma unroll
  for (int k = 0; k < 16; k++) {
    int i = b * kCdfBlk + k * 256 + threadIdx.x;
    v[k] = i < V ? l[i] : 0.0f;
  }
#pragma unroll
  for (int k = 0; k < 16; k++) {
    int i = b * kCdfBlk + k * 256 + threadIdx.x;
    if (i < V) e[(size_t)(i & 7) * v8 + (i >> 3)] = exp_clamped(v[k] - mx);
  }
}

// Z = sum_f32_ref(e): chain c (i = c mod 8, ascending) runs on the 16-lane
// row c % 4 of wave c / 4 as a DPP chain (chain_group_lds), over a three-deep
// LDS ring that waves 2-3 fill from the chain-major buffer.
__global__ void __launch_bounds__(256) k_cdf_z(int V, CdfScratch cs) {
  // A producer thread holds the next segment in registers for a whole
  // segment's worth of adds before it stores it, so the global-load latency
  // never reaches the chains.  Entries past a chain's own length are stored
  // as +0.0, so all eight chains add the same number of terms (the longest
  // chain's) without changing any sum's bits: a sum of non-negative exps
  // that starts at +0.0 is never -0.0.
  constexpr int kSeg = 1024;  // elements per chain per ring slot
  constexpr int kSlots = 3;
  constexpr int kChainThreads = 128;
  constexpr int kProducers = 256 - kChainThreads;
  constexpr int kF4 = 8 * kSeg / 4;                            // float4 per segment
  constexpr int kPer = kF4 / kProducers;                       // per producer thread
  static_assert(kF4 % kProducers == 0, "whole float4 rounds per producer");
  extern __shared__ __align__(16) float zring[];               // [kSlots][8][kSeg]
  __shared__ float zc[8];
  const int r = blockIdx.x, tid = threadIdx.x;
  const int v8 = cdf_v8(V);
  const float* e = cs.ebuf + (size_t)r * 8 * v8;
  const int cnt_max = (V + 7) / 8;  // chain 0, the longest
  const int nseg = (cnt_max + kSeg - 1) / kSeg;
  float4 pre[kPer];
  auto load = [&](int sg) {
#pragma unroll
    for (int k = 0; k < kPer; k++) {
      const int x = tid - kChainThreads + kProducers * k;
      const int c = x / (kSeg / 4), j = sg * kSeg + 4 * (x % (kSeg / 4));
      const int cnt = (V - c + 7) / 8;  // elements of chain c (at most v8)
      // unconditional: a load under a branch waits for every load before it
      float4 f = *reinterpret_cast<const float4*>(e + (size_t)c * v8 + (j < v8 ? j : 0));
      f.x = j < cnt ? f.x : 0.0f;
      f.y = j + 1 < cnt ? f.y : 0.0f;
      f.z = j + 2 < cnt ? f.z : 0.0f;
      f.w = j + 3 < cnt ? f.w : 0.0f;
      pre[k] = f;
    }
  };
  auto store = [&](int sg) {
    float* dst = zring + (size_t)(sg % kSlots) * 8 * kSeg;
#pragma unroll
    for (int k = 0; k < kPer; k++) {
      const int x = tid - kChainThreads + kProducers * k;
      reinterpret_cast<float4*>(dst)[x] = pre[k];  // [c][j]: x = c * kSeg / 4 + j / 4
    }
  };
  if (tid >= kChainThreads) {
    load(0);
    store(0);
    if (nseg > 1) {
      load(1);
      store(1);
    }
    if (nseg > 2) load(2);
  }
  __syncthreads();
  const int c = 4 * (tid >> 6) + ((tid & 63) >> 4);  // chain waves only
  float acc = 0.0f;
  for (int sg = 0; sg < nseg; sg++) {
    if (tid >= kChainThreads) {
      if (sg + 2 < nseg) store(sg + 2);  // slot of segment sg - 1, released at the last barrier
      if (sg + 3 < nseg) load(sg + 3);
    } else {
      int n = cnt_max - sg * kSeg;  // the same for every lane of the wave
      n = n < kSeg ? n : kSeg;
      acc = chain_group_lds<16>(acc, zring + (size_t)(sg % kSlots) * 8 * kSeg + (size_t)c * kSeg, n);
    }
    __syncthreads();
  }
  if (tid < kChainThreads && (tid & 15) == 0) zc[c] = acc;
  __syncthreads();
  if (tid == 0) cs.z[r] = finish_8lane(zc);
}

// Block sums of f_i = (u32)(e_i / Z * 2^24) + 1 (exact integers): all, and
// (mode 0) those below the symbol, plus the symbol's own f.
__global__ void __launch_bounds__(256) k_cdf_bfreq(int V, int mode, const uint32_t* symbols,
                                                   CdfScratch cs) {
  __shared__ uint64_t red[4];
  const int r = blockIdx.y, b = blockIdx.x, nb = gridDim.x;
  const int v8 = cdf_v8(V);
  const float* e = cs.ebuf + (size_t)r * 8 * v8;
  const float z = cs.z[r];
  const uint32_t want = mode == 0 ? symbols[r] : 0xffffffffu;
  // This block's elements b*4096 .. +4096 sit at chain positions
  // [c][512 b .. 512 b + 511]; thread x takes c = x / 32 and 16 consecutive j.
  const int c = threadIdx.x >> 5, j0 = b * (kCdfBlk / 8) + (threadIdx.x & 31) * 16;
  uint64_t sum = 0, below = 0;
#pragma unroll
  for (int k = 0; k < 16; k += 4) {
    float4 f4 = make_float4(0.f, 0.f, 0.f, 0.f);
    if (j0 + k + 3 < v8) f4 = *reinterpret_cast<const float4*>(e + (size_t)c * v8 + j0 + k);
    const float ev[4] = {f4.x, f4.y, f4.z, f4.w};
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int i = 8 * (j0 + k + u) + c;
      if (i < V) {
        const uint32_t f = cdf_freq(ev[u], z);
        sum += f;
        if ((uint32_t)i < want) below += f;
        if ((uint32_t)i == want) cs.symf[r] = f;
      }
    }
  }
  sum = block_sum_u64_256(sum, red);
  if (mode == 0) below = block_sum_u64_256(below, red);
  if (threadIdx.x == 0) {
    cs.bsum[(size_t)r * nb + b] = sum;
    if (mode == 0) cs.bbelow[(size_t)r * nb + b] = below;
  }
}

// Per-row finish: totals (and the CdfError::TotalTooLarge check), the
// symbol range (mode 0) or the decoder lookup (mode 2: block search, then a
// scan of the f_i of that block in symbol order).  Mode 4 (one row) is the
// lookup of RangeDecoder::decode_freq's value (det-coder range.rs:110-126),
// formed here from the decoder's window cml = code - low and rng = range:
// value = cml / (rng / total), valid when 0 < total < 2^31, rng / total > 0
// and value < total (the host's decode_freq accepts exactly these).  Its
// results go to pack[0..6]: symbol, cum, freq, total, error bits, value,
// valid (1 or 0), for one copy to the host.
__global__ void __launch_bounds__(256) k_cdf_finish(int V, int nb, int tail, int mode,
                                                    const uint32_t* symbols,
                                                    const uint64_t* values, uint64_t* cum,
                                                    uint32_t* freq, uint64_t* total, uint32_t* sym,
                                                    CdfScratch cs, int* err, uint64_t cml,
                                                    uint64_t rng, uint64_t* pack) {
  __shared__ uint64_t scan[256];
  __shared__ int blk_sh;
  __shared__ uint64_t off_sh;
  __shared__ uint64_t found[3];  // mode 4: symbol, cum, freq
  const int r = blockIdx.x, tid = threadIdx.x;
  // Row totals: the block sums in order (exact, order free).
  uint64_t run = 0, below = 0;
  for (int b = 0; b < nb; b++) {
    run += cs.bsum[(size_t)r * nb + b];
    if (mode == 0) below += cs.bbelow[(size_t)r * nb + b];
  }
  const uint64_t tot_all = run + (uint64_t)tail;
  int mybits = 0;  // thread 0's own flags, for the pack
  if (tid == 0 && (run >= (1ull << 31) || tot_all >= (1ull << 31))) {
    flag(err, ERRBIT_CDF_TOTAL);
    mybits |= ERRBIT_CDF_TOTAL;
  }
  if (mode == 0) {
    if (tid == 0) {
      const uint32_t s = symbols[r];
      if (s < (uint32_t)V) {
        cum[r] = below;
        freq[r] = cs.symf[r];
      } else {
        cum[r] = run + (s - (uint32_t)V);
        freq[r] = 1;
      }
      total[r] = tot_all;
    }
    return;
  }
  if (mode == 3) {
    if (tid == 0) total[r] = tot_all;
    return;
  }
  // modes 2 and 4; every thread forms the same target
  uint64_t target;
  bool valid = true;
  if (mode == 4) {
    valid = tot_all != 0 && tot_all < (1ull << 31);
    const uint64_t q = valid ? rng / tot_all : 0;
    valid = valid && q != 0;
    target = valid ? cml / q : 0;
    valid = valid && target < tot_all;
  } else {
    target = values[r];
  }
  auto put = [&](uint32_t sy, uint64_t cu, uint32_t fr) {
    if (mode == 4) {
      found[0] = sy;
      found[1] = cu;
      found[2] = fr;
    } else {
      sym[r] = sy;
      cum[r] = cu;
      freq[r] = fr;
    }
  };
  if (tid == 0) {
    if (mode != 4) total[r] = tot_all;
    found[0] = found[1] = found[2] = 0;
    int blk = -1;
    uint64_t off = 0;
    if (!valid) {
    } else if (target < run) {
      for (int b = 0; b < nb; b++) {
        const uint64_t sb = cs.bsum[(size_t)r * nb + b];
        if (target < off + sb) {
          blk = b;
          break;
        }
        off += sb;
      }
    } else {
      const uint64_t o = target - run;
      if (o < (uint64_t)tail) {
        put((uint32_t)(V + o), target, 1u);
      } else {
        flag(err, ERRBIT_CDF_LOOKUP);
        mybits |= ERRBIT_CDF_LOOKUP;
      }
    }
    blk_sh = blk;
    off_sh = off;
  }
  __syncthreads();
  const int blk = blk_sh;
  if (blk >= 0) {
    const int v8 = cdf_v8(V);
    const float* e = cs.ebuf + (size_t)r * 8 * v8;
    const float z = cs.z[r];
    // thread tid owns symbols blk*4096 + 16 tid .. +15 (ascending)
    uint32_t f[16];
    uint64_t local = 0;
    const int i0 = blk * kCdfBlk + 16 * tid;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const int i = i0 + k;
      f[k] = i < V ? cdf_freq(e[(size_t)(i & 7) * v8 + (i >> 3)], z) : 0u;
      local += f[k];
    }
    uint64_t tot;
    const uint64_t incl = block_scan_u64(local, scan, &tot);
    uint64_t c0 = off_sh + incl - local;
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const int i = i0 + k;
      if (i < V && target >= c0 && target < c0 + f[k]) put((uint32_t)i, c0, f[k]);
      c0 += f[k];
    }
  }
  if (mode != 4) return;
  __syncthreads();
  if (tid == 0) {
    // the flags of the launches before this one (the forward's, the block
    // kernels'), read past the L1, and this thread's own
    const int prior = __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    pack[0] = found[0];
    pack[1] = found[1];
    pack[2] = found[2];
    pack[3] = tot_all;
    pack[4] = (uint64_t)(uint32_t)(prior | mybits);
    pack[5] = target;
    pack[6] = valid ? 1u : 0u;
  }
}

// The block kernels of launch_cdf_blocks: block maxima, exps, Z and block
// sums (mode 0: also the sums below symbols[r]).
void launch_cdf_block_pass(const float* logits, const uint32_t* rows, int R, int V, int mode,
                           const uint32_t* symbols, const CdfScratch& cs, int* err, hipStream_t s) {
  const int nb = cdf_nblk(V);
  launch_kernel(k_cdf_bmax, dim3(nb, R), dim3(256), 0, s, logits, rows, V, cs, err);
  launch_kernel(k_cdf_bexp, dim3(nb, R), dim3(256), 0, s, logits, rows, V, cs);
  constexpr size_t kZRing = 3 * 8 * 1024 * sizeof(float);  // k_cdf_z's segment ring
  static bool z_attr_set = false;
  if (!z_attr_set) {
    (void)hipFuncSetAttribute((const void*)k_cdf_z, hipFuncAttributeMaxDynamicSharedMemorySize,
                              (int)kZRing);
    z_attr_set = true;
  }
  launch_kernel(k_cdf_z, dim3(R), dim3(256), kZRing, s, V, cs);
  launch_kernel(k_cdf_bfreq, dim3(nb, R), dim3(256), 0, s, V, mode, symbols, cs);
}

void launch_cdf_blocks(const float* logits, const uint32_t* rows, int R, int V, int tail, int mode,
                       const uint32_t* symbols, const uint64_t* values, uint64_t* cum,
                       uint32_t* freq, uint64_t* total, uint32_t* sym, void* scratch,
                       bool finish_only, int* err, hipStream_t s) {
  const int nb = cdf_nblk(V);
  CdfScratch cs = cdf_scratch(scratch, R, V);
  if (!finish_only) launch_cdf_block_pass(logits, rows, R, V, mode, symbols, cs, err, s);
  launch_kernel(k_cdf_finish, dim3(R), dim3(256), 0, s, V, nb, tail, mode, symbols, values, cum,
                freq, total, sym, cs, err, (uint64_t)0, (uint64_t)0, (uint64_t*)nullptr);
}

void launch_cdf_decode(const float* logits, int V, int tail, uint64_t cml, uint64_t rng, void* scratch,
                       uint64_t* pack, int* err, hipStream_t s) {
  const int nb = cdf_nblk(V);
  CdfScratch cs = cdf_scratch(scratch, 1, V);
  launch_cdf_block_pass(logits, nullptr, 1, V, 4, nullptr, cs, err, s);
  launch_kernel(k_cdf_finish, dim3(1), dim3(256), 0, s, V, nb, tail, 4, (const uint32_t*)nullptr,
                (const uint64_t*)nullptr, (uint64_t*)nullptr, (uint32_t*)nullptr, (uint64_t*)nullptr,
                (uint32_t*)nullptr, cs, err, cml, rng, pack);
}

void launch_cdf(const float* logits, int R, int V, int tail, int mode, const uint32_t* symbols,
                const uint64_t* values, uint64_t* cum, uint32_t* freq, uint64_t* total,
                uint32_t* sym, uint32_t* freq_tab, uint64_t* cum_tab, int* err, hipStream_t s) {
  launch_kernel(k_cdf, dim3(R), dim3(kCdfThreads), 0, s, logits, V, tail, mode, symbols,
                     values, cum, freq, total, sym, freq_tab, cum_tab, err);
}

// ---------------------------------------------------------------------------
// parity entry points
__global__ void k_exp(const float* in, float* out, int n, int which) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  // which 2: the softmax / CDF exp restated for t <= 0 (t > 0 is outside
  // its domain; callers of the parity entry pass t <= 0 or NaN)
  out[i] = which == 0 ? expf_det(in[i]) : which == 1 ? silu_det(in[i]) : exp_clamped(in[i]);
}

void launch_exp_f32(const float* in, float* out, int n, int which, hipStream_t s) {
  launch_kernel(k_exp, dim3((n + 255) / 256), dim3(256), 0, s, in, out, n, which);
}

__global__ void k_f16(const uint16_t* in, float* out, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = f16_to_f32(in[i]);
}

void launch_f16_to_f32(const uint16_t* in, float* out, int n, hipStream_t s) {
  launch_kernel(k_f16, dim3((n + 255) / 256), dim3(256), 0, s, in, out, n);
}

__global__ void k_div_sqrt(const float* a, const float* b, float* q, float* r, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  q[i] = a[i] / b[i];
  r[i] = sqrtf(a[i]);
}

void launch_div_sqrt(const float* a, const float* b, float* q, float* r, int n, hipStream_t s) {
  launch_kernel(k_div_sqrt, dim3((n + 255) / 256), dim3(256), 0, s, a, b, q, r, n);
}

// ---------------------------------------------------------------------------
// Measurement support: the issue rate of the instruction mix of the
// reference's f32 chains, separately rounded multiplies and adds (no FMA, no
// packed math).  Every lane runs eight independent multiply chains and eight
// independent add chains, 16 VALU instructions per iteration, so the rate
// is the VALU's, not a dependency's.  Both operands are per-lane registers,
// as in the kernels (their operands come from LDS and memory): a SIMD
// issues two such instructions from different waves at once, where an
// operand read from a scalar register halves the rate.  The result is
// written only for a value no input produces, which keeps the work live.
__global__ void __launch_bounds__(1024) k_valu_probe(float* out, float a0, float b0, int iters) {
  float x[8], y[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    x[i] = (float)threadIdx.x * 1e-3f + (float)i;
    y[i] = x[i] * 0.5f;
  }
  // per-lane copies of the operands (the asm hides that they are uniform)
  float a = a0, b = b0;
  asm volatile("" : "+v"(a), "+v"(b));
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      x[i] = x[i] * a;
      y[i] = y[i] + b;
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; i++) s = s + (x[i] + y[i]);
  if (s == -1.0f) out[threadIdx.x] = s;
}

void launch_valu_probe(float* out, int workgroups, int iters, hipStream_t s) {
  launch_kernel(k_valu_probe, dim3(workgroups), dim3(1024), 0, s, out, 1.0001f, 1e-7f, iters);
}

}  // namespace dtl
