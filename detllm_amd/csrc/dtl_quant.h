// Activation quantisation shared by the kernels that form Q8A / Q8_K
// activations: Q8A (det-quant lib.rs:111-137) per 32-element block and Q8_K
// (lib.rs:139-172) per 256-element block.  One wave quantises one
// 256-element span: lane l holds elements 4l..4l+3, so a Q8A block is 8
// lanes and a Q8_K block the whole wave; every reduction is a wave shuffle.
// The outputs may live in global memory or in LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dtl_numerics.h"

namespace dtl {

struct QuantOut {
  int8_t* qa;
  float* da;
  float* af;
  int8_t* qk;
  float* dk;
};

// v: the lane's four elements; in: whether they exist; base: element offset
// of the span (a multiple of 256 within the [T][n] array).
__device__ __forceinline__ void quantize_span(const float v[4], bool in, size_t base, bool want_q8a,
                                              bool want_q8k, const QuantOut& q) {
  const int lane = threadIdx.x & 63;
  const size_t off = base + 4 * lane;
  float ax[4];
#pragma unroll
  for (int c = 0; c < 4; c++) ax[c] = v[c] < 0.0f ? -v[c] : v[c];
  if (want_q8a) {
    // amax over the 32-element block (max is order independent).
    float amax = fmaxf(fmaxf(ax[0], ax[1]), fmaxf(ax[2], ax[3]));
#pragma unroll
    for (int m = 4; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m));
    if (in) {
      int8_t qv[4];
      float fv[4];
      float d = amax / 127.0f;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        if (amax == 0.0f) {
          qv[c] = 0;
          fv[c] = 0.0f;
        } else {
          float y = v[c] / d;
          int r = y < 0.0f ? f32_as_i32(y - 0.5f) : f32_as_i32(y + 0.5f);
          r = r < -127 ? -127 : (r > 127 ? 127 : r);
          qv[c] = (int8_t)r;
          fv[c] = d * (float)r;
        }
      }
      uint32_t packed = (uint32_t)(uint8_t)qv[0] | ((uint32_t)(uint8_t)qv[1] << 8) |
                        ((uint32_t)(uint8_t)qv[2] << 16) | ((uint32_t)(uint8_t)qv[3] << 24);
      *reinterpret_cast<uint32_t*>(q.qa + off) = packed;
      if (q.af) *reinterpret_cast<float4*>(q.af + off) = make_float4(fv[0], fv[1], fv[2], fv[3]);
      if ((lane & 7) == 0) q.da[off / 32] = amax == 0.0f ? 0.0f : d;
    }
  }
  if (want_q8k) {
    // Signed max: the first element with the strictly largest |x|.  Reduce
    // (|x|, index, x) taking the larger |x| and, on ties, the smaller index.
    float bx = -1.0f, bv = 0.0f;
    int bi = 0;
#pragma unroll
    for (int c = 0; c < 4; c++)
      if (in && ax[c] > bx) {
        bx = ax[c];
        bv = v[c];
        bi = 4 * lane + c;
      }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      float ox = __shfl_xor(bx, m), ov = __shfl_xor(bv, m);
      int oi = __shfl_xor(bi, m);
      if (ox > bx || (ox == bx && oi < bi)) {
        bx = ox;
        bi = oi;
        bv = ov;
      }
    }
    float mx = bx == 0.0f ? 0.0f : bv;
    if (in) {
      // Stored class-major inside the 256-block (element e at (e % 8) * 32 + e / 8),
      // the order the Q6_K kernels consume the eight lane sums in.
      float iscale = -127.0f / mx;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        int e = 4 * lane + c;
        int r = 0;
        if (mx != 0.0f) {
          float val = iscale * v[c] + 12582912.0f;
          r = (int)(f2u(val) & 0x007fffffu) - 0x00400000;
          if (r > 127) r = 127;
        }
        q.qk[base + (e & 7) * 32 + (e >> 3)] = (int8_t)r;
      }
      if (lane == 0) q.dk[base / 256] = mx == 0.0f ? 0.0f : 1.0f / iscale;
    }
  }
}

// Q8A of one value per lane, 32-lane blocks (lanes 0-31 and 32-63 of a
// wave are two blocks): the same amax, scale and rounding as quantize_span.
// base: element offset of lane 0 (a multiple of 32).  Lanes with store off
// take part in the reductions only.
__device__ __forceinline__ void quantize_q8a_lanes(float v, size_t base, const QuantOut& q,
                                                   bool store = true) {
  const int lane = threadIdx.x & 63;
  float amax = v < 0.0f ? -v : v;
#pragma unroll
  for (int m = 16; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m));
  int8_t qv = 0;
  float fv = 0.0f;
  const float d = amax / 127.0f;
  if (amax != 0.0f) {
    const float y = v / d;
    int r = y < 0.0f ? f32_as_i32(y - 0.5f) : f32_as_i32(y + 0.5f);
    r = r < -127 ? -127 : (r > 127 ? 127 : r);
    qv = (int8_t)r;
    fv = d * (float)r;
  }
  if (!store) return;
  q.qa[base + lane] = qv;
  if (q.af) q.af[base + lane] = fv;
  if ((lane & 31) == 0) q.da[(base + lane) / 32] = amax == 0.0f ? 0.0f : d;
}

}  // namespace dtl
