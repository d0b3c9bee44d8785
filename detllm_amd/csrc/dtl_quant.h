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

// Null outputs are not written.  With af_skew, the f32 values d q go to
// af[e + 4 (e / 64)] (a row with four floats of padding after every 64).
struct QuantOut {
  int8_t* qa;
  float* da;
  float* af;
  int8_t* qk;
  float* dk;
  int af_skew = 0;
};

// v: the lane's four elements; in: whether they exist; base: element offset
// of the span (a multiple of 256 within the [T][n] array).
__device__ __forceinline__ void quantize_span(const float v[4], bool in, size_t base, bool want_q8a,
                                              bool want_q8k, const QuantOut& q) {
  // (every lane of the wave must be active: the reductions exchange lanes by DPP)
  const int lane = threadIdx.x & 63;
  const size_t off = base + 4 * lane;
  float ax[4];
#pragma unroll
  for (int c = 0; c < 4; c++) ax[c] = v[c] < 0.0f ? -v[c] : v[c];
  if (want_q8a) {
    // amax over the 32-element block (max is order independent).
    float amax = fmaxf(fmaxf(ax[0], ax[1]), fmaxf(ax[2], ax[3]));
    amax = fmaxf(amax, dpp_f32<kDppXor1>(amax));
    amax = fmaxf(amax, dpp_f32<kDppXor2>(amax));
    amax = fmaxf(amax, dpp_f32<kDppMirror8>(amax));
    if (in) {
      int8_t qv[4];
      float fv[4];
      // d = amax / 127 and the quotients v / d, each rounded to nearest.
      // From amax = 2^-92 up, by reciprocals and one fma correction
      // (div_recip); below, and for amax = 0, by division.
      float d, yv[4];
      if (amax >= 0x1p-92f) {
        d = div_recip(amax, 127.0f, 1.0f / 127.0f);
        const float rd = 1.0f / d;
#pragma unroll
        for (int c = 0; c < 4; c++) yv[c] = div_recip(v[c], d, rd);
      } else {
        d = amax / 127.0f;
#pragma unroll
        for (int c = 0; c < 4; c++) yv[c] = v[c] / d;
      }
      // Selects, not branches (per-element branches cost a mask round trip
      // each): y - 0.5 and y + (-0.5) are the same rounded sum, and an
      // all-zero block (whose quotients are 0 / 0) stores 0.
      const bool zero = amax == 0.0f;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const float y = yv[c];
        int r = f32_as_i32(y + (y < 0.0f ? -0.5f : 0.5f));
        r = r < -127 ? -127 : (r > 127 ? 127 : r);
        qv[c] = zero ? (int8_t)0 : (int8_t)r;
        fv[c] = zero ? 0.0f : d * (float)r;
      }
      uint32_t packed = (uint32_t)(uint8_t)qv[0] | ((uint32_t)(uint8_t)qv[1] << 8) |
                        ((uint32_t)(uint8_t)qv[2] << 16) | ((uint32_t)(uint8_t)qv[3] << 24);
      if (q.qa) *reinterpret_cast<uint32_t*>(q.qa + off) = packed;
      if (q.af)
        *reinterpret_cast<float4*>(q.af + (q.af_skew ? off + ((off >> 6) << 2) : off)) =
            make_float4(fv[0], fv[1], fv[2], fv[3]);
      if (q.da && (lane & 7) == 0) q.da[off / 32] = amax == 0.0f ? 0.0f : d;
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
    // the combine is commutative and associative: DPP steps within each
    // sixteen lanes, then the two exchanges across rows
    auto take = [&](float ox, float ov, int oi) {
      if (ox > bx || (ox == bx && oi < bi)) {
        bx = ox;
        bi = oi;
        bv = ov;
      }
    };
    take(dpp_f32<kDppXor1>(bx), dpp_f32<kDppXor1>(bv), dpp_i32<kDppXor1>(bi));
    take(dpp_f32<kDppXor2>(bx), dpp_f32<kDppXor2>(bv), dpp_i32<kDppXor2>(bi));
    take(dpp_f32<kDppMirror8>(bx), dpp_f32<kDppMirror8>(bv), dpp_i32<kDppMirror8>(bi));
    take(dpp_f32<kDppMirror16>(bx), dpp_f32<kDppMirror16>(bv), dpp_i32<kDppMirror16>(bi));
    // across the four rows by DPP row broadcasts: rows 1 and 3 take rows 0
    // and 2 (lane 15, lane 47), then rows 2 and 3 take lane 31 (rows 0-1),
    // so lane 63 holds the wave's; rows not written keep their own values
    // and combine with themselves
    take(__int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(bx), __float_as_int(bx), kDppRowBcast15, 0xa, 0xf, false)),
         __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(bv), __float_as_int(bv), kDppRowBcast15, 0xa, 0xf, false)),
         __builtin_amdgcn_update_dpp(bi, bi, kDppRowBcast15, 0xa, 0xf, false));
    take(__int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(bx), __float_as_int(bx), kDppRowBcast31, 0xc, 0xf, false)),
         __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(bv), __float_as_int(bv), kDppRowBcast31, 0xc, 0xf, false)),
         __builtin_amdgcn_update_dpp(bi, bi, kDppRowBcast31, 0xc, 0xf, false));
    bx = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bx), 63));
    bv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), 63));
    float mx = bx == 0.0f ? 0.0f : bv;
    if (in) {
      // Stored class-major inside the 256-block (element e at (e % 8) * 32 + e / 8),
      // the order the Q6_K kernels consume the eight lane sums in.
      float iscale = -127.0f / mx;
#pragma unroll
      for (int c = 0; c < 4; c++) {
        int e = 4 * lane + c;
        const float val = iscale * v[c] + 12582912.0f;
        int r = (int)(f2u(val) & 0x007fffffu) - 0x00400000;
        r = r > 127 ? 127 : r;
        q.qk[base + (e & 7) * 32 + (e >> 3)] = mx != 0.0f ? (int8_t)r : (int8_t)0;
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
