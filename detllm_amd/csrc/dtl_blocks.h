// Element accessors of ggml quant blocks shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dtl {

// det-quant lib.rs:531-552: 6-bit quant of element e (0..255) of a Q6_K body.
__device__ __forceinline__ int q6k_quant(const uint8_t* body, int e) {
  int half = e >> 7, within = e & 127, l = within & 31, part = within >> 5;
  uint8_t qlb = body[half * 64 + l + (part & 1) * 32];
  int ql = (part < 2) ? (qlb & 0x0f) : (qlb >> 4);
  int qh = (body[128 + half * 32 + l] >> (2 * part)) & 3;
  return (ql | (qh << 4)) - 32;
}

// Scale index of element e: q6_k_scale_index (lib.rs:554-568) equals e/16.
__device__ __forceinline__ int q6k_scale(const uint8_t* body, int e) {
  return (int)(int8_t)body[192 + (e >> 4)];
}

}  // namespace dtl
