// Q4_K chunk GEMMs (teacher-forced encode) with the products formed on the
// matrix cores and the chains' adds on the VALU: the rows x positions of
// k_q4k_f32m (dtl_gemm.hip), value for value, at one VALU instruction per
// multiply-add instead of two.  Built with the VGPR form of the MFMA
// results (-mllvm -amdgpu-mfma-vgpr-form): the VALU adds read them
// directly, where results in accumulation registers would need a copy
// (v_accvgpr_read) per product.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dtl_device.h"
#include "dtl_numerics.h"

namespace dtl {

namespace {

__device__ __forceinline__ void flag(int* err, int bit) { atomicOr(err, bit); }

__device__ __forceinline__ bool store_epilogue(float v, float* out, size_t o, const float* bias, int r,
                                               int epi) {
  bool ok = finite(v);
  if (epi == EPI_BIAS) v = v + bias[r];
  else if (epi == EPI_RESIDUAL) v = out[o] + v;
  out[o] = v;
  return ok && finite(v);
}

}  // namespace

// The same chains with the products formed on the matrix cores.  An f32
// MFMA with one element of K and a zero accumulator is an outer product:
// v_mfma_f32_16x16x1f32 forms, in four blocks, D_b[i][j] = A_b[i] B_b[j]
// + 0, each rounded once, which is the rounded product w a (bit for bit,
// denormals included; a product of -0 comes out +0, which no chain that
// starts at +0.0 can tell apart, as x + -0 = x + +0 for every x but -0,
// and a sum of products from +0.0 is never -0).  The VALU then does only
// the chains' adds, one instruction per multiply-add instead of two.
//   wave tile  16 rows x 16 positions, 4 chains per lane: lane l holds rows
//              4 (l / 16) + c (c < 4) at position l % 16 (the D layout:
//              lane j + 16 (i / 4), register 4 b + i % 4)
//   16 elements per four MFMAs: MFMA m's block b takes element k0 + 4 b + m,
//              so a lane's A operands over the four are one float4 of its
//              row at k0 + 4 (l / 16) (A_b[i] comes from lane i + 16 b), and
//              its B operands one float4 of its position there; register
//              4 b + c of MFMA m is chain c's product at k0 + 4 b + m, and
//              the adds run b-major, then m: element order
//   pair       the wave's 16 tile rows alternate gate and up rows (tile row
//              i is matrix i % 2, row i / 2), so each lane holds a gate and
//              an up chain of two rows for the SwiGLU epilogue
// A workgroup of WP x WR waves stages 16 WP positions and 16 WR tile rows
// per 64-element slice in LDS, double-buffered as in k_q4k_f32m.
typedef float dtl_v4f __attribute__((ext_vector_type(4)));
typedef float dtl_v16f __attribute__((ext_vector_type(16)));

template <int WP, int WR, int MODE>
__global__ void __launch_bounds__(64 * WP * WR) k_q4k_mfp(Q4kF32Args p) {
  constexpr int NT = 64 * WP * WR;
  constexpr int PB = WP * 16;        // positions per workgroup
  constexpr int TR = WR * 16;        // tile rows per workgroup
  constexpr int NR = PB + TR;        // staged LDS rows per slice
  constexpr int SL = 64, LD = SL + 4;
  constexpr int F = NR * SL / 4;
  constexpr int PERT = (F + NT - 1) / NT;
  static_assert(PERT >= 1 && PERT <= 8, "staging slots per thread");
  static_assert(2 * NR * LD * 4 <= 64 * 1024, "LDS tile");
  __shared__ __align__(16) float st[2][NR][LD];
  const int cols = p.cols, T = p.T;
  const int rows_total = MODE == MODE_CAT ? p.rows0 + p.rows1 : p.rows0;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wp = wave % WP, wr = wave / WP;
  const int l16 = lane & 15, q = lane >> 4;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};

  // Staging slot k of thread x moves float4 f = x + k NT of the slice: LDS
  // row f / 16 (the positions, then the tile rows), columns 4 (f % 16);
  // clamped sources and unconditional loads as in k_q4k_f32m.
  auto slot_src = [&](int f) -> const float* {
    const int sr = f < F ? f >> 4 : 0, c4 = f & 15;
    if (sr < PB) {
      const int tt = blockIdx.y * PB + sr;
      return p.af + (size_t)(tt < T ? tt : T - 1) * cols + c4 * 4;
    }
    const int tr = sr - PB;
    if (MODE == MODE_PAIR) {
      const int rr = blockIdx.x * (TR / 2) + (tr >> 1);
      return ((tr & 1) ? p.w1 : p.w0) + (size_t)(rr < p.rows0 ? rr : p.rows0 - 1) * cols + c4 * 4;
    }
    int gg = blockIdx.x * TR + tr;
    gg = gg < rows_total ? gg : rows_total - 1;
    const bool m = MODE == MODE_CAT && gg >= p.rows0;
    return (m ? p.w1 : p.w0) + (size_t)(m ? gg - p.rows0 : gg) * cols + c4 * 4;
  };
  const int x = threadIdx.x;
#define DTL_SLOT_DECL(n)                                                      \
  const float* s##n = slot_src(x + (n) * NT);                                 \
  const int d##n = ((x + (n) * NT) >> 4) * LD + ((x + (n) * NT) & 15) * 4;    \
  const bool k##n = x + (n) * NT < F;                                         \
  float4 q##n;
  DTL_SLOT_DECL(0) DTL_SLOT_DECL(1) DTL_SLOT_DECL(2) DTL_SLOT_DECL(3)
  DTL_SLOT_DECL(4) DTL_SLOT_DECL(5) DTL_SLOT_DECL(6) DTL_SLOT_DECL(7)
#undef DTL_SLOT_DECL
#define DTL_ISSUE_M(e0)                                                       \
  do {                                                                        \
    q0 = *(const float4*)(s0 + (e0));                                         \
    if (PERT > 1) q1 = *(const float4*)(s1 + (e0));                           \
    if (PERT > 2) q2 = *(const float4*)(s2 + (e0));                           \
    if (PERT > 3) q3 = *(const float4*)(s3 + (e0));                           \
    if (PERT > 4) q4 = *(const float4*)(s4 + (e0));                           \
    if (PERT > 5) q5 = *(const float4*)(s5 + (e0));                           \
    if (PERT > 6) q6 = *(const float4*)(s6 + (e0));                           \
    if (PERT > 7) q7 = *(const float4*)(s7 + (e0));                           \
  } while (0)
#define DTL_COMMIT_M(b)                                                       \
  do {                                                                        \
    float* sb_ = &st[b][0][0];                                                \
    if (k0) *(float4*)(sb_ + d0) = q0;                                        \
    if (PERT > 1 && k1) *(float4*)(sb_ + d1) = q1;                            \
    if (PERT > 2 && k2) *(float4*)(sb_ + d2) = q2;                            \
    if (PERT > 3 && k3) *(float4*)(sb_ + d3) = q3;                            \
    if (PERT > 4 && k4) *(float4*)(sb_ + d4) = q4;                            \
    if (PERT > 5 && k5) *(float4*)(sb_ + d5) = q5;                            \
    if (PERT > 6 && k6) *(float4*)(sb_ + d6) = q6;                            \
    if (PERT > 7 && k7) *(float4*)(sb_ + d7) = q7;                            \
  } while (0)
  DTL_ISSUE_M(0);
  DTL_COMMIT_M(0);
  __syncthreads();
  dtl_v16f zero;
#pragma unroll
  for (int i = 0; i < 16; i++) zero[i] = 0.0f;
  const int boff = (wp * 16 + l16) * LD + 4 * q;       // this lane's position
  const int aoff = (PB + wr * 16 + l16) * LD + 4 * q;  // this lane's tile row
  int buf = 0;
  for (int e0 = 0; e0 < cols; e0 += SL) {
    const bool more = e0 + SL < cols;
    if (more) DTL_ISSUE_M(e0 + SL);
    const float* sb = &st[buf][0][0];
    dtl_v4f a4 = *(const dtl_v4f*)(sb + boff);
    dtl_v4f w4 = *(const dtl_v4f*)(sb + aoff);
#pragma unroll
    for (int g = 0; g < SL; g += 16) {
      dtl_v16f d[4];
#pragma unroll
      for (int m = 0; m < 4; m++) d[m] = __builtin_amdgcn_mfma_f32_16x16x1f32(w4[m], a4[m], zero, 0, 0, 0);
      // the next group's operands read while these products are added
      if (g + 16 < SL) {
        a4 = *(const dtl_v4f*)(sb + boff + g + 16);
        w4 = *(const dtl_v4f*)(sb + aoff + g + 16);
      }
      // the four MFMAs issue back to back, ahead of the adds: an add placed
      // right after the MFMA it reads waits out that MFMA's latency
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int b = 0; b < 4; b++)
#pragma unroll
        for (int m = 0; m < 4; m++)
#pragma unroll
          for (int c = 0; c < 4; c++) acc[c] += d[m][4 * b + c];
      // The next group's MFMAs take operands that pass through this empty
      // asm with the sums, so they follow these adds: one group's 64
      // results are live at a time (hoisted, the sixteen MFMAs of a slice
      // needed 256 registers).
      asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]), "+v"(a4), "+v"(w4));
    }
    if (more) DTL_COMMIT_M(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
#undef DTL_ISSUE_M
#undef DTL_COMMIT_M
  const int t = blockIdx.y * PB + wp * 16 + l16;
  if (t >= T) return;
  bool ok = true;
  if (MODE == MODE_PAIR) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int row = blockIdx.x * (TR / 2) + wr * 8 + 2 * q + h;
      if (row >= p.rows0) continue;
      const float gv = acc[2 * h], uv = acc[2 * h + 1];
      const float v = silu_det(gv) * uv;
      ok &= finite(gv) && finite(uv) && finite(v);
      p.ffo[(size_t)t * p.rows0 + row] = v;
    }
  } else {
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int g = blockIdx.x * TR + wr * 16 + 4 * q + c;
      if (g >= rows_total) continue;
      const bool m = MODE == MODE_CAT && g >= p.rows0;
      const int local = m ? g - p.rows0 : g;
      const int R = m ? p.rows1 : p.rows0;
      ok &= store_epilogue(acc[c], m ? p.out1 : p.out0, (size_t)t * R + local, m ? p.bias1 : p.bias0,
                           local, p.epi);
    }
  }
  if (!ok) flag(p.err, ERRBIT_NON_FINITE);
}

namespace {
template <int WP, int WR, int MODE>
void launch_mfp(const Q4kF32Args& a, hipStream_t s) {
  constexpr int PB = WP * 16, TR = WR * 16;
  const int rows_grid = MODE == MODE_PAIR ? 2 * a.rows0 : (MODE == MODE_CAT ? a.rows0 + a.rows1 : a.rows0);
  dim3 grid((rows_grid + TR - 1) / TR, (a.T + PB - 1) / PB);
  launch_kernel(k_q4k_mfp<WP, WR, MODE>, grid, dim3(64 * WP * WR), 0, s, a);
}
}  // namespace

// Measurement support: the rate of k_q4k_mfp's inner pattern on a chip
// with nothing else to do, four 16x16x1 outer products (4096 products per
// wave) and the 64 ordered adds per lane that take them into four chains,
// with operands the compiler must treat as new each iteration.  A SIMD runs
// the f32 MFMAs and the VALU adds one after the other, not side by side, so
// this, not either unit's own peak, bounds the Q4_K chunk GEMMs.  Four
// waves per SIMD (k_q4k_mfp's occupancy); the result is written only for a
// value no input produces, which keeps the work live.
__global__ void __launch_bounds__(256) k_mfp_probe(float* out, float a0, float b0, int iters) {
  const int lane = threadIdx.x & 63;
  dtl_v4f a4, w4;
#pragma unroll
  for (int m = 0; m < 4; m++) {
    a4[m] = a0 + (float)(lane + m);
    w4[m] = b0 - (float)(lane * m);
  }
  dtl_v16f zero;
#pragma unroll
  for (int i = 0; i < 16; i++) zero[i] = 0.0f;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int it = 0; it < iters; it++) {
    dtl_v16f d[4];
#pragma unroll
    for (int m = 0; m < 4; m++) d[m] = __builtin_amdgcn_mfma_f32_16x16x1f32(w4[m], a4[m], zero, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int b = 0; b < 4; b++)
#pragma unroll
      for (int m = 0; m < 4; m++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[c] += d[m][4 * b + c];
    asm volatile("" : "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]), "+v"(acc[3]), "+v"(a4), "+v"(w4));
  }
  const float s = acc[0] + acc[1] + acc[2] + acc[3];
  if (s == -1.0f) out[threadIdx.x] = s;
}

void launch_mfp_probe(float* out, int workgroups, int iters, hipStream_t s) {
  launch_kernel(k_mfp_probe, dim3(workgroups), dim3(256), 0, s, out, 1.0001f, 0.5f, iters);
}

// Tiles (waves over positions x rows), chosen on the pipelined TinyLlama
// encode (64 positions, four chunks in flight; ms per step): gate + up
// 2 x 2 (98.5; 4 x 1 100.5, 2 x 1 105.8, 1 x 2 106.0), the other matrices
// 4 x 1 (98.5; 2 x 2 100.5, 2 x 1 106.4, 1 x 2 106.4, 1 x 1 109.2).
void launch_q4k_mfp(const Q4kF32Args& a, int mode, hipStream_t s) {
  if (mode == MODE_PAIR) return launch_mfp<2, 2, MODE_PAIR>(a, s);
  if (mode == MODE_CAT) return launch_mfp<4, 1, MODE_CAT>(a, s);
  launch_mfp<4, 1, MODE_SINGLE>(a, s);
}

}  // namespace dtl
