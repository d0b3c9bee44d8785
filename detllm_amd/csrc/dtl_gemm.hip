// Token-parallel GEMMs for chunks of positions (teacher-forced encode).
//
// Mapping: one lane = one position (token) of the chunk, one wave = up to 64
// positions x R weight rows.  Every (row, position) output is a dependent
// f32 chain that its lane walks in the reference's order; the wave
// dequantises each weight once into LDS and all 64 lanes read it back as a
// broadcast, so the decode cost is shared by the whole chunk and the inner
// loop is one multiply + one add per weight (Q4_K) or one int8 dot4 per four
// weights (Q6_K, Q8_0).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <array>

#include "dtl_blocks.h"
#include "dtl_device.h"
#include "dtl_numerics.h"

namespace dtl {

namespace {

constexpr int kWaves = 4;  // waves per workgroup
constexpr int kGgmlQ4_0 = 2, kGgmlQ4K = 12, kGgmlQ6K = 14, kGgmlQ8_0 = 8;

__device__ __forceinline__ void flag(int* err, int bit) { atomicOr(err, bit); }

__device__ __forceinline__ uint32_t byte_of(const uint32_t w[3], int i) {
  return (w[i >> 2] >> (8 * (i & 3))) & 0xffu;
}

// Q4_K 6-bit scale and min of sub-block j from the 12 packed bytes held as
// three little-endian words (det-quant lib.rs:519-529).
__device__ __forceinline__ void q4k_scale_min_w(const uint32_t s[3], int j, int* sc, int* mn) {
  if (j < 4) {
    *sc = (int)(byte_of(s, j) & 0x3f);
    *mn = (int)(byte_of(s, j + 4) & 0x3f);
  } else {
    *sc = (int)((byte_of(s, j + 4) & 0x0f) | ((byte_of(s, j - 4) >> 6) << 4));
    *mn = (int)((byte_of(s, j + 4) >> 4) | ((byte_of(s, j) >> 6) << 4));
  }
}

__device__ __forceinline__ bool store_epilogue(float v, float* out, size_t o, const float* bias, int r,
                                               int epi) {
  bool ok = finite(v);
  if (epi == EPI_BIAS) v = v + bias[r];
  else if (epi == EPI_RESIDUAL) v = out[o] + v;
  out[o] = v;
  return ok && finite(v);
}

// The value the epilogue adds (bias[r], or the residual out[o]), read
// without a branch so that a kernel can load it ahead, long before its
// store: a load under a branch is waited for at once, and one such wait per
// output put a round trip per output on the kernel's tail.  With EPI_STORE
// the read (of out[o]) goes unused.
__device__ __forceinline__ float epilogue_operand(const float* out, size_t o, const float* bias, int r,
                                                  int epi) {
  return *(epi == EPI_BIAS ? bias + r : out + o);
}

__device__ __forceinline__ bool store_epilogue_pre(float v, float pre, float* out, size_t o, int epi) {
  bool ok = finite(v);
  if (epi == EPI_BIAS) v = v + pre;
  else if (epi == EPI_RESIDUAL) v = pre + v;
  out[o] = v;
  return ok && finite(v);
}

}  // namespace

// ---------------------------------------------------------------------------
// Q4_K: dot_q4_k_q8a (det-quant lib.rs:281-315).  Each lane's chain adds
// weight*activation for every element of the row in ascending order.
// PAIR computes rows of two matrices with the same shape (gate and up) and
// writes silu(gate)*up (det-model lib.rs:2420-2434) in the epilogue.
template <int R, bool PAIR>
__global__ void __launch_bounds__(256) k_q4k_tok(DevMat W0, DevMat W1, const float* __restrict__ af,
                                                 int T, float* out0, float* out1, float* ffo,
                                                 const float* bias, int epi, int* err) {
  constexpr int NM = PAIR ? 2 : 1;
  __shared__ __align__(16) float wl[kWaves][NM * R][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * kWaves + wave) * R;
  const int t = blockIdx.y * 64 + lane;
  const bool tok = t < T;
  const int rows = W0.rows, cols = W0.cols, nsb = W0.nb;
  const float* arow = af + (size_t)(tok ? t : 0) * cols;
  float acc[NM * R];
#pragma unroll
  for (int k = 0; k < NM * R; k++) acc[k] = 0.0f;
  // lane -> four consecutive elements of one sub-block
  const int wi = lane & 31, hh = lane >> 5;
  const int sub = 2 * (wi >> 3) + hh;
  const int e0 = sub * 32 + (wi & 7) * 4;

  for (int sb = 0; sb < nsb; sb++) {
#pragma unroll
    for (int m = 0; m < NM; m++) {
      const DevMat& W = m ? W1 : W0;
#pragma unroll
      for (int r = 0; r < R; r++) {
        int row = row0 + r;
        float4 w4 = make_float4(0.f, 0.f, 0.f, 0.f);
        if (row < rows) {
          size_t blk = (size_t)row * nsb + sb;
          const uint32_t* h = (const uint32_t*)(W.hdr + blk * 16);
          uint32_t h0 = h[0];
          uint32_t s[3] = {h[1], h[2], h[3]};
          float d = f16_to_f32((uint16_t)(h0 & 0xffff));
          float dmin = f16_to_f32((uint16_t)(h0 >> 16));
          int sc, mn;
          q4k_scale_min_w(s, sub, &sc, &mn);
          float dsc = d * (float)sc, dm = dmin * (float)mn;
          uint32_t qw = ((const uint32_t*)((const uint8_t*)W.w + blk * 128))[wi];
          uint32_t q = (qw >> (4 * hh)) & 0x0f0f0f0fu;
          w4.x = dsc * (float)(q & 0xff) - dm;
          w4.y = dsc * (float)((q >> 8) & 0xff) - dm;
          w4.z = dsc * (float)((q >> 16) & 0xff) - dm;
          w4.w = dsc * (float)(q >> 24) - dm;
        }
        *(float4*)&wl[wave][m * R + r][e0] = w4;
      }
    }
    __builtin_amdgcn_wave_barrier();
    // 16 activations per slice held in registers; each row's 16 weights
    // come from LDS as four broadcast 128-bit reads.
#pragma unroll 1
    for (int s = 0; s < 16; s++) {
      float a[16];
      const float4* ap = (const float4*)(arow + sb * 256 + s * 16);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        float4 v = ap[i];  // rows past T read row 0 and are never stored
        a[4 * i] = v.x;
        a[4 * i + 1] = v.y;
        a[4 * i + 2] = v.z;
        a[4 * i + 3] = v.w;
      }
#pragma unroll
      for (int k = 0; k < NM * R; k++) {
        const float4* wp = (const float4*)&wl[wave][k][s * 16];
        float c = acc[k];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          float4 w = wp[i];
          c += w.x * a[4 * i];
          c += w.y * a[4 * i + 1];
          c += w.z * a[4 * i + 2];
          c += w.w * a[4 * i + 3];
        }
        acc[k] = c;
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
  if (!tok) return;
  bool ok = true;
#pragma unroll
  for (int r = 0; r < R; r++) {
    int row = row0 + r;
    if (row >= rows) continue;
    size_t o = (size_t)t * rows + row;
    if (PAIR) {
      float g = acc[r], u = acc[R + r];
      float v = silu_det(g) * u;
      ok &= finite(g) && finite(u) && finite(v);
      if (out0) out0[o] = g;
      if (out1) out1[o] = u;
      ffo[o] = v;
    } else {
      ok &= store_epilogue(acc[r], out0, o, bias, row, epi);
    }
  }
  if (!ok) flag(err, ERRBIT_NON_FINITE);
}

// ---------------------------------------------------------------------------
// Q6_K: dot_q6_k_q8k (det-quant lib.rs:353-397).  The eight lane sums
// aux32[l] (l = element index mod 8) are exact integers: with the Q8_K
// activations stored class-major (class l at bytes 32l..32l+31 of each
// 256-block) and W' = scale*q6 split into int8 planes hi = W' >> 6 and
// lo = W' & 63 in the same order, aux32[l] = 64*dot(hi_l, q_l) + dot(lo_l, q_l),
// eight dot4 per plane.  Then sums[l] += (dw*da)*aux32[l] per superblock and
// the final sequential combine 0 + s0 + ... + s7.
template <int R>
__global__ void __launch_bounds__(256) k_q6k_tok(DevMat W, const int8_t* __restrict__ qk,
                                                 const float* __restrict__ dk, int T, float* out,
                                                 const float* bias, int epi, int* err) {
  __shared__ __align__(16) int8_t hl[kWaves][R][2][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * kWaves + wave) * R;
  const int t = blockIdx.y * 64 + lane;
  const bool tok = t < T;
  const int rows = W.rows, cols = W.cols, nsb = W.nb;
  const int8_t* arow = qk + (size_t)(tok ? t : 0) * cols;
  const float* drow = dk + (size_t)(tok ? t : 0) * nsb;
  float sums[R][8];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int l = 0; l < 8; l++) sums[r][l] = 0.0f;
  // lane -> elements e0..e0+3 (same half, part and 16-element scale group)
  const int e0 = lane * 4;
  const int half = e0 >> 7, within = e0 & 127, l0 = within & 31, part = within >> 5;

  for (int sb = 0; sb < nsb; sb++) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      int row = row0 + r;
      uint32_t hiw = 0, low = 0;
      if (row < rows) {
        const uint8_t* body = (const uint8_t*)W.w + ((size_t)row * nsb + sb) * 208;
        uint32_t qlw = *(const uint32_t*)(body + half * 64 + l0 + (part & 1) * 32);
        uint32_t qhw = *(const uint32_t*)(body + 128 + half * 32 + l0);
        int scale = (int)(int8_t)body[192 + (e0 >> 4)];
        uint32_t nib = (part < 2 ? qlw : (qlw >> 4)) & 0x0f0f0f0fu;
        uint32_t two = (qhw >> (2 * part)) & 0x03030303u;
        uint32_t q6 = nib | (two << 4);  // four 6-bit codes
#pragma unroll
        for (int k = 0; k < 4; k++) {
          int v = (int)((q6 >> (8 * k)) & 0xff) - 32;
          int wp = scale * v;           // in [-4064, 4096]
          int hi = wp >> 6, lo = wp & 63;
          hiw |= (uint32_t)(uint8_t)hi << (8 * k);
          low |= (uint32_t)(uint8_t)lo << (8 * k);
        }
      }
      // scatter the four bytes to their class-major positions
#pragma unroll
      for (int k = 0; k < 4; k++) {
        int e = e0 + k;
        int p = (e & 7) * 32 + (e >> 3);
        hl[wave][r][0][p] = (int8_t)(hiw >> (8 * k));
        hl[wave][r][1][p] = (int8_t)(low >> (8 * k));
      }
    }
    __builtin_amdgcn_wave_barrier();
    float da = drow[sb];
    float d[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      int row = row0 + r < rows ? row0 + r : rows - 1;
      d[r] = f16_to_f32(W.d16[(size_t)row * nsb + sb]) * da;
    }
#pragma unroll
    for (int l = 0; l < 8; l++) {
      // the 32 class-l activation quants of this superblock
      const int4* ap = (const int4*)(arow + sb * 256 + l * 32);
      int4 a0 = ap[0];
      int4 a1 = ap[1];
#pragma unroll
      for (int r = 0; r < R; r++) {
        const int4* hp = (const int4*)&hl[wave][r][0][l * 32];
        const int4* lp = (const int4*)&hl[wave][r][1][l * 32];
        int4 h0 = hp[0], h1 = hp[1], q0 = lp[0], q1 = lp[1];
        int dh = 0, dl = 0;
        dh = __builtin_amdgcn_sdot4(h0.x, a0.x, dh, false);
        dh = __builtin_amdgcn_sdot4(h0.y, a0.y, dh, false);
        dh = __builtin_amdgcn_sdot4(h0.z, a0.z, dh, false);
        dh = __builtin_amdgcn_sdot4(h0.w, a0.w, dh, false);
        dh = __builtin_amdgcn_sdot4(h1.x, a1.x, dh, false);
        dh = __builtin_amdgcn_sdot4(h1.y, a1.y, dh, false);
        dh = __builtin_amdgcn_sdot4(h1.z, a1.z, dh, false);
        dh = __builtin_amdgcn_sdot4(h1.w, a1.w, dh, false);
        dl = __builtin_amdgcn_sdot4(q0.x, a0.x, dl, false);
        dl = __builtin_amdgcn_sdot4(q0.y, a0.y, dl, false);
        dl = __builtin_amdgcn_sdot4(q0.z, a0.z, dl, false);
        dl = __builtin_amdgcn_sdot4(q0.w, a0.w, dl, false);
        dl = __builtin_amdgcn_sdot4(q1.x, a1.x, dl, false);
        dl = __builtin_amdgcn_sdot4(q1.y, a1.y, dl, false);
        dl = __builtin_amdgcn_sdot4(q1.z, a1.z, dl, false);
        dl = __builtin_amdgcn_sdot4(q1.w, a1.w, dl, false);
        int aux = dh * 64 + dl;
        sums[r][l] += d[r] * (float)aux;
      }
      // keep the loads of one class from being hoisted over the previous one
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_wave_barrier();
  }
  if (!tok) return;
  bool ok = true;
#pragma unroll
  for (int r = 0; r < R; r++) {
    int row = row0 + r;
    if (row >= rows) continue;
    float v = 0.0f;
#pragma unroll
    for (int l = 0; l < 8; l++) v += sums[r][l];
    ok &= store_epilogue(v, out, (size_t)t * rows + row, bias, row, epi);
  }
  if (!ok) flag(err, ERRBIT_NON_FINITE);
}

// ---------------------------------------------------------------------------
// Q8_0: dot_q8_0_q8a (det-quant lib.rs:237-257): exact i32 block sums by
// dot4, (dw*da)*isum, block-ordered f32 chain per lane.
template <int R>
__global__ void __launch_bounds__(256) k_q8_0_tok(DevMat W, const int8_t* __restrict__ qa,
                                                  const float* __restrict__ da, int T, float* out,
                                                  const float* bias, int epi, int* err) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = (blockIdx.x * kWaves + wave) * R;
  const int t = blockIdx.y * 64 + lane;
  const bool tok = t < T;
  const int rows = W.rows, cols = W.cols, nb = W.nb;
  const int8_t* arow = qa + (size_t)(tok ? t : 0) * cols;
  const float* drow = da + (size_t)(tok ? t : 0) * nb;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; r++) acc[r] = 0.0f;
  for (int b = 0; b < nb; b++) {
    int4 a0 = ((const int4*)(arow + b * 32))[0];
    int4 a1 = ((const int4*)(arow + b * 32))[1];
    float dab = drow[b];
#pragma unroll
    for (int r = 0; r < R; r++) {
      int row = row0 + r < rows ? row0 + r : rows - 1;
      const int4* wp = (const int4*)((const int8_t*)W.w + (size_t)row * cols + b * 32);
      int4 w0 = wp[0], w1 = wp[1];
      int is = 0;
      is = __builtin_amdgcn_sdot4(w0.x, a0.x, is, false);
      is = __builtin_amdgcn_sdot4(w0.y, a0.y, is, false);
      is = __builtin_amdgcn_sdot4(w0.z, a0.z, is, false);
      is = __builtin_amdgcn_sdot4(w0.w, a0.w, is, false);
      is = __builtin_amdgcn_sdot4(w1.x, a1.x, is, false);
      is = __builtin_amdgcn_sdot4(w1.y, a1.y, is, false);
      is = __builtin_amdgcn_sdot4(w1.z, a1.z, is, false);
      is = __builtin_amdgcn_sdot4(w1.w, a1.w, is, false);
      float scale = f16_to_f32(W.d16[(size_t)row * nb + b]) * dab;
      acc[r] += scale * (float)is;
    }
  }
  if (!tok) return;
  bool ok = true;
#pragma unroll
  for (int r = 0; r < R; r++) {
    int row = row0 + r;
    if (row >= rows) continue;
    ok &= store_epilogue(acc[r], out, (size_t)t * rows + row, bias, row, epi);
  }
  if (!ok) flag(err, ERRBIT_NON_FINITE);
}

// ---------------------------------------------------------------------------
// Q4_K from an exact f32 copy of the weights (Q4kF32Args, the modes in
// dtl_device.h; one matrix, or two concatenated), every output one chain of
// products in element order.  The lanes of a wave are split over positions and rows, and each lane
// holds a PP x RP block of chains: lane = (p = lane % PW, r = lane / PW),
// RW = 64 / PW; the lane's positions are p + PW i (i < PP) and its rows
// r + RW j (j < RP), one chain per (position, row), every chain in
// element order.  A wave covers PW PP positions of RW RP
// rows; a workgroup is WP x WR waves covering PB positions of RB rows and
// stages each 64-element slice of those positions' activations and rows'
// weights in LDS once (double-buffered, the next slice's global loads in
// flight).  Per four elements a lane reads PP activation and RP weight
// float4 for PP RP chains: the blocking divides the LDS bytes per
// multiply-add, which bound the one-chain mapping, by the block's size
// over its perimeter.
template <int PW, int PP, int RP, int WP, int WR, int MODE>
__global__ void __launch_bounds__(64 * WP * WR) k_q4k_f32m(Q4kF32Args p) {
  static_assert(MODE != MODE_PAIR, "gate + up runs on k_q4k_mfp");
  constexpr int NT = 64 * WP * WR;
  constexpr int NM = 1;
  constexpr int RW = 64 / PW;
  constexpr int PWV = PW * PP, RWV = RW * RP;  // positions, rows per wave
  constexpr int PB = WP * PWV;                 // positions per workgroup
  constexpr int RB = WR * RWV;                 // rows per workgroup
  constexpr int NR = PB + NM * RB;             // staged LDS rows per slice
  constexpr int SL = 64, LD = SL + 4;          // elements per slice, padded LDS row
  constexpr int F = NR * SL / 4;               // float4 per slice
  constexpr int PERT = (F + NT - 1) / NT;
  static_assert(PERT >= 1 && PERT <= 8, "staging slots per thread");
  static_assert(2 * NR * LD * 4 <= 64 * 1024, "LDS tile");
  __shared__ __align__(16) float st[2][NR][LD];
  const int cols = p.cols, T = p.T;
  const int rows_total = MODE == MODE_CAT ? p.rows0 + p.rows1 : p.rows0;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wp = wave % WP, wr = wave / WP;
  const int pl = lane % PW, rl = lane / PW;
  const int prow = wp * PWV + pl;   // LDS row of position i: prow + PW i
  const int rrow = wr * RWV + rl;   // workgroup row of row j: rrow + RW j
  float acc[NM][PP][RP];
#pragma unroll
  for (int m = 0; m < NM; m++)
#pragma unroll
    for (int i = 0; i < PP; i++)
#pragma unroll
      for (int j = 0; j < RP; j++) acc[m][i][j] = 0.0f;

  // Staging slot k of thread x moves float4 f = x + k NT of the slice: LDS
  // row f / 16 (activations of position f / 16 first, then the weight rows,
  // matrix by matrix), columns 4 (f % 16).  Out-of-range positions and rows
  // read the last valid one; slots past the slice load a valid address and
  // store nothing, so every load is unconditional.
  auto slot_src = [&](int f) -> const float* {
    const int sr = f < F ? f >> 4 : 0, c4 = f & 15;
    if (sr < PB) {
      const int tt = blockIdx.y * PB + sr;
      return p.af + (size_t)(tt < T ? tt : T - 1) * cols + c4 * 4;
    }
    const int wrow = sr - PB;
    int gg = blockIdx.x * RB + wrow;
    gg = gg < rows_total ? gg : rows_total - 1;
    const bool m = MODE == MODE_CAT && gg >= p.rows0;
    return (m ? p.w1 : p.w0) + (size_t)(m ? gg - p.rows0 : gg) * cols + c4 * 4;
  };
  // Up to eight slots as named registers (an indexed array of them is not
  // kept in registers by the compiler across the conditional load/store).
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
  int buf = 0;
  for (int e0 = 0; e0 < cols; e0 += SL) {
    const bool more = e0 + SL < cols;
    if (more) DTL_ISSUE_M(e0 + SL);
    const float* sb = &st[buf][0][0];
#pragma unroll 4
    for (int e = 0; e < SL; e += 4) {
      float4 a[PP], w[NM][RP];
#pragma unroll
      for (int i = 0; i < PP; i++) a[i] = *(const float4*)(sb + (prow + PW * i) * LD + e);
#pragma unroll
      for (int m = 0; m < NM; m++)
#pragma unroll
        for (int j = 0; j < RP; j++)
          w[m][j] = *(const float4*)(sb + (PB + m * RB + rrow + RW * j) * LD + e);
#pragma unroll
      for (int m = 0; m < NM; m++)
#pragma unroll
        for (int i = 0; i < PP; i++)
#pragma unroll
          for (int j = 0; j < RP; j++) {
            float c = acc[m][i][j];
            c += w[m][j].x * a[i].x;
            c += w[m][j].y * a[i].y;
            c += w[m][j].z * a[i].z;
            c += w[m][j].w * a[i].w;
            acc[m][i][j] = c;
          }
    }
    if (more) DTL_COMMIT_M(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
#undef DTL_ISSUE_M
#undef DTL_COMMIT_M
  bool ok = true;
#pragma unroll
  for (int i = 0; i < PP; i++) {
    const int t = blockIdx.y * PB + prow + PW * i;
    if (t >= T) continue;
#pragma unroll
    for (int j = 0; j < RP; j++) {
      const int g = blockIdx.x * RB + rrow + RW * j;  // row of the concatenation
      if (g >= rows_total) continue;
      const bool m = MODE == MODE_CAT && g >= p.rows0;
      const int local = m ? g - p.rows0 : g;
      const int R = m ? p.rows1 : p.rows0;
      ok &= store_epilogue(acc[0][i][j], m ? p.out1 : p.out0, (size_t)t * R + local,
                           m ? p.bias1 : p.bias0, local, p.epi);
    }
  }
  if (!ok) flag(p.err, ERRBIT_NON_FINITE);
}

// Exact f32 copy of a Q4_K matrix: q4_k_value for every element.
__global__ void k_dequant_q4k(DevMat W, float* out) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t total = (size_t)W.rows * W.cols;
  if (i >= total) return;
  int row = (int)(i / W.cols), c = (int)(i % W.cols);
  int sb = c / 256, idx = c % 256, sub = idx / 32, within = idx % 32;
  size_t blk = (size_t)row * W.nb + sb;
  const uint32_t* h = (const uint32_t*)(W.hdr + blk * 16);
  uint32_t h0 = h[0];
  uint32_t s[3] = {h[1], h[2], h[3]};
  float d = f16_to_f32((uint16_t)(h0 & 0xffff)), dmin = f16_to_f32((uint16_t)(h0 >> 16));
  int sc, mn;
  q4k_scale_min_w(s, sub, &sc, &mn);
  uint8_t byte = ((const uint8_t*)W.w)[blk * 128 + (sub / 2) * 32 + within];
  int q = (sub & 1) ? (byte >> 4) : (byte & 0x0f);
  out[i] = (d * (float)sc) * (float)q - (dmin * (float)mn);
}

void launch_dequant_q4k(const DevMat& W, float* out, hipStream_t s) {
  size_t total = (size_t)W.rows * W.cols;
  launch_kernel(k_dequant_q4k, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, W, out);
}

// ---------------------------------------------------------------------------
// Q6_K on the int8 matrix cores (dot_q6_k_q8k, det-quant lib.rs:353-397).
// Per superblock sb and class c (element index mod 8) the reference's exact
// integer sums aux_c = sum_j W'[8j+c] * qa[8j+c] over the 32 elements of
// the class form a [rows x positions] product with K = 32.  With
// W' = scale*q6 = 64*hi + lo held as two int8 planes, aux_c is
// 64*(hi . qa) + (lo . qa): two v_mfma_i32_16x16x64_i8 (K quarters 2 and 3
// zero), exact in i32.  The f32 part, sums[c] += (dw*da)*aux_c per
// superblock in order and the final 0 + sums[0] + ... + sums[7], runs on the
// VALU as in the reference.  The Q8_K activations are class-major within
// each 256-block, so class c's 32 bytes are contiguous.
//
// One workgroup per 16-row tile x NT tiles of 16 positions.  MFMA
// operand layout (16x16x64 i8): lane l supplies row / position l % 16 and
// K quarter l / 16 (16 bytes); result register i of lane l is row
// 4 (l / 16) + i, position l % 16.
typedef int dtl_v4i __attribute__((ext_vector_type(4)));

__global__ void k_q6k_planes(DevMat W, int rows_pad, int8_t* planes) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int nb = W.nb;
  const size_t total = (size_t)rows_pad * nb * 256;
  if (idx >= total) return;
  const int row = (int)(idx / ((size_t)nb * 256));
  const int rem = (int)(idx % ((size_t)nb * 256));
  const int sb = rem >> 8, k = rem & 255;
  const int c = k >> 5, j = k & 31;
  int wp = 0;
  if (row < W.rows) {
    const uint8_t* body = (const uint8_t*)W.w + ((size_t)row * nb + sb) * 208;
    const int e = 8 * j + c;
    wp = q6k_scale(body, e) * q6k_quant(body, e);
  }
  const size_t base = ((((size_t)(row >> 4) * nb + sb) * 8 + c) * 2) * 512 + (row & 15) * 32 + j;
  planes[base] = (int8_t)(wp >> 6);
  planes[base + 512] = (int8_t)(wp & 63);
}

size_t q6k_planes_bytes(const DevMat& W) {
  return (size_t)((W.rows + 15) / 16) * 16 * W.nb * 256 * 2;
}

void launch_q6k_planes(const DevMat& W, int8_t* planes, hipStream_t s) {
  const int rows_pad = (W.rows + 15) / 16 * 16;
  const size_t total = (size_t)rows_pad * W.nb * 256;
  launch_kernel(k_q6k_planes, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, W, rows_pad,
                planes);
}

// K steps in flight per wave in the int8 MFMA GEMMs (slots r0, r1, ...):
// the Q6_K superblock's operands are four times a Q8_0 block pair's.
constexpr int kQ6kRing = 2;
constexpr int kMfmaRing = 4;

template <int NT>
__global__ void __launch_bounds__(256) k_q6k_mfma(const int8_t* __restrict__ planes,
                                                  const uint16_t* __restrict__ d16, int rows,
                                                  int nb, const int8_t* __restrict__ qk,
                                                  const float* __restrict__ dk, int T, float* out,
                                                  const float* bias, int epi, int* err) {
  // The eight class chains are independent until the final combine: wave w
  // runs classes 2w and 2w+1 of the workgroup's tile.
  __shared__ float part[8][NT][4][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int rt = blockIdx.x;
  const int p0 = blockIdx.y * 16 * NT;
  const int q = lane >> 4, li = lane & 15;
  const int cols = nb * 256;
  const dtl_v4i zero = {0, 0, 0, 0};
  // A operand: row li of the tile, bytes 16 (q & 1) .. of the class run
  // (quarters 2 and 3 read the same bytes and are zeroed).
  const int8_t* abase = planes + (size_t)rt * nb * 8192 + (size_t)(2 * wave) * 1024 + li * 32 +
                        (q & 1) * 16;
  // B operand: position p0 + 16 j + li (clamped to T - 1; not stored).
  const int8_t* bsrc[NT];
  const float* dsrc[NT];
#pragma unroll
  for (int j = 0; j < NT; j++) {
    int pos = p0 + 16 * j + li;
    pos = pos < T ? pos : T - 1;
    bsrc[j] = qk + (size_t)pos * cols + (2 * wave) * 32 + (q & 1) * 16;
    dsrc[j] = dk + (size_t)pos * nb;
  }
  // Rows of this lane's results: 16 rt + 4 q + i.
  const uint16_t* dwsrc[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    int row = rt * 16 + 4 * q + i;
    row = row < rows ? row : rows - 1;
    dwsrc[i] = d16 + (size_t)row * nb;
  }
  float sums[NT][2][4];
#pragma unroll
  for (int j = 0; j < NT; j++)
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
      for (int i = 0; i < 4; i++) sums[j][c][i] = 0.0f;
  // Operands of one superblock for this wave's two classes; the next
  // superblock's are in flight while the current one is multiplied.
  struct Ops {
    dtl_v4i a[2][2];
    dtl_v4i b[NT][2];
    uint16_t dw[4];
    float da[NT];
  };
  auto load = [&](Ops& o, int sb) {
    const int8_t* ab = abase + (size_t)sb * 8192;
#pragma unroll
    for (int c = 0; c < 2; c++) {
      o.a[c][0] = *(const dtl_v4i*)(ab + (2 * c) * 512);
      o.a[c][1] = *(const dtl_v4i*)(ab + (2 * c + 1) * 512);
    }
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
      for (int c = 0; c < 2; c++) o.b[j][c] = *(const dtl_v4i*)(bsrc[j] + sb * 256 + c * 32);
#pragma unroll
    for (int i = 0; i < 4; i++) o.dw[i] = dwsrc[i][sb];
#pragma unroll
    for (int j = 0; j < NT; j++) o.da[j] = dsrc[j][sb];
  };
  // valid false (a ring slot past the last superblock): every term added is
  // +0.0f, which leaves the sums' bits unchanged (a sum that starts at +0.0f
  // is never -0.0f), so the loop needs no branch around it.
  auto compute = [&](const Ops& o, bool valid) {
    float dd[NT][4];
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
      for (int i = 0; i < 4; i++) dd[j][i] = f16_to_f32(o.dw[i]) * o.da[j];
#pragma unroll
    for (int c = 0; c < 2; c++) {
      const dtl_v4i ahi = q < 2 ? o.a[c][0] : zero;
      const dtl_v4i alo = q < 2 ? o.a[c][1] : zero;
#pragma unroll
      for (int j = 0; j < NT; j++) {
        dtl_v4i acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi, o.b[j][c], zero, 0, 0, 0);
        acc = acc * 64;
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo, o.b[j][c], acc, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float term = dd[j][i] * (float)acc[i];
          sums[j][c][i] += valid ? term : 0.0f;
        }
      }
    }
  };
  // kQ6kRing superblocks in flight.  Every pass refills its slot (the
  // index clamped to the last superblock): with the refill under a branch
  // the compiler waits for every load in flight before the next compute.
  // (Named slots, not an array, and each refill after the last use of the
  // slot: otherwise the loop-carried registers get copies at the back edge,
  // and the copies wait for the loads.)
  auto last = [&](int i) { return i < nb ? i : nb - 1; };
  Ops r0, r1;
  load(r0, last(0));
  load(r1, last(1));
  // the epilogue's operands of this wave's outputs (see the final combine),
  // in flight with the first superblocks
  float pre[NT];
#pragma unroll
  for (int k = 0; k < NT; k++) {
    const int o = wave + 4 * k, j = o >> 2, i = o & 3;
    int pos = p0 + 16 * j + li;
    pos = pos < T ? pos : T - 1;
    int row = rt * 16 + 4 * q + i;
    row = row < rows ? row : rows - 1;
    pre[k] = epilogue_operand(out, (size_t)pos * rows + row, bias, row, epi);
  }
#define DTL_MFMA_STEP(r, i)                                                                \
  compute(r, (i) < nb);                                                                    \
  __builtin_amdgcn_sched_barrier(0);                                                       \
  load(r, last((i) + kQ6kRing));                                                           \
  __builtin_amdgcn_sched_barrier(0)
  for (int s0 = 0; s0 < nb; s0 += kQ6kRing) {
    DTL_MFMA_STEP(r0, s0);
    DTL_MFMA_STEP(r1, s0 + 1);
  }
#undef DTL_MFMA_STEP
#pragma unroll
  for (int c = 0; c < 2; c++)
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
      for (int i = 0; i < 4; i++) part[2 * wave + c][j][i][lane] = sums[j][c][i];
  __syncthreads();
  // Final combine 0 + sums[0] + ... + sums[7] in class order; the four
  // waves split the (position tile, register) outputs.
  bool ok = true;
#pragma unroll
  for (int k = 0; k < NT; k++) {
    const int o = wave + 4 * k, j = o >> 2, i = o & 3;
    const int pos = p0 + 16 * j + li;
    const int row = rt * 16 + 4 * q + i;
    if (row < rows && pos < T) {
      float v = 0.0f;
#pragma unroll
      for (int c = 0; c < 8; c++) v += part[c][j][i][lane];
      ok &= store_epilogue_pre(v, pre[k], out, (size_t)pos * rows + row, epi);
    }
  }
  if (!ok) flag(err, ERRBIT_NON_FINITE);
}

// ---------------------------------------------------------------------------
// Q8_0 / Q4_0 on the int8 matrix cores: dot_q8_0_q8a / dot_q4_0_q8a
// (det-quant lib.rs:237-279).  Per 32-element block b the reference forms
// the exact integer isum = sum_e qw[e] * qa[e], then c = (dw * da) * isum
// and one f32 chain per (row, position) over the blocks in order.  With K =
// 64 covering blocks 2p and 2p+1, v_mfma_i32_16x16x64_i8 gives block 2p's
// isum when the A operand's K quarters 2 and 3 are zero and block 2p+1's
// when quarters 0 and 1 are: both exact in i32.  The f32 part runs on the
// VALU in the reference's order.  Q4_0 uses the int8 copy of its weights
// (nibble - 8, element order) built at load.
//
// MFMA operand layout (16x16x64 i8): lane l supplies row / position l % 16
// and K quarter l / 16 (16 bytes); result register i of lane l is row
// 4 (l / 16) + i, position l % 16.  A wave covers 16 rows x 16 NT
// positions; a workgroup 4 / (4 / NT) row tiles x 64 positions.
template <int NT, bool EVEN>
__global__ void __launch_bounds__(256) k_q8_mfma(const int8_t* __restrict__ w8,
                                                 const uint16_t* __restrict__ d16, int rows, int nb,
                                                 const int8_t* __restrict__ qa,
                                                 const float* __restrict__ da, int T, float* out,
                                                 const float* bias, int epi, int* err) {
  constexpr int PT = 4 / NT;  // position tiles (of 16 NT) per workgroup
  constexpr int RT = 4 / PT;  // row tiles per workgroup
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int q = lane >> 4, li = lane & 15;
  const int row0 = (blockIdx.x * RT + wave / PT) * 16;
  const int p0 = blockIdx.y * 64 + (wave % PT) * 16 * NT;
  const int cols = nb * 32;
  const dtl_v4i zero = {0, 0, 0, 0};
  int arow = row0 + li;
  arow = arow < rows ? arow : rows - 1;
  const int8_t* asrc = w8 + (size_t)arow * cols + 16 * q;
  const int8_t* bsrc[NT];
  const float* dsrc[NT];
#pragma unroll
  for (int j = 0; j < NT; j++) {
    int pos = p0 + 16 * j + li;
    pos = pos < T ? pos : T - 1;
    bsrc[j] = qa + (size_t)pos * cols + 16 * q;
    dsrc[j] = da + (size_t)pos * nb;
  }
  const uint16_t* dwsrc[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    int row = row0 + 4 * q + i;
    row = row < rows ? row : rows - 1;
    dwsrc[i] = d16 + (size_t)row * nb;
  }
  float sums[NT][4];
#pragma unroll
  for (int j = 0; j < NT; j++)
#pragma unroll
    for (int i = 0; i < 4; i++) sums[j][i] = 0.0f;
  // Operands of one block pair; the next pair's are in flight while the
  // current one is multiplied.  In an odd last pair the second block's
  // quarters re-read the first block's bytes and are zeroed.
  // EVEN (an even block count, so every pair is whole and starts at an even
  // block): the pair's two weight scales of a row are one 32-bit load and
  // its two activation scales one 64-bit load (each load costs issue time;
  // a value packed from two loads would be waited for as soon as loaded).
  struct Ops {
    dtl_v4i a;
    dtl_v4i b[NT];
    uint32_t dw[2][4];  // EVEN: dw[0][i] holds both halves
    float dav[2][NT];
  };
  auto load = [&](Ops& o, int pr) {
    const int b0 = 2 * pr;
    const bool two = b0 + 1 < nb;
    const int off = b0 * 32 + (two || q < 2 ? 0 : -32);
    o.a = *(const dtl_v4i*)(asrc + off);
#pragma unroll
    for (int j = 0; j < NT; j++) o.b[j] = *(const dtl_v4i*)(bsrc[j] + off);
    const int b1 = two ? b0 + 1 : b0;
    if constexpr (EVEN) {
#pragma unroll
      for (int i = 0; i < 4; i++) o.dw[0][i] = *(const uint32_t*)(dwsrc[i] + b0);
#pragma unroll
      for (int j = 0; j < NT; j++) {
        const float2 d2 = *(const float2*)(dsrc[j] + b0);
        o.dav[0][j] = d2.x;
        o.dav[1][j] = d2.y;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        o.dw[0][i] = dwsrc[i][b0];
        o.dw[1][i] = dwsrc[i][b1];
      }
#pragma unroll
      for (int j = 0; j < NT; j++) {
        o.dav[0][j] = dsrc[j][b0];
        o.dav[1][j] = dsrc[j][b1];
      }
    }
  };
  // valid[h]: whether block 2 pr + h exists; a missing block adds +0.0f
  // terms, which leave the sums' bits unchanged (as in k_q6k_mfma).
  auto compute = [&](const Ops& o, bool valid0, bool valid1) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const bool valid = h == 0 ? valid0 : valid1;
      const dtl_v4i a = (q >> 1) == h ? o.a : zero;
      float dw[4];
#pragma unroll
      for (int i = 0; i < 4; i++)
        dw[i] = f16_to_f32((uint16_t)(EVEN ? (h == 0 ? o.dw[0][i] & 0xffffu : o.dw[0][i] >> 16) : o.dw[h][i]));
#pragma unroll
      for (int j = 0; j < NT; j++) {
        const dtl_v4i acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, o.b[j], zero, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float dd = dw[i] * o.dav[h][j];
          const float term = dd * (float)acc[i];
          sums[j][i] += valid ? term : 0.0f;
        }
      }
    }
  };
  // Block pairs in flight, refilled unconditionally as in k_q6k_mfma
  const int np = (nb + 1) / 2;
  // (four slots with one position tile per wave, two with more)
  constexpr int D = NT == 1 ? kMfmaRing : 2;
  auto last = [&](int i) { return i < np ? i : np - 1; };
  Ops r0, r1, r2, r3;
  load(r0, last(0));
  load(r1, last(1));
  if (D == 4) {
    load(r2, last(2));
    load(r3, last(3));
  }
  // the epilogue's operands (clamped positions and rows), in flight with the
  // first block pairs
  float pre[NT][4];
#pragma unroll
  for (int j = 0; j < NT; j++) {
    int pos = p0 + 16 * j + li;
    pos = pos < T ? pos : T - 1;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      int row = row0 + 4 * q + i;
      row = row < rows ? row : rows - 1;
      pre[j][i] = epilogue_operand(out, (size_t)pos * rows + row, bias, row, epi);
    }
  }
#define DTL_MFMA_STEP(r, i)                                                                \
  compute(r, (i) < np, 2 * (i) + 1 < nb);                                                  \
  __builtin_amdgcn_sched_barrier(0);                                                       \
  load(r, last((i) + D));                                                                  \
  __builtin_amdgcn_sched_barrier(0)
  for (int p0 = 0; p0 < np; p0 += D) {
    DTL_MFMA_STEP(r0, p0);
    DTL_MFMA_STEP(r1, p0 + 1);
    if (D == 4) {
      DTL_MFMA_STEP(r2, p0 + 2);
      DTL_MFMA_STEP(r3, p0 + 3);
    }
  }
#undef DTL_MFMA_STEP
  bool ok = true;
#pragma unroll
  for (int j = 0; j < NT; j++) {
    const int pos = p0 + 16 * j + li;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = row0 + 4 * q + i;
      if (row < rows && pos < T)
        ok &= store_epilogue_pre(sums[j][i], pre[j][i], out, (size_t)pos * rows + row, epi);
    }
  }
  if (!ok) flag(err, ERRBIT_NON_FINITE);
}

// int8 copy of a Q4_0 matrix in element order (nibble - 8; det-quant
// lib.rs:259-279: element i < 16 is the low nibble of byte i, element
// i + 16 its high nibble), the A operand of k_q8_mfma.
__global__ void k_q4_0_i8(DevMat W, int8_t* out) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t total = (size_t)W.rows * W.cols;
  if (idx >= total) return;
  const size_t blk = idx / 32;
  const int e = (int)(idx % 32);
  const uint8_t b = ((const uint8_t*)W.w)[blk * 16 + (e & 15)];
  out[idx] = (int8_t)((e < 16 ? (b & 15) : (b >> 4)) - 8);
}

void launch_q4_0_i8(const DevMat& W, int8_t* out, hipStream_t s) {
  const size_t total = (size_t)W.rows * W.cols;
  launch_kernel(k_q4_0_i8, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, s, W, out);
}

// ---------------------------------------------------------------------------
// launchers

namespace {
// Rows per wave: enough waves to cover every SIMD, more rows when the
// matrix is tall so the per-row decode is amortised over fewer LDS refills.
int rows_per_wave(int rows) {
  if (rows >= 8192) return 4;
  if (rows >= 4096) return 2;
  return 1;
}

// Which Q4_K chunk GEMM serves a launch.  The products on the matrix cores
// (k_q4k_mfp) own 16 x 16 (row, position) chains per wave, so a launch of
// wo / ffn_down or wq + wk at 64 positions has 512-576 waves: with other
// chunks' launches in flight (the pipelined encode) they and the gate + up
// pair (2816 waves) run there, the pipelined TinyLlama step taking 98.5 ms
// against 118.5 with k_q4k_f32m.  A launch alone on the chip
// (dtl_forward_chunk, the decode-size chunks) keeps one chain per lane of
// k_q4k_f32m for wo / ffn_down and wq + wk, 8 x 8 lanes, 2 x 2 waves over
// 16 positions x 16 rows, which fills the chip (chunk-at-a-time step: wo /
// ffn_down 39.9 ms against 58.1 on the matrix cores, wq + wk 23.1 against
// 24.9); gate + up takes the matrix cores there too (45.4 against 56.3 ms).
template <int PW, int PP, int RP, int WP, int WR, int MODE>
void launch_q4k_f32m(const Q4kF32Args& a, int rows_total, hipStream_t s) {
  constexpr int RB = WR * RP * 64 / PW, PB = WP * PW * PP;
  dim3 grid((rows_total + RB - 1) / RB, (a.T + PB - 1) / PB);
  launch_kernel(k_q4k_f32m<PW, PP, RP, WP, WR, MODE>, grid, dim3(64 * WP * WR), 0, s, a);
}

template <int MODE>
void launch_q4k_f32w(const Q4kF32Args& a, bool overlapped, hipStream_t s) {
  if (MODE == MODE_PAIR || overlapped) return launch_q4k_mfp(a, MODE, s);
  const int rows_total = MODE == MODE_CAT ? a.rows0 + a.rows1 : a.rows0;
  launch_q4k_f32m<8, 1, 1, 2, 2, MODE == MODE_CAT ? MODE_CAT : MODE_SINGLE>(a, rows_total, s);
}

Q4kF32Args q4k_args(const DevMat& W0, const DevMat* W1, const DevAct& A, int T, float* out0,
                    float* out1, float* ffo, const float* bias0, const float* bias1, int epi,
                    int* err) {
  Q4kF32Args a{};
  a.w0 = W0.w32;
  a.w1 = W1 ? W1->w32 : nullptr;
  a.rows0 = W0.rows;
  a.rows1 = W1 ? W1->rows : 0;
  a.cols = W0.cols;
  a.af = A.af;
  a.T = T;
  a.out0 = out0;
  a.out1 = out1;
  a.ffo = ffo;
  a.bias0 = bias0;
  a.bias1 = bias1;
  a.epi = epi;
  a.err = err;
  return a;
}
}  // namespace

namespace {
template <bool EVEN>
void launch_q8_mfma(const int8_t* w8, const DevMat& W, const DevAct& A, int T, float* out, const float* bias,
                    int epi, int* err, hipStream_t s) {
  const int py = (T + 63) / 64;
  if (W.rows >= 8192)
    launch_kernel((k_q8_mfma<4, EVEN>), dim3((W.rows + 63) / 64, py), dim3(256), 0, s, w8, W.d16, W.rows,
                  W.nb, A.qa, A.da, T, out, bias, epi, err);
  else if (W.rows >= 2048)
    launch_kernel((k_q8_mfma<2, EVEN>), dim3((W.rows + 31) / 32, py), dim3(256), 0, s, w8, W.d16, W.rows,
                  W.nb, A.qa, A.da, T, out, bias, epi, err);
  else
    launch_kernel((k_q8_mfma<1, EVEN>), dim3((W.rows + 15) / 16, py), dim3(256), 0, s, w8, W.d16, W.rows,
                  W.nb, A.qa, A.da, T, out, bias, epi, err);
}
}  // namespace

bool gemm_tok_supported(const DevMat& W) {
  return W.type == kGgmlQ4K || W.type == kGgmlQ6K || W.type == kGgmlQ8_0 ||
         (W.type == kGgmlQ4_0 && W.i8);
}

void launch_gemm_tok(const DevMat& W, const DevAct& A, int T, float* out, const float* bias,
                     int epi, int* err, hipStream_t s) {
  DevMat none{};
  if (W.type == kGgmlQ4K && W.w32) {
    launch_q4k_f32w<MODE_SINGLE>(
        q4k_args(W, nullptr, A, T, out, nullptr, nullptr, bias, nullptr, epi, err), A.overlapped, s);
    return;
  }
  if (W.type == kGgmlQ6K && W.planes) {
    // Matrices of 2048 rows and more: 32 positions per wave share each
    // weight-plane load; shorter ones split positions over waves to fill the
    // chip.  (The TinyLlama encode's 2048-row ffn_down: 98.5 against 99.1 ms
    // per pipelined step with 16 positions per wave, in a same-box A/B.)
    const int rt = (W.rows + 15) / 16;
    if (W.rows >= 2048) {
      launch_kernel(k_q6k_mfma<2>, dim3(rt, (T + 31) / 32), dim3(256), 0, s, W.planes, W.d16,
                    W.rows, W.nb, A.qk, A.dk, T, out, bias, epi, err);
    } else {
      launch_kernel(k_q6k_mfma<1>, dim3(rt, (T + 15) / 16), dim3(256), 0, s, W.planes, W.d16,
                    W.rows, W.nb, A.qk, A.dk, T, out, bias, epi, err);
    }
    return;
  }
  if ((W.type == kGgmlQ8_0 || (W.type == kGgmlQ4_0 && W.i8)) && T >= 16) {
    // Q8_0 / Q4_0 on the int8 matrix cores: one workgroup per 64 positions
    // and 16 (short matrices: every wave its own 16 positions), 32 or 64 rows.
    const int8_t* w8 = W.type == kGgmlQ8_0 ? (const int8_t*)W.w : W.i8;
    if (W.nb % 2 == 0)
      launch_q8_mfma<true>(w8, W, A, T, out, bias, epi, err, s);
    else
      launch_q8_mfma<false>(w8, W, A, T, out, bias, epi, err, s);
    return;
  }
  int R = rows_per_wave(W.rows);
  dim3 grid((W.rows + kWaves * R - 1) / (kWaves * R), (T + 63) / 64);
  dim3 block(kWaves * 64);
  switch (W.type) {
    case kGgmlQ4K:
      if (R == 4)
        launch_kernel((k_q4k_tok<4, false>), grid, block, 0, s, W, none, A.af, T, out, nullptr, nullptr, bias, epi, err);
      else if (R == 2)
        launch_kernel((k_q4k_tok<2, false>), grid, block, 0, s, W, none, A.af, T, out, nullptr, nullptr, bias, epi, err);
      else
        launch_kernel((k_q4k_tok<1, false>), grid, block, 0, s, W, none, A.af, T, out, nullptr, nullptr, bias, epi, err);
      break;
    case kGgmlQ6K:
      if (R == 4)
        launch_kernel((k_q6k_tok<4>), grid, block, 0, s, W, A.qk, A.dk, T, out, bias, epi, err);
      else if (R == 2)
        launch_kernel((k_q6k_tok<2>), grid, block, 0, s, W, A.qk, A.dk, T, out, bias, epi, err);
      else
        launch_kernel((k_q6k_tok<1>), grid, block, 0, s, W, A.qk, A.dk, T, out, bias, epi, err);
      break;
    default:
      if (R == 4)
        launch_kernel((k_q8_0_tok<4>), grid, block, 0, s, W, A.qa, A.da, T, out, bias, epi, err);
      else if (R == 2)
        launch_kernel((k_q8_0_tok<2>), grid, block, 0, s, W, A.qa, A.da, T, out, bias, epi, err);
      else
        launch_kernel((k_q8_0_tok<1>), grid, block, 0, s, W, A.qa, A.da, T, out, bias, epi, err);
      break;
  }
}

void launch_gemm_pair_swiglu_q4k(const DevMat& G, const DevMat& U, const DevAct& A, int T, float* g,
                                 float* u, float* ffo, int* err, hipStream_t s) {
  if (G.w32 && U.w32 && !g && !u) {
    launch_q4k_f32w<MODE_PAIR>(
        q4k_args(G, &U, A, T, nullptr, nullptr, ffo, nullptr, nullptr, EPI_STORE, err), A.overlapped, s);
    return;
  }
  int R = rows_per_wave(2 * G.rows) >= 2 ? 2 : 1;
  dim3 grid((G.rows + kWaves * R - 1) / (kWaves * R), (T + 63) / 64);
  dim3 block(kWaves * 64);
  if (R == 2)
    launch_kernel((k_q4k_tok<2, true>), grid, block, 0, s, G, U, A.af, T, g, u, ffo, nullptr, 0, err);
  else
    launch_kernel((k_q4k_tok<1, true>), grid, block, 0, s, G, U, A.af, T, g, u, ffo, nullptr, 0, err);
}

bool launch_gemm_cat_q4k(const DevMat& W0, const DevMat& W1, const DevAct& A, int T, float* out0,
                         float* out1, const float* bias0, const float* bias1, int epi, int* err,
                         hipStream_t s) {
  if (T < 16 || W0.type != kGgmlQ4K || W1.type != kGgmlQ4K || !W0.w32 || !W1.w32 ||
      W0.cols != W1.cols)
    return false;
  launch_q4k_f32w<MODE_CAT>(q4k_args(W0, &W1, A, T, out0, out1, nullptr, bias0, bias1, epi, err),
                            A.overlapped, s);
  return true;
}

}  // namespace dtl
