// Decode GEMVs: a handful of positions (single-token decode, short chunks),
// so every weight byte streams from HBM once per position and the kernels
// are shaped for memory-level parallelism rather than weight reuse.
//
//   Q8_0 / Q4_0  dot_q8_0_q8a / dot_q4_0_q8a (det-quant lib.rs:237-279):
//                the per-block integer sums are exact, so lanes compute them
//                in parallel from coalesced 16-byte loads (int8 dot4); the
//                per-block f32 terms (dw*da)*isum land in LDS and one lane
//                per row adds them in block order.
//   Q6_K         dot_q6_k_q8k (lib.rs:353-397): one lane per (row,
//                superblock) forms the eight exact class sums of its
//                superblock; one lane per row then runs the per-superblock
//                f32 chain sums[l] += (dw*da)*aux[l] and the final combine.
//   Q4_K         dot_q4_k_q8a (lib.rs:281-315) is one serial f32 chain per
//                row: one lane per row walks the exact f32 weights (the
//                values q4_k_value yields) with the activations as scalar
//                operands.  Its time is bounded by the chain length (cols
//                dependent adds), not by HBM.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dtl_device.h"
#include "dtl_numerics.h"
#include "dtl_quant.h"

namespace dtl {

namespace {

// Q4_K 6-bit scale and min of sub-block j (det-quant lib.rs:519-529) from
// the 12 packed bytes held as three little-endian words; the words are
// selected, not indexed, so that they stay in registers.
__device__ __forceinline__ void q4k_scale_min3(uint32_t s0, uint32_t s1, uint32_t s2, int j, int* sc,
                                               int* mn) {
  auto byte = [&](int i) -> uint32_t {
    const uint32_t w = i < 4 ? s0 : (i < 8 ? s1 : s2);
    return (w >> (8 * (i & 3))) & 0xffu;
  };
  if (j < 4) {
    *sc = (int)(byte(j) & 0x3f);
    *mn = (int)(byte(j + 4) & 0x3f);
  } else {
    *sc = (int)((byte(j + 4) & 0x0f) | ((byte(j - 4) >> 6) << 4));
    *mn = (int)((byte(j + 4) >> 4) | ((byte(j) >> 6) << 4));
  }
}

constexpr int kGgmlQ4_0 = 2, kGgmlQ8_0 = 8, kGgmlQ4K = 12, kGgmlQ6K = 14;

__device__ __forceinline__ void flag(int* err, int bit) { atomicOr(err, bit); }

// add_optional_bias / residual_add (det-model lib.rs:1967-1998) on a finished dot.
__device__ __forceinline__ bool epilogue(float v, float* out, size_t o, const float* bias, int r,
                                         int epi) {
  bool ok = finite(v);
  if (epi == EPI_BIAS) v = v + bias[r];
  else if (epi == EPI_RESIDUAL) v = out[o] + v;
  out[o] = v;
  return ok && finite(v);
}

// The value the epilogue adds (bias[r], or the residual out[o]), read without
// a branch so that a kernel can load it at its start: read at the end it put
// a round trip after the last chain.  With EPI_STORE the read (of out[o])
// goes unused.
__device__ __forceinline__ float epilogue_operand(const float* out, size_t o, const float* bias, int r,
                                                  int epi) {
  return *(epi == EPI_BIAS ? bias + r : out + o);
}

__device__ __forceinline__ bool epilogue_pre(float v, float pre, float* out, size_t o, int epi) {
  bool ok = finite(v);
  if (epi == EPI_BIAS) v = v + pre;
  else if (epi == EPI_RESIDUAL) v = pre + v;
  out[o] = v;
  return ok && finite(v);
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Sequential sum of n block terms (block order), from LDS.
// Block-term rows in LDS start on 16-byte boundaries (chain_sum_lds reads
// them four at a time): row stride nb rounded up to a multiple of 4.
__host__ __device__ inline int nb_stride(int nb) { return (nb + 3) & ~3; }

// A 16-byte load marked non-temporal (streamed once, not kept in the caches).
typedef unsigned int dtl_v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_nt16(const void* p) {
  const dtl_v4u v = __builtin_nontemporal_load(reinterpret_cast<const dtl_v4u*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Byte B of x as f32 (exact), one v_cvt_f32_ubyteB: written out because the
// compiler turns (x >> 8 B) & 0xff of a nibble-masked dword into a bit-field
// extract and a conversion of byte 0.
template <int B>
__device__ __forceinline__ float ubyte_f32(uint32_t x) {
  float f;
  if (B == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f) : "v"(x));
  else if (B == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f) : "v"(x));
  else if (B == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f) : "v"(x));
  else asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f) : "v"(x));
  return f;
}
}  // namespace

// ---------------------------------------------------------------------------
// Q8_0 / Q4_0.  Four waves per workgroup, R rows per wave.  Dynamic LDS:
// float[4][R][nb] block terms.
template <int TYPE, int R>
__global__ void __launch_bounds__(256) k_gemv_q8(DevMat W, const int8_t* __restrict__ qa,
                                                 const float* __restrict__ da, float* out,
                                                 const float* bias, int epi, int* err) {
  extern __shared__ __align__(16) float vb[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.y;
  const int rows = W.rows, cols = W.cols, nb = W.nb;
  const int row0 = (blockIdx.x * 4 + wave) * R;
  const int nbs = nb_stride(nb);
  float* mine = vb + (size_t)wave * R * nbs;
  const int8_t* arow = qa + (size_t)t * cols;
  const float* drow = da + (size_t)t * nb;
  // the epilogue operand of this lane's row (lanes below R), loaded first
  int prow = row0 + (lane < R ? lane : 0);
  prow = prow < rows ? prow : rows - 1;
  const float pre = epilogue_operand(out, (size_t)t * rows + prow, bias, prow, epi);
  // Q8_0: a 32-byte block is two 16-byte chunks (lanes c, c^1); Q4_0: one
  // 16-byte block of nibbles per lane.  A pass covers 64 chunks.
  const int nchunk = TYPE == kGgmlQ8_0 ? 2 * nb : nb;
  struct Pass {
    uint4 w4[R];
    uint32_t dsc[R];  // 32-bit: packed two to a register, a pair is waited for when loaded
    uint4 a0, a1;
    float dact;
  };
  // Every load of a pass (R weight chunks, their block scales, the
  // activation and its scale) is issued before any of its arithmetic, and
  // unconditionally: lanes past the row's chunks read its last chunk and
  // store nothing (a load under a branch is waited for before the next one).
  auto load = [&](Pass& P, int c0) __attribute__((always_inline)) {
    const int c = c0 + lane;
    const int cl = c < nchunk ? c : nchunk - 1;
    const int b = TYPE == kGgmlQ8_0 ? cl >> 1 : cl;
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int row = row0 + r < rows ? row0 + r : rows - 1;
      if (TYPE == kGgmlQ8_0)
        P.w4[r] = *(const uint4*)((const int8_t*)W.w + (size_t)row * cols + (size_t)cl * 16);
      else
        P.w4[r] = *(const uint4*)((const uint8_t*)W.w + ((size_t)row * nb + cl) * 16);
      P.dsc[r] = W.d16[(size_t)row * nb + b];
    }
    if (TYPE == kGgmlQ8_0) {
      P.a0 = *(const uint4*)(arow + (size_t)cl * 16);
      P.a1 = make_uint4(0, 0, 0, 0);
    } else {
      P.a0 = *(const uint4*)(arow + (size_t)cl * 32);
      P.a1 = *(const uint4*)(arow + (size_t)cl * 32 + 16);
    }
    P.dact = drow[b];
  };
  auto reduce = [&](const Pass& P, int c0) __attribute__((always_inline)) {
    const int c = c0 + lane;
    const bool cv = c < nchunk;
    const int b = TYPE == kGgmlQ8_0 ? c >> 1 : c;
    int asum = 0;
    if (TYPE != kGgmlQ8_0) {
      // Q4_0 nibbles are offset by 8: isum = sum(lo*a) + sum(hi*a') - 8*sum(a).
      const uint32_t ones = 0x01010101u;
      asum = dot4(ones, P.a0.x, asum);
      asum = dot4(ones, P.a0.y, asum);
      asum = dot4(ones, P.a0.z, asum);
      asum = dot4(ones, P.a0.w, asum);
      asum = dot4(ones, P.a1.x, asum);
      asum = dot4(ones, P.a1.y, asum);
      asum = dot4(ones, P.a1.z, asum);
      asum = dot4(ones, P.a1.w, asum);
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
      int isum = 0;
      if (TYPE == kGgmlQ8_0) {
        isum = dot4(P.w4[r].x, P.a0.x, isum);
        isum = dot4(P.w4[r].y, P.a0.y, isum);
        isum = dot4(P.w4[r].z, P.a0.z, isum);
        isum = dot4(P.w4[r].w, P.a0.w, isum);
        isum += dpp_i32<kDppXor1>(isum);
      } else {
        const uint32_t m = 0x0f0f0f0fu;
        isum = dot4(P.w4[r].x & m, P.a0.x, isum);
        isum = dot4(P.w4[r].y & m, P.a0.y, isum);
        isum = dot4(P.w4[r].z & m, P.a0.z, isum);
        isum = dot4(P.w4[r].w & m, P.a0.w, isum);
        isum = dot4((P.w4[r].x >> 4) & m, P.a1.x, isum);
        isum = dot4((P.w4[r].y >> 4) & m, P.a1.y, isum);
        isum = dot4((P.w4[r].z >> 4) & m, P.a1.z, isum);
        isum = dot4((P.w4[r].w >> 4) & m, P.a1.w, isum);
        isum -= 8 * asum;
      }
      const bool writer = TYPE == kGgmlQ8_0 ? cv && !(c & 1) : cv;
      if (writer && row0 + r < rows) mine[r * nbs + b] = (f16_to_f32((uint16_t)P.dsc[r]) * P.dact) * (float)isum;
    }
  };
  // Rows of up to kPre passes (8192 Q8_0 columns) with few rows per wave:
  // all passes' loads go out before the first pass's arithmetic.
  constexpr int kPre = R <= 2 ? 8 : 1;
  const int npass = (nchunk + 63) / 64;
  if (kPre > 1 && npass <= kPre) {
    Pass P[kPre];
    // passes past npass reload pass 0 (unconditional loads) and are not reduced
#pragma unroll
    for (int p = 0; p < kPre; p++) load(P[p], p < npass ? 64 * p : 0);
#pragma unroll
    for (int p = 0; p < kPre; p++)
      if (p < npass) reduce(P[p], 64 * p);
  } else {
    for (int c0 = 0; c0 < nchunk; c0 += 64) {
      Pass P;
      load(P, c0);
      reduce(P, c0);
    }
  }
  __syncthreads();
  if (lane < R) {
    const int row = row0 + lane;
    if (row < rows) {
      float v = chain_sum_lds(0.0f, mine + lane * nbs, nb);
      if (!epilogue_pre(v, pre, out, (size_t)t * rows + row, epi)) flag(err, ERRBIT_NON_FINITE);
    }
  }
}

// ---------------------------------------------------------------------------
// Q8_0 streaming variant for tall matrices with at most 1024 columns (the
// output projection of the small-vocabulary-heavy shapes): every wave walks
// groups of R rows in a grid-stride loop with two groups' weights and scales
// in flight, refilling a slot as soon as its group is reduced.  Lane c owns
// 16-byte chunk c of every row (nchunk <= 64), so the activation chunk is
// loaded once per wave.  Every load is unconditional (lanes past the row's
// chunks and groups past the end read valid addresses whose values are not
// stored): a load under a branch makes the compiler wait for every load in
// flight at the branch, which took the prefetch away.  The weight loads are
// non-temporal (the matrix is read once per position and is larger than the
// last-level cache), and the rows' chains use the short ring of
// chain_sum_lds32: with four rows per group (and the waves-per-SIMD hint,
// without which the epilogue's registers tip it to 73) that leaves 68
// registers and seven waves per SIMD (the 145 MB Qwen2.5 output projection: 26.7 us per
// launch by events, against 30.5 with eight rows, the general chain and
// cached loads).
template <int R>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(7))) k_gemv_q8_0_stream(DevMat W, const int8_t* __restrict__ qa,
                                                          const float* __restrict__ da, float* out,
                                                          const float* bias, int epi, int* err) {
  extern __shared__ __align__(16) float vb[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.y;
  const int rows = W.rows, cols = W.cols, nb = W.nb;
  const int nchunk = 2 * nb;
  const int c = lane, b = c >> 1;
  const bool cv = c < nchunk;
  const int cc = cv ? c : 0, bc = cv ? b : 0;  // clamped chunk and block of this lane
  const int nbs = nb_stride(nb);
  float* mine = vb + (size_t)wave * R * nbs;
  const int ngroups = (rows + R - 1) / R;
  const int stride = gridDim.x * 4;
  int g = blockIdx.x * 4 + wave;
  if (g >= ngroups) return;
  const uint4 a0 = *(const uint4*)(qa + (size_t)t * cols + (size_t)cc * 16);
  const float dact = da[(size_t)t * nb + bc];
  const int8_t* wbase = (const int8_t*)W.w + (size_t)cc * 16;
  const uint16_t* dbase = W.d16 + bc;
  uint4 w0[R], w1[R];
  // scales as 32-bit values: packed two to a register, each pair would be
  // waited for right after its loads are issued
  uint32_t s0[R], s1[R];
  // group gg's rows, the group clamped to the last one
#define DTL_STREAM_LOAD(WV, SV, GG)                                        \
  do {                                                                    \
    const int gc_ = (GG) < ngroups ? (GG) : ngroups - 1;                  \
    _Pragma("unroll") for (int r = 0; r < R; r++) {                       \
      int row = gc_ * R + r;                                              \
      row = row < rows ? row : rows - 1;                                  \
      WV[r] = load_nt16(wbase + (size_t)row * cols);                      \
      SV[r] = dbase[(size_t)row * nb];                                    \
    }                                                                     \
  } while (0)
#define DTL_STREAM_REDUCE(WV, SV, GG)                                                           \
  do {                                                                                         \
    _Pragma("unroll") for (int r = 0; r < R; r++) {                                            \
      int isum = 0;                                                                            \
      isum = dot4(WV[r].x, a0.x, isum);                                                         \
      isum = dot4(WV[r].y, a0.y, isum);                                                         \
      isum = dot4(WV[r].z, a0.z, isum);                                                         \
      isum = dot4(WV[r].w, a0.w, isum);                                                         \
      isum += dpp_i32<kDppXor1>(isum); /* lane c^1's half block, by DPP */                     \
      if (cv && !(c & 1)) mine[r * nbs + b] = (f16_to_f32((uint16_t)SV[r]) * dact) * (float)isum;        \
    }                                                                                          \
    __builtin_amdgcn_wave_barrier();                                                           \
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");                                     \
    if (lane < R) {                                                                            \
      const int row = (GG) * R + lane;                                                         \
      if (row < rows) {                                                                        \
        float v = chain_sum_lds32(0.0f, mine + lane * nbs, nb);                                  \
        if (!epilogue(v, out, (size_t)t * rows + row, bias, row, epi)) flag(err, ERRBIT_NON_FINITE); \
      }                                                                                        \
    }                                                                                          \
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");                                     \
    __builtin_amdgcn_wave_barrier();                                                           \
  } while (0)
  DTL_STREAM_LOAD(w0, s0, g);
  DTL_STREAM_LOAD(w1, s1, g + stride);
  for (;;) {
    DTL_STREAM_REDUCE(w0, s0, g);
    __builtin_amdgcn_sched_barrier(0);
    DTL_STREAM_LOAD(w0, s0, g + 2 * stride);
    __builtin_amdgcn_sched_barrier(0);
    g += stride;
    if (g >= ngroups) break;
    DTL_STREAM_REDUCE(w1, s1, g);
    __builtin_amdgcn_sched_barrier(0);
    DTL_STREAM_LOAD(w1, s1, g + 2 * stride);
    __builtin_amdgcn_sched_barrier(0);
    g += stride;
    if (g >= ngroups) break;
  }
#undef DTL_STREAM_LOAD
#undef DTL_STREAM_REDUCE
}

// ---------------------------------------------------------------------------
// Q6_K.  One wave per workgroup; lane = (row_local, superblock) with
// rpw = 64 / nsb rows per wave.  Q8_K activations are class-major inside each
// 256-block (element e at (e % 8) * 32 + e / 8).
__global__ void __launch_bounds__(64) k_gemv_q6k(DevMat W, const int8_t* __restrict__ qk,
                                                 const float* __restrict__ dk, float* out,
                                                 const float* bias, int epi, int* err) {
  __shared__ int aux_s[64][9];
  __shared__ float d_s[64];
  const int lane = threadIdx.x;
  const int t = blockIdx.y;
  const int rows = W.rows, cols = W.cols, nsb = W.nb;
  const int rpw = 64 / nsb;
  const int rl = lane / nsb, sb = lane % nsb;
  const int row = blockIdx.x * rpw + rl;
  const bool active = rl < rpw && row < rows;
  // Every load (both halves of the superblock, its activations and both
  // scales) is issued before any arithmetic; inactive lanes read row 0.
  const int lrow = active ? row : 0, lsb = active ? sb : 0;
  const uint32_t* body =
      (const uint32_t*)((const uint8_t*)W.w + ((size_t)lrow * nsb + lsb) * 208);
  const uint32_t* act = (const uint32_t*)(qk + (size_t)t * cols + (size_t)lsb * 256);
  uint32_t ql[2][16], qh[2][8], sc[2][2], a[2][8][4];
#pragma unroll
  for (int h = 0; h < 2; h++) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      uint4 v = ((const uint4*)(body + 16 * h))[i];
      ql[h][4 * i] = v.x;
      ql[h][4 * i + 1] = v.y;
      ql[h][4 * i + 2] = v.z;
      ql[h][4 * i + 3] = v.w;
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
      uint4 v = ((const uint4*)(body + 32 + 8 * h))[i];
      qh[h][4 * i] = v.x;
      qh[h][4 * i + 1] = v.y;
      qh[h][4 * i + 2] = v.z;
      qh[h][4 * i + 3] = v.w;
    }
    sc[h][0] = body[48 + 2 * h];
    sc[h][1] = body[48 + 2 * h + 1];
    // class k, half h: elements e = 128h + 8j + k for j in 0..15 sit at
    // bytes 32k + 16h .. +15 of the block; dword p holds l0 = k + 8i, i = 0..3
    // of part p.
#pragma unroll
    for (int k = 0; k < 8; k++) {
      uint4 v = *(const uint4*)(act + 8 * k + 4 * h);
      a[h][k][0] = v.x;
      a[h][k][1] = v.y;
      a[h][k][2] = v.z;
      a[h][k][3] = v.w;
    }
  }
  const uint16_t dw = W.d16[(size_t)lrow * nsb + lsb];
  const float da = dk[(size_t)t * nsb + lsb];
  int aux[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int h = 0; h < 2; h++) {
#pragma unroll
    for (int k = 0; k < 8; k++) {
      int acc = 0;
#pragma unroll
      for (int p = 0; p < 4; p++) {
#pragma unroll
        for (int pair = 0; pair < 2; pair++) {
          // scale index 8h + l0/16 + 2p (l0 = k + 8i: i = 0,1 -> 0; 2,3 -> 1)
          const int si = pair + 2 * p;
          const int scale = (int)(int8_t)((sc[h][si >> 2] >> (8 * (si & 3))) & 0xffu);
          int s = 0;
#pragma unroll
          for (int ii = 0; ii < 2; ii++) {
            const int i = 2 * pair + ii;
            const int l0 = k + 8 * i;
            const int qlb = l0 + 32 * (p & 1);
            const uint32_t lo = (ql[h][qlb >> 2] >> (8 * (qlb & 3) + 4 * (p >> 1))) & 0x0fu;
            const uint32_t hi = (qh[h][l0 >> 2] >> (8 * (l0 & 3) + 2 * p)) & 0x03u;
            const int q6 = (int)(lo | (hi << 4)) - 32;
            const int av = (int)(int8_t)((a[h][k][p] >> (8 * i)) & 0xffu);
            s += q6 * av;
          }
          acc += scale * s;
        }
      }
      aux[k] += acc;
    }
  }
#pragma unroll
  for (int k = 0; k < 8; k++) aux_s[lane][k] = aux[k];
  d_s[lane] = f16_to_f32(dw) * da;
  __syncthreads();
  if (lane < rpw && (int)blockIdx.x * rpw + lane < rows) {
    const int r = blockIdx.x * rpw + lane;
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int b = 0; b < nsb; b++) {
      const float d = d_s[lane * nsb + b];
      const int* ax = aux_s[lane * nsb + b];
#pragma unroll
      for (int l = 0; l < 8; l++) sums[l] += d * (float)ax[l];
    }
    float v = 0.0f;
#pragma unroll
    for (int l = 0; l < 8; l++) v += sums[l];
    if (!epilogue(v, out, (size_t)t * rows + r, bias, r, epi)) flag(err, ERRBIT_NON_FINITE);
  }
}

// ---------------------------------------------------------------------------
// Q6_K decode layout (see q6k_decode_layout_applies): one thread per
// (superblock, class) of the padded groups writes its class's low nibbles and
// high bit pairs; class 0 also writes the scales.  Quant q6u of element e
// decoded as q6_k_quant does (det-quant lib.rs:537-556); its bit 5 is stored
// flipped (q6u ^ 32), so that the kernel's byte with the six bits at the top
// is the signed 4 (q6u - 32).
__global__ void k_q6k_decode_layout(DevMat W, uint32_t* out, int groups) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  const int c = i & 7, s = (i >> 3) & 15, g = i >> 7;
  if (g >= groups) return;
  const int nb = W.nb, rpg = 16 / nb;
  const int row = g * rpg + s / nb, sb = s % nb;
  const int p = c >> 1, ci = c & 1;
  uint32_t* grp = out + (size_t)g * kQ6dGroupWords * 4;  // dwords
  uint32_t lo[4] = {0, 0, 0, 0}, hi[2] = {0, 0}, sc[4] = {0, 0, 0, 0};
  if (row < W.rows) {
    const uint8_t* body = (const uint8_t*)W.w + ((size_t)row * nb + sb) * 208;
    for (int j = 0; j < 32; j++) {
      const int e = c + 8 * j, half = e / 128, within = e % 128, l = within % 32, part = within / 32;
      const uint8_t qlb = body[64 * half + l + 32 * (part & 1)];
      const uint32_t nib = (part >> 1) ? (qlb >> 4) : (qlb & 0x0fu);
      // the high pair with its top bit (bit 5 of q) flipped: the kernel's
      // byte (q ^ 0x20) << 2 is then the signed value 4 (q - 32)
      const uint32_t h2 = ((body[128 + 32 * half + l] >> (2 * part)) & 0x03u) ^ 0x02u;
      lo[j >> 3] |= nib << (8 * (j & 3) + 4 * ((j >> 2) & 1));
      hi[j >> 4] |= h2 << (8 * (j & 3) + 2 * ((j >> 2) & 3));
    }
    for (int k = 0; k < 16; k++) sc[k >> 2] |= (uint32_t)body[192 + k] << (8 * (k & 3));
  }
  uint32_t* lw = grp + (size_t)(ci * 64 + s * 4 + p) * 4;
  for (int k = 0; k < 4; k++) lw[k] = lo[k];
  uint32_t* hw = grp + (size_t)(2 * 64 + s * 4 + p) * 4 + 2 * ci;
  hw[0] = hi[0];
  hw[1] = hi[1];
  if (c == 0) {
    uint32_t* sw = grp + (size_t)(192 + s) * 4;
    for (int k = 0; k < 4; k++) sw[k] = sc[k];
  }
}

void launch_q6k_decode_layout(const DevMat& W, uint4* out, hipStream_t s) {
  const int rpg = 16 / W.nb, groups = (W.rows + rpg - 1) / rpg;
  const int threads = groups * 128;
  launch_kernel(k_q6k_decode_layout, dim3((threads + 255) / 256), dim3(256), 0, s, W, (uint32_t*)out, groups);
}

// dot_q6_k_q8k (det-quant lib.rs:353-397) over the decode layout, for tall
// matrices (the output projection).  Lane (s, p) = (lane / 4, lane % 4) of a
// wave owns class pair p of superblock s of the wave's 16-superblock group
// (one group per wave, every group its own wave: a resident grid walking
// groups in a loop streamed slower here, 12.2 against 11.4 us on the
// 32000 x 2048 TinyLlama output, since its activation operands held in
// registers left four waves per SIMD where this kernel has eight).  The
// group's four words are loaded non-temporally (read once per position).
// For elements j = 4m .. 4m + 3 of a class, the quant bytes are built with
// the six bits at the top, the stored bit 5 flipped: the signed byte
// 4 (q - 32).  The activation dword is masked to its first and second halves
// (the two scales j >> 1 = 2m, 2m + 1), and dot4(quants, half) =
// 4 sum (q - 32) * a, times the half's scale, exact in 32 bits; the class
// sum is that total shifted right by two (exact: a multiple of four).  Each lane forms d * aux[c]
// (d = w.d * a.d) for its two classes; then one lane per (row, class) runs
// sums[c] += ... over the row's superblocks in order, and one lane per row
// the final sum of sums[0..7], as the reference does.
template <int NB>
__global__ void __launch_bounds__(256) k_gemv_q6k_cm(const uint4* __restrict__ q6d,
                                                     const uint16_t* __restrict__ d16, int rows,
                                                     const int8_t* __restrict__ qk,
                                                     const float* __restrict__ dk, float* out,
                                                     const float* bias, int epi, int* err) {
  constexpr int RPG = 16 / NB;
  __shared__ float terms[4][16][9];
  __shared__ float sums_s[4][RPG][8];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.y;
  const int s = lane >> 2, p = lane & 3, sb = s % NB;
  const int ngroups = (rows + RPG - 1) / RPG;
  const int g = blockIdx.x * 4 + wave;
  if (g >= ngroups) return;
  const uint4* gp = q6d + (size_t)g * kQ6dGroupWords;
  const uint4 l0 = load_nt16(gp + lane), l1 = load_nt16(gp + 64 + lane), hw = load_nt16(gp + 128 + lane),
              sw = load_nt16(gp + 192 + s);
  int row = g * RPG + s / NB;
  row = row < rows ? row : rows - 1;
  const uint16_t dw = d16[(size_t)row * NB + sb];
  // the Q8_K activations of classes 2p, 2p + 1 of superblock column sb
  uint4 av[4];
  {
    const uint4* ap = (const uint4*)(qk + (size_t)t * NB * 256 + (size_t)sb * 256 + p * 64);
#pragma unroll
    for (int k = 0; k < 4; k++) av[k] = ap[k];
  }
  const float d = f16_to_f32(dw) * dk[(size_t)t * NB + sb];
  float(*mine)[9] = terms[wave];
  const uint32_t scw[4] = {sw.x, sw.y, sw.z, sw.w};
#pragma unroll
  for (int ci = 0; ci < 2; ci++) {
    const uint4 lw4 = ci ? l1 : l0;
    const uint32_t L[4] = {lw4.x, lw4.y, lw4.z, lw4.w};
    const uint32_t H[2] = {ci ? hw.z : hw.x, ci ? hw.w : hw.y};
    const uint32_t A[8] = {av[2 * ci].x,     av[2 * ci].y,     av[2 * ci].z,     av[2 * ci].w,
                           av[2 * ci + 1].x, av[2 * ci + 1].y, av[2 * ci + 1].z, av[2 * ci + 1].w};
    int acc = 0;  // four times the class sum
#pragma unroll
    for (int m = 0; m < 8; m++) {
      const uint32_t lw = (m & 1) ? L[m >> 1] >> 2 : L[m >> 1] << 2;
      const uint32_t h = H[m >> 2];
      const uint32_t hs = (m & 3) == 0 ? h << 6 : (m & 3) == 1 ? h << 4 : (m & 3) == 2 ? h << 2 : h;
      const uint32_t q = (hs & 0xc0c0c0c0u) | (lw & 0x3c3c3c3cu);
      const uint32_t a0 = A[m] & 0x0000ffffu, a1 = A[m] & 0xffff0000u;
      const int c0 = dot4(q, a0, 0);
      const int c1 = dot4(q, a1, 0);
      const int s0 = (int)(int8_t)((scw[m >> 1] >> (16 * (m & 1))) & 0xffu);
      const int s1 = (int)(int8_t)((scw[m >> 1] >> (16 * (m & 1) + 8)) & 0xffu);
      acc += __mul24(s0, c0) + __mul24(s1, c1);
    }
    mine[s][2 * p + ci] = d * (float)(acc >> 2);
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  for (int rc = lane; rc < 8 * RPG; rc += 64) {  // (row, class) pairs: 128 when NB = 1
    const int rl = rc >> 3, c = rc & 7;
    float sm = 0.0f;
#pragma unroll
    for (int b = 0; b < NB; b++) sm += mine[rl * NB + b][c];
    sums_s[wave][rl][c] = sm;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  if (lane < RPG) {
    const int r = g * RPG + lane;
    if (r < rows) {
      float v = 0.0f;
#pragma unroll
      for (int c = 0; c < 8; c++) v += sums_s[wave][lane][c];
      if (!epilogue(v, out, (size_t)t * rows + r, bias, r, epi)) flag(err, ERRBIT_NON_FINITE);
    }
  }
}

template <int NB>
void launch_q6k_cm_nb(const DevMat& W, const DevAct& A, int T, float* out, const float* bias, int epi,
                      int* err, hipStream_t s) {
  const int ngroups = (W.rows + 16 / NB - 1) / (16 / NB);
  launch_kernel(k_gemv_q6k_cm<NB>, dim3((ngroups + 3) / 4, T), dim3(256), 0, s, W.q6d, W.d16, W.rows, A.qk,
                A.dk, out, bias, epi, err);
}

void launch_q6k_cm(const DevMat& W, const DevAct& A, int T, float* out, const float* bias, int epi, int* err,
                   hipStream_t s) {
  switch (W.nb) {
    case 1: launch_q6k_cm_nb<1>(W, A, T, out, bias, epi, err, s); break;
    case 2: launch_q6k_cm_nb<2>(W, A, T, out, bias, epi, err, s); break;
    case 4: launch_q6k_cm_nb<4>(W, A, T, out, bias, epi, err, s); break;
    case 8: launch_q6k_cm_nb<8>(W, A, T, out, bias, epi, err, s); break;
    default: launch_q6k_cm_nb<16>(W, A, T, out, bias, epi, err, s); break;
  }
}

// Q6_K with each superblock split over eight lanes: one row per workgroup
// of 8 * nsb lanes (rounded up to whole waves), lane = (superblock sb, half
// h, part pp) as in the fused wv rows of k_gemv_q4k_pc.  A lane forms its
// share (32 elements) of the eight exact class sums, the eight lanes of a
// superblock add theirs (integers: any order), and thread 0 runs the
// per-superblock f32 chain and the final combine as k_gemv_q6k does.  A
// lane thus does an eighth of k_gemv_q6k's per-lane unpacking.
__global__ void __launch_bounds__(256) k_gemv_q6k_split(DevMat W, const int8_t* __restrict__ qk,
                                                       const float* __restrict__ dk, float* out,
                                                       const float* bias, int epi, int* err) {
  __shared__ int aux_s[32][8];
  __shared__ float d_s[32];
  const int tid = threadIdx.x, lane = tid & 63;
  const int t = blockIdx.y, r = blockIdx.x;
  const int rows = W.rows, cols = W.cols, nsb = W.nb;
  const int sb = tid >> 3, h = (tid >> 2) & 1, pp = tid & 3;
  const int sbl = sb < nsb ? sb : 0;
  const uint32_t* body = (const uint32_t*)((const uint8_t*)W.w + ((size_t)r * nsb + sbl) * 208);
  const uint4 qa4 = reinterpret_cast<const uint4*>(body + 16 * h + 8 * (pp & 1))[0];
  const uint4 qb4 = reinterpret_cast<const uint4*>(body + 16 * h + 8 * (pp & 1))[1];
  const uint4 ha4 = reinterpret_cast<const uint4*>(body + 32 + 8 * h)[0];
  const uint4 hb4 = reinterpret_cast<const uint4*>(body + 32 + 8 * h)[1];
  const uint32_t scw = body[48 + 2 * h + (pp >> 1)];
  const uint32_t* act = (const uint32_t*)(qk + (size_t)t * cols + (size_t)sbl * 256);
  uint32_t aw[8];
#pragma unroll
  for (int k = 0; k < 8; k++) aw[k] = act[8 * k + 4 * h + pp];
  const uint16_t dw = W.d16[(size_t)r * nsb + sbl];
  const float da = dk[(size_t)t * nsb + sbl];
  // the epilogue operand (thread 0 stores the row), loaded with the weights
  const float pre = epilogue_operand(out, (size_t)t * rows + r, bias, r, epi);
  const uint32_t qlw[8] = {qa4.x, qa4.y, qa4.z, qa4.w, qb4.x, qb4.y, qb4.z, qb4.w};
  const uint32_t qhw[8] = {ha4.x, ha4.y, ha4.z, ha4.w, hb4.x, hb4.y, hb4.z, hb4.w};
  int aux[8];
#pragma unroll
  for (int k = 0; k < 8; k++) {
    int acc = 0;
#pragma unroll
    for (int pair = 0; pair < 2; pair++) {
      const int scale = (int)(int8_t)((scw >> (8 * (pair + 2 * (pp & 1)))) & 0xffu);
      int sum = 0;
#pragma unroll
      for (int ii = 0; ii < 2; ii++) {
        const int i = 2 * pair + ii;
        const int l0 = k + 8 * i;
        const uint32_t lo = (qlw[l0 >> 2] >> (8 * (l0 & 3) + 4 * (pp >> 1))) & 0x0fu;
        const uint32_t hi = (qhw[l0 >> 2] >> (8 * (l0 & 3) + 2 * pp)) & 0x03u;
        const int q6 = (int)(lo | (hi << 4)) - 32;
        const int av = (int)(int8_t)((aw[k] >> (8 * i)) & 0xffu);
        sum += q6 * av;
      }
      acc += scale * sum;
    }
    aux[k] = acc;
  }
#pragma unroll
  for (int k = 0; k < 8; k++) {
    // the eight lanes of the superblock, by DPP: quads, then the other quad
    aux[k] += dpp_i32<kDppXor1>(aux[k]);
    aux[k] += dpp_i32<kDppXor2>(aux[k]);
    aux[k] += dpp_i32<kDppMirror8>(aux[k]);
  }
  if ((lane & 7) == 0 && sb < nsb) {
#pragma unroll
    for (int k = 0; k < 8; k++) aux_s[sb][k] = aux[k];
    d_s[sb] = f16_to_f32(dw) * da;
  }
  __syncthreads();
  if (tid == 0) {
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int b = 0; b < nsb; b++) {
      const float d = d_s[b];
#pragma unroll
      for (int l = 0; l < 8; l++) sums[l] += d * (float)aux_s[b][l];
    }
    float v = 0.0f;
#pragma unroll
    for (int l = 0; l < 8; l++) v += sums[l];
    if (!epilogue_pre(v, pre, out, (size_t)t * rows + r, epi)) flag(err, ERRBIT_NON_FINITE);
  }
}

// ---------------------------------------------------------------------------
// Q4_K from the exact f32 weights.  One wave per workgroup, RL rows (lanes)
// per wave so that the short-lived chains spread over many CUs; the
// activation addresses are wave-uniform (scalar loads).  Each lane keeps an
// eight-deep ring of 16-element weight chunks in flight (cols is a multiple
// of 256, one ring turn), so HBM latency overlaps the serial chain.
template <int RL>
__global__ void __launch_bounds__(64) k_gemv_q4k(const float* __restrict__ w32, int rows, int cols,
                                                 const float* __restrict__ af, float* out,
                                                 const float* bias, int epi, int* err) {
  constexpr int CH = 16, D = 8;
  const int lane = threadIdx.x;
  const int t = blockIdx.y;
  const int row = blockIdx.x * RL + lane;
  if (lane >= RL || row >= rows) return;
  const float* wr = w32 + (size_t)row * cols;
  const float* a = af + (size_t)t * cols;
  float4 ring[D][CH / 4];
#pragma unroll
  for (int c = 0; c < D - 1; c++)
#pragma unroll
    for (int i = 0; i < CH / 4; i++) ring[c][i] = *(const float4*)(wr + c * CH + 4 * i);
  const int last = cols - CH;  // clamp for prefetches past the row end
  float sum = 0.0f;
  for (int base = 0; base < cols; base += D * CH) {
#pragma unroll
    for (int k = 0; k < D; k++) {
      int ep = base + (k + D - 1) * CH;
      ep = ep < last ? ep : last;
#pragma unroll
      for (int i = 0; i < CH / 4; i++) ring[(k + D - 1) % D][i] = *(const float4*)(wr + ep + 4 * i);
      const int e = base + k * CH;
#pragma unroll
      for (int i = 0; i < CH / 4; i++) {
        const float4 w = ring[k][i];
        sum += w.x * a[e + 4 * i];
        sum += w.y * a[e + 4 * i + 1];
        sum += w.z * a[e + 4 * i + 2];
        sum += w.w * a[e + 4 * i + 3];
      }
    }
  }
  if (!epilogue(sum, out, (size_t)t * rows + row, bias, row, epi)) flag(err, ERRBIT_NON_FINITE);
}

// ---------------------------------------------------------------------------
// Fused decode GEMV for Q8_0 / Q4_0 weights.  Every workgroup first forms
// the Q8A activations of its position in LDS from the f32 input: after
// rmsnorm (det-model lib.rs:2053-2073: ss = sum_squares_f32_ref(x), r =
// 1 / sqrt(ss / n + eps), y = (x * r) * w) when a norm weight is given,
// else straight from x (the re-quantisation of wo / down inputs,
// lib.rs:1310-1316, 1366-1372).  The weight loads of the first chunk
// column are issued before that prologue.  The matrices of one launch share
// the input: either concatenated rows (q, k, v: up to three outputs with
// their own bias / epilogue) or two matrices over the same rows whose dots
// finish as swiglu (gate, up: out = silu(g) * u, lib.rs:2420-2434).  Every
// value is computed exactly as by the separate launches.
namespace {

// Float4s per thread (norm pass) or 256-element spans per wave (plain
// pass) loaded at once: inputs of up to 4096 elements take one round trip
// (with 4 waves; one batch already covers that with 16).
template <int NW>
constexpr int pro_batch() { return NW >= 16 ? 1 : 4; }

// The first batch of a prologue's row loads, issued ahead (q8a_row_loads)
// by a kernel that then issues its first weight loads: those are younger
// than the row's, so the in-order wait for the row does not wait for them.
// (named members, not an array: the row's registers must not go to scratch)
template <int NW>
struct RowLoads {
  static constexpr int kX = pro_batch<NW>() < 3 ? pro_batch<NW>() : 3;  // plain pass: x only
  float4 x0, x1, x2, w0;                                               // norm pass: x0 and w0
  __device__ float4 x(int k) const { return k == 0 ? x0 : (k == 1 ? x1 : x2); }
};

// The loads of the first batch, in the order and with the clamped
// addresses q8a_prologue uses (the norm pass: its first float4 of x and of
// the weights; the plain pass: the first kX of its spans).
template <int NW>
__device__ __forceinline__ void q8a_row_loads(const FusedIn& in, int t, int cols, bool norm,
                                              RowLoads<NW>& rl) {
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const float* x = in.x + (size_t)t * cols;
  auto ld = [&](int i) { return *reinterpret_cast<const float4*>(x + (i < cols ? i : 0)); };
  if (norm) {
    rl.x0 = ld(4 * tid);
    rl.w0 = *reinterpret_cast<const float4*>(in.norm_w + (4 * tid < cols ? 4 * tid : 0));
  } else {
    rl.x0 = ld(wave * 256 + 4 * lane);
    if (RowLoads<NW>::kX > 1) rl.x1 = ld((wave + NW) * 256 + 4 * lane);
    if (RowLoads<NW>::kX > 2) rl.x2 = ld((wave + 2 * NW) * 256 + 4 * lane);
  }
}

// NW: waves per workgroup.  k_qk / k_dk (optional): also the Q8_K form of
// the (normed) row, written to memory for position t.  With use_pre, pre
// holds the first batch's loads, issued by q8a_row_loads.  af_s (optional):
// the f32 values d q of the Q8A form, in the skewed row layout of QuantOut.
// DPP_CHAIN: the eight sum-of-squares chains on DPP rows of waves 0 and 1
// (needs the whole of both waves and cols % 8 == 0), else on lanes 0-7.
template <int NW, bool DPP_CHAIN = false>
__device__ __forceinline__ bool q8a_prologue(const FusedIn& in, int t, int cols, bool norm,
                                             float* xs, float* ws, float* sq, int cs,
                                             int8_t* qa_s, float* da_s, float* misc,
                                             int8_t* k_qk = nullptr, float* k_dk = nullptr,
                                             bool use_pre = false, RowLoads<NW> pre = {},
                                             float* af_s = nullptr) {
  constexpr int kProBatch = pro_batch<NW>();
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const float* x = in.x + (size_t)t * cols;
  const bool want_k = k_qk != nullptr;
  const QuantOut q{qa_s, da_s, af_s, want_k ? k_qk + (size_t)t * cols : nullptr,
                   want_k ? k_dk + (size_t)t * (cols / 256) : nullptr, 1};
  bool bad = false;
  if (norm) {
    constexpr int kStep = 4 * 64 * NW;  // elements per float4 pass of the workgroup
    for (int base = 0; base < cols; base += kStep * kProBatch) {
      float4 xv[kProBatch], wv[kProBatch];
#pragma unroll
      for (int k = 0; k < kProBatch; k++) {
        const int i = base + kStep * k + 4 * tid;
        const int il = i < cols ? i : 0;  // unconditional loads (see above), unused past cols
        if (use_pre && base == 0 && k == 0) {
          xv[k] = pre.x0;
          wv[k] = pre.w0;
        } else {
          xv[k] = *reinterpret_cast<const float4*>(x + il);
          wv[k] = *reinterpret_cast<const float4*>(in.norm_w + il);
        }
      }
#pragma unroll
      for (int k = 0; k < kProBatch; k++) {
        const int i = base + kStep * k + 4 * tid;
        if (i < cols) {
          const float xe[4] = {xv[k].x, xv[k].y, xv[k].z, xv[k].w};
          const float we[4] = {wv[k].x, wv[k].y, wv[k].z, wv[k].w};
          *reinterpret_cast<float4*>(xs + i) = xv[k];
          *reinterpret_cast<float4*>(ws + i) = wv[k];
          // the element index through an empty asm: the four chain-major
          // addresses are formed here, not at the kernel's start and held
          // through the loads (at a 1024-thread launch's 128 registers they
          // went to scratch)
          int ia = i;
          asm volatile("" : "+v"(ia));
#pragma unroll
          for (int c = 0; c < 4; c++) {
            bad |= any_nonfinite(xe[c], we[c]);
            sq[((ia & 7) + c) * cs + (ia >> 3)] = xe[c] * xe[c];
          }
        }
      }
    }
    __syncthreads();
    if (DPP_CHAIN && cols % 8 == 0) {
      if (wave < 2) {
        const int c = 4 * wave + (lane >> 4);
        const float sum = chain_group_lds<16>(0.0f, sq + c * cs, cols / 8);
        if ((lane & 15) == 0) misc[c] = sum;
      }
    } else if (tid < 8) {
      misc[tid] = chain_sum_lds(0.0f, sq + tid * cs, (cols - tid + 7) / 8);
    }
    __syncthreads();
    // every thread forms r from the eight sums (no thread-0 pass and barrier)
    const float ss = finish_8lane(misc);
    const float m = ss / (float)cols;
    const float r = 1.0f / sqrtf(m + in.eps);
    if (!finite(r)) bad = true;
    for (int span = wave; span * 256 < cols; span += NW) {
      const int e = span * 256 + 4 * lane;
      const bool inb = e < cols;
      float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if (inb) {
        const float4 xf = *reinterpret_cast<const float4*>(xs + e);
        const float4 wf = *reinterpret_cast<const float4*>(ws + e);
        v[0] = (xf.x * r) * wf.x;
        v[1] = (xf.y * r) * wf.y;
        v[2] = (xf.z * r) * wf.z;
        v[3] = (xf.w * r) * wf.w;
#pragma unroll
        for (int c = 0; c < 4; c++) bad |= !finite(v[c]);
      }
      quantize_span(v, inb, (size_t)span * 256, true, want_k, q);
    }
  } else {
    for (int s0 = wave; s0 * 256 < cols; s0 += NW * kProBatch) {
      float4 f[kProBatch];
#pragma unroll
      for (int k = 0; k < kProBatch; k++) {
        const int e = (s0 + NW * k) * 256 + 4 * lane;
        const float4 v = use_pre && s0 == wave && k < RowLoads<NW>::kX
                             ? pre.x(k)
                             : *reinterpret_cast<const float4*>(x + (e < cols ? e : 0));
        f[k] = e < cols ? v : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int k = 0; k < kProBatch; k++) {
        const int span = s0 + NW * k;
        if (span * 256 < cols) {
          const int e = span * 256 + 4 * lane;
          const bool inb = e < cols;
          float v[4] = {f[k].x, f[k].y, f[k].z, f[k].w};
          if (inb) bad |= any_nonfinite(v[0], v[1], v[2], v[3]);
          quantize_span(v, inb, (size_t)span * 256, true, want_k, q);
        }
      }
    }
  }
  __syncthreads();
  return bad;
}

}  // namespace

// Q4_K decode with the products and the chains on different lanes.  A
// workgroup of eight waves owns RB rows.  Waves 1-7 stream their share of
// the packed weight rows (16 quant bytes, i.e. 16 elements of two adjacent
// sub-blocks, plus the superblock's header per unit) through an NS-deep
// register ring (one SL-column stage per slot, loads issued
// unconditionally), dequantise them in registers to q4_k_value's
// (d sc) q - dmin m (det-quant lib.rs:506-517), multiply them by the
// activations (all T positions, staged in LDS once) and store the rounded
// products row-major in LDS; after the stage's barrier, wave 0's lanes
// (row r, position t) add their row of products in element order, twelve
// float4 ahead of the adds, while the other waves already form the next
// stage.  The chain, the one serial part, therefore runs one add per
// element with its operands in LDS; the weights' HBM latency is covered by
// NS stages, and the weights cost their packed 0.5625 bytes per element.
template <int N4>
__device__ __forceinline__ float chain_sum_lds_n(float a, const float* v) {
  constexpr int kRing = N4 < 12 ? N4 : 12;
  constexpr int kLoop = (N4 - kRing) / kRing;  // ring turns with a refill per slot
  constexpr int kRem = N4 - kLoop * kRing;     // then kRem float4, kRing of them in the ring
  const float4* v4 = reinterpret_cast<const float4*>(v);
  float4 r[kRing];
#pragma unroll
  for (int q = 0; q < kRing; q++) r[q] = v4[q];
  // a rolled loop: fully unrolled, the reads would be hoisted out of the ring
#pragma unroll 1
  for (int it = 0; it < kLoop; it++) {
#pragma unroll
    for (int q = 0; q < kRing; q++) {
      a += r[q].x;
      a += r[q].y;
      a += r[q].z;
      a += r[q].w;
      r[q] = v4[(it + 1) * kRing + q];
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int q = 0; q < kRem; q++) {
    const int slot = q % kRing;
    a += r[slot].x;
    a += r[slot].y;
    a += r[slot].z;
    a += r[slot].w;
    if (q + kRing < kRem) r[slot] = v4[kLoop * kRing + kRing + q];
    __builtin_amdgcn_sched_barrier(0);
  }
  return a;
}

// Matrices of one launch: one matrix (rows0), two over the same input with
// their rows concatenated (wq and wk: rows0 + rows1, each its own output,
// bias and epilogue), or gate and up (rows0 each) finishing as
// silu(gate) * up (det-model lib.rs:2420-2434).
enum { PC_SINGLE = 0, PC_CAT = 1, PC_PAIR = 2 };

struct Q4kPcArgs {
  // packed Q4_K: per superblock 128 quant bytes (q0/q1) and a 16-byte header
  // (h0/h1: d, dmin, the 12 scale bytes), nb superblocks per row
  const uint8_t* q0;
  const uint8_t* q1;
  const uint8_t* h0;
  const uint8_t* h1;
  int nb;
  int rows0, rows1, cols, T;
  const float* af;      // the Q8A values of the input, or null: formed from x
  const float* x;       // raw input (with af null), normed first when norm_w is set
  const float* norm_w;
  float eps;
  int8_t* side_qk;      // with x: the first workgroup also writes the input's Q8_K form
  float* side_dk;
  // With x: a Q6_K matrix over the same normed input (wv), one row per
  // wave 1-7 of each workgroup (row blockIdx.x + (wave - 1) * gridDim.x),
  // at most eight superblocks per row.
  const uint32_t* v6w;  // 208-byte superblock bodies as 52 words
  const uint16_t* v6d;
  int v6rows, v6nb;
  float* v6out;
  const float* v6bias;
  int v6epi;
  float* out0;
  float* out1;
  const float* bias0;
  const float* bias1;
  int epi0, epi1;
  int* err;
};

// Floats of the input prologue's scratch: row, norm weights, chain-major
// squares and 16 of scratch.
__host__ __device__ constexpr size_t q4k_pc_prologue_floats(int cols) {
  return 2 * (size_t)cols + 8 * (size_t)((((cols + 7) / 8) + 3) & ~3) + 16;
}

constexpr int kPcThreads = 512;    // eight waves
constexpr int kPcChainWaves = 3;   // waves 0-2 run the chains
constexpr int kPcProducers = kPcThreads - 64 * kPcChainWaves;  // waves 3-7 form the products
constexpr int kPcMaxUnits = 2;     // 16-byte quant units per producer thread and stage
// With PT threads per workgroup (512, or 1024 for the gate+up pair): the
// producer lanes, and the units each forms per stage (one at 1024: 832
// lanes cover every stage the plan allows).
__host__ __device__ constexpr int pc_producers(int PT) { return PT - 64 * kPcChainWaves; }
__host__ __device__ constexpr int pc_max_units(int PT) { return PT > 512 ? 1 : kPcMaxUnits; }

// Chains per chain wave: a DPP row of 16 lanes per chain (CR = 16) while
// they fit, else a quad of 4 (CR = 4).
__host__ __device__ constexpr int q4k_pc_chains(int CR) { return kPcChainWaves * (64 / CR); }

// LDS bytes: activations, two product buffers and, when the kernel forms
// the activations itself, the prologue's row, norm weights, chain-major
// squares and scratch.
// Activation rows and product rows keep four floats of padding after every
// 64 columns (column c at c + 4 (c / 64)): the sixteen-float units a
// producer wave writes and reads then fall on different LDS banks.
__host__ __device__ constexpr int q4k_pc_skew(int c) { return c + ((c >> 6) << 2); }
__host__ __device__ constexpr int q4k_pc_ldp(int SL) { return q4k_pc_skew(SL) + 4; }

__host__ __device__ inline size_t q4k_pc_smem(int T, int cols, int NR, int SL, bool prologue, bool v6,
                                              int pt = kPcThreads) {
  const int pw = pt / 64 - kPcChainWaves;  // producer waves
  size_t f = (size_t)T * q4k_pc_skew(cols) + (size_t)2 * NR * T * q4k_pc_ldp(SL);
  if (prologue || v6) f += q4k_pc_prologue_floats(cols);
  if (v6) f += (size_t)T * cols / 4 + (size_t)T * (cols / 256) + (size_t)pw * 64 + (size_t)pw * 8;
  return f * sizeof(float);
}

template <int SL, int NS, int MODE, int CR, int PT = kPcThreads>
__global__ void __launch_bounds__(PT) k_gemv_q4k_pc(Q4kPcArgs p, int RB) {
  constexpr int kPcProducers = pc_producers(PT);  // this launch's producer lanes
  constexpr int kPcMaxUnits = pc_max_units(PT);
  constexpr int NM = MODE == PC_PAIR ? 2 : 1;
  // fused Q6_K rows: wq+wk launches with 512-column stages only (the
  // 128-column variants have no registers to spare for them)
  constexpr bool V6 = MODE == PC_CAT && SL == 512;
  constexpr int LDP = q4k_pc_ldp(SL);     // product row stride (floats)
  constexpr int G = 64 / CR;              // chains per chain wave
  const int NR = NM * RB;                 // staged rows (gate rows, then up rows)
  extern __shared__ __align__(16) float smem[];
  const int cols = p.cols, T = p.T;
  const int rows_total = MODE == PC_CAT ? p.rows0 + p.rows1 : p.rows0;
  const int ACS = q4k_pc_skew(cols);      // activation row stride
  float* as = smem;                       // [T][ACS] activations
  float* prod = smem + (size_t)T * ACS;   // [2][NR * T][LDP] products
  // fused Q6_K rows: the input's Q8_K form [T][cols] (int8) and scales
  // [T][cols / 256], then per producer wave eight superblocks' class sums and scales
  float* v6area = prod + (size_t)2 * NR * T * LDP + q4k_pc_prologue_floats(cols);
  int8_t* v6q = reinterpret_cast<int8_t*>(v6area);
  float* v6dk = v6area + (size_t)T * cols / 4;
  // [producer waves][8][8], then [producer waves][8]
  int* v6aux = reinterpret_cast<int*>(v6dk + (size_t)T * (cols / 256));
  float* v6ds = reinterpret_cast<float*>(v6aux + (PT / 64 - kPcChainWaves) * 64);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool producer = wave >= kPcChainWaves;
  const int row0 = blockIdx.x * RB;
  const int nst = cols / SL;
  // Unit j of producer thread x = tid - 64 kPcChainWaves is f = x + kPcProducers j:
  // staged row f / UPR, bytes 16 (f % UPR) of the row's SL / 2 quant bytes of
  // the stage.  Rows past the end read the last row, units past WPU read the
  // workgroup's first row and store nothing.
  constexpr int UPR = SL / 32;            // units per row and stage
  const int WPU = NR * UPR;               // units per stage
  const int nb = p.nb;
  auto row_of = [&](int f, int* m) {
    const int j = f < WPU ? f / UPR : 0;
    int row;
    if (MODE == PC_PAIR) {
      *m = j < RB ? 0 : 1;
      row = row0 + j % RB;
      row = row < p.rows0 ? row : p.rows0 - 1;
    } else {
      int g = row0 + j;
      g = g < rows_total ? g : rows_total - 1;
      *m = MODE == PC_CAT && g >= p.rows0 ? 1 : 0;
      row = *m ? g - p.rows0 : g;
    }
    return row;
  };
  const int ptid = producer ? tid - 64 * kPcChainWaves : 0;
  // The fused Q6_K row's superblock words of this lane (see below), loaded
  // now so that they arrive during the stages; waves past the rows load row 0.
  uint4 v6a{}, v6b{}, v6c{}, v6e{};
  uint32_t v6sc = 0;
  uint16_t v6dw = 0;
  // (at 1024 threads there are no registers to hold them through the
  // stages: they are loaded where they are used)
  constexpr bool kV6Early = PT <= 512;
  auto v6_loads = [&]() {
    int r6 = blockIdx.x + (wave - kPcChainWaves) * gridDim.x;
    r6 = r6 < p.v6rows ? r6 : 0;
    const int sb = lane >> 3, h = (lane >> 2) & 1, pp = lane & 3;
    const int sbl = sb < p.v6nb ? sb : 0;
    const uint32_t* body = p.v6w + ((size_t)r6 * p.v6nb + sbl) * 52;
    v6a = reinterpret_cast<const uint4*>(body + 16 * h + 8 * (pp & 1))[0];
    v6b = reinterpret_cast<const uint4*>(body + 16 * h + 8 * (pp & 1))[1];
    v6c = reinterpret_cast<const uint4*>(body + 32 + 8 * h)[0];
    v6e = reinterpret_cast<const uint4*>(body + 32 + 8 * h)[1];
    v6sc = body[48 + 2 * h + (pp >> 1)];
    v6dw = p.v6d[(size_t)r6 * p.v6nb + sbl];
  };
  if (V6 && kV6Early && p.v6w && producer) v6_loads();
  // the producers' weights: the first NS stages are in flight before the
  // activations load
  // Units past the first round of kPcProducers: when there are at most half
  // as many, each goes to two lanes as halves (the sixteen elements of one
  // of its two sub-blocks), so that a wave's second round costs half a unit
  // (the gate+up launch: 352 units, 32 past the first round).
  const int E = WPU - kPcProducers;
  const bool halves = E > 0 && 2 * E <= kPcProducers;
  const int f2 = halves ? (ptid < 2 * E ? kPcProducers + (ptid >> 1) : WPU) : ptid + kPcProducers;
  const int hi2 = ptid & 1;
  // Gate+up with one unit per lane (1024 threads) and at most half as many
  // units as producer lanes: every unit goes to two lanes as halves (lane
  // 2 f + h: sub-block h of unit f's two).  There the chains waited on the
  // producers (384 units for 832 lanes): stages of 2.5-2.9k cycles became
  // 2.3-2.6k and the launch 16.3 -> 15.8 us; the other launches, whose
  // chains set the pace, gained nothing and keep whole units.
  const bool split = MODE == PC_PAIR && kPcMaxUnits == 1 && 2 * WPU <= kPcProducers;
  const int f0 = split ? ptid >> 1 : ptid;
  const int hi0 = ptid & 1;
  int m0, m1;
  const int r0 = row_of(f0, &m0), r1 = row_of(f2, &m1);
  const uint8_t* qr0 = (m0 ? p.q1 : p.q0) + (size_t)r0 * nb * 128;
  const uint8_t* hr0 = (m0 ? p.h1 : p.h0) + (size_t)r0 * nb * 16;
  const uint8_t* qr1 = (m1 ? p.q1 : p.q0) + (size_t)r1 * nb * 128;
  const uint8_t* hr1 = (m1 ? p.h1 : p.h0) + (size_t)r1 * nb * 16;
  const int u0 = f0 < WPU ? f0 % UPR : 0;
  const int u1 = f2 < WPU ? f2 % UPR : 0;
  uint4 qa0[NS], ha0[NS], qa1[NS], ha1[NS];
#define DTL_PC_LOAD(slot, k)                                                                \
  do {                                                                                      \
    const int kk_ = (k) < nst ? (k) : nst - 1;                                              \
    const int b0_ = kk_ * (SL / 2) + 16 * u0, b1_ = kk_ * (SL / 2) + 16 * u1;               \
    qa0[slot] = *reinterpret_cast<const uint4*>(qr0 + b0_);                                 \
    ha0[slot] = *reinterpret_cast<const uint4*>(hr0 + (b0_ >> 7) * 16);                     \
    if (kPcMaxUnits > 1) {                                                                  \
      qa1[slot] = *reinterpret_cast<const uint4*>(qr1 + b1_);                               \
      ha1[slot] = *reinterpret_cast<const uint4*>(hr1 + (b1_ >> 7) * 16);                   \
    }                                                                                       \
  } while (0)
  // The input row's first loads, then the first NS stages' weights (younger,
  // so the prologue's wait for the row does not wait for them).
  const FusedIn in{p.x, p.norm_w, p.eps};
  // (at 1024 threads the registers for holding them are not there)
  constexpr bool kPre = PT <= 512;
  RowLoads<PT / 64> pre;
  if (kPre && !p.af) q8a_row_loads<PT / 64>(in, 0, cols, p.norm_w != nullptr, pre);
  // Stage 0 of gate+up on the chain waves: each chain's lanes load their
  // own first-stage weights here (lane k of a group of CR: the quant dword
  // holding its elements 4 k .. 4 k + 3 of every group, and the stage's
  // superblock headers) and, after the prologue, form those products just
  // before their adds, so the chains start without waiting for a producer
  // pass and its barrier; the producers begin at stage 1.  Only gate+up,
  // whose chains waited on the producers, gains (14.95 -> 14.6 us); where
  // the chains set the pace (wq+wk, wo, ffn_down: sixteen-lane chains),
  // the chain waves' own dequantisation in front of every group of adds
  // cost more than the first stage's wait (12.4 -> 14.5 us, 9.2 -> 10.1).
  constexpr int G0 = SL / (4 * CR);        // groups of 4 CR terms per stage
  constexpr bool kDirect0 = MODE == PC_PAIR && G0 <= 16;
  constexpr int H0 = (SL + 255) / 256;     // superblock headers per stage
  constexpr int K0 = kDirect0 ? 1 : 0;     // the producers' first stage
  // Groups (and headers) loaded at the start: at most 256 columns' worth,
  // the rest when stage 0 begins, behind the first groups' adds (held
  // through the prologue, a 512-column stage's sixteen registers spilled
  // at the 1024-thread cap).
  constexpr int GE = G0 * 4 * CR > 256 ? 256 / (4 * CR) : G0;
  constexpr int HE = (GE * 4 * CR + 255) / 256;
  // Chain c = G wave + group: staged row c % NR, position c / NR (with
  // the gate and up chains of one row and position in adjacent groups for
  // the pair).  Groups past the chains add chain 0's products and store
  // nothing, so the whole wave runs every DPP add.
  const int grp = lane / CR, cidx = G * wave + grp;
  int chain_row;
  if (MODE == PC_PAIR) {
    const int pc = cidx >> 1, j = pc % RB, t = pc / RB;
    chain_row = pc < RB * T ? ((cidx & 1) ? RB + j : j) + NR * t : 0;
  } else {
    chain_row = cidx < NR * T ? cidx : 0;
  }
  uint32_t cq[kDirect0 ? G0 : 1];
  uint4 ch[kDirect0 ? H0 : 1];
  if (kDirect0 && !producer) {
    int mc;
    const int rc = row_of((chain_row % NR) * UPR, &mc);
    const uint8_t* qrow = (mc ? p.q1 : p.q0) + (size_t)rc * nb * 128;
    const uint8_t* hrow = (mc ? p.h1 : p.h0) + (size_t)rc * nb * 16;
    const int kl = lane & (CR - 1);
#pragma unroll
    for (int g = 0; g < GE; g++) {
      // element e0 of the row lies in 32-byte block e0 / 64, byte e0 % 32
      // (the low nibbles hold the block's first 32 elements)
      const int e0 = 4 * CR * g + 4 * kl;
      cq[g] = *reinterpret_cast<const uint32_t*>(qrow + (e0 >> 6) * 32 + (e0 & 31));
    }
#pragma unroll
    for (int hh = 0; hh < HE; hh++) ch[hh] = *reinterpret_cast<const uint4*>(hrow + hh * 16);
  }
  if (producer) {
#pragma unroll
    for (int u = 0; u < NS; u++) DTL_PC_LOAD(u, u + K0);
  }
  if (p.af) {
    for (int i = tid; i < T * cols / 4; i += PT) {
      const int t = 4 * i / cols, e = 4 * i - t * cols;
      *reinterpret_cast<float4*>(as + (size_t)t * ACS + q4k_pc_skew(e)) =
          reinterpret_cast<const float4*>(p.af)[i];
    }
  } else {
    // The input's rmsnorm (with norm_w) and Q8A quantisation, as the
    // separate kernels form them, into the f32 values d * q.
    const int cs = (((cols + 7) / 8) + 3) & ~3;
    float* xs = prod + (size_t)2 * NR * T * LDP;
    float* ws = xs + cols;
    float* sq = ws + cols;
    float* misc = sq + 8 * cs;
    bool bad = false;
    for (int t = 0; t < T; t++) {
      // the Q8_K form: to LDS for the fused Q6_K rows, else (first
      // workgroup) to memory for a separate Q6_K launch
      const bool side = blockIdx.x == 0 && p.side_qk;
      int8_t* kq = p.v6w ? v6q : (side ? p.side_qk : nullptr);
      float* kd = p.v6w ? v6dk : (side ? p.side_dk : nullptr);
      // the Q8A values d q straight into the activation rows
      bad |= q8a_prologue<PT / 64, true>(in, t, cols, p.norm_w != nullptr, xs, ws, sq, cs,
                                                 nullptr, nullptr, misc, kq, kd, kPre && t == 0, pre,
                                                 as + (size_t)t * ACS);
    }
    if (bad && tid == 0) flag(p.err, ERRBIT_NON_FINITE);
  }
  __syncthreads();
  // The 32 products of unit f (staged row r, quant bytes b.. b+15 of the
  // row): elements b % 32 + [0, 16) of sub-blocks 2 g and 2 g + 1 of
  // superblock b / 128, g = (b % 128) / 32, at stage columns c and c + 32.
  auto products = [&](float* pb, int k, int f, uint4 qv, uint4 hv) {
    if (f >= WPU) return;
    const int r = f / UPR;
    const int b = k * (SL / 2) + 16 * (f % UPR);
    const int g = (b & 127) >> 5;
    const int c = (b >> 7) * 256 + 64 * g + (b & 31) - k * SL;
    const float d = f16_to_f32((uint16_t)(hv.x & 0xffffu)), dmin = f16_to_f32((uint16_t)(hv.x >> 16));
    int sc0, mn0, sc1, mn1;
    q4k_scale_min3(hv.y, hv.z, hv.w, 2 * g, &sc0, &mn0);
    q4k_scale_min3(hv.y, hv.z, hv.w, 2 * g + 1, &sc1, &mn1);
    const float dsc0 = d * (float)sc0, dm0 = dmin * (float)mn0;
    const float dsc1 = d * (float)sc1, dm1 = dmin * (float)mn1;
    const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
    float wl[16], wh[16];
    // the nibbles of a dword masked at once, each byte then converted by
    // v_cvt_f32_ubyte0-3 (no per-element extraction)
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t lo = qw[j] & 0x0f0f0f0fu, hi = (qw[j] >> 4) & 0x0f0f0f0fu;
      const float fl[4] = {ubyte_f32<0>(lo), ubyte_f32<1>(lo), ubyte_f32<2>(lo), ubyte_f32<3>(lo)};
      const float fh[4] = {ubyte_f32<0>(hi), ubyte_f32<1>(hi), ubyte_f32<2>(hi), ubyte_f32<3>(hi)};
#pragma unroll
      for (int b = 0; b < 4; b++) {
        wl[4 * j + b] = dsc0 * fl[b] - dm0;
        wh[4 * j + b] = dsc1 * fh[b] - dm1;
      }
    }
    // columns c and c + 32 lie in one 64-column group, k SL is a multiple of 64
    const int cs = q4k_pc_skew(c);
    const int e = q4k_pc_skew(k * SL);
    for (int t = 0; t < T; t++) {
      const float* at = as + (size_t)t * ACS + e;
      float* pr = pb + (r + NR * t) * LDP;
      // all eight activation reads before the first product store (the
      // compiler cannot move a read above a store to the same LDS)
      float4 a[4], h[4];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        a[q] = *reinterpret_cast<const float4*>(at + cs + 4 * q);
        h[q] = *reinterpret_cast<const float4*>(at + cs + 32 + 4 * q);
      }
#pragma unroll
      for (int q = 0; q < 4; q++) {
        *reinterpret_cast<float4*>(pr + cs + 4 * q) = make_float4(
            wl[4 * q] * a[q].x, wl[4 * q + 1] * a[q].y, wl[4 * q + 2] * a[q].z, wl[4 * q + 3] * a[q].w);
        *reinterpret_cast<float4*>(pr + cs + 32 + 4 * q) = make_float4(
            wh[4 * q] * h[q].x, wh[4 * q + 1] * h[q].y, wh[4 * q + 2] * h[q].z, wh[4 * q + 3] * h[q].w);
      }
    }
  };
  // One sub-block of unit f (hi: the high nibbles, columns c + 32 ..), with
  // the values and order of the full unit's.
  auto products_half = [&](float* pb, int k, int f, int hi, uint4 qv, uint4 hv) {
    if (f >= WPU) return;
    const int r = f / UPR;
    const int b = k * (SL / 2) + 16 * (f % UPR);
    const int g = (b & 127) >> 5;
    const int c = (b >> 7) * 256 + 64 * g + (b & 31) - k * SL;
    const float d = f16_to_f32((uint16_t)(hv.x & 0xffffu)), dmin = f16_to_f32((uint16_t)(hv.x >> 16));
    int sc, mn;
    q4k_scale_min3(hv.y, hv.z, hv.w, 2 * g + hi, &sc, &mn);
    const float dsc = d * (float)sc, dm = dmin * (float)mn;
    const uint32_t qw[4] = {qv.x, qv.y, qv.z, qv.w};
    float w[16];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t nib = (qw[j] >> (4 * hi)) & 0x0f0f0f0fu;
      const float f[4] = {ubyte_f32<0>(nib), ubyte_f32<1>(nib), ubyte_f32<2>(nib), ubyte_f32<3>(nib)};
#pragma unroll
      for (int b = 0; b < 4; b++) w[4 * j + b] = dsc * f[b] - dm;
    }
    // c + 32 lies in the 64-column group of c
    const int cs = q4k_pc_skew(c) + 32 * hi;
    const int e = q4k_pc_skew(k * SL);
    for (int t = 0; t < T; t++) {
      const float* at = as + (size_t)t * ACS + e;
      float* pr = pb + (r + NR * t) * LDP;
      float4 a[4];
#pragma unroll
      for (int q = 0; q < 4; q++) a[q] = *reinterpret_cast<const float4*>(at + cs + 4 * q);
#pragma unroll
      for (int q = 0; q < 4; q++)
        *reinterpret_cast<float4*>(pr + cs + 4 * q) = make_float4(
            w[4 * q] * a[q].x, w[4 * q + 1] * a[q].y, w[4 * q + 2] * a[q].z, w[4 * q + 3] * a[q].w);
    }
  };
  if (producer) {
    // Stage k's products go to buffer k & 1; the barrier after them hands
    // the buffer to the chain waves, which add it while the next stage forms.
    for (int base = K0; base < nst; base += NS) {
#pragma unroll
      for (int u = 0; u < NS; u++) {
        const int k = base + u;  // stages past the end form unused products
        float* pb = prod + (size_t)(k & 1) * NR * T * LDP;
        const int kk = k < nst ? k : nst - 1;
        if (split)
          products_half(pb, kk, f0, hi0, qa0[u], ha0[u]);
        else
          products(pb, kk, ptid, qa0[u], ha0[u]);
        if (kPcMaxUnits > 1) {
          if (halves)
            products_half(pb, kk, f2, hi2, qa1[u], ha1[u]);
          else
            products(pb, kk, f2, qa1[u], ha1[u]);
        }
        DTL_PC_LOAD(u, k + NS);
        __syncthreads();
      }
    }
  } else {
    const int c = cidx;
    float sum = 0.0f;
    if (kDirect0) {
      // stage 0: the products of this lane's four terms of each group,
      // formed as the producers form them ((d sc) q - dmin m, times the
      // activation), then the group's adds
      const float* arow = as + (size_t)(chain_row / NR) * ACS;
      const int kl = lane & (CR - 1);
      if (GE < G0) {
        int mc;
        const int rc = row_of((chain_row % NR) * UPR, &mc);
        const uint8_t* qrow = (mc ? p.q1 : p.q0) + (size_t)rc * nb * 128;
        const uint8_t* hrow = (mc ? p.h1 : p.h0) + (size_t)rc * nb * 16;
#pragma unroll
        for (int g = GE; g < G0; g++) {
          const int e0 = 4 * CR * g + 4 * kl;
          cq[g] = *reinterpret_cast<const uint32_t*>(qrow + (e0 >> 6) * 32 + (e0 & 31));
        }
#pragma unroll
        for (int hh = HE; hh < H0; hh++) ch[hh] = *reinterpret_cast<const uint4*>(hrow + hh * 16);
      }
#pragma unroll
      for (int g = 0; g < G0; g++) {
        const int e0 = 4 * CR * g + 4 * kl;
        const uint4 h = ch[(4 * CR * g) >> 8];
        const float d = f16_to_f32((uint16_t)(h.x & 0xffffu)), dmin = f16_to_f32((uint16_t)(h.x >> 16));
        int sc, mn;
        q4k_scale_min3(h.y, h.z, h.w, (e0 & 255) >> 5, &sc, &mn);
        const float dsc = d * (float)sc, dm = dmin * (float)mn;
        const uint32_t nib = (cq[g] >> (4 * ((e0 >> 5) & 1))) & 0x0f0f0f0fu;
        const float4 a = *reinterpret_cast<const float4*>(arow + q4k_pc_skew(e0));
        const float w0 = dsc * ubyte_f32<0>(nib) - dm, w1 = dsc * ubyte_f32<1>(nib) - dm;
        const float w2 = dsc * ubyte_f32<2>(nib) - dm, w3 = dsc * ubyte_f32<3>(nib) - dm;
        sum = chain_group_add<CR>(sum, make_float4(w0 * a.x, w1 * a.y, w2 * a.z, w3 * a.w));
      }
    }
    for (int base = K0; base < nst; base += NS) {
#pragma unroll
      for (int u = 0; u < NS; u++) {
        const int k = base + u;
        __syncthreads();
        if (k < nst)
          sum = chain_group_lds<CR, true>(sum, prod + (size_t)(k & 1) * NR * T * LDP + (size_t)chain_row * LDP, SL);
      }
    }
    if ((lane & (CR - 1)) != 0) return;
    if (MODE == PC_PAIR) {
      const float u = __shfl(sum, lane + CR);  // the up chain of the same row and position
      const int pc = c >> 1, j = pc % RB, t = pc / RB;
      const int row = row0 + j;
      if ((c & 1) || pc >= RB * T || row >= p.rows0) return;
      const float v = silu_det(sum) * u;
      p.out0[(size_t)t * p.rows0 + row] = v;
      if (!(finite(sum) && finite(u) && finite(v))) flag(p.err, ERRBIT_NON_FINITE);
      return;
    }
    if (c >= NR * T) return;
    const int j = c % NR, t = c / NR;
    const int g = row0 + j;
    if (g >= rows_total) return;
    const bool m = MODE == PC_CAT && g >= p.rows0;
    const int row = m ? g - p.rows0 : g, R = m ? p.rows1 : p.rows0;
    if (!epilogue(sum, m ? p.out1 : p.out0, (size_t)t * R + row, m ? p.bias1 : p.bias0, row,
                  m ? p.epi1 : p.epi0))
      flag(p.err, ERRBIT_NON_FINITE);
    return;
  }
#undef DTL_PC_LOAD
  if (V6 && p.v6w) {
    if (!kV6Early) v6_loads();
    const int r6 = blockIdx.x + (wave - kPcChainWaves) * gridDim.x;
    if (r6 < p.v6rows) {
      // dot_q6_k_q8k (det-quant lib.rs:353-397): lane = (superblock sb,
      // half h, part pp) forms its share of the eight class sums (exact
      // integers, reduced over the eight lanes of the superblock); lane 0
      // then runs sums[l] += (dw * da) * aux[l] over the superblocks in order
      // and adds the eight sums.
      const int nsb = p.v6nb;
      const int sb = lane >> 3, h = (lane >> 2) & 1, pp = lane & 3;
      const int sbl = sb < nsb ? sb : 0;
      const uint32_t qlw[8] = {v6a.x, v6a.y, v6a.z, v6a.w, v6b.x, v6b.y, v6b.z, v6b.w};
      const uint32_t qhw[8] = {v6c.x, v6c.y, v6c.z, v6c.w, v6e.x, v6e.y, v6e.z, v6e.w};
      const uint32_t scw = v6sc;
      const float dwf = f16_to_f32(v6dw);
      int* aux_w = v6aux + (wave - kPcChainWaves) * 64;
      float* ds_w = v6ds + (wave - kPcChainWaves) * 8;
      for (int t = 0; t < T; t++) {
        const uint32_t* act = reinterpret_cast<const uint32_t*>(v6q + (size_t)t * cols + (size_t)sbl * 256);
        int aux[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
          const uint32_t aw = act[8 * k + 4 * h + pp];
          int acc = 0;
#pragma unroll
          for (int pair = 0; pair < 2; pair++) {
            const int scale = (int)(int8_t)((scw >> (8 * (pair + 2 * (pp & 1)))) & 0xffu);
            int sum = 0;
#pragma unroll
            for (int ii = 0; ii < 2; ii++) {
              const int i = 2 * pair + ii;
              const int l0 = k + 8 * i;
              const uint32_t lo = (qlw[l0 >> 2] >> (8 * (l0 & 3) + 4 * (pp >> 1))) & 0x0fu;
              const uint32_t hi = (qhw[l0 >> 2] >> (8 * (l0 & 3) + 2 * pp)) & 0x03u;
              const int q6 = (int)(lo | (hi << 4)) - 32;
              const int av = (int)(int8_t)((aw >> (8 * i)) & 0xffu);
              sum += q6 * av;
            }
            acc += scale * sum;
          }
          aux[k] = acc;
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
          aux[k] += dpp_i32<kDppXor1>(aux[k]);
          aux[k] += dpp_i32<kDppXor2>(aux[k]);
          aux[k] += dpp_i32<kDppMirror8>(aux[k]);
        }
        if ((lane & 7) == 0 && sb < nsb) {
#pragma unroll
          for (int k = 0; k < 8; k++) aux_w[sb * 8 + k] = aux[k];
          ds_w[sb] = dwf * v6dk[(size_t)t * (cols / 256) + sb];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (lane == 0) {
          float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
          for (int b = 0; b < nsb; b++) {
            const float d = ds_w[b];
#pragma unroll
            for (int l = 0; l < 8; l++) sums[l] += d * (float)aux_w[b * 8 + l];
          }
          float v = 0.0f;
#pragma unroll
          for (int l = 0; l < 8; l++) v += sums[l];
          if (!epilogue(v, p.v6out, (size_t)t * p.v6rows + r6, p.v6bias, r6, p.v6epi))
            flag(p.err, ERRBIT_NON_FINITE);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    }
  }
}

// Rows per workgroup, columns per stage and the chain grouping.  A chain
// wave runs far slower when it shares its SIMD with another busy wave, so
// the rows are spread over at most one workgroup per CU (at least eight
// rows each); the chains (staged rows x positions) must fit the chain waves
// (twelve as DPP rows, 48 as quads) and the stage's weights kPcMaxUnits
// 16-byte quant units per producer thread.
bool q4k_pc_plan(int mode, int rows_total, int cols, int T, bool prologue, bool v6, int* RB,
                 int* SL, int* CR, size_t* smem, int pt = kPcThreads) {
  if (cols % 256 != 0 || T < 1) return false;
  static const int cus = [] {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      return 256;
    return n;
  }();
  const int NM = mode == PC_PAIR ? 2 : 1;
  int rb = (rows_total + cus - 1) / cus;  // rows_total: of each matrix for the pair
  rb = rb < 8 ? 8 : rb;
  if (NM * rb * T > q4k_pc_chains(4)) rb = q4k_pc_chains(4) / (NM * T);
  if (rb < 1) return false;
  const int NR = NM * rb;
  *CR = NR * T <= q4k_pc_chains(16) ? 16 : 4;
  // the longest stage (fewest barriers and ring refills) whose weights and
  // products fit
  int sl = 512;
  const int units = pc_max_units(pt) * pc_producers(pt);
  while (sl > 128 && (NR * (sl / 32) > units ||
                      q4k_pc_smem(T, cols, NR, sl, prologue, v6, pt) > 150 * 1024 || cols % sl != 0))
    sl /= 2;
  if (NR * (sl / 32) > units || cols % sl != 0) return false;
  if (v6 && (mode != PC_CAT || sl != 512)) return false;  // where the kernel has the fused rows
  *RB = rb;
  *SL = sl;
  *smem = q4k_pc_smem(T, cols, NR, sl, prologue, v6, pt);
  return *smem <= 150 * 1024;
}

template <int MODE>
bool launch_q4k_pc(const Q4kPcArgs& a, hipStream_t s) {
  const int rows_total = MODE == PC_CAT ? a.rows0 + a.rows1 : a.rows0;
  int RB, SL, CR;
  size_t smem;
  // Sixteen waves (thirteen producing) where the plan fits, else eight.
  int pt = 1024;
  if (!q4k_pc_plan(MODE, rows_total, a.cols, a.T, a.af == nullptr, a.v6w != nullptr, &RB, &SL, &CR, &smem, pt))
    pt = kPcThreads;
  if (!q4k_pc_plan(MODE, rows_total, a.cols, a.T, a.af == nullptr, a.v6w != nullptr, &RB, &SL, &CR, &smem, pt))
    return false;
  const dim3 grid((rows_total + RB - 1) / RB);
  // the fused Q6_K rows need the producer waves of the grid to cover them
  if (a.v6w && (a.af || a.v6nb > 8 || (int)grid.x * (pt / 64 - kPcChainWaves) < a.v6rows))
    return false;
#define DTL_Q4K_PC(sl, ns, cr, npt)                                                               \
  do {                                                                                           \
    static const bool attr = hipFuncSetAttribute((const void*)k_gemv_q4k_pc<sl, ns, MODE, cr, npt>, \
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,      \
                                                 150 * 1024) == hipSuccess;                       \
    (void)attr;                                                                                  \
    launch_kernel((k_gemv_q4k_pc<sl, ns, MODE, cr, npt>), grid, dim3(npt), smem, s, a, RB);       \
  } while (0)
  // At sixteen waves: two stages of weights in flight (three measured 1602
  // against 1584 us per TinyLlama decode token with the gate+up launch
  // alone at sixteen waves)
  if (pt == 1024) {
    if (CR == 16) {
      if (SL == 512) DTL_Q4K_PC(512, 2, 16, 1024);
      else if (SL == 256) DTL_Q4K_PC(256, 2, 16, 1024);
      else DTL_Q4K_PC(128, 2, 16, 1024);
    } else {
      if (SL == 512) DTL_Q4K_PC(512, 2, 4, 1024);
      else if (SL == 256) DTL_Q4K_PC(256, 2, 4, 1024);
      else DTL_Q4K_PC(128, 2, 4, 1024);
    }
    return true;
  }
  if (CR == 16) {
    if (SL == 512) DTL_Q4K_PC(512, 3, 16, 512);
    else if (SL == 256) DTL_Q4K_PC(256, 4, 16, 512);
    else DTL_Q4K_PC(128, 4, 16, 512);
  } else {
    if (SL == 512) DTL_Q4K_PC(512, 3, 4, 512);
    else if (SL == 256) DTL_Q4K_PC(256, 4, 4, 512);
    else DTL_Q4K_PC(128, 4, 4, 512);
  }
#undef DTL_Q4K_PC
  return true;
}

// LDS bytes of k_gemv_q8f: block terms, the Q8A activations and, with a
// norm, its scratch (the row, the weights, the chain-major squares).
size_t gemv_fused_smem(int nr, int cols, int nb, bool norm, int nw) {
  const size_t cs = (size_t)((((cols + 7) / 8) + 3) & ~3);
  size_t b = (size_t)nw * nr * nb_stride(nb) * 4 + (size_t)((cols + 15) & ~15) + (size_t)((nb + 3) & ~3) * 4;
  if (norm) b += 2 * (size_t)((cols + 3) & ~3) * 4 + 8 * cs * 4 + 16 * 4;
  return b;
}

template <int TYPE, int R, bool PAIR, bool QOUT = false, int NW = 4>
__global__ void __launch_bounds__(64 * NW) k_gemv_q8f(FusedMats M, FusedIn in, int* err) {
  constexpr int NR = PAIR ? 2 * R : R;
  static_assert(!QOUT || (PAIR && NW * R == 32), "quantized output: one 32-row Q8A block per workgroup");
  extern __shared__ __align__(16) float lds[];
  __shared__ float vq[QOUT ? 32 : 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.y;
  const int cols = M.cols, nb = M.nb;
  const int cs = (((cols + 7) / 8) + 3) & ~3;
  const int nbs = nb_stride(nb);
  float* vb = lds;
  int8_t* qa_s = reinterpret_cast<int8_t*>(lds + NW * NR * nbs);
  float* da_s = reinterpret_cast<float*>(qa_s + ((cols + 15) & ~15));
  float* xs = da_s + ((nb + 3) & ~3);
  float* ws = xs + ((cols + 3) & ~3);
  float* sq = ws + ((cols + 3) & ~3);
  float* misc = sq + 8 * cs;
  float* mine = vb + (size_t)wave * NR * nbs;
  const int row0 = (blockIdx.x * NW + wave) * R;
  // Slot r: (matrix, row) of the r-th dot of this wave.  Matrix choice is
  // wave-uniform, so the selects below stay scalar.
  const void* wp[NR];
  const uint16_t* dp[NR];
  int srow[NR];
  bool sval[NR];
#pragma unroll
  for (int r = 0; r < NR; r++) {
    int mi, row;
    if (PAIR) {
      mi = r < R ? 0 : 1;
      row = row0 + (r < R ? r : r - R);
      sval[r] = row < M.rows[0];
    } else {
      const int gr = row0 + r;
      mi = gr < M.row_end[0] ? 0 : (gr < M.row_end[1] ? 1 : 2);
      row = gr - (mi == 0 ? 0 : (mi == 1 ? M.row_end[0] : M.row_end[1]));
      sval[r] = gr < M.total_rows;
    }
    if (!sval[r]) {
      mi = 0;
      row = 0;
    }
    wp[r] = mi == 0 ? M.w[0] : (mi == 1 ? M.w[1] : M.w[2]);
    dp[r] = mi == 0 ? M.d16[0] : (mi == 1 ? M.d16[1] : M.d16[2]);
    srow[r] = row;
  }
  const int nchunk = TYPE == kGgmlQ8_0 ? 2 * nb : nb;
  bool bad = false;
  // the epilogue operand of this lane's row (lanes below R; the pair stores
  // its SwiGLU product and reads nothing)
  float pre = 0.0f;
  if (!PAIR) {
    int gr = row0 + (lane < R ? lane : 0);
    gr = gr < M.total_rows ? gr : M.total_rows - 1;
    const int mi = gr < M.row_end[0] ? 0 : (gr < M.row_end[1] ? 1 : 2);
    const int row = gr - (mi == 0 ? 0 : (mi == 1 ? M.row_end[0] : M.row_end[1]));
    const int rows = mi == 0 ? M.rows[0] : (mi == 1 ? M.rows[1] : M.rows[2]);
    pre = epilogue_operand(mi == 0 ? M.out[0] : (mi == 1 ? M.out[1] : M.out[2]), (size_t)t * rows + row,
                           mi == 0 ? M.bias[0] : (mi == 1 ? M.bias[1] : M.bias[2]), row,
                           mi == 0 ? M.epi[0] : (mi == 1 ? M.epi[1] : M.epi[2]));
  }
  // One chunk column of 64 lanes per pass (batching several passes' loads
  // measured slower: the extra registers cost more than the round trips).
  constexpr int NI = 1;
  for (int cb = 0; cb < nchunk; cb += 64 * NI) {
    uint4 w4[NI][NR];
    uint16_t dsc[NI][NR];
#pragma unroll
    for (int ii = 0; ii < NI; ii++) {
      // lanes past the row load its last chunk and store nothing: loads under
      // a condition would each be waited for before the next is issued
      const int c = cb + 64 * ii + lane;
      const int cl = c < nchunk ? c : nchunk - 1;
      const int b = TYPE == kGgmlQ8_0 ? cl >> 1 : cl;
#pragma unroll
      for (int r = 0; r < NR; r++) {
        if (TYPE == kGgmlQ8_0)
          w4[ii][r] = *(const uint4*)((const int8_t*)wp[r] + (size_t)srow[r] * cols + (size_t)cl * 16);
        else
          w4[ii][r] = *(const uint4*)((const uint8_t*)wp[r] + ((size_t)srow[r] * nb + cl) * 16);
        dsc[ii][r] = dp[r][(size_t)srow[r] * nb + b];
      }
    }
    if (cb == 0)
      bad |= q8a_prologue<NW>(in, t, cols, in.norm_w != nullptr, xs, ws, sq, cs, qa_s, da_s, misc);
#pragma unroll
    for (int ii = 0; ii < NI; ii++) {
      const int c = cb + 64 * ii + lane;
      const bool cv = c < nchunk;
      const int b = TYPE == kGgmlQ8_0 ? c >> 1 : c;
      uint4 a0 = make_uint4(0, 0, 0, 0), a1 = make_uint4(0, 0, 0, 0);
      float dact = 0.0f;
      if (cv) {
        if (TYPE == kGgmlQ8_0) {
          a0 = *(const uint4*)(qa_s + (size_t)c * 16);
        } else {
          a0 = *(const uint4*)(qa_s + (size_t)c * 32);
          a1 = *(const uint4*)(qa_s + (size_t)c * 32 + 16);
        }
        dact = da_s[b];
      }
      int asum = 0;
      if (TYPE != kGgmlQ8_0) {
        const uint32_t ones = 0x01010101u;
        asum = dot4(ones, a0.x, asum);
        asum = dot4(ones, a0.y, asum);
        asum = dot4(ones, a0.z, asum);
        asum = dot4(ones, a0.w, asum);
        asum = dot4(ones, a1.x, asum);
        asum = dot4(ones, a1.y, asum);
        asum = dot4(ones, a1.z, asum);
        asum = dot4(ones, a1.w, asum);
      }
#pragma unroll
      for (int r = 0; r < NR; r++) {
        int isum = 0;
        if (TYPE == kGgmlQ8_0) {
          isum = dot4(w4[ii][r].x, a0.x, isum);
          isum = dot4(w4[ii][r].y, a0.y, isum);
          isum = dot4(w4[ii][r].z, a0.z, isum);
          isum = dot4(w4[ii][r].w, a0.w, isum);
          isum += dpp_i32<kDppXor1>(isum);
        } else {
          const uint32_t m = 0x0f0f0f0fu;
          isum = dot4(w4[ii][r].x & m, a0.x, isum);
          isum = dot4(w4[ii][r].y & m, a0.y, isum);
          isum = dot4(w4[ii][r].z & m, a0.z, isum);
          isum = dot4(w4[ii][r].w & m, a0.w, isum);
          isum = dot4((w4[ii][r].x >> 4) & m, a1.x, isum);
          isum = dot4((w4[ii][r].y >> 4) & m, a1.y, isum);
          isum = dot4((w4[ii][r].z >> 4) & m, a1.z, isum);
          isum = dot4((w4[ii][r].w >> 4) & m, a1.w, isum);
          isum -= 8 * asum;
        }
        const bool writer = TYPE == kGgmlQ8_0 ? cv && !(c & 1) : cv;
        if (writer) mine[r * nbs + b] = (f16_to_f32(dsc[ii][r]) * dact) * (float)isum;
      }
    }
  }
  __syncthreads();
  if (lane < R) {
    if (PAIR) {
      const int row = row0 + lane;
      if (row < M.rows[0]) {
        const float g = chain_sum_lds(0.0f, mine + lane * nbs, nb);
        const float u = chain_sum_lds(0.0f, mine + (R + lane) * nbs, nb);
        const float v = silu_det(g) * u;
        if (!finite(g) || !finite(u) || !finite(v)) bad = true;
        M.out[0][(size_t)t * M.rows[0] + row] = v;
        if (QOUT) vq[wave * R + lane] = v;
      }
    } else {
      const int gr = row0 + lane;
      if (gr < M.total_rows) {
        const int mi = gr < M.row_end[0] ? 0 : (gr < M.row_end[1] ? 1 : 2);
        const int row = gr - (mi == 0 ? 0 : (mi == 1 ? M.row_end[0] : M.row_end[1]));
        float* out = mi == 0 ? M.out[0] : (mi == 1 ? M.out[1] : M.out[2]);
        const float* bias = mi == 0 ? M.bias[0] : (mi == 1 ? M.bias[1] : M.bias[2]);
        const int epi = mi == 0 ? M.epi[0] : (mi == 1 ? M.epi[1] : M.epi[2]);
        const int rows = mi == 0 ? M.rows[0] : (mi == 1 ? M.rows[1] : M.rows[2]);
        const float v = chain_sum_lds(0.0f, mine + lane * nbs, nb);
        (void)bias;
        if (!epilogue_pre(v, pre, out, (size_t)t * rows + row, epi)) bad = true;
      }
    }
  }
  if (QOUT) {
    // The workgroup's 32 rows are one Q8A block of the SwiGLU output
    // (quantize_q8a_into, det-quant lib.rs:111-137): lanes 0-31 of wave 0
    // form it, lanes 32-63 only take part in the reductions.
    __syncthreads();
    if (wave == 0) {
      const QuantOut q{in.out_qa, in.out_da, nullptr, nullptr, nullptr};
      quantize_q8a_lanes(lane < 32 ? vq[lane] : 0.0f, (size_t)t * M.rows[0] + (size_t)blockIdx.x * 32,
                         q, lane < 32);
    }
  }
  if (bad) flag(err, ERRBIT_NON_FINITE);
}

// ---------------------------------------------------------------------------
namespace {
template <int TYPE>
void launch_q8(const DevMat& W, const DevAct& A, int T, float* out, const float* bias, int epi,
               int* err, hipStream_t s, int R) {
  size_t smem = (size_t)4 * R * nb_stride(W.nb) * sizeof(float);
  dim3 grid((W.rows + 4 * R - 1) / (4 * R), T);
  if (R == 8)
    launch_kernel((k_gemv_q8<TYPE, 8>), grid, dim3(256), smem, s, W, A.qa, A.da, out, bias, epi, err);
  else if (R == 4)
    launch_kernel((k_gemv_q8<TYPE, 4>), grid, dim3(256), smem, s, W, A.qa, A.da, out, bias, epi, err);
  else if (R == 2)
    launch_kernel((k_gemv_q8<TYPE, 2>), grid, dim3(256), smem, s, W, A.qa, A.da, out, bias, epi, err);
  else
    launch_kernel((k_gemv_q8<TYPE, 1>), grid, dim3(256), smem, s, W, A.qa, A.da, out, bias, epi, err);
}
}  // namespace

bool launch_gemv(const DevMat& W, const DevAct& A, int T, float* out, const float* bias, int epi,
                 int* err, hipStream_t s) {
  if (W.type == kGgmlQ8_0 && W.nb <= 32 && W.rows >= 16384) {
    // Tall, narrow Q8_0 (the output projection): streaming waves, as many
    // workgroups as stay resident at once (a second round of workgroups
    // would start only when the first ones end, doubling the launch).
    constexpr int R = 4;
    const int ngroups = (W.rows + R - 1) / R;
    size_t smem = (size_t)4 * R * nb_stride(W.nb) * sizeof(float);
    static const int resident = [] {
      int dev = 0, cus = 0, per_cu = 0;
      if (hipGetDevice(&dev) != hipSuccess ||
          hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
          hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_gemv_q8_0_stream<R>, 256,
                                                       4 * R * 32 * sizeof(float)) != hipSuccess ||
          cus <= 0 || per_cu <= 0)
        return 256;
      return cus * per_cu;
    }();
    int wgs = (ngroups + 3) / 4;
    if (wgs > resident) wgs = resident;
    launch_kernel(k_gemv_q8_0_stream<R>, dim3(wgs, T), dim3(256), smem, s, W, A.qa, A.da, out,
                  bias, epi, err);
    return true;
  }
  if (W.type == kGgmlQ8_0 || W.type == kGgmlQ4_0) {
    // Rows per wave: enough waves to fill the chip on small matrices, more
    // rows per wave (fewer chain tails) on tall ones; LDS holds R*nb terms per wave.
    int R = W.rows >= 65536 ? 8 : (W.rows >= 16384 ? 4 : (W.rows >= 4096 ? 2 : 1));
    while (R > 1 && (size_t)4 * R * nb_stride(W.nb) * sizeof(float) > 64 * 1024) R >>= 1;
    if ((size_t)4 * R * nb_stride(W.nb) * sizeof(float) > 64 * 1024) return false;
    if (W.type == kGgmlQ8_0)
      launch_q8<kGgmlQ8_0>(W, A, T, out, bias, epi, err, s, R);
    else
      launch_q8<kGgmlQ4_0>(W, A, T, out, bias, epi, err, s, R);
    return true;
  }
  if (W.type == kGgmlQ6K && W.q6d) {
    launch_q6k_cm(W, A, T, out, bias, epi, err, s);
    return true;
  }
  // Split superblocks for the per-layer matrices (ffn_down: 11.9 -> 10.0 us
  // per launch); the tall output projection keeps k_gemv_q6k (24.6 us, the
  // split's one workgroup per row measured 29.1).
  if (W.type == kGgmlQ6K && W.nb <= 32 && W.rows <= 16384) {
    const int threads = (8 * W.nb + 63) / 64 * 64;
    launch_kernel(k_gemv_q6k_split, dim3(W.rows, T), dim3(threads), 0, s, W, A.qk, A.dk, out, bias,
                  epi, err);
    return true;
  }
  if (W.type == kGgmlQ6K) {
    if (W.nb > 64) return false;
    int rpw = 64 / W.nb;
    dim3 grid((W.rows + rpw - 1) / rpw, T);
    launch_kernel(k_gemv_q6k, grid, dim3(64), 0, s, W, A.qk, A.dk, out, bias, epi, err);
    return true;
  }
  if (W.type == kGgmlQ4K) {
    Q4kPcArgs a{static_cast<const uint8_t*>(W.w), nullptr, W.hdr, nullptr, W.nb,
                W.rows, 0, W.cols, T, A.af, nullptr, nullptr, 0.0f, nullptr, nullptr,
                nullptr, nullptr, 0, 0, nullptr, nullptr, 0, out, nullptr, bias, nullptr, epi, 0, err};
    if (launch_q4k_pc<PC_SINGLE>(a, s)) return true;
  }
  if (W.type == kGgmlQ4K && W.w32 && W.cols % 256 == 0) {
    // Rows per wave: the chain length fixes the time, so spread rows thin
    // enough to use every CU.
    dim3 grid8((W.rows + 7) / 8, T), grid32((W.rows + 31) / 32, T);
    if (W.rows <= 8192)
      launch_kernel(k_gemv_q4k<8>, grid8, dim3(64), 0, s, W.w32, W.rows, W.cols, A.af, out, bias, epi, err);
    else
      launch_kernel(k_gemv_q4k<32>, grid32, dim3(64), 0, s, W.w32, W.rows, W.cols, A.af, out, bias, epi, err);
    return true;
  }
  return false;
}

namespace {
template <int TYPE, bool PAIR>
void launch_q8f(const FusedMats& M, const FusedIn& in, int T, int R, bool norm, int* err,
                hipStream_t s) {
  const int nr = PAIR ? 2 * R : R;
  const int rows = PAIR ? M.rows[0] : M.total_rows;
  dim3 grid((rows + 4 * R - 1) / (4 * R), T);
  const size_t smem = gemv_fused_smem(nr, M.cols, M.nb, norm, 4);
  if constexpr (PAIR) {
    if (in.out_qa) {
      // two rows per wave, sixteen waves: one 32-row Q8A block per workgroup
      launch_kernel((k_gemv_q8f<TYPE, 2, true, true, 16>), dim3(rows / 32, T), dim3(1024),
                    gemv_fused_smem(4, M.cols, M.nb, norm, 16), s, M, in, err);
      return;
    }
  }
  if (R == 4)
    launch_kernel((k_gemv_q8f<TYPE, 4, PAIR>), grid, dim3(256), smem, s, M, in, err);
  else if (R == 2)
    launch_kernel((k_gemv_q8f<TYPE, 2, PAIR>), grid, dim3(256), smem, s, M, in, err);
  else
    launch_kernel((k_gemv_q8f<TYPE, 1, PAIR>), grid, dim3(256), smem, s, M, in, err);
}
}  // namespace

bool gemv_fused_fits(const DevMat* const* mats, int nm, bool pair_swiglu, bool norm, int T) {
  if (nm < 1 || nm > 3 || (pair_swiglu && nm != 2) || T < 1 || T > kGemvMaxT) return false;
  const DevMat& m0 = *mats[0];
  if (m0.type != kGgmlQ8_0 && m0.type != kGgmlQ4_0) return false;
  for (int i = 0; i < nm; i++) {
    const DevMat& m = *mats[i];
    if (m.type != m0.type || m.cols != m0.cols || m.nb != m0.nb) return false;
    if (pair_swiglu && m.rows != m0.rows) return false;
  }
  return m0.cols % 32 == 0 && gemv_fused_smem(pair_swiglu ? 2 : 1, m0.cols, m0.nb, norm, 4) <= 64 * 1024;
}

bool gemv_fused_pair_quantizes(const DevMat& gate, const DevMat& up, bool norm, int T) {
  const DevMat* mats[2] = {&gate, &up};
  return gemv_fused_fits(mats, 2, true, norm, T) && gate.rows % 32 == 0 &&
         gemv_fused_smem(4, gate.cols, gate.nb, norm, 16) <= 64 * 1024;
}

bool launch_gemv_fused(const DevMat* const* mats, int nm, bool pair_swiglu, float* const* outs,
                       const float* const* biases, const int* epis, const FusedIn& in, int T,
                       int* err, hipStream_t s) {
  const bool norm = in.norm_w != nullptr;
  if (!gemv_fused_fits(mats, nm, pair_swiglu, norm, T)) return false;
  const DevMat& m0 = *mats[0];
  FusedMats M{};
  int acc = 0;
  for (int i = 0; i < nm; i++) {
    const DevMat& m = *mats[i];
    if (m.type != m0.type || m.cols != m0.cols || m.nb != m0.nb) return false;
    if (pair_swiglu && m.rows != m0.rows) return false;
    M.w[i] = m.w;
    M.d16[i] = m.d16;
    M.rows[i] = m.rows;
    acc += m.rows;
    M.row_end[i] = acc;
    if (!pair_swiglu) {
      M.out[i] = outs[i];
      M.bias[i] = biases[i];
      M.epi[i] = epis[i];
    }
  }
  for (int i = nm; i < 3; i++) M.row_end[i] = acc;
  if (pair_swiglu) M.out[0] = outs[0];
  M.total_rows = acc;
  M.cols = m0.cols;
  M.nb = m0.nb;
  const int rows = pair_swiglu ? m0.rows : acc;
  // Rows per wave as the unfused kernel chooses them; LDS bounds the rest.
  int R = rows >= 16384 ? 4 : (rows >= 4096 ? 2 : 1);
  const int mult = pair_swiglu ? 2 : 1;
  if (in.out_qa && (!pair_swiglu || !gemv_fused_pair_quantizes(*mats[0], *mats[1], norm, T)))
    return false;
  while (R > 1 && gemv_fused_smem(mult * R, m0.cols, m0.nb, norm, 4) > 64 * 1024) R >>= 1;
  if (gemv_fused_smem(mult * R, m0.cols, m0.nb, norm, 4) > 64 * 1024) return false;
  if (m0.type == kGgmlQ8_0) {
    if (pair_swiglu) launch_q8f<kGgmlQ8_0, true>(M, in, T, R, norm, err, s);
    else launch_q8f<kGgmlQ8_0, false>(M, in, T, R, norm, err, s);
  } else {
    if (pair_swiglu) launch_q8f<kGgmlQ4_0, true>(M, in, T, R, norm, err, s);
    else launch_q8f<kGgmlQ4_0, false>(M, in, T, R, norm, err, s);
  }
  return true;
}

bool gemv_q4k_fit(const DevMat& W0, const DevMat* W1, bool pair, bool prologue, int T,
                  const DevMat* v6) {
  int RB, SL;
  size_t smem;
  if (T > kGemvMaxT || W0.type != kGgmlQ4K) return false;
  if (W1 && (W1->type != kGgmlQ4K || W1->cols != W0.cols || (pair && W1->rows != W0.rows)))
    return false;
  if (v6 && (!prologue || v6->type != kGgmlQ6K || v6->cols != W0.cols || v6->nb > 8)) return false;
  const int mode = pair ? PC_PAIR : (W1 ? PC_CAT : PC_SINGLE);
  const int rows = pair || !W1 ? W0.rows : W0.rows + W1->rows;
  int CR;
  if (!q4k_pc_plan(mode, rows, W0.cols, T, prologue, v6 != nullptr, &RB, &SL, &CR, &smem)) return false;
  return !v6 || ((rows + RB - 1) / RB) * (kPcThreads / 64 - kPcChainWaves) >= v6->rows;
}

bool launch_gemv_q4k(const DevMat& W0, const DevMat* W1, bool pair, const Q4kIn& in, int T,
                     float* out0, float* out1, const float* bias0, const float* bias1, int epi0,
                     int epi1, int* err, hipStream_t s) {
  if (!gemv_q4k_fit(W0, W1, pair, in.af == nullptr, T, in.v6)) return false;
  if (in.side_qk && (in.af || W0.cols % 256 != 0)) return false;
  const DevMat* v6 = in.v6;
  Q4kPcArgs a{static_cast<const uint8_t*>(W0.w), W1 ? static_cast<const uint8_t*>(W1->w) : nullptr,
              W0.hdr, W1 ? W1->hdr : nullptr, W0.nb, W0.rows, W1 && !pair ? W1->rows : 0, W0.cols, T,
              in.af, in.x, in.norm_w, in.eps, in.side_qk, in.side_dk,
              v6 ? static_cast<const uint32_t*>(v6->w) : nullptr, v6 ? v6->d16 : nullptr,
              v6 ? v6->rows : 0, v6 ? v6->nb : 0, in.v6out, in.v6bias, in.v6epi,
              out0, out1, bias0, bias1, epi0, epi1, err};
  if (pair) return launch_q4k_pc<PC_PAIR>(a, s);
  if (W1) return launch_q4k_pc<PC_CAT>(a, s);
  return launch_q4k_pc<PC_SINGLE>(a, s);
}

}  // namespace dtl
