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

namespace dtl {

namespace {

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

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Sequential sum of n block terms (block order), from LDS.
__device__ __forceinline__ float chain_sum(const float* v, int n) {
  float s = 0.0f;
  int b = 0;
  for (; b + 4 <= n; b += 4) {
    s += v[b];
    s += v[b + 1];
    s += v[b + 2];
    s += v[b + 3];
  }
  for (; b < n; b++) s += v[b];
  return s;
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
  float* mine = vb + (size_t)wave * R * nb;
  const int8_t* arow = qa + (size_t)t * cols;
  const float* drow = da + (size_t)t * nb;
  // Q8_0: a 32-byte block is two 16-byte chunks (lanes c, c^1); Q4_0: one
  // 16-byte block of nibbles per lane.
  const int nchunk = TYPE == kGgmlQ8_0 ? 2 * nb : nb;
  for (int c0 = 0; c0 < nchunk; c0 += 64) {
    const int c = c0 + lane;
    const bool cv = c < nchunk;
    const int b = TYPE == kGgmlQ8_0 ? c >> 1 : c;
    // Every load of this chunk column (R weight chunks, their block scales,
    // the activation and its scale) is issued before any arithmetic.
    uint4 w4[R];
    uint16_t dsc[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int row = row0 + r < rows ? row0 + r : rows - 1;
      w4[r] = make_uint4(0, 0, 0, 0);
      dsc[r] = 0;
      if (cv) {
        if (TYPE == kGgmlQ8_0)
          w4[r] = *(const uint4*)((const int8_t*)W.w + (size_t)row * cols + (size_t)c * 16);
        else
          w4[r] = *(const uint4*)((const uint8_t*)W.w + ((size_t)row * nb + c) * 16);
        dsc[r] = W.d16[(size_t)row * nb + b];
      }
    }
    uint4 a0 = make_uint4(0, 0, 0, 0), a1 = make_uint4(0, 0, 0, 0);
    float dact = 0.0f;
    if (cv) {
      if (TYPE == kGgmlQ8_0) {
        a0 = *(const uint4*)(arow + (size_t)c * 16);
      } else {
        a0 = *(const uint4*)(arow + (size_t)c * 32);
        a1 = *(const uint4*)(arow + (size_t)c * 32 + 16);
      }
      dact = drow[b];
    }
    int asum = 0;
    if (TYPE != kGgmlQ8_0) {
      // Q4_0 nibbles are offset by 8: isum = sum(lo*a) + sum(hi*a') - 8*sum(a).
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
    for (int r = 0; r < R; r++) {
      int isum = 0;
      if (TYPE == kGgmlQ8_0) {
        isum = dot4(w4[r].x, a0.x, isum);
        isum = dot4(w4[r].y, a0.y, isum);
        isum = dot4(w4[r].z, a0.z, isum);
        isum = dot4(w4[r].w, a0.w, isum);
        isum += __shfl_xor(isum, 1);
      } else {
        const uint32_t m = 0x0f0f0f0fu;
        isum = dot4(w4[r].x & m, a0.x, isum);
        isum = dot4(w4[r].y & m, a0.y, isum);
        isum = dot4(w4[r].z & m, a0.z, isum);
        isum = dot4(w4[r].w & m, a0.w, isum);
        isum = dot4((w4[r].x >> 4) & m, a1.x, isum);
        isum = dot4((w4[r].y >> 4) & m, a1.y, isum);
        isum = dot4((w4[r].z >> 4) & m, a1.z, isum);
        isum = dot4((w4[r].w >> 4) & m, a1.w, isum);
        isum -= 8 * asum;
      }
      const bool writer = TYPE == kGgmlQ8_0 ? cv && !(c & 1) : cv;
      if (writer && row0 + r < rows) mine[r * nb + b] = (f16_to_f32(dsc[r]) * dact) * (float)isum;
    }
  }
  __syncthreads();
  if (lane < R) {
    const int row = row0 + lane;
    if (row < rows) {
      float v = chain_sum(mine + lane * nb, nb);
      if (!epilogue(v, out, (size_t)t * rows + row, bias, row, epi)) flag(err, ERRBIT_NON_FINITE);
    }
  }
}

// ---------------------------------------------------------------------------
// Q8_0 streaming variant for tall matrices with at most 1024 columns (the
// output projection of the small-vocabulary-heavy shapes): every wave walks
// groups of R rows in a grid-stride loop, loading the next group's weights
// and scales while it reduces the current one, so HBM sees a steady stream
// rather than one burst per wave.  Lane c owns 16-byte chunk c of every row
// (nchunk <= 64), so the activation chunk is loaded once per wave.
template <int R>
__global__ void __launch_bounds__(256) k_gemv_q8_0_stream(DevMat W, const int8_t* __restrict__ qa,
                                                          const float* __restrict__ da, float* out,
                                                          const float* bias, int epi, int* err) {
  extern __shared__ __align__(16) float vb[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.y;
  const int rows = W.rows, cols = W.cols, nb = W.nb;
  const int nchunk = 2 * nb;
  const int c = lane, b = c >> 1;
  const bool cv = c < nchunk;
  float* mine = vb + (size_t)wave * R * nb;
  const int ngroups = (rows + R - 1) / R;
  const int stride = gridDim.x * 4;
  uint4 a0 = make_uint4(0, 0, 0, 0);
  float dact = 0.0f;
  if (cv) {
    a0 = *(const uint4*)(qa + (size_t)t * cols + (size_t)c * 16);
    dact = da[(size_t)t * nb + b];
  }
  uint4 w4[2][R];
  uint16_t dsc[2][R];
  auto load = [&](int slot, int g) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      int row = g * R + r;
      row = row < rows ? row : rows - 1;
      w4[slot][r] = make_uint4(0, 0, 0, 0);
      dsc[slot][r] = 0;
      if (cv) {
        w4[slot][r] = *(const uint4*)((const int8_t*)W.w + (size_t)row * cols + (size_t)c * 16);
        dsc[slot][r] = W.d16[(size_t)row * nb + b];
      }
    }
  };
  auto reduce = [&](int slot, int g) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      int isum = 0;
      isum = dot4(w4[slot][r].x, a0.x, isum);
      isum = dot4(w4[slot][r].y, a0.y, isum);
      isum = dot4(w4[slot][r].z, a0.z, isum);
      isum = dot4(w4[slot][r].w, a0.w, isum);
      isum += __shfl_xor(isum, 1);
      if (cv && !(c & 1)) mine[r * nb + b] = (f16_to_f32(dsc[slot][r]) * dact) * (float)isum;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    if (lane < R) {
      const int row = g * R + lane;
      if (row < rows) {
        float v = chain_sum(mine + lane * nb, nb);
        if (!epilogue(v, out, (size_t)t * rows + row, bias, row, epi)) flag(err, ERRBIT_NON_FINITE);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    __builtin_amdgcn_wave_barrier();
  };
  int g = blockIdx.x * 4 + wave;
  if (g >= ngroups) return;
  load(0, g);
  for (;;) {
    const int gn = g + stride;
    if (gn < ngroups) load(1, gn);
    reduce(0, g);
    if (gn >= ngroups) break;
    g = gn;
    const int gn2 = g + stride;
    if (gn2 < ngroups) load(0, gn2);
    reduce(1, g);
    if (gn2 >= ngroups) break;
    g = gn2;
  }
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
  if (lane < rpw && blockIdx.x * rpw + lane < rows) {
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
namespace {
template <int TYPE>
void launch_q8(const DevMat& W, const DevAct& A, int T, float* out, const float* bias, int epi,
               int* err, hipStream_t s, int R) {
  size_t smem = (size_t)4 * R * W.nb * sizeof(float);
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
    // workgroups as stay resident (four per CU at this kernel's occupancy).
    constexpr int R = 8;
    const int ngroups = (W.rows + R - 1) / R;
    int wgs = (ngroups + 3) / 4;
    if (wgs > 256 * 4) wgs = 256 * 4;
    size_t smem = (size_t)4 * R * W.nb * sizeof(float);
    launch_kernel(k_gemv_q8_0_stream<R>, dim3(wgs, T), dim3(256), smem, s, W, A.qa, A.da, out,
                  bias, epi, err);
    return true;
  }
  if (W.type == kGgmlQ8_0 || W.type == kGgmlQ4_0) {
    // Rows per wave: enough waves to fill the chip on small matrices, more
    // rows per wave (fewer chain tails) on tall ones; LDS holds R*nb terms per wave.
    int R = W.rows >= 65536 ? 8 : (W.rows >= 16384 ? 4 : (W.rows >= 4096 ? 2 : 1));
    while (R > 1 && (size_t)4 * R * W.nb * sizeof(float) > 64 * 1024) R >>= 1;
    if ((size_t)4 * R * W.nb * sizeof(float) > 64 * 1024) return false;
    if (W.type == kGgmlQ8_0)
      launch_q8<kGgmlQ8_0>(W, A, T, out, bias, epi, err, s, R);
    else
      launch_q8<kGgmlQ4_0>(W, A, T, out, bias, epi, err, s, R);
    return true;
  }
  if (W.type == kGgmlQ6K) {
    if (W.nb > 64) return false;
    int rpw = 64 / W.nb;
    dim3 grid((W.rows + rpw - 1) / rpw, T);
    launch_kernel(k_gemv_q6k, grid, dim3(64), 0, s, W, A.qk, A.dk, out, bias, epi, err);
    return true;
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

}  // namespace dtl
