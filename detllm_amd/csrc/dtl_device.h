// Device-side data layouts and kernel launchers shared by the library's
// translation units.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

namespace dtl {

// Kernel-boundary timing.  While a LaunchTiming is installed on the calling
// thread, launch_kernel binds `start` to the first kernel's start and `stop`
// to the last kernel's end (hipExtLaunchKernel events carry the kernels' own
// timestamps, so the interval excludes launch overhead).
struct LaunchTiming {
  hipEvent_t start, stop;
  bool launched;
};
extern thread_local LaunchTiming* tl_timing;

template <typename... KArgs, typename... Args>
inline void launch_kernel(void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t smem,
                          hipStream_t stream, Args&&... args) {
  if (LaunchTiming* lt = tl_timing) {
    hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)smem, stream,
                          lt->launched ? nullptr : lt->start, lt->stop, 0u,
                          std::forward<Args>(args)...);
    lt->launched = true;
  } else {
    hipLaunchKernelGGL(kernel, grid, block, smem, stream, std::forward<Args>(args)...);
  }
}

// Sticky device error bits, OR-ed into the session's flag word and read at
// synchronisation points (the reference returns the matching error on the
// first non-finite value it meets).
enum : int {
  ERRBIT_NON_FINITE = 1,         // ModelError::NonFinite
  ERRBIT_CDF_NON_FINITE = 2,     // CdfError::NonFiniteLogit
  ERRBIT_CDF_TOTAL = 4,          // CdfError::TotalTooLarge
  ERRBIT_CDF_LOOKUP = 8,         // decoder value outside every symbol
  ERRBIT_CDF_SYMBOL = 16,        // CdfError::SymbolOutOfRange (symbols held on the device)
};

// One weight matrix in device layout.  Values are the GGUF values exactly;
// only the byte arrangement changes so that rows stream with wide loads:
//   F32  : w = float[rows][cols]
//   Q8_0 : w = int8[rows][cols],          d16 = f16[rows][cols/32]
//   Q4_0 : w = uint8[rows][cols/32][16],  d16 = f16[rows][cols/32]
//   Q4_K : w = uint8[rows][cols/256][128] (nibbles), hdr = uint8[rows][cols/256][16]
//          ({f16 d, f16 dmin, u8 scales[12]})
//   Q6_K : w = uint8[rows][cols/256][208] ({ql[128], qh[64], i8 scales[16]}),
//          d16 = f16[rows][cols/256]
struct DevMat {
  int32_t type;
  int32_t rows;
  int32_t cols;
  int32_t nb;  // blocks per row (32-element for Q8_0/Q4_0, 256 for K types, cols for F32)
  const void* w;
  const uint16_t* d16;
  const uint8_t* hdr;
  // Q4_K only (optional): float[rows][cols] holding q4_k_value of every
  // element, used by the chunked-encode GEMM as scalar-path operands.
  const float* w32;
  // Q6_K only (optional): the int8 matrix-core operands of the chunked-encode
  // GEMM.  For 16-row tile rt, superblock sb, class c (element index mod 8)
  // and plane p, 512 bytes at (((rt*nb + sb)*8 + c)*2 + p)*512 hold, for
  // row r of the tile, bytes [r*32, r*32+32): W' = scale*q6 of elements
  // 8j + c (j = 0..31) split as W' = 64*hi + lo (p = 0: hi in [-64, 64],
  // p = 1: lo in [0, 63]).  Rows are padded with zeros to a multiple of 16.
  const int8_t* planes;
  // Q4_0 only (optional): int8[rows][cols], nibble - 8 of every element in
  // element order, the A operand of the chunked-encode GEMM on the int8
  // matrix cores (Q8_0 uses w itself).
  const int8_t* i8;
  // Q6_K only (tall matrices whose superblocks per row divide 16): the
  // decode GEMV's layout of the 208-byte bodies (q6k_decode_layout_*).
  const uint4* q6d;
};

// Q6_K decode layout.  Inside a superblock the 208 body bytes are re-cut
// into 13 words of 16 bytes with the 6-bit quants class-major (class c =
// element index mod 8, elements c + 8j, j = 0..31): for class pair p
// (classes 2p, 2p + 1), word (p, 0) holds the low nibbles of class 2p and
// word (p, 1) those of class 2p + 1 (dword k, byte i: j = 8k + i in bits
// 0-3, j = 8k + 4 + i in bits 4-7), word (p, 2) their high bit pairs (dwords
// 0-1 for class 2p, 2-3 for 2p + 1; dword k, byte i: j = 16k + 4m + i in
// bits 2m, 2m + 1); the 16 scales are the 13th word.  16 consecutive (row,
// superblock) pairs form a group (16 / nb rows, superblock s = row % (16 /
// nb) * nb + superblock) of 13 * 16 words: word (p, k) of superblock s at
// group * 208 + k * 64 + s * 4 + p, the scales at group * 208 + 192 + s, so
// that the wave load of word k of the group's 16 * 4 (superblock, class
// pair) lanes reads one contiguous KiB.  Superblocks past the last row are
// zero.
constexpr int kQ6dGroupWords = 208;
inline bool q6k_decode_layout_applies(const DevMat& W) {
  return W.nb > 0 && 16 % W.nb == 0 && W.rows > 16384;
}
inline size_t q6k_decode_layout_bytes(const DevMat& W) {
  const size_t rpg = 16 / (size_t)W.nb, groups = ((size_t)W.rows + rpg - 1) / rpg;
  return groups * kQ6dGroupWords * 16;
}
void launch_q6k_decode_layout(const DevMat& W, uint4* out, hipStream_t s);

// Activations of T positions for one GEMM input of width cols, in every
// form a weight type consumes (det-quant Q8A for Q8_0/Q4_0/Q4_K, Q8_K for Q6_K).
struct DevAct {
  const float* x;    // [T][cols] raw f32 (F32 weights)
  const int8_t* qa;  // [T][cols]      Q8A quants
  const float* da;   // [T][cols/32]   Q8A scales
  const float* af;   // [T][cols]      Q8A dequantised: da * qa (Q4_K chain input)
  const int8_t* qk;  // [T][cols]      Q8_K quants
  const float* dk;   // [T][cols/256]  Q8_K scales
  // Other chunks' launches share the chip with this one (the pipelined
  // encode): the GEMMs then pick tiles for an occupied chip.
  bool overlapped = false;
};

enum GemmEpilogue : int { EPI_STORE = 0, EPI_BIAS = 1, EPI_RESIDUAL = 2 };

// Q4_K chunk GEMMs from the exact f32 weight copy (the values q4_k_value
// yields, det-quant lib.rs:506-517), every output one chain of products in
// element order:
//   MODE_SINGLE  one matrix
//   MODE_PAIR    gate and up (same shape): silu(gate)*up (det-model
//                lib.rs:2420-2434) written in the epilogue
//   MODE_CAT     two matrices with the same input (e.g. wq and wk), their
//                rows concatenated into one grid, separate outputs
enum { MODE_SINGLE = 0, MODE_PAIR = 1, MODE_CAT = 2 };

struct Q4kF32Args {
  const float* w0;
  const float* w1;
  int rows0, rows1, cols;
  const float* af;
  int T;
  float* out0;
  float* out1;
  float* ffo;
  const float* bias0;
  const float* bias1;
  int epi;
  int* err;
};

// The products on the matrix cores (k_q4k_mfp, dtl_mfp.hip), and the probe
// of their inner pattern's rate.
void launch_q4k_mfp(const Q4kF32Args& a, int mode, hipStream_t s);
void launch_mfp_probe(float* out, int workgroups, int iters, hipStream_t s);

// Positions up to which the decode GEMVs (one weight pass per position)
// replace the chunked-encode GEMMs.
constexpr int kGemvMaxT = 8;

// Matrices of one fused decode GEMV launch (same type, cols and input).
struct FusedMats {
  const void* w[3];
  const uint16_t* d16[3];
  float* out[3];
  const float* bias[3];
  int epi[3];
  int rows[3];
  int row_end[3];  // prefix sums of rows (concatenated launches)
  int total_rows;
  int cols, nb;
};

// Input of a fused decode GEMV: f32 rows [T][cols], normalised first when
// norm_w is set.  out_qa / out_da (gate/up pair only): also write the Q8A
// form of the SwiGLU output (the next projection's input), [T][rows] and
// [T][rows / 32]; gemv_fused_pair_quantizes says when a pair can.
struct FusedIn {
  const float* x;
  const float* norm_w;
  float eps;
  int8_t* out_qa = nullptr;
  float* out_da = nullptr;
};

// ---- launchers (dtl_kernels.hip) -------------------------------------------
void launch_embed(const DevMat& E, const uint32_t* tokens, int T, float* x, int* err,
                  hipStream_t s);
void launch_rmsnorm(const float* x, const float* w, float eps, int T, int n, float* out, int* err,
                    hipStream_t s);
// rmsnorm followed by the activation quantisation of the normalised row, in
// one pass (out keeps the f32 row).
void launch_rmsnorm_quant(const float* x, const float* w, float eps, int T, int n, float* out,
                          bool want_q8a, bool want_q8k, int8_t* qa, float* da, float* af,
                          int8_t* qk, float* dk, int* err, hipStream_t s);
// want_q8a / want_q8k select which quantisations to produce.
void launch_quantize(const float* x, int T, int n, bool want_q8a, bool want_q8k, int8_t* qa,
                     float* da, float* af, int8_t* qk, float* dk, int* err, hipStream_t s);
void launch_gemm(const DevMat& W, const DevAct& A, int T, float* out, const float* bias, int epi,
                 int* err, hipStream_t s);
// Decode GEMVs (dtl_gemv.hip) for a few positions; false when the matrix
// shape or type has no GEMV kernel.
bool launch_gemv(const DevMat& W, const DevAct& A, int T, float* out, const float* bias, int epi,
                 int* err, hipStream_t s);
// Q8_0 / Q4_0 decode GEMV with its activation quantisation (and rmsnorm when
// in.norm_w is set) fused in: nm matrices over concatenated rows, or gate and
// up (nm == 2, pair_swiglu) whose dots finish as swiglu into outs[0].
// Returns false when the shapes do not fit (the caller uses separate launches).
bool gemv_fused_fits(const DevMat* const* mats, int nm, bool pair_swiglu, bool norm, int T);
bool gemv_fused_pair_quantizes(const DevMat& gate, const DevMat& up, bool norm, int T);
bool launch_gemv_fused(const DevMat* const* mats, int nm, bool pair_swiglu, float* const* outs,
                       const float* const* biases, const int* epis, const FusedIn& in, int T,
                       int* err, hipStream_t s);
// Q4_K decode GEMVs (T <= kGemvMaxT) with the products and chains split:
// one matrix (W1 null), two over concatenated rows with the same input (wq
// and wk: each its own output, bias and epilogue), or gate and up (pair)
// finishing as silu(gate) * up into out0.  The input is either the Q8A
// values (in.af) or the raw f32 rows the kernel normalises (in.norm_w) and
// quantises itself (in.x).  false (nothing launched) when the shapes or
// types do not qualify.
struct Q4kIn {
  const float* af;
  const float* x;
  const float* norm_w;
  float eps;
  int8_t* side_qk = nullptr;  // with x: also the input's Q8_K form (for a Q6_K consumer)
  float* side_dk = nullptr;
  // with x: a Q6_K matrix over the same normed input computed in the same
  // launch (at most eight superblocks per row), its output, bias and epilogue
  const DevMat* v6 = nullptr;
  float* v6out = nullptr;
  const float* v6bias = nullptr;
  int v6epi = 0;
};
bool gemv_q4k_fit(const DevMat& W0, const DevMat* W1, bool pair, bool prologue, int T,
                  const DevMat* v6 = nullptr);
bool launch_gemv_q4k(const DevMat& W0, const DevMat* W1, bool pair, const Q4kIn& in, int T,
                     float* out0, float* out1, const float* bias0, const float* bias1, int epi0,
                     int epi1, int* err, hipStream_t s);
// Token-parallel GEMMs (dtl_gemm.hip) for chunks of positions.
bool gemm_tok_supported(const DevMat& W);
void launch_gemm_tok(const DevMat& W, const DevAct& A, int T, float* out, const float* bias,
                     int epi, int* err, hipStream_t s);
// Fills out[rows*cols] with the exact f32 value of every Q4_K weight.
void launch_dequant_q4k(const DevMat& W, float* out, hipStream_t s);
// Bytes of the Q6_K matrix-core planes of W (see DevMat::planes).
size_t q6k_planes_bytes(const DevMat& W);
// Fills planes (q6k_planes_bytes(W) bytes) from W's Q6_K superblocks.
void launch_q6k_planes(const DevMat& W, int8_t* planes, hipStream_t s);
// Fills out (rows * cols bytes) with the int8 values of W's Q4_0 blocks.
void launch_q4_0_i8(const DevMat& W, int8_t* out, hipStream_t s);
// Two Q4_K matrices with the same input and column count (wq, wk) in one
// launch of at least 16 positions, each with its own output, bias and
// epilogue; false (nothing launched) when the pair does not qualify.
bool launch_gemm_cat_q4k(const DevMat& W0, const DevMat& W1, const DevAct& A, int T, float* out0,
                         float* out1, const float* bias0, const float* bias1, int epi, int* err,
                         hipStream_t s);
// gate and up (both Q4_K, same shape) in one pass with silu(gate)*up written to ffo.
void launch_gemm_pair_swiglu_q4k(const DevMat& G, const DevMat& U, const DevAct& A, int T, float* g,
                                 float* u, float* ffo, int* err, hipStream_t s);
// pos_dev (optional): device int holding pos0, read by the kernels instead of
// the pos0 argument (lets one captured graph serve every position).
void launch_rope_store(float* q, float* k, const float* v, const float* rope_cos,
                       const float* rope_sin, int T, int pos0, int H, int KV, int hd, int rope_dim,
                       int split_half, float* kc, float* vc, int layer, int n_ctx,
                       const int* pos_dev, int* err, hipStream_t s);
// The chunk's raw keys / values and RoPE tables for the decode attention,
// which applies RoPE and stores the chunk's cache rows itself.
struct RopeIn {
  const float* k;  // [T][KV][hd] keys before RoPE
  const float* v;  // [T][KV][hd] values
  const float* rc;  // [n_ctx][rope_dim / 2] cos / sin tables
  const float* rs;
  int rope_dim;
  int split_half;
  float* kc;  // [layer][KV][n_ctx][hd] caches
  float* vc;
};
// Whether launch_attention_dec takes this shape (hd 64, at most four
// positions, the score row within LDS).
bool attention_dec_applies(int hd, int T, int pos0, int n_ctx, bool pos_in_device);
// Rows up to this many keys run the decode attention in one launch (scores
// in LDS); longer rows run the split pair (scores through memory).
int attention_fused_max_len();
// scores: scratch of T * H * n_ctx floats.  maxlen_dev: with pos_dev, the
// longest row (pos + 1) the launches may see; the caller keeps every
// position it copies to pos_dev below it.
void launch_attention_dec(const float* q, const RopeIn& R, int layer, int T, int pos0, int H,
                          int KV, int n_ctx, int maxlen_dev, float scale, float* scores, float* out,
                          const int* pos_dev, int* err, hipStream_t s);
// Whether the decode attention (launch_attention_dec) takes the position
// from device memory for this shape (graph replay of single-position forwards).
bool attention_pos_dev_supported(int hd, int T, int n_ctx);
// Whether launch_attention writes the Q8A form of its output itself (the
// chunked kernel, when qa / da / af are passed).
bool attention_quantizes_q8a(int hd, int H, int KV, int T, int pos0, int n_ctx);
void launch_attention(const float* q, const float* kc, const float* vc, int layer, int T, int pos0,
                      int H, int KV, int hd, int n_ctx, float scale, float* scores, float* out,
                      int* err, hipStream_t s, int8_t* qa = nullptr, float* da = nullptr,
                      float* af = nullptr);
void launch_swiglu(const float* g, const float* u, int count, float* out, int* err, hipStream_t s);
void launch_rope_table(float base, int rope_dim, int positions, float* cos_out, float* sin_out,
                       int* err, hipStream_t s);

// CDF over rows of logits [R][V].
//   mode 0: symbol range for symbols[r]        -> cum[r], freq[r], total[r]
//   mode 1: full table for one row             -> freq_tab[V+tail], cum_tab[V+tail], total[0]
//   mode 2: decoder lookup of values[r]        -> sym[r], cum[r], freq[r], total[r]
//   mode 3: decoder total only                 -> total[r]
void launch_cdf(const float* logits, int R, int V, int tail, int mode, const uint32_t* symbols,
                const uint64_t* values, uint64_t* cum, uint32_t* freq, uint64_t* total,
                uint32_t* sym, uint32_t* freq_tab, uint64_t* cum_tab, int* err, hipStream_t s);

// Modes 0, 2 and 3 of launch_cdf spread over many workgroups per row;
// scratch holds cdf_scratch_bytes(R, V) bytes of device memory.  rows
// (device, optional): row r of the launch is logits row rows[r].
// finish_only: the scratch already holds this row's block results (a
// decoder total for the same row and tail): only the per-row finish runs.
constexpr size_t kCdfBlockElems = 4096;  // logits per workgroup of the block kernels
constexpr size_t cdf_scratch_bytes_for(size_t R, size_t V) {
  // per row: block maxima (f32), exps chain-major (8 x v8 f32, v8 = V/8
  // rounded up to a multiple of 4), Z, block sums and sums below (u64),
  // the symbol's frequency; + 256 for the 16-byte rounding of each part
  return R * (((V + kCdfBlockElems - 1) / kCdfBlockElems) * 4 + 8 * ((((V + 7) / 8) + 3) & ~(size_t)3) * 4 + 4 +
              ((V + kCdfBlockElems - 1) / kCdfBlockElems) * 16 + 4) +
         256;
}
size_t cdf_scratch_bytes(int R, int V);
void launch_cdf_blocks(const float* logits, const uint32_t* rows, int R, int V, int tail, int mode,
                       const uint32_t* symbols, const uint64_t* values, uint64_t* cum,
                       uint32_t* freq, uint64_t* total, uint32_t* sym, void* scratch,
                       bool finish_only, int* err, hipStream_t s);
// One row's decoder step: the block pass, then the lookup of the value
// RangeDecoder::decode_freq forms from the decoder's window (cml = code -
// low, rng = range) against the row's total.  pack[0..6]: symbol, cum, freq,
// total, error bits (with those already set in *err), value, valid.
void launch_cdf_decode(const float* logits, int V, int tail, uint64_t cml, uint64_t rng, void* scratch,
                       uint64_t* pack, int* err, hipStream_t s);

// Kernel-level parity entry points.
void launch_exp_f32(const float* in, float* out, int n, int which, hipStream_t s);
void launch_f16_to_f32(const uint16_t* in, float* out, int n, hipStream_t s);
void launch_div_sqrt(const float* a, const float* b, float* q, float* r, int n, hipStream_t s);
// 1024-thread workgroups of 16 VALU instructions (8 f32 multiplies, 8 f32
// adds, independent chains) per iteration per lane.
void launch_valu_probe(float* out, int workgroups, int iters, hipStream_t s);

}  // namespace dtl
