// Device numerics for gfx950: bit-exact restatements of the detllm CPU
// arithmetic.  Every routine uses only IEEE-754 operations that the device
// rounds exactly like the host (add, sub, mul, correctly rounded div and
// sqrt, conversions); the translation units are compiled with
// -ffp-contract=off so no multiply-add is ever fused.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dtl {

__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ double u2d(uint64_t u) { return __longlong_as_double((long long)u); }
__device__ __forceinline__ uint64_t d2u(double d) { return (uint64_t)__double_as_longlong(d); }

__device__ __forceinline__ bool finite(float x) { return (f2u(x) & 0x7f800000u) != 0x7f800000u; }
// Whether any argument is Inf/NaN, without short-circuit branches (so the
// loads behind the arguments are not serialised).
__device__ __forceinline__ bool any_nonfinite(float a, float b) {
  return ((int)!finite(a) | (int)!finite(b)) != 0;
}
__device__ __forceinline__ bool any_nonfinite(float a, float b, float c, float d) {
  return ((int)!finite(a) | (int)!finite(b) | (int)!finite(c) | (int)!finite(d)) != 0;
}

// Rust `f32 as i32`: truncation toward zero, saturating, NaN -> 0.  Written
// with selects (no branches): the conversion sees a value clamped into
// [-2^31, largest float below 2^31], which truncates exactly as the
// unclamped in-range value would, and the two out-of-range cases and NaN
// are selected afterwards.
__device__ __forceinline__ int32_t f32_as_i32(float x) {
  const float xc = fminf(fmaxf(x, -2147483648.0f), 2147483520.0f);
  int32_t r = (int32_t)xc;
  r = x >= 2147483648.0f ? INT32_MAX : r;
  return x != x ? 0 : r;
}

// f16 bits -> f32 by integer construction (det-num f16.rs:6-34); exact for
// every input including subnormals, independent of the hardware f16 mode.
// Written with selects: a subnormal f16 is frac * 2^-24 (exact in f32), a
// normal one rebiases its exponent, Inf / NaN keep their fraction.
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  const uint32_t frac = h & 0x3ffu;
  const uint32_t normal = sign | ((exp + 112u) << 23) | (frac << 13);
  const uint32_t sub = sign | f2u((float)frac * 0x1p-24f);
  const uint32_t special = sign | 0x7f800000u | (frac << 13);
  return u2f(exp == 0 ? sub : (exp == 0x1f ? special : normal));
}

// 8-lane finishing tree (det-num reduce.rs:36-38).
__device__ __forceinline__ float finish_8lane(const float a[8]) {
  return ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
}

// scalbnf with the two-step range handling of det-num vendored_libm.rs:94-119,
// written with selects: the upward steps apply when the original n is above
// 127, the downward ones when it is below -126, each step exactly as the
// branches take it.
__device__ __forceinline__ float scalbnf(float x, int n) {
  const float x1p127 = u2f(0x7f000000u);
  const float x1p_126 = u2f(0x00800000u);
  const int n0 = n;
  const bool up1 = n0 > 127;
  x = up1 ? x * x1p127 : x;
  n = up1 ? n - 127 : n;
  const bool up2 = up1 && n > 127;
  x = up2 ? x * x1p127 : x;
  n = up2 ? n - 127 : n;
  n = up2 && n > 127 ? 127 : n;
  const bool dn1 = n0 < -126;
  x = dn1 ? x * x1p_126 : x;
  n = dn1 ? n + 126 : n;
  const bool dn2 = dn1 && n < -126;
  x = dn2 ? x * x1p_126 : x;
  n = dn2 ? n + 126 : n;
  n = dn2 && n < -126 ? -126 : n;
  return x * u2f((uint32_t)(0x7f + n) << 23);
}

// v / d rounded to nearest, given rd = 1 / d rounded to nearest: q0 = v rd,
// then one fma correction, q0 + (v - q0 d) rd (Markstein's theorem: with rd
// correctly rounded and q0 within an ulp of the quotient, the corrected
// value is the rounded quotient while nothing underflows).  Three
// instructions where the division takes about ten, for a caller that
// divides by one d many times.  tests/div_recip_check.c compares it with
// the division over its caller's operands (the Q8A quantiser's).
__device__ __forceinline__ float div_recip(float v, float d, float rd) {
  const float q0 = v * rd;
  const float r = __builtin_fmaf(-q0, d, v);
  return __builtin_fmaf(r, rd, q0);
}

// exp_f32 (det-num math.rs:5-7): the FreeBSD e_expf method restated from
// its published description -- round x/ln2 to k, reduce with a two-part
// ln2, approximate with x*c/(2-c), c = x - x^2(P1 + x^2 P2), scale by 2^k.
//
// Every path is computed and the result selected, so a wave of mixed inputs
// runs one straight sequence (the branches of the method became selects;
// each path's arithmetic is unchanged).
__device__ __forceinline__ float expf_det(float x) {
  const float ln2_hi = u2f(0x3f317200u);
  const float ln2_lo = u2f(0x35bfbe8eu);
  const float inv_ln2 = u2f(0x3fb8aa3bu);
  const float p1 = u2f(0x3e2aaa8fu);
  const float p2 = u2f(0xbb355215u);
  const uint32_t ux = f2u(x);
  const int sign = (int)(ux >> 31);
  const uint32_t hx = ux & 0x7fffffffu;
  // |x| > 0.5 ln2: reduce by k ln2 (k from the rounding of x / ln2 above
  // 1.5 ln2, else +-1)
  const int kr = hx > 0x3f851592u ? f32_as_i32(inv_ln2 * x + (sign ? -0.5f : 0.5f)) : 1 - sign - sign;
  const float kf = (float)kr;
  const float hi_r = x - kf * ln2_hi;
  const float lo_r = kf * ln2_lo;
  const bool reduce = hx > 0x3eb17218u;
  const int k = reduce ? kr : 0;
  const float hi = reduce ? hi_r : x;
  const float lo = reduce ? lo_r : 0.0f;
  const float xr = reduce ? hi_r - lo_r : x;
  const float xx = xr * xr;
  const float c = xr - xx * (p1 + xx * p2);
  const float y = 1.0f + (xr * c / (2.0f - c) - lo + hi);
  float r = k == 0 ? y : scalbnf(y, k);
  r = hx > 0x39000000u ? r : 1.0f + x;  // |x| < 2^-14
  // special cases, lowest priority first
  r = sign && hx >= 0x42cff1b5u ? 0.0f : r;                 // underflow
  r = !sign && hx >= 0x42b17218u ? x * u2f(0x7f000000u) : r;  // overflow
  return hx > 0x7f800000u ? x : r;                          // NaN
}

// a + v[0] + v[1] + ... + v[n - 1], one add at a time in that order, from
// 16-byte aligned LDS.  The serial chain waits on its own adds, not on LDS:
// whole float4 go through a ring of twelve reads issued twelve float4 ahead
// of their adds (the slot's adds first, then its refill into the same
// registers, so a loop-carried ring needs no copies; the scheduling barrier
// keeps each refill where it is).  The last n % 4 terms are added singly.
__device__ __forceinline__ float chain_sum_lds(float a, const float* v, int n) {
  constexpr int kRing = 12;
  const float4* v4 = reinterpret_cast<const float4*>(v);
  const int n4 = n >> 2;
  int q4 = 0;
  if (n4 >= kRing) {
    float4 r[kRing];
#pragma unroll
    for (int q = 0; q < kRing; q++) r[q] = v4[q];
    for (; q4 + 2 * kRing <= n4; q4 += kRing) {
#pragma unroll
      for (int q = 0; q < kRing; q++) {
        a += r[q].x;
        a += r[q].y;
        a += r[q].z;
        a += r[q].w;
        r[q] = v4[q4 + kRing + q];
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int q = 0; q < kRing; q++) {
      a += r[q].x;
      a += r[q].y;
      a += r[q].z;
      a += r[q].w;
    }
    q4 += kRing;
  }
  for (; q4 < n4; q4++) {
    const float4 w = v4[q4];
    a += w.x;
    a += w.y;
    a += w.z;
    a += w.w;
  }
  for (int i = 4 * n4; i < n; i++) a += v[i];
  return a;
}

// chain_sum_lds for n <= 32 (at most eight float4): the same adds in the
// same order from a ring of four reads, sixteen registers where the general
// ring holds forty-eight (which a streaming kernel spends on loads in flight).
__device__ __forceinline__ float chain_sum_lds32(float a, const float* v, int n) {
  const float4* v4 = reinterpret_cast<const float4*>(v);
  const int n4 = n >> 2;
  float4 r[4];
#pragma unroll
  for (int q = 0; q < 4; q++) r[q] = v4[q < n4 ? q : 0];
#pragma unroll
  for (int q = 0; q < 8; q++) {
    if (q < n4) {
      const float4 w = r[q & 3];
      if (q + 4 < 8) r[q & 3] = v4[q + 4 < n4 ? q + 4 : 0];
      a += w.x;
      a += w.y;
      a += w.z;
      a += w.w;
    }
  }
  for (int i = 4 * n4; i < n; i++) a += v[i];
  return a;
}

// Lane exchanges by DPP (a VALU operand modifier, no LDS round trip), for
// reductions whose combine is commutative and associative or exact: after
// the two quad steps every quad holds its result, the half-row mirror (lane
// i <-> 7 - i) then pairs each quad with the other quad of its eight lanes,
// and the row mirror (i <-> 15 - i) each eight with the other eight of its
// sixteen.  Every lane of the group must be active.
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
  return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(dpp_i32<CTRL>(__float_as_int(v)));
}
constexpr int kDppXor1 = 0xb1;      // quad_perm:[1,0,3,2]
constexpr int kDppXor2 = 0x4e;      // quad_perm:[2,3,0,1]
constexpr int kDppMirror8 = 0x141;  // row_half_mirror
constexpr int kDppMirror16 = 0x140; // row_mirror
constexpr int kDppRowBcast15 = 0x142;  // row_bcast:15 (lane 15 of each row to the next row)
constexpr int kDppRowBcast31 = 0x143;  // row_bcast:31 (lane 31 to rows 2 and 3)

// The maximum over the wave's 64 lanes, returned to every lane (fmax is
// exact in any order): within rows by DPP, across rows by row broadcasts
// (lane 63 ends with the wave's), then read from lane 63.  Every lane of the
// wave must be active.
__device__ __forceinline__ float wave_fmax(float v) {
  v = fmaxf(v, dpp_f32<kDppXor1>(v));
  v = fmaxf(v, dpp_f32<kDppXor2>(v));
  v = fmaxf(v, dpp_f32<kDppMirror8>(v));
  v = fmaxf(v, dpp_f32<kDppMirror16>(v));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v),
                                                         kDppRowBcast15, 0xa, 0xf, false)));
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v),
                                                         kDppRowBcast31, 0xc, 0xf, false)));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// finish_8lane over the eight lanes 8 i .. 8 i + 7 holding a[0..7] of one
// dot product, by DPP: ((a0 + a1) + (a2 + a3)) + ((a4 + a5) + (a6 + a7)),
// exact at the group's first lane (whose partner in the last step, lane 7,
// holds (a7 + a6) + (a5 + a4): the same sums, each operand pair swapped,
// and IEEE addition commutes).  Every lane of the wave must be active.
__device__ __forceinline__ float finish_8lane_dpp(float a) {
  const float s1 = a + dpp_f32<kDppXor1>(a);
  const float s2 = s1 + dpp_f32<kDppXor2>(s1);
  return s2 + dpp_f32<kDppMirror8>(s2);
}

// Serial chains whose terms reach the adding lane by DPP broadcast.  A wave
// issues an LDS read in about 14 cycles and a dependent add in about 4.6, so
// a chain that reads its own terms (one float4 per four adds) runs at about
// 9 cycles per term.  Here the R lanes of a group (a DPP row of 16, or a
// quad of 4) read 4R consecutive terms of the group's chain with one float4
// each, and every add takes its term from lane k of the group
// (v_add_f32_dpp with row_newbcast:k or quad_perm:[k,k,k,k]): one LDS read
// per 4R terms, and each term costs one add.  All R lanes of a group run the
// same chain (the same sums, in the same order).
//
// a + v[0] + ... + v[n - 1] in order, per group; v points at the group's
// chain (the same pointer on its R lanes), 16-byte aligned, with
// ((n + 3) & ~3) floats readable; terms past n count as +0.0f (exact: a sum
// that starts at +0.0f and adds rounded terms is never -0.0f).  n must be the
// same on every lane of the wave, and the whole wave must be active (DPP
// reads other lanes' registers).
#define DTL_RNB(k)                                                                    \
  "v_add_f32_dpp %0, %1, %0 row_newbcast:" #k " row_mask:0xf bank_mask:0xf\n"         \
  "v_add_f32_dpp %0, %2, %0 row_newbcast:" #k " row_mask:0xf bank_mask:0xf\n"         \
  "v_add_f32_dpp %0, %3, %0 row_newbcast:" #k " row_mask:0xf bank_mask:0xf\n"         \
  "v_add_f32_dpp %0, %4, %0 row_newbcast:" #k " row_mask:0xf bank_mask:0xf\n"
#define DTL_QB(k)                                                                     \
  "v_add_f32_dpp %0, %1, %0 quad_perm:[" #k "," #k "," #k "," #k "] row_mask:0xf bank_mask:0xf\n" \
  "v_add_f32_dpp %0, %2, %0 quad_perm:[" #k "," #k "," #k "," #k "] row_mask:0xf bank_mask:0xf\n" \
  "v_add_f32_dpp %0, %3, %0 quad_perm:[" #k "," #k "," #k "," #k "] row_mask:0xf bank_mask:0xf\n" \
  "v_add_f32_dpp %0, %4, %0 quad_perm:[" #k "," #k "," #k "," #k "] row_mask:0xf bank_mask:0xf\n"

// The 4R terms held by the group's lanes (lane k: terms 4k .. 4k + 3), added
// in order.  The leading s_nop covers the two wait states a DPP source
// needs after a VALU write.
template <int R>
__device__ __forceinline__ float chain_group_add(float a, float4 x) {
  static_assert(R == 16 || R == 4, "DPP rows or quads");
  if (R == 16) {
    asm("s_nop 1\n" DTL_RNB(0) DTL_RNB(1) DTL_RNB(2) DTL_RNB(3) DTL_RNB(4) DTL_RNB(5) DTL_RNB(6)
            DTL_RNB(7) DTL_RNB(8) DTL_RNB(9) DTL_RNB(10) DTL_RNB(11) DTL_RNB(12) DTL_RNB(13)
                DTL_RNB(14) DTL_RNB(15)
        : "+v"(a)
        : "v"(x.x), "v"(x.y), "v"(x.z), "v"(x.w));
  } else {
    asm("s_nop 1\n" DTL_QB(0) DTL_QB(1) DTL_QB(2) DTL_QB(3)
        : "+v"(a)
        : "v"(x.x), "v"(x.y), "v"(x.z), "v"(x.w));
  }
  return a;
}
#undef DTL_RNB
#undef DTL_QB

// With SKEW, term e sits at v[e + 4 (e / 64)] (four floats of padding after
// every 64 terms, which spreads the writers of a 64-term group over the LDS
// banks).
template <int R, bool SKEW = false>
__device__ __forceinline__ float chain_group_lds(float a, const float* v, int n) {
  constexpr int B = 4 * R;  // terms per group read
  const int k = threadIdx.x & (R - 1);
  const int nb = (n + B - 1) / B;
  auto load = [&](int b) {
    const int e = b * B + 4 * k;
    const int ec = e < n ? e : 0;
    return *reinterpret_cast<const float4*>(v + (SKEW ? ec + ((ec >> 6) << 2) : ec));
  };
  // Terms past n are zeroed just before their group's adds, not at the
  // read: a select on a value right after its read would wait for the read.
  auto live = [&](float4 x, int b) {
    const int e = b * B + 4 * k;
    x.x = e < n ? x.x : 0.0f;
    x.y = e + 1 < n ? x.y : 0.0f;
    x.z = e + 2 < n ? x.z : 0.0f;
    x.w = e + 3 < n ? x.w : 0.0f;
    return x;
  };
  // Two reads in flight ahead of the adds, over pairs of full groups (every
  // term below n).  The scheduling barrier after each read keeps it where it
  // is: without one the compiler merges the reads that feed the loop-carried
  // slot into one read at the top of the loop, next to the adds that wait
  // for it.
  const int nfull = n / B;
  if constexpr (R == 4) {
    // Quads: a read feeds only sixteen adds (about 80 cycles), less than an
    // LDS read takes while producer waves load the LDS, so six reads are in
    // flight (slot i holds group b + i).
    constexpr int A = 6;
    float4 x[A];
#pragma unroll
    for (int i = 0; i < A; i++) x[i] = load(i);
    __builtin_amdgcn_sched_barrier(0);
    int b = 0;
    for (; b + A <= nfull; b += A) {
#pragma unroll
      for (int i = 0; i < A; i++) {
        a = chain_group_add<R>(a, x[i]);
        x[i] = load(b + A + i);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int i = 0; i < A; i++) {
      if (b + i < nfull) a = chain_group_add<R>(a, x[i]);
      else if (b + i < nb) a = chain_group_add<R>(a, live(x[i], b + i));
    }
    return a;
  }
  float4 x0 = load(0), x1 = load(1);
  __builtin_amdgcn_sched_barrier(0);
  int b = 0;
  for (; b + 1 < nfull; b += 2) {
    a = chain_group_add<R>(a, x0);
    x0 = load(b + 2);
    __builtin_amdgcn_sched_barrier(0);
    a = chain_group_add<R>(a, x1);
    x1 = load(b + 3);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (b < nfull) {  // one full group, then perhaps a partial one
    a = chain_group_add<R>(a, x0);
    if (b + 1 < nb) a = chain_group_add<R>(a, live(x1, b + 1));
  } else if (b < nb) {  // a partial group
    a = chain_group_add<R>(a, live(x0, b));
  }
  return a;
}

// a += p[j] * v[j] for j = 0 .. n-1 in order as a DPP chain (one chain per
// row of R lanes, as chain_group_lds): each lane reads a float4 of p and of
// v, forms the four rounded products fl(p[j] * v[j]) just before the group's
// adds, and the adds take them from the lanes holding them.  Same values as
// forming the products into LDS first and running chain_group_lds over them.
template <int R>
__device__ __forceinline__ float chain_group_dot_lds(float a, const float* p, const float* v, int n) {
  constexpr int B = 4 * R;
  const int k = threadIdx.x & (R - 1);
  const int nb = (n + B - 1) / B;
  auto load = [&](const float* base, int b) {
    const int e = b * B + 4 * k;
    return *reinterpret_cast<const float4*>(base + (e < n ? e : 0));
  };
  auto prod = [&](float4 x, float4 y) { return make_float4(x.x * y.x, x.y * y.y, x.z * y.z, x.w * y.w); };
  auto live = [&](float4 x, int b) {
    const int e = b * B + 4 * k;
    x.x = e < n ? x.x : 0.0f;
    x.y = e + 1 < n ? x.y : 0.0f;
    x.z = e + 2 < n ? x.z : 0.0f;
    x.w = e + 3 < n ? x.w : 0.0f;
    return x;
  };
  const int nfull = n / B;
  float4 p0 = load(p, 0), v0 = load(v, 0), p1 = load(p, 1), v1 = load(v, 1);
  __builtin_amdgcn_sched_barrier(0);
  int b = 0;
  for (; b + 1 < nfull; b += 2) {
    a = chain_group_add<R>(a, prod(p0, v0));
    p0 = load(p, b + 2);
    v0 = load(v, b + 2);
    __builtin_amdgcn_sched_barrier(0);
    a = chain_group_add<R>(a, prod(p1, v1));
    p1 = load(p, b + 3);
    v1 = load(v, b + 3);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (b < nfull) {
    a = chain_group_add<R>(a, prod(p0, v0));
    if (b + 1 < nb) a = chain_group_add<R>(a, live(prod(p1, v1), b + 1));
  } else if (b < nb) {
    a = chain_group_add<R>(a, live(prod(p0, v0), b));
  }
  return a;
}

// a += p[j] * v[j] for j = 0 .. n-1 in order, each product rounded and
// added on its own (the P.V chain, det-model lib.rs:2390-2420), with both
// operand rows in LDS (16-byte aligned).  Software-pipelined in blocks of 16
// elements: the products of block b + 1 are formed (independent multiplies)
// and the operands of block b + 3 read before the 16 dependent adds of block
// b, so neither the LDS latency nor the multiplies sit on the chain.
// Operands (four float4 of each row) of one block of 16 elements.
struct ChainOps16 {
  float4 p[4], v[4];
};

__device__ __forceinline__ void chain_load16(ChainOps16& o, const float4* __restrict__ p4,
                                             const float4* __restrict__ v4, int b) {
#pragma unroll
  for (int k = 0; k < 4; k++) {
    o.p[k] = p4[4 * b + k];
    o.v[k] = v4[4 * b + k];
  }
}

__device__ __forceinline__ void chain_mul16(float (&d)[16], const ChainOps16& o) {
#pragma unroll
  for (int k = 0; k < 4; k++) {
    d[4 * k + 0] = o.p[k].x * o.v[k].x;
    d[4 * k + 1] = o.p[k].y * o.v[k].y;
    d[4 * k + 2] = o.p[k].z * o.v[k].z;
    d[4 * k + 3] = o.p[k].w * o.v[k].w;
  }
}

__device__ __forceinline__ float chain_dot_lds(float a, const float4* __restrict__ p4,
                                               const float4* __restrict__ v4, int n) {
  const int nb = n >> 4;  // blocks of 16
  int b = 0;
  if (nb >= 4) {
    // Operands are read two blocks ahead of their multiplies and products
    // one block ahead of their adds; loads past the last block re-read it.
    const int last = nb - 1;
    ChainOps16 A, B;
    float x[16], y[16];
    chain_load16(A, p4, v4, 0);
    chain_load16(B, p4, v4, 1);
    chain_mul16(x, A);                 // block 0
    chain_load16(A, p4, v4, 2);
    for (; b + 4 <= nb; b += 2) {
      // x: products of block b; B: operands of b + 1; A: operands of b + 2
      chain_mul16(y, B);               // block b + 1
      chain_load16(B, p4, v4, b + 3 < last ? b + 3 : last);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 16; i++) a += x[i];
      chain_mul16(x, A);               // block b + 2
      chain_load16(A, p4, v4, b + 4 < last ? b + 4 : last);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 16; i++) a += y[i];
    }
    // x: products of block b; B: operands of b + 1 (b + 1 < nb)
#pragma unroll
    for (int i = 0; i < 16; i++) a += x[i];
    chain_mul16(y, B);
#pragma unroll
    for (int i = 0; i < 16; i++) a += y[i];
    b += 2;
  }
  const float* p = reinterpret_cast<const float*>(p4);
  const float* v = reinterpret_cast<const float*>(v4);
  for (int i = 16 * b; i < n; i++) a += p[i] * v[i];
  return a;
}

// silu_f32 (det-num math.rs:30-34).
__device__ __forceinline__ float silu_det(float x) {
  float t = expf_det(-x);
  float d = 1.0f + t;
  return x / d;
}

// exp clamped at -88, as used by softmax (det-model lib.rs:2375) and the
// CDF (det-coder cdf.rs:291).
// exp_clamped(t) = exp_f32(max(t, -88)) (det-model softmax_in_place,
// lib.rs:2361-2388, and det-coder cdf.rs: every caller passes t = l - max
// <= 0).  For t <= 0 the method above restated for that domain: no
// overflow, underflow or NaN paths, k in [-127, 0], the k = 0 reduction as
// the general one (x - 0 ln2_hi = x, 0 ln2_lo = 0) and scalbnf as one
// multiply (two for k = -127, as its downward step takes them).  About a
// third of expf_det's instructions.  Checks: a host restatement of this
// function equals the host restatement of expf_det on all 2^31 floats with
// the sign bit set and on +0 (tests/exp_nonpos_check.c); this device
// function equals the oracle's exp_f32(max(t, -88)) on every 61st such
// pattern and on dense bands around its branch points
// (tests/test_gpu_kernels.py::test_exp_clamped_device_matches_oracle), and
// through the softmax and CDF parity tests.  NaN gives NaN; t > 0 is
// outside the domain.
__device__ __forceinline__ float exp_clamped(float t) {
  const float ln2_hi = u2f(0x3f317200u);
  const float ln2_lo = u2f(0x35bfbe8eu);
  const float inv_ln2 = u2f(0x3fb8aa3bu);
  const float p1 = u2f(0x3e2aaa8fu);
  const float p2 = u2f(0xbb355215u);
  const float x = t < -88.0f ? -88.0f : t;
  const uint32_t hx = f2u(x) & 0x7fffffffu;
  const int kr = f32_as_i32(inv_ln2 * x - 0.5f);
  const int k = hx > 0x3f851592u ? kr : (hx > 0x3eb17218u ? -1 : 0);
  const float kf = (float)k;
  const float hi = x - kf * ln2_hi;
  const float lo = kf * ln2_lo;
  const float xr = hi - lo;
  const float xx = xr * xr;
  const float c = xr - xx * (p1 + xx * p2);
  const float y = 1.0f + (xr * c / (2.0f - c) - lo + hi);
  const float r = k >= -126 ? y * u2f((uint32_t)(127 + k) << 23) : (y * 0x1p-126f) * 0.5f;
  const float e = hx > 0x39000000u ? r : 1.0f + x;
  return t != t ? t : e;
}

// ---- f64 transcendentals for RoPE tables (det-num vendored_libm) --------
// fdlibm methods: e_exp.c, e_log.c, k_sin.c, k_cos.c and the Cody-Waite
// branch of e_rem_pio2.c.

__device__ inline double scalbn64(double x, int n) {
  const double x1p1023 = u2d(0x7fe0000000000000ull);
  const double x1p_1022 = u2d(0x0010000000000000ull);
  if (n > 1023) {
    x *= x1p1023;
    n -= 1023;
    if (n > 1023) {
      x *= x1p1023;
      n -= 1023;
      if (n > 1023) n = 1023;
    }
  } else if (n < -1022) {
    x *= x1p_1022;
    n += 1022;
    if (n < -1022) {
      x *= x1p_1022;
      n += 1022;
      if (n < -1022) n = -1022;
    }
  }
  return x * u2d((uint64_t)(0x3ff + n) << 52);
}

__device__ inline int32_t f64_as_i32(double x) {
  if (x != x) return 0;
  if (x >= 2147483648.0) return INT32_MAX;
  if (x <= -2147483649.0) return INT32_MIN;
  return (int32_t)x;
}

__device__ inline double exp64(double x) {
  const double ln2hi = u2d(0x3fe62e42fee00000ull);
  const double ln2lo = u2d(0x3dea39ef35793c76ull);
  const double invln2 = u2d(0x3ff71547652b82feull);
  const double P1 = u2d(0x3fc555555555553eull);
  const double P2 = u2d(0xbf66c16c16bebd93ull);
  const double P3 = u2d(0x3f11566aaf25de2cull);
  const double P4 = u2d(0xbebbbd41c5d26bf1ull);
  const double P5 = u2d(0x3e66376972bea4d0ull);
  uint32_t hx = (uint32_t)(d2u(x) >> 32);
  int sign = (int)(hx >> 31);
  hx &= 0x7fffffffu;
  if (hx >= 0x4086232bu) {
    if (x != x) return x;
    if (x > 709.782712893383973096) return x * u2d(0x7fe0000000000000ull);
    if (x < -745.13321910194110842) return 0.0;
  }
  int k;
  double hi, lo;
  if (hx > 0x3fd62e42u) {
    if (hx >= 0x3ff0a2b2u) {
      k = f64_as_i32(invln2 * x + (sign ? -0.5 : 0.5));
    } else {
      k = 1 - sign - sign;
    }
    hi = x - (double)k * ln2hi;
    lo = (double)k * ln2lo;
    x = hi - lo;
  } else if (hx > 0x3e300000u) {
    k = 0;
    hi = x;
    lo = 0.0;
  } else {
    return 1.0 + x;
  }
  double xx = x * x;
  double c = x - xx * (P1 + xx * (P2 + xx * (P3 + xx * (P4 + xx * P5))));
  double y = 1.0 + (x * c / (2.0 - c) - lo + hi);
  return k == 0 ? y : scalbn64(y, k);
}

__device__ inline double log64(double x) {
  const double ln2_hi = u2d(0x3fe62e42fee00000ull);
  const double ln2_lo = u2d(0x3dea39ef35793c76ull);
  const double Lg1 = u2d(0x3fe5555555555593ull), Lg2 = u2d(0x3fd999999997fa04ull);
  const double Lg3 = u2d(0x3fd2492494229359ull), Lg4 = u2d(0x3fcc71c51d8e78afull);
  const double Lg5 = u2d(0x3fc7466496cb03deull), Lg6 = u2d(0x3fc39a09d078c69full);
  const double Lg7 = u2d(0x3fc2f112df3e5244ull);
  uint64_t ui = d2u(x);
  uint32_t hx = (uint32_t)(ui >> 32);
  int k = 0;
  if (hx < 0x00100000u || (hx >> 31) != 0) {
    if ((ui << 1) == 0) return -1.0 / (x * x);
    if (hx >> 31) return (x - x) / 0.0;
    k -= 54;
    x *= u2d(0x4350000000000000ull);
    ui = d2u(x);
    hx = (uint32_t)(ui >> 32);
  } else if (hx >= 0x7ff00000u) {
    return x;
  } else if (hx == 0x3ff00000u && (ui << 32) == 0) {
    return 0.0;
  }
  hx += 0x3ff00000u - 0x3fe6a09eu;
  k += (int)(hx >> 20) - 0x3ff;
  hx = (hx & 0x000fffffu) + 0x3fe6a09eu;
  ui = ((uint64_t)hx << 32) | (ui & 0xffffffffull);
  x = u2d(ui);
  double f = x - 1.0;
  double hfsq = 0.5 * f * f;
  double s = f / (2.0 + f);
  double z = s * s;
  double w = z * z;
  double t1 = w * (Lg2 + w * (Lg4 + w * Lg6));
  double t2 = z * (Lg1 + w * (Lg3 + w * (Lg5 + w * Lg7)));
  double r = t2 + t1;
  double dk = (double)k;
  return s * (hfsq + r) + dk * ln2_lo - hfsq + f + dk * ln2_hi;
}

__device__ inline double ksin64(double x, double y, int iy) {
  const double S1 = u2d(0xbfc5555555555549ull), S2 = u2d(0x3f8111111110f8a6ull);
  const double S3 = u2d(0xbf2a01a019c161d5ull), S4 = u2d(0x3ec71de357b1fe7dull);
  const double S5 = u2d(0xbe5ae5e68a2b9cebull), S6 = u2d(0x3de5d93a5acfd57cull);
  double z = x * x;
  double w = z * z;
  double r = S2 + z * (S3 + z * S4) + z * w * (S5 + z * S6);
  double v = z * x;
  if (iy == 0) return x + v * (S1 + z * r);
  return x - ((z * (0.5 * y - v * r) - y) - v * S1);
}

__device__ inline double kcos64(double x, double y) {
  const double C1 = u2d(0x3fa555555555554cull), C2 = u2d(0xbf56c16c16c15177ull);
  const double C3 = u2d(0x3efa01a019cb1590ull), C4 = u2d(0xbe927e4f809c52adull);
  const double C5 = u2d(0x3e21ee9ebdb4b1c4ull), C6 = u2d(0xbda8fae9be8838d4ull);
  double z = x * x;
  double w = z * z;
  double r = z * (C1 + z * (C2 + z * C3)) + w * w * (C4 + z * (C5 + z * C6));
  double hz = 0.5 * z;
  double ww = 1.0 - hz;
  return ww + (((1.0 - ww) - hz) + (z * r - x * y));
}

// Argument reduction by pi/2 for |x| < 2^20*pi/2; returns n, y0 + y1 = x - n*pi/2.
// Larger arguments (beyond every supported RoPE phase) yield NaN.
__device__ inline int rem_pio2(double x, double* y0o, double* y1o) {
  const double TO_INT = 1.5 / 2.2204460492503131e-16;
  const double INV_PIO2 = u2d(0x3fe45f306dc9c883ull);
  const double PIO2_1 = u2d(0x3ff921fb54400000ull), PIO2_1T = u2d(0x3dd0b4611a626331ull);
  const double PIO2_2 = u2d(0x3dd0b4611a600000ull), PIO2_2T = u2d(0x3ba3198a2e037073ull);
  const double PIO2_3 = u2d(0x3ba3198a2e000000ull), PIO2_3T = u2d(0x397b839a252049c1ull);
  int sign = (int)(d2u(x) >> 63);
  uint32_t ix = (uint32_t)(d2u(x) >> 32) & 0x7fffffffu;
  bool medium = false;
  int mult = 0;
  if (ix <= 0x400f6a7au) {
    if ((ix & 0xfffffu) == 0x921fbu) medium = true;
    else mult = ix <= 0x4002d97cu ? 1 : 2;
  } else if (ix <= 0x401c463bu) {
    if (ix <= 0x4015fdbcu) {
      if (ix == 0x4012d97cu) medium = true;
      else mult = 3;
    } else {
      if (ix == 0x401921fbu) medium = true;
      else mult = 4;
    }
  } else if (ix < 0x413921fbu) {
    medium = true;
  } else {
    *y0o = __longlong_as_double(0x7ff8000000000000ll);
    *y1o = *y0o;
    return 0;
  }
  if (!medium) {
    double m = (double)mult;
    if (sign == 0) {
      double z = x - m * PIO2_1;
      double y0 = z - m * PIO2_1T;
      *y0o = y0;
      *y1o = (z - y0) - m * PIO2_1T;
      return mult;
    }
    double z = x + m * PIO2_1;
    double y0 = z + m * PIO2_1T;
    *y0o = y0;
    *y1o = (z - y0) + m * PIO2_1T;
    return -mult;
  }
  double tmp = x * INV_PIO2 + TO_INT;
  double f_n = tmp - TO_INT;
  int n = f64_as_i32(f_n);
  double r = x - f_n * PIO2_1;
  double w = f_n * PIO2_1T;
  double y0 = r - w;
  int ey = (int)(d2u(y0) >> 52) & 0x7ff;
  int ex = (int)(ix >> 20);
  if (ex - ey > 16) {
    double t = r;
    w = f_n * PIO2_2;
    r = t - w;
    w = f_n * PIO2_2T - ((t - r) - w);
    y0 = r - w;
    ey = (int)(d2u(y0) >> 52) & 0x7ff;
    if (ex - ey > 49) {
      t = r;
      w = f_n * PIO2_3;
      r = t - w;
      w = f_n * PIO2_3T - ((t - r) - w);
      y0 = r - w;
    }
  }
  *y0o = y0;
  *y1o = (r - y0) - w;
  return n;
}

__device__ inline double sin64(double x) {
  uint32_t ix = (uint32_t)(d2u(x) >> 32) & 0x7fffffffu;
  if (ix <= 0x3fe921fbu) {
    if (ix < 0x3e500000u) return x;
    return ksin64(x, 0.0, 0);
  }
  if (ix >= 0x7ff00000u) return x - x;
  double y0, y1;
  int n = rem_pio2(x, &y0, &y1);
  switch (n & 3) {
    case 0: return ksin64(y0, y1, 1);
    case 1: return kcos64(y0, y1);
    case 2: return -ksin64(y0, y1, 1);
    default: return -kcos64(y0, y1);
  }
}

__device__ inline double cos64(double x) {
  uint32_t ix = (uint32_t)(d2u(x) >> 32) & 0x7fffffffu;
  if (ix <= 0x3fe921fbu) {
    if (ix < 0x3e46a09eu && f64_as_i32(x) == 0) return 1.0;
    return kcos64(x, 0.0);
  }
  if (ix >= 0x7ff00000u) return x - x;
  double y0, y1;
  int n = rem_pio2(x, &y0, &y1);
  switch (n & 3) {
    case 0: return kcos64(y0, y1);
    case 1: return -ksin64(y0, y1, 1);
    case 2: return -kcos64(y0, y1);
    default: return ksin64(y0, y1, 1);
  }
}

}  // namespace dtl
