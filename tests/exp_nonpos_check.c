/* Host check of exp_clamped (detllm_amd/csrc/dtl_numerics.h), restated for
 * t <= 0: against the general expf_det path (the FreeBSD expf restated, as in
 * oracle/detref_num.c) applied to max(t, -88), for every float with the sign
 * bit set (all 2^31 patterns: -0, subnormals, normals, -inf) and +0.  Exit
 * status 0 when all agree bit for bit (NaN inputs go to the general path and
 * are not compared).  About 40 s on 8 cores. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static int32_t f32_as_i32(float x) {
  if (x != x) return 0;
  if (x >= 2147483648.0f) return INT32_MAX;
  if (x <= -2147483648.0f) return INT32_MIN;
  return (int32_t)x;
}
static float scalbn_f32(float x, int32_t n) {
  const float x1p127 = u2f(0x7f000000u), x1p_126 = u2f(0x00800000u);
  if (n > 127) { x *= x1p127; n -= 127; if (n > 127) { x *= x1p127; n -= 127; if (n > 127) n = 127; } }
  else if (n < -126) { x *= x1p_126; n += 126; if (n < -126) { x *= x1p_126; n += 126; if (n < -126) n = -126; } }
  return x * u2f((uint32_t)(0x7f + n) << 23);
}
static float expf_ref(float x) {
  const float half[2] = {0.5f, -0.5f};
  const float ln2_hi = u2f(0x3f317200u), ln2_lo = u2f(0x35bfbe8eu), inv_ln2 = u2f(0x3fb8aa3bu);
  const float p1 = 1.6666625440e-1f, p2 = -2.7667332906e-3f, x1p127 = u2f(0x7f000000u);
  uint32_t hx = f2u(x);
  int32_t sign = (int32_t)(hx >> 31);
  hx &= 0x7fffffffu;
  if (hx >= 0x42aeac50u) {
    if (hx > 0x7f800000u) return x;
    if (hx >= 0x42b17218u && !sign) return x * x1p127;
    if (sign && hx >= 0x42cff1b5u) return 0.0f;
  }
  int32_t k;
  float hi, lo;
  if (hx > 0x3eb17218u) {
    k = hx > 0x3f851592u ? f32_as_i32(inv_ln2 * x + half[sign]) : 1 - sign - sign;
    float kf = (float)k;
    hi = x - kf * ln2_hi;
    lo = kf * ln2_lo;
    x = hi - lo;
  } else if (hx > 0x39000000u) {
    k = 0; hi = x; lo = 0.0f;
  } else {
    return 1.0f + x;
  }
  float xx = x * x;
  float c = x - xx * (p1 + xx * p2);
  float y = 1.0f + (x * c / (2.0f - c) - lo + hi);
  return k == 0 ? y : scalbn_f32(y, k);
}
/* the restatement in dtl_numerics.h (t <= 0) */
static float exp_nonpos(float t) {
  const float ln2_hi = u2f(0x3f317200u), ln2_lo = u2f(0x35bfbe8eu), inv_ln2 = u2f(0x3fb8aa3bu);
  const float p1 = u2f(0x3e2aaa8fu), p2 = u2f(0xbb355215u);
  const float x = t < -88.0f ? -88.0f : t;
  const uint32_t hx = f2u(x) & 0x7fffffffu;
  const int32_t kr = f32_as_i32(inv_ln2 * x - 0.5f);
  const int32_t k = hx > 0x3f851592u ? kr : (hx > 0x3eb17218u ? -1 : 0);
  const float kf = (float)k;
  const float hi = x - kf * ln2_hi, lo = kf * ln2_lo, xr = hi - lo;
  const float xx = xr * xr;
  const float c = xr - xx * (p1 + xx * p2);
  const float y = 1.0f + (xr * c / (2.0f - c) - lo + hi);
  float r = k >= -126 ? y * u2f((uint32_t)(127 + k) << 23) : (y * 0x1p-126f) * 0.5f;
  return hx > 0x39000000u ? r : 1.0f + x;
}

int main(void) {
  long bad = 0, n = 0;
#pragma omp parallel for reduction(+ : bad, n) schedule(static)
  for (long u = 0x80000000L; u <= 0xffffffffL; u += 1) {
    float t = u2f((uint32_t)u);
    if (t != t) continue;
    float want = expf_ref(t < -88.0f ? -88.0f : t), got = exp_nonpos(t);
    n++;
    if (f2u(want) != f2u(got)) bad++;
  }
  if (f2u(exp_nonpos(0.0f)) != f2u(expf_ref(0.0f))) bad++;
  printf("%ld inputs, %ld mismatches\n", n, bad);
  return bad != 0;
}
