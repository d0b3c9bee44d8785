/* Host check of div_recip (detllm_amd/csrc/dtl_numerics.h): q0 = v * rd,
 * q1 = fma(fma(-q0, d, v), rd, q0) with rd = 1 / d must equal the rounded
 * quotient v / d for the Q8A quantiser's operands: d = amax / 127 with
 * amax >= 2^-92 and 2^-100 <= |v| <= amax; and d itself, amax / 127 by the
 * same correction from rd = 1 / 127, for every amax in [2^-100, 2^127).
 * Exit status 0 when every compared value agrees bit for bit. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static uint64_t rs = 88172645463325252ull;
static uint64_t rnd(void) { rs ^= rs << 13; rs ^= rs >> 7; rs ^= rs << 17; return rs; }
static float div_recip(float v, float d, float rd) {
  float q0 = v * rd;
  float r = fmaf(-q0, d, v);
  return fmaf(r, rd, q0);
}

int main(int argc, char **argv) {
  volatile float one = 1.0f, c127 = 127.0f;
  const float r127 = one / c127;
  long bad = 0, n = 0;
  /* every third float v in [2^-100, amax] for these amax (every one of
   * them, and a dozen more amax, agreed when this check was first run) */
  const float amaxs[] = {1.0f, 0x1.fffffep0f, 0x1.4cccccp-92f, 7.77e5f};
  for (unsigned k = 0; k < sizeof amaxs / sizeof amaxs[0]; k++) {
    float amax = amaxs[k], d = div_recip(amax, c127, r127), rd = one / d;
    if (f2u(d) != f2u(amax / c127)) bad++;
    for (uint32_t u = f2u(0x1p-100f) + k; u <= f2u(amax); u += 3) {
      float v = u2f(u);
      n++;
      if (f2u(div_recip(v, d, rd)) != f2u(v / d)) bad++;
    }
  }
  /* random pairs, amax from 2^-92 to 2^127 */
  for (long it = 0; it < (1L << 24); it++) {
    uint32_t ea = 127 - 92 + (uint32_t)(rnd() % 219);
    float amax = u2f((ea << 23) | (uint32_t)(rnd() & 0x7fffff));
    float d = amax / c127, rd = one / d;
    uint32_t span = f2u(amax) - f2u(0x1p-100f);
    float v = u2f(f2u(amax) - (uint32_t)(rnd() % (span + 1u)));
    if (rnd() & 1) v = -v;
    n++;
    if (f2u(div_recip(v, d, rd)) != f2u(v / d)) bad++;
  }
  /* d = amax / 127 itself, every seventh amax in [2^-100, 2^127) */
  for (uint32_t u = f2u(0x1p-100f); u < 0x7f800000u; u += 7) {
    float a = u2f(u);
    n++;
    if (f2u(div_recip(a, c127, r127)) != f2u(a / c127)) bad++;
  }
  printf("%ld comparisons, %ld mismatches\n", n, bad);
  return bad != 0;
}
