/*
 * detref numeric core — TEST INFRASTRUCTURE ONLY (the oracle).
 *
 * Restates crates/det-num of mii443/detllm: the 8-lane f32 reductions
 * (src/reduce.rs:2-38), f16 decoding (src/f16.rs:6-34), explicit rounding
 * (src/round.rs:2-39), SHA-256 (src/hash.rs), the numeric canary
 * (src/canary.rs:14-53) and the vendored FreeBSD/fdlibm transcendentals
 * (src/vendored_libm.rs, src/vendored_libm/{expf,exp,log,sin,cos,k_sin,
 * k_cos,rem_pio2}.rs).  Compiled with -ffp-contract=off and without
 * -ffast-math so every C operator is one IEEE-754 rounding.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "detref.h"
#include "detref_internal.h"

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static inline uint64_t d2u(double x) { uint64_t u; memcpy(&u, &x, 8); return u; }
static inline double u2d(uint64_t u) { double x; memcpy(&x, &u, 8); return x; }

/* Rust `f32 as i32`: truncation toward zero, saturating, NaN -> 0. */
int32_t ref_f32_as_i32(float x) {
    if (x != x) return 0;
    if (x >= 2147483648.0f) return INT32_MAX;
    if (x <= -2147483904.0f) return INT32_MIN;
    if (x < -2147483648.0f) return INT32_MIN;
    return (int32_t)x;
}

static int64_t f64_as_i64(double x) {
    if (x != x) return 0;
    if (x >= 9223372036854775808.0) return INT64_MAX;
    if (x < -9223372036854775808.0) return INT64_MIN;
    return (int64_t)x;
}

/* ---- reductions: crates/det-num/src/reduce.rs:2-38 --------------------- */
float ref_finish_8lane(const float acc[8]) {
    return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

float ref_dot_f32(const float *x, const float *y, size_t n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t i = 0; i < n; i++) acc[i & 7] += x[i] * y[i];
    return ref_finish_8lane(acc);
}

float ref_sum_f32(const float *x, size_t n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t i = 0; i < n; i++) acc[i & 7] += x[i];
    return ref_finish_8lane(acc);
}

float ref_sum_squares_f32(const float *x, size_t n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t i = 0; i < n; i++) acc[i & 7] += x[i] * x[i];
    return ref_finish_8lane(acc);
}

/* ---- f16: crates/det-num/src/f16.rs:6-34 -------------------------------- */
float ref_f16_to_f32(uint16_t bits) {
    uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
    uint32_t exp = (bits >> 10) & 0x1f;
    uint32_t frac = bits & 0x03ffu;
    uint32_t out;
    if (exp == 0) {
        if (frac == 0) {
            out = sign;
        } else {
            uint32_t f = frac;
            int32_t e = -14;
            while ((f & 0x0400u) == 0) {
                f <<= 1;
                e -= 1;
            }
            f &= 0x03ffu;
            out = sign | ((uint32_t)(e + 127) << 23) | (f << 13);
        }
    } else if (exp == 0x1f) {
        out = sign | 0x7f800000u | (frac << 13);
    } else {
        out = sign | ((exp - 15 + 127) << 23) | (frac << 13);
    }
    return u2f(out);
}

int ref_f16_is_finite(uint16_t bits) { return (bits & 0x7c00) != 0x7c00; }

/* ---- rounding: crates/det-num/src/round.rs:2-39 ------------------------- */
int32_t ref_round_ties_even_i32(float x) {
    if (!isfinite(x)) return ref_f32_as_i32(x);
    if (!(x >= -8388608.0f && x < 8388608.0f)) return ref_f32_as_i32(x);
    int32_t t = (int32_t)x;
    float frac = x - (float)t;
    if (frac > 0.5f || (frac == 0.5f && (t & 1) != 0)) return t + 1;
    if (frac < -0.5f || (frac == -0.5f && (t & 1) != 0)) return t - 1;
    return t;
}

int64_t ref_round_ties_even_i64(double x) {
    if (!isfinite(x)) return f64_as_i64(x);
    if (!(x >= -4503599627370496.0 && x < 4503599627370496.0)) return f64_as_i64(x);
    int64_t t = (int64_t)x;
    double frac = x - (double)t;
    if (frac > 0.5 || (frac == 0.5 && (t & 1) != 0)) return t + 1;
    if (frac < -0.5 || (frac == -0.5 && (t & 1) != 0)) return t - 1;
    return t;
}

/* ---- scalbn: crates/det-num/src/vendored_libm.rs:94-146 ----------------- */
static float scalbn_f32(float x, int32_t n) {
    const float x1p127 = u2f(0x7f000000u);
    const float x1p_126 = u2f(0x00800000u);
    if (n > 127) {
        x *= x1p127;
        n -= 127;
        if (n > 127) {
            x *= x1p127;
            n -= 127;
            if (n > 127) n = 127;
        }
    } else if (n < -126) {
        x *= x1p_126;
        n += 126;
        if (n < -126) {
            x *= x1p_126;
            n += 126;
            if (n < -126) n = -126;
        }
    }
    return x * u2f((uint32_t)(0x7f + n) << 23);
}

static double scalbn_f64(double x, int32_t n) {
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

/* ---- expf: crates/det-num/src/vendored_libm/expf.rs:33-106 --------------
 * FreeBSD e_expf.c: k = round(x/ln2), x = hi - lo with ln2 split in two,
 * rational approximation R(x) = x*c/(2-c) with c = x - x^2 (P1 + x^2 P2). */
float ref_exp_f32(float x) {
    const float half[2] = {0.5f, -0.5f};
    const float ln2_hi = u2f(0x3f317200u);
    const float ln2_lo = u2f(0x35bfbe8eu);
    const float inv_ln2 = u2f(0x3fb8aa3bu);
    const float p1 = 1.6666625440e-1f;
    const float p2 = -2.7667332906e-3f;
    const float x1p127 = u2f(0x7f000000u);
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
        if (hx > 0x3f851592u) {
            k = ref_f32_as_i32(inv_ln2 * x + half[sign]);
        } else {
            k = 1 - sign - sign;
        }
        float kf = (float)k;
        hi = x - kf * ln2_hi;
        lo = kf * ln2_lo;
        x = hi - lo;
    } else if (hx > 0x39000000u) {
        k = 0;
        hi = x;
        lo = 0.0f;
    } else {
        return 1.0f + x;
    }
    float xx = x * x;
    float c = x - xx * (p1 + xx * p2);
    float y = 1.0f + (x * c / (2.0f - c) - lo + hi);
    return k == 0 ? y : scalbn_f32(y, k);
}

/* exp_f32 over an array; clamp != 0 applies max(x, -88) first, as
 * softmax_in_place (det-model lib.rs:2375) and the CDF (det-coder
 * cdf.rs:291) do before calling exp_f32. */
void ref_exp_f32_array(const float *x, float *out, size_t n, int clamp) {
    for (size_t i = 0; i < n; i++) {
        float v = x[i];
        if (clamp && v < -88.0f) v = -88.0f;
        out[i] = ref_exp_f32(v);
    }
}

/* silu: crates/det-num/src/math.rs:30-34 */
float ref_silu_f32(float x) {
    float t = ref_exp_f32(-x);
    float d = 1.0f + t;
    return x / d;
}

/* ---- exp (f64): crates/det-num/src/vendored_libm/exp.rs ----------------- */
double ref_exp_f64(double x) {
    const double half[2] = {0.5, -0.5};
    const double ln2hi = u2d(0x3fe62e42fee00000ull);
    const double ln2lo = u2d(0x3dea39ef35793c76ull);
    const double invln2 = u2d(0x3ff71547652b82feull);
    const double P1 = u2d(0x3FC555555555553Eull);
    const double P2 = u2d(0xBF66C16C16BEBD93ull);
    const double P3 = u2d(0x3F11566AAF25DE2Cull);
    const double P4 = u2d(0xBEBBBD41C5D26BF1ull);
    const double P5 = u2d(0x3E66376972BEA4D0ull);
    const double x1p1023 = u2d(0x7fe0000000000000ull);
    uint32_t hx = (uint32_t)(d2u(x) >> 32);
    int32_t sign = (int32_t)(hx >> 31);
    hx &= 0x7fffffffu;
    if (hx >= 0x4086232bu) {
        if (x != x) return x;
        if (x > 709.782712893383973096) return x * x1p1023;
        if (x < -708.39641853226410622) {
            if (x < -745.13321910194110842) return 0.0;
        }
    }
    int32_t k;
    double hi, lo;
    if (hx > 0x3fd62e42u) {
        if (hx >= 0x3ff0a2b2u) {
            k = (int32_t)f64_as_i64(invln2 * x + half[sign]);
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
    return k == 0 ? y : scalbn_f64(y, k);
}

/* ---- log (f64): crates/det-num/src/vendored_libm/log.rs ----------------- */
double ref_ln_f64(double x) {
    const double ln2_hi = u2d(0x3fe62e42fee00000ull);
    const double ln2_lo = u2d(0x3dea39ef35793c76ull);
    const double Lg1 = u2d(0x3FE5555555555593ull);
    const double Lg2 = u2d(0x3FD999999997FA04ull);
    const double Lg3 = u2d(0x3FD2492494229359ull);
    const double Lg4 = u2d(0x3FCC71C51D8E78AFull);
    const double Lg5 = u2d(0x3FC7466496CB03DEull);
    const double Lg6 = u2d(0x3FC39A09D078C69Full);
    const double Lg7 = u2d(0x3FC2F112DF3E5244ull);
    const double x1p54 = u2d(0x4350000000000000ull);
    uint64_t ui = d2u(x);
    uint32_t hx = (uint32_t)(ui >> 32);
    int32_t k = 0;
    if (hx < 0x00100000u || (hx >> 31) != 0) {
        if ((ui << 1) == 0) return -1.0 / (x * x);
        if (hx >> 31) return (x - x) / 0.0;
        k -= 54;
        x *= x1p54;
        ui = d2u(x);
        hx = (uint32_t)(ui >> 32);
    } else if (hx >= 0x7ff00000u) {
        return x;
    } else if (hx == 0x3ff00000u && (ui << 32) == 0) {
        return 0.0;
    }
    hx += 0x3ff00000u - 0x3fe6a09eu;
    k += (int32_t)(hx >> 20) - 0x3ff;
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

/* ---- sin/cos kernels: vendored_libm/k_sin.rs, k_cos.rs ------------------ */
static double k_sin(double x, double y, int iy) {
    const double S1 = u2d(0xBFC5555555555549ull);
    const double S2 = u2d(0x3F8111111110F8A6ull);
    const double S3 = u2d(0xBF2A01A019C161D5ull);
    const double S4 = u2d(0x3EC71DE357B1FE7Dull);
    const double S5 = u2d(0xBE5AE5E68A2B9CEBull);
    const double S6 = u2d(0x3DE5D93A5ACFD57Cull);
    double z = x * x;
    double w = z * z;
    double r = S2 + z * (S3 + z * S4) + z * w * (S5 + z * S6);
    double v = z * x;
    if (iy == 0) return x + v * (S1 + z * r);
    return x - ((z * (0.5 * y - v * r) - y) - v * S1);
}

static double k_cos(double x, double y) {
    const double C1 = u2d(0x3FA555555555554Cull);
    const double C2 = u2d(0xBF56C16C16C15177ull);
    const double C3 = u2d(0x3EFA01A019CB1590ull);
    const double C4 = u2d(0xBE927E4F809C52ADull);
    const double C5 = u2d(0x3E21EE9EBDB4B1C4ull);
    const double C6 = u2d(0xBDA8FAE9BE8838D4ull);
    double z = x * x;
    double w = z * z;
    double r = z * (C1 + z * (C2 + z * C3)) + w * w * (C4 + z * (C5 + z * C6));
    double hz = 0.5 * z;
    double ww = 1.0 - hz;
    return ww + (((1.0 - ww) - hz) + (z * r - x * y));
}

/* ---- rem_pio2: vendored_libm/rem_pio2.rs --------------------------------
 * Cody-Waite reduction for |x| < 2^20*pi/2.  The Payne-Hanek path the
 * reference keeps for larger arguments (rem_pio2_large.rs) is not restated:
 * RoPE phases are pos*omega with omega <= 1, so they stay below 2^20*pi/2
 * for every context below 1.6M positions.  Larger arguments return NaN,
 * which the RoPE table builder reports as NonFinite. */
static int rem_pio2(double x, double *y0o, double *y1o) {
    const double EPS = 2.2204460492503131e-16;
    const double TO_INT = 1.5 / EPS;
    const double INV_PIO2 = u2d(0x3FE45F306DC9C883ull);
    const double PIO2_1 = u2d(0x3FF921FB54400000ull);
    const double PIO2_1T = u2d(0x3DD0B4611A626331ull);
    const double PIO2_2 = u2d(0x3DD0B4611A600000ull);
    const double PIO2_2T = u2d(0x3BA3198A2E037073ull);
    const double PIO2_3 = u2d(0x3BA3198A2E000000ull);
    const double PIO2_3T = u2d(0x397B839A252049C1ull);
    int32_t sign = (int32_t)(d2u(x) >> 63);
    uint32_t ix = (uint32_t)(d2u(x) >> 32) & 0x7fffffffu;
    int medium = 0;
    if (ix <= 0x400f6a7au) {
        if ((ix & 0xfffffu) == 0x921fbu) {
            medium = 1;
        } else if (ix <= 0x4002d97cu) {
            if (sign == 0) {
                double z = x - PIO2_1;
                double y0 = z - PIO2_1T;
                *y0o = y0;
                *y1o = (z - y0) - PIO2_1T;
                return 1;
            } else {
                double z = x + PIO2_1;
                double y0 = z + PIO2_1T;
                *y0o = y0;
                *y1o = (z - y0) + PIO2_1T;
                return -1;
            }
        } else if (sign == 0) {
            double z = x - 2.0 * PIO2_1;
            double y0 = z - 2.0 * PIO2_1T;
            *y0o = y0;
            *y1o = (z - y0) - 2.0 * PIO2_1T;
            return 2;
        } else {
            double z = x + 2.0 * PIO2_1;
            double y0 = z + 2.0 * PIO2_1T;
            *y0o = y0;
            *y1o = (z - y0) + 2.0 * PIO2_1T;
            return -2;
        }
    } else if (ix <= 0x401c463bu) {
        if (ix <= 0x4015fdbcu) {
            if (ix == 0x4012d97cu) {
                medium = 1;
            } else if (sign == 0) {
                double z = x - 3.0 * PIO2_1;
                double y0 = z - 3.0 * PIO2_1T;
                *y0o = y0;
                *y1o = (z - y0) - 3.0 * PIO2_1T;
                return 3;
            } else {
                double z = x + 3.0 * PIO2_1;
                double y0 = z + 3.0 * PIO2_1T;
                *y0o = y0;
                *y1o = (z - y0) + 3.0 * PIO2_1T;
                return -3;
            }
        } else {
            if (ix == 0x401921fbu) {
                medium = 1;
            } else if (sign == 0) {
                double z = x - 4.0 * PIO2_1;
                double y0 = z - 4.0 * PIO2_1T;
                *y0o = y0;
                *y1o = (z - y0) - 4.0 * PIO2_1T;
                return 4;
            } else {
                double z = x + 4.0 * PIO2_1;
                double y0 = z + 4.0 * PIO2_1T;
                *y0o = y0;
                *y1o = (z - y0) + 4.0 * PIO2_1T;
                return -4;
            }
        }
    } else if (ix < 0x413921fbu) {
        medium = 1;
    }
    if (!medium) {
        *y0o = NAN;
        *y1o = NAN;
        return 0;
    }
    double tmp = x * INV_PIO2 + TO_INT;
    double f_n = tmp - TO_INT;
    int32_t n = (int32_t)f64_as_i64(f_n);
    double r = x - f_n * PIO2_1;
    double w = f_n * PIO2_1T;
    double y0 = r - w;
    int32_t ey = (int32_t)(d2u(y0) >> 52) & 0x7ff;
    int32_t ex = (int32_t)(ix >> 20);
    if (ex - ey > 16) {
        double t = r;
        w = f_n * PIO2_2;
        r = t - w;
        w = f_n * PIO2_2T - ((t - r) - w);
        y0 = r - w;
        ey = (int32_t)(d2u(y0) >> 52) & 0x7ff;
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

/* sin.rs */
double ref_sin_f64(double x) {
    uint32_t ix = (uint32_t)(d2u(x) >> 32) & 0x7fffffffu;
    if (ix <= 0x3fe921fbu) {
        if (ix < 0x3e500000u) return x;
        return k_sin(x, 0.0, 0);
    }
    if (ix >= 0x7ff00000u) return x - x;
    double y0, y1;
    int n = rem_pio2(x, &y0, &y1);
    switch (n & 3) {
    case 0: return k_sin(y0, y1, 1);
    case 1: return k_cos(y0, y1);
    case 2: return -k_sin(y0, y1, 1);
    default: return -k_cos(y0, y1);
    }
}

/* cos.rs */
double ref_cos_f64(double x) {
    uint32_t ix = (uint32_t)(d2u(x) >> 32) & 0x7fffffffu;
    if (ix <= 0x3fe921fbu) {
        if (ix < 0x3e46a09eu) {
            if ((int32_t)f64_as_i64(x) == 0) return 1.0;
        }
        return k_cos(x, 0.0);
    }
    if (ix >= 0x7ff00000u) return x - x;
    double y0, y1;
    int n = rem_pio2(x, &y0, &y1);
    switch (n & 3) {
    case 0: return k_cos(y0, y1);
    case 1: return -k_sin(y0, y1, 1);
    case 2: return -k_cos(y0, y1);
    default: return k_sin(y0, y1, 1);
    }
}

/* ---- SHA-256 (FIPS 180-4), as used by crates/det-num/src/hash.rs ------- */
static const uint32_t K256[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};

static inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

static void sha256_compress(uint32_t st[8], const uint8_t *p) {
    uint32_t w[64];
    for (int i = 0; i < 16; i++)
        w[i] = ((uint32_t)p[4 * i] << 24) | ((uint32_t)p[4 * i + 1] << 16) |
               ((uint32_t)p[4 * i + 2] << 8) | p[4 * i + 3];
    for (int i = 16; i < 64; i++) {
        uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
        uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
        w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = st[0], b = st[1], c = st[2], d = st[3], e = st[4], f = st[5], g = st[6], h = st[7];
    for (int i = 0; i < 64; i++) {
        uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
        uint32_t ch = (e & f) ^ (~e & g);
        uint32_t t1 = h + S1 + ch + K256[i] + w[i];
        uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
        uint32_t mj = (a & b) ^ (a & c) ^ (b & c);
        uint32_t t2 = S0 + mj;
        h = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
    }
    st[0] += a; st[1] += b; st[2] += c; st[3] += d;
    st[4] += e; st[5] += f; st[6] += g; st[7] += h;
}

void ref_sha256_init(ref_sha256_ctx *c) {
    static const uint32_t iv[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                   0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    memcpy(c->st, iv, sizeof iv);
    c->len = 0;
    c->buf_len = 0;
}

void ref_sha256_update(ref_sha256_ctx *c, const void *data, size_t len) {
    const uint8_t *p = (const uint8_t *)data;
    c->len += len;
    if (c->buf_len) {
        size_t n = 64 - c->buf_len;
        if (n > len) n = len;
        memcpy(c->buf + c->buf_len, p, n);
        c->buf_len += n;
        p += n;
        len -= n;
        if (c->buf_len == 64) {
            sha256_compress(c->st, c->buf);
            c->buf_len = 0;
        }
    }
    while (len >= 64) {
        sha256_compress(c->st, p);
        p += 64;
        len -= 64;
    }
    if (len) {
        memcpy(c->buf, p, len);
        c->buf_len = len;
    }
}

void ref_sha256_final(ref_sha256_ctx *c, uint8_t out[32]) {
    uint64_t bits = c->len * 8;
    c->buf[c->buf_len++] = 0x80;
    if (c->buf_len > 56) {
        memset(c->buf + c->buf_len, 0, 64 - c->buf_len);
        sha256_compress(c->st, c->buf);
        c->buf_len = 0;
    }
    memset(c->buf + c->buf_len, 0, 56 - c->buf_len);
    for (int i = 0; i < 8; i++) c->buf[56 + i] = (uint8_t)(bits >> (56 - 8 * i));
    sha256_compress(c->st, c->buf);
    for (int i = 0; i < 8; i++) {
        out[4 * i] = (uint8_t)(c->st[i] >> 24);
        out[4 * i + 1] = (uint8_t)(c->st[i] >> 16);
        out[4 * i + 2] = (uint8_t)(c->st[i] >> 8);
        out[4 * i + 3] = (uint8_t)c->st[i];
    }
}

void ref_sha256(const void *data, size_t len, uint8_t out[32]) {
    ref_sha256_ctx c;
    ref_sha256_init(&c);
    ref_sha256_update(&c, data, len);
    ref_sha256_final(&c, out);
}

void ref_sha256_f32(ref_sha256_ctx *c, float v) {
    uint32_t u = f2u(v);
    uint8_t b[4] = {(uint8_t)u, (uint8_t)(u >> 8), (uint8_t)(u >> 16), (uint8_t)(u >> 24)};
    ref_sha256_update(c, b, 4);
}

/* ---- numeric canary: crates/det-num/src/canary.rs:26-53 ----------------- */
void ref_numeric_canary(uint8_t out[32]) {
    float x[9] = {u2f(1), u2f(2), -0.0f, 1.0f, -2.5f, 3.25f, 1024.0f, -4096.0f, 0.125f};
    float y[9] = {2.0f, -3.0f, 4.0f, 0.5f, -8.0f, 16.0f, -0.25f, 0.03125f, -64.0f};
    float values[6] = {
        ref_dot_f32(x, y, 9),        ref_exp_f32(-1.0f),
        ref_exp_f32(0.0f),           ref_f16_to_f32(0x3555),
        (float)ref_round_ties_even_i32(2.5f), u2f(1) + u2f(1),
    };
    ref_sha256_ctx c;
    ref_sha256_init(&c);
    for (int i = 0; i < 6; i++) ref_sha256_f32(&c, values[i]);
    ref_sha256_final(&c, out);
}
