/*
 * detref quantisation kernels — TEST INFRASTRUCTURE ONLY (the oracle).
 *
 * Restates the scalar paths of crates/det-quant/src/lib.rs of
 * mii443/detllm: Q8A / Q8_K activation quantisers (lib.rs:111-187), the
 * Q8_0 / Q4_0 block dots (lib.rs:237-279, 443-504), the per-element Q4_K
 * chain (lib.rs:281-315, 506-529) and the lane-split Q6_K dot
 * (lib.rs:353-397, 531-568), plus the det-cli known-answer generators
 * (crates/det-cli/src/main.rs:146-388).
 */
#include <math.h>
#include <string.h>

#include "detref.h"
#include "detref_internal.h"

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* lib.rs:175-181 */
static int32_t round_half_away_from_zero_i32(float x) {
    if (x < 0.0f) return ref_f32_as_i32(x - 0.5f);
    return ref_f32_as_i32(x + 0.5f);
}

/* lib.rs:184-187: the 1.5*2^23 magic-number rounding of ggml. */
static int32_t nearest_i32_ggml(float x) {
    float val = x + 12582912.0f;
    return (int32_t)(f2u(val) & 0x007fffffu) - 0x00400000;
}

/* lib.rs:111-137 */
int ref_q8a_block_quantize(const float *x, ref_q8a_block *out) {
    float amax = 0.0f;
    for (int i = 0; i < QK; i++) {
        if (!isfinite(x[i])) return QERR_NON_FINITE_INPUT;
        float ax = x[i] < 0.0f ? -x[i] : x[i];
        if (ax > amax) amax = ax;
    }
    memset(out->q, 0, QK);
    if (amax == 0.0f) {
        out->d = 0.0f;
        return QERR_OK;
    }
    float d = amax / 127.0f;
    for (int i = 0; i < QK; i++) {
        int32_t r = round_half_away_from_zero_i32(x[i] / d);
        if (r < -127) r = -127;
        if (r > 127) r = 127;
        out->q[i] = (int8_t)r;
    }
    out->d = d;
    return QERR_OK;
}

/* lib.rs:139-172 (bsums are not used by any dot and are omitted) */
int ref_q8k_block_quantize(const float *x, ref_q8k_block *out) {
    float amax = 0.0f, max = 0.0f;
    for (int i = 0; i < QKK; i++) {
        if (!isfinite(x[i])) return QERR_NON_FINITE_INPUT;
        float ax = x[i] < 0.0f ? -x[i] : x[i];
        if (ax > amax) {
            amax = ax;
            max = x[i];
        }
    }
    memset(out->q, 0, QKK);
    if (amax == 0.0f) {
        out->d = 0.0f;
        return QERR_OK;
    }
    float iscale = -127.0f / max;
    for (int i = 0; i < QKK; i++) {
        int32_t r = nearest_i32_ggml(iscale * x[i]);
        if (r > 127) r = 127;
        out->q[i] = (int8_t)r;
    }
    out->d = 1.0f / iscale;
    return QERR_OK;
}

/* lib.rs:443-452 */
float ref_dot_q8_0_q8a_block(const ref_q8_0_block *w, const ref_q8a_block *a) {
    int32_t isum = 0;
    for (int i = 0; i < QK; i++) isum += (int32_t)w->q[i] * (int32_t)a->q[i];
    float scale = w->d * a->d;
    return scale * (float)isum;
}

/* lib.rs:492-504 */
float ref_dot_q4_0_q8a_block(const ref_q4_0_block *w, const ref_q8a_block *a) {
    int32_t isum = 0;
    for (int i = 0; i < QK / 2; i++) {
        uint8_t packed = w->qs[i];
        int32_t lo = (int32_t)(packed & 0x0f) - 8;
        int32_t hi = (int32_t)(packed >> 4) - 8;
        isum += lo * (int32_t)a->q[i];
        isum += hi * (int32_t)a->q[i + QK / 2];
    }
    float scale = w->d * a->d;
    return scale * (float)isum;
}

/* lib.rs:237-257 */
int ref_dot_q8_0_q8a(const ref_q8_0_block *w, const ref_q8a_block *a, size_t nb, float *out) {
    if (nb == 0) return QERR_INVALID_BLOCK_LENGTH;
    float sum = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        if (!isfinite(w[b].d) || !isfinite(a[b].d)) return QERR_NON_FINITE_SCALE;
        float block = ref_dot_q8_0_q8a_block(&w[b], &a[b]);
        if (!isfinite(block)) return QERR_NON_FINITE_OUTPUT;
        sum += block;
        if (!isfinite(sum)) return QERR_NON_FINITE_OUTPUT;
    }
    *out = sum;
    return QERR_OK;
}

/* lib.rs:259-279 */
int ref_dot_q4_0_q8a(const ref_q4_0_block *w, const ref_q8a_block *a, size_t nb, float *out) {
    if (nb == 0) return QERR_INVALID_BLOCK_LENGTH;
    float sum = 0.0f;
    for (size_t b = 0; b < nb; b++) {
        if (!isfinite(w[b].d) || !isfinite(a[b].d)) return QERR_NON_FINITE_SCALE;
        float block = ref_dot_q4_0_q8a_block(&w[b], &a[b]);
        if (!isfinite(block)) return QERR_NON_FINITE_OUTPUT;
        sum += block;
        if (!isfinite(sum)) return QERR_NON_FINITE_OUTPUT;
    }
    *out = sum;
    return QERR_OK;
}

/* lib.rs:519-529: 6-bit scale/min unpacking of the 12-byte Q4_K header. */
int ref_q4_k_scale_min(const uint8_t scales[12], size_t index, uint8_t *mn) {
    uint8_t sc, m;
    if (index < 4) {
        sc = scales[index] & 0x3f;
        m = scales[index + 4] & 0x3f;
    } else {
        sc = (uint8_t)((scales[index + 4] & 0x0f) | ((scales[index - 4] >> 6) << 4));
        m = (uint8_t)((scales[index + 4] >> 4) | ((scales[index] >> 6) << 4));
    }
    *mn = m;
    return sc;
}

/* lib.rs:506-517 */
float ref_q4_k_value(const ref_q4k_block *w, size_t index) {
    size_t sub = index / 32, within = index % 32;
    uint8_t m;
    uint8_t sc = (uint8_t)ref_q4_k_scale_min(w->scales, sub, &m);
    uint8_t q = (sub % 2 == 0) ? (uint8_t)(w->qs[(sub / 2) * 32 + within] & 0x0f)
                               : (uint8_t)(w->qs[(sub / 2) * 32 + within] >> 4);
    return (w->d * (float)sc) * (float)q - (w->dmin * (float)m);
}

/* lib.rs:281-315: one sequential f32 chain over every element of the row. */
int ref_dot_q4_k_q8a(const ref_q4k_block *w, const ref_q8a_block *a, size_t nsb, float *out) {
    if (nsb == 0) return QERR_INVALID_BLOCK_LENGTH;
    float sum = 0.0f;
    for (size_t b = 0; b < nsb; b++) {
        if (!isfinite(w[b].d) || !isfinite(w[b].dmin)) return QERR_NON_FINITE_SCALE;
        const ref_q8a_block *ab = a + b * (QKK / QK);
        for (size_t sub = 0; sub < 8; sub++) {
            uint8_t m;
            uint8_t sc = (uint8_t)ref_q4_k_scale_min(w[b].scales, sub, &m);
            float dsc = w[b].d * (float)sc;
            float dm = w[b].dmin * (float)m;
            const ref_q8a_block *blk = &ab[sub];
            if (!isfinite(blk->d)) return QERR_NON_FINITE_SCALE;
            for (size_t within = 0; within < 32; within++) {
                uint8_t byte = w[b].qs[(sub / 2) * 32 + within];
                uint8_t q = (sub % 2 == 0) ? (uint8_t)(byte & 0x0f) : (uint8_t)(byte >> 4);
                float weight = dsc * (float)q - dm;
                float activation = blk->d * (float)blk->q[within];
                float product = weight * activation;
                if (!isfinite(product)) return QERR_NON_FINITE_OUTPUT;
                sum += product;
                if (!isfinite(sum)) return QERR_NON_FINITE_OUTPUT;
            }
        }
    }
    *out = sum;
    return QERR_OK;
}

/* lib.rs:531-568 */
int8_t ref_q6_k_quant(const ref_q6k_block *w, size_t index) {
    size_t half = index / 128, within = index % 128;
    size_t l = within % 32, part = within / 32;
    size_t ql_base = half * 64, qh_base = half * 32;
    uint8_t ql;
    int shift;
    switch (part) {
    case 0: ql = w->ql[ql_base + l] & 0x0f; shift = 0; break;
    case 1: ql = w->ql[ql_base + l + 32] & 0x0f; shift = 2; break;
    case 2: ql = w->ql[ql_base + l] >> 4; shift = 4; break;
    default: ql = w->ql[ql_base + l + 32] >> 4; shift = 6; break;
    }
    uint8_t high = (uint8_t)(((w->qh[qh_base + l] >> shift) & 0x03) << 4);
    return (int8_t)((int8_t)(ql | high) - 32);
}

static size_t q6_k_scale_index(size_t index) {
    size_t half = index / 128, within = index % 128;
    size_t l = within % 32, part = within / 32;
    return half * 8 + l / 16 + 2 * part;
}

float ref_q6_k_value(const ref_q6k_block *w, size_t index) {
    return (w->d * (float)w->scales[q6_k_scale_index(index)]) * (float)ref_q6_k_quant(w, index);
}

/* lib.rs:353-397: exact i32 sums per lane (element index mod 8), one f32
 * accumulator per lane across superblocks, then a sequential lane combine. */
int ref_dot_q6_k_q8k(const ref_q6k_block *w, const ref_q8k_block *a, size_t nsb, float *out) {
    if (nsb == 0) return QERR_INVALID_BLOCK_LENGTH;
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (size_t b = 0; b < nsb; b++) {
        if (!isfinite(w[b].d) || !isfinite(a[b].d)) return QERR_NON_FINITE_SCALE;
        int32_t aux[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        size_t offset = 0;
        for (int s = 0; s < 16; s++) {
            int32_t scale = w[b].scales[s];
            for (int rep = 0; rep < 2; rep++) {
                for (int lane = 0; lane < 8; lane++)
                    aux[lane] += scale * (int32_t)a[b].q[offset + lane] *
                                 (int32_t)ref_q6_k_quant(&w[b], offset + lane);
                offset += 8;
            }
        }
        float d = w[b].d * a[b].d;
        if (!isfinite(d)) return QERR_NON_FINITE_OUTPUT;
        for (int lane = 0; lane < 8; lane++) {
            sums[lane] += d * (float)aux[lane];
            if (!isfinite(sums[lane])) return QERR_NON_FINITE_OUTPUT;
        }
    }
    float sum = 0.0f;
    for (int lane = 0; lane < 8; lane++) {
        sum += sums[lane];
        if (!isfinite(sum)) return QERR_NON_FINITE_OUTPUT;
    }
    *out = sum;
    return QERR_OK;
}

/* ---- AVX2 integer dot (the reference's simd feature, lib.rs:621-682) ---- */
#if defined(__x86_64__)
#include <immintrin.h>
__attribute__((target("avx2"))) float ref_dot_q8_0_q8a_block_avx2(const ref_q8_0_block *w,
                                                                   const ref_q8a_block *a) {
    __m256i x0 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)w->q));
    __m256i x1 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(w->q + 16)));
    __m256i y0 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)a->q));
    __m256i y1 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(a->q + 16)));
    __m256i s = _mm256_add_epi32(_mm256_madd_epi16(x0, y0), _mm256_madd_epi16(x1, y1));
    int32_t lanes[8];
    _mm256_storeu_si256((__m256i *)lanes, s);
    int32_t isum = 0;
    for (int i = 0; i < 8; i++) isum += lanes[i];
    float scale = w->d * a->d;
    return scale * (float)isum;
}
int ref_cpu_has_avx2(void) { return __builtin_cpu_supports("avx2"); }
#else
float ref_dot_q8_0_q8a_block_avx2(const ref_q8_0_block *w, const ref_q8a_block *a) {
    return ref_dot_q8_0_q8a_block(w, a);
}
int ref_cpu_has_avx2(void) { return 0; }
#endif

/* ---- public wrappers ---------------------------------------------------- */
int ref_quantize_q8a(const float *x, size_t n, float *d, int8_t *q) {
    if (n == 0 || n % QK) return REF_ERR_SHAPE;
    for (size_t b = 0; b < n / QK; b++) {
        ref_q8a_block blk;
        if (ref_q8a_block_quantize(x + b * QK, &blk)) return REF_ERR_NON_FINITE;
        d[b] = blk.d;
        memcpy(q + b * QK, blk.q, QK);
    }
    return REF_OK;
}

int ref_quantize_q8k(const float *x, size_t n, float *d, int8_t *q) {
    if (n == 0 || n % QKK) return REF_ERR_SHAPE;
    for (size_t b = 0; b < n / QKK; b++) {
        ref_q8k_block blk;
        if (ref_q8k_block_quantize(x + b * QKK, &blk)) return REF_ERR_NON_FINITE;
        d[b] = blk.d;
        memcpy(q + b * QKK, blk.q, QKK);
    }
    return REF_OK;
}

/* ---- det-cli known-answer generators (crates/det-cli/src/main.rs:273-388) */
static ref_q8_0_block gen_q8_block(uint32_t seed) {
    ref_q8_0_block b;
    uint32_t x = seed;
    for (int i = 0; i < QK; i++) {
        x = x * 1103515245u + 12345u;
        b.q[i] = (int8_t)((int16_t)((x >> 16) % 255) - 127);
    }
    b.d = u2f(0x3c000000u + (seed & 0xff));
    return b;
}

static ref_q8a_block gen_q8a_block(uint32_t seed) {
    ref_q8a_block b;
    uint32_t x = seed;
    for (int i = 0; i < QK; i++) {
        x = x * 22695477u + 1u;
        b.q[i] = (int8_t)((int16_t)((x >> 17) % 255) - 127);
    }
    b.d = u2f(0x3d000000u + (seed & 0xff));
    return b;
}

static ref_q4_0_block gen_q4_block(uint32_t seed) {
    ref_q4_0_block b;
    uint32_t x = seed;
    for (int i = 0; i < 16; i++) {
        x = x * 747796405u + 2891336453u;
        uint8_t lo = (uint8_t)((x >> 8) & 0x0f);
        uint8_t hi = (uint8_t)((x >> 20) & 0x0f);
        b.qs[i] = (uint8_t)(lo | (hi << 4));
    }
    b.d = u2f(0x3c800000u + (seed & 0xff));
    return b;
}

static ref_q4k_block gen_q4k_block(uint32_t seed) {
    ref_q4k_block b;
    memset(&b, 0, sizeof b);
    uint32_t x = seed;
    for (int i = 0; i < 4; i++) {
        x = x * 1664525u + 1013904223u;
        uint8_t scale = (uint8_t)((x >> 10) & 0x3f);
        x = x * 22695477u + 1u;
        uint8_t min = (uint8_t)((x >> 11) & 0x3f);
        b.scales[i] = scale & 0x3f;
        b.scales[i + 4] = min & 0x3f;
    }
    for (int i = 4; i < 8; i++) {
        x = x * 747796405u + 2891336453u;
        uint8_t scale = (uint8_t)((x >> 8) & 0x3f);
        x = x * 1103515245u + 12345u;
        uint8_t min = (uint8_t)((x >> 12) & 0x3f);
        b.scales[i + 4] = (uint8_t)((scale & 0x0f) | ((min & 0x0f) << 4));
        b.scales[i - 4] |= (uint8_t)((scale >> 4) << 6);
        b.scales[i] |= (uint8_t)((min >> 4) << 6);
    }
    for (int i = 0; i < 128; i++) {
        x = x * 1103515245u + 12345u;
        uint8_t lo = (uint8_t)((x >> 16) & 0x0f);
        x = x * 747796405u + 2891336453u;
        uint8_t hi = (uint8_t)((x >> 20) & 0x0f);
        b.qs[i] = (uint8_t)(lo | (hi << 4));
    }
    b.d = u2f(0x3b000000u + (seed & 0xff));
    b.dmin = u2f(0x3a800000u + ((seed >> 8) & 0xff));
    return b;
}

static ref_q6k_block gen_q6_block(uint32_t seed) {
    ref_q6k_block b;
    uint32_t x = seed;
    for (int i = 0; i < 128; i++) {
        x = x * 1664525u + 1013904223u;
        b.ql[i] = (uint8_t)(x >> 13);
    }
    for (int i = 0; i < 64; i++) {
        x = x * 22695477u + 1u;
        b.qh[i] = (uint8_t)(x >> 11);
    }
    for (int i = 0; i < 16; i++) {
        x = x * 747796405u + 2891336453u;
        b.scales[i] = (int8_t)((int16_t)((x >> 16) % 127) - 63);
    }
    b.d = u2f(0x3b800000u + (seed & 0xff));
    return b;
}

static void gen_q8a_blocks_for_q4k(uint32_t seed, ref_q8a_block out[8]) {
    for (uint32_t i = 0; i < 8; i++) out[i] = gen_q8a_block(seed + i * 0x85ebca6bu);
}

static int gen_q8k_block_for_q6(uint32_t seed, ref_q8k_block *out) {
    float input[QKK];
    for (uint32_t i = 0; i < QKK; i++) {
        uint32_t x = (seed + i * 0x9e3779b9u) * 747796405u + 2891336453u;
        input[i] = (float)(((int32_t)(x >> 9) % 4093) - 2046) / 257.0f;
    }
    return ref_q8k_block_quantize(input, out);
}

int ref_quant_kernel_hash(uint8_t out[32]) {
    ref_sha256_ctx c;
    ref_sha256_init(&c);
    for (uint32_t seed = 0; seed < 1000000u; seed++) {
        ref_q8_0_block q8 = gen_q8_block(seed);
        ref_q4_0_block q4 = gen_q4_block(seed ^ 0xa5a55a5au);
        ref_q8a_block a = gen_q8a_block(seed * 1664525u + 1013904223u);
        float y8 = ref_dot_q8_0_q8a_block(&q8, &a);
        float y4 = ref_dot_q4_0_q8a_block(&q4, &a);
        if (!isfinite(y8) || !isfinite(y4)) return REF_ERR_QUANT;
        ref_sha256_f32(&c, y8);
        ref_sha256_f32(&c, y4);
    }
    for (uint32_t seed = 0; seed < 4096u; seed++) {
        ref_q4k_block q4k = gen_q4k_block(seed ^ 0x9e3779b9u);
        ref_q8a_block a4k[8];
        gen_q8a_blocks_for_q4k(seed, a4k);
        float y;
        if (ref_dot_q4_k_q8a(&q4k, a4k, 1, &y)) return REF_ERR_QUANT;
        ref_sha256_f32(&c, y);
    }
    for (uint32_t seed = 0; seed < 4096u; seed++) {
        ref_q6k_block q6 = gen_q6_block(seed ^ 0x517cc1b7u);
        ref_q8k_block a6;
        if (gen_q8k_block_for_q6(seed, &a6)) return REF_ERR_QUANT;
        float y;
        if (ref_dot_q6_k_q8k(&q6, &a6, 1, &y)) return REF_ERR_QUANT;
        ref_sha256_f32(&c, y);
    }
    ref_sha256_final(&c, out);
    return REF_OK;
}

/* main.rs:146-224 (the rmsnorm and CDF pieces call the model/coder code). */
int ref_rmsnorm(const float *x, const float *w, float eps, size_t n, float *out);
int ref_logits_to_cdf(const float *logits, size_t n, size_t tail, uint32_t *freq, uint64_t *cum,
                      uint64_t *total);

int ref_runtime_canary(uint8_t out[32]) {
    ref_sha256_ctx c;
    ref_sha256_init(&c);
    for (uint32_t seed = 0; seed < 16; seed++) {
        ref_q8_0_block q8 = gen_q8_block(seed);
        ref_q4_0_block q4 = gen_q4_block(seed ^ 0xa5a55a5au);
        ref_q8a_block a = gen_q8a_block(seed * 1664525u + 1013904223u);
        ref_q4k_block q4k = gen_q4k_block(seed ^ 0x9e3779b9u);
        ref_q8a_block a4k[8];
        gen_q8a_blocks_for_q4k(seed, a4k);
        ref_q6k_block q6 = gen_q6_block(seed ^ 0x517cc1b7u);
        ref_q8k_block a6;
        if (gen_q8k_block_for_q6(seed, &a6)) return REF_ERR_QUANT;
        float y8 = ref_dot_q8_0_q8a_block(&q8, &a);
        float y4 = ref_dot_q4_0_q8a_block(&q4, &a);
        float y4k, y6;
        if (ref_dot_q4_k_q8a(&q4k, a4k, 1, &y4k)) return REF_ERR_QUANT;
        if (ref_dot_q6_k_q8k(&q6, &a6, 1, &y6)) return REF_ERR_QUANT;
        ref_sha256_f32(&c, y8);
        ref_sha256_f32(&c, y4);
        ref_sha256_f32(&c, y4k);
        ref_sha256_f32(&c, y6);
    }
    float q_input[QK];
    for (int i = 0; i < QK; i++) {
        if (i == 0) q_input[i] = u2f(1);
        else if (i == 1) q_input[i] = -u2f(2);
        else q_input[i] = (float)((i % 11) - 5) * 0.03125f;
    }
    ref_q8a_block q;
    if (ref_q8a_block_quantize(q_input, &q)) return REF_ERR_QUANT;
    ref_sha256_f32(&c, q.d);
    ref_sha256_update(&c, q.q, QK);

    float x[8] = {u2f(1), -0.75f, 1.25f, -2.0f, 3.5f, -4.25f, 0.5f, -0.125f};
    float w[8] = {1.0f, -0.5f, 0.25f, -1.5f, 2.0f, -2.5f, 0.75f, -0.25f};
    float rms[8];
    if (ref_rmsnorm(x, w, 1e-5f, 8, rms)) return REF_ERR_NON_FINITE;
    for (int i = 0; i < 8; i++) ref_sha256_f32(&c, rms[i]);

    float logits[11] = {0.0f, -1.0f, 3.25f, 3.25f, -88.5f, u2f(1), -12.0f, 0.5f, -0.25f, 2.0f,
                        -1000.0f};
    uint32_t freq[11];
    uint64_t cum[11], total;
    int st = ref_logits_to_cdf(logits, 11, 0, freq, cum, &total);
    if (st) return st;
    for (int i = 0; i < 11; i++) {
        uint8_t b[4] = {(uint8_t)freq[i], (uint8_t)(freq[i] >> 8), (uint8_t)(freq[i] >> 16),
                        (uint8_t)(freq[i] >> 24)};
        ref_sha256_update(&c, b, 4);
    }
    for (int i = 0; i < 11; i++) {
        uint8_t b[8];
        for (int k = 0; k < 8; k++) b[k] = (uint8_t)(cum[i] >> (8 * k));
        ref_sha256_update(&c, b, 8);
    }
    {
        uint8_t b[8];
        for (int k = 0; k < 8; k++) b[k] = (uint8_t)(total >> (8 * k));
        ref_sha256_update(&c, b, 8);
    }
    ref_sha256_final(&c, out);
    return REF_OK;
}
