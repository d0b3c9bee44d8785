/* Internal declarations shared by the oracle's translation units
 * (TEST INFRASTRUCTURE ONLY). */
#ifndef DETREF_INTERNAL_H
#define DETREF_INTERNAL_H

#include <stddef.h>
#include <stdint.h>

typedef struct {
    uint32_t st[8];
    uint64_t len;
    uint8_t buf[64];
    size_t buf_len;
} ref_sha256_ctx;

void ref_sha256_init(ref_sha256_ctx *c);
void ref_sha256_update(ref_sha256_ctx *c, const void *data, size_t len);
void ref_sha256_final(ref_sha256_ctx *c, uint8_t out[32]);
void ref_sha256_f32(ref_sha256_ctx *c, float v);

float ref_finish_8lane(const float acc[8]);
int32_t ref_f32_as_i32(float x);
int ref_f16_is_finite(uint16_t bits);

/* det-quant block types (crates/det-quant/src/lib.rs:20-59); scales are
 * held as f32 exactly like the reference's in-memory structs. */
#define QK 32
#define QKK 256
typedef struct { float d; int8_t q[QK]; } ref_q8a_block;
typedef struct { float d; int8_t q[QKK]; } ref_q8k_block;
typedef struct { float d; int8_t q[QK]; } ref_q8_0_block;
typedef struct { float d; uint8_t qs[16]; } ref_q4_0_block;
typedef struct { float d; float dmin; uint8_t scales[12]; uint8_t qs[128]; } ref_q4k_block;
typedef struct { float d; uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; } ref_q6k_block;

enum { QERR_OK = 0, QERR_LENGTH_MISMATCH, QERR_INVALID_BLOCK_LENGTH, QERR_NON_FINITE_INPUT,
       QERR_NON_FINITE_SCALE, QERR_NON_FINITE_OUTPUT };

int ref_q8a_block_quantize(const float *x, ref_q8a_block *out);
int ref_q8k_block_quantize(const float *x, ref_q8k_block *out);
float ref_dot_q8_0_q8a_block(const ref_q8_0_block *w, const ref_q8a_block *a);
float ref_dot_q4_0_q8a_block(const ref_q4_0_block *w, const ref_q8a_block *a);
int ref_dot_q8_0_q8a(const ref_q8_0_block *w, const ref_q8a_block *a, size_t nb, float *out);
int ref_dot_q4_0_q8a(const ref_q4_0_block *w, const ref_q8a_block *a, size_t nb, float *out);
int ref_dot_q4_k_q8a(const ref_q4k_block *w, const ref_q8a_block *a, size_t nsb, float *out);
int ref_dot_q6_k_q8k(const ref_q6k_block *w, const ref_q8k_block *a, size_t nsb, float *out);
float ref_q4_k_value(const ref_q4k_block *w, size_t index);
float ref_q6_k_value(const ref_q6k_block *w, size_t index);
int ref_q4_k_scale_min(const uint8_t scales[12], size_t index, uint8_t *mn);
int8_t ref_q6_k_quant(const ref_q6k_block *w, size_t index);

/* AVX2 exact integer block dot used by the threaded CPU baseline; it
 * returns the same bits as the scalar block dot (integer sums are exact). */
float ref_dot_q8_0_q8a_block_avx2(const ref_q8_0_block *w, const ref_q8a_block *a);
int ref_cpu_has_avx2(void);

#endif
