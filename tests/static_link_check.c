/* A C host linked against libdetllm_amd.a (not the shared library) through
 * include/detllm.h, calling host-only entry points: the range coder, the DTLZ
 * header, the codec window schedule, the uniform symbol range and the status
 * strings.  It prints one line per result for tests/test_static_lib.py,
 * which compares them with the oracle and the shared library.
 *
 * Symbols: a fixed 64-bit LCG draws `n` (cum, freq, total) triples with
 * total in [2, 2^31), freq in [1, total - cum].  The same generator is
 * restated in the test. */
#include <inttypes.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "detllm.h"

static uint64_t lcg(uint64_t *s) {
    *s = *s * 6364136223846793005ull + 1442695040888963407ull;
    return *s >> 17;
}

static void draw(uint64_t *s, uint64_t *cum, uint64_t *freq, uint64_t *total) {
    uint64_t t = 2 + lcg(s) % ((1ull << 31) - 2);
    uint64_t c = lcg(s) % t;
    uint64_t room = t - c;
    uint64_t f = 1 + lcg(s) % (room < 4096 ? room : 4096);
    *cum = c;
    *freq = f;
    *total = t;
}

static int fail(const char *what, int st) {
    printf("FAIL %s %d %s\n", what, st, dtl_status_string(st));
    return 1;
}

int main(int argc, char **argv) {
    size_t n = argc > 1 ? (size_t)strtoull(argv[1], 0, 10) : 1000;
    uint64_t seed = argc > 2 ? strtoull(argv[2], 0, 10) : 7;

    /* range coder: encode n triples, print the payload, decode it back */
    dtl_range_encoder *enc = 0;
    int st = dtl_range_encoder_new(&enc);
    if (st) return fail("encoder_new", st);
    uint64_t s = seed;
    for (size_t i = 0; i < n; i++) {
        uint64_t c, f, t;
        draw(&s, &c, &f, &t);
        st = dtl_range_encode(enc, c, f, t);
        if (st) return fail("encode", st);
    }
    size_t len = 0;
    st = dtl_range_encoder_finish(enc, 0, 0, &len);
    if (st && st != DTL_ERR_BUFFER_TOO_SMALL) return fail("finish_size", st);
    uint8_t *payload = (uint8_t *)malloc(len ? len : 1);
    st = dtl_range_encoder_finish(enc, payload, len, &len);
    if (st) return fail("finish", st);
    dtl_range_encoder_free(enc);
    printf("payload ");
    for (size_t i = 0; i < len; i++) printf("%02x", payload[i]);
    printf("\n");

    dtl_range_decoder *dec = 0;
    st = dtl_range_decoder_new(payload, len, &dec);
    if (st) return fail("decoder_new", st);
    s = seed;
    for (size_t i = 0; i < n; i++) {
        uint64_t c, f, t, v;
        draw(&s, &c, &f, &t);
        st = dtl_range_decode_freq(dec, t, &v);
        if (st) return fail("decode_freq", st);
        if (v < c || v >= c + f) {
            printf("FAIL decode symbol %zu: value %" PRIu64 " outside [%" PRIu64 ", %" PRIu64 ")\n", i, v,
                   c, c + f);
            return 1;
        }
        st = dtl_range_decode_advance(dec, c, f, t);
        if (st) return fail("decode_advance", st);
    }
    dtl_range_decoder_free(dec);
    printf("roundtrip ok %zu\n", n);
    free(payload);

    /* an invalid frequency is refused with the reference's error */
    st = dtl_range_encoder_new(&enc);
    if (st) return fail("encoder_new", st);
    printf("zero_freq_status %d\n", dtl_range_encode(enc, 0, 0, 10));
    dtl_range_encoder_free(enc);

    /* DTLZ header */
    uint8_t sha[32], hdr[DTL_DTLZ_HEADER_LEN];
    for (int i = 0; i < 32; i++) sha[i] = (uint8_t)(3 * i + 1);
    st = dtl_dtlz_header_encode(DTL_DTLZ_FLAG_BYTE_ESCAPES, sha, 2048, 512, 1048576, hdr);
    if (st) return fail("header_encode", st);
    printf("header ");
    for (unsigned i = 0; i < DTL_DTLZ_HEADER_LEN; i++) printf("%02x", hdr[i]);
    printf("\n");
    uint16_t flags = 0;
    uint8_t sha2[32];
    uint32_t n_ctx = 0, overlap = 0;
    uint64_t orig = 0;
    st = dtl_dtlz_header_decode(hdr, sizeof hdr, &flags, sha2, &n_ctx, &overlap, &orig);
    if (st) return fail("header_decode", st);
    printf("header_fields %u %u %u %" PRIu64 " %d\n", flags, n_ctx, overlap, orig, memcmp(sha, sha2, 32) == 0);
    hdr[0] = 'X';
    printf("bad_magic_status %d\n", dtl_dtlz_header_decode(hdr, sizeof hdr, &flags, sha2, &n_ctx, &overlap, &orig));

    /* codec window schedule (n_ctx 8, overlap 2) over the first 20 positions */
    printf("windows");
    size_t ws = 0;
    for (size_t pos = 0; pos < 20; pos++) {
        ws = dtl_codec_next_window_start(pos, ws, 8, 2);
        printf(" %zu", ws);
    }
    printf("\n");

    /* uniform symbol range over vocab 256 + 256 escapes */
    uint64_t cum = 0, total = 0;
    uint32_t freq = 0;
    st = dtl_uniform_symbol_range(300, 512, &cum, &freq, &total);
    printf("uniform %d %" PRIu64 " %u %" PRIu64 "\n", st, cum, freq, total);

    /* status strings */
    int codes[] = {0, 1, 20, 30, 45, 80, 81};
    for (unsigned i = 0; i < sizeof codes / sizeof codes[0]; i++)
        printf("status %d %s\n", codes[i], dtl_status_string(codes[i]));
    return 0;
}
