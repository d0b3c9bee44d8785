"""Pins the CPU oracle against everything the reference fixes.

Golden values come from the reference's own files (testdata/*.sha256,
det-num canary.rs EXPECTED, det-cli RUNTIME_CANARY_EXPECTED, the recorded
quant-kernel-hash in docs/validation.md:343, det-num / det-quant / det-coder
unit anchors).  Where those leave a gap (multi-block rows, RoPE tables at
large positions), closed forms and library math pin it instead.
"""
import ctypes as C
import math
import struct

import numpy as np
import pytest

import detref
import qblocks
from conftest import GOLDEN

L = detref.lib()


def bits(v: float) -> int:
    return struct.unpack("<I", struct.pack("<f", v))[0]


def dbits(v: float) -> int:
    return struct.unpack("<Q", struct.pack("<d", v))[0]


def h32(fn):
    out = (C.c_uint8 * 32)()
    rc = fn(out)
    assert rc in (None, 0)
    return bytes(out).hex()


# ---- det-num ------------------------------------------------------------------

def test_numeric_canary_matches_reference():
    # crates/det-num/src/canary.rs:3-6
    assert h32(L.ref_numeric_canary) == "2e42e5507cc1bfd7111a5a0f3c28056d669e05ea0f627d1b92d92ec7fec17a5d"


def test_runtime_canary_matches_reference():
    # crates/det-cli/src/main.rs:5-8 (Q8_0/Q4_0/Q4_K/Q6_K dots, Q8A, rmsnorm, CDF)
    assert h32(L.ref_runtime_canary) == "055d04e336f748129f5d80250fe945eba6c82893c289ce284dc09ecbc8035095"


def test_quant_kernel_hash_matches_recorded_value():
    # docs/validation.md:343 (1M Q8_0+Q4_0 blocks, 4096 Q4_K, 4096 Q6_K)
    assert h32(L.ref_quant_kernel_hash) == "99832eb2ac8ddeb15731805e876a36b4013ae41c2aca0783ea02890fe9b0efba"


def test_exp_f32_anchors():
    # crates/det-num/src/math.rs:41-46
    assert bits(L.ref_exp_f32(-88.0)) == 0x0041EDC4
    assert bits(L.ref_exp_f32(0.0)) == 0x3F800000
    assert bits(L.ref_exp_f32(1.0)) == 0x402DF854
    assert bits(L.ref_exp_f32(-1.0)) == 0x3EBC5AB2


def test_exp_f32_is_within_one_ulp_of_true_exp():
    # FreeBSD expf is accurate to < 1 ulp: a dropped term or wrong constant fails.
    xs = np.linspace(-103.0, 88.5, 20001).astype(np.float32)
    got = detref.exp_f32(xs).astype(np.float64)
    want = np.exp(xs.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    ulp = np.maximum(ulp, 2.0 ** -149)
    assert np.all(np.abs(got - want) <= ulp)


def test_f64_transcendental_anchors():
    # crates/det-num/src/math.rs:49-62
    assert dbits(L.ref_exp_f64(1.0)) == 0x4005BF0A8B14576A
    assert dbits(L.ref_ln_f64(10000.0)) == 0x40226BB1BBB55516
    assert dbits(L.ref_sin_f64(0.0)) == 0
    assert dbits(L.ref_cos_f64(0.0)) == dbits(1.0)
    assert dbits(L.ref_sin_f64(math.pi / 2)) == dbits(1.0)
    assert dbits(L.ref_cos_f64(math.pi / 2)) == 0x3C91A62633145C07


def test_f64_transcendentals_agree_with_libm():
    rng = np.random.default_rng(1)
    for x in rng.uniform(-2100.0, 2100.0, 4000):
        assert abs(L.ref_sin_f64(x) - math.sin(x)) <= 2 * math.ulp(1.0)
        assert abs(L.ref_cos_f64(x) - math.cos(x)) <= 2 * math.ulp(1.0)
    for x in rng.uniform(1e-3, 2e6, 2000):
        assert abs(L.ref_ln_f64(x) - math.log(x)) <= 2 * math.ulp(math.log(x))
    for x in rng.uniform(-700, 700, 2000):
        assert abs(L.ref_exp_f64(x) - math.exp(x)) <= 2 * math.ulp(math.exp(x))


def test_f16_conversion():
    # crates/det-num/src/f16.rs:41-49; all 65536 codes against numpy's IEEE half
    assert bits(L.ref_f16_to_f32(0x0000)) == 0
    assert bits(L.ref_f16_to_f32(0x8000)) == 0x80000000
    assert L.ref_f16_to_f32(0x3C00) == 1.0
    assert L.ref_f16_to_f32(0xC000) == -2.0
    assert L.ref_f16_to_f32(0x7BFF) == 65504.0
    codes = np.arange(65536, dtype=np.uint16)
    want = codes.view(np.float16).astype(np.float32)
    got = np.array([L.ref_f16_to_f32(int(c)) for c in codes], np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.array_equal(np.isinf(got), np.isinf(want))


def test_round_ties_even():
    # crates/det-num/src/round.rs:46-57
    for x, y in [(0.5, 0), (1.5, 2), (2.5, 2), (-0.5, 0), (-1.5, -2), (-2.5, -2)]:
        assert L.ref_round_ties_even_i32(x) == y
    for x, y in [(2.5, 2), (3.5, 4), (-2.5, -2), (-3.5, -4)]:
        assert L.ref_round_ties_even_i64(x) == y


def test_dot_uses_8_lane_order():
    # crates/det-num/src/reduce.rs:44-61 with a case where order changes bits
    x = np.array([1e8, 1.0, -1e8, 1.0, 3.0, 5.0, 7.0, 11.0, 1.0], np.float32)
    y = np.ones_like(x)
    acc = [np.float32(0)] * 8
    for i in range(x.size):
        acc[i % 8] = np.float32(acc[i % 8] + np.float32(x[i] * y[i]))
    a = acc
    want = np.float32(np.float32(np.float32(a[0] + a[1]) + np.float32(a[2] + a[3]))
                      + np.float32(np.float32(a[4] + a[5]) + np.float32(a[6] + a[7])))
    got = L.ref_dot_f32(x.ctypes.data_as(C.POINTER(C.c_float)), y.ctypes.data_as(C.POINTER(C.c_float)), x.size)
    assert bits(got) == bits(float(want))
    assert got != float(np.sum(x.astype(np.float64)))  # a naive order would give 29


# ---- det-quant --------------------------------------------------------------------

def test_q8a_quantizer_anchors():
    # crates/det-quant/src/lib.rs:825-842: zero block and half-away rounding
    d, q = detref.quantize_q8a(np.zeros(32, np.float32))
    assert bits(d[0]) == 0 and not q.any()
    x = np.zeros(32, np.float32)
    x[0], x[1], x[2] = 127.0, 0.5, -0.5
    d, q = detref.quantize_q8a(x)
    assert d[0] == 1.0 and q[0] == 127 and q[1] == 1 and q[2] == -1


def test_q8k_uses_first_signed_max():
    x = np.zeros(256, np.float32)
    x[5], x[9] = -3.0, 3.0  # same |x|: the first one (negative) sets the sign
    d, q = detref.quantize_q8k(x)
    assert d[0] == np.float32(1.0) / (np.float32(-127.0) / np.float32(-3.0))
    assert q[5] == -127 and q[9] == 127
    x[5], x[9] = 3.0, -3.0  # now the positive one comes first: signs flip
    d2, q2 = detref.quantize_q8k(x)
    assert d2[0] == -d[0] and q2[5] == -127 and q2[9] == 127


def _exact_activation(rng, cols):
    """Integer activations with amax 127 in every 32-block: Q8A d == 1."""
    x = rng.integers(-127, 128, cols).astype(np.float32)
    x[::32] = 127.0
    return x


@pytest.mark.parametrize("nb", [1, 3, 7])
def test_q8_0_row_closed_form(nb):
    rng = np.random.default_rng(nb)
    cols = 32 * nb
    q = rng.integers(-127, 128, (nb, 32))
    row = qblocks.q8_0_row(np.full(nb, qblocks.F16_ONE, np.uint16), q)
    x = _exact_activation(rng, cols)
    assert detref.dot_row(8, row, cols, x) == float(np.dot(q.reshape(-1), x.astype(np.int64)))


@pytest.mark.parametrize("nb", [1, 4])
def test_q4_0_row_closed_form(nb):
    rng = np.random.default_rng(10 + nb)
    cols = 32 * nb
    nib = rng.integers(0, 16, (nb, 32))
    row = qblocks.q4_0_row(np.full(nb, qblocks.F16_ONE, np.uint16), nib)
    x = _exact_activation(rng, cols)
    w = nib.reshape(-1) - 8
    assert detref.dot_row(2, row, cols, x) == float(np.dot(w, x.astype(np.int64)))


@pytest.mark.parametrize("nsb", [1, 2, 3])
def test_q4_k_row_closed_form(nsb):
    # Multi-superblock rows: the element order and nibble/scale layout are
    # fixed by an independent integer decode of the GGUF bytes.
    rng = np.random.default_rng(20 + nsb)
    cols = 256 * nsb
    sc = rng.integers(0, 8, (nsb, 8))
    mn = rng.integers(0, 8, (nsb, 8))
    nib = rng.integers(0, 16, (nsb, 256))
    one = np.full(nsb, qblocks.F16_ONE, np.uint16)
    row = qblocks.q4_k_row(one, one, sc, mn, nib)
    q, s, m = qblocks.decode_q4_k_codes(row, cols)
    assert np.array_equal(q, nib.reshape(-1))
    x = _exact_activation(rng, cols)
    want = float(np.dot(s * q - m, x.astype(np.int64)))
    assert detref.dot_row(12, row, cols, x) == want


@pytest.mark.parametrize("nsb", [1, 2, 3])
def test_q6_k_row_closed_form(nsb):
    rng = np.random.default_rng(30 + nsb)
    cols = 256 * nsb
    sc = rng.integers(-7, 8, (nsb, 16))
    q6 = rng.integers(-32, 32, (nsb, 256))
    row = qblocks.q6_k_row(np.full(nsb, qblocks.F16_ONE, np.uint16), sc, q6)
    qd, sd = qblocks.decode_q6_k(row, cols)
    assert np.array_equal(qd, q6.reshape(-1))
    x = rng.integers(-126, 127, cols).astype(np.float32)
    x[::256] = 127.0  # first max |x| of every superblock is +127: Q8_K d == -1
    want = float(np.dot(sd * qd, x.astype(np.int64)))
    assert detref.dot_row(14, row, cols, x) == want


# ---- det-model ----------------------------------------------------------------------

def _hash_fixture(name, chunk=1):
    m = detref.Model((GOLDEN / f"{name}.gguf").read_bytes())
    toks = [int(t) for t in (GOLDEN / "tiny.tokens.txt").read_text().strip().split(",")]
    return m.logits_hash(toks, chunk).hex(), (GOLDEN / f"{name}.logits.sha256").read_text().strip()


@pytest.mark.parametrize("name", ["tiny-f32", "tiny-qmix"])
def test_fixture_logits_hash_matches_reference(name):
    got, want = _hash_fixture(name)
    assert got == want


@pytest.mark.parametrize("threads", [1, 2, 7])
def test_fixture_hash_is_thread_invariant(threads):
    detref.set_threads(threads)
    try:
        got, want = _hash_fixture("tiny-qmix", 3)
    finally:
        detref.set_threads(0)
    assert got == want


def test_rope_pairing_anchors():
    # det-model lib.rs:2751-2820: position 1 of a table with cos (0, 0.5),
    # sin (1, -0.25); adjacent and split-half pairs, and a non-rotary tail.
    c, s = [0.0, 0.5], [1.0, -0.25]
    bits = lambda a: np.asarray(a, np.float32).view(np.uint32)
    got = detref.apply_rope([1, 2, 3, 4, 5, 6, 7, 8], 2, 4, 4, False, c, s)
    assert np.array_equal(bits(got), bits([-2.0, 1.0, 2.5, 1.25, -6.0, 5.0, 5.5, 2.25]))
    got = detref.apply_rope([1, 2, 3, 4], 1, 4, 4, True, c, s)
    assert np.array_equal(bits(got), bits([-3.0, 2.0, 1.0, 1.5]))
    got = detref.apply_rope([1, 2, 3, 4, 9, -9], 1, 6, 4, False, c, s)
    assert np.array_equal(bits(got), bits([-2.0, 1.0, 2.5, 1.25, 9.0, -9.0]))
    got = detref.apply_rope([1, 2, 3, 4, 9, -9], 1, 6, 4, True, c, s)
    assert np.array_equal(bits(got), bits([-3.0, 2.0, 1.0, 1.5, 9.0, -9.0]))
    # A swapped pairing or sign is caught by the same anchors.
    assert not np.array_equal(bits(detref.apply_rope([1, 2, 3, 4], 1, 4, 4, False, c, s)),
                              bits([-3.0, 2.0, 1.0, 1.5]))


def test_rmsnorm_order():
    # det-model lib.rs:2442-2459
    x = np.array([1.0, -2.0, 3.0, -4.0], np.float32)
    w = np.array([0.5, 1.0, 1.5, 2.0], np.float32)
    ss = np.float32(30.0)
    r = np.float32(1.0) / np.sqrt(np.float32(ss / np.float32(4.0) + np.float32(1e-5)))
    want = ((x * r) * w).astype(np.float32)
    assert np.array_equal(detref.rmsnorm(x, w, 1e-5).view(np.uint32), want.view(np.uint32))


def test_rope_table_tracks_libm_at_long_context():
    # Positions up to 2047 and theta 1e4 / 1e5 / 1e6: fdlibm agrees with
    # glibc to within one f64 ulp, so the f32 tables agree except on rare
    # double-rounding ties.
    from detllm_amd import synth
    for name in ("tiny", "smollm2"):
        w = synth.WORKLOADS[name]
        m = detref.Model(synth.build_model(w, layers=1))
        positions = min(w.ctx, 2048)
        c, s = m.rope_table(positions)
        half = c.size // positions
        j = np.arange(half)
        omega = np.exp(-(2.0 * j / (2 * half)) * math.log(np.float32(w.rope_base)))
        phi = np.arange(positions)[:, None] * omega[None, :]
        assert np.mean(c.reshape(positions, half) == np.cos(phi).astype(np.float32)) > 0.9999
        assert np.mean(s.reshape(positions, half) == np.sin(phi).astype(np.float32)) > 0.9999


# ---- det-coder ------------------------------------------------------------------------

def test_cdf_uniform_logits_closed_form():
    # det-coder cdf.rs:447-462: no renormalisation to a fixed total
    freq, cum, total = detref.logits_to_cdf(np.zeros(4, np.float32))
    assert list(freq) == [4194305] * 4
    assert list(cum) == [0, 4194305, 8388610, 12582915]
    assert total == 16777220


def test_cdf_clamp_equivalence():
    # cdf.rs:464-481
    a = detref.logits_to_cdf(np.array([0.0, -88.0, -88.0, -0.5], np.float32))
    b = detref.logits_to_cdf(np.array([0.0, -1000.0, -1.0e30, -0.5], np.float32))
    assert all(np.array_equal(x, y) for x, y in zip(a[:2], b[:2])) and a[2] == b[2]


def test_symbol_range_and_decoder_agree_with_full_cdf():
    rng = np.random.default_rng(5)
    lg = rng.normal(0, 3, 300).astype(np.float32)
    for tail in (0, 256):
        freq, cum, total = detref.logits_to_cdf(lg, tail)
        for s in list(range(0, 300, 37)) + [299 + tail]:
            assert detref.symbol_range(lg, s, tail) == (int(cum[s]), int(freq[s]), total)
            for v in (int(cum[s]), int(cum[s]) + int(freq[s]) - 1):
                assert detref.decoder_lookup(lg, v, tail) == (s, int(cum[s]), int(freq[s]), total)


def test_range_coder_roundtrip():
    rng = np.random.default_rng(7)
    triples = []
    for _ in range(2000):
        total = int(rng.integers(2, 1 << 30))
        cum = int(rng.integers(0, total - 1))
        freq = int(rng.integers(1, total - cum + 1))
        triples.append((cum, freq, total))
    data = detref.range_encode(triples)
    st = C.c_int()
    buf = (C.c_uint8 * len(data)).from_buffer_copy(data)
    d = L.ref_range_decoder_new(buf, len(data), C.byref(st))
    assert d
    v = C.c_uint64()
    for cum, freq, total in triples:
        assert L.ref_range_decode_freq(d, total, C.byref(v)) == 0
        assert cum <= v.value < cum + freq
        assert L.ref_range_decode_advance(d, cum, freq, total) == 0
    L.ref_range_decoder_free(d)


def test_oracle_exp_array_matches_scalar_binding():
    """The array form of the oracle's exp_f32 (used to check the device's
    exp over millions of bit patterns) agrees with the scalar form, which
    the reference's anchors above pin, on a strided sweep of both signs;
    with clamp it is exp_f32(max(x, -88))."""
    bits = np.arange(0, 2**32, 65521, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    assert np.array_equal(detref.exp_f32_array(x).view(np.uint32), detref.exp_f32(x).view(np.uint32))
    want = detref.exp_f32(np.maximum(x, np.float32(-88.0)))
    assert np.array_equal(detref.exp_f32_array(x, clamp=True).view(np.uint32), want.view(np.uint32))
