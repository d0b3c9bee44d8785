"""Kernel-level parity of the HIP implementation against the oracle (bit-exact)."""
import ctypes as C

import numpy as np
import pytest

import detref
import qblocks

pytestmark = pytest.mark.gpu


def _lib():
    from detllm_amd import _lib

    return _lib


def _p(a, t):
    return a.ctypes.data_as(C.POINTER(t))


def gpu_exp(x, which="exp"):
    L = _lib()
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    fn = L.lib.dtl_kernel_exp_f32 if which == "exp" else L.lib.dtl_kernel_silu_f32
    L.check(fn(_p(x, C.c_float), _p(out, C.c_float), x.size), which)
    return out


def test_exp_f32_bitexact_sweep():
    rng = np.random.default_rng(0)
    # every f32 in [-1, 0] spaced by 64 ulps, a dense band near the clamp,
    # random values over the whole range and the special cases
    a = np.arange(0xBF800000, 0x80000000, -64, dtype=np.uint64).astype(np.uint32).view(np.float32)
    b = np.linspace(-104.0, 89.0, 400000, dtype=np.float32)
    c = rng.uniform(-120, 100, 200000).astype(np.float32)
    special = np.array([0.0, -0.0, -88.0, -87.33655, -88.72284, 88.72284, 88.7229, -103.972084,
                        -103.97209, 1e-30, -1e-30, np.float32(2 ** -149), 0.3465735, -0.3465735,
                        1.0397208, -1.0397208, np.inf, -np.inf], np.float32)
    x = np.concatenate([a, b, c, special])
    got = gpu_exp(x)
    want = detref.exp_f32(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_exp_f32_strided_all_bit_patterns():
    """Every 257th f32 bit pattern (both signs, subnormals, infinities, NaN
    payloads) against the oracle: the device exp is branch-free, every path
    selected, so each range must land on the reference's path."""
    bits = np.arange(0, 2**32, 257, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    got = gpu_exp(x).view(np.uint32)
    # NaN inputs come back as they are (expf.rs:50-53 returns x).  The oracle
    # binding passes values through a C double, which quiets signalling
    # NaNs, so those are checked against the input bits instead.
    nan = (bits & 0x7fffffff) > 0x7f800000
    assert np.array_equal(got[nan], bits[nan])
    want = detref.exp_f32(x[~nan]).view(np.uint32)
    assert np.array_equal(got[~nan], want)


def test_exp_clamped_device_matches_oracle():
    """The device's exp for softmax and the CDF (exp_f32(max(t, -88)) restated
    for t <= 0) against the oracle's exp_f32 of max(t, -88): every 61st
    pattern with the sign bit set (-0, subnormals, normals, -inf), every
    pattern in the bands around its branch points (|t| near 2^-13, ln2/2,
    1.5 ln2, the -88 clamp and the k = -126 / -127 scaling steps), and +0.
    The host check tests/exp_nonpos_check.c covers all 2^31 patterns of the
    same restatement."""
    L = _lib()
    bits = np.arange(0x80000000, 0x100000000, 61, dtype=np.uint64).astype(np.uint32)
    bands = [np.arange(c - 4096, c + 4096, dtype=np.uint64).astype(np.uint32) | np.uint32(0x80000000)
             for c in (0x39000000, 0x3EB17218, 0x3F851592, 0x42B00000, 0x42AEAC50, 0x42AF0000, 0x42AE0000)]
    x = np.concatenate([bits, *bands, np.array([0], np.uint32)]).view(np.float32)
    x = np.ascontiguousarray(x[~np.isnan(x)])
    out = np.empty_like(x)
    L.check(L.lib.dtl_kernel_exp_clamped_f32(_p(x, C.c_float), _p(out, C.c_float), x.size), "exp_clamped")
    want = detref.exp_f32_array(x, clamp=True)
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))
    # outside the domain: refused on the host
    y = np.array([-1.0, 0.5], np.float32)
    assert L.lib.dtl_kernel_exp_clamped_f32(_p(y, C.c_float), _p(out, C.c_float), 2) == 42


def test_silu_bitexact():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.normal(0, 4, 100000), rng.uniform(-100, 100, 50000)]).astype(np.float32)
    got = gpu_exp(x, "silu")
    f = detref.lib().ref_silu_f32
    want = np.array([f(float(v)) for v in x], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_f16_to_f32_exhaustive():
    L = _lib()
    codes = np.arange(65536, dtype=np.uint16)
    out = np.empty(65536, np.float32)
    L.check(L.lib.dtl_kernel_f16_to_f32(_p(codes, C.c_uint16), _p(out, C.c_float), 65536), "f16")
    f = detref.lib().ref_f16_to_f32
    # The oracle returns through a C double, which quiets signalling NaNs, so
    # NaN codes are checked against numpy's bit-level half -> single widening.
    nan = np.isnan(codes.view(np.float16))
    want = np.array([f(int(c)) for c in codes], np.float32)
    assert np.array_equal(out[~nan].view(np.uint32), want[~nan].view(np.uint32))
    want_nan = codes[nan].view(np.float16).astype(np.float32)
    assert np.array_equal(out[nan].view(np.uint32), want_nan.view(np.uint32))


def test_div_and_sqrt_are_correctly_rounded():
    L = _lib()
    rng = np.random.default_rng(2)
    n = 1 << 20
    a = rng.uniform(-1e3, 1e3, n).astype(np.float32)
    b = rng.uniform(-1e3, 1e3, n).astype(np.float32)
    a[:1000] = np.abs(rng.normal(0, 1e-38, 1000)).astype(np.float32)  # subnormal range
    b[1000:2000] = np.float32(2 ** -140)
    q = np.empty(n, np.float32)
    r = np.empty(n, np.float32)
    L.check(L.lib.dtl_kernel_div_sqrt(_p(a, C.c_float), _p(b, C.c_float), _p(q, C.c_float), _p(r, C.c_float), n), "div")
    with np.errstate(all="ignore"):
        assert np.array_equal(q.view(np.uint32), (a / b).view(np.uint32))
        pos = a >= 0
        assert np.array_equal(r[pos].view(np.uint32), np.sqrt(a[pos]).view(np.uint32))


def test_quantize_q8a_q8k_bitexact():
    L = _lib()
    rng = np.random.default_rng(3)
    rows, n = 5, 2048
    x = rng.normal(0, 2, (rows, n)).astype(np.float32)
    x[0, :256] = 0.0                       # all-zero blocks
    x[1, 10], x[1, 20] = -7.5, 7.5         # |x| tie: first one wins in Q8_K
    x[2, 0:32] = np.float32(2 ** -140)     # subnormal block
    x[3, 64:96] = rng.integers(-3, 4, 32)  # many exact .5 ratios
    # |x| ties across the rows of sixteen lanes of a 256-block (lane = local
    # index / 4): row 0 against row 3, row 0 against row 2, row 2 against
    # row 3; the first index wins
    x[4, 3], x[4, 200] = -20.0, 20.0
    x[4, 560], x[4, 700] = -19.0, 19.0
    x[4, 900], x[4, 1000] = 18.0, -18.0
    da = np.empty(rows * n // 32, np.float32)
    qa = np.empty(rows * n, np.int8)
    dk = np.empty(rows * n // 256, np.float32)
    qk = np.empty(rows * n, np.int8)
    L.check(L.lib.dtl_kernel_quantize(_p(x, C.c_float), rows, n, _p(da, C.c_float), _p(qa, C.c_int8),
                                      _p(dk, C.c_float), _p(qk, C.c_int8)), "quantize")
    for r in range(rows):
        wd, wq = detref.quantize_q8a(x[r])
        assert np.array_equal(da[r * n // 32:(r + 1) * n // 32].view(np.uint32), wd.view(np.uint32))
        assert np.array_equal(qa[r * n:(r + 1) * n], wq)
        kd, kq = detref.quantize_q8k(x[r])
        assert np.array_equal(dk[r * n // 256:(r + 1) * n // 256].view(np.uint32), kd.view(np.uint32))
        assert np.array_equal(qk[r * n:(r + 1) * n], kq)


def test_quantize_q8a_only_partial_span():
    # 896 = 3.5 spans of 256: the last wave quantises half a span.
    L = _lib()
    rng = np.random.default_rng(5)
    rows, n = 3, 896
    x = rng.normal(0, 1, (rows, n)).astype(np.float32)
    x[1, 864:] = 0.0
    da = np.empty(rows * n // 32, np.float32)
    qa = np.empty(rows * n, np.int8)
    L.check(L.lib.dtl_kernel_quantize(_p(x, C.c_float), rows, n, _p(da, C.c_float), _p(qa, C.c_int8),
                                      None, None), "quantize")
    for r in range(rows):
        wd, wq = detref.quantize_q8a(x[r])
        assert np.array_equal(da[r * n // 32:(r + 1) * n // 32].view(np.uint32), wd.view(np.uint32))
        assert np.array_equal(qa[r * n:(r + 1) * n], wq)


def test_rmsnorm_bitexact():
    L = _lib()
    rng = np.random.default_rng(4)
    for n, eps in [(64, 1e-5), (576, 1e-5), (896, 1e-6), (2048, 1e-5), (13, 1e-5), (4, 1e-5), (16384, 1e-5)]:
        x = rng.normal(0, 30, (3, n)).astype(np.float32)
        w = rng.normal(1, 0.02, n).astype(np.float32)
        out = np.empty_like(x)
        L.check(L.lib.dtl_kernel_rmsnorm(_p(x, C.c_float), _p(w, C.c_float), eps, 3, n, _p(out, C.c_float)), "rms")
        for r in range(3):
            assert np.array_equal(out[r].view(np.uint32), detref.rmsnorm(x[r], w, eps).view(np.uint32))


# (type, rows, cols, positions): T <= 8 runs the decode GEMVs (rows per wave
# grows with the row count: Q8_0/Q4_0 1/2/4/8, Q6_K 64/nsb, Q4_K 8/32),
# T >= 16 the token-parallel GEMMs (Q8_0 / Q4_0 / Q6_K on the matrix
# cores), T in between the row-lane kernel.
GEMV_CASES = [
    (0, 37, 64, 3), (0, 20, 128, 1),
    (8, 61, 576, 1), (8, 33, 896, 5), (8, 9, 4864, 2), (8, 5000, 64, 1), (8, 17000, 64, 2),
    (8, 66000, 32, 1), (8, 300, 8192, 1), (8, 20, 576, 12),
    # the streaming Q8_0 kernel (tall, at most 32 blocks per row): the Qwen2.5
    # output width (28 blocks), the 32-block maximum, and 3 blocks (a chain
    # shorter than one float4 read)
    (8, 20001, 896, 1), (8, 16390, 1024, 2), (8, 16400, 96, 3),
    (2, 40, 64, 2), (2, 17, 512, 1), (2, 66000, 64, 1), (2, 5000, 96, 3),
    (12, 45, 2048, 1), (12, 7, 5632, 3), (12, 30, 512, 64), (12, 9000, 256, 1), (12, 13, 256, 8),
    (12, 45, 256, 37), (12, 100, 768, 20),
    # Q4_K chunk GEMMs: partial row and position tiles, one and several
    # slices per superblock, the ffn_down width
    (12, 17, 2048, 16), (12, 130, 1024, 33), (12, 48, 5632, 64), (12, 1, 256, 17),
    # 8 positions x 5632 columns: the split decode kernel's LDS does not hold
    # the activations, so the one-lane-per-row Q4_K kernel serves it
    (12, 20, 5632, 8),
    (14, 50, 2048, 1), (14, 9, 5632, 2), (14, 20, 512, 64), (14, 300, 256, 1), (14, 33, 4096, 1),
    # Q6_K decode at full TinyLlama ffn_down size (T = 8), odd row counts, and
    # a 16384-row matrix (the split-superblock kernel's largest)
    (14, 2048, 5632, 8), (14, 1000, 5632, 3), (14, 2049, 5632, 1), (14, 16384, 2048, 1),
    # tall Q6_K on the decode layout (k_gemv_q6k_cm): the TinyLlama output
    # projection, every superblock count that divides 16 (1 to 16 per row),
    # partial last groups and several positions
    (14, 32000, 2048, 1), (14, 16385, 256, 3), (14, 17000, 512, 1), (14, 20001, 1024, 2),
    (14, 16400, 4096, 1), (14, 16390, 8192, 2), (14, 16401, 256, 1), (14, 8, 16384, 1),
    # Q8_0 / Q4_0 on the int8 matrix cores (T >= 16): odd block counts (a
    # half block pair), row tiles of 16 / 32 / 64, partial position tiles
    (8, 40, 32, 16), (8, 37, 96, 33), (8, 2100, 160, 17), (8, 8200, 64, 16), (8, 100, 896, 64),
    (8, 64, 576, 100), (2, 40, 64, 16), (2, 33, 96, 70), (2, 2050, 64, 16),
]


@pytest.mark.parametrize("ggml_type,rows,cols,T", GEMV_CASES)
def test_gemv_bitexact_against_oracle(ggml_type, rows, cols, T):
    L = _lib()
    rng = np.random.default_rng(ggml_type * 1000 + cols + T)
    w = qblocks.random_row(rng, ggml_type, rows, cols)
    x = rng.normal(0, 3, (T, cols)).astype(np.float32)
    out = np.empty((T, rows), np.float32)
    wb = np.frombuffer(w, np.uint8).copy()
    L.check(L.lib.dtl_kernel_gemv(ggml_type, _p(wb, C.c_uint8), rows, cols, _p(x, C.c_float), T,
                                  _p(out, C.c_float)), "gemv")
    rb = qblocks.ROW_BYTES[ggml_type](cols)
    for t in range(T):
        want = np.array([detref.dot_row(ggml_type, w[r * rb:(r + 1) * rb], cols, x[t]) for r in range(rows)],
                        np.float32)
        assert np.array_equal(out[t].view(np.uint32), want.view(np.uint32)), (t,)


# (mode, overlapped, rows0, rows1, cols, T): the Q4_K chunk GEMMs of the
# encode.  mode 0 one matrix, 1 gate + up + SwiGLU, 2 two matrices (wq + wk)
# in one launch; overlapped 1 runs the products on the matrix cores
# (k_q4k_mfp), 0 a launch alone (k_q4k_f32m for modes 0 and 2).  Partial row
# tiles (16 per wave, 8 of each matrix for gate + up), partial position
# tiles, a wq + wk boundary inside a tile, one to 22 superblocks per row.
Q4K_CHUNK_CASES = [
    (0, 1, 17, 0, 256, 16), (0, 1, 130, 0, 1024, 33), (0, 1, 48, 0, 5632, 64), (0, 1, 1, 0, 512, 70),
    (0, 0, 37, 0, 512, 20),
    (1, 1, 13, 0, 256, 16), (1, 1, 40, 0, 2048, 64), (1, 1, 9, 0, 768, 37), (1, 0, 21, 0, 512, 17),
    (2, 1, 40, 8, 512, 16), (2, 1, 64, 16, 2048, 64), (2, 1, 23, 5, 256, 33), (2, 0, 30, 9, 512, 19),
]


@pytest.mark.parametrize("mode,overlapped,rows0,rows1,cols,T", Q4K_CHUNK_CASES)
def test_q4k_chunk_gemm_bitexact_against_oracle(mode, overlapped, rows0, rows1, cols, T):
    L = _lib()
    rng = np.random.default_rng(mode * 100 + rows0 + cols + T)
    if mode == 1:
        rows1 = rows0
    w0 = qblocks.random_row(rng, 12, rows0, cols)
    w1 = qblocks.random_row(rng, 12, rows1, cols) if mode else bytes(1)
    x = rng.normal(0, 3, (T, cols)).astype(np.float32)
    out0 = np.empty((T, rows0), np.float32)
    out1 = np.empty((T, max(rows1, 1)), np.float32)
    b0 = np.frombuffer(w0, np.uint8).copy()
    b1 = np.frombuffer(w1, np.uint8).copy()
    L.check(L.lib.dtl_kernel_q4k_chunk(mode, overlapped, _p(b0, C.c_uint8), rows0, _p(b1, C.c_uint8),
                                       rows1, cols, _p(x, C.c_float), T, _p(out0, C.c_float),
                                       _p(out1, C.c_float)), "q4k chunk")
    rb = qblocks.ROW_BYTES[12](cols)
    silu = detref.lib().ref_silu_f32
    for t in range(T):
        d0 = np.array([detref.dot_row(12, w0[r * rb:(r + 1) * rb], cols, x[t]) for r in range(rows0)],
                      np.float32)
        if mode == 1:
            d1 = np.array([detref.dot_row(12, w1[r * rb:(r + 1) * rb], cols, x[t]) for r in range(rows1)],
                          np.float32)
            want = np.array([silu(float(g)) for g in d0], np.float32) * d1
            assert np.array_equal(out0[t].view(np.uint32), want.view(np.uint32)), (t,)
            continue
        assert np.array_equal(out0[t].view(np.uint32), d0.view(np.uint32)), (t,)
        if mode == 2:
            d1 = np.array([detref.dot_row(12, w1[r * rb:(r + 1) * rb], cols, x[t]) for r in range(rows1)],
                          np.float32)
            assert np.array_equal(out1[t, :rows1].view(np.uint32), d1.view(np.uint32)), (t,)


@pytest.mark.parametrize("theta,rope_dim", [(1e4, 64), (1e5, 64), (1e6, 64), (1e4, 16)])
def test_rope_table_bitexact(theta, rope_dim):
    L = _lib()
    from detllm_amd import synth
    import dataclasses

    positions = 2048
    half = rope_dim // 2
    c = np.empty(positions * half, np.float32)
    s = np.empty(positions * half, np.float32)
    L.check(L.lib.dtl_kernel_rope_table(theta, rope_dim, positions, _p(c, C.c_float), _p(s, C.c_float)), "rope")
    base = synth.WORKLOADS["tiny"]
    w = dataclasses.replace(base, rope_base=theta, d=rope_dim * 4, heads=4, kv_heads=2, ff=64, ctx=positions)
    m = detref.Model(synth.build_model(w, layers=1))
    wc, ws = m.rope_table(positions)
    assert np.array_equal(c.view(np.uint32), wc.view(np.uint32))
    assert np.array_equal(s.view(np.uint32), ws.view(np.uint32))


def test_valu_probe_rate_is_the_unfused_f32_issue_rate():
    """dtl_valu_probe (measurement support for the bench's roofline): separately
    rounded f32 multiplies and adds with per-lane register operands on eight
    waves of every SIMD.  A SIMD issues such instructions from two waves at
    once, 16 lanes each per clock: 256 CU x 4 SIMD x 32 lanes at up to 2.4 GHz
    is at most 78.6 T lane-operations/s, and the rate must exceed what one
    issue per SIMD allows at that clock (39.3 T)."""
    L = _lib()
    r = C.c_double()
    L.check(L.lib.dtl_valu_probe(C.byref(r)), "valu probe")
    assert 39.4e12 < r.value <= 78.7e12, r.value


def test_mfp_probe_rate_is_between_the_units_alone():
    """dtl_mfp_probe: k_q4k_mfp's inner pattern (four f32 16x16x1 outer
    products, 64 ordered adds per lane) on four waves of every SIMD.  The
    MFMAs alone would allow 32 products per clock per SIMD (78.6 T/s at
    2.4 GHz); the adds share the SIMD with them, and the pattern must still
    beat the two VALU instructions per multiply-add of the VALU-only chains
    at one issue per SIMD (19.7 T/s)."""
    L = _lib()
    r = C.c_double()
    L.check(L.lib.dtl_mfp_probe(C.byref(r)), "mfp probe")
    assert 19.7e12 < r.value <= 78.7e12, r.value
