"""The C-ABI library loads without a GPU and exports everything the header declares;
its host-only parts (range coder, argument checks) run on the CPU."""
import ctypes as C
import re

import numpy as np
import pytest

import detref
from conftest import ROOT


def declared_symbols():
    text = (ROOT / "include" / "detllm.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dtl_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from detllm_amd import _lib

    names = declared_symbols()
    assert len(names) >= 30
    for name in names:
        assert hasattr(_lib.lib, name), name
    assert set(names) == set(_lib.EXPORTED)


def test_library_is_built_for_gfx950():
    from detllm_amd import _lib

    data = _lib.LIB_PATH.read_bytes()
    assert b"gfx950" in data


def test_status_strings():
    from detllm_amd._lib import status_name

    assert status_name(0) == "ok"
    assert status_name(2) == "non-finite"
    assert status_name(25) == "cdf: total too large"


def test_host_range_coder_matches_oracle_bytes():
    from detllm_amd.coder import RangeDecoder, RangeEncoder

    rng = np.random.default_rng(11)
    triples = []
    for _ in range(5000):
        total = int(rng.integers(2, 1 << 30))
        cum = int(rng.integers(0, total - 1))
        freq = int(rng.integers(1, total - cum + 1))
        triples.append((cum, freq, total))
    enc = RangeEncoder()
    for t in triples:
        enc.encode(*t)
    data = enc.finish()
    assert data == detref.range_encode(triples)
    dec = RangeDecoder(data)
    for cum, freq, total in triples:
        v = dec.decode_freq(total)
        assert cum <= v < cum + freq
        dec.advance(cum, freq, total)


def test_range_coder_rejects_bad_triples_and_truncation():
    from detllm_amd._lib import DetllmError
    from detllm_amd.coder import RangeDecoder, RangeEncoder

    enc = RangeEncoder()
    for bad in [(0, 0, 10), (5, 6, 10), (0, 1, 1 << 31), (0, 1, 0)]:
        try:
            enc.encode(*bad)
            raise AssertionError(bad)
        except DetllmError as e:
            assert e.status == 30
    try:
        RangeDecoder(b"\x01\x02\x03")
        raise AssertionError("short payload accepted")
    except DetllmError as e:
        assert e.status == 31


def test_dtlz_header_roundtrip():
    from detllm_amd.coder import HEADER_LEN, DtlzHeader

    h = DtlzHeader(1, bytes(range(32)), 2048, 512, 1 << 20)
    raw = h.encode_checked()
    assert len(raw) == HEADER_LEN == 56 and raw[:4] == b"DTLZ"
    assert raw == h.encode()
    assert DtlzHeader.decode(raw) == h


def test_range_decoder_snapshot_resumes_mid_stream():
    """A decoder restored from a snapshot taken between two symbols decodes
    the rest of the stream as the uninterrupted decoder does, through the
    renormalisations the stream holds; a snapshot between decode_freq and
    advance, a position before the 8 code bytes or past the input, and a
    zero range are rejected."""
    from detllm_amd._lib import DetllmError, RangeDecoderState
    from detllm_amd.coder import RangeDecoder, RangeEncoder

    rng = np.random.default_rng(11)
    triples = []
    for _ in range(3000):
        total = int(rng.integers(2, 1 << 20))
        f = int(rng.integers(1, total + 1))
        triples.append((int(rng.integers(0, total - f + 1)), f, total))
    enc = RangeEncoder()
    for t in triples:
        enc.encode(*t)
    data = enc.finish()

    def run(dec, ts):
        got = []
        for c, f, t in ts:
            v = dec.decode_freq(t)
            assert c <= v < c + f
            dec.advance(c, f, t)
            got.append(v)
        return got

    whole = RangeDecoder(data)
    want = run(whole, triples)
    end = whole.snapshot()
    for cut in (0, 1, 777, 2999):
        dec = RangeDecoder(data)
        got = run(dec, triples[:cut])
        resumed = RangeDecoder.from_snapshot(data, dec.snapshot())
        got += run(resumed, triples[cut:])
        assert got == want
        fin = resumed.snapshot()
        assert (fin.low, fin.range, fin.code, fin.pos) == (end.low, end.range, end.code, end.pos)
    dec = RangeDecoder(data)
    dec.decode_freq(triples[0][2])
    with pytest.raises(DetllmError):
        dec.snapshot()
    good = RangeDecoder(data).snapshot()
    for bad in (RangeDecoderState(good.low, good.range, good.code, 7),
                RangeDecoderState(good.low, good.range, good.code, len(data) + 1),
                RangeDecoderState(good.low, 0, good.code, good.pos)):
        with pytest.raises(DetllmError):
            RangeDecoder.from_snapshot(data, bad)


def test_range_encoder_snapshot_resumes_canonical_stream():
    # det-coder range.rs:208-230: encode a prefix, snapshot, restore, encode
    # the rest: the same bytes as one uninterrupted encoder.
    from detllm_amd._lib import DetllmError
    from detllm_amd.coder import RangeEncoder, RangeEncoderSnapshot

    cum = [0, 1, 0, 2, 1, 3, 0, 2]
    freq = [1, 1, 2, 1, 2, 1, 1, 2]
    one = RangeEncoder()
    for c, f in zip(cum, freq):
        one.encode(c, f, 4)
    part = RangeEncoder()
    for c, f in zip(cum[:4], freq[:4]):
        part.encode(c, f, 4)
    snap = part.snapshot()
    resumed = RangeEncoder.from_snapshot(snap)
    for c, f in zip(cum[4:], freq[4:]):
        resumed.encode(c, f, 4)
    assert resumed.finish() == one.finish()
    # a long stream through several snapshots equals the oracle's bytes
    rng = np.random.default_rng(3)
    triples = []
    for _ in range(5000):
        total = int(rng.integers(2, 1 << 20))
        f = int(rng.integers(1, total + 1))
        triples.append((int(rng.integers(0, total - f + 1)), f, total))
    enc = RangeEncoder()
    for i, t in enumerate(triples):
        if i % 997 == 0:
            enc = RangeEncoder.from_snapshot(enc.snapshot())
        enc.encode(*t)
    assert enc.finish() == detref.range_encode(triples)
    try:
        RangeEncoder.from_snapshot(RangeEncoderSnapshot(snap.low, 0, snap.out))
        raise AssertionError("range 0 accepted")
    except DetllmError as e:
        assert e.status == 30  # RangeError::InvalidFrequency


def test_uniform_cdf():
    # det-coder cdf.rs:684-705
    from detllm_amd._lib import DetllmError
    from detllm_amd.coder import uniform_cdf, uniform_cdf_with_byte_escapes

    c = uniform_cdf(4)
    assert c.freq.tolist() == [1, 1, 1, 1] and c.cum.tolist() == [0, 1, 2, 3] and c.total == 4
    c = uniform_cdf_with_byte_escapes(151936)
    assert c.total == 152192 and c.cum[-1] == 152191 and int(c.freq.sum()) == 152192
    for n, st in ((0, 20), ((1 << 18) + 1, 24)):
        try:
            uniform_cdf(n)
            raise AssertionError(n)
        except DetllmError as e:
            assert e.status == st
