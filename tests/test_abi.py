"""The C-ABI library loads without a GPU and exports everything the header declares;
its host-only parts (range coder, argument checks) run on the CPU."""
import ctypes as C
import re

import numpy as np

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
