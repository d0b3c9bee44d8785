"""Host side of the windowed codec: DTLZ header, window schedule, byte-fallback
tokenizer (all inside libdetllm_amd.so, no GPU needed) and the oracle's
codec restatement, pinned by the reference's own codec tests.

Reference tests followed: det-coder src/file.rs:96-214 (header),
det-cli src/main.rs:1244-1306 (token codec, replay payload, window
rollover), det-token src/lib.rs tests (byte-fallback construction).
"""
import ctypes as C
import struct

import numpy as np
import pytest

import detref
from detllm_amd import synth
from detllm_amd._lib import DetllmError, lib


# ---- DTLZ header (file.rs:96-214) -------------------------------------------
def _hdr(flags=1, n_ctx=2048, overlap=512, orig_len=123456789):
    from detllm_amd.coder import DtlzHeader

    return DtlzHeader(flags, bytes([7] * 32), n_ctx, overlap, orig_len)


def _status(fn, *args):
    try:
        fn(*args)
    except DetllmError as e:
        return e.status
    return 0


def test_header_round_trips_and_layout():
    from detllm_amd.coder import DtlzHeader

    h = _hdr()
    raw = h.encode_checked()
    # layout fixed by DtlzHeader::encode: magic, u16 version, u16 flags,
    # sha[32], u32 n_ctx, u32 overlap, u64 orig_len, little-endian
    assert raw == b"DTLZ" + struct.pack("<HH", 1, 1) + bytes([7] * 32) + struct.pack("<IIQ", 2048, 512, 123456789)
    assert DtlzHeader.decode(raw) == h
    assert DtlzHeader.decode(raw + b"payload") == h


def test_header_accepts_known_flags_rejects_unsupported():
    from detllm_amd.coder import DtlzHeader

    for flags in (0, 1):
        h = _hdr(flags=flags)
        assert DtlzHeader.decode(h.encode_checked()) == h
    bad = _hdr(flags=2)
    assert _status(bad.encode_checked) == 83
    raw = bytearray(_hdr().encode_checked())
    raw[6:8] = struct.pack("<H", 2)
    assert _status(DtlzHeader.decode, bytes(raw)) == 83


def test_header_rejects_malformed_envelope():
    from detllm_amd.coder import DtlzHeader

    assert _status(DtlzHeader.decode, b"") == 80
    assert _status(DtlzHeader.decode, bytes(55)) == 80
    raw = bytearray(_hdr(flags=0).encode_checked())
    raw[0:4] = b"NOPE"
    assert _status(DtlzHeader.decode, bytes(raw)) == 81
    raw = bytearray(_hdr(flags=0).encode_checked())
    raw[4:6] = struct.pack("<H", 2)
    assert _status(DtlzHeader.decode, bytes(raw)) == 82


def test_header_rejects_invalid_window_fields():
    from detllm_amd.coder import DtlzHeader

    for n_ctx, overlap, want in ((0, 0, 84), (8, 8, 85)):
        h = _hdr(flags=0, n_ctx=n_ctx, overlap=overlap)
        assert _status(h.encode_checked) == want
        raw = b"DTLZ" + struct.pack("<HH", 1, 0) + bytes(32) + struct.pack("<IIQ", n_ctx, overlap, 5)
        assert _status(DtlzHeader.decode, raw) == want


def test_decompress_rejects_malformed_header_before_model():
    """cli_decompress_rejects_malformed_header_before_model_load
    (main.rs:1431-1554): no model is needed to fail on the header."""
    from detllm_amd.codec import decompress

    def hdr(flags, n_ctx, overlap, version=1):
        return b"DTLZ" + struct.pack("<HH", version, flags) + bytes(32) + struct.pack("<IIQ", n_ctx, overlap, 0)

    cases = [
        (b"NOPE" + bytes(52), 81),
        (hdr(1, 8, 1, version=2), 82),
        (hdr(2, 8, 1), 83),
        (hdr(1, 0, 0), 84),
        (hdr(1, 8, 8), 85),
        (b"DTLZ", 80),
    ]
    for raw, want in cases:
        assert _status(decompress, None, raw) == want, raw[:8]


# ---- window schedule (main.rs:1289-1304) -------------------------------------
def test_window_rolls_over_when_context_reaches_n_ctx():
    from detllm_amd.codec import next_window_start

    start, seen = 0, []
    for pos in range(18):
        start = next_window_start(pos, start, 8, 2)
        seen.append((pos, start, pos - start))
    assert seen[7] == (7, 0, 7)
    assert seen[8] == (8, 6, 2)
    assert seen[13] == (13, 6, 7)
    assert seen[14] == (14, 12, 2)
    # library and oracle agree over a sweep, overlap 0 included
    for n_ctx, overlap in ((1, 0), (3, 1), (8, 0), (8, 7), (64, 16)):
        a = b = 0
        for pos in range(200):
            a = next_window_start(pos, a, n_ctx, overlap)
            b = detref.next_window_start(pos, b, n_ctx, overlap)
            assert a == b
            assert pos - a <= n_ctx


# ---- byte-fallback tokenizer (det-token) --------------------------------------
def _writer_with_tokens(tokens, types=None, extra=None):
    from detllm_amd.gguf import GgufWriter

    g = GgufWriter()
    g.add_str("general.architecture", "llama")
    if tokens is not None:
        g.add_str_array("tokenizer.ggml.tokens", tokens)
    if types is not None:
        g.add_i32_array("tokenizer.ggml.token_type", types)
    for fn in extra or []:
        fn(g)
    return g.to_bytes()


def test_tokenizer_from_cli_fixture_maps_every_byte():
    from detllm_amd.codec import Tokenizer

    tok = Tokenizer.from_gguf(synth.cli_fixture_gguf())
    assert tok.vocab_len == 256
    data = bytes(range(256)) + b"detllm"
    sym = tok.codec_symbols(data, 256)
    assert list(sym) == list(data)
    for s in (0, 0x41, 255, 256 + 7, 256 + 255):
        assert tok.decode_codec_symbol(s, 256) == bytes([s % 256])
    assert _status(tok.decode_codec_symbol, 512, 256) == 61
    assert Tokenizer.codec_symbol_is_token(255, 256) and not Tokenizer.codec_symbol_is_token(256, 256)


def test_tokenizer_matches_oracle_with_non_emittable_bytes():
    """Bytes whose <0xHH> token is not emittable (token type 3) become byte
    escapes vocab + byte; the tables match the oracle's restatement."""
    from detllm_amd.codec import Tokenizer

    vocab = 600
    tokens, types = synth.vocabulary(vocab)
    tok = Tokenizer.from_gguf(_writer_with_tokens(tokens, types))
    emit = [1 if t in (1, 4, 6) else 0 for t in types]
    b2t, t2b = detref.byte_fallback_tables(tokens, emit)
    rng = np.random.default_rng(5)
    data = bytes(rng.integers(0, 256, 4000, dtype=np.uint8)) + b"zz~~"
    got = tok.codec_symbols(data, vocab)
    want = detref.codec_symbols(b2t, data, vocab)
    assert np.array_equal(got, want)
    for b in synth.ESCAPED_BYTES:
        assert got[data.index(bytes([b]))] == vocab + b
    # decoding: token ids decode through token_to_byte, escapes to their byte
    for s in list(range(0, 300, 7)) + [vocab + 0x7A, vocab + 3]:
        if s < vocab and t2b[s] < 0:
            assert _status(tok.decode_codec_symbol, s, vocab) == 61
        else:
            exp = bytes([t2b[s]]) if s < vocab else bytes([s - vocab])
            assert tok.decode_codec_symbol(s, vocab) == exp


@pytest.mark.parametrize(
    "case,want",
    [
        ("missing_vocabulary", 62),
        ("incomplete", 65),
        ("duplicate_plus_sign", 72),
        ("bpe_model", 77),
        ("bpe_merges", 77),
        ("type_length", 67),
        ("invalid_type", 68),
        ("type_not_ints", 66),
    ],
)
def test_tokenizer_construction_errors(case, want):
    from detllm_amd.codec import Tokenizer

    base = [f"<0x{b:02X}>" for b in range(256)]
    if case == "missing_vocabulary":
        raw = _writer_with_tokens(None)
    elif case == "incomplete":
        toks = list(base)
        toks[255] = "not-a-byte"
        raw = _writer_with_tokens(toks)
    elif case == "duplicate_plus_sign":
        raw = _writer_with_tokens(base + ["<0x+F>"])  # u8::from_str_radix("+F", 16) == 15
    elif case == "bpe_model":
        raw = _writer_with_tokens(base + ["ab"], extra=[lambda g: g.add_str("tokenizer.ggml.model", "gpt2")])
    elif case == "bpe_merges":
        raw = _writer_with_tokens(base + ["ab"],
                                  extra=[lambda g: g.add_str_array("tokenizer.ggml.merges", ["<0x61> <0x62>"])])
    elif case == "type_length":
        raw = _writer_with_tokens(base, [6] * 255)
    elif case == "invalid_type":
        raw = _writer_with_tokens(base, [6] * 255 + [7])
    else:
        raw = _writer_with_tokens(base, extra=[lambda g: g.add_str_array("tokenizer.ggml.token_type", ["6"] * 256)])
    assert _status(Tokenizer.from_gguf, raw) == want


def test_canonical_byte_token_forms():
    # canonical_byte_fallback_token (lib.rs:841-847), checked on the oracle
    # restatement and through the library's tokenizer on the same strings
    cases = {"<0x00>": 0, "<0xff>": 255, "<0xAb>": 0xAB, "<0x+7>": 7, "<0x-1>": -1, "<0x1>": -1,
             "<0x100>": -1, "<0xg1>": -1, "0x41": -1, "<0x41": -1, "<0X41>": -1, "<0x é>": -1}
    for t, want in cases.items():
        assert detref.canonical_byte_token(t) == want, t


# ---- oracle codec pins (main.rs:1244-1262, 1306-1366, 1806-1858) ------------
def _replay_payload(model, symbols, n_ctx, overlap, tail=256):
    """encode_tokens_with_replayed_context (main.rs:1346-1361): every
    position's CDF from a fresh cache over its window's context."""
    trip, ws, V = [], 0, model.vocab
    assert all(int(s) < V for s in symbols), "token streams only: escapes do not enter the context"
    for pos, s in enumerate(symbols):
        ws = detref.next_window_start(pos, ws, n_ctx, overlap)
        ctx = [int(t) for t in symbols[ws:pos]]
        if not ctx:
            trip.append((int(s), 1, V + tail))
        else:
            trip.append(detref.symbol_range(detref.Model.logits(model, ctx)[-1], int(s), tail))
    return detref.range_encode(trip)


def test_oracle_token_codec_round_trips_and_matches_replay():
    m = detref.Model(synth.codec_fixture_gguf())
    toks = [0, 1, 2, 3, 0, 2, 1, 3, 2, 0]
    enc = detref.codec_encode(m, toks, 3, 1, True)
    assert enc == _replay_payload(m, toks, 3, 1)
    syms, _ = detref.codec_decode(m, np.arange(4, dtype=np.int16), enc, len(toks), 3, 1, True)
    assert list(syms) == toks


def test_oracle_byte_codec_multi_window_round_trips():
    m = detref.Model(synth.cli_fixture_gguf())
    b2t, t2b = detref.byte_fallback_tables([f"<0x{b:02X}>" for b in range(256)])
    for data in (b"", b"detllm windowed roundtrip", bytes(range(256)) + bytes(range(255, -1, -1))):
        sym = detref.codec_symbols(b2t, data, 256)
        enc = detref.codec_encode(m, sym, 8, 2, True)
        if len(data) <= 40:
            assert enc == _replay_payload(m, list(sym), 8, 2)
        got_sym, got = detref.codec_decode(m, t2b, enc, len(data), 8, 2, True)
        assert got == data and list(got_sym) == list(sym)


# Payload sizes the reference records for its bundled fixtures
# (docs/validation.md:511 and 1263-1264): n_ctx 8, overlap 2, byte escapes.
SIZE_PINS = [
    ("tiny-f32", b"detllm deterministic compression smoke\n", 102 - 56),
    ("tiny-f32", None, 19),   # None: the bundled tiny.tokens.txt (12 bytes)
    ("tiny-qmix", None, 19),
]


@pytest.mark.parametrize("model,data,payload", SIZE_PINS)
def test_oracle_codec_payload_sizes_match_reference_records(model, data, payload):
    from conftest import GOLDEN

    g = (GOLDEN / f"{model}.gguf").read_bytes()
    if data is None:
        data = (GOLDEN / "tiny.tokens.txt").read_bytes()
        assert len(data) == 12
    m = detref.Model(g)
    b2t, t2b = detref.byte_fallback_tables([f"<0x{b:02X}>" for b in range(256)])
    sym = detref.codec_symbols(b2t, data, m.vocab)
    enc = detref.codec_encode(m, sym, 8, 2, True)
    assert len(enc) == payload
    _, back = detref.codec_decode(m, t2b, enc, len(data), 8, 2, True)
    assert back == data
