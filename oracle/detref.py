"""ctypes binding of the CPU oracle (TEST INFRASTRUCTURE ONLY).

The oracle is the plain-C restatement of the detllm reference CPU path in
this directory.  Only tests/, the smoke check and the CPU-baseline leg of
bench.py load it; the product library never does.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "libdetref.so"


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def load() -> C.CDLL:
    if not LIB.exists():
        build()
    L = C.CDLL(str(LIB))
    f32p, u8p, u32p, u64p, i8p = (C.POINTER(C.c_float), C.POINTER(C.c_uint8), C.POINTER(C.c_uint32),
                                  C.POINTER(C.c_uint64), C.POINTER(C.c_int8))
    sz = C.c_size_t
    sigs = {
        "ref_exp_f32": (C.c_float, [C.c_float]),
        "ref_exp_f32_array": (None, [C.POINTER(C.c_float), C.POINTER(C.c_float), sz, C.c_int]),
        "ref_silu_f32": (C.c_float, [C.c_float]),
        "ref_exp_f64": (C.c_double, [C.c_double]),
        "ref_ln_f64": (C.c_double, [C.c_double]),
        "ref_sin_f64": (C.c_double, [C.c_double]),
        "ref_cos_f64": (C.c_double, [C.c_double]),
        "ref_f16_to_f32": (C.c_float, [C.c_uint16]),
        "ref_round_ties_even_i32": (C.c_int32, [C.c_float]),
        "ref_round_ties_even_i64": (C.c_int64, [C.c_double]),
        "ref_dot_f32": (C.c_float, [f32p, f32p, sz]),
        "ref_sum_f32": (C.c_float, [f32p, sz]),
        "ref_sum_squares_f32": (C.c_float, [f32p, sz]),
        "ref_sha256": (None, [C.c_void_p, sz, u8p]),
        "ref_numeric_canary": (None, [u8p]),
        "ref_runtime_canary": (C.c_int, [u8p]),
        "ref_quant_kernel_hash": (C.c_int, [u8p]),
        "ref_quantize_q8a": (C.c_int, [f32p, sz, f32p, i8p]),
        "ref_quantize_q8k": (C.c_int, [f32p, sz, f32p, i8p]),
        "ref_dot_row": (C.c_int, [C.c_int, u8p, sz, f32p, f32p]),
        "ref_rmsnorm": (C.c_int, [f32p, f32p, C.c_float, sz, f32p]),
        "ref_model_load": (C.c_void_p, [C.c_char_p, sz, C.POINTER(C.c_int)]),
        "ref_model_free": (None, [C.c_void_p]),
        "ref_model_config": (None, [C.c_void_p, C.POINTER(C.c_int64)]),
        "ref_model_bias": (sz, [C.c_void_p, sz, C.c_int, f32p, sz]),
        "ref_session_new": (C.c_void_p, [C.c_void_p, sz, C.POINTER(C.c_int)]),
        "ref_session_free": (None, [C.c_void_p]),
        "ref_session_reset": (C.c_int, [C.c_void_p]),
        "ref_forward_one": (C.c_int, [C.c_void_p, sz, sz, f32p]),
        "ref_logits_hash": (C.c_int, [C.c_void_p, u32p, sz, sz, u8p]),
        "ref_logits": (C.c_int, [C.c_void_p, u32p, sz, f32p]),
        "ref_rope_table": (C.c_int, [C.c_void_p, sz, f32p, f32p]),
        "ref_apply_rope": (C.c_int, [f32p, sz, sz, sz, C.c_int, f32p, f32p]),
        "ref_set_threads": (None, [sz]),
        "ref_set_simd": (None, [C.c_int]),
        "ref_logits_to_cdf": (C.c_int, [f32p, sz, sz, u32p, u64p, u64p]),
        "ref_symbol_range": (C.c_int, [f32p, sz, sz, sz, u64p, u32p, u64p]),
        "ref_decoder_lookup": (C.c_int, [f32p, sz, sz, C.c_uint64, u64p, u64p, u32p, u64p]),
        "ref_decoder_total": (C.c_int, [f32p, sz, sz, u64p]),
        "ref_uniform_symbol_range": (C.c_int, [sz, sz, u64p, u32p, u64p]),
        "ref_range_encoder_new": (C.c_void_p, []),
        "ref_range_encode": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64]),
        "ref_range_encoder_finish": (sz, [C.c_void_p, u8p, sz]),
        "ref_range_encoder_free": (None, [C.c_void_p]),
        "ref_range_decoder_new": (C.c_void_p, [u8p, sz, C.POINTER(C.c_int)]),
        "ref_range_decode_freq": (C.c_int, [C.c_void_p, C.c_uint64, u64p]),
        "ref_range_decode_advance": (C.c_int, [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64]),
        "ref_range_decoder_free": (None, [C.c_void_p]),
        "ref_canonical_byte_token": (C.c_int, [C.c_char_p, sz]),
        "ref_byte_fallback_tables": (C.c_int, [C.c_char_p, C.POINTER(sz), sz, u8p,
                                               C.POINTER(C.c_int32), C.POINTER(C.c_int16)]),
        "ref_codec_symbols": (None, [C.POINTER(C.c_int32), u8p, sz, sz, u32p]),
        "ref_next_window_start": (sz, [sz, sz, sz, sz]),
        "ref_codec_encode": (C.c_int, [C.c_void_p, u32p, sz, sz, sz, C.c_int, u8p, sz, C.POINTER(sz)]),
        "ref_codec_decode": (C.c_int, [C.c_void_p, C.POINTER(C.c_int16), u8p, sz, sz, sz, sz, C.c_int,
                                       u32p, u8p, C.POINTER(sz)]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


_L = None


def lib() -> C.CDLL:
    global _L
    if _L is None:
        _L = load()
    return _L


def _p(a, t):
    return a.ctypes.data_as(C.POINTER(t))


class OracleError(RuntimeError):
    def __init__(self, status: int, where: str):
        self.status = status
        super().__init__(f"{where}: oracle status {status}")


def _chk(st: int, where: str) -> None:
    if st:
        raise OracleError(st, where)


class Model:
    """The oracle's F32Llama (det-model lib.rs restated in C)."""

    def __init__(self, gguf: bytes):
        self._buf = bytes(gguf)
        st = C.c_int()
        h = lib().ref_model_load(self._buf, len(self._buf), C.byref(st))
        if not h:
            raise OracleError(st.value, "ref_model_load")
        self._h = C.c_void_p(h)
        cfg = (C.c_int64 * 16)()
        lib().ref_model_config(self._h, cfg)
        self.cfg = list(cfg)
        self.vocab = int(cfg[9])

    def __del__(self):
        try:
            lib().ref_model_free(self._h)
        except Exception:
            pass

    def bias(self, layer: int, which: int):
        """Layer bias q (0), k (1) or v (2) as loaded, or None when absent."""
        buf = np.empty(1 << 16, np.float32)
        n = lib().ref_model_bias(self._h, layer, which, _p(buf, C.c_float), buf.size)
        return buf[:n].copy() if n else None

    def logits(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
        out = np.empty((t.size, self.vocab), np.float32)
        _chk(lib().ref_logits(self._h, _p(t, C.c_uint32), t.size, _p(out, C.c_float)), "ref_logits")
        return out

    def logits_hash(self, tokens, chunk: int = 1) -> bytes:
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.uint32))
        out = (C.c_uint8 * 32)()
        _chk(lib().ref_logits_hash(self._h, _p(t, C.c_uint32), t.size, chunk, out), "ref_logits_hash")
        return bytes(out)

    def forward_at(self, tokens, positions, next_symbols=None, tail: int = 0):
        """forward_one (det-model lib.rs:1249-1400) of tokens[i] at positions[i]
        in one session, in the order given: the cache rows below each position
        are whatever the session holds (zeros, or earlier calls' rows).  With
        next_symbols, also the symbol range of next_symbols[i] under each
        position's logits.  Used to time positions spread over a window."""
        st = C.c_int()
        s = lib().ref_session_new(self._h, int(max(positions)) + 1, C.byref(st))
        if not s:
            raise OracleError(st.value, "ref_session_new")
        out = np.empty(self.vocab, np.float32)
        try:
            for i, (t, p) in enumerate(zip(tokens, positions)):
                _chk(lib().ref_forward_one(s, int(t), int(p), _p(out, C.c_float)), "ref_forward_one")
                if next_symbols is not None:
                    symbol_range(out, int(next_symbols[i]), tail)
        finally:
            lib().ref_session_free(s)
        return out

    def rope_table(self, positions: int):
        half = int(self.cfg[6]) // 2
        c = np.empty(positions * half, np.float32)
        s = np.empty(positions * half, np.float32)
        _chk(lib().ref_rope_table(self._h, positions, _p(c, C.c_float), _p(s, C.c_float)), "ref_rope_table")
        return c, s


def set_threads(n: int) -> None:
    lib().ref_set_threads(n)


def set_simd(on: bool) -> None:
    lib().ref_set_simd(1 if on else 0)


def logits_to_cdf(logits, tail: int = 0):
    lg = np.ascontiguousarray(np.asarray(logits, np.float32))
    n = lg.size + tail
    freq = np.empty(n, np.uint32)
    cum = np.empty(n, np.uint64)
    total = C.c_uint64()
    _chk(lib().ref_logits_to_cdf(_p(lg, C.c_float), lg.size, tail, _p(freq, C.c_uint32), _p(cum, C.c_uint64),
                                 C.byref(total)), "ref_logits_to_cdf")
    return freq, cum, int(total.value)


def symbol_range(logits, symbol: int, tail: int = 0):
    lg = np.ascontiguousarray(np.asarray(logits, np.float32))
    cum, total = C.c_uint64(), C.c_uint64()
    freq = C.c_uint32()
    _chk(lib().ref_symbol_range(_p(lg, C.c_float), lg.size, symbol, tail, C.byref(cum), C.byref(freq),
                                C.byref(total)), "ref_symbol_range")
    return int(cum.value), int(freq.value), int(total.value)


def decoder_lookup(logits, value: int, tail: int = 0):
    lg = np.ascontiguousarray(np.asarray(logits, np.float32))
    sym, cum, total = C.c_uint64(), C.c_uint64(), C.c_uint64()
    freq = C.c_uint32()
    _chk(lib().ref_decoder_lookup(_p(lg, C.c_float), lg.size, tail, value, C.byref(sym), C.byref(cum),
                                  C.byref(freq), C.byref(total)), "ref_decoder_lookup")
    return int(sym.value), int(cum.value), int(freq.value), int(total.value)


def quantize_q8a(x):
    x = np.ascontiguousarray(np.asarray(x, np.float32))
    d = np.empty(x.size // 32, np.float32)
    q = np.empty(x.size, np.int8)
    _chk(lib().ref_quantize_q8a(_p(x, C.c_float), x.size, _p(d, C.c_float), _p(q, C.c_int8)), "ref_quantize_q8a")
    return d, q


def quantize_q8k(x):
    x = np.ascontiguousarray(np.asarray(x, np.float32))
    d = np.empty(x.size // 256, np.float32)
    q = np.empty(x.size, np.int8)
    _chk(lib().ref_quantize_q8k(_p(x, C.c_float), x.size, _p(d, C.c_float), _p(q, C.c_int8)), "ref_quantize_q8k")
    return d, q


def dot_row(ggml_type: int, row: bytes, cols: int, x) -> float:
    rb = np.frombuffer(bytes(row), np.uint8).copy()
    x = np.ascontiguousarray(np.asarray(x, np.float32))
    out = C.c_float()
    _chk(lib().ref_dot_row(ggml_type, _p(rb, C.c_uint8), cols, _p(x, C.c_float), C.byref(out)), "ref_dot_row")
    return out.value


def rmsnorm(x, w, eps: float):
    x = np.ascontiguousarray(np.asarray(x, np.float32))
    w = np.ascontiguousarray(np.asarray(w, np.float32))
    out = np.empty_like(x)
    _chk(lib().ref_rmsnorm(_p(x, C.c_float), _p(w, C.c_float), eps, x.size, _p(out, C.c_float)), "ref_rmsnorm")
    return out


def apply_rope(x, heads: int, head_dim: int, rope_dim: int, split_half: bool, cos_row, sin_row):
    """apply_rope on a copy of x (heads*head_dim values) with one table row."""
    x = np.array(x, np.float32)
    c = np.ascontiguousarray(np.asarray(cos_row, np.float32))
    s = np.ascontiguousarray(np.asarray(sin_row, np.float32))
    _chk(lib().ref_apply_rope(_p(x, C.c_float), heads, head_dim, rope_dim, int(split_half),
                              _p(c, C.c_float), _p(s, C.c_float)), "ref_apply_rope")
    return x


def exp_f32(x: np.ndarray) -> np.ndarray:
    f = lib().ref_exp_f32
    return np.array([f(float(v)) for v in np.asarray(x, np.float32)], np.float32)


def exp_f32_array(x: np.ndarray, clamp: bool = False) -> np.ndarray:
    """exp_f32 of every element in C (bit patterns pass unchanged, NaN
    payloads included); clamp: of max(x, -88)."""
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().ref_exp_f32_array(_p(x, C.c_float), _p(out, C.c_float), x.size, int(clamp))
    return out


def range_encode(triples) -> bytes:
    L = lib()
    e = L.ref_range_encoder_new()
    try:
        for cum, freq, total in triples:
            _chk(L.ref_range_encode(e, cum, freq, total), "ref_range_encode")
        n = L.ref_range_encoder_finish(e, None, 0)
        buf = (C.c_uint8 * n)()
        L.ref_range_encoder_finish(e, buf, n)
        return bytes(buf)
    finally:
        L.ref_range_encoder_free(e)


# ---- det-token byte fallback + det-cli windowed codec -----------------------
def canonical_byte_token(tok: str) -> int:
    """canonical_byte_fallback_token: the byte, or -1."""
    b = tok.encode()
    return int(lib().ref_canonical_byte_token(b, len(b)))


def byte_fallback_tables(tokens, emit=None):
    """(byte_to_token int32[256], token_to_byte int16[n]) of a vocabulary."""
    enc = [t.encode() for t in tokens]
    off = np.zeros(len(enc) + 1, np.uint64)
    off[1:] = np.cumsum([len(e) for e in enc]) if enc else []
    text = b"".join(enc)
    b2t = np.empty(256, np.int32)
    t2b = np.empty(max(len(enc), 1), np.int16)
    em = None if emit is None else np.ascontiguousarray(np.asarray(emit, np.uint8))
    _chk(lib().ref_byte_fallback_tables(text, off.ctypes.data_as(C.POINTER(C.c_size_t)), len(enc),
                                        None if em is None else _p(em, C.c_uint8),
                                        _p(b2t, C.c_int32), _p(t2b, C.c_int16)),
         "ref_byte_fallback_tables")
    return b2t, t2b[: len(enc)]


def codec_symbols(byte_to_token, data: bytes, vocab_len: int) -> np.ndarray:
    b2t = np.ascontiguousarray(np.asarray(byte_to_token, np.int32))
    src = np.frombuffer(bytes(data), np.uint8).copy()
    out = np.empty(max(src.size, 1), np.uint32)
    lib().ref_codec_symbols(_p(b2t, C.c_int32), _p(src, C.c_uint8), src.size, vocab_len,
                            _p(out, C.c_uint32))
    return out[: src.size]


def next_window_start(pos: int, window_start: int, n_ctx: int, overlap: int) -> int:
    return int(lib().ref_next_window_start(pos, window_start, n_ctx, overlap))


def codec_encode(model: Model, symbols, n_ctx: int, overlap: int, escapes: bool = True) -> bytes:
    """encode_symbols_with_model, one forward per token as the reference runs it."""
    sym = np.ascontiguousarray(np.asarray(symbols, np.uint32))
    n = C.c_size_t()
    _chk(lib().ref_codec_encode(model._h, _p(sym, C.c_uint32), sym.size, n_ctx, overlap, int(escapes),
                                None, 0, C.byref(n)), "ref_codec_encode")
    buf = (C.c_uint8 * n.value)()
    _chk(lib().ref_codec_encode(model._h, _p(sym, C.c_uint32), sym.size, n_ctx, overlap, int(escapes),
                                buf, n.value, C.byref(n)), "ref_codec_encode")
    return bytes(buf)


def codec_decode(model: Model, token_to_byte, payload: bytes, byte_len: int, n_ctx: int, overlap: int,
                 escapes: bool = True):
    """decode_bytes_with_model for a byte-fallback vocabulary: (symbols, bytes)."""
    t2b = np.ascontiguousarray(np.asarray(token_to_byte, np.int16))
    pl = np.frombuffer(bytes(payload), np.uint8).copy()
    syms = np.empty(max(byte_len, 1), np.uint32)
    out = np.empty(max(byte_len, 1), np.uint8)
    n = C.c_size_t()
    _chk(lib().ref_codec_decode(model._h, _p(t2b, C.c_int16), _p(pl, C.c_uint8), pl.size, byte_len, n_ctx,
                                overlap, int(escapes), _p(syms, C.c_uint32), _p(out, C.c_uint8),
                                C.byref(n)), "ref_codec_decode")
    return syms[: n.value], bytes(out[: n.value])
