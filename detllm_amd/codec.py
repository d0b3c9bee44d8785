"""det-token byte-fallback tokenizer + det-cli windowed codec mirror.

Mirrors, on top of the C ABI of include/detllm.h:

* ``Tokenizer`` — det-token ``Tokenizer::from_gguf`` for the byte-fallback
  kind, ``codec_symbols``, ``decode_codec_symbol``, ``codec_symbol_is_token``
  (crates/det-token/src/lib.rs:85-209, 258-325, 841-847);
* ``LoadedModel`` — det-cli ``LoadedModel::load`` (main.rs:926-1000): model
  SHA-256, tokenizer, device model and the vocabulary checks;
* ``encode_symbols_with_model`` / ``decode_tokens_with_model`` /
  ``decode_bytes_with_model`` (main.rs:514-632) over a device ``Session``
  whose n_ctx is the codec window;
* ``compress`` / ``decompress`` (main.rs:431-512) producing / consuming the
  DTLZ file (header + payload).

Every step runs in libdetllm_amd.so: forwards and CDFs on the GPU, the range
coder and the window bookkeeping on the host side of the library.
"""
from __future__ import annotations

import ctypes as C
import enum
import hashlib
from dataclasses import dataclass
from typing import List, Optional, Sequence

import numpy as np

from . import _lib
from ._lib import DetllmError, check, lib, ptr
from .coder import BYTE_ESCAPE_SYMBOLS, DtlzHeader, FLAG_BYTE_ESCAPES, HEADER_LEN
from .model import F32Llama, Session


class TokenError(enum.IntEnum):
    """det-token TokenError (lib.rs:6-25) with the C ABI status values."""

    MissingByteFallback = 60
    InvalidToken = 61
    MissingVocabulary = 62
    MissingTokenBytes = 63
    MissingMergeToken = 64
    IncompleteByteFallback = 65
    MetadataType = 66
    TokenTypeLength = 67
    InvalidTokenType = 68
    ScoresLength = 69
    NonFiniteScore = 70
    TokenIndexOverflow = 71
    DuplicateByteFallback = 72
    DuplicateTokenId = 73
    DuplicateTokenBytes = 74
    InvalidMerge = 75
    DuplicateMerge = 76
    UnsupportedModel = 77


class CodecError(enum.IntEnum):
    ModelMismatch = 90
    NotCanonical = 91
    EscapeInTokenStream = 92
    VocabMismatch = 93


def _u8(data: bytes):
    buf = bytes(data)
    return (C.c_uint8 * max(len(buf), 1)).from_buffer_copy(buf or b"\0"), len(buf)


class Tokenizer:
    """Tokenizer::from_gguf for a byte-fallback vocabulary (no tokenizer
    model, merges or scores)."""

    def __init__(self, handle: int):
        self._h = C.c_void_p(handle)

    @classmethod
    def from_gguf(cls, data: bytes) -> "Tokenizer":
        buf = bytes(data)
        h = C.c_void_p()
        check(lib.dtl_tokenizer_from_gguf(buf, len(buf), C.byref(h)), "Tokenizer::from_gguf")
        return cls(h.value)

    def close(self) -> None:
        if self._h:
            lib.dtl_tokenizer_free(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def vocab_len(self) -> int:
        return int(lib.dtl_tokenizer_vocab_len(self._h))

    def codec_symbols(self, data: bytes, vocab_len: int) -> np.ndarray:
        """One symbol per byte: its emittable token, else vocab_len + byte."""
        src, n = _u8(data)
        out = np.empty(max(n, 1), np.uint32)
        got = C.c_size_t()
        check(lib.dtl_tokenizer_codec_symbols(self._h, src, n, vocab_len, ptr(out, C.c_uint32), out.size,
                                              C.byref(got)), "Tokenizer::codec_symbols")
        return out[: got.value]

    def decode_codec_symbol(self, symbol: int, vocab_len: int) -> bytes:
        if symbol < 0 or symbol >= 1 << 32:
            raise DetllmError(int(TokenError.InvalidToken), "Tokenizer::decode_codec_symbol")
        out = (C.c_uint8 * 1)()
        n = C.c_size_t()
        check(lib.dtl_tokenizer_decode_symbol(self._h, symbol, vocab_len, out, 1, C.byref(n)),
              "Tokenizer::decode_codec_symbol")
        return bytes(out[: n.value])

    @staticmethod
    def codec_symbol_is_token(symbol: int, vocab_len: int) -> bool:
        return symbol < vocab_len


@dataclass
class LoadedModel:
    """LoadedModel (main.rs:926-1000): model hash, tokenizer, device model."""

    model_sha256: bytes
    model: F32Llama
    tokenizer: Tokenizer

    @classmethod
    def load(cls, gguf: bytes) -> "LoadedModel":
        data = bytes(gguf)
        sha = hashlib.sha256(data).digest()
        tok = Tokenizer.from_gguf(data)
        model = F32Llama.from_gguf(data)
        if tok.vocab_len != model.vocab:
            raise DetllmError(int(CodecError.VocabMismatch),
                              f"tokenizer vocabulary length {tok.vocab_len} does not match model "
                              f"vocabulary {model.vocab}")
        if model.vocab + BYTE_ESCAPE_SYMBOLS > 1 << 18:
            raise DetllmError(24, "validate_codec_vocab_len")
        return cls(sha, model, tok)


def encode_symbols_with_model(session: Session, symbols: Sequence[int], overlap: int,
                              use_byte_escapes: bool = True) -> bytes:
    """encode_symbols_with_model with window n_ctx = session.n_ctx."""
    sym = np.ascontiguousarray(np.asarray(symbols, dtype=np.uint32))
    n = C.c_size_t()
    st = lib.dtl_codec_encode(session._h, ptr(sym, C.c_uint32), sym.size, overlap, int(use_byte_escapes),
                              None, 0, C.byref(n))
    check(st, "encode_symbols_with_model")
    buf = (C.c_uint8 * max(n.value, 1))()
    check(lib.dtl_codec_encode(session._h, ptr(sym, C.c_uint32), sym.size, overlap, int(use_byte_escapes),
                               buf, n.value, C.byref(n)), "encode_symbols_with_model")
    return bytes(buf[: n.value])


def encode_tokens_with_model(session: Session, tokens: Sequence[int], overlap: int) -> bytes:
    """encode_tokens_with_model (main.rs:514-519): byte escapes on."""
    return encode_symbols_with_model(session, tokens, overlap, True)


def _decode(session: Session, payload: bytes, overlap: int, escapes: bool, piece_len, byte_len: int,
            max_symbols: int) -> np.ndarray:
    pl, plen = _u8(payload)
    out = np.empty(max(max_symbols, 1), np.uint32)
    n = C.c_size_t()
    pieces = None
    if piece_len is not None:
        pieces = np.ascontiguousarray(np.asarray(piece_len, np.uint8))
    st = lib.dtl_codec_decode(session._h, pl, plen, overlap, int(escapes),
                              None if pieces is None else ptr(pieces, C.c_uint8), byte_len, max_symbols,
                              ptr(out, C.c_uint32), C.byref(n))
    check(st, "decode_with_model")
    return out[: n.value]


def decode_tokens_with_model(session: Session, payload: bytes, token_len: int, overlap: int) -> List[int]:
    """decode_tokens_with_model (main.rs:553-572): token_len tokens; a byte
    escape is an error."""
    syms = _decode(session, payload, overlap, True, None, 0, token_len)
    V = session.model.vocab
    for s in syms:
        if not Tokenizer.codec_symbol_is_token(int(s), V):
            raise DetllmError(int(CodecError.EscapeInTokenStream), "decode_tokens_with_model")
    return [int(s) for s in syms]


@dataclass
class DecodedBytes:
    bytes: bytes
    symbols: List[int]


def decode_bytes_with_model(session: Session, tokenizer: Tokenizer, payload: bytes, byte_len: int,
                            overlap: int, use_byte_escapes: bool = True) -> DecodedBytes:
    """decode_bytes_with_model (main.rs:573-632) for a byte-fallback
    vocabulary: every symbol decodes to one byte."""
    V = session.model.vocab
    pieces = np.zeros(V + BYTE_ESCAPE_SYMBOLS, np.uint8)
    one = np.zeros(V + BYTE_ESCAPE_SYMBOLS, np.uint8)
    for s in range(V + BYTE_ESCAPE_SYMBOLS):
        try:
            b = tokenizer.decode_codec_symbol(s, V)
        except DetllmError:
            continue
        pieces[s] = len(b)
        one[s] = b[0]
    syms = _decode(session, payload, overlap, use_byte_escapes, pieces, byte_len, byte_len)
    return DecodedBytes(bytes(one[syms].tobytes()), [int(s) for s in syms])


def _take(p, n: int) -> bytes:
    try:
        return C.string_at(p, n)
    finally:
        lib.dtl_bytes_free(p)


# Positions per forward chunk of the codec's sessions.  The bytes do not
# depend on it (every position's logits are the same whatever the chunking);
# 512 measured fastest on the Qwen2.5-0.5B shape (8 KiB compress: 8.9 KB/s at
# 64, 10.0k at 128, 11.2k at 512, 11.4k at 1024).
CODEC_CHUNK = 512


def compress(loaded: LoadedModel, data: bytes, n_ctx: Optional[int] = None,
             max_chunk: int = CODEC_CHUNK) -> bytes:
    """compress (main.rs:431-462): DTLZ header + payload."""
    src, n = _u8(data)
    sha, _ = _u8(loaded.model_sha256)
    out = _lib.u8p()
    size = C.c_size_t()
    check(lib.dtl_compress(loaded.model._h, loaded.tokenizer._h, sha, src, n, n_ctx or 0, max_chunk,
                           C.byref(out), C.byref(size)), "compress")
    return _take(out, size.value)


def decompress(loaded: Optional[LoadedModel], file: bytes, max_chunk: int = CODEC_CHUNK) -> bytes:
    """decompress (main.rs:464-512).  The header is validated first, so a
    malformed file fails even without a model."""
    src, n = _u8(file)
    out = _lib.u8p()
    size = C.c_size_t()
    if loaded is None:
        st = lib.dtl_decompress(None, None, None, src, n, max_chunk, C.byref(out), C.byref(size))
        check(st, "decompress")
        raise DetllmError(42, "decompress: a model is required")
    sha, _ = _u8(loaded.model_sha256)
    check(lib.dtl_decompress(loaded.model._h, loaded.tokenizer._h, sha, src, n, max_chunk, C.byref(out),
                             C.byref(size)), "decompress")
    return _take(out, size.value)


@dataclass
class DecompressPart:
    symbols: np.ndarray              # the symbols this call decoded
    state: "_lib.RangeDecoderState"  # the range decoder's state after them
    done: bool
    data: Optional[bytes]            # the decompressed bytes once done


def decompress_part(loaded: LoadedModel, file: bytes, prior: Sequence[int] = (),
                    state: Optional["_lib.RangeDecoderState"] = None, max_new: int = 1 << 16,
                    max_chunk: int = CODEC_CHUNK) -> DecompressPart:
    """decompress over several calls (no counterpart in the reference): up to
    max_new symbols after `prior` (all symbols of the earlier calls), resuming
    the range decoder from `state`; once the symbols cover the original
    length, the canonical check runs and `data` holds the bytes."""
    src, n = _u8(file)
    sha, _ = _u8(loaded.model_sha256)
    pr = np.ascontiguousarray(np.asarray(prior, dtype=np.uint32))
    out_sym = np.empty(max(max_new, 1), np.uint32)
    n_new = C.c_size_t()
    st_out = _lib.RangeDecoderState()
    done = C.c_int()
    out = _lib.u8p()
    size = C.c_size_t()
    check(lib.dtl_decompress_part(loaded.model._h, loaded.tokenizer._h, sha, src, n, max_chunk,
                                  ptr(pr, C.c_uint32) if pr.size else None, pr.size,
                                  C.byref(state) if state is not None else None, max_new,
                                  ptr(out_sym, C.c_uint32), out_sym.size, C.byref(n_new), C.byref(st_out),
                                  C.byref(done), C.byref(out), C.byref(size)), "decompress_part")
    data = _take(out, size.value) if done.value else None
    return DecompressPart(out_sym[: n_new.value].copy(), st_out, bool(done.value), data)


def next_window_start(pos: int, window_start: int, n_ctx: int, overlap: int) -> int:
    """next_window_start (main.rs:801-808)."""
    return int(lib.dtl_codec_next_window_start(pos, window_start, n_ctx, overlap))


__all__ = [
    "BYTE_ESCAPE_SYMBOLS", "CodecError", "DecodedBytes", "DtlzHeader", "FLAG_BYTE_ESCAPES", "HEADER_LEN",
    "DecompressPart", "LoadedModel", "TokenError", "Tokenizer", "compress", "decode_bytes_with_model",
    "decode_tokens_with_model", "decompress", "decompress_part", "encode_symbols_with_model",
    "encode_tokens_with_model",
    "next_window_start",
]
