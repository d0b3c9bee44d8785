"""det-coder API mirror: logits -> integer CDF on the device, range coder on the host.

Mirrors crates/det-coder of mii443/detllm: ``logits_to_cdf*`` /
``logits_to_symbol_range*`` / ``uniform_*`` (src/cdf.rs:47-341),
``RangeEncoder`` / ``RangeDecoder`` (src/range.rs:10-159) and the 56-byte
``DtlzHeader`` (src/file.rs:1-89).
"""
from __future__ import annotations

import ctypes as C
import enum
import struct
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._lib import DetllmError, check, lib, ptr

M = 16_777_216
MAX_SYMBOLS = 1 << 18
BYTE_ESCAPE_SYMBOLS = 256


class CdfError(enum.IntEnum):
    Empty = 20
    Malformed = 21
    NonFiniteLogit = 22
    SymbolOutOfRange = 23
    TooManySymbols = 24
    TotalTooLarge = 25


class RangeError(enum.IntEnum):
    InvalidFrequency = 30
    UnexpectedEof = 31


@dataclass(frozen=True)
class SymbolRange:
    cum: int
    freq: int
    total: int


@dataclass
class Cdf:
    freq: np.ndarray  # u32
    cum: np.ndarray   # u64
    total: int


def _logits(x) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


def _cdf(logits, tail: int) -> Cdf:
    lg = _logits(logits)
    n = lg.size + tail
    freq = np.empty(max(n, 1), np.uint32)
    cum = np.empty(max(n, 1), np.uint64)
    total = C.c_uint64()
    check(lib.dtl_logits_to_cdf(ptr(lg, C.c_float), lg.size, tail, ptr(freq, C.c_uint32),
                                ptr(cum, C.c_uint64), C.byref(total)), "logits_to_cdf")
    return Cdf(freq[:n], cum[:n], int(total.value))


def logits_to_cdf(logits) -> Cdf:
    """logits_to_cdf (cdf.rs:47-106)."""
    return _cdf(logits, 0)


def logits_to_cdf_with_byte_escapes(logits) -> Cdf:
    """logits_to_cdf_with_byte_escapes (cdf.rs:95-106, 255-286)."""
    return _cdf(logits, BYTE_ESCAPE_SYMBOLS)


def _range(logits, symbol: int, tail: int) -> SymbolRange:
    lg = _logits(logits)
    if symbol < 0:
        raise DetllmError(int(CdfError.SymbolOutOfRange), "logits_to_symbol_range")
    cum, total = C.c_uint64(), C.c_uint64()
    freq = C.c_uint32()
    check(lib.dtl_logits_to_symbol_range(ptr(lg, C.c_float), lg.size, int(symbol), tail, C.byref(cum),
                                         C.byref(freq), C.byref(total)), "logits_to_symbol_range")
    return SymbolRange(int(cum.value), int(freq.value), int(total.value))


def logits_to_symbol_range(logits, symbol: int) -> SymbolRange:
    """logits_to_symbol_range_with_scratch (cdf.rs:123-130, 138-199)."""
    return _range(logits, symbol, 0)


def logits_to_symbol_range_with_byte_escapes(logits, symbol: int) -> SymbolRange:
    """logits_to_symbol_range_with_byte_escapes (cdf.rs:131-136)."""
    return _range(logits, symbol, BYTE_ESCAPE_SYMBOLS)


def uniform_cdf(symbols: int) -> Cdf:
    """uniform_cdf (cdf.rs:302-320)."""
    freq = np.empty(max(symbols, 1), np.uint32)
    cum = np.empty(max(symbols, 1), np.uint64)
    total = C.c_uint64()
    check(lib.dtl_uniform_cdf(symbols, ptr(freq, C.c_uint32), ptr(cum, C.c_uint64), C.byref(total)),
          "uniform_cdf")
    return Cdf(freq[:symbols], cum[:symbols], int(total.value))


def uniform_cdf_with_byte_escapes(vocab_len: int) -> Cdf:
    """uniform_cdf_with_byte_escapes (cdf.rs:102-106): vocabulary + 256 escape symbols."""
    return uniform_cdf(vocab_len + BYTE_ESCAPE_SYMBOLS)


def uniform_symbol_range(symbol: int, symbols: int) -> SymbolRange:
    """uniform_symbol_range (cdf.rs:322-341)."""
    cum, total = C.c_uint64(), C.c_uint64()
    freq = C.c_uint32()
    check(lib.dtl_uniform_symbol_range(symbol, symbols, C.byref(cum), C.byref(freq), C.byref(total)),
          "uniform_symbol_range")
    return SymbolRange(int(cum.value), int(freq.value), int(total.value))


@dataclass
class RangeEncoderSnapshot:
    """RangeEncoderSnapshot (range.rs:17-22)."""
    low: int
    range: int
    out: bytes


class RangeEncoder:
    """RangeEncoder (range.rs:10-92): 64-bit low/range, carry-less renormalisation."""

    def __init__(self):
        h = C.c_void_p()
        check(lib.dtl_range_encoder_new(C.byref(h)), "RangeEncoder::new")
        self._h = h

    def encode(self, cum: int, freq: int, total: int) -> None:
        check(lib.dtl_range_encode(self._h, cum, freq, total), "RangeEncoder::encode")

    def snapshot(self) -> RangeEncoderSnapshot:
        """RangeEncoder::snapshot (range.rs:48-54)."""
        low, rng, n = C.c_uint64(), C.c_uint64(), C.c_size_t()
        check(lib.dtl_range_encoder_snapshot(self._h, C.byref(low), C.byref(rng), None, 0, C.byref(n)),
              "RangeEncoder::snapshot")
        buf = (C.c_uint8 * max(n.value, 1))()
        check(lib.dtl_range_encoder_snapshot(self._h, C.byref(low), C.byref(rng), buf, n.value, C.byref(n)),
              "RangeEncoder::snapshot")
        return RangeEncoderSnapshot(int(low.value), int(rng.value), bytes(buf)[:n.value])

    @classmethod
    def from_snapshot(cls, snap: "RangeEncoderSnapshot") -> "RangeEncoder":
        """RangeEncoder::from_snapshot (range.rs:37-46)."""
        self = cls.__new__(cls)
        data = (C.c_uint8 * max(len(snap.out), 1)).from_buffer_copy(bytes(snap.out) or b"\0")
        h = C.c_void_p()
        self._h = C.c_void_p()
        check(lib.dtl_range_encoder_from_snapshot(snap.low, snap.range, data, len(snap.out), C.byref(h)),
              "RangeEncoder::from_snapshot")
        self._h = h
        return self

    def finish(self) -> bytes:
        n = C.c_size_t()
        check(lib.dtl_range_encoder_finish(self._h, None, 0, C.byref(n)), "RangeEncoder::finish")
        buf = (C.c_uint8 * n.value)()
        check(lib.dtl_range_encoder_finish(self._h, buf, n.value, C.byref(n)), "RangeEncoder::finish")
        return bytes(buf)

    def __del__(self):
        try:
            if self._h:
                lib.dtl_range_encoder_free(self._h)
                self._h = C.c_void_p()
        except Exception:
            pass


class RangeDecoder:
    """RangeDecoder (range.rs:94-159)."""

    def __init__(self, data: bytes):
        self._buf = (C.c_uint8 * max(len(data), 1)).from_buffer_copy(bytes(data) or b"\0")
        h = C.c_void_p()
        check(lib.dtl_range_decoder_new(self._buf, len(data), C.byref(h)), "RangeDecoder::new")
        self._h = h

    def decode_freq(self, total: int) -> int:
        v = C.c_uint64()
        check(lib.dtl_range_decode_freq(self._h, total, C.byref(v)), "RangeDecoder::decode_freq")
        return int(v.value)

    def advance(self, cum: int, freq: int, total: int) -> None:
        check(lib.dtl_range_decode_advance(self._h, cum, freq, total), "RangeDecoder::advance")

    def snapshot(self) -> "_lib.RangeDecoderState":
        """The state between two symbols (low, range, code, bytes consumed); no
        counterpart in the reference, for a decode continued in a later call."""
        st = _lib.RangeDecoderState()
        check(lib.dtl_range_decoder_snapshot(self._h, C.byref(st)), "RangeDecoder::snapshot")
        return st

    @classmethod
    def from_snapshot(cls, data: bytes, state: "_lib.RangeDecoderState") -> "RangeDecoder":
        self = cls.__new__(cls)
        self._buf = (C.c_uint8 * max(len(data), 1)).from_buffer_copy(bytes(data) or b"\0")
        h = C.c_void_p()
        check(lib.dtl_range_decoder_from_snapshot(self._buf, len(data), C.byref(state), C.byref(h)),
              "RangeDecoder::from_snapshot")
        self._h = h
        return self

    def __del__(self):
        try:
            if self._h:
                lib.dtl_range_decoder_free(self._h)
                self._h = C.c_void_p()
        except Exception:
            pass


MAGIC = b"DTLZ"
VERSION = 1
FLAG_BYTE_ESCAPES = 1
HEADER_LEN = 56


class FileError(enum.IntEnum):
    """det-coder FileError (file.rs:18-26) with the C ABI status values."""

    TooShort = 80
    BadMagic = 81
    UnsupportedVersion = 82
    UnsupportedFlags = 83
    InvalidContext = 84
    InvalidOverlap = 85


@dataclass(frozen=True)
class DtlzHeader:
    """DtlzHeader (file.rs:8-89): 56-byte little-endian container header,
    encoded and validated by dtl_dtlz_header_{encode,decode}."""

    flags: int
    model_sha256: bytes
    n_ctx: int
    overlap: int
    orig_len: int

    def encode_checked(self) -> bytes:
        sha = (C.c_uint8 * 32).from_buffer_copy(bytes(self.model_sha256).ljust(32, b"\0")[:32])
        out = (C.c_uint8 * HEADER_LEN)()
        check(lib.dtl_dtlz_header_encode(self.flags, sha, self.n_ctx, self.overlap, self.orig_len, out),
              "DtlzHeader::encode_checked")
        return bytes(out)

    def encode(self) -> bytes:
        """DtlzHeader::encode: the 56 bytes without validation (for writing
        deliberately malformed files)."""
        return (MAGIC + struct.pack("<HH", VERSION, self.flags) + bytes(self.model_sha256)
                + struct.pack("<IIQ", self.n_ctx, self.overlap, self.orig_len))

    def validate(self) -> None:
        self.encode_checked()

    @classmethod
    def decode(cls, data: bytes) -> "DtlzHeader":
        buf = (C.c_uint8 * max(len(data), 1)).from_buffer_copy(bytes(data) or b"\0")
        flags, n_ctx, overlap = C.c_uint16(), C.c_uint32(), C.c_uint32()
        orig_len = C.c_uint64()
        sha = (C.c_uint8 * 32)()
        check(lib.dtl_dtlz_header_decode(buf, len(data), C.byref(flags), sha, C.byref(n_ctx),
                                         C.byref(overlap), C.byref(orig_len)), "DtlzHeader::decode")
        return cls(int(flags.value), bytes(sha), int(n_ctx.value), int(overlap.value),
                   int(orig_len.value))
