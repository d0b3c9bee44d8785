"""det-model API mirror on top of the MI355X library.

Mirrors the public surface of crates/det-model/src/lib.rs (mii443/detllm):
``F32Llama::from_gguf`` (lib.rs:1035), ``forward_workspace`` (1244),
``forward_one[_with_workspace]`` (1228-1400) and the logits visitors
``logits_hash_for_tokens[_chunked]`` / ``logits_bytes_for_tokens_chunked`` /
``visit_logits_for_tokens_chunked`` (1402-1465).  A ``Session`` bundles the
reference's ``KvCache`` + ``ForwardWorkspace`` + ``RopeTables`` and lives on
the device; logits stay in HBM unless a caller asks for them.
"""
from __future__ import annotations

import ctypes as C
import enum
from dataclasses import dataclass
from typing import Callable, Iterable, Optional, Sequence

import numpy as np

from . import _lib
from ._lib import DetllmError, check, lib, ptr


class ModelError(enum.IntEnum):
    """det-model ModelError (lib.rs:48-59) with the C ABI status values."""

    Shape = 1
    NonFinite = 2
    UnsupportedArchitecture = 3
    UnsupportedAttentionHeadLength = 4
    UnsupportedModelFeature = 5
    UnsupportedRopeScaling = 6
    MissingMetadata = 7
    Gguf = 8
    UnsupportedTensorType = 9
    ThreadPanicked = 10


class RopePairing(enum.IntEnum):
    Adjacent = 0
    SplitHalf = 1


@dataclass(frozen=True)
class LlamaConfig:
    """LlamaConfig (lib.rs:27-39)."""

    block_count: int
    embedding_length: int
    feed_forward_length: int
    head_count: int
    head_count_kv: int
    rms_epsilon: float
    attention_scale: float
    rope_freq_base: float
    rope_dimension_count: int
    rope_pairing: RopePairing
    context_length: int

    @property
    def head_dim(self) -> int:
        return self.embedding_length // self.head_count


def _tokens(tokens: Iterable[int]) -> np.ndarray:
    arr = np.ascontiguousarray(np.asarray(list(tokens) if not isinstance(tokens, np.ndarray) else tokens,
                                          dtype=np.int64))
    if arr.ndim != 1:
        raise ValueError("tokens must be one-dimensional")
    if (arr < 0).any() or (arr >= 2**32).any():
        raise DetllmError(int(ModelError.Shape), "tokens")
    return arr.astype(np.uint32)


class F32Llama:
    """A Llama / Qwen2 decoder whose weights live in device memory."""

    def __init__(self, handle: int, gguf_bytes_len: int):
        self._h = C.c_void_p(handle)
        cfg = _lib.ModelConfig()
        check(lib.dtl_model_get_config(self._h, C.byref(cfg)), "dtl_model_get_config")
        self._cfg = cfg
        self.config = LlamaConfig(
            block_count=cfg.block_count,
            embedding_length=cfg.embedding_length,
            feed_forward_length=cfg.feed_forward_length,
            head_count=cfg.head_count,
            head_count_kv=cfg.head_count_kv,
            rms_epsilon=cfg.rms_epsilon,
            attention_scale=cfg.attention_scale,
            rope_freq_base=cfg.rope_freq_base,
            rope_dimension_count=cfg.rope_dimension_count,
            rope_pairing=RopePairing(cfg.rope_split_half),
            context_length=cfg.context_length,
        )
        self.vocab = int(cfg.vocab)
        self.device_bytes = int(cfg.device_bytes)
        self.embedding_type = int(cfg.embedding_type)
        self.output_type = int(cfg.output_type)

    @classmethod
    def from_gguf(cls, data: bytes) -> "F32Llama":
        """F32Llama::from_gguf: parse, validate and upload a GGUF model."""
        buf = bytes(data)
        h = C.c_void_p()
        check(lib.dtl_model_load(buf, len(buf), C.byref(h)), "dtl_model_load")
        return cls(h.value, len(buf))

    def close(self) -> None:
        if self._h:
            lib.dtl_model_free(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ---- sessions -------------------------------------------------------------
    def forward_workspace(self, max_context: int, max_chunk: int = 1) -> "Session":
        """forward_workspace + KvCache::new + RopeTables::llama, on the device."""
        return Session(self, max_context, max_chunk)

    def forward_one(self, token: int, pos: int, session: "Session") -> np.ndarray:
        return session.forward_one(token, pos)

    # ---- logits visitors (lib.rs:1402-1465) -------------------------------------
    def logits_hash_for_tokens(self, tokens: Sequence[int]) -> bytes:
        return self.logits_hash_for_tokens_chunked(tokens, 1)

    def logits_hash_for_tokens_chunked(self, tokens: Sequence[int], chunk_size: int) -> bytes:
        toks = _tokens(tokens)
        out = (C.c_uint8 * 32)()
        check(
            lib.dtl_logits_hash(self._h, ptr(toks, C.c_uint32), toks.size, int(chunk_size), out),
            "dtl_logits_hash",
        )
        return bytes(out)

    def visit_logits_for_tokens_chunked(
        self, tokens: Sequence[int], chunk_size: int, visit: Callable[[np.ndarray], None]
    ) -> None:
        toks = _tokens(tokens)
        if toks.size == 0 or chunk_size == 0 or toks.size > self.config.context_length:
            raise DetllmError(int(ModelError.Shape), "visit_logits_for_tokens_chunked")
        chunk = min(int(chunk_size), toks.size)
        with Session(self, toks.size, chunk) as s:
            for p in range(0, toks.size, chunk):
                block = s.forward_chunk(toks[p : p + chunk], p, want_logits=True)
                for row in block:
                    visit(row)

    def logits_bytes_for_tokens_chunked(self, tokens: Sequence[int], chunk_size: int) -> bytes:
        parts: list[bytes] = []
        self.visit_logits_for_tokens_chunked(tokens, chunk_size, lambda r: parts.append(r.tobytes()))
        return b"".join(parts)


class Session:
    """KvCache + ForwardWorkspace + RopeTables of one decode stream (device)."""

    def __init__(self, model: F32Llama, n_ctx: int, max_chunk: int = 1):
        self.model = model
        self.n_ctx = int(n_ctx)
        self.max_chunk = max(1, min(int(max_chunk), self.n_ctx))
        h = C.c_void_p()
        check(lib.dtl_session_new(model._h, self.n_ctx, self.max_chunk, C.byref(h)), "dtl_session_new")
        self._h = h
        self.rows = 0

    def close(self) -> None:
        if self._h:
            lib.dtl_session_free(self._h)
            self._h = C.c_void_p()

    def __enter__(self) -> "Session":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self) -> None:
        """A fresh KvCache (window replay restarts from position 0)."""
        check(lib.dtl_session_reset(self._h), "dtl_session_reset")
        self.rows = 0

    def forward_one(self, token: int, pos: int, want_logits: bool = True) -> Optional[np.ndarray]:
        out = self.forward_chunk([token], pos, want_logits)
        return None if out is None else out[0]

    def forward_chunk(self, tokens: Sequence[int], pos0: int, want_logits: bool = False) -> Optional[np.ndarray]:
        toks = _tokens(tokens)
        V = self.model.vocab
        out = np.empty((toks.size, V), dtype=np.float32) if want_logits else None
        check(
            lib.dtl_forward_chunk(
                self._h, ptr(toks, C.c_uint32), toks.size, int(pos0),
                ptr(out, C.c_float) if out is not None else None,
            ),
            "dtl_forward_chunk",
        )
        self.rows = toks.size
        return out

    def logits(self, first: int = 0, n: Optional[int] = None) -> np.ndarray:
        n = self.rows - first if n is None else n
        out = np.empty((n, self.model.vocab), dtype=np.float32)
        check(lib.dtl_session_logits(self._h, first, n, ptr(out, C.c_float)), "dtl_session_logits")
        return out

    # ---- device timing ----------------------------------------------------------------
    def set_profiling(self, enable: bool) -> None:
        """HIP-event timing of every launch on this session's stream."""
        check(lib.dtl_session_set_profiling(self._h, 1 if enable else 0), "dtl_session_set_profiling")

    def profile_only(self, kernel_class: Optional[str]) -> None:
        """Restricts timing to one kernel class (None: every class)."""
        arg = kernel_class.encode() if kernel_class else None
        check(lib.dtl_session_profile_only(self._h, arg), "dtl_session_profile_only")

    def profile(self) -> dict:
        """{kernel class: {launches, total_ms, bytes, macs}} since profiling was enabled."""
        n = C.c_size_t()
        check(lib.dtl_session_profile(self._h, None, 0, C.byref(n)), "dtl_session_profile")
        arr = (_lib.KernelStat * max(n.value, 1))()
        check(lib.dtl_session_profile(self._h, arr, n.value, C.byref(n)), "dtl_session_profile")
        return {
            s.name.decode(): {"launches": int(s.launches), "total_ms": float(s.total_ms),
                              "bytes": float(s.bytes), "macs": float(s.macs)}
            for s in arr[: n.value]
        }

    # ---- det-coder on the device-resident logits -----------------------------------
    def symbol_ranges(self, symbols: Sequence[int], first: int = 0, tail_symbols: int = 0):
        """logits_to_symbol_range_* for rows first.. of the last forward."""
        sym = np.ascontiguousarray(np.asarray(symbols, dtype=np.uint32))
        n = sym.size
        cum = np.empty(n, np.uint64)
        freq = np.empty(n, np.uint32)
        total = np.empty(n, np.uint64)
        check(
            lib.dtl_symbol_ranges(self._h, first, n, ptr(sym, C.c_uint32), tail_symbols,
                                  ptr(cum, C.c_uint64), ptr(freq, C.c_uint32), ptr(total, C.c_uint64)),
            "dtl_symbol_ranges",
        )
        return cum, freq, total

    def symbol_ranges_rows(self, rows: Sequence[int], symbols: Sequence[int], tail_symbols: int = 0):
        """logits_to_symbol_range_* of symbols[i] against row rows[i] of the last forward."""
        r = np.ascontiguousarray(np.asarray(rows, dtype=np.uint32))
        sym = np.ascontiguousarray(np.asarray(symbols, dtype=np.uint32))
        if r.size != sym.size:
            raise ValueError("rows and symbols differ in length")
        n = sym.size
        cum = np.empty(n, np.uint64)
        freq = np.empty(n, np.uint32)
        total = np.empty(n, np.uint64)
        check(
            lib.dtl_symbol_ranges_rows(self._h, n, ptr(r, C.c_uint32), ptr(sym, C.c_uint32), tail_symbols,
                                       ptr(cum, C.c_uint64), ptr(freq, C.c_uint32), ptr(total, C.c_uint64)),
            "dtl_symbol_ranges_rows",
        )
        return cum, freq, total

    def forward_ranges(self, tokens: Sequence[int], pos0: int, rows: Sequence[int], symbols: Sequence[int],
                       tail_symbols: int = 0):
        """Forwards of tokens at pos0.. (chunks of max_chunk, three in flight) and the
        range of symbols[i] under the logits of token rows[i]: (cum, freq, total)."""
        toks = _tokens(tokens)
        r = np.ascontiguousarray(np.asarray(rows, dtype=np.uint32))
        sym = np.ascontiguousarray(np.asarray(symbols, dtype=np.uint32))
        if r.size != sym.size:
            raise ValueError("rows and symbols differ in length")
        n = sym.size
        cum = np.empty(max(n, 1), np.uint64)
        freq = np.empty(max(n, 1), np.uint32)
        total = np.empty(max(n, 1), np.uint64)
        check(
            lib.dtl_forward_ranges(self._h, ptr(toks, C.c_uint32), toks.size, int(pos0), n,
                                   ptr(r, C.c_uint32), ptr(sym, C.c_uint32), tail_symbols,
                                   ptr(cum, C.c_uint64), ptr(freq, C.c_uint32), ptr(total, C.c_uint64)),
            "dtl_forward_ranges",
        )
        return cum[:n], freq[:n], total[:n]

    def cdf(self, row: int = 0, tail_symbols: int = 0):
        """logits_to_cdf_* of one row: (freq[u32], cum[u64], total)."""
        n = self.model.vocab + tail_symbols
        freq = np.empty(n, np.uint32)
        cum = np.empty(n, np.uint64)
        total = C.c_uint64()
        check(lib.dtl_cdf(self._h, row, tail_symbols, ptr(freq, C.c_uint32), ptr(cum, C.c_uint64),
                          C.byref(total)), "dtl_cdf")
        return freq, cum, int(total.value)

    def decoder_total(self, row: int = 0, tail_symbols: int = 0) -> int:
        total = C.c_uint64()
        check(lib.dtl_decoder_total(self._h, row, tail_symbols, C.byref(total)), "dtl_decoder_total")
        return int(total.value)

    def decoder_lookup(self, value: int, row: int = 0, tail_symbols: int = 0):
        """DecoderDistribution::symbol_range on the device: (symbol, cum, freq, total)."""
        sym = C.c_uint32()
        cum = C.c_uint64()
        freq = C.c_uint32()
        total = C.c_uint64()
        check(lib.dtl_decoder_lookup(self._h, row, tail_symbols, int(value), C.byref(sym), C.byref(cum),
                                     C.byref(freq), C.byref(total)), "dtl_decoder_lookup")
        return int(sym.value), int(cum.value), int(freq.value), int(total.value)

    def decode_symbol(self, dec, row: int = 0, tail_symbols: int = 0) -> int:
        """decode_symbol's model branch (det-cli main.rs:724-750) on row `row`:
        distribution, decode_freq, symbol_range and advance of the
        coder.RangeDecoder `dec`, one wait for the device."""
        sym = C.c_uint32()
        check(lib.dtl_decoder_decode(self._h, row, tail_symbols, dec._h, C.byref(sym)), "dtl_decoder_decode")
        return int(sym.value)

    def forward_decode(self, token: int, pos: int, dec, tail_symbols: int = 0) -> int:
        """advance(token) then decode_symbol (det-cli main.rs:570-575): the
        forward of `token` at `pos` and the next symbol from its logits."""
        sym = C.c_uint32()
        check(lib.dtl_forward_decode(self._h, int(token), int(pos), tail_symbols, dec._h, C.byref(sym)),
              "dtl_forward_decode")
        self.rows = 1
        return int(sym.value)
