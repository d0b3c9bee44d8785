"""GGUF v3 writer for synthetic models.

Writes the container that crates/det-gguf/src/lib.rs (mii443/detllm) reads:
little-endian header, metadata table, tensor infos with dims [cols, rows],
32-byte aligned data section.  The layout choices (alignment, tokenizer
token array) follow the reference's fixture encoder
(xtask/src/main.rs:4939-4984).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field
from typing import Dict, List, Tuple, Union

import numpy as np

ALIGN = 32

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 0, 1, 2, 8, 12, 14

# (bytes per block, elements per block)
TYPE_SIZE = {GGML_F32: (4, 1), GGML_F16: (2, 1), GGML_Q4_0: (18, 32), GGML_Q8_0: (34, 32),
             GGML_Q4_K: (144, 256), GGML_Q6_K: (210, 256)}

_U32, _I32, _F32, _BOOL, _STR, _ARR, _U64, _F64 = 4, 5, 6, 7, 8, 9, 10, 12


@dataclass
class Tensor:
    name: str
    dims: Tuple[int, ...]  # GGUF order: [cols, rows] for matrices
    ggml_type: int
    data: bytes


@dataclass
class GgufWriter:
    metadata: List[Tuple[str, int, object]] = field(default_factory=list)
    tensors: List[Tensor] = field(default_factory=list)

    def add_u32(self, key: str, v: int) -> None:
        self.metadata.append((key, _U32, int(v)))

    def add_f32(self, key: str, v: float) -> None:
        self.metadata.append((key, _F32, float(v)))

    def add_bool(self, key: str, v: bool) -> None:
        self.metadata.append((key, _BOOL, bool(v)))

    def add_str(self, key: str, v: str) -> None:
        self.metadata.append((key, _STR, v))

    def add_str_array(self, key: str, v: List[str]) -> None:
        self.metadata.append((key, _ARR, (_STR, list(v))))

    def add_i32_array(self, key: str, v: List[int]) -> None:
        self.metadata.append((key, _ARR, (_I32, [int(x) for x in v])))

    def add_tensor(self, name: str, dims: Tuple[int, ...], ggml_type: int, data: Union[bytes, np.ndarray]) -> None:
        raw = data.tobytes() if isinstance(data, np.ndarray) else bytes(data)
        n = 1
        for d in dims:
            n *= d
        bpb, epb = TYPE_SIZE[ggml_type]
        if n % epb or len(raw) != n // epb * bpb:
            raise ValueError(f"{name}: {len(raw)} bytes do not match dims {dims} type {ggml_type}")
        self.tensors.append(Tensor(name, tuple(dims), ggml_type, raw))

    @staticmethod
    def _str(s: str) -> bytes:
        b = s.encode()
        return struct.pack("<Q", len(b)) + b

    def to_bytes(self) -> bytes:
        out = bytearray()
        out += b"GGUF" + struct.pack("<IQQ", 3, len(self.tensors), len(self.metadata))
        for key, ty, v in self.metadata:
            out += self._str(key) + struct.pack("<I", ty)
            if ty == _U32:
                out += struct.pack("<I", v)
            elif ty == _F32:
                out += struct.pack("<f", v)
            elif ty == _BOOL:
                out += struct.pack("<B", 1 if v else 0)
            elif ty == _STR:
                out += self._str(v)
            elif ty == _ARR:
                ety, items = v
                out += struct.pack("<IQ", ety, len(items))
                if ety == _STR:
                    for s in items:
                        out += self._str(s)
                else:
                    out += struct.pack(f"<{len(items)}i", *items)
            else:
                raise ValueError(ty)
        offset = 0
        offsets = []
        for t in self.tensors:
            offsets.append(offset)
            offset += len(t.data)
            offset = (offset + ALIGN - 1) // ALIGN * ALIGN
        for t, off in zip(self.tensors, offsets):
            out += self._str(t.name) + struct.pack("<I", len(t.dims))
            for d in t.dims:
                out += struct.pack("<Q", d)
            out += struct.pack("<IQ", t.ggml_type, off)
        pad = (-len(out)) % ALIGN
        out += b"\0" * pad
        base = len(out)
        buf = bytearray(base + offset)
        buf[:base] = out
        for t, off in zip(self.tensors, offsets):
            buf[base + off: base + off + len(t.data)] = t.data
        return bytes(buf)
