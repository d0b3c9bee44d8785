"""GGUF block encoders and an independent integer decoder for tests.

Builds raw GGUF rows (Q8_0 34 B, Q4_0 18 B, Q4_K 144 B, Q6_K 210 B per
block) from explicit fields, and decodes them with numpy straight from the
GGUF block format, so closed-form checks do not reuse the oracle's code.
"""
from __future__ import annotations

import numpy as np

F16_ONE = 0x3C00


def f16(v: float) -> int:
    return int(np.array([v], np.float16).view(np.uint16)[0])


# ---- encoders -------------------------------------------------------------------

def q8_0_row(d16: np.ndarray, q: np.ndarray) -> bytes:
    nb = d16.size
    out = np.empty((nb, 34), np.uint8)
    out[:, :2] = d16.astype(np.uint16).view(np.uint8).reshape(nb, 2)
    out[:, 2:] = q.astype(np.int8).view(np.uint8).reshape(nb, 32)
    return out.tobytes()


def q4_0_row(d16: np.ndarray, nib: np.ndarray) -> bytes:
    """nib[b][i] for i < 32 is the 4-bit code of element i of block b."""
    nb = d16.size
    nib = nib.reshape(nb, 32)
    out = np.empty((nb, 18), np.uint8)
    out[:, :2] = d16.astype(np.uint16).view(np.uint8).reshape(nb, 2)
    out[:, 2:] = (nib[:, :16] | (nib[:, 16:] << 4)).astype(np.uint8)
    return out.tobytes()


def pack_q4k_scales(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Eight 6-bit scales and mins into the 12-byte Q4_K header (ggml layout)."""
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = sc[j] & 63
        s[j + 4] = mn[j] & 63
    for j in range(4, 8):
        s[j + 4] = (sc[j] & 15) | ((mn[j] & 15) << 4)
        s[j - 4] |= (sc[j] >> 4) << 6
        s[j] |= (mn[j] >> 4) << 6
    return s


def q4_k_row(d16, dmin16, sc, mn, nib) -> bytes:
    """sc, mn: [nsb][8]; nib: [nsb][256] codes in element order."""
    nsb = len(d16)
    out = np.empty((nsb, 144), np.uint8)
    for b in range(nsb):
        out[b, 0:2] = np.array([d16[b]], np.uint16).view(np.uint8)
        out[b, 2:4] = np.array([dmin16[b]], np.uint16).view(np.uint8)
        out[b, 4:16] = pack_q4k_scales(np.asarray(sc[b]), np.asarray(mn[b]))
        n = np.asarray(nib[b]).reshape(8, 32)
        for pair in range(4):
            out[b, 16 + 32 * pair: 16 + 32 * (pair + 1)] = n[2 * pair] | (n[2 * pair + 1] << 4)
    return out.tobytes()


def q6_k_row(d16, sc, q6) -> bytes:
    """sc: [nsb][16] int8; q6: [nsb][256] values in [-32, 31], element order."""
    nsb = len(d16)
    out = np.zeros((nsb, 210), np.uint8)
    for b in range(nsb):
        u = (np.asarray(q6[b]) + 32).astype(np.uint8)
        ql = np.zeros(128, np.uint8)
        qh = np.zeros(64, np.uint8)
        for e in range(256):
            half, within = divmod(e, 128)
            part, l = divmod(within, 32)
            lo, hi = u[e] & 15, u[e] >> 4
            idx = half * 64 + l + (32 if part in (1, 3) else 0)
            ql[idx] |= lo if part < 2 else lo << 4
            qh[half * 32 + l] |= hi << (2 * part)
        out[b, :128] = ql
        out[b, 128:192] = qh
        out[b, 192:208] = np.asarray(sc[b], np.int8).view(np.uint8)
        out[b, 208:210] = np.array([d16[b]], np.uint16).view(np.uint8)
    return out.tobytes()


# ---- independent decoders (integer codes, scales) ---------------------------------

def decode_q4_k_codes(row: bytes, cols: int):
    """Per element: (q code, sub-block scale, sub-block min) from raw bytes."""
    nsb = cols // 256
    raw = np.frombuffer(row, np.uint8).reshape(nsb, 144)
    q = np.empty(cols, np.int64)
    scale = np.empty(cols, np.int64)
    mins = np.empty(cols, np.int64)
    for b in range(nsb):
        s = raw[b, 4:16].astype(np.int64)
        qs = raw[b, 16:]
        for j in range(8):
            if j < 4:
                sc, mn = s[j] & 63, s[j + 4] & 63
            else:
                sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4)
                mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4)
            byte = qs[(j // 2) * 32:(j // 2) * 32 + 32].astype(np.int64)
            codes = (byte >> 4) if j % 2 else (byte & 15)
            sl = slice(256 * b + 32 * j, 256 * b + 32 * j + 32)
            q[sl], scale[sl], mins[sl] = codes, sc, mn
    return q, scale, mins


def decode_q6_k(row: bytes, cols: int):
    """Per element: (q6 value in [-32,31], int8 scale)."""
    nsb = cols // 256
    raw = np.frombuffer(row, np.uint8).reshape(nsb, 210)
    q = np.empty(cols, np.int64)
    sc = np.empty(cols, np.int64)
    for b in range(nsb):
        ql, qh = raw[b, :128].astype(np.int64), raw[b, 128:192].astype(np.int64)
        s = raw[b, 192:208].view(np.int8).astype(np.int64)
        for e in range(256):
            half, within = divmod(e, 128)
            part, l = divmod(within, 32)
            byte = ql[half * 64 + l + (32 if part in (1, 3) else 0)]
            lo = (byte & 15) if part < 2 else (byte >> 4)
            hi = (qh[half * 32 + l] >> (2 * part)) & 3
            q[256 * b + e] = (lo | (hi << 4)) - 32
            sc[256 * b + e] = s[e // 16]
    return q, sc


def random_row(rng: np.random.Generator, ggml_type: int, rows: int, cols: int) -> bytes:
    """Random GGUF rows with realistic scales (for parity against the oracle)."""
    out = []
    for _ in range(rows):
        if ggml_type == 0:
            out.append(rng.normal(0, 0.1, cols).astype(np.float32).tobytes())
        elif ggml_type == 8:
            nb = cols // 32
            d = np.abs(rng.normal(0, 2e-3, nb)).astype(np.float16).view(np.uint16)
            out.append(q8_0_row(d, rng.integers(-127, 128, (nb, 32))))
        elif ggml_type == 2:
            nb = cols // 32
            d = np.abs(rng.normal(0, 2e-2, nb)).astype(np.float16).view(np.uint16)
            out.append(q4_0_row(d, rng.integers(0, 16, (nb, 32))))
        elif ggml_type == 12:
            nsb = cols // 256
            raw = rng.integers(0, 256, (nsb, 144)).astype(np.uint8)
            raw[:, 0:2] = np.abs(rng.normal(0, 1e-3, nsb)).astype(np.float16).view(np.uint8).reshape(nsb, 2)
            raw[:, 2:4] = np.abs(rng.normal(0, 1e-3, nsb)).astype(np.float16).view(np.uint8).reshape(nsb, 2)
            out.append(raw.tobytes())
        elif ggml_type == 14:
            nsb = cols // 256
            raw = rng.integers(0, 256, (nsb, 210)).astype(np.uint8)
            raw[:, 192:208] = rng.integers(-63, 64, (nsb, 16)).astype(np.int8).view(np.uint8)
            raw[:, 208:210] = np.abs(rng.normal(0, 1e-3, nsb)).astype(np.float16).view(np.uint8).reshape(nsb, 2)
            out.append(raw.tobytes())
        else:
            raise ValueError(ggml_type)
    return b"".join(out)


ROW_BYTES = {0: lambda c: 4 * c, 8: lambda c: c // 32 * 34, 2: lambda c: c // 32 * 18,
             12: lambda c: c // 256 * 144, 14: lambda c: c // 256 * 210}
