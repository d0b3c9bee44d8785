"""dtl_symbol_ranges_static: the allocation-free symbol ranges.

Checks it through the C ABI against dtl_logits_to_symbol_range (the same
ranges from host logits, det-coder cdf.rs:122-199) on two calls in a row,
the second smaller than the first, so a stale scratch from the first call
would show; then its limits and its error bits.  Device buffers come from
the HIP runtime the library itself uses (plain hipMalloc through ctypes);
the entry point allocates nothing.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


class _Hip:
    def __init__(self):
        from detllm_amd._lib import lib  # loads libdetllm_amd.so and its HIP runtime

        self.dtl = lib
        self.rt = C.CDLL("libamdhip64.so.7")
        self.rt.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.rt.hipFree.argtypes = [C.c_void_p]
        self.rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.rt.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.rt.hipStreamDestroy.argtypes = [C.c_void_p]
        self.rt.hipStreamSynchronize.argtypes = [C.c_void_p]
        self.bufs = []

    def alloc(self, nbytes):
        p = C.c_void_p()
        assert self.rt.hipMalloc(C.byref(p), max(nbytes, 16)) == 0
        self.bufs.append(p)
        return p

    def put(self, arr):
        arr = np.ascontiguousarray(arr)
        p = self.alloc(arr.nbytes)
        assert self.rt.hipMemcpy(p, arr.ctypes.data, arr.nbytes, 1) == 0  # host to device
        return p

    def get(self, p, dtype, n):
        out = np.empty(n, dtype)
        assert self.rt.hipMemcpy(out.ctypes.data, p, out.nbytes, 2) == 0  # device to host
        return out

    def close(self):
        for p in self.bufs:
            self.rt.hipFree(p)


def _reference(logits, symbols, tail):
    from detllm_amd.coder import logits_to_symbol_range, logits_to_symbol_range_with_byte_escapes

    f = logits_to_symbol_range_with_byte_escapes if tail else logits_to_symbol_range
    return [(r.cum, r.freq, r.total) for r in (f(row, int(s)) for row, s in zip(logits, symbols))]


def _call(h, stream, logits, symbols, tail):
    R, V = logits.shape
    dl, ds = h.put(logits.astype(np.float32)), h.put(symbols.astype(np.uint32))
    dc, df, dt, db = h.alloc(8 * R), h.alloc(4 * R), h.alloc(8 * R), h.alloc(4)
    st = h.dtl.dtl_symbol_ranges_static(dl, R, V, ds, tail, dc, df, dt, db, stream)
    assert st == 0, st
    assert h.rt.hipStreamSynchronize(stream) == 0
    bits = int(h.get(db, np.int32, 1)[0])
    got = list(zip(h.get(dc, np.uint64, R).tolist(), h.get(df, np.uint32, R).tolist(),
                   h.get(dt, np.uint64, R).tolist()))
    return bits, got


def test_static_symbol_ranges_match_host_entry_point():
    h = _Hip()
    stream = C.c_void_p()
    assert h.rt.hipStreamCreate(C.byref(stream)) == 0
    try:
        rng = np.random.default_rng(7)
        # first call: the largest size the scratch takes; second: smaller
        for R, V, tail in ((8, 151936, 256), (3, 49152, 0)):
            logits = rng.normal(0, 4, (R, V)).astype(np.float32)
            symbols = rng.integers(0, V + tail, R)
            symbols[0] = V + tail - 1 if tail else V - 1
            print(f"static symbol ranges: {R} rows, vocab {V}, tail {tail}", flush=True)
            bits, got = _call(h, stream, logits, symbols, tail)
            assert bits == 0
            assert got == _reference(logits, symbols, tail)
        # limits: rejected on the host before anything is enqueued
        dummy = h.alloc(64)
        st = h.dtl.dtl_symbol_ranges_static(dummy, 9, 1000, dummy, 0, dummy, dummy, dummy, dummy, stream)
        assert st == 45
        st = h.dtl.dtl_symbol_ranges_static(dummy, 1, (1 << 18) - 255, dummy, 256, dummy, dummy, dummy,
                                            dummy, stream)
        assert st == 24
        # error bits: a symbol past vocab + tail, then a non-finite logit
        logits = rng.normal(0, 1, (2, 1000)).astype(np.float32)
        bits, _ = _call(h, stream, logits, np.array([3, 1000]), 0)
        assert h.dtl.dtl_status_from_bits(bits) == 23
        logits[1, 17] = np.inf
        bits, _ = _call(h, stream, logits, np.array([3, 4]), 0)
        assert h.dtl.dtl_status_from_bits(bits) == 22
        # and a clean call after the failures clears the word
        logits[1, 17] = 0.5
        bits, got = _call(h, stream, logits, np.array([3, 4]), 0)
        assert bits == 0 and got == _reference(logits, [3, 4], 0)
    finally:
        h.rt.hipStreamDestroy(stream)
        h.close()
