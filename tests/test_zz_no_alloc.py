"""dtl_symbol_ranges_static: the allocation-free symbol ranges.

Checks it through the C ABI against the oracle's symbol_range
(logits_to_symbol_range_*, det-coder cdf.rs:122-199 restated) and against
dtl_logits_to_symbol_range (the same ranges from host logits) on calls in a
row, each smaller than the one before, so a stale scratch from an earlier
call would show; the first calls sit exactly on the documented limit (8 rows,
vocab + tail = 2^18).  Then the limits, the error bits, and the call captured
into a HIP graph (the first test of the file, so that in a fresh process the
entry point's first-call symbol lookup runs under capture), replayed several
times with new logits and eager work in between.  Device buffers come from
the HIP runtime the library itself uses (plain hipMalloc through ctypes); the
entry point allocates nothing.
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
        self.rt.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
        self.rt.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
        self.rt.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p,
                                                C.c_size_t]
        self.rt.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
        self.rt.hipGraphExecDestroy.argtypes = [C.c_void_p]
        self.rt.hipGraphDestroy.argtypes = [C.c_void_p]
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


def _host_entry(logits, symbols, tail):
    from detllm_amd.coder import logits_to_symbol_range, logits_to_symbol_range_with_byte_escapes

    f = logits_to_symbol_range_with_byte_escapes if tail else logits_to_symbol_range
    return [(r.cum, r.freq, r.total) for r in (f(row, int(s)) for row, s in zip(logits, symbols))]


def _oracle(logits, symbols, tail):
    import detref

    return [tuple(int(v) for v in detref.symbol_range(row, int(s), tail)) for row, s in zip(logits, symbols)]


def _outputs(h, R):
    return h.alloc(8 * R), h.alloc(4 * R), h.alloc(8 * R), h.alloc(4)


def _read(h, R, dc, df, dt, db):
    bits = int(h.get(db, np.int32, 1)[0])
    got = list(zip(h.get(dc, np.uint64, R).tolist(), h.get(df, np.uint32, R).tolist(),
                   h.get(dt, np.uint64, R).tolist()))
    return bits, got


def _call(h, stream, logits, symbols, tail):
    R, V = logits.shape
    dl, ds = h.put(logits.astype(np.float32)), h.put(symbols.astype(np.uint32))
    dc, df, dt, db = _outputs(h, R)
    st = h.dtl.dtl_symbol_ranges_static(dl, R, V, ds, tail, dc, df, dt, db, stream)
    assert st == 0, st
    assert h.rt.hipStreamSynchronize(stream) == 0
    return _read(h, R, dc, df, dt, db)


def test_static_symbol_ranges_captured_in_a_graph():
    h = _Hip()
    stream = C.c_void_p()
    assert h.rt.hipStreamCreate(C.byref(stream)) == 0
    graph, exe = C.c_void_p(), C.c_void_p()
    try:
        rng = np.random.default_rng(11)
        R, V, tail = 5, 32000, 256
        logits = rng.normal(0, 3, (R, V)).astype(np.float32)
        symbols = rng.integers(0, V + tail, R).astype(np.uint32)
        dl, ds = h.put(logits), h.put(symbols)
        dc, df, dt, db = _outputs(h, R)
        print("static symbol ranges under graph capture", flush=True)
        assert h.rt.hipStreamBeginCapture(stream, 0) == 0  # global capture mode
        try:
            st = h.dtl.dtl_symbol_ranges_static(dl, R, V, ds, tail, dc, df, dt, db, stream)
        finally:
            end = h.rt.hipStreamEndCapture(stream, C.byref(graph))
        assert st == 0, st
        assert end == 0
        assert h.rt.hipGraphInstantiate(C.byref(exe), graph, None, None, 0) == 0
        for replay in range(4):
            # new inputs, and eager work of the entry point itself, between replays
            logits = rng.normal(0, 1 + replay, (R, V)).astype(np.float32)
            symbols = rng.integers(0, V + tail, R).astype(np.uint32)
            assert h.rt.hipMemcpy(dl, logits.ctypes.data, logits.nbytes, 1) == 0
            assert h.rt.hipMemcpy(ds, symbols.ctypes.data, symbols.nbytes, 1) == 0
            eager_bits, eager = _call(h, stream, logits[:2], symbols[:2], tail)
            print(f"graph replay {replay}", flush=True)
            assert h.rt.hipGraphLaunch(exe, stream) == 0
            assert h.rt.hipStreamSynchronize(stream) == 0
            bits, got = _read(h, R, dc, df, dt, db)
            assert bits == 0 and eager_bits == 0
            want = _oracle(logits, symbols, tail)
            assert got == want
            assert eager == want[:2]
    finally:
        if exe:
            h.rt.hipGraphExecDestroy(exe)
        if graph:
            h.rt.hipGraphDestroy(graph)
        h.rt.hipStreamDestroy(stream)
        h.close()


def test_static_symbol_ranges_match_oracle_and_host_entry_point():
    h = _Hip()
    stream = C.c_void_p()
    assert h.rt.hipStreamCreate(C.byref(stream)) == 0
    try:
        rng = np.random.default_rng(7)
        # the documented limit first (8 rows; vocab 2^18 takes the most
        # scratch, vocab + tail = 2^18 the most symbols), then smaller calls
        for R, V, tail in ((8, 1 << 18, 0), (8, (1 << 18) - 256, 256), (8, 151936, 256), (3, 49152, 0)):
            logits = rng.normal(0, 4, (R, V)).astype(np.float32)
            symbols = rng.integers(0, V + tail, R)
            symbols[0] = V + tail - 1
            print(f"static symbol ranges: {R} rows, vocab {V}, tail {tail}", flush=True)
            bits, got = _call(h, stream, logits, symbols, tail)
            assert bits == 0
            assert got == _oracle(logits, symbols, tail)
            assert got == _host_entry(logits, symbols, tail)
        # limits: rejected on the host before anything is enqueued
        dummy = h.alloc(64)
        st = h.dtl.dtl_symbol_ranges_static(dummy, 9, 1000, dummy, 0, dummy, dummy, dummy, dummy, stream)
        assert st == 45
        st = h.dtl.dtl_symbol_ranges_static(dummy, 1, (1 << 18) - 255, dummy, 256, dummy, dummy, dummy,
                                            dummy, stream)
        assert st == 24
        st = h.dtl.dtl_symbol_ranges_static(dummy, 1, (1 << 18) + 1, dummy, 0, dummy, dummy, dummy,
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
        assert bits == 0 and got == _oracle(logits, [3, 4], 0) == _host_entry(logits, [3, 4], 0)
    finally:
        h.rt.hipStreamDestroy(stream)
        h.close()
