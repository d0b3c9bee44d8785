"""dtl_forward_ranges: the codec window's forwards and symbol ranges with several
chunks in flight on separate streams.  Every range must equal the oracle's
(det-coder logits_to_symbol_range over det-model logits) and the
chunk-at-a-time path's, whatever the chunk split, the final chunk's size
(the decode-attention path below five positions) or the start position.
"""
import dataclasses

import numpy as np
import pytest

import detref

pytestmark = pytest.mark.gpu


def _rows_symbols(n, vocab, tail, seed):
    """Rows 0..n-1 in order, some repeated (byte escapes share the logits of
    the last token) and some skipped; symbols over the whole alphabet."""
    rng = np.random.default_rng(seed)
    rows = []
    for r in range(n):
        k = int(rng.integers(0, 3))  # 0, 1 or 2 symbols coded against row r
        rows += [r] * k
    rows = np.array(rows, np.uint32)
    syms = rng.integers(0, vocab + tail, rows.size).astype(np.uint32)
    return rows, syms


def _oracle_ranges(data, tokens, pos0, rows, syms, tail):
    logits = detref.Model(data).logits(tokens)
    return [detref.symbol_range(logits[pos0 + int(r)], int(s), tail) for r, s in zip(rows, syms)]


@pytest.mark.parametrize("n,chunk,pos0", [(17, 3, 0), (17, 4, 5), (9, 8, 0), (3, 1, 2)])
@pytest.mark.parametrize("tail", [0, 256])
def test_forward_ranges_matches_oracle(n, chunk, pos0, tail):
    from detllm_amd import synth
    from detllm_amd.model import F32Llama

    # the tiny all-F32 shape with room for 22 positions
    w = dataclasses.replace(synth.WORKLOADS["tiny"], ctx=32)
    data = synth.build_model(w)
    toks = synth.tokens(w, pos0 + n)
    m = F32Llama.from_gguf(data)
    rows, syms = _rows_symbols(n, m.vocab, tail, seed=n * 31 + chunk)
    print(f"forward_ranges tiny n={n} chunk={chunk} pos0={pos0} tail={tail}", flush=True)
    with m.forward_workspace(pos0 + n, chunk) as s:
        for p in range(0, pos0, chunk):
            s.forward_chunk(toks[p:min(p + chunk, pos0)], p)
        cum, freq, total = s.forward_ranges(toks[pos0:], pos0, rows, syms, tail)
    got = [(int(c), int(f), int(t)) for c, f, t in zip(cum, freq, total)]
    assert got == _oracle_ranges(data, toks, pos0, rows, syms, tail)


@pytest.mark.parametrize("name,layers,n,chunk,lanes", [
    ("tinyllama", 2, 194, 64, None),  # final chunk of 2: decode attention with its own K/V store
    ("tinyllama", 1, 197, 64, None),  # final chunk of 5: chunked attention
    ("qwen05", 2, 70, 16, None),      # Q8_0 with bias
    ("qwen05", 1, 90, 16, "4"),       # four chunks in flight, whatever the queue count
    ("qwen05", 1, 90, 16, "1"),
])
def test_forward_ranges_equals_chunk_at_a_time(monkeypatch, name, layers, n, chunk, lanes):
    from detllm_amd import synth
    from detllm_amd.model import F32Llama

    if lanes:
        monkeypatch.setenv("DETLLM_LANES", lanes)  # read when the session is created

    w = synth.WORKLOADS[name]
    data = synth.build_model(w, layers=layers)
    toks = synth.tokens(w, n)
    m = F32Llama.from_gguf(data)
    tail = 256
    rows, syms = _rows_symbols(n, m.vocab, tail, seed=n)
    print(f"forward_ranges {name} layers={layers} n={n} chunk={chunk} lanes={lanes}", flush=True)
    with m.forward_workspace(n, chunk) as s:
        cum, freq, total = s.forward_ranges(toks, 0, rows, syms, tail)
        again = s.forward_ranges(toks, 0, rows, syms, tail)
        want = [], [], []
        for p in range(0, n, chunk):
            T = min(chunk, n - p)
            s.forward_chunk(toks[p:p + T], p)
            sel = (rows >= p) & (rows < p + T)
            if sel.any():
                for dst, src in zip(want, s.symbol_ranges_rows(rows[sel] - p, syms[sel], tail)):
                    dst.append(src)
    for got, rep, ref in zip((cum, freq, total), again, want):
        ref = np.concatenate(ref)
        assert np.array_equal(got, ref)
        assert np.array_equal(rep, got)
    # spot-check a few rows against the oracle at full width
    if name == "qwen05":
        pick = [0, rows.size // 2, rows.size - 1]
        ref = _oracle_ranges(data, toks, 0, rows[pick], syms[pick], tail)
        assert [(int(cum[i]), int(freq[i]), int(total[i])) for i in pick] == ref


def test_forward_ranges_errors():
    from detllm_amd import synth
    from detllm_amd._lib import DetllmError
    from detllm_amd.model import F32Llama

    w = synth.WORKLOADS["tiny"]
    m = F32Llama.from_gguf(synth.build_model(w))
    toks = synth.tokens(w, 6)
    with m.forward_workspace(8, 3) as s:
        with pytest.raises(DetllmError) as e:       # rows must not decrease
            s.forward_ranges(toks, 0, [2, 1], [0, 0], 0)
        assert e.value.status == 1
        with pytest.raises(DetllmError) as e:       # row past the tokens
            s.forward_ranges(toks, 0, [6], [0], 0)
        assert e.value.status == 1
        with pytest.raises(DetllmError) as e:       # symbol outside vocab + tail
            s.forward_ranges(toks, 0, [0], [m.vocab], 0)
        assert e.value.status == 23
        with pytest.raises(DetllmError) as e:       # past n_ctx
            s.forward_ranges(toks, 4, [0], [0], 0)
        assert e.value.status == 1
        # the session still works afterwards, on its first lane
        cum, freq, total = s.forward_ranges(toks, 0, [0, 5], [1, 2], 0)
        logits = s.forward_chunk(toks[:3], 0, want_logits=True)
        assert logits.shape == (3, m.vocab)
