"""Full decoder forward on the GPU: logits bit-identical to the reference.

The tiny-f32 / tiny-qmix fixtures are checked against the reference's own
committed SHA-256 values; the SmolLM2-, Qwen2.5- and TinyLlama-shaped synthetic models against the
oracle at full width (a few positions, truncated depth where noted) and
through size-independent properties (chunk invariance, repeatability).
"""
import numpy as np
import pytest

import detref
from conftest import GOLDEN

pytestmark = pytest.mark.gpu


def _model(data):
    from detllm_amd.model import F32Llama

    return F32Llama.from_gguf(data)


def _fixture_tokens():
    return [int(t) for t in (GOLDEN / "tiny.tokens.txt").read_text().strip().split(",")]


@pytest.mark.parametrize("name", ["tiny-f32", "tiny-qmix"])
@pytest.mark.parametrize("chunk", [1, 2, 3, 6])
def test_fixture_hash_matches_reference_golden(name, chunk):
    m = _model((GOLDEN / f"{name}.gguf").read_bytes())
    want = (GOLDEN / f"{name}.logits.sha256").read_text().strip()
    assert m.logits_hash_for_tokens_chunked(_fixture_tokens(), chunk).hex() == want


def _compare_with_oracle(data, tokens, chunk):
    m = _model(data)
    ref = detref.Model(data).logits(tokens)
    got = []
    m.visit_logits_for_tokens_chunked(tokens, chunk, lambda row: got.append(row.copy()))
    got = np.stack(got)
    assert got.shape == ref.shape
    bad = np.nonzero(got.view(np.uint32) != ref.view(np.uint32))
    assert bad[0].size == 0, f"first mismatch at position {bad[0][:1]}, index {bad[1][:1]}"
    return m, got


def test_tiny_workload_matches_oracle_all_chunks():
    from detllm_amd import synth

    w = synth.WORKLOADS["tiny"]
    data = synth.build_model(w)
    toks = synth.tokens(w)
    m, got = _compare_with_oracle(data, toks, w.chunk)
    ref_hash = detref.Model(data).logits_hash(toks)
    for chunk in (1, 2, 3, 8):
        assert m.logits_hash_for_tokens_chunked(toks, chunk) == ref_hash


@pytest.mark.parametrize("name,layers,n_tok,chunk", [
    ("smollm2", 4, 5, 2),
    ("qwen05", 3, 5, 3),
    ("tinyllama", 2, 4, 4),
    # chunks of >= 16 positions run the token-parallel kernels (and the fused
    # gate/up/SwiGLU pass for Q4_K), including a partial final chunk
    ("smollm2", 2, 40, 32),
    ("qwen05", 1, 21, 21),
    ("tinyllama", 1, 70, 64),
    ("tinyllama", 1, 37, 37),   # Q4_K GEMM tiles with positions past the chunk
])
def test_baseline_shapes_match_oracle(name, layers, n_tok, chunk):
    from detllm_amd import synth

    w = synth.WORKLOADS[name]
    data = synth.build_model(w, layers=layers)
    _compare_with_oracle(data, synth.tokens(w, n_tok), chunk)


@pytest.mark.parametrize("name,chunk", [("qwen05", 1), ("qwen05", 8), ("smollm2", 5)])
@pytest.mark.parametrize("fused", [True, False])
def test_decode_gemv_fusion_matches_oracle(monkeypatch, name, chunk, fused):
    # Up to eight positions the Q8_0 layers run the fused decode GEMVs
    # (rmsnorm / quantisation in the GEMV prologue, q/k/v in one launch,
    # gate/up finishing as swiglu); both that and the separate launches must
    # give the reference bits.
    from detllm_amd import synth

    if not fused:
        monkeypatch.setenv("DETLLM_NO_FUSED_DECODE", "1")
    monkeypatch.setenv("DETLLM_NO_GRAPH", "1")
    w = synth.WORKLOADS[name]
    _compare_with_oracle(synth.build_model(w, layers=2), synth.tokens(w, 10), chunk)


def test_fused_decode_mixed_q8_0_q4_0_fixture():
    # tiny-qmix mixes Q8_0 and Q4_0 within q/k/v and gate/up: each matrix
    # gets its own fused launch; the reference's golden hash must hold.
    m = _model((GOLDEN / "tiny-qmix.gguf").read_bytes())
    want = (GOLDEN / "tiny-qmix.logits.sha256").read_text().strip()
    assert m.logits_hash_for_tokens_chunked(_fixture_tokens(), 1).hex() == want


@pytest.mark.parametrize("env", ["DETLLM_NO_F32_MIRROR", "DETLLM_NO_Q6K_PLANES"])
def test_packed_chunk_paths_match_oracle(monkeypatch, env):
    # Without the encode copies (Q4_K f32 weights, Q6_K matrix-core planes)
    # the chunked GEMMs decode the packed superblocks themselves; every path
    # must give the reference bits.
    from detllm_amd import synth

    monkeypatch.setenv(env, "1")
    w = synth.WORKLOADS["tinyllama"]
    _compare_with_oracle(synth.build_model(w, layers=1), synth.tokens(w, 40), 40)


@pytest.mark.parametrize("name", ["qwen05", "tinyllama"])
def test_single_position_graph_replay_matches_oracle(monkeypatch, name):
    # One-position forwards replay a captured graph (the position reaches the
    # kernels through device memory); every replay, a reset session and the
    # eager launches must give the reference bits.
    from detllm_amd import synth

    w = synth.WORKLOADS[name]
    data = synth.build_model(w, layers=1)
    toks = [int(t) for t in synth.tokens(w, 12)]
    ref = detref.Model(data).logits(toks)
    m = _model(data)
    with m.forward_workspace(16, 1) as s:
        for rep in range(2):
            for p, tok in enumerate(toks):
                got = s.forward_one(tok, p)
                assert np.array_equal(got.view(np.uint32), ref[p].view(np.uint32)), (rep, p)
            s.reset()
    monkeypatch.setenv("DETLLM_NO_GRAPH", "1")
    with m.forward_workspace(16, 1) as s:
        for p, tok in enumerate(toks[:4]):
            assert np.array_equal(s.forward_one(tok, p).view(np.uint32), ref[p].view(np.uint32))


def test_repeat_runs_are_bitwise_identical():
    from detllm_amd import synth

    w = synth.WORKLOADS["smollm2"]
    m = _model(synth.build_model(w, layers=2))
    toks = synth.tokens(w, 16)
    hashes = {m.logits_hash_for_tokens_chunked(toks, c) for c in (1, 5, 16, 16)}
    assert len(hashes) == 1


def test_session_errors_mirror_reference_shape_checks():
    from detllm_amd._lib import DetllmError

    m = _model((GOLDEN / "tiny-f32.gguf").read_bytes())
    with m.forward_workspace(4, 2) as s:
        with pytest.raises(DetllmError) as e:
            s.forward_chunk([0, 1, 2], 0)  # more positions than max_chunk
        assert e.value.status == 1
        with pytest.raises(DetllmError) as e:
            s.forward_one(10_000, 0)      # token outside the vocabulary
        assert e.value.status == 1
        with pytest.raises(DetllmError) as e:
            s.forward_one(0, 4)           # position outside the window
        assert e.value.status == 1


def test_cdf_on_device_logits_matches_oracle():
    from detllm_amd import synth

    w = synth.WORKLOADS["smollm2"]
    data = synth.build_model(w, layers=2)
    m = _model(data)
    toks = synth.tokens(w, 6)
    with m.forward_workspace(8, 6) as s:
        logits = s.forward_chunk(toks, 0, want_logits=True)
        syms = [int(t) for t in synth.tokens(w, 7)[1:7]]
        for tail in (0, 256):
            cum, freq, total = s.symbol_ranges(syms, 0, tail)
            for i in range(6):
                assert (int(cum[i]), int(freq[i]), int(total[i])) == detref.symbol_range(logits[i], syms[i], tail)
            f, c, t = s.cdf(2, tail)
            rf, rc, rt = detref.logits_to_cdf(logits[2], tail)
            assert np.array_equal(f, rf) and np.array_equal(c, rc) and t == rt
            # values inside, at the start and at the end of symbols, including the
            # 4096-symbol work-block edges, the last vocab symbol and the escapes
            values = {0, rt - 1, int(rc[100]), int(rc[100]) + int(rf[100]) - 1}
            for sym in (4095, 4096, 4097, 8191, 8192, len(rf) - tail - 1):
                values |= {int(rc[sym]), int(rc[sym]) + int(rf[sym]) - 1}
            if tail:
                values |= {int(rc[len(rf) - tail]), int(rc[len(rf) - 1])}
            for value in sorted(values):
                assert s.decoder_lookup(value, 2, tail) == detref.decoder_lookup(logits[2], value, tail), value
            assert s.decoder_total(2, tail) == rt


@pytest.mark.parametrize("tail", [0, 256])
def test_fused_decode_steps_match_oracle_ranges(tail):
    """dtl_forward_decode / dtl_decoder_decode against a payload coded with
    the oracle's symbol ranges: the symbols and, after every step, the range
    decoder's state equal a host decoder fed the oracle's ranges.  The
    symbols sit on the 4096-symbol work-block edges, at the vocabulary's end,
    on the most likely token and (tail 256) on byte escapes, which are not
    forwarded, so the next decode reads the same row again."""
    from detllm_amd import coder, synth
    from detllm_amd._lib import DetllmError

    w = synth.WORKLOADS["smollm2"]
    data = synth.build_model(w, layers=2)
    m = _model(data)
    V = w.vocab
    t0 = int(synth.tokens(w, 1)[0])
    esc = (V + 3, V + 255) if tail else (17, 30000)
    with m.forward_workspace(16, 1) as s:
        lg = s.forward_one(t0, 0)
        syms = [4095, 4096, V - 1, esc[0], None, 8192, 0, esc[1], 12345, 4097]  # None: the argmax
        enc, ranges, pos = coder.RangeEncoder(), [], 1
        for i, want in enumerate(syms):
            if want is None:
                want = syms[i] = int(np.argmax(lg))
            r = detref.symbol_range(lg, want, tail)
            enc.encode(*r)
            ranges.append(r)
            if want < V:
                lg = s.forward_one(want, pos)
                pos += 1
        payload = enc.finish()

    def state(d):
        st = d.snapshot()
        return st.low, st.range, st.code, st.pos

    with m.forward_workspace(16, 1) as s:
        dec, host = coder.RangeDecoder(payload), coder.RangeDecoder(payload)
        s.forward_one(t0, 0, want_logits=False)
        pos, pend = 1, None
        for want, (cum, freq, total) in zip(syms, ranges):
            if pend is None:
                got = s.decode_symbol(dec, 0, tail)
            else:
                got = s.forward_decode(pend, pos, dec, tail)
                pos += 1
            v = host.decode_freq(total)
            assert cum <= v < cum + freq
            host.advance(cum, freq, total)
            assert got == want
            assert state(dec) == state(host)
            pend = got if got < V else None
        # a decoder between decode_freq and advance, a token outside the vocabulary
        host.decode_freq(ranges[0][2])
        with pytest.raises(DetllmError) as e:
            s.decode_symbol(host, 0, tail)
        assert e.value.status == 30
        with pytest.raises(DetllmError) as e:
            s.forward_decode(V, pos, dec, tail)
        assert e.value.status == 1


@pytest.mark.parametrize("V", [4, 256, 32000, 151936])
def test_standalone_cdf_kernel_matches_oracle(V):
    from detllm_amd import coder

    rng = np.random.default_rng(V)
    lg = rng.normal(0, 4, V).astype(np.float32)
    if V == 4:
        lg[:] = 0.0
    else:
        lg[:11] = [0.0, -1.0, 3.25, 3.25, -88.5, np.float32(2 ** -149), -12.0, 0.5, -0.25, 2.0, -1000.0]
    for tail in (0, 256):
        got = coder._cdf(lg, tail)
        rf, rc, rt = detref.logits_to_cdf(lg, tail)
        assert np.array_equal(got.freq, rf) and np.array_equal(got.cum, rc) and got.total == rt
        for s in (0, V // 2, V - 1, V + tail - 1):
            r = coder._range(lg, s, tail)
            assert (r.cum, r.freq, r.total) == detref.symbol_range(lg, s, tail)


@pytest.mark.parametrize("graph", [True, False])
def test_decode_attention_regimes_match_oracle(monkeypatch, graph):
    """Single-position forwards in a 4096-position window (1-layer SmolLM2
    shape) through every decode attention they can take, bit for bit against
    the oracle.

    graph: positions below 512 replay the graph whose attention is one launch
    (k_attn_fused); from 512 on, the graph sized for the whole window, whose
    attention runs one workgroup per (head, position) (k_attention_dec).
    eager (DETLLM_NO_GRAPH=1, the path under profiling or after a failed
    capture): the launch is sized by the row: k_attn_fused up to 512 keys,
    the split pair (k_attn_split_scores + k_attn_split_pv) up to 2048,
    k_attention_dec beyond; the positions between are forwarded in chunks of
    64 (chunk attention)."""
    import dataclasses

    from detllm_amd import synth

    if not graph:
        monkeypatch.setenv("DETLLM_NO_GRAPH", "1")
    w = dataclasses.replace(synth.WORKLOADS["smollm2"], ctx=4096)
    data = synth.build_model(w, layers=1)
    if graph:
        singles = list(range(524))
        n = 524
    else:
        singles = [0, 1, 2, 3, 600, 601, 602, 603, 2048, 2049, 2050, 2051, 2052, 2053]
        n = 2054
    toks = [int(t) for t in synth.tokens(w, n)]
    print(f"oracle logits of {n} positions", flush=True)
    ref = detref.Model(data).logits(toks)
    m = _model(data)
    with m.forward_workspace(4096, 64) as s:
        p = 0
        while p < n:
            if p in singles:
                if p in (0, 512, 600, 2048):
                    print(f"{'graph' if graph else 'eager'} single-position forwards from {p}", flush=True)
                got = s.forward_one(toks[p], p)
                assert np.array_equal(got.view(np.uint32), ref[p].view(np.uint32)), p
                p += 1
            else:
                end = min(n, p + 64, min((q for q in singles if q > p), default=n))
                lg = s.forward_chunk(toks[p:end], p, want_logits=True)
                assert np.array_equal(lg[-1].view(np.uint32), ref[end - 1].view(np.uint32)), end - 1
                p = end
