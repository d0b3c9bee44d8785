"""Full-depth, full-length parity of the benchmark workloads.

Each workload's whole token stream runs through the HIP path and is compared
with the goldens the oracle wrote in the build container
(tests/golden/make_goldens.py): the SHA-256 of all positions' logits (the
reference's logits hash, det-model lib.rs:1402-1465), a digest per position
(so a mismatch names its first position), qwen05's next-token symbol ranges
(det-coder cdf.rs:130-199) and the windowed codec payload of a 6 KiB prefix
of the end-to-end byte stream (det-cli main.rs:521-551).  The reference's
invariance tests (lib.rs:3727-3796) are followed by running every stream
through more than one path: the captured single-position graph, the chunked
forward and the pipelined encode (several chunks in flight).
"""
import hashlib
import json
import struct

import numpy as np
import pytest

from conftest import GOLDEN
from detllm_amd import synth

pytestmark = pytest.mark.gpu


def _golden(name):
    f = GOLDEN / f"workload_{name}.json"
    if not f.exists():  # written by tests/golden/make_goldens.py (CPU-hours for the largest)
        pytest.skip(f"{f.name} not generated: python tests/golden/make_goldens.py {name}")
    return json.loads(f.read_text())


def _check_rows(rows, gold, path):
    """rows: per-position logits in order; compares digests, then the hash."""
    h = hashlib.sha256()
    for i, r in enumerate(rows):
        b = np.ascontiguousarray(r, np.float32).tobytes()
        h.update(b)
        d = hashlib.sha256(b).hexdigest()[:16]
        assert d == gold["position_digests"][i], f"{path}: first mismatch at position {i}"
    assert h.hexdigest() == gold["logits_sha256"], path


def _setup(name):
    from detllm_amd.model import F32Llama

    gold = _golden(name)
    w = synth.WORKLOADS[gold["workload"]]
    layers = gold["layers"] if gold["layers"] != w.layers else None
    g = synth.build_model(w, layers)
    assert hashlib.sha256(g).hexdigest() == gold["model_sha256"]
    toks = [int(t) for t in synth.tokens(w, gold["positions"])]
    return gold, w, F32Llama.from_gguf(g), toks


def _decode_rows(m, toks, n_ctx):
    from detllm_amd.model import Session

    rows = []
    with Session(m, n_ctx, 1) as s:
        for p, t in enumerate(toks):
            rows.append(s.forward_one(t, p))
    return rows


def _ranges_hash(cum, freq, total):
    h = hashlib.sha256()
    for c, f, t in zip(cum, freq, total):
        h.update(struct.pack("<QIQ", int(c), int(f), int(t)))
    return h.hexdigest()


@pytest.mark.parametrize("name", ["smollm2", "smollm2_l1"])
def test_smollm2_decode_and_chunks_match_golden(name):
    gold, w, m, toks = _setup(name)
    print(f"{name}: {gold['layers']} layers, {len(toks)} positions, single-token decode", flush=True)
    _check_rows(_decode_rows(m, toks, len(toks)), gold, "decode")
    print(f"{name}: chunks of 64", flush=True)
    assert m.logits_hash_for_tokens_chunked(toks, 64).hex() == gold["logits_sha256"]


def test_qwen05_decode_ranges_and_pipeline_match_golden():
    from detllm_amd.model import Session

    gold, w, m, toks = _setup("qwen05")
    n = len(toks)
    nxt = toks[1:] + [0]
    print(f"qwen05: 24 layers, {n} positions: decode with a symbol range each", flush=True)
    h = hashlib.sha256()
    cum, freq, total = [], [], []
    with Session(m, 2048, 1) as s:
        for p, t in enumerate(toks):
            row = s.forward_one(t, p)
            b = row.tobytes()
            h.update(b)
            assert hashlib.sha256(b).hexdigest()[:16] == gold["position_digests"][p], f"position {p}"
            c, f, tt = s.symbol_ranges([nxt[p]], 0, 256)
            cum.append(c[0]), freq.append(f[0]), total.append(tt[0])
    assert h.hexdigest() == gold["logits_sha256"]
    assert _ranges_hash(cum, freq, total) == gold["next_token_ranges_sha256"]
    print("qwen05: pipelined encode, chunks of 64", flush=True)
    with Session(m, 2048, 64) as s:
        c, f, tt = s.forward_ranges(toks, 0, list(range(n)), nxt, 256)
    assert _ranges_hash(c, f, tt) == gold["next_token_ranges_sha256"]
    print("qwen05: chunks of 64 (logits hash)", flush=True)
    assert m.logits_hash_for_tokens_chunked(toks, 64).hex() == gold["logits_sha256"]


def test_tinyllama_encode_and_decode_match_golden(monkeypatch):
    """The benchmark's own workload end to end: the timed encode
    (dtl_forward_ranges, chunks of 64 in flight on 4 lanes as the bench
    runs it, and on 3) must code every one of the 2048 next tokens with the
    reference's (cum, freq, total), as det-cli's encode loop does
    (main.rs:521-551; cdf.rs:130-199).  Expected ranges: the golden's
    (the oracle's logits and symbol_range in the build container), and the
    oracle's symbol_range over this run's chunked logits once every row's
    digest equals the golden's."""
    import detref
    from detllm_amd.model import Session

    gold, w, m, toks = _setup("tinyllama")
    n = len(toks)
    nxt = toks[1:] + [0]
    print(f"tinyllama: 22 layers, {n} positions, chunks of 64", flush=True)
    want = []

    def visit(r):
        i = len(want)
        b = np.ascontiguousarray(r, np.float32).tobytes()
        assert hashlib.sha256(b).hexdigest()[:16] == gold["position_digests"][i], f"chunk 64: position {i}"
        want.append(tuple(int(v) for v in detref.symbol_range(r, nxt[i], 256)))

    assert m.logits_hash_for_tokens_chunked(toks, 64).hex() == gold["logits_sha256"]
    m.visit_logits_for_tokens_chunked(toks, 64, visit)
    assert len(want) == n
    if "next_token_ranges" in gold:
        assert [tuple(t) for t in gold["next_token_ranges"]] == want
    if "next_token_ranges_sha256" in gold:
        assert _ranges_hash(*zip(*want)) == gold["next_token_ranges_sha256"]
    for lanes in ("4", "3"):
        monkeypatch.setenv("DETLLM_LANES", lanes)  # read when the session is created
        print(f"tinyllama: pipelined encode on {lanes} lanes", flush=True)
        with Session(m, 2048, 64) as s:
            c, f, tt = s.forward_ranges(toks, 0, list(range(n)), nxt, 256)
        got = [(int(a), int(b), int(d)) for a, b, d in zip(c, f, tt)]
        bad = [i for i in range(n) if got[i] != want[i]]
        assert not bad, f"{lanes} lanes: {len(bad)} rows differ, first {bad[0]}"
    monkeypatch.delenv("DETLLM_LANES")
    print("tinyllama: single-token decode", flush=True)
    _check_rows(_decode_rows(m, toks, 2048), gold, "decode")


def test_codec_prefix_payload_matches_golden():
    from detllm_amd.codec import LoadedModel, compress, decompress
    from detllm_amd.coder import DtlzHeader

    gold = _golden("codec")
    w = synth.WORKLOADS[gold["workload"]]
    lm = LoadedModel.load(synth.build_model(w))
    data = synth.markov_bytes(gold["markov_seed"], gold["bytes"])
    print(f"codec: {len(data)} bytes, qwen05 24 layers, n_ctx {gold['n_ctx']}", flush=True)
    out = compress(lm, data, gold["n_ctx"])
    h = DtlzHeader.decode(out)
    assert (h.n_ctx, h.overlap, h.orig_len) == (gold["n_ctx"], gold["overlap"], len(data))
    assert len(out) - 56 == gold["payload_len"]
    assert hashlib.sha256(out[56:]).hexdigest() == gold["payload_sha256"]
    print("codec: decompress", flush=True)
    assert decompress(lm, out) == data
