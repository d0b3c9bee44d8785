"""DET-4 on the device: non-finite values are errors, never results.

Follows det-model's checks (ensure_finite at load, lib.rs:1140-1160 and the
read_*_matrix scale checks 1812-1953; gemv / rmsnorm / residual / bias
results, lib.rs:237-242, 282-284, 2053-2073, 1967-1998; the kernel tests
public_kernels_reject_nonfinite_inputs, 2481-2523) and det-coder's
NonFiniteLogit (cdf.rs:65, 156, 215).  Every case is planted on the host in
the GGUF bytes or in host logits; the kernels run to completion and report
through the sticky error flag, so nothing faults.  The oracle must return the
same status for each model.
"""
import numpy as np
import pytest

import detref
from detllm_amd import synth

pytestmark = pytest.mark.gpu

NON_FINITE = 2
CDF_NON_FINITE_LOGIT = 22


def _edit(name, fn):
    def e(t):
        if t.name == name:
            t.data = fn(bytearray(t.data))
    return e


def _f32_set(idx, v):
    def f(b):
        a = np.frombuffer(bytes(b), np.float32).copy()
        a[idx] = v
        return a.tobytes()
    return f


def _f32_scale(k):
    def f(b):
        return (np.frombuffer(bytes(b), np.float32) * np.float32(k)).astype(np.float32).tobytes()
    return f


def _f32_fill(v):
    def f(b):
        return np.full(len(b) // 4, v, np.float32).tobytes()
    return f


def _f16_at(off, bits):
    def f(b):
        b[off:off + 2] = bits.to_bytes(2, "little")
        return bytes(b)
    return f


def _status(fn):
    from detllm_amd._lib import DetllmError

    try:
        fn()
    except DetllmError as e:
        return e.status
    return 0


def _oracle_status(fn):
    try:
        fn()
    except detref.OracleError as e:
        return e.status
    return 0


W = synth.WORKLOADS

LOAD_CASES = {
    "f32 weight NaN": (W["tiny"], None, _edit("blk.0.attn_q.weight", _f32_set(5, np.nan))),
    "f32 norm +inf": (W["tiny"], None, _edit("blk.1.ffn_norm.weight", _f32_set(3, np.inf))),
    "q8_0 scale +inf": (W["smollm2"], 1, _edit("blk.0.ffn_up.weight", _f16_at(34 * 7, 0x7C00))),
    "q8_0 embedding scale NaN": (W["smollm2"], 1, _edit("token_embd.weight", _f16_at(34 * 3, 0x7E00))),
    "q4_k d +inf": (W["tinyllama"], 1, _edit("blk.0.attn_q.weight", _f16_at(144 * 2, 0x7C00))),
    "q4_k dmin NaN": (W["tinyllama"], 1, _edit("blk.0.ffn_gate.weight", _f16_at(144 * 2 + 2, 0x7E00))),
    "q6_k d +inf": (W["tinyllama"], 1, _edit("blk.0.attn_v.weight", _f16_at(210 * 2 + 208, 0x7C00))),
    "qkv bias NaN": (W["qwen05"], 1, _edit("blk.0.attn_k.bias", _f32_set(7, np.nan))),
}


@pytest.mark.parametrize("case", list(LOAD_CASES))
def test_load_rejects_non_finite_weights(case):
    from detllm_amd.model import F32Llama

    w, layers, edit = LOAD_CASES[case]
    g = synth.build_model(w, layers, edit)
    print(f"load {case}", flush=True)
    assert _oracle_status(lambda: detref.Model(g)) == NON_FINITE
    assert _status(lambda: F32Llama.from_gguf(g)) == NON_FINITE


FORWARD_CASES = {
    # the output projection's dot overflows (F32 GEMV result check)
    "f32 logits overflow": (W["tiny"], None, _edit("output.weight", _f32_fill(3e38))),
    # normed activations of 1e37 overflow the q/k/v block terms (Q8_0)
    "q8_0 gemv overflow": (W["smollm2"], 1, _edit("blk.0.attn_norm.weight", _f32_scale(1e37))),
    # rmsnorm's own output overflows (Q4_K layers: attention and FFN norms)
    "q4_k attn rmsnorm overflow": (W["tinyllama"], 1, _edit("blk.0.attn_norm.weight", _f32_scale(3e38))),
    "q4_k ffn rmsnorm overflow": (W["tinyllama"], 1, _edit("blk.0.ffn_norm.weight", _f32_scale(3e38))),
    "qwen2 q8_0 gemv overflow": (W["qwen05"], 1, _edit("blk.0.ffn_norm.weight", _f32_scale(1e37))),
}


@pytest.mark.parametrize("case", list(FORWARD_CASES))
def test_forward_overflow_returns_non_finite(case):
    from detllm_amd.model import F32Llama, Session

    w, layers, edit = FORWARD_CASES[case]
    g = synth.build_model(w, layers, edit)
    toks = [int(t) for t in synth.tokens(w, 20)]
    assert _oracle_status(lambda: detref.Model(g).logits(toks[:3])) == NON_FINITE
    m = F32Llama.from_gguf(g)
    n = min(16, w.ctx)  # the tiny model's context is 8
    print(f"forward {case}: single-token (graph) and chunk paths", flush=True)
    with Session(m, n, n) as s:
        assert _status(lambda: s.forward_one(toks[0], 0)) == NON_FINITE
        # a session that reported the error still serves later calls
        assert _status(lambda: s.forward_one(toks[1], 1)) == NON_FINITE
        # the decode step (forward and CDF in one wait) reports the forward's
        # error first and leaves the range decoder where it was; no row is
        # valid afterwards
        from detllm_amd import coder

        dec = coder.RangeDecoder(bytes(range(16)))
        before = dec.snapshot()
        assert _status(lambda: s.forward_decode(toks[2], 2, dec, 256)) == NON_FINITE
        after = dec.snapshot()
        assert (after.low, after.range, after.code, after.pos) == (before.low, before.range, before.code, before.pos)
        assert _status(lambda: s.decode_symbol(dec, 0, 256)) == 1
        s.reset()
        assert _status(lambda: s.forward_chunk(toks[:n], 0)) == NON_FINITE
        assert _status(lambda: s.forward_chunk(toks[:3], 0)) == NON_FINITE
    with Session(m, n, n) as s:
        syms = [int(t) for t in toks[1:n + 1]]
        assert _status(lambda: s.forward_ranges(toks[:n], 0, list(range(n)), syms, 256)) == NON_FINITE


def test_healthy_model_after_failures_is_unaffected():
    """The sticky flag is per call: a clean model still matches the oracle
    after another model's forward failed in the same process."""
    from detllm_amd.model import F32Llama

    w = W["tiny"]
    bad = F32Llama.from_gguf(synth.build_model(w, None, _edit("output.weight", _f32_fill(3e38))))
    toks = [int(t) for t in synth.tokens(w)]
    assert _status(lambda: bad.logits_hash_for_tokens_chunked(toks, 3)) == NON_FINITE
    g = synth.build_model(w)
    assert F32Llama.from_gguf(g).logits_hash_for_tokens_chunked(toks, 3) == detref.Model(g).logits_hash(toks)


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
@pytest.mark.parametrize("tail", [0, 256])
def test_cdf_entry_points_reject_non_finite_logits(bad, tail):
    from detllm_amd import coder

    for n in (4, 1000, 151936):
        lg = np.linspace(-3.0, 3.0, n).astype(np.float32)
        lg[n // 3] = bad
        with pytest.raises(Exception) as e:
            detref.logits_to_cdf(lg, tail)
        assert getattr(e.value, "status", None) == CDF_NON_FINITE_LOGIT
        f = coder.logits_to_cdf_with_byte_escapes if tail else coder.logits_to_cdf
        assert _status(lambda: f(lg)) == CDF_NON_FINITE_LOGIT
        r = coder.logits_to_symbol_range_with_byte_escapes if tail else coder.logits_to_symbol_range
        assert _status(lambda: r(lg, 1)) == CDF_NON_FINITE_LOGIT
