"""Pins the oracle's qwen2 path and the Q4_K / Q6_K superblock scale fields.

- The qwen2 metadata test of det-model (lib.rs:3178-3213) restated against
  the oracle: architecture prefix, split-half RoPE pairing, epsilon, RoPE
  base and the three bias vectors as loaded.
- A closed form for the order "GEMV, + bias, RoPE" (lib.rs:1295-1320) and
  for the split-half pairing: a one-layer qwen2 model whose q and k are
  their biases alone (zero wq, wk), so the position-1 attention weights are
  fixed by the rotation of the biases.  An independent float64 forward
  gives the expected logits; the two plausible mistakes (bias added after
  RoPE, adjacent pairs) move the attention weight of position 0 from 0.022
  to 0.5 and are checked to land far from the oracle.
- Multi-superblock Q4_K rows with d != dmin (and different per superblock),
  Q6_K rows with d != 1: a swapped f16 field or superblock index fails.
"""
import math

import numpy as np
import pytest

import detref
import qblocks
from detllm_amd.gguf import GGML_F32, GgufWriter


def _f32_gguf(arch, cfg, tensors):
    w = GgufWriter()
    w.add_str("general.architecture", arch)
    for key, kind, v in cfg:
        (w.add_u32 if kind == "u32" else w.add_f32)(f"{arch}.{key}", v)
    for name, arr in tensors:
        a = np.ascontiguousarray(arr, np.float32)
        dims = (a.shape[1], a.shape[0]) if a.ndim == 2 else (a.shape[0],)
        w.add_tensor(name, dims, GGML_F32, a)
    return w.to_bytes()


def _pattern(rows, cols, scale):
    # push_tensor (det-model lib.rs:4160-4179): ((i % 11) - 5) * scale
    i = np.arange(rows * cols)
    return (((i % 11).astype(np.float32) - np.float32(5.0)) * np.float32(scale)).reshape(rows, cols)


def test_qwen2_metadata_restated():
    # det-model lib.rs:3178-3213 with the builder of lib.rs:3921-4033
    cfg = [("block_count", "u32", 1), ("embedding_length", "u32", 4), ("feed_forward_length", "u32", 6),
           ("attention.head_count", "u32", 2), ("attention.head_count_kv", "u32", 1),
           ("attention.layer_norm_rms_epsilon", "f32", 1e-6), ("rope.freq_base", "f32", 1_000_000.0),
           ("rope.dimension_count", "u32", 2), ("context_length", "u32", 4), ("vocab_size", "u32", 3)]
    tensors = [("token_embd.weight", _pattern(3, 4, 0.01)),
               ("blk.0.attn_norm.weight", np.ones(4)),
               ("blk.0.attn_q.weight", _pattern(4, 4, 0.02)),
               ("blk.0.attn_q.bias", np.full(4, 0.001)),
               ("blk.0.attn_k.weight", _pattern(2, 4, -0.015)),
               ("blk.0.attn_k.bias", np.full(2, -0.002)),
               ("blk.0.attn_v.weight", _pattern(2, 4, 0.025)),
               ("blk.0.attn_v.bias", np.full(2, 0.003)),
               ("blk.0.attn_output.weight", _pattern(4, 4, -0.02)),
               ("blk.0.ffn_norm.weight", np.ones(4)),
               ("blk.0.ffn_gate.weight", _pattern(6, 4, 0.03)),
               ("blk.0.ffn_up.weight", _pattern(6, 4, -0.025)),
               ("blk.0.ffn_down.weight", _pattern(4, 6, 0.018)),
               ("output_norm.weight", np.ones(4)),
               ("output.weight", _pattern(3, 4, 0.022))]
    m = detref.Model(_f32_gguf("qwen2", cfg, tensors))
    c = m.cfg
    f = lambda b: float(np.array([b], np.uint32).view(np.float32)[0])
    assert c[:10] == [1, 4, 6, 2, 1, 2, 2, 1, 4, 3]  # ... rope_dim 2, SplitHalf (1), ctx 4, vocab 3
    assert f(c[10]) == np.float32(1e-6)
    assert f(c[11]) == np.float32(1.0) / np.float32(math.sqrt(2.0))  # default_attention_scale(2)
    assert f(c[12]) == np.float32(1_000_000.0)
    assert m.bias(0, 0).view(np.uint32).tolist() == np.full(4, 0.001, np.float32).view(np.uint32).tolist()
    assert m.bias(0, 1).view(np.uint32).tolist() == np.full(2, -0.002, np.float32).view(np.uint32).tolist()
    assert m.bias(0, 2).view(np.uint32).tolist() == np.full(2, 0.003, np.float32).view(np.uint32).tolist()
    assert any(m.logits_hash([0, 1]))
    # the same model under "llama" pairs adjacent dimensions and has no bias
    llama = detref.Model(_f32_gguf("llama", cfg, [t for t in tensors if not t[0].endswith(".bias")]))
    assert llama.cfg[7] == 0 and llama.bias(0, 0) is None


# ---- bias before RoPE, split-half pairs: closed form -------------------------------

C = 3.0
THETA = 1e6
EMB = np.array([[1.0, 0.5, -0.25, 2.0], [-1.0, 2.0, 0.5, 0.25], [0.3, -0.7, 1.1, 0.2]])
BQ = np.array([0.0, 0.0, C, 0.0])
BK = np.array([C, 0.0, 0.0, 0.0])
BV = np.array([0.1, -0.2, 0.3, 0.05])
OUT = np.array([[1.0, 0.0, 0.0, 0.0], [0.0, 1.0, 0.0, 0.0], [0.5, 0.5, -1.0, 1.0]])


def _rope64(x, pos, split_half):
    """Rotates a 4-vector at `pos`, theta 1e6, rope_dim 4, in float64."""
    x = x.copy()
    for j in range(2):
        ang = pos * THETA ** (-(2.0 * j) / 4.0)
        a, b = (j, j + 2) if split_half else (2 * j, 2 * j + 1)
        x0, x1 = x[a], x[b]
        x[a] = x0 * math.cos(ang) - x1 * math.sin(ang)
        x[b] = x0 * math.sin(ang) + x1 * math.cos(ang)
    return x


def _forward64(tokens, split_half=True, bias_after_rope=False):
    """Float64 forward of the model below: wq = wk = 0, wv = wo = I, zero FFN."""
    eps = 1e-6

    def norm(v):
        return v / math.sqrt(float(np.mean(v * v)) + eps)

    ks, vs, out, p0 = [], [], [], None
    for pos, t in enumerate(tokens):
        x = EMB[t].copy()
        h = norm(x)
        if bias_after_rope:
            q, k = _rope64(np.zeros(4), pos, split_half) + BQ, _rope64(np.zeros(4), pos, split_half) + BK
        else:
            q, k = _rope64(BQ, pos, split_half), _rope64(BK, pos, split_half)
        ks.append(k)
        vs.append(h + BV)
        if pos == 0:
            att = vs[0]
        else:
            s = np.array([q @ kj for kj in ks]) * 0.5
            e = np.exp(s - s.max())
            p = e / e.sum()
            p0 = p[0] if pos == 1 else p0
            att = sum(pj * vj for pj, vj in zip(p, vs))
        x = x + att  # the FFN adds silu(0) * 0 = 0 through a zero down matrix
        out.append(OUT @ norm(x))
    return np.array(out), p0


def _closed_form_model():
    cfg = [("block_count", "u32", 1), ("embedding_length", "u32", 4), ("feed_forward_length", "u32", 4),
           ("attention.head_count", "u32", 1), ("attention.head_count_kv", "u32", 1),
           ("attention.layer_norm_rms_epsilon", "f32", 1e-6), ("rope.freq_base", "f32", THETA),
           ("rope.dimension_count", "u32", 4), ("context_length", "u32", 4), ("vocab_size", "u32", 3)]
    z = np.zeros((4, 4))
    tensors = [("token_embd.weight", EMB), ("blk.0.attn_norm.weight", np.ones(4)),
               ("blk.0.attn_q.weight", z), ("blk.0.attn_q.bias", BQ),
               ("blk.0.attn_k.weight", z), ("blk.0.attn_k.bias", BK),
               ("blk.0.attn_v.weight", np.eye(4)), ("blk.0.attn_v.bias", BV),
               ("blk.0.attn_output.weight", np.eye(4)), ("blk.0.ffn_norm.weight", np.ones(4)),
               ("blk.0.ffn_gate.weight", z), ("blk.0.ffn_up.weight", z), ("blk.0.ffn_down.weight", z),
               ("output_norm.weight", np.ones(4)), ("output.weight", OUT)]
    return _f32_gguf("qwen2", cfg, tensors)


def test_qwen2_bias_before_split_half_rope_closed_form():
    m = detref.Model(_closed_form_model())
    toks = [0, 1, 2]
    got = m.logits(toks).astype(np.float64)
    want, p0 = _forward64(toks)
    assert abs(p0 - 0.0220) < 1e-3  # softmax(-c^2 sin(1) / 2, 0) at position 1
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5)
    for wrong in (dict(split_half=False), dict(bias_after_rope=True)):
        bad, p0_bad = _forward64(toks, **wrong)
        assert abs(p0_bad - 0.5) < 1e-12
        assert np.max(np.abs(got[1:] - bad[1:])) > 0.05, wrong


# ---- Q4_K with d != dmin, Q6_K with d != 1 ------------------------------------------

def _exact_activation(rng, cols):
    x = rng.integers(-127, 128, cols).astype(np.float32)
    x[::32] = 127.0  # Q8A d == 1 in every block
    return x


@pytest.mark.parametrize("nsb", [1, 2, 3])
def test_q4_k_row_closed_form_distinct_d_dmin(nsb):
    # q4_k_value (det-quant lib.rs:506-529): (d * sc) * q - dmin * m, d at
    # bytes 0-1 and dmin at bytes 2-3 of the superblock; powers of two keep
    # every product and partial sum exact, so the dot is an integer closed form.
    rng = np.random.default_rng(40 + nsb)
    cols = 256 * nsb
    d = np.array([2.0, 0.5, 4.0][:nsb])
    dmin = np.array([0.25, 8.0, 1.0][:nsb])
    sc = rng.integers(0, 16, (nsb, 8))
    mn = rng.integers(0, 16, (nsb, 8))
    nib = rng.integers(0, 16, (nsb, 256))
    row = qblocks.q4_k_row([qblocks.f16(v) for v in d], [qblocks.f16(v) for v in dmin], sc, mn, nib)
    x = _exact_activation(rng, cols)
    w = np.concatenate([np.repeat(d[b] * sc[b], 32) * nib[b] - np.repeat(dmin[b] * mn[b], 32)
                        for b in range(nsb)])
    want = float(np.dot(w, x.astype(np.float64)))
    assert abs(want) < 2 ** 24
    assert detref.dot_row(12, row, cols, x) == want
    swapped = float(np.dot(np.concatenate([np.repeat(dmin[b] * sc[b], 32) * nib[b] -
                                           np.repeat(d[b] * mn[b], 32) for b in range(nsb)]),
                           x.astype(np.float64)))
    assert swapped != want


@pytest.mark.parametrize("nsb", [2, 3])
def test_q6_k_row_closed_form_scaled_d(nsb):
    # dot_q6_k_q8k (det-quant lib.rs:353-397) with a different power-of-two d
    # per superblock: sums[l] += (d * dq) * aux[l]; a superblock-index slip fails.
    rng = np.random.default_rng(50 + nsb)
    cols = 256 * nsb
    d = np.array([2.0, 0.25, 8.0][:nsb])
    sc = rng.integers(-7, 8, (nsb, 16))
    q6 = rng.integers(-32, 32, (nsb, 256))
    row = qblocks.q6_k_row([qblocks.f16(v) for v in d], sc, q6)
    x = rng.integers(-126, 127, cols).astype(np.float32)
    x[::256] = 127.0  # Q8_K d == -1
    w = np.concatenate([np.repeat(sc[b], 16) * q6[b] * d[b] for b in range(nsb)])
    want = float(np.dot(w, x.astype(np.float64)))
    assert detref.dot_row(14, row, cols, x) == want
    assert float(np.dot(np.concatenate([np.repeat(sc[b], 16) * q6[b] * d[::-1][b] for b in range(nsb)]),
                        x.astype(np.float64))) != want
