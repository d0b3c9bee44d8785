"""Seeded synthetic models and token streams for the benchmark workloads.

Every random quantity comes from a counter-based SplitMix64 stream that
numpy evaluates in bulk, and every floating-point step is an IEEE-754 basic
operation (add, multiply, divide, sqrt, float16 rounding), so the generated
GGUF bytes are identical on every machine.  "Normal" draws use the sum of
four uniforms scaled to unit variance; Zipf draws invert a cumulative table
whose powers k^-s are evaluated with series built from basic operations.

Workloads (shapes of well-known checkpoints, random weights):
  tiny     Llama, 2 layers, d=64, 4/2 heads (hd 16), FFN 128, vocab 256, all F32
  smollm2  SmolLM2-135M shape, Q8_0, 30 layers, d=576, 9/3 heads, FFN 1536, vocab 49152
  qwen05   Qwen2.5-0.5B shape, Q8_0 + f32 QKV bias, 24 layers, d=896, 14/2 heads,
           FFN 4864, vocab 151936, split-half RoPE
  tinyllama TinyLlama-1.1B shape, Q4_K (Q6_K for attn_v, ffn_down of even layers and
           output), 22 layers, d=2048, 32/4 heads, FFN 5632, vocab 32000
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Dict, List, Optional, Tuple

import numpy as np

from .gguf import GGML_F32, GGML_Q4_K, GGML_Q6_K, GGML_Q8_0, GgufWriter, Tensor

GAMMA = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * M1
    z = (z ^ (z >> np.uint64(27))) * M2
    return z ^ (z >> np.uint64(31))


def _fnv1a(key: str) -> int:
    h = 0xCBF29CE484222325
    for b in key.encode():
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


class Stream:
    """Counter-based SplitMix64: value i = mix(start + (i+1)*gamma)."""

    def __init__(self, seed: int, key: str):
        base = np.array([(seed ^ _fnv1a(key)) & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64)
        self.start = _mix(base)[0]
        self.pos = 0

    def u64(self, n: int) -> np.ndarray:
        with np.errstate(over="ignore"):
            idx = np.arange(self.pos + 1, self.pos + n + 1, dtype=np.uint64)
            out = _mix(self.start + idx * GAMMA)
        self.pos += n
        return out

    def bytes(self, n: int) -> np.ndarray:
        words = self.u64((n + 7) // 8)
        return words.view(np.uint8)[:n].copy()

    def unit(self, n: int) -> np.ndarray:
        """Uniform doubles in [0, 1) with 53 random bits."""
        return (self.u64(n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)

    def ints(self, n: int, lo: int, hi: int) -> np.ndarray:
        """Uniform integers in [lo, hi] (inclusive)."""
        span = np.uint64(hi - lo + 1)
        return (self.u64(n) % span).astype(np.int64) + lo

    def normal(self, n: int) -> np.ndarray:
        """Approximately N(0, 1): (u1+u2+u3+u4-2) * sqrt(3)."""
        u = self.unit(4 * n).reshape(n, 4)
        s = ((u[:, 0] + u[:, 1]) + (u[:, 2] + u[:, 3])) - 2.0
        return s * 1.7320508075688772


def _ln(x: np.ndarray) -> np.ndarray:
    """Natural log from frexp and the atanh series (basic operations only)."""
    m, e = np.frexp(x)  # x = m * 2^e, m in [0.5, 1)
    m = m * 2.0
    e = e - 1
    s = (m - 1.0) / (m + 1.0)
    s2 = s * s
    term = s
    acc = np.zeros_like(s)
    for k in range(0, 40):
        acc = acc + term / (2 * k + 1)
        term = term * s2
    return 2.0 * acc + e * 0.6931471805599453


def _exp(y: np.ndarray) -> np.ndarray:
    """exp(y): y = k*ln2 + r with r in [0, ln2), Taylor series for e^r, ldexp by k."""
    ln2 = 0.6931471805599453
    k = np.floor(y / ln2)
    r = y - k * ln2
    acc = np.ones_like(r)
    term = np.ones_like(r)
    for i in range(1, 25):
        term = term * r / i
        acc = acc + term
    return np.ldexp(acc, k.astype(np.int64))


def zipf_tokens(seed: int, key: str, n: int, vocab: int, s: float = 1.1) -> np.ndarray:
    """n token ids whose ranks follow Zipf(s) over the vocabulary."""
    ranks = np.arange(1, vocab + 1, dtype=np.float64)
    weights = _exp(-s * _ln(ranks))
    cdf = np.cumsum(weights)
    cdf = cdf / cdf[-1]
    st = Stream(seed, key)
    u = st.unit(n)
    r = np.searchsorted(cdf, u, side="right")
    r = np.minimum(r, vocab - 1)
    perm = np.argsort(Stream(seed, key + ".perm").u64(vocab), kind="stable")
    return perm[r].astype(np.uint32)


# ---- block encoders ------------------------------------------------------------

def _f16_abs_normal(st: Stream, n: int, sigma: float) -> np.ndarray:
    v = np.abs(st.normal(n) * sigma).astype(np.float32).astype(np.float16)
    return v.view(np.uint16)


def q8_0_bytes(st: Stream, rows: int, cols: int, sigma: float) -> bytes:
    nb = rows * cols // 32
    blocks = np.empty((nb, 34), dtype=np.uint8)
    blocks[:, 0:2] = _f16_abs_normal(st, nb, sigma).view(np.uint8).reshape(nb, 2)
    # One random byte per quant folded onto [-127, 127] (bytes 0 and 255 share -127).
    q = (st.bytes(nb * 32).astype(np.int16) % 255) - 127
    blocks[:, 2:] = q.astype(np.int8).view(np.uint8).reshape(nb, 32)
    return blocks.tobytes()


def q4_k_bytes(st: Stream, rows: int, cols: int, sigma: float) -> bytes:
    nb = rows * cols // 256
    blocks = np.empty((nb, 144), dtype=np.uint8)
    blocks[:, 0:2] = _f16_abs_normal(st, nb, sigma).view(np.uint8).reshape(nb, 2)
    blocks[:, 2:4] = _f16_abs_normal(st, nb, sigma).view(np.uint8).reshape(nb, 2)
    # Every bit pattern of the 12 packed bytes is a valid set of eight 6-bit
    # scales and eight 6-bit mins, so uniform bytes give U{0..63} for each.
    blocks[:, 4:16] = st.bytes(nb * 12).reshape(nb, 12)
    blocks[:, 16:] = st.bytes(nb * 128).reshape(nb, 128)
    return blocks.tobytes()


def q6_k_bytes(st: Stream, rows: int, cols: int, sigma: float) -> bytes:
    nb = rows * cols // 256
    blocks = np.empty((nb, 210), dtype=np.uint8)
    blocks[:, 0:192] = st.bytes(nb * 192).reshape(nb, 192)
    blocks[:, 192:208] = st.ints(nb * 16, -63, 63).astype(np.int8).view(np.uint8).reshape(nb, 16)
    blocks[:, 208:210] = _f16_abs_normal(st, nb, sigma).view(np.uint8).reshape(nb, 2)
    return blocks.tobytes()


def f32_normal(st: Stream, n: int, sigma: float, mean: float = 0.0) -> np.ndarray:
    return (st.normal(n) * sigma + mean).astype(np.float32)


@dataclass(frozen=True)
class Workload:
    name: str
    arch: str
    layers: int
    d: int
    heads: int
    kv_heads: int
    ff: int
    vocab: int
    rope_base: float
    eps: float
    ctx: int
    weight: str              # "f32" | "q8_0" | "q4k_mix"
    tied: bool
    qkv_bias: bool
    seed: int
    n_tokens: int
    token_dist: str          # "uniform" | "zipf"
    chunk: int
    description: str


WORKLOADS: Dict[str, Workload] = {
    "tiny": Workload("tiny", "llama", 2, 64, 4, 2, 128, 256, 1e4, 1e-5, 8, "f32", False, False,
                     0xDE711001, 8, "uniform", 3,
                     "Llama 2L d64 4/2 heads hd16 FFN128 V256, all F32, untied lm_head; 8 tokens, n_ctx 8, chunk 3"),
    "smollm2": Workload("smollm2", "llama", 30, 576, 9, 3, 1536, 49152, 1e5, 1e-5, 2048, "q8_0", True,
                        False, 0xDE711002, 512, "zipf", 1,
                        "SmolLM2-135M-shaped Llama, Q8_0, tied embeddings; 512 Zipf tokens, n_ctx 2048, single-token decode"),
    "qwen05": Workload("qwen05", "qwen2", 24, 896, 14, 2, 4864, 151936, 1e6, 1e-6, 2048, "q8_0", True,
                       True, 0xDE711003, 1024, "zipf", 1,
                       "Qwen2.5-0.5B-shaped decoder, Q8_0 + f32 QKV bias, tied; 1024 Zipf tokens, n_ctx 2048"),
    "tinyllama": Workload("tinyllama", "llama", 22, 2048, 32, 4, 5632, 32000, 1e4, 1e-5, 2048, "q4k_mix",
                          False, False, 0xDE711004, 2048, "zipf", 64,
                          "TinyLlama-1.1B-shaped Llama, Q4_K with Q6_K attn_v / even-layer ffn_down / output; 2048 Zipf tokens, n_ctx 2048, chunk 64"),
}


# Byte tokens the synthetic vocabularies mark non-emittable (GGUF token type
# 3, control): the byte-fallback tokenizer codes these bytes as escapes.
ESCAPED_BYTES = (0x7A, 0x7E)


def vocabulary(vocab: int) -> Tuple[List[str], List[int]]:
    """Synthetic vocabulary: ids 0..255 are the byte-fallback tokens <0x00>
    .. <0xFF> (type 6, byte; ESCAPED_BYTES type 3), the rest plain tokens
    (type 1) that the byte-fallback path never emits."""
    tokens = [f"<0x{b:02X}>" for b in range(256)] + [f"<synth_{i}>" for i in range(256, vocab)]
    types = [3 if b in ESCAPED_BYTES else 6 for b in range(256)] + [1] * (vocab - 256)
    return tokens, types


def build_model(w: Workload, layers: Optional[int] = None,
                edit: Optional[Callable[[Tensor], None]] = None) -> bytes:
    """Writes the workload's model as GGUF bytes.  `layers` truncates depth
    (used by quick tests); the benchmark always uses the full depth.
    `edit`, when given, may rewrite each tensor's bytes before the file is
    written (tests plant non-finite or out-of-range values with it)."""
    L = w.layers if layers is None else layers
    hd = w.d // w.heads
    g = GgufWriter()
    g.add_str("general.architecture", w.arch)
    p = w.arch + "."
    g.add_u32(p + "block_count", L)
    g.add_u32(p + "context_length", w.ctx)
    g.add_u32(p + "embedding_length", w.d)
    g.add_u32(p + "feed_forward_length", w.ff)
    g.add_u32(p + "attention.head_count", w.heads)
    g.add_u32(p + "attention.head_count_kv", w.kv_heads)
    g.add_f32(p + "rope.freq_base", w.rope_base)
    g.add_f32(p + "attention.layer_norm_rms_epsilon", w.eps)
    g.add_u32(p + "vocab_size", w.vocab)
    tokens, types = vocabulary(w.vocab)
    g.add_str_array("tokenizer.ggml.tokens", tokens)
    g.add_i32_array("tokenizer.ggml.token_type", types)

    def mat(name: str, rows: int, cols: int, kind: str) -> None:
        st = Stream(w.seed, name)
        if kind == "f32":
            g.add_tensor(name, (cols, rows), GGML_F32, f32_normal(st, rows * cols, 0.02))
        elif kind == "q8_0":
            g.add_tensor(name, (cols, rows), GGML_Q8_0, q8_0_bytes(st, rows, cols, 2e-3))
        elif kind == "q4_k":
            g.add_tensor(name, (cols, rows), GGML_Q4_K, q4_k_bytes(st, rows, cols, 1e-3))
        elif kind == "q6_k":
            g.add_tensor(name, (cols, rows), GGML_Q6_K, q6_k_bytes(st, rows, cols, 1e-3))
        else:
            raise ValueError(kind)

    def norm(name: str, n: int) -> None:
        g.add_tensor(name, (n,), GGML_F32, f32_normal(Stream(w.seed, name), n, 0.02, 1.0))

    def kind_of(role: str, layer: int) -> str:
        if w.weight == "f32":
            return "f32"
        if w.weight == "q8_0":
            return "q8_0"
        if role == "v" or role == "output" or (role == "down" and layer % 2 == 0):
            return "q6_k"
        return "q4_k"

    mat("token_embd.weight", w.vocab, w.d, kind_of("embd", -1))
    for l in range(L):
        b = f"blk.{l}."
        norm(b + "attn_norm.weight", w.d)
        mat(b + "attn_q.weight", w.heads * hd, w.d, kind_of("q", l))
        mat(b + "attn_k.weight", w.kv_heads * hd, w.d, kind_of("k", l))
        mat(b + "attn_v.weight", w.kv_heads * hd, w.d, kind_of("v", l))
        if w.qkv_bias:
            for nm, n in (("attn_q.bias", w.heads * hd), ("attn_k.bias", w.kv_heads * hd),
                          ("attn_v.bias", w.kv_heads * hd)):
                g.add_tensor(b + nm, (n,), GGML_F32, f32_normal(Stream(w.seed, b + nm), n, 0.02))
        mat(b + "attn_output.weight", w.d, w.heads * hd, kind_of("o", l))
        norm(b + "ffn_norm.weight", w.d)
        mat(b + "ffn_gate.weight", w.ff, w.d, kind_of("gate", l))
        mat(b + "ffn_up.weight", w.ff, w.d, kind_of("up", l))
        mat(b + "ffn_down.weight", w.d, w.ff, kind_of("down", l))
    norm("output_norm.weight", w.d)
    if not w.tied:
        mat("output.weight", w.vocab, w.d, kind_of("output", -1))
    if edit is not None:
        for t in g.tensors:
            edit(t)
    return g.to_bytes()


def tokens(w: Workload, n: Optional[int] = None) -> np.ndarray:
    n = w.n_tokens if n is None else n
    if w.token_dist == "uniform":
        return Stream(w.seed, "tokens").ints(n, 0, w.vocab - 1).astype(np.uint32)
    return zipf_tokens(w.seed, "tokens", n, w.vocab)


def _pattern(n: int, period: int, scale: float) -> np.ndarray:
    """((i % period) - period // 2) * scale in f32, the fixture weight pattern."""
    i = np.arange(n)
    return (((i % period).astype(np.float32) - np.float32(period // 2)) * np.float32(scale)).astype(np.float32)


def cli_fixture_gguf(vocab_size: int = 256, token_override: Optional[Tuple[int, str]] = None,
                     include_bpe: bool = False) -> bytes:
    """The byte-fallback test model of the reference codec tests
    (det-cli main.rs:1976-2047): Llama 1 layer, d 4, FFN 6, 2/1 heads,
    rope_dim 2, n_ctx 16, F32 weights ((i % 13) - 6) * scale; the
    vocabulary is <0x00>..<0xFF> (+ "ab" and a merge with include_bpe)."""
    g = GgufWriter()
    g.add_str("general.architecture", "llama")
    for k, v in (("block_count", 1), ("embedding_length", 4), ("feed_forward_length", 6),
                 ("attention.head_count", 2), ("attention.head_count_kv", 1)):
        g.add_u32("llama." + k, v)
    g.add_f32("llama.attention.layer_norm_rms_epsilon", 1e-5)
    g.add_f32("llama.rope.freq_base", 10_000.0)
    g.add_u32("llama.rope.dimension_count", 2)
    g.add_u32("llama.context_length", 16)
    g.add_u32("llama.vocab_size", vocab_size)
    toks = [f"<0x{b:02X}>" for b in range(256)]
    if token_override is not None:
        toks[token_override[0]] = token_override[1]
    if include_bpe:
        toks.append("ab")
    g.add_str_array("tokenizer.ggml.tokens", toks)
    if include_bpe:
        g.add_str("tokenizer.ggml.model", "gpt2")
        g.add_str_array("tokenizer.ggml.merges", ["<0x61> <0x62>"])

    def mat(name: str, rows: int, cols: int, scale: float) -> None:
        g.add_tensor(name, (cols, rows), GGML_F32, _pattern(rows * cols, 13, scale))

    def vec(name: str, n: int) -> None:
        g.add_tensor(name, (n,), GGML_F32, np.ones(n, np.float32))

    mat("token_embd.weight", vocab_size, 4, 0.001)
    vec("blk.0.attn_norm.weight", 4)
    mat("blk.0.attn_q.weight", 4, 4, 0.002)
    mat("blk.0.attn_k.weight", 2, 4, -0.0015)
    mat("blk.0.attn_v.weight", 2, 4, 0.0025)
    mat("blk.0.attn_output.weight", 4, 4, -0.002)
    vec("blk.0.ffn_norm.weight", 4)
    mat("blk.0.ffn_gate.weight", 6, 4, 0.003)
    mat("blk.0.ffn_up.weight", 6, 4, -0.0025)
    mat("blk.0.ffn_down.weight", 4, 6, 0.0018)
    vec("output_norm.weight", 4)
    mat("output.weight", vocab_size, 4, 0.0022)
    return g.to_bytes()


def codec_fixture_gguf() -> bytes:
    """The 4-token model of the reference's token-codec tests
    (det-cli main.rs:390-431): d 4, FFN 6, 2/1 heads, rope_dim 2, n_ctx 8,
    F32 weights ((i % 9) - 4) * scale."""
    g = GgufWriter()
    g.add_str("general.architecture", "llama")
    for k, v in (("block_count", 1), ("embedding_length", 4), ("feed_forward_length", 6),
                 ("attention.head_count", 2), ("attention.head_count_kv", 1)):
        g.add_u32("llama." + k, v)
    g.add_f32("llama.attention.layer_norm_rms_epsilon", 1e-5)
    g.add_f32("llama.rope.freq_base", 10_000.0)
    g.add_u32("llama.rope.dimension_count", 2)
    g.add_u32("llama.context_length", 8)
    g.add_u32("llama.vocab_size", 4)

    def mat(name: str, rows: int, cols: int, scale: float) -> None:
        g.add_tensor(name, (cols, rows), GGML_F32, _pattern(rows * cols, 9, scale))

    def vec(name: str, n: int) -> None:
        g.add_tensor(name, (n,), GGML_F32, np.ones(n, np.float32))

    mat("token_embd.weight", 4, 4, 0.01)
    vec("blk.0.attn_norm.weight", 4)
    mat("blk.0.attn_q.weight", 4, 4, 0.02)
    mat("blk.0.attn_k.weight", 2, 4, -0.015)
    mat("blk.0.attn_v.weight", 2, 4, 0.025)
    mat("blk.0.attn_output.weight", 4, 4, -0.02)
    vec("blk.0.ffn_norm.weight", 4)
    mat("blk.0.ffn_gate.weight", 6, 4, 0.03)
    mat("blk.0.ffn_up.weight", 6, 4, -0.025)
    mat("blk.0.ffn_down.weight", 4, 6, 0.018)
    vec("output_norm.weight", 4)
    mat("output.weight", 4, 4, 0.022)
    return g.to_bytes()


# Seed of the end-to-end codec workload's byte stream (1 MiB compressed and
# decompressed with the Qwen2.5-0.5B-shaped model at n_ctx 2048).
C5_SEED = 0xDE711005


def markov_bytes(seed: int, n: int) -> bytes:
    """n bytes of seeded order-3 Markov text over printable ASCII + newline.

    Words have Zipf(1.1) lengths in 1..16 and are separated by spaces;
    lines hold Zipf(1.1) 1..20 words.  Each word character is drawn by
    rank from a Zipf(1.1) law over the 94 visible characters, and the
    rank -> character map is a seeded permutation chosen by the previous
    three bytes (4096 hashed contexts), which makes the source order-3."""
    visible = np.arange(0x21, 0x7F, dtype=np.uint8)  # 94 characters
    nctx = 4096
    perms = np.argsort(Stream(seed, "markov.perm").u64(nctx * 94).reshape(nctx, 94), axis=1, kind="stable")
    table = visible[perms]  # [ctx][rank] -> byte

    def zipf_ranks(key: str, count: int, k: int) -> np.ndarray:
        w = _exp(-1.1 * _ln(np.arange(1, k + 1, dtype=np.float64)))
        cdf = np.cumsum(w)
        cdf = cdf / cdf[-1]
        return np.minimum(np.searchsorted(cdf, Stream(seed, key).unit(count), side="right"), k - 1)

    ranks = zipf_ranks("markov.char", n, 94)
    word_len = zipf_ranks("markov.word", n // 2 + 2, 16) + 1
    line_words = zipf_ranks("markov.line", n // 2 + 2, 20) + 1
    out = bytearray(n)
    c1 = c2 = c3 = 0x0A
    i = wi = li = ri = 0
    left_in_word = int(word_len[0])
    left_in_line = int(line_words[0])
    while i < n:
        if left_in_word == 0:
            left_in_line -= 1
            if left_in_line == 0:
                b = 0x0A
                li += 1
                left_in_line = int(line_words[li])
            else:
                b = 0x20
            wi += 1
            left_in_word = int(word_len[wi])
        else:
            b = int(table[((c1 * 961) + (c2 * 31) + c3) & (nctx - 1), ranks[ri]])
            ri += 1
            left_in_word -= 1
        out[i] = b
        c1, c2, c3 = c2, c3, b
        i += 1
    return bytes(out)
