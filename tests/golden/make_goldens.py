"""Writes the full-depth, full-length workload goldens with the CPU oracle.

Run in the build container (CPU only; about 20 minutes on 8 cores):

    python tests/golden/make_goldens.py [smollm2 qwen05 tinyllama smollm2_l1 codec]

For every workload the full-depth synthetic model (detllm_amd.synth) runs
its whole token stream through the oracle, one position after another as
det-model's logits_hash_for_tokens_chunked does (crates/det-model/src/
lib.rs:1402-1465).  Each JSON file records the SHA-256 of all positions'
logits (f32 little-endian bits, positions ascending: the reference's logits
hash) and a 16-hex-digit digest of every single position, so a GPU mismatch
names its first position.  qwen05 and tinyllama also record the next-token
symbol range (cum, freq, total) of every position with the 256 byte-escape
symbols (det-coder cdf.rs:130-199): their SHA-256 (u64 cum, u32 freq, u64
total, little-endian, positions ascending), and for tinyllama every row's
triple, so a mismatch names its row.  The next token of the last position
is 0.  The codec file is the windowed payload of a
prefix of the byte stream of the end-to-end workload on the qwen05 model at
n_ctx 2048 (det-cli main.rs:521-551), long enough for three window
rollovers.
"""
from __future__ import annotations

import hashlib
import json
import os
import struct
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
for p in (ROOT, ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

import detref  # noqa: E402
from detllm_amd import synth  # noqa: E402

CODEC_SEED = 0xDE711005
CODEC_BYTES = 6144
CODEC_N_CTX = 2048


def _digests(rows: np.ndarray):
    full = hashlib.sha256()
    per = []
    for r in rows:
        b = np.ascontiguousarray(r, np.float32).tobytes()
        full.update(b)
        per.append(hashlib.sha256(b).hexdigest()[:16])
    return full.hexdigest(), per


# name -> (workload, layers, positions); None keeps the workload's own value.
# smollm2_l1: one layer over a whole 2048-position window, so that every
# 128-key block of the decode attention is compared at least once.
LOGITS = {"smollm2": ("smollm2", None, None), "qwen05": ("qwen05", None, None),
          "tinyllama": ("tinyllama", None, None), "smollm2_l1": ("smollm2", 1, 2048)}


def logits_golden(name: str) -> dict:
    wname, layers, positions = LOGITS[name]
    w = synth.WORKLOADS[wname]
    g = synth.build_model(w, layers)
    toks = synth.tokens(w, positions)
    t0 = time.time()
    rows = detref.Model(g).logits(toks)
    out = {"workload": wname, "layers": layers or w.layers, "positions": int(len(toks)),
           "model_sha256": hashlib.sha256(g).hexdigest()}
    out["logits_sha256"], out["position_digests"] = _digests(rows)
    if wname in ("qwen05", "tinyllama"):
        nxt = [int(t) for t in toks[1:]] + [0]
        h = hashlib.sha256()
        triples = []
        for i in range(len(toks)):
            cum, freq, total = detref.symbol_range(rows[i], nxt[i], 256)
            h.update(struct.pack("<QIQ", cum, freq, total))
            triples.append([cum, freq, total])
        out["next_token_ranges_sha256"] = h.hexdigest()
        out["range_tail"] = 256
        if wname == "tinyllama":
            out["next_token_ranges"] = triples
    out["oracle_seconds"] = round(time.time() - t0, 1)
    return out


def codec_golden() -> dict:
    w = synth.WORKLOADS["qwen05"]
    g = synth.build_model(w)
    data = synth.markov_bytes(CODEC_SEED, CODEC_BYTES)
    m = detref.Model(g)
    tokens, types = synth.vocabulary(w.vocab)
    emit = [1 if ty in (1, 4, 6) else 0 for ty in types]  # det-token lib.rs:258-325
    b2t, _ = detref.byte_fallback_tables(tokens, emit)
    sym = detref.codec_symbols(b2t, data, m.vocab)
    t0 = time.time()
    payload = detref.codec_encode(m, sym, CODEC_N_CTX, CODEC_N_CTX // 4, True)
    n_tok = int((sym < m.vocab).sum())
    return {"workload": "qwen05", "layers": w.layers, "markov_seed": CODEC_SEED, "bytes": CODEC_BYTES,
            "symbols": int(len(sym)), "escapes": int(len(sym) - n_tok), "n_ctx": CODEC_N_CTX,
            "overlap": CODEC_N_CTX // 4, "payload_len": len(payload),
            "payload_sha256": hashlib.sha256(payload).hexdigest(),
            "oracle_seconds": round(time.time() - t0, 1)}


def dumps(res: dict) -> str:
    """JSON with one-space indents, and the per-row range triples one per line."""
    triples = res.get("next_token_ranges")
    if triples is None:
        return json.dumps(res, indent=1) + "\n"
    head = dict(res)
    head["next_token_ranges"] = "@RANGES@"
    rows = ",\n  ".join(json.dumps(t) for t in triples)
    return json.dumps(head, indent=1).replace('"@RANGES@"', "[\n  " + rows + "\n ]") + "\n"


def main(argv) -> None:
    detref.set_threads(int(os.environ.get("GOLDEN_THREADS", 0)) or os.cpu_count() or 1)
    todo = argv or ["smollm2", "qwen05", "tinyllama", "smollm2_l1", "codec"]
    for name in todo:
        t0 = time.time()
        res = codec_golden() if name == "codec" else logits_golden(name)
        res["generator"] = "tests/golden/make_goldens.py"
        path = HERE / f"workload_{name}.json"
        path.write_text(dumps(res))
        print(f"{name}: {time.time() - t0:.0f} s -> {path.name}", flush=True)


if __name__ == "__main__":
    main(sys.argv[1:])
