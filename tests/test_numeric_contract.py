"""Static check of the numeric contract on the device code this build ships.

The reference enforces its determinism rules with `xtask check-determinism`
(xtask/src/main.rs:21-436): it bans FMA, fast-math flags and intrinsics,
hardware approximate reciprocals and platform transcendentals from its
sources.  The device code here is compiled by LLVM, so the same rules are
checked where they take effect, on every .hip source of the library compiled
for gfx950 with the library's own flags (detllm_amd.build.NUMERIC_FLAGS):

LLVM IR of the device pass (before instruction selection):
- no fast-math flag (contract, reassoc, afn, arcp, nnan, ninf, nsz, fast)
  on any instruction, and no llvm.fmuladd: the backend may then fuse no
  multiply into an add;
- no !fpmath accuracy relaxation on a divide or square root, no
  approximate or platform math intrinsic (amdgcn rcp/rsq/exp2/log/sin/cos,
  llvm.exp/log/pow/sin/cos, device-library calls);
- every explicit llvm.fma.f32 is one half of the Markstein quotient
  correction div_recip(v, d, 1/d): r = fma(-q0, d, v) then fma(r, 1/d, q0)
  (its equality with correctly rounded division is checked exhaustively on
  the host by tests/test_div_recip.py).

gfx950 assembly:
- no packed FP32 instruction (v_pk_add/mul/fma_f32);
- no write through the scalar data cache (scalar stores and atomics, its
  write-back and discard);
- no hardware transcendental approximation (v_exp/v_log/v_sin/v_cos/v_rsq;
  v_rcp_f32 and v_rcp_iflag_f32 remain as the seeds of the correctly rounded
  divide expansion and of integer division, whose results are exact);
- matrix-core instructions only in the chunked encode GEMMs: the exact int8
  form (dtl_gemm.hip), and the f32 outer product with one element of K
  (dtl_mfp.hip), every one with the literal 0 as its accumulator, so that
  each result is one rounded product and no MFMA adds.

Sources: no platform transcendental or fast intrinsic is called, and the
only explicit fma is div_recip's.
"""
import re
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

from detllm_amd import build as B

HIP_SOURCES = [s for s in B.SOURCES if s.endswith(".hip")]
FLAGS = [f"--offload-arch={B.ARCH}", "-O3", "-std=c++17", *B.NUMERIC_FLAGS, "--cuda-device-only",
         "-Wno-unused-result"]


@pytest.fixture(scope="module")
def device_code(tmp_path_factory):
    """{source: (llvm_ir_text, gfx950_asm_text)} for every .hip source."""
    d = tmp_path_factory.mktemp("contract")
    cc = B.hipcc()

    def one(src, kind):
        out = d / f"{Path(src).stem}.{kind}"
        extra = ["-emit-llvm", "-S"] if kind == "ll" else ["-S"]
        res = subprocess.run([cc, *FLAGS, *B.EXTRA_FLAGS.get(src, []), *extra, str(B.CSRC / src), "-o", str(out)],
                             capture_output=True, text=True)
        assert res.returncode == 0, res.stderr[-2000:]
        return out.read_text()

    jobs = [(s, k) for s in HIP_SOURCES for k in ("ll", "s")]
    with ThreadPoolExecutor(max_workers=8) as ex:
        texts = list(ex.map(lambda a: one(*a), jobs))
    res = {}
    for (s, k), t in zip(jobs, texts):
        res.setdefault(s, {})[k] = t
    return {s: (v["ll"], v["s"]) for s, v in res.items()}


def test_build_flags_pin_the_contract():
    flags = " ".join(B.NUMERIC_FLAGS)
    for f in ("-ffp-contract=off", "-fno-fast-math", "-fhip-fp32-correctly-rounded-divide-sqrt",
              "-fno-gpu-flush-denormals-to-zero", "-packed-fp32-ops"):
        assert f in flags
    assert "-ffast-math" not in flags.replace("-fno-fast-math", "")


_FM_FLAG = re.compile(
    r"\b(?:fadd|fsub|fmul|fdiv|frem|fneg|fcmp|call|select|phi|fptrunc|fpext|uitofp|sitofp)"
    r"\s+(?:fast|contract|reassoc|nnan|ninf|nsz|arcp|afn)\b")
_APPROX = re.compile(
    r"@(?:llvm\.amdgcn\.(?:rcp|rsq|sqrt|exp2|log|sin|cos|fract|frexp)\b"
    r"|llvm\.(?:exp|exp2|exp10|log|log2|log10|pow|powi|sin|cos|tan)\."
    r"|__ocml_)")


def test_ir_has_no_contraction_fast_math_or_approximation(device_code):
    for src, (ir, _) in device_code.items():
        assert "@llvm.fmuladd" not in ir, src
        m = _FM_FLAG.search(ir)
        assert m is None, f"{src}: fast-math flag: {ir[max(0, m.start() - 80):m.end() + 80]}"
        assert "!fpmath" not in ir, src
        m = _APPROX.search(ir)
        assert m is None, f"{src}: approximate or platform math: {ir[m.start():m.start() + 120]}"
        assert "@llvm.fma.v" not in ir, src


_FMA_CALL = re.compile(
    r"^\s*(%[\w.]+) = (?:tail )?call (?:noundef )?float @llvm\.fma\.f32\("
    r"float (?:noundef )?([^,]+), float (?:noundef )?([^,]+), float (?:noundef )?([^)]+)\)")
_FNEG = re.compile(r"^\s*(%[\w.]+) = fneg float (%[\w.]+)")


def _fma_pairs(ir):
    """(fma calls, div_recip pairs, unexplained calls) over every function."""
    total = pairs = 0
    unexplained = []
    fn = None
    for line in ir.splitlines():
        if line.startswith("define "):
            fn = {"fma": {}, "neg": {}, "name": line.split("@", 1)[1].split("(", 1)[0]}
            continue
        if fn is None:
            continue
        if line.startswith("}"):
            fmas, negs = fn["fma"], fn["neg"]
            total += len(fmas)
            firsts, seconds = set(), set()
            for res, (a, _b, c) in fmas.items():
                # second half fma(r, 1/d, q0) whose r = fma(-q0, d, v)
                if a in fmas and negs.get(fmas[a][0]) == c:
                    firsts.add(a)
                    seconds.add(res)
            pairs += len(seconds)
            unexplained += [(fn["name"], r) for r in fmas if r not in firsts and r not in seconds]
            fn = None
            continue
        if "@llvm.fma.f32(" in line:
            m = _FMA_CALL.match(line)
            assert m, line
            fn["fma"][m.group(1)] = tuple(x.strip() for x in m.groups()[1:])
        m = _FNEG.match(line)
        if m:
            fn["neg"][m.group(1)] = m.group(2)
    return total, pairs, unexplained


def test_every_explicit_fma_is_a_div_recip_pair(device_code):
    seen = 0
    for src, (ir, _) in device_code.items():
        total, pairs, unexplained = _fma_pairs(ir)
        assert not unexplained, f"{src}: fma outside div_recip: {unexplained[:5]}"
        assert total == 2 * pairs, src
        seen += pairs
    # the Q8A quantiser (the only user of div_recip) is inlined into the
    # rmsnorm, quantise and fused decode GEMV kernels
    assert seen > 0


_SCALAR_WRITE = re.compile(r"^\s*s_(?:store|buffer_store|scratch_store|atomic|buffer_atomic|dcache_wb|dcache_discard)",
                           re.M)
_PACKED_F32 = re.compile(r"^\s*v_pk_(?:add|mul|fma|mov)_f32", re.M)
_HW_APPROX = re.compile(r"^\s*v_(?:exp|log|sin|cos|rsq|exp_legacy|log_legacy)_f32", re.M)
_MFMA = re.compile(r"^\s*(v_mfma_\w+)", re.M)
_MFMA_F32_LINE = re.compile(r"^\s*v_mfma_f32_\w+[^\n]*", re.M)


def test_asm_has_no_packed_f32_scalar_writes_or_hw_approximations(device_code):
    for src, (_, asm) in device_code.items():
        for name, rx in (("packed FP32", _PACKED_F32), ("scalar-cache write", _SCALAR_WRITE),
                         ("hardware approximation", _HW_APPROX)):
            m = rx.search(asm)
            assert m is None, f"{src}: {name}: {asm[m.start():m.start() + 80]!r}"
        mfma = set(_MFMA.findall(asm))
        if src == "dtl_gemm.hip":
            assert mfma == {"v_mfma_i32_16x16x64_i8"}, mfma
        elif src == "dtl_mfp.hip":
            assert mfma == {"v_mfma_f32_16x16x1_4b_f32"}, mfma
            lines = _MFMA_F32_LINE.findall(asm)
            assert lines and all(ln.split(";")[0].rstrip().endswith(", 0") for ln in lines), lines[:4]
        else:
            assert not mfma, (src, mfma)


_SRC_BANNED = re.compile(
    r"\b(?:expf|exp2f|exp10f|logf|log2f|log10f|powf|sinf|cosf|tanf|tanhf|rsqrtf|__expf|__logf|__powf"
    r"|__fdividef|__frcp_r[nduz]|__frsqrt_rn|__fmaf_r[nduz]|fmaf|__builtin_amdgcn_(?:rcp|rsq|exp2|log|sin|cos)f?"
    r"|std::(?:exp|log|pow|sin|cos|tan|fma))\s*\(")


def test_sources_call_no_platform_transcendental_or_fast_intrinsic():
    for path in sorted(B.CSRC.iterdir()):
        text = path.read_text()
        code = re.sub(r"//[^\n]*|/\*.*?\*/", "", text, flags=re.S)
        m = _SRC_BANNED.search(code)
        assert m is None, f"{path.name}: {code[m.start():m.end() + 40]!r}"
        for bad in ("-ffast-math", "fp contract(fast)", "unsafe-fp-math", "__attribute__((optimize"):
            assert bad not in code, (path.name, bad)
        fma_sites = len(re.findall(r"__builtin_fmaf\s*\(", code))
        assert fma_sites == (2 if path.name == "dtl_numerics.h" else 0), (path.name, fma_sites)


_PROBE = r"""
#include <hip/hip_runtime.h>
typedef float f2 __attribute__((ext_vector_type(2)));
__global__ void probe_madd(const float* a, const float* b, float* c) {
  int i = threadIdx.x;
  c[i] = a[i] * b[i] + c[i];
}
__global__ void probe_pk(const f2* a, const f2* b, f2* c) {
  int i = threadIdx.x;
  c[i] = a[i] * b[i] + c[i];
}
"""


def test_checks_catch_planted_violations(tmp_path):
    """The checks above reject what they exist to reject: a multiply-add
    compiled with contraction allowed, and packed FP32 selected when the
    packed-ops feature is left on."""
    src = tmp_path / "probe.hip"
    src.write_text(_PROBE)
    cc = B.hipcc()

    def compile_(flags, kind):
        out = tmp_path / f"probe.{kind}"
        extra = ["-emit-llvm", "-S"] if kind == "ll" else ["-S"]
        subprocess.run([cc, f"--offload-arch={B.ARCH}", "-O3", "--cuda-device-only", *flags, *extra, str(src),
                        "-o", str(out)], check=True, capture_output=True)
        return out.read_text()

    fast = [f for f in B.NUMERIC_FLAGS if f != "-ffp-contract=off"] + ["-ffp-contract=fast"]
    ir = compile_(fast, "ll")
    assert "@llvm.fmuladd" in ir or _FM_FLAG.search(ir) is not None
    ir = compile_(B.NUMERIC_FLAGS, "ll")
    assert "@llvm.fmuladd" not in ir and _FM_FLAG.search(ir) is None

    no_pk_flag = [f for f in B.NUMERIC_FLAGS if f not in ("-Xclang", "-target-feature", "-packed-fp32-ops")]
    assert _PACKED_F32.search(compile_(no_pk_flag, "s")) is not None
    assert _PACKED_F32.search(compile_(B.NUMERIC_FLAGS, "s")) is None
