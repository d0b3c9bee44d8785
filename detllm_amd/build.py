"""Builds libdetllm_amd.so (gfx950 HIP kernels + C ABI) in-tree.

Usage: python -m detllm_amd.build   (or detllm_amd.build.build_library()).

Numeric flags are part of the contract: -ffp-contract=off keeps every
multiply and add separately rounded (the reference forbids FMA), the
correctly-rounded f32 divide/sqrt stays on, denormals stay enabled, and
packed-FP32 instruction selection is disabled.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_build"
LIB_NAME = "libdetllm_amd.so"
STATIC_LIB_NAME = "libdetllm_amd.a"
ARCH = os.environ.get("DETLLM_AMD_ARCH", "gfx950")

SOURCES = [
    "dtl_kernels.hip",
    "dtl_gemm.hip",
    "dtl_gemv.hip",
    "dtl_api.hip",
    "dtl_mfp.hip",
    "dtl_gguf.cpp",
    "dtl_range.cpp",
    "dtl_token.cpp",
    "dtl_codec.cpp",
]

NUMERIC_FLAGS = [
    "-ffp-contract=off",
    "-fno-fast-math",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

# Per-source additions: the MFMA-product GEMMs take their results in VGPRs
# (the VALU adds read them; in accumulation registers each would need a copy).
EXTRA_FLAGS = {
    "dtl_mfp.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: a ROCm toolchain is required to build detllm_amd")


def _run(cmd, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"{Path(cmd[0]).name} failed with exit code {res.returncode}: {' '.join(cmd[-3:])}")


def build_library(verbose: bool = False, jobs: int = 0) -> Path:
    """Compiles every source (one hipcc per file, in parallel), links them
    into one shared library and archives the same objects as the static
    library libdetllm_amd.a; returns the shared library's path.

    The archive's objects are ordinary (non-relocatable-device-code) HIP
    objects: each carries its own gfx950 code object and registers it from
    a static constructor, so a host linker pulling them from the archive
    needs only -lamdhip64 and the C++ runtime beside it."""
    OUT_DIR.mkdir(exist_ok=True)
    out = OUT_DIR / LIB_NAME
    tmp = OUT_DIR / (LIB_NAME + ".tmp")
    common = [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", *NUMERIC_FLAGS,
              "-Wno-unused-result"]
    objs = [OUT_DIR / (Path(s).stem + ".o") for s in SOURCES]
    cmds = [common + EXTRA_FLAGS.get(s, []) + ["-c", str(CSRC / s), "-o", str(o)]
            for s, o in zip(SOURCES, objs)]
    jobs = jobs or min(len(cmds), os.cpu_count() or 1, 16)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        for f in [ex.submit(_run, c, verbose) for c in cmds]:
            f.result()
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *[str(o) for o in objs], "-o", str(tmp)],
         verbose)
    os.replace(tmp, out)
    archive = OUT_DIR / STATIC_LIB_NAME
    archive_tmp = OUT_DIR / (STATIC_LIB_NAME + ".tmp")
    archive_tmp.unlink(missing_ok=True)
    _run(["ar", "rcs", str(archive_tmp), *[str(o) for o in objs]], verbose)
    os.replace(archive_tmp, archive)
    return out


if __name__ == "__main__":
    path = build_library(verbose=True)
    print(path)
