"""exp_clamped restated for non-positive arguments (detllm_amd/csrc/
dtl_numerics.h) against the general expf_det path, on the host:
tests/exp_nonpos_check.c compares both for every float t <= 0 (all 2^31
patterns with the sign bit set, and +0).  The device function itself is
checked against the oracle's exp_f32 by
tests/test_gpu_kernels.py::test_exp_clamped_device_matches_oracle."""
import shutil
import subprocess

import pytest


def test_exp_nonpos_matches_expf(tmp_path):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    src = __file__.replace("test_exp_nonpos.py", "exp_nonpos_check.c")
    exe = tmp_path / "exp_nonpos_check"
    subprocess.run([cc, "-O2", "-fopenmp", "-ffp-contract=off", src, "-o", str(exe), "-lm"], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stdout + res.stderr
    assert " 0 mismatches" in res.stdout
