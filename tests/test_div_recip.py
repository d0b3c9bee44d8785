"""Division by reciprocal and fma correction (div_recip in
detllm_amd/csrc/dtl_numerics.h) against correctly rounded division, on the
host: tests/div_recip_check.c compares both over its caller's operands (the
Q8A quantiser: every third float dividend for four scales, 2^24 random
pairs of both signs, every seventh scale for the scale's own division)."""
import shutil
import subprocess

import pytest


def test_div_recip_matches_division(tmp_path):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    src = __file__.replace("test_div_recip.py", "div_recip_check.c")
    exe = tmp_path / "div_recip_check"
    subprocess.run([cc, "-O2", "-ffp-contract=off", src, "-o", str(exe), "-lm"], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stdout + res.stderr
    assert " 0 mismatches" in res.stdout
