"""The static library: a C host linked against libdetllm_amd.a through
include/detllm.h (as a Rust `build.rs` would link `static=detllm_amd`,
`dylib=amdhip64`, `dylib=stdc++`), calling host-only entry points.

Its range-coder payload must equal the oracle's (det-coder range.rs:30-92
restated) on the same triples and decode back; the header, window schedule,
uniform range and status strings must equal the shared library's.  No GPU
call is made.
"""
import ctypes as C
import shutil
import subprocess
from pathlib import Path

import pytest

import detref
from detllm_amd import build as B
from detllm_amd._lib import lib

ROOT = Path(__file__).resolve().parents[1]
ROCM_LIB = Path("/opt/rocm/lib")


def _lcg_triples(n, seed):
    """The generator of tests/static_link_check.c, restated."""
    s = seed
    mask = (1 << 64) - 1

    def nxt():
        nonlocal s
        s = (s * 6364136223846793005 + 1442695040888963407) & mask
        return s >> 17

    out = []
    for _ in range(n):
        t = 2 + nxt() % ((1 << 31) - 2)
        c = nxt() % t
        room = t - c
        f = 1 + nxt() % min(room, 4096)
        out.append((c, f, t))
    return out


@pytest.fixture(scope="module")
def static_prog(tmp_path_factory):
    archive = B.OUT_DIR / B.STATIC_LIB_NAME
    if not archive.exists():
        pytest.fail(f"{archive} is missing: build() produces it beside the shared library")
    if shutil.which("gcc") is None or shutil.which("g++") is None:
        pytest.skip("gcc/g++ not available")
    d = tmp_path_factory.mktemp("static")
    obj, exe = d / "check.o", d / "check"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-O2", f"-I{ROOT / 'include'}", "-c",
                    str(ROOT / "tests" / "static_link_check.c"), "-o", str(obj)], check=True)
    subprocess.run(["g++", str(obj), str(archive), f"-L{ROCM_LIB}", "-lamdhip64",
                    f"-Wl,-rpath,{ROCM_LIB}", "-o", str(exe)], check=True)
    # the archive, not the shared library, provides the entry points
    ldd = subprocess.run(["ldd", str(exe)], capture_output=True, text=True, check=True).stdout
    assert "libdetllm_amd" not in ldd
    return exe


def _run(exe, *args):
    res = subprocess.run([str(exe), *map(str, args)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    out = {}
    for line in res.stdout.splitlines():
        key, _, rest = line.partition(" ")
        assert key != "FAIL", line
        out.setdefault(key, []).append(rest)
    return out


@pytest.mark.parametrize("n,seed", [(0, 1), (1, 2), (1000, 7), (20000, 11)])
def test_static_range_coder_matches_oracle(static_prog, n, seed):
    out = _run(static_prog, n, seed)
    want = detref.range_encode(_lcg_triples(n, seed))
    assert bytes.fromhex(out["payload"][0]) == want
    assert out["roundtrip"] == [f"ok {n}"]
    assert out["zero_freq_status"] == ["30"]


def test_static_header_schedule_and_strings_match_shared_library(static_prog):
    out = _run(static_prog, 4, 3)
    sha = bytes((3 * i + 1) & 0xFF for i in range(32))
    hdr = (C.c_uint8 * 56)()
    assert lib.dtl_dtlz_header_encode(1, (C.c_uint8 * 32)(*sha), 2048, 512, 1048576, hdr) == 0
    assert bytes.fromhex(out["header"][0]) == bytes(hdr)
    assert out["header_fields"] == ["1 2048 512 1048576 1"]
    assert out["bad_magic_status"] == ["81"]

    ws, want = 0, []
    for pos in range(20):
        ws = detref.next_window_start(pos, ws, 8, 2)
        want.append(str(ws))
    assert out["windows"] == [" ".join(want)]

    assert out["uniform"] == ["0 300 1 512"]
    for line in out["status"]:
        code, _, text = line.partition(" ")
        assert text == lib.dtl_status_string(int(code)).decode()
