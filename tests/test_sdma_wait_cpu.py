"""The copy-engine wait gives up at its deadline instead of hanging.

Builds tests/native/sdma_wait_check.cpp with g++ against
flexkv_amd/csrc/kv_wait.h (header-only, no HIP) and runs it: stub signals
that complete, an interrupt signal and a polled signal that never do, an
empty half, and the host-row ledger of a device-to-host transfer whose
halves stall (the host blocks their copies write are reported unsafe).  No
device is involved.
"""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_bounded_sdma_wait(tmp_path):
    exe = tmp_path / "sdma_wait_check"
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", "-I", os.path.join(ROOT, "flexkv_amd", "csrc"),
           "-I", "/opt/rocm/include", os.path.join(ROOT, "tests", "native", "sdma_wait_check.cpp"),
           "-o", str(exe), "-lpthread"]
    build = subprocess.run(cmd, capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "FAIL" not in res.stdout
    assert res.stdout.count("ok:") == 14
