"""The device ceiling program (flexkv_amd/csrc/hbm_ceiling.hip) that bench.py
runs before it touches the GPU: it prints one JSON line whose best rates are
the maxima of its runs, and refuses buffers below 64 MiB."""
import json
import os
import subprocess

import pytest

EXE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "flexkv_amd",
                   "hbm_ceiling")


@pytest.mark.gpu
def test_ceiling_program_reports_consistent_rates():
    assert os.path.exists(EXE), "build first: python -c 'import __graft_entry__ as g; g.build()'"
    res = subprocess.run([EXE, str(64 << 20)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stderr
    out = json.loads(res.stdout.strip().splitlines()[-1])
    assert out["bytes"] == 64 << 20 and out["cus"] > 0
    for kind in ("read", "write", "copy"):
        rates = [r["gbps"] for r in out["runs"] if r["kind"] == kind]
        assert rates and out[f"{kind}_gbps"] == max(rates) > 0


def test_ceiling_program_refuses_small_buffers():
    if not os.path.exists(EXE):
        pytest.skip("hbm_ceiling not built")
    res = subprocess.run([EXE, str(1 << 20)], capture_output=True, text=True, timeout=60)
    assert res.returncode == 2 and "64 MiB" in res.stderr
