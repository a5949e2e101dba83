"""Compile libflexkv_hip.so in-tree with hipcc for gfx950, the hbm_ceiling
program that measures the device's plain read / write / copy rates
(bench.py reports them beside the gather's roofline), and the call_latency
program that times small fkv_transfer_kv_blocks calls against the launch
floors beside them.

    python -m flexkv_amd.build_ext
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SOURCES = [os.path.join(HERE, "csrc", f)
           for f in ("kv_transfer.hip", "kv_host.cpp", "kv_sdma.cpp", "kv_ssd.cpp")]
OUT = os.path.join(HERE, "libflexkv_hip.so")
CEILING_SOURCE = os.path.join(HERE, "csrc", "hbm_ceiling.hip")
CEILING_OUT = os.path.join(HERE, "hbm_ceiling")
LATENCY_SOURCE = os.path.join(HERE, "csrc", "call_latency.hip")
LATENCY_OUT = os.path.join(HERE, "call_latency")
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


# no packed fp32 instructions anywhere in device code
COMMON = ["-O3", "-std=c++17", "-Wall", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def command() -> list:
    return [
        hipcc(), f"--offload-arch={ARCH}", *COMMON, "-fPIC", "-shared",
        "-I", os.path.join(ROOT, "include"),
        *SOURCES, "-o", OUT + ".tmp", "-ldl",
    ]


def ceiling_command() -> list:
    return [hipcc(), f"--offload-arch={ARCH}", *COMMON, CEILING_SOURCE, "-o", CEILING_OUT + ".tmp"]


def latency_command() -> list:
    return [hipcc(), f"--offload-arch={ARCH}", *COMMON, "-I", os.path.join(ROOT, "include"),
            LATENCY_SOURCE, "-o", LATENCY_OUT + ".tmp", "-L", HERE, "-lflexkv_hip",
            "-Wl,-rpath,$ORIGIN"]


def _run(cmd: list, out: str, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    os.replace(out + ".tmp", out)


def build(verbose: bool = False) -> str:
    _run(command(), OUT, verbose)
    _run(ceiling_command(), CEILING_OUT, verbose)
    _run(latency_command(), LATENCY_OUT, verbose)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
