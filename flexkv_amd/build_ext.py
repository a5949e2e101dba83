"""Compile libflexkv_hip.so in-tree with hipcc for gfx950, the hbm_ceiling
program that measures the device's plain read / write / copy rates
(bench.py reports them beside the gather's roofline), and the call_latency
program that times small fkv_transfer_kv_blocks calls against the launch
floors beside them, libresident_probe.so (a kernel that only occupies compute
units, which bench.py runs beside GEMMs), and the CPython module _fkv_py (host
C++ against torch's headers, built with g++) that carries
c_ext.transfer_kv_blocks' per-call path.

    python -m flexkv_amd.build_ext
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SOURCES = [os.path.join(HERE, "csrc", f)
           for f in ("kv_transfer.hip", "kv_host.cpp", "kv_sdma.cpp", "kv_ssd.cpp",
                     "kv_tp_group.cpp")]
OUT = os.path.join(HERE, "libflexkv_hip.so")
CEILING_SOURCE = os.path.join(HERE, "csrc", "hbm_ceiling.hip")
CEILING_OUT = os.path.join(HERE, "hbm_ceiling")
LATENCY_SOURCE = os.path.join(HERE, "csrc", "call_latency.hip")
LATENCY_OUT = os.path.join(HERE, "call_latency")
PROBE_SOURCE = os.path.join(HERE, "csrc", "resident_probe.hip")
PROBE_OUT = os.path.join(HERE, "libresident_probe.so")
PY_SOURCE = os.path.join(HERE, "csrc", "py_fastcall.cpp")
PY_OUT = os.path.join(HERE, "_fkv_py" + sysconfig.get_config_var("EXT_SUFFIX"))
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


def probe_command() -> list:
    return [hipcc(), f"--offload-arch={ARCH}", *COMMON, "-fPIC", "-shared", PROBE_SOURCE,
            "-o", PROBE_OUT + ".tmp"]


def py_command() -> list:
    import torch
    tdir = os.path.dirname(os.path.abspath(torch.__file__))
    tlib = os.path.join(tdir, "lib")
    abi = int(bool(torch._C._GLIBCXX_USE_CXX11_ABI))
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-Wall", "-fPIC", "-shared",
            f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__",
            "-I", sysconfig.get_paths()["include"], "-I", os.path.join(tdir, "include"),
            "-I", os.path.join(tdir, "include", "torch", "csrc", "api", "include"),
            "-I", os.path.join(rocm, "include"),
            PY_SOURCE, "-o", PY_OUT + ".tmp", "-L", tlib, "-ltorch_python", "-lc10", "-lc10_hip",
            f"-Wl,-rpath,{tlib}"]


def _run(cmd: list, out: str, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{os.path.basename(cmd[0])} failed ({res.returncode}):\n"
                           f"{res.stdout}\n{res.stderr}")
    os.replace(out + ".tmp", out)


def build(verbose: bool = False) -> str:
    _run(command(), OUT, verbose)
    _run(ceiling_command(), CEILING_OUT, verbose)
    _run(latency_command(), LATENCY_OUT, verbose)
    _run(probe_command(), PROBE_OUT, verbose)
    _run(py_command(), PY_OUT, verbose)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
