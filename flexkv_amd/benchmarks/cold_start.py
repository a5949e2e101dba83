"""First-transfer cost of the copy-engine path in a fresh process.

Each run starts a child process that sets up the Llama-3-8B KV workload of
bench.py (32 layers, 1024 random blocks, 2 GiB per op, pinned block-wise host
cache) and times its first three copy-engine D2H and H2D transfers, with or
without fkv_prepare first; the parent touches no GPU.  Prints one JSON line:

    python -m flexkv_amd.benchmarks.cold_start [--runs 2]
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))


def child(prepare: bool) -> dict:
    sys.path.insert(0, ROOT)
    import torch

    import bench
    from flexkv_amd import _lib
    wl = bench.Workload("llama3-8b", 1001)
    torch.cuda.synchronize()
    out = {"prepare": prepare}
    if prepare:
        t0 = time.perf_counter()
        _lib.prepare(torch.cuda.current_device())
        out["prepare_ms"] = round((time.perf_counter() - t0) * 1e3, 2)

    def timed(h2d: bool) -> float:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        wl.transfer(h2d, True)
        return round((time.perf_counter() - t0) * 1e3, 2)
    out["d2h_ms"] = [timed(False) for _ in range(3)]
    out["h2d_ms"] = [timed(True) for _ in range(3)]
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--runs", type=int, default=2, help="fresh processes per mode")
    ap.add_argument("--child", choices=["cold", "prepared"], help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.child:
        print(json.dumps(child(args.child == "prepared")), flush=True)
        return 0
    runs = []
    for _ in range(args.runs):
        for mode in ("cold", "prepared"):
            res = subprocess.run([sys.executable, "-m", "flexkv_amd.benchmarks.cold_start",
                                  "--child", mode], cwd=ROOT, capture_output=True, text=True,
                                 timeout=300)
            if res.returncode != 0:
                print(res.stderr[-2000:], file=sys.stderr)
                return res.returncode
            runs.append(json.loads(res.stdout.strip().splitlines()[-1]))
    print(json.dumps({"cold_start": runs,
                      "what": "first three copy-engine D2H and H2D transfers (2 GiB each, "
                              "Llama-3-8B KV shape) in fresh processes, without and with "
                              "fkv_prepare first"}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
