"""Memory-traffic profile of the transfer kernels from two rocprofv3 PMC
passes over `bench.py --counters` (one with FETCH_SIZE, one with
WRITE_SIZE), written to profiles/kv_gather_<workload>_counters.{json,md}.
bench.py reads the JSON for its roofline line's `traffic`, when the profile
was taken with the current kernel source.

    cd /tmp && export TMPDIR=/tmp
    rocprofv3 --pmc FETCH_SIZE -f csv -d <fetch> -o pmc -- python <repo>/bench.py --counters --workload W
    rocprofv3 --pmc WRITE_SIZE -f csv -d <write> -o pmc -- python <repo>/bench.py --counters --workload W
    python -m flexkv_amd.benchmarks.counter_profile <fetch>/..._counter_collection.csv \\
        <write>/..._counter_collection.csv --workload W

The run's dispatches in order: a plain 1 GiB device copy (calibration: a
copy of known size reads and writes 1 GiB, which fixes each counter's
scale), 3 device gathers, 3 device scatters, 3 zero-copy D2H and 3
zero-copy H2D transfers of the workload's step, then one copy-engine D2H and
one H2D, whose gather and scatter pieces are summed per transfer.
"""
from __future__ import annotations

import argparse
import csv
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

DESC = {
    "llama3-8b": ("Llama-3-8B KV shape",
                  "1024 blocks x 32 layers x K/V x 32 KiB = 2 GiB moved per launch", 2147483648),
    "llama3-70b-tp8": ("Llama-3-70B TP-8 shard KV shape",
                       "2048 blocks x 80 layers x K/V x 4 KiB = 1.25 GiB moved per launch",
                       1342177280),
    "mla-dsv3": ("MLA latent (DeepSeek-V3) shape",
                 "2048 blocks x 61 layers x 72 KiB = 8.6 GiB moved per launch", 9210691584),
}
CAL_BYTES = 1 << 30


def kind_of(name: str) -> str:
    """Which transfer kernel a dispatch is: staging gather / scatter,
    zero-copy D2H / H2D, or '' for anything else (the calibration copy,
    id staging, cache acquires, torch's own kernels)."""
    if "kv_pack_kernel<false" in name or "kv_pack_span_kernel<false" in name or \
            "kv_chunk_copy_kernel<false, true" in name:
        return "gather"
    if "kv_pack_kernel<true" in name or "kv_pack_span_kernel<true" in name or \
            "kv_chunk_copy_kernel<true, true" in name:
        return "scatter"
    if "kv_chunk_copy_kernel<false, false" in name or "kv_small_copy_kernel<false>" in name:
        return "zero_copy_d2h"
    if "kv_chunk_copy_kernel<true, false" in name or "kv_small_copy_kernel<true>" in name:
        return "zero_copy_h2d"
    return ""


def load(path: str, counter: str) -> list:
    rows = []
    with open(path) as fh:
        for r in csv.DictReader(fh):
            if r["Counter_Name"] == counter:
                rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
    return sorted(rows)


def summarize(fetch_csv: str, write_csv: str, workload: str) -> dict:
    fetch = load(fetch_csv, "FETCH_SIZE")
    write = load(write_csv, "WRITE_SIZE")
    if [d for d, _, _ in fetch] != [d for d, _, _ in write]:
        raise ValueError("the two passes saw different dispatches")
    pairs = [(n, f, w) for (_, n, f), (_, _, w) in zip(fetch, write)]
    cal = next(p for p in pairs if "copyBuffer" in p[0])
    fs = CAL_BYTES / (cal[1] * 1024)
    ws = CAL_BYTES / (cal[2] * 1024)
    moved = DESC[workload][2]
    alg = 2 * moved
    out = {"workload": f"{DESC[workload][0]}, {DESC[workload][1]}",
           "calibration": {"kernel": cal[0][:80], "bytes": CAL_BYTES, "fetch_kib": cal[1],
                           "write_kib": cal[2], "fetch_scale": round(fs, 4),
                           "write_scale": round(ws, 4)}}
    seen = {"gather": [], "scatter": [], "zero_copy_d2h": [], "zero_copy_h2d": []}
    pieces = {"ce_gather_pieces": [], "ce_scatter_pieces": []}
    for p in pairs:
        k = kind_of(p[0])
        if not k:
            continue
        if len(seen[k]) < 3:
            seen[k].append(p)
        elif k in ("gather", "scatter"):
            pieces["ce_" + k + "_pieces"].append(p)
    for k, g in seen.items():
        if len(g) != 3:
            raise ValueError(f"expected 3 {k} dispatches, found {len(g)}")
        fk = [x[1] for x in g]
        wk = [x[2] for x in g]
        rd = round(sum(fk) / 3 * 1024 * fs)
        wr = round(sum(wk) / 3 * 1024 * ws)
        out[k] = {"kernel": g[0][0][:160], "fetch_kib_per_dispatch": fk,
                  "write_kib_per_dispatch": wk, "read_bytes": rd, "write_bytes": wr,
                  "traffic_bytes_per_launch": rd + wr, "algorithmic_bytes_per_launch": alg,
                  "traffic_over_algorithmic": round((rd + wr) / alg, 4)}
    for k, g in pieces.items():
        fk = [x[1] for x in g]
        wk = [x[2] for x in g]
        rd = round(sum(fk) * 1024 * fs)
        wr = round(sum(wk) * 1024 * ws)
        out[k] = {"kernel": g[0][0][:160] if g else "", "pieces": len(g),
                  "fetch_kib_per_dispatch": fk, "write_kib_per_dispatch": wk,
                  "read_bytes_per_transfer": rd, "write_bytes_per_transfer": wr,
                  "algorithmic_bytes_per_transfer": alg,
                  "traffic_over_algorithmic": round((rd + wr) / alg, 4) if g else None}
    sys.path.insert(0, ROOT)
    import bench
    out["kernel_sha16"] = bench.kernel_section_sha16()
    return out


def markdown(out: dict, workload: str) -> str:
    title, desc, moved = DESC[workload]
    alg = 2 * moved
    wl_arg = f" --workload {workload}"
    short = {"gather": "gather (HBM → HBM)", "scatter": "scatter (HBM → HBM)",
             "zero_copy_d2h": "zero-copy D2H (HBM → host)",
             "zero_copy_h2d": "zero-copy H2D (host → HBM)"}
    cal = out["calibration"]
    L = [f"# Memory traffic of the transfer kernels, {title}", "",
         "Two PMC passes (one counter each) over `bench.py --counters`. It runs a 1 GiB plain",
         "device copy (calibration), then 3 device gathers, 3 device scatters, 3 zero-copy D2H",
         f"and 3 zero-copy H2D transfers, each of {desc}, then one copy-engine",
         "transfer each way:", "", "```", "cd /tmp && export TMPDIR=/tmp",
         "timeout -s KILL 150 rocprofv3 --pmc FETCH_SIZE -f csv -d <fetch> -o pmc -- "
         f"python /root/repo/bench.py --counters{wl_arg}",
         "timeout -s KILL 150 rocprofv3 --pmc WRITE_SIZE -f csv -d <write> -o pmc -- "
         f"python /root/repo/bench.py --counters{wl_arg}",
         "python -m flexkv_amd.benchmarks.counter_profile <fetch>/<...>_counter_collection.csv "
         f"<write>/<...>_counter_collection.csv{wl_arg}",
         "```", "", "| Kernel | Name | FETCH_SIZE (KiB) per dispatch | WRITE_SIZE (KiB) per dispatch |",
         "|---|---|---|---|",
         f"| calibration copy, 1 GiB | `{cal['kernel'][:40]}` | {cal['fetch_kib']:.1f} | "
         f"{cal['write_kib']:.1f} |"]
    for k in short:
        o = out[k]
        name = o["kernel"].replace("void (anonymous namespace)::", "").split("((")[0]
        L.append(f"| {short[k]} | `{name}` | "
                 f"{', '.join(f'{x:.1f}' for x in o['fetch_kib_per_dispatch'])} | "
                 f"{', '.join(f'{x:.1f}' for x in o['write_kib_per_dispatch'])} |")
    L += ["", "Scale factors from the calibration copy (a known 1 GiB read and 1 GiB written): "
          f"FETCH_SIZE x {cal['fetch_scale']:.4f}, WRITE_SIZE x {cal['write_scale']:.4f}.", "",
          "| Kernel | Read (bytes) | Written (bytes) | Traffic / launch | Algorithmic / launch "
          "| Ratio |", "|---|---|---|---|---|---|"]
    for k in short:
        o = out[k]
        L.append(f"| {short[k]} | {o['read_bytes']} | {o['write_bytes']} | "
                 f"{o['traffic_bytes_per_launch']} | {alg} | {o['traffic_over_algorithmic']:.4f} |")
    L += ["", "Copy-engine transfers (one each way): their gather and scatter pieces, summed per",
          "transfer:", "", "| Pieces | Count | Read (bytes) | Written (bytes) | Algorithmic | "
          "Ratio |", "|---|---|---|---|---|---|"]
    for k in ("ce_gather_pieces", "ce_scatter_pieces"):
        o = out[k]
        ratio = f"{o['traffic_over_algorithmic']:.4f}" if o["traffic_over_algorithmic"] else "—"
        L.append(f"| {k[3:].replace('_', ' ')} | {o['pieces']} | {o['read_bytes_per_transfer']} | "
                 f"{o['write_bytes_per_transfer']} | {alg} | {ratio} |")
    ratios = [out[k]["traffic_over_algorithmic"] for k in list(short) +
              ["ce_gather_pieces", "ce_scatter_pieces"] if out[k]["traffic_over_algorithmic"]]
    L += ["", f"Kernel source: sha256 prefix {out['kernel_sha16']} of "
          "`flexkv_amd/csrc/kv_transfer.hip` from its start to the end of the transfer kernels,",
          "comments and blank lines left out (`bench.kernel_section_sha16`).", "",
          f"Traffic over algorithmic bytes: {min(ratios):.4f}-{max(ratios):.4f}. The counters "
          "count requests to",
          "host memory as well as to HBM, so for the zero-copy kernels they also give the",
          f"host-link bytes ({moved} bytes per launch each way).", ""]
    return "\n".join(L)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("fetch_csv")
    ap.add_argument("write_csv")
    ap.add_argument("--workload", default="llama3-8b", choices=sorted(DESC))
    args = ap.parse_args()
    out = summarize(args.fetch_csv, args.write_csv, args.workload)
    base = os.path.join(ROOT, "profiles", f"kv_gather_{args.workload}_counters")
    with open(base + ".json", "w") as fh:
        json.dump(out, fh, indent=2)
    with open(base + ".md", "w") as fh:
        fh.write(markdown(out, args.workload))
    print(json.dumps({k: out[k]["traffic_over_algorithmic"] for k in out
                      if isinstance(out[k], dict) and "traffic_over_algorithmic" in out[k]}))
    return 0


if __name__ == "__main__":
    sys.exit(main())
