"""One results table from a full `bench.py` run: profiles/results.md.

    python bench.py > bench.json
    python -m flexkv_amd.benchmarks.results_table bench.json [--out profiles/results.md]

Every figure in the table is read from the bench's JSON line.
profiles/results.json keeps the line the committed table was made from.
"""
from __future__ import annotations

import argparse
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
HBM_PEAK = 8000.0


def _f(x, nd=1):
    return "—" if x is None else f"{x:.{nd}f}"


def _pair(d, a, b, nd=1):
    if not d:
        return "—"
    return f"{_f(d.get(a), nd)} / {_f(d.get(b), nd)}"


def _frac(d, a, b):
    if not d:
        return "—"
    return f"{_f(d.get(a), 3)} / {_f(d.get(b), 3)}"


def config_rows(cfg: dict) -> list:
    names = [("cfg0_plumbing", "cfg0 CPU-plumbing shape (16 MiB)"),
             ("cfg1_llama3-8b", "cfg1 Llama-3-8B (2 GiB)"),
             ("cfg1_llama3-8b_layerwise_host", "cfg1 on a layer-wise host cache"),
             ("cfg3_llama3-70b-tp8", "cfg3 Llama-3-70B TP-8 shard (1.25 GiB)"),
             ("cfg4_mla-dsv3", "cfg4 MLA DeepSeek-V3 (8.6 GiB)")]
    rows = []
    for key, label in names:
        c = cfg.get(key)
        if not c:
            continue
        ce, k, dg = c.get("ce", {}), c.get("kernel", {}), c.get("device_gather", {})
        moved = ce.get("d2h_moved_by")
        ce_cell = _pair(ce, "d2h_gbps", "h2d_gbps") + (" (zero-copy kernel by policy)" if moved
                                                        else "")
        pieces = "—"
        if "gather_piece_frac_hbm" in ce:
            pieces = _frac(ce, "gather_piece_frac_hbm", "scatter_piece_frac_hbm")
        rows.append(f"| {label} | {ce_cell} | {_frac(ce, 'd2h_frac_link', 'h2d_frac_link')} | "
                    f"{_pair(k, 'd2h_gbps', 'h2d_gbps')} | {pieces} | "
                    f"{_frac(dg, 'gather_frac_hbm', 'scatter_frac_hbm')} | "
                    f"{'yes' if c.get('bit_exact') else 'no'} |")
        if "ce_rect_copies" in c:
            r = c["ce_rect_copies"]
            rows.append(f"| … rect copies (`layerwise_scattered=\"rect_copies\"`) | "
                        f"{_pair(r, 'd2h_gbps', 'h2d_gbps')} | "
                        f"{_frac(r, 'd2h_frac_link', 'h2d_frac_link')} | — | "
                        f"{_frac(r, 'gather_piece_frac_hbm', 'scatter_piece_frac_hbm')} | — | — |")
    frag = cfg.get("cfg2_llama3-8b_fragmentation", {})
    for run, c in frag.items():
        ce, k = c.get("ce", {}), c.get("kernel", {})
        rows.append(f"| cfg2 Llama-3-8B, id runs of {run.split('_')[1]} | "
                    f"{_pair(ce, 'd2h_gbps', 'h2d_gbps')} | "
                    f"{_frac(ce, 'd2h_frac_link', 'h2d_frac_link')} | "
                    f"{_pair(k, 'd2h_gbps', 'h2d_gbps')} | "
                    f"{_frac(ce, 'gather_piece_frac_hbm', 'scatter_piece_frac_hbm')} | — | "
                    f"{'yes' if c.get('bit_exact') else 'no'} |")
    return rows


def overlap_rows(o: dict, label: str) -> list:
    rows = []
    tf = o.get("transfer_first", {})
    for key in sorted(k for k in o if k.startswith(("d2h", "h2d"))):
        a, b = o[key], tf.get(key, {})
        rows.append(f"| {label} | {key} | {_f(a.get('transfer_gbps'), 1)} | "
                    f"{_f(a.get('gemm_slowdown'), 3)} | {_f(b.get('gemm_slowdown'), 3)} |")
    if "resident_spin" in o:
        rows.append(f"| {label} | one-thread spin kernel (no memory access) | — | "
                    f"{_f(o['resident_spin'].get('gemm_slowdown'), 3)} | "
                    f"{_f(tf.get('resident_spin', {}).get('gemm_slowdown'), 3)} |")
    for key, what in (("resident_sleep_1wave", "one sleeping wavefront (no memory access)"),
                      ("resident_sleep_256wg", "256 sleeping workgroups of 256 threads")):
        if key in o:
            rows.append(f"| {label} | {what} | — | {_f(o[key].get('gemm_slowdown'), 3)} | "
                        f"{_f(tf.get(key, {}).get('gemm_slowdown'), 3)} |")
    return rows


def _traffic_row(r: dict) -> str:
    alg = r["algorithmic_bytes_per_launch"]
    t = r.get("traffic")
    if not t:
        why = r.get("traffic_source", "no counter profile")
        return f"| HBM traffic per gather launch (counters) | — ({why}) |"
    return (f"| HBM traffic per gather launch (counters) | {t} B for {alg} algorithmic "
            f"(ratio {t / alg:.4f}) |")


def _ceiling_row(r: dict) -> str:
    c = r.get("device_ceilings")
    if not c:
        return "| Device ceilings | — |"
    return (f"| Device ceilings: read only / write only / plain copy (16 B per lane, 4 GiB) | "
            f"{_f(c.get('read_gbps'))} / {_f(c.get('write_gbps'))} / {_f(c.get('copy_gbps'))} "
            f"GB/s; gather / scatter at {_f(c.get('gather_frac_of_copy'), 3)} / "
            f"{_f(c.get('scatter_frac_of_copy'), 3)} of the copy |")


def table(p: dict, label: str) -> str:
    r = p["roofline"]
    hl = p.get("host_link", {})
    cpu = p.get("cpu_baseline", {})
    L = [f"# Results ({label})", "",
         "Generated from one full `python bench.py` run on one MI355X by",
         "`python -m flexkv_amd.benchmarks.results_table <bench.json>`. GB/s are 10^9 B/s.", "",
         "## Headline", "",
         "| Figure | Value |", "|---|---|",
         f"| D2H, default path (copy engines), Llama-3-8B step | {p['value']} GB/s "
         f"({_f(hl.get('d2h_frac'), 3)} of the measured link, "
         f"{_f(hl.get('d2h_frac_pcie_gen5_x16'), 3)} of nominal PCIe Gen5 x16) |",
         f"| H2D, default path | {_f(p['h2d']['gbps'], 2)} GB/s ({_f(hl.get('h2d_frac'), 3)} "
         f"of the link) |",
         f"| Measured link peak D2H / H2D (1 GiB contiguous pinned copy) | "
         f"{_f(hl.get('d2h_peak_gbps_measured'), 2)} / {_f(hl.get('h2d_peak_gbps_measured'), 2)} "
         f"GB/s |",
         f"| Device gather (roofline kernel), 2 GiB in one launch | {_f(r['achieved'])} GB/s of "
         f"HBM = {_f(r['frac'], 4)} of 8 TB/s; {r['avg_launch_ms']} ms per launch |",
         f"| Device scatter, same | {_f(r['scatter']['achieved'])} GB/s = "
         f"{_f(r['scatter']['frac'], 4)} |",
         f"| Gather / scatter pieces inside the copy-engine transfers | "
         f"{_f(r['in_path']['gather']['frac'], 4)} / {_f(r['in_path']['scatter']['frac'], 4)} "
         f"of 8 TB/s |" if r.get("in_path") else "| In-path pieces | — |",
         _traffic_row(r),
         _ceiling_row(r),
         f"| CPU baseline ({cpu.get('kind')}, {cpu.get('cores')} threads) | "
         f"{cpu.get('value')} GB/s; one thread {cpu.get('single_thread_gbps')} GB/s |",
         f"| Reference copy-engine loop (one copy per chunk) | "
         f"{_f(p.get('ce_per_chunk_loop', {}).get('gbps'), 2)} GB/s |", "",
         "## Benchmark configurations", "",
         "Fractions of the link are of the measured per-direction peak; piece and device",
         "fractions are of the 8 TB/s HBM peak.", "",
         "| Configuration | Copy-engine D2H / H2D GB/s | of link | Zero-copy D2H / H2D GB/s | "
         "Pieces gather / scatter | Device gather / scatter | Bit-exact |",
         "|---|---|---|---|---|---|---|"]
    L += config_rows(p.get("configs", {}))
    mla = p.get("configs", {}).get("cfg4_mla-dsv3", {}).get("request_batch")
    if mla:
        L += ["", f"MLA request mix ({mla['requests']} requests, {mla['blocks']} blocks): copy "
              f"engines per request {mla['ce']['d2h_per_request_gbps']} / "
              f"{mla['ce']['h2d_per_request_gbps']} GB/s, batched "
              f"{mla['ce']['d2h_batched_gbps']} / {mla['ce']['h2d_batched_gbps']} GB/s "
              f"(D2H / H2D)."]
    tpg = p.get("configs", {}).get("cfg3_llama3-70b-tp8_group")
    if tpg:
        L += ["", f"Llama-3-70B TP-8 group on this GPU ({tpg['ranks']} ranks sharing its link, "
              f"{tpg['bytes_per_op'] / 2**30:.0f} GiB per op, zero-copy kernel): group "
              f"{tpg['group_d2h_gbps']} / {tpg['group_h2d_gbps']} GB/s "
              f"({tpg['group_d2h_frac_link']} / {tpg['group_h2d_frac_link']} of the link), "
              f"the ranks' calls in turn {tpg['ranks_in_turn_d2h_gbps']} / "
              f"{tpg['ranks_in_turn_h2d_gbps']} GB/s (D2H / H2D); bit-exact "
              f"{'yes' if tpg.get('bit_exact') else 'no'}."]
    L += ["", "## Beside compute", "",
          "160 bf16 GEMMs [8192x4096]x[4096x4096] beside one 2 GiB transfer, against the same",
          "GEMMs alone started the same way. `h2d_kernel_spread`: the zero-copy H2D with its",
          "grid spread over the chip (`transfer_cus` = CUs / 8, about one workgroup per CU)",
          "instead of the automatic 8 CUs' worth.", "",
          "| Host cache | Path | Transfer GB/s | GEMMs first | Transfer first |",
          "|---|---|---|---|---|"]
    L += overlap_rows(p.get("overlap_with_compute", {}), "block-wise")
    lw = p.get("configs", {}).get("cfg1_llama3-8b_layerwise_host", {}).get(
        "overlap_with_compute")
    if lw:
        L += overlap_rows(lw, "layer-wise")
    lh = p.get("layerwise_h2d", {})
    if lh:
        L += ["", "## Layer-wise asynchronous H2D (one layer per group)", "",
              "| Handle | GB/s | First group ms | Overlapped prefill ms (bound) | "
              "GEMMs beside, GEMMs first / handle first |", "|---|---|---|---|---|"]
        for k in ("kernel", "ce"):
            h = lh.get(k, {})
            L.append(f"| {k} | {_f(h.get('async_gbps'), 2)} | {_f(h.get('async_first_group_ms'), 2)}"
                     f" | {_f(h.get('layerwise_overlapped_ms'), 2)} "
                     f"({_f(h.get('bound_transfer_plus_one_layer_ms'), 2)}) | "
                     f"{_f(h.get('gemm_slowdown'), 3)} / "
                     f"{_f(h.get('gemm_slowdown_transfer_first'), 3)} |")
    du = p.get("duplex", {})
    ep = p.get("engine_put_get", {})
    wo = p.get("worker_ops", {})
    L += ["", "## Other measurements", "", "| Figure | Value |", "|---|---|"]
    if du:
        peak = hl.get("duplex_peak_gbps_measured")
        L.append(f"| D2H and H2D at once, copy engines / zero-copy | "
                 f"{du.get('ce_aggregate_gbps')} / {du.get('kernel_aggregate_gbps')} GB/s"
                 + (f" ({du.get('ce_frac_duplex_peak')} / {du.get('kernel_frac_duplex_peak')} of "
                    f"{peak} GB/s, two 1 GiB runtime copies at once)" if peak else "") + " |")
    if ep:
        L.append(f"| TransferEngine put / get / both | {ep['put']['gbps']} / {ep['get']['gbps']} / "
                 f"{ep['put_and_get']['gbps']} GB/s |")
    for key, lab in (("thread_ce", "thread worker, copy engines"),
                     ("thread_kernel", "thread worker, zero-copy"),
                     ("process_ce", "spawned worker, copy engines"),
                     ("process_kernel", "spawned worker, zero-copy")):
        w = wo.get(key)
        if w:
            L.append(f"| 16-block worker ops, {lab} (D2H / H2D) | {w['d2h_16blk']['gbps']} / "
                     f"{w['h2d_16blk']['gbps']} GB/s |")
    cl = p.get("call_latency_c_abi") or {}
    if cl:
        L.append(f"| One block, one layer through the C-ABI (D2H / H2D) | {cl.get('fkv_1x1_d2h_us')}"
                 f" / {cl.get('fkv_1x1_h2d_us')} µs (empty kernel with arguments "
                 f"{cl.get('args_kernel_us')} µs) |")
    cp = p.get("call_latency") or {}
    if cp:
        L.append(f"| Same from Python (D2H / H2D) | {cp.get('zc_1blk_1layer_d2h_us')} / "
                 f"{cp.get('zc_1blk_1layer_h2d_us')} µs |")
    ssd = p.get("ssd_tier") or {}
    if ssd.get("threads"):
        L.append(f"| Host cache ⇄ SSD, threads: write (fsync) / random read | "
                 f"{ssd['threads']['write_gbps_with_fsync']} / "
                 f"{ssd['threads']['read_gbps_random_host_blocks']} GB/s (disk "
                 f"{ssd['disk']['seq_write_gbps_with_fsync']} / {ssd['disk']['seq_read_gbps']}) |")
    if ssd.get("io_uring"):
        L.append(f"| Host cache ⇄ SSD, io_uring: write (fsync) / random read | "
                 f"{ssd['io_uring']['write_gbps_with_fsync']} / "
                 f"{ssd['io_uring']['read_gbps_random_host_blocks']} GB/s |")
    L.append(f"| Every moved block bit-exact (whole run) | {'yes' if p.get('bit_exact') else 'no'} |")
    if "procs_at_end" in p:
        L.append(f"| Helper processes left at exit | {p['procs_at_end']} |")
    L.append("")
    return "\n".join(L)


def load(path: str) -> dict:
    """The bench's result: a file holding the JSON object, or bench.py's
    output with the JSON line last."""
    with open(path) as fh:
        text = fh.read()
    try:
        return json.loads(text)
    except json.JSONDecodeError:
        lines = [ln for ln in text.splitlines() if ln.strip().startswith("{")]
        return json.loads(lines[-1])


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("bench_json")
    ap.add_argument("--out", default=os.path.join(ROOT, "profiles", "results.md"))
    ap.add_argument("--label", default="one MI355X")
    args = ap.parse_args()
    with open(args.out, "w") as fh:
        fh.write(table(load(args.bench_json), args.label))
    print(args.out)
    return 0


if __name__ == "__main__":
    sys.exit(main())
