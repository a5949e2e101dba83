#!/usr/bin/env python3
"""KV-block transfer benchmark (GPU<->CPU) on one MI355X.

Default workload (Llama-3-8B KV shape): 32 layers, per-layer K/V device tensors
[2, 4096 blocks, 16 tokens, 8 kv heads, 128] bf16 ~N(0,1), pinned block-wise
host cache [16384, 32, 2, 16, 8, 128] bf16 (32 GiB); one step = one transfer
op of 1024 distinct random GPU block ids <-> 1024 distinct random host ids
(2 GiB).  `value` is D2H GB/s (1e9 B/s) of the default path; H2D is measured on
the same tensors and ids.  Bytes per op follow the reference's accounting,
chunk * layers * blocks * kv (flexkv/transfer/worker.py:334-335).

Also reported, in the same run: every transfer path, the measured host-link
peak (1 GiB contiguous pinned copies) and device-to-device copy rate, the
reference's one-DMA-per-chunk copy-engine loop, the host cache <-> SSD file
tier (write, fsync, O_DIRECT read, bit-exact), the CPU baseline (the oracle's
block-partitioned memcpy on this host's cores), a per-kernel roofline from
HIP events recorded by the library around each launch, and a bit-exact check
of every moved block.

    python bench.py [--steps K] [--warmup W] [--workload NAME] [--gpus 1]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import subprocess
import sys
import time

import torch

# per-op transfer logs of the workers would drown the bench's own lines
os.environ.setdefault("FLEXKV_LOG_LEVEL", "WARNING")

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "KV-block transfer GB/s D2H & H2D at Llama-3-8B shape; % of host-link/HBM peak"
HBM_PEAK_GBS = 8000.0
# PCIe Gen5 x16, per direction: 32 GT/s x 16 lanes x 128/130 line coding
PCIE_GEN5_X16_GBS = 63.0

WORKLOADS = {
    "plumbing": dict(layers=4, kv=2, ng=256, nh=512, tokens=16, heads=8, dim=128, n=64,
                     dtype="float16",
                     desc="CPU-plumbing shape: 4 layers, K/V [256,16,8,128] fp16 <-> host "
                          "[512,4,2,16,8,128]; 64 random distinct ids"),
    "llama3-8b": dict(layers=32, kv=2, ng=4096, nh=16384, tokens=16, heads=8, dim=128, n=1024,
                      desc="Llama-3-8B KV: 32 layers, K/V [4096,16,8,128] bf16 <-> pinned "
                           "block-wise host [16384,32,2,16,8,128]; 1024 random distinct ids"),
    "llama3-70b-tp8": dict(layers=80, kv=2, ng=8192, nh=16384, tokens=16, heads=1, dim=128,
                           n=2048, desc="Llama-3-70B TP-8 shard KV: 80 layers, K/V "
                                        "[8192,16,1,128] bf16 <-> host [16384,80,2,16,1,128]; "
                                        "2048 random distinct ids"),
    "mla-dsv3": dict(layers=61, kv=1, ng=4096, nh=8192, tokens=64, heads=1, dim=576, n=2048,
                     desc="MLA latent (DeepSeek-V3): 61 layers, [4096,64,576] bf16 <-> host "
                          "[8192,61,64,576]; 2048 random distinct ids"),
}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def release_device_memory() -> None:
    """Return torch's cached device memory to the driver, then wait while
    the driver clears it.  The amdgpu driver clears freed VRAM in the
    background on a copy engine that device-to-host copies share: on MI355X
    copy-engine D2H ran at 15.5 GB/s instead of 46 GB/s for 630 ms after a
    16 GiB free and 157 ms after a 4 GiB free (about 26 GB/s of clearing),
    which would be charged to whatever is measured next."""
    import gc
    gc.collect()
    before = torch.cuda.memory_reserved()
    torch.cuda.empty_cache()
    freed = max(0, before - torch.cuda.memory_reserved())
    torch.cuda.synchronize()
    if freed:
        time.sleep(0.05 + freed / 20e9)


class Workload:
    def __init__(self, name: str, seed: int, run: int = 0, host: bool = True,
                 host_layout: str = "BLOCKWISE"):
        from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType
        from flexkv_amd.storage.allocator import CPUAllocator

        w = WORKLOADS[name]
        self.name, self.w = name, w
        self.dev = torch.device("cuda:0")
        L, kv = w["layers"], w["kv"]
        mla = kv == 1
        self.dtype = getattr(torch, w.get("dtype", "bfloat16"))
        gl = KVCacheLayout(KVCacheLayoutType.LAYERWISE, L, w["ng"], w["tokens"], w["heads"],
                           w["dim"], is_mla=mla)
        cl = KVCacheLayout(KVCacheLayoutType[host_layout], L, w["nh"], w["tokens"], w["heads"],
                           w["dim"], is_mla=mla)
        self.cl = cl
        self.chunk, self.gkv, _, self.gblk = gl.div_layer(L).byte_strides(self.dtype)
        _, self.ckv, self.clay, self.cblk = cl.byte_strides(self.dtype)
        self.mla = mla
        t0 = time.time()
        gen = torch.Generator(device=self.dev).manual_seed(seed)
        self.layers = []
        for _ in range(L):
            t = torch.empty(tuple(gl.kv_shape[1:]), dtype=self.dtype, device=self.dev)
            t.normal_(generator=gen)
            self.layers.append(t)
        torch.cuda.synchronize()
        log(f"device layers ready ({L} x {self.layers[0].numel() * 2 / 2**30:.2f} GiB) "
            f"in {time.time() - t0:.1f}s")
        t0 = time.time()
        self.host = CPUAllocator.allocate(cl, self.dtype).get_tensor() if host else None
        if host:
            log(f"pinned host cache {self.host.numel() * 2 / 2**30:.2f} GiB in "
                f"{time.time() - t0:.1f}s")
        self.seed = seed
        cpu_gen = torch.Generator().manual_seed(seed + 1)
        n = w["n"]
        if run:
            self.gids = _run_ids(cpu_gen, n, w["ng"], run)
            self.cids = _run_ids(cpu_gen, n, w["nh"], run)
        else:
            self.gids = torch.randperm(w["ng"], generator=cpu_gen)[:n].to(torch.int64)
            self.cids = torch.randperm(w["nh"], generator=cpu_gen)[:n].to(torch.int64)
        self.gids_p = self.gids.pin_memory()
        self.cids_p = self.cids.pin_memory()
        self.ptrs = torch.tensor([t.data_ptr() for t in self.layers], dtype=torch.int64).pin_memory()
        self.bytes_per_op = self.chunk * L * kv * n

    def transfer(self, h2d: bool, use_ce, cus: int = -1) -> None:
        from flexkv_amd import c_ext
        c_ext.transfer_kv_blocks(self.gids_p, self.ptrs, self.gkv, self.gblk, self.cids_p,
                                 self.host, self.ckv, self.clay, self.cblk, self.chunk, 0, cus,
                                 h2d, use_ce, self.mla)

    def gather(self, buf: torch.Tensor, scatter: bool = False) -> None:
        from flexkv_amd import c_ext
        fn = c_ext.scatter_kv_blocks if scatter else c_ext.gather_kv_blocks
        fn(self.gids_p, self.ptrs, self.gkv, self.gblk, self.chunk, buf, self.mla)

    def packed_expected(self) -> torch.Tensor:
        """The moved blocks packed [block][layer][K|V][chunk], by torch indexing."""
        L, kv = self.w["layers"], self.w["kv"]
        g = self.gids.to(self.dev)
        want = torch.stack([t[:, g] for t in self.layers], dim=1)
        return want.permute(2, 1, 0, *range(3, want.dim())).reshape(-1).contiguous()

    def host_rows(self, ids: torch.Tensor) -> torch.Tensor:
        """Host blocks `ids` as int16 rows [n, layers, kv, chunk], any layout."""
        L, kv, nh = self.w["layers"], self.w["kv"], self.w["nh"]
        ce = self.chunk // 2
        h = self.host.view(torch.int16)
        if self.cl.type.name == "BLOCKWISE":
            return h.view(nh, L, kv, ce)[ids]
        return h.view(L, kv, nh, ce)[:, :, ids].permute(2, 0, 1, 3)

    def set_host_rows(self, ids: torch.Tensor, rows: torch.Tensor) -> None:
        L, kv, nh = self.w["layers"], self.w["kv"], self.w["nh"]
        ce = self.chunk // 2
        h = self.host.view(torch.int16)
        if self.cl.type.name == "BLOCKWISE":
            h.view(nh, L, kv, ce)[ids] = rows
        else:
            h.view(L, kv, nh, ce)[:, :, ids] = rows.permute(1, 2, 0, 3)

    def check(self) -> bool:
        """Every moved block: host block == the GPU blocks, bit for bit."""
        L, kv = self.w["layers"], self.w["kv"]
        ok = True
        step = 128
        for s in range(0, len(self.gids), step):
            g = self.gids[s:s + step].to(self.dev)
            c = self.cids[s:s + step]
            want = torch.stack([t[:, g] for t in self.layers], dim=1)  # [kv, L, b, ...]
            want = want.permute(2, 1, 0, *range(3, want.dim())).reshape(len(c), L, kv, -1)
            got = self.host_rows(c).to(self.dev)
            ok &= bool(torch.equal(got, want.view(torch.int16)))
        return ok


def _run_ids(gen, n, universe, run):
    slots = torch.randperm(universe // run, generator=gen)[: n // run]
    return (slots[:, None] * run + torch.arange(run)[None, :]).reshape(-1).to(torch.int64)


def time_steps(fn, steps: int, warmup: int):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    times = []
    t_all = time.perf_counter()
    for _ in range(steps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    torch.cuda.synchronize()
    total = time.perf_counter() - t_all
    return total / steps, statistics.median(times), min(times)


def device_ceilings(timeout_s: float = 180.0):
    """The device's plain HBM stream rates (read only, write only, copy) from
    the hbm_ceiling program built beside the library, run as a child process
    before this process touches the GPU.  None when the program is missing or
    fails."""
    exe = os.path.join(ROOT, "flexkv_amd", "hbm_ceiling")
    if not os.path.exists(exe):
        log("hbm_ceiling not built; device ceilings not measured")
        return None
    try:
        res = subprocess.run([exe], capture_output=True, text=True, timeout=timeout_s)
    except subprocess.TimeoutExpired:
        log("hbm_ceiling timed out")
        return None
    if res.returncode != 0:
        log(f"hbm_ceiling failed ({res.returncode}): {res.stderr.strip()[-300:]}")
        return None
    out = json.loads(res.stdout.strip().splitlines()[-1])
    log(f"device ceilings: read {out['read_gbps']:.0f}, write {out['write_gbps']:.0f}, "
        f"copy {out['copy_gbps']:.0f} GB/s")
    return out


def c_abi_latency(timeout_s: float = 120.0):
    """Per-call latency through the C-ABI from the call_latency program built
    beside the library (1-block and 16-block kernel-mode calls with their
    stream synchronisation, and the launch floors beside them), run as a
    child process before this process touches the GPU.  None when the
    program is missing or fails."""
    exe = os.path.join(ROOT, "flexkv_amd", "call_latency")
    if not os.path.exists(exe):
        log("call_latency not built; C-ABI latency not measured")
        return None
    try:
        res = subprocess.run([exe], capture_output=True, text=True, timeout=timeout_s)
    except subprocess.TimeoutExpired:
        log("call_latency timed out")
        return None
    if res.returncode != 0:
        log(f"call_latency failed ({res.returncode}): {res.stderr.strip()[-300:]}")
        return None
    out = json.loads(res.stdout.strip().splitlines()[-1])
    out["what"] = ("flexkv_amd/call_latency: median of 400 calls, each with "
                   "hipStreamSynchronize, in a C++ process")
    log(f"C-ABI call latency: 1 block {out['fkv_1x1_h2d_us']} / {out['fkv_1x1_d2h_us']} us "
        f"(H2D / D2H), empty kernel with arguments {out['args_kernel_us']} us")
    return out


def link_peaks(wl: Workload, reps: int = 8):
    """Best-of-reps 1 GiB contiguous pinned copies each way, and a 4 GiB
    device-to-device copy, timed with events on one stream."""
    nbytes = 1 << 30
    host = wl.host.view(torch.uint8)[:nbytes]
    dbuf = torch.empty(nbytes, dtype=torch.uint8, device=wl.dev)
    s = torch.cuda.current_stream()
    res = {}
    for name, fn in (("d2h", lambda: host.copy_(dbuf, non_blocking=True)),
                     ("h2d", lambda: dbuf.copy_(host, non_blocking=True))):
        best = 0.0
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(s)
            fn()
            b.record(s)
            b.synchronize()
            best = max(best, nbytes / (a.elapsed_time(b) * 1e-3) / 1e9)
        res[name] = best
    big = torch.empty(4 << 30, dtype=torch.uint8, device=wl.dev)
    big2 = torch.empty_like(big)
    best = 0.0
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(s)
        big2.copy_(big)
        b.record(s)
        b.synchronize()
        best = max(best, 2 * big.numel() / (a.elapsed_time(b) * 1e-3) / 1e9)
    res["d2d_copy_read_plus_write"] = best
    del big, big2
    # both directions at once: a 1 GiB D2H and a 1 GiB H2D of other memory
    # on two streams, started together; bytes of both over the wall time
    host2 = wl.host.view(torch.uint8)[nbytes:2 * nbytes]
    dbuf2 = torch.empty(nbytes, dtype=torch.uint8, device=wl.dev)
    streams = (torch.cuda.Stream(), torch.cuda.Stream())
    best = 0.0
    for _ in range(reps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        with torch.cuda.stream(streams[0]):
            host.copy_(dbuf, non_blocking=True)
        with torch.cuda.stream(streams[1]):
            dbuf2.copy_(host2, non_blocking=True)
        torch.cuda.synchronize()
        best = max(best, 2 * nbytes / (time.perf_counter() - t0) / 1e9)
    res["duplex"] = best
    del dbuf, dbuf2
    release_device_memory()
    return res


GEMM_WARM = 200   # GEMMs run before each measured window (about 40 ms)
GEMM_LEAD = 20    # of which the last GEMM_LEAD run after the transfer starts


def gemm_window(a, b, c, comp, start=None, n: int = 160):
    """Time n bf16 GEMMs on `comp` with the GPU already at its working clocks.

    The GFX clock drops within about 10 ms of idle compute and takes some
    30 ms of GEMMs to climb back, so a batch started from a quiet GPU runs
    6-9% slower than the same batch in a busy one.  Both the alone and the
    beside measurement therefore queue GEMM_WARM GEMMs ahead of the window
    with no gap; `start` (the transfer) is called when the warm-up has
    GEMM_LEAD GEMMs left, so the window runs entirely under the transfer
    for transfers longer than the window.  Returns (window ms, start's
    return value)."""
    with torch.cuda.stream(comp):
        ready = torch.cuda.Event()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for i in range(GEMM_WARM):
            torch.mm(a, b, out=c)
            if i == GEMM_WARM - GEMM_LEAD - 1:
                ready.record()
        e0.record()
        for _ in range(n):
            torch.mm(a, b, out=c)
        e1.record()
    ready.synchronize()
    started = start() if start is not None else None
    e1.synchronize()
    return e0.elapsed_time(e1), started


GEMM_QUIET_S = 0.05   # idle time before a transfer-first window


def gemm_window_transfer_first(a, b, c, comp, start=None, n: int = 160):
    """The other order: from a GPU idle for GEMM_QUIET_S, `start` (the
    transfer) is called first and the n GEMMs are queued right after it.
    The alone measurement starts from the same idle state, so the clock
    ramp is in both.  A zero-copy kernel launched first spreads its
    workgroups over idle compute units, where every GEMM wave then meets
    them; launched into running GEMMs it takes units as they free up."""
    torch.cuda.synchronize()
    time.sleep(GEMM_QUIET_S)
    started = None
    if start is not None:
        started = start()
        time.sleep(0.001)   # a transfer started on a thread has launched by now
    with torch.cuda.stream(comp):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            torch.mm(a, b, out=c)
        e1.record()
    e1.synchronize()
    return e0.elapsed_time(e1), started


def layerwise_h2d(wl: Workload, steps: int):
    """H2D of the step's blocks one layer group per layer.

    * reference schedule: one synchronous call per layer (the layer-wise read
      graph's ops, each run by the worker with its own stream sync);
    * async: fkv_transfer_kv_blocks_layerwise, host waits per group, on the
      zero-copy kernel ("kernel") and on the copy-engine pipeline ("ce");
    * overlap: a compute stream waits on each group's event, then runs a
      per-layer GEMM; compared with the transfer alone plus one layer's
      compute (the bound) and with the same GEMMs after a synchronous
      transfer;
    * GEMMs beside: 160 GEMMs with no waits, alone and beside one async
      layer-wise transfer on each path, both behind the same warm-up
      (gemm_window).
    """
    import threading

    from flexkv_amd import c_ext
    L = wl.w["layers"]
    args = (wl.gkv, wl.gblk, wl.cids_p, wl.host, wl.ckv, wl.clay, wl.cblk, wl.chunk)
    layer_ptrs = [wl.ptrs[l:l + 1].clone().pin_memory() for l in range(L)]

    def per_layer_sync():
        for l in range(L):
            c_ext.transfer_kv_blocks(wl.gids_p, layer_ptrs[l], wl.gkv, wl.gblk, wl.cids_p,
                                     wl.host, wl.ckv, wl.clay, wl.cblk, wl.chunk, l, -1, True,
                                     False, wl.mla)

    ref_s, _, _ = time_steps(per_layer_sync, steps, 1)
    xfer = c_ext.transfer_stream()   # own hardware queue, every CU
    # compute proxy: per layer, bf16 GEMMs of [8192 x 4096] x [4096 x 4096]
    a = torch.randn(8192, 4096, device=wl.dev, dtype=torch.bfloat16)
    b = torch.randn(4096, 4096, device=wl.dev, dtype=torch.bfloat16)
    c = torch.empty(8192, 4096, device=wl.dev, dtype=torch.bfloat16)
    reps = 4
    comp = torch.cuda.Stream()
    gb = wl.bytes_per_op / 1e9

    def start(ce):
        with torch.cuda.stream(xfer):
            return c_ext.transfer_kv_blocks_layerwise(wl.gids_p, wl.ptrs, wl.gkv, wl.gblk,
                                                      *args[2:], 0, 1, -1, True, wl.mla,
                                                      use_ce_transfer=ce)

    def compute_layers(hnd=None):
        with torch.cuda.stream(comp):
            for l in range(L):
                if hnd is not None:
                    hnd.stream_wait(l, comp)
                for _ in range(reps):
                    torch.mm(a, b, out=c)

    def compute_only():
        compute_layers()
        comp.synchronize()

    comp_s, _, _ = time_steps(compute_only, steps, 1)
    gemm_alone = statistics.median(gemm_window(a, b, c, comp)[0] for _ in range(3))
    gemm_alone_tf = statistics.median(gemm_window_transfer_first(a, b, c, comp)[0]
                                      for _ in range(3))
    out = {"granularity_layers": 1,
           "reference_schedule_ms": round(ref_s * 1e3, 2),
           "reference_schedule_gbps": round(gb / ref_s, 2),
           "compute_only_ms": round(comp_s * 1e3, 2),
           "compute_proxy": f"{reps} bf16 GEMMs [8192x4096]x[4096x4096] per layer",
           "gemm_window": (f"160 GEMMs after {GEMM_WARM} back-to-back warm-up GEMMs; beside: "
                           f"the handle starts {GEMM_LEAD} GEMMs before the window"),
           "gemm_alone_ms": round(gemm_alone, 2),
           "gemm_window_transfer_first": (f"160 GEMMs queued right after the handle starts, "
                                          f"from a GPU idle {GEMM_QUIET_S * 1e3:.0f} ms; alone "
                                          "from the same idle state"),
           "gemm_alone_transfer_first_ms": round(gemm_alone_tf, 2)}
    for name, ce in (("kernel", False), ("ce", True)):
        first, total = [], []
        for _ in range(steps + 1):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            h = start(ce)
            h.wait(0)
            t1 = time.perf_counter()
            h.wait()
            t2 = time.perf_counter()
            h.release()
            first.append(t1 - t0)
            total.append(t2 - t0)
        first, total = first[1:], total[1:]

        def serial():
            wl.transfer(True, ce)
            compute_layers()
            comp.synchronize()

        def overlapped():
            hnd = start(ce)
            compute_layers(hnd)
            comp.synchronize()
            hnd.release()

        ser_s, _, _ = time_steps(serial, steps, 1)
        ovl_s, _, _ = time_steps(overlapped, steps, 1)
        beside, beside_tf = [], []
        for _ in range(3):
            ms, hnd = gemm_window(a, b, c, comp, start=lambda: start(ce))
            beside.append(ms)
            hnd.release()
            ms, hnd = gemm_window_transfer_first(a, b, c, comp, start=lambda: start(ce))
            beside_tf.append(ms)
            hnd.release()
        xfer_ms = statistics.median(total) * 1e3
        bound = xfer_ms + comp_s * 1e3 / L
        out[name] = {"async_total_ms": round(xfer_ms, 2),
                     "async_gbps": round(gb / (xfer_ms * 1e-3), 2),
                     "async_first_group_ms": round(statistics.median(first) * 1e3, 3),
                     "transfer_then_compute_ms": round(ser_s * 1e3, 2),
                     "layerwise_overlapped_ms": round(ovl_s * 1e3, 2),
                     "bound_transfer_plus_one_layer_ms": round(bound, 2),
                     "overlapped_over_bound": round(ovl_s * 1e3 / bound, 4),
                     "gemm_beside_ms": round(statistics.median(beside), 2),
                     "gemm_slowdown": round(statistics.median(beside) / gemm_alone, 4),
                     "gemm_beside_transfer_first_ms": round(statistics.median(beside_tf), 2),
                     "gemm_slowdown_transfer_first": round(statistics.median(beside_tf)
                                                           / gemm_alone_tf, 4)}
    c_ext.release_transfer_stream(xfer)
    return out


def engine_layerwise(wl: Workload, steps: int):
    """A layer-wise read graph (one H2D op per layer, each after the previous,
    convert_read_graph_to_layer_wise_graph) through TransferEngine with a
    thread worker; submit-to-graph-complete time, with and without eager
    dispatch of same-worker chains."""
    from flexkv_amd.cache.transfer_pattern import (convert_read_graph_to_layer_wise_graph,
                                                   create_read_graph_cpu_storage)
    from flexkv_amd.common.config import CacheConfig, ModelConfig
    from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType
    from flexkv_amd.storage.allocator import AccessHandleType, StorageHandle
    from flexkv_amd.transfer.transfer_engine import TransferEngine
    w = wl.w
    L = w["layers"]
    gl = KVCacheLayout(KVCacheLayoutType.LAYERWISE, L, w["ng"], w["tokens"], w["heads"],
                       w["dim"], is_mla=wl.mla)
    cl = wl.cl
    gpu_h = StorageHandle(AccessHandleType.TENSOR, wl.layers, gl, wl.dtype, gpu_device_id=0)
    cpu_h = StorageHandle(AccessHandleType.TENSOR, wl.host, cl, wl.dtype)
    mc = ModelConfig(num_layers=L, num_kv_heads=w["heads"], head_size=w["dim"],
                     use_mla=wl.mla, dtype=wl.dtype)
    out = {}
    for eager in (False, True):
        eng = TransferEngine([gpu_h], mc, CacheConfig(use_ce_transfer_h2d=False), cpu_handle=cpu_h, eager_dispatch=eager)
        eng.start()
        times = []
        try:
            for _ in range(steps + 1):
                rg, ends = create_read_graph_cpu_storage(wl.gids, wl.cids,
                                                         torch.empty(0, dtype=torch.int64),
                                                         layer_num=L)
                lw, _ = convert_read_graph_to_layer_wise_graph(rg, ends, L, 1)
                t0 = time.perf_counter()
                eng.submit_transfer_graph(lw)
                seen = []
                while (lw.graph_id, -1) not in seen:
                    seen += eng.get_completed_graphs_and_ops(timeout=0.05)
                times.append(time.perf_counter() - t0)
        finally:
            eng.shutdown()
        med = statistics.median(times[1:])
        out["eager" if eager else "reference_scheduling"] = {
            "ms": round(med * 1e3, 2), "gbps": round(wl.bytes_per_op / med / 1e9, 2)}
    out["what"] = f"{L} one-layer H2D ops chained layer by layer, thread worker, zero-copy path"
    return out


def engine_put_get(wl: Workload, steps: int):
    """A write graph (D2H of the step's blocks) and a read graph (H2D of as
    many other blocks) submitted together to TransferEngine with thread
    workers and the default copy-engine path: submit-to-both-complete time,
    and each graph alone.  The engine runs one worker per direction, so the
    two overlap on the full-duplex link."""
    from flexkv_amd.cache.transfer_pattern import (create_read_graph_cpu_storage,
                                                   create_write_graph_cpu_storage)
    from flexkv_amd.common.config import CacheConfig, ModelConfig
    from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType
    from flexkv_amd.storage.allocator import AccessHandleType, StorageHandle
    from flexkv_amd.transfer.transfer_engine import TransferEngine
    w = wl.w
    L = w["layers"]
    n = len(wl.gids)
    gl = KVCacheLayout(KVCacheLayoutType.LAYERWISE, L, w["ng"], w["tokens"], w["heads"],
                       w["dim"], is_mla=wl.mla)
    gpu_h = StorageHandle(AccessHandleType.TENSOR, wl.layers, gl, wl.dtype, gpu_device_id=0)
    cpu_h = StorageHandle(AccessHandleType.TENSOR, wl.host, wl.cl, wl.dtype)
    mc = ModelConfig(num_layers=L, num_kv_heads=w["heads"], head_size=w["dim"],
                     use_mla=wl.mla, dtype=wl.dtype)
    g = torch.Generator().manual_seed(wl.seed + 6)
    free_g = torch.tensor(sorted(set(range(w["ng"])) - set(wl.gids.tolist())), dtype=torch.int64)
    free_c = torch.tensor(sorted(set(range(w["nh"])) - set(wl.cids.tolist())), dtype=torch.int64)
    g2 = free_g[torch.randperm(len(free_g), generator=g)[:n]]
    c2 = free_c[torch.randperm(len(free_c), generator=g)[:n]]
    none = torch.empty(0, dtype=torch.int64)
    eng = TransferEngine([gpu_h], mc, CacheConfig(), cpu_handle=cpu_h)
    eng.start()

    def run(kinds):
        graphs = []
        for kind in kinds:
            if kind == "put":
                graphs.append(create_write_graph_cpu_storage(wl.gids, wl.cids, none,
                                                             layer_num=L)[0])
            else:
                graphs.append(create_read_graph_cpu_storage(g2, c2, none, layer_num=L)[0])
        t0 = time.perf_counter()
        for gr in graphs:
            eng.submit_transfer_graph(gr)
        left = {gr.graph_id for gr in graphs}
        while left:
            for gid, op in eng.get_completed_graphs_and_ops(timeout=0.05):
                if op == -1:
                    left.discard(gid)
        return time.perf_counter() - t0

    out = {}
    try:
        for name, kinds in (("put", ["put"]), ("get", ["get"]), ("put_and_get", ["put", "get"])):
            ts = [run(kinds) for _ in range(steps + 1)][1:]
            med = statistics.median(ts)
            out[name] = {"ms": round(med * 1e3, 2),
                         "gbps": round(len(kinds) * wl.bytes_per_op / med / 1e9, 2)}
    finally:
        eng.shutdown()
    out["what"] = ("TransferEngine, thread workers, copy-engine path: a 2 GiB write graph, a "
                   "2 GiB read graph of other blocks, and both submitted together")
    return out


def worker_ops(wl: Workload, reps: int = 40, process: bool = True):
    """Ops through GPUCPUTransferWorker, each submitted and waited for on the
    finished-ops queue before the next, as the reference's worker benchmark
    does (benchmarks/benchmark_workers.py:159-167,232-240): 16 blocks
    (32 MiB at the Llama-3-8B shape) and the full step, both directions, on
    the copy-engine and the zero-copy path; on a worker thread of this
    process (this package's engine default) and, for 16 blocks, in a spawned
    worker process fed IPC handles of the device layers (the reference's
    worker model; its own pinned host cache of 1024 blocks), reporting
    finished ops over a pipe as TransferEngine's process mode does.  Each op
    runs inside a roctx range named as the reference names its NVTX range."""
    import multiprocessing as mp
    import queue

    from flexkv_amd.common.memory_handle import TensorSharedHandle
    from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType
    from flexkv_amd.common.transfer import TransferDescriptor, TransferOp, TransferType
    from flexkv_amd.storage.allocator import HostCacheSpec
    from flexkv_amd.transfer.worker import FinishedOpsChannel, GPUCPUTransferWorker
    w = wl.w
    L = w["layers"]
    gl = KVCacheLayout(KVCacheLayoutType.LAYERWISE, L, w["ng"], w["tokens"], w["heads"],
                       w["dim"], is_mla=wl.mla)

    def op(kind, gids, cids):
        src, dst = (gids, cids) if kind == TransferType.D2H else (cids, gids)
        return TransferOp(graph_id=0, transfer_type=kind, layer_id=0, layer_granularity=L,
                          src_descriptor=TransferDescriptor(physical_block_ids=src),
                          dst_descriptor=TransferDescriptor(physical_block_ids=dst))

    def timed(handle, q, kind, gids, cids, n_reps):
        o = op(kind, gids, cids)
        handle.submit_transfer(o)
        assert q.get(timeout=120) == o.op_id
        ts = []
        for _ in range(n_reps):
            o = op(kind, gids, cids)
            t0 = time.perf_counter()
            handle.submit_transfer(o)
            got = q.get(timeout=120)
            ts.append(time.perf_counter() - t0)
            assert got == o.op_id
        med = statistics.median(ts)
        nbytes = len(gids) * L * w["kv"] * wl.chunk
        return {"ms": round(med * 1e3, 3), "gbps": round(nbytes / med / 1e9, 2)}

    out = {}
    g16, c16 = wl.gids[:16].clone(), wl.cids[:16].clone()
    for path, ce in (("ce", True), ("kernel", False)):
        q = queue.Queue()
        h = GPUCPUTransferWorker.create_worker_thread(
            0, q, wl.layers, wl.host, gl, wl.cl, wl.dtype, 0, use_ce_transfer_h2d=ce,
            use_ce_transfer_d2h=ce)
        h.wait_ready()
        try:
            res = {}
            for kind in (TransferType.D2H, TransferType.H2D):
                d = kind.name.lower()
                res[f"{d}_16blk"] = timed(h, q, kind, g16, c16, reps)
                res[f"{d}_step"] = timed(h, q, kind, wl.gids, wl.cids, 3)
            out[f"thread_{path}"] = res
        finally:
            h.shutdown()
    if process:
        ctx = mp.get_context("spawn")
        q = FinishedOpsChannel(ctx)
        small = KVCacheLayout(wl.cl.type, L, 1024, w["tokens"], w["heads"], w["dim"],
                              is_mla=wl.mla)
        for path, ce in (("ce", True), ("kernel", False)):
            h = GPUCPUTransferWorker.create_worker(
                0, q, [TensorSharedHandle(t) for t in wl.layers], HostCacheSpec(small, wl.dtype),
                gl, small, wl.dtype, 0, use_ce_transfer_h2d=ce, use_ce_transfer_d2h=ce)
            try:
                if not h.ready_event.wait(180):
                    out[f"process_{path}"] = {"skipped": "worker process did not start"}
                    continue
                c_small = torch.randperm(1024, generator=torch.Generator().manual_seed(8))[:16]
                out[f"process_{path}"] = {
                    f"{k.name.lower()}_16blk": timed(h, q, k, g16, c_small, reps)
                    for k in (TransferType.D2H, TransferType.H2D)}
            finally:
                h.shutdown()
        q.close()
    out["what"] = ("16-block ops (32 MiB at this shape) and full-step ops, one at a time, "
                   "submit to finished-ops queue (spawned workers: a pipe, FinishedOpsChannel); "
                   "copy engines take ops of 32 MiB or more (the default policy)")
    return out


def call_latency(wl: Workload, reps: int = 200):
    """Wall time of small synchronous calls from Python (1 block x 1 layer,
    16 blocks x 1 layer, 16 blocks x all layers), zero-copy and copy-engine
    paths, each direction, median of `reps` on the current stream; beside
    them a one-element torch fill plus stream synchronisation, the cost of
    the smallest torch device op from Python."""
    from flexkv_amd import c_ext
    out = {}
    L = wl.w["layers"]
    warm = 50   # untimed calls first: the first of a series ran about 1 us slower
    for path, ce in (("zc", False), ("ce", True)):
        for nb, nl in ((1, 1), (16, 1), (16, L)):
            g = wl.gids_p[:nb].clone().pin_memory()
            c = wl.cids_p[:nb].clone().pin_memory()
            p = wl.ptrs[:nl].clone().pin_memory()
            for name, h2d in (("h2d", True), ("d2h", False)):
                ts = []
                for i in range(reps + warm):
                    t0 = time.perf_counter()
                    c_ext.transfer_kv_blocks(g, p, wl.gkv, wl.gblk, c, wl.host, wl.ckv, wl.clay,
                                             wl.cblk, wl.chunk, 0, -1, h2d, ce, wl.mla)
                    ts.append(time.perf_counter() - t0)
                out[f"{path}_{nb}blk_{nl}layer_{name}_us"] = round(statistics.median(ts[warm:]) * 1e6, 1)
    x = torch.zeros(1, device=wl.dev)
    st = torch.cuda.current_stream()
    ts = []
    for i in range(reps + warm):
        t0 = time.perf_counter()
        x.fill_(1.0)
        st.synchronize()
        ts.append(time.perf_counter() - t0)
    out["torch_fill_sync_us"] = round(statistics.median(ts[warm:]) * 1e6, 1)
    return out


def duplex(wl: Workload, reps: int = 3):
    """A D2H of the step's blocks and an H2D of as many other blocks (other
    GPU and host ids) at once, from two host threads on two streams, per
    path: aggregate GB/s over both directions (best of `reps`).  PCIe is
    full duplex; each copy-engine direction has its own staging and
    engines."""
    import threading

    from flexkv_amd import c_ext
    w = wl.w
    n = len(wl.gids)
    g = torch.Generator().manual_seed(wl.seed + 5)
    free_g = torch.tensor(sorted(set(range(w["ng"])) - set(wl.gids.tolist())), dtype=torch.int64)
    free_c = torch.tensor(sorted(set(range(w["nh"])) - set(wl.cids.tolist())), dtype=torch.int64)
    g2 = free_g[torch.randperm(len(free_g), generator=g)[:n]].pin_memory()
    c2 = free_c[torch.randperm(len(free_c), generator=g)[:n]].pin_memory()
    # streams on hardware queues of their own: two ordinary streams can share
    # one of the process's queues, and then the two zero-copy kernels run in turn
    streams = [c_ext.transfer_stream(), c_ext.transfer_stream()]
    out = {}
    for name, ce in (("kernel", False), ("ce", True)):
        best = None
        for _ in range(reps):
            torch.cuda.synchronize()
            errs = []
            took = [0.0, 0.0]

            def move(i):
                try:
                    with torch.cuda.stream(streams[i]):
                        ids = (wl.gids_p, wl.cids_p) if i == 0 else (g2, c2)
                        t0 = time.perf_counter()
                        c_ext.transfer_kv_blocks(ids[0], wl.ptrs, wl.gkv, wl.gblk, ids[1],
                                                 wl.host, wl.ckv, wl.clay, wl.cblk, wl.chunk,
                                                 0, -1, i == 1, ce, wl.mla)
                        took[i] = time.perf_counter() - t0
                except Exception as e:   # reported below
                    errs.append(e)
            th = [threading.Thread(target=move, args=(i,)) for i in range(2)]
            t0 = time.perf_counter()
            for t in th:
                t.start()
            for t in th:
                t.join()
            el = time.perf_counter() - t0
            if errs:
                raise errs[0]
            run = (2 * wl.bytes_per_op / el / 1e9, wl.bytes_per_op / took[0] / 1e9,
                   wl.bytes_per_op / took[1] / 1e9)
            if best is None or run[0] > best[0]:
                best = run
        out[f"{name}_aggregate_gbps"] = round(best[0], 3)
        out[f"{name}_d2h_gbps"] = round(best[1], 2)
        out[f"{name}_h2d_gbps"] = round(best[2], 2)
    for st in streams:
        c_ext.release_transfer_stream(st)
    out["what"] = ("one D2H and one H2D of 2 GiB each at once, two threads and streams; "
                   "aggregate: bytes of both over the wall time; per direction: its bytes "
                   "over its own call time (best run by aggregate)")
    return out


def overlap_with_compute(wl: Workload, steps: int = 3, gemms: int = 160,
                         rect_copies: bool = False, resident_probe: bool = True):
    """One full transfer op on its own stream (from a second host thread)
    while the main thread runs bf16 GEMMs [8192x4096]x[4096x4096] on a compute
    stream: GEMM time alone and beside each path and direction.  The
    zero-copy kernel shares compute units with the GEMMs; the copy-engine
    path leaves the PCIe copies to the SDMA engines.  Alone and beside, the
    GEMMs run behind the same warm-up (gemm_window).  `rect_copies`: the
    copy-engine runs use the rect-copy policy (layer-wise host caches with
    scattered ids).  `resident_probe`: also time the GEMMs beside a kernel
    that only spins in one single-thread workgroup (torch.cuda._sleep), as
    long as a transfer, which shows what residency alone costs them."""
    import threading

    from flexkv_amd import c_ext
    xfer = c_ext.transfer_stream()
    comp = torch.cuda.Stream()
    a = torch.randn(8192, 4096, device=wl.dev, dtype=torch.bfloat16)
    b = torch.randn(4096, 4096, device=wl.dev, dtype=torch.bfloat16)
    c = torch.empty(8192, 4096, device=wl.dev, dtype=torch.bfloat16)

    def once(h2d, ce, with_xfer=True, window=gemm_window, cus=-1):
        torch.cuda.synchronize()
        res = {}

        def move():
            with torch.cuda.stream(xfer):
                t0 = time.perf_counter()
                wl.transfer(h2d, ce, cus)
                res["xfer"] = time.perf_counter() - t0

        def start():
            th = threading.Thread(target=move)
            th.start()
            return th
        ms, th = window(a, b, c, comp, start=start if with_xfer else None, n=gemms)
        if th:
            th.join()
        torch.cuda.synchronize()
        res["gemm"] = ms / 1e3
        return res

    once(True, False, with_xfer=False)
    def med_ms(rs, key):
        return round(statistics.median(r[key] for r in rs) * 1e3, 2)

    out = {"gemm_alone_ms": med_ms([once(True, False, with_xfer=False)
                                    for _ in range(steps)], "gemm")}
    tf = {"gemm_alone_ms": med_ms([once(True, False, False, gemm_window_transfer_first)
                                   for _ in range(steps)], "gemm")}
    ce_name = "_ce_rect" if rect_copies else "_ce"
    for h2d in (False, True):
        for ce in (False, True):
            key = ("h2d" if h2d else "d2h") + (ce_name if ce else "_kernel")
            if ce and rect_copies:
                c_ext.set_copy_engine_policy(layerwise_scattered="rect_copies")
            try:
                rs = [once(h2d, ce) for _ in range(steps)]
                out[key] = {"gemm_ms": med_ms(rs, "gemm"), "transfer_ms": med_ms(rs, "xfer"),
                            "gemm_slowdown": round(med_ms(rs, "gemm") / out["gemm_alone_ms"], 4),
                            "transfer_gbps": round(wl.bytes_per_op / med_ms(rs, "xfer") / 1e6,
                                                   2)}
                rs = [once(h2d, ce, True, gemm_window_transfer_first) for _ in range(steps)]
                tf[key] = {"gemm_ms": med_ms(rs, "gemm"), "transfer_ms": med_ms(rs, "xfer"),
                           "gemm_slowdown": round(med_ms(rs, "gemm") / tf["gemm_alone_ms"], 4),
                           "transfer_gbps": round(wl.bytes_per_op / med_ms(rs, "xfer") / 1e6, 2)}
            finally:
                if ce and rect_copies:
                    c_ext.set_copy_engine_policy(layerwise_scattered="unset")
    # The zero-copy H2D with its grid spread over the chip (transfer_cus = a
    # CU count / 8: about one workgroup per compute unit) instead of 8 CUs'
    # worth: the automatic grid keeps 8, and this shows the trade.
    spread = max(1, torch.cuda.get_device_properties(wl.dev).multi_processor_count // 8)
    for key, window, store, alone in (("h2d_kernel_spread", gemm_window, out, out),
                                      ("h2d_kernel_spread", gemm_window_transfer_first, tf,
                                       tf)):
        rs = [once(True, False, True, window, cus=spread) for _ in range(steps)]
        store[key] = {"gemm_ms": med_ms(rs, "gemm"), "transfer_ms": med_ms(rs, "xfer"),
                      "gemm_slowdown": round(med_ms(rs, "gemm") / alone["gemm_alone_ms"], 4),
                      "transfer_gbps": round(wl.bytes_per_op / med_ms(rs, "xfer") / 1e6, 2),
                      "transfer_cus": spread}
    if resident_probe:
        spin = resident_spin_probe(a, b, c, comp, steps, gemms)
        out["resident_spin"] = {k: v for k, v in spin.items() if k != "transfer_first"}
        tf["resident_spin"] = spin["transfer_first"]
        for key, grid, block in (("resident_sleep_1wave", 1, 64),
                                 ("resident_sleep_256wg", 256, 256)):
            res = resident_sleep_probe(a, b, c, comp, steps, gemms, grid, block)
            if res is None:
                break
            out[key], tf[key] = res
    c_ext.release_transfer_stream(xfer)
    out["transfer_first"] = tf
    out["what"] = (f"{gemms} GEMMs on a compute stream beside one {wl.bytes_per_op / 2**30:.0f} "
                   f"GiB transfer on a transfer stream, started {GEMM_LEAD} GEMMs before the "
                   f"window; alone and beside after {GEMM_WARM - GEMM_LEAD} warm-up GEMMs. "
                   f"transfer_first: the transfer starts on a GPU idle "
                   f"{GEMM_QUIET_S * 1e3:.0f} ms and the GEMMs are queued after it; alone from "
                   "the same idle state")
    return out


def resident_spin_probe(a, b, c, comp, steps: int, gemms: int, target_ms: float = 38.0):
    """The GEMM windows of overlap_with_compute beside a kernel that touches
    no memory: torch.cuda._sleep, one workgroup of one thread spinning on
    the clock for about target_ms (the length of a 2 GiB transfer; the spin
    count is calibrated first).  Both launch orders; alone from the same
    state.  Any workgroup that stays resident on a compute unit slows these
    GEMMs, which run one 256-thread workgroup per compute unit."""
    spin_stream = torch.cuda.Stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    cycles = 1 << 20
    for _ in range(3):                          # calibrate the spin's clock
        with torch.cuda.stream(spin_stream):
            e0.record()
            torch.cuda._sleep(cycles)
            e1.record()
        e1.synchronize()
        ms = max(e0.elapsed_time(e1), 1e-3)
        cycles = int(cycles * min(64.0, target_ms / ms))
    cycles = min(cycles, 1 << 40)

    def start():
        with torch.cuda.stream(spin_stream):
            torch.cuda._sleep(cycles)

    def med(fn):
        return round(statistics.median(fn() for _ in range(steps)), 2)
    out = {}
    for key, window in (("gemm_first", gemm_window), ("transfer_first",
                                                       gemm_window_transfer_first)):
        alone = med(lambda: window(a, b, c, comp, None, gemms)[0])
        beside = med(lambda: window(a, b, c, comp, start, gemms)[0])
        torch.cuda.synchronize()
        out[key] = {"gemm_alone_ms": alone, "gemm_ms": beside,
                    "gemm_slowdown": round(beside / alone, 4)}
    with torch.cuda.stream(spin_stream):
        e0.record()
        torch.cuda._sleep(cycles)
        e1.record()
    e1.synchronize()
    res = out["gemm_first"]
    res["spin_ms"] = round(e0.elapsed_time(e1), 2)
    res["transfer_first"] = out["transfer_first"]
    res["what"] = ("torch.cuda._sleep: one workgroup of one thread spinning on the clock, "
                   "no memory access, started as the transfer would be")
    return res


def resident_sleep_probe(a, b, c, comp, steps: int, gemms: int, grid: int, block: int,
                         target_ms: float = 38.0):
    """The GEMM windows beside a kernel whose wavefronts only sleep
    (flexkv_amd/libresident_probe.so: s_sleep between wall-clock reads for
    target_ms, no memory access), `grid` workgroups of `block` threads, in
    both launch orders against GEMMs alone started the same way.  Set beside
    resident_spin, it shows whether a resident kernel costs the GEMMs by what
    it issues or by occupying compute units.  None when the probe library is
    not built."""
    import ctypes
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "flexkv_amd",
                        "libresident_probe.so")
    if not os.path.exists(path):
        return None
    lib = ctypes.CDLL(path)
    lib.fkv_probe_resident.argtypes = [ctypes.c_void_p, ctypes.c_double, ctypes.c_int,
                                       ctypes.c_int]
    side = torch.cuda.Stream()

    def start():
        rc = lib.fkv_probe_resident(ctypes.c_void_p(side.cuda_stream), target_ms, grid, block)
        if rc != 0:
            raise RuntimeError(f"fkv_probe_resident failed ({rc})")

    def med(fn):
        return round(statistics.median(fn() for _ in range(steps)), 2)
    out = []
    for window in (gemm_window, gemm_window_transfer_first):
        alone = med(lambda: window(a, b, c, comp, None, gemms)[0])

        def beside():
            ms = window(a, b, c, comp, start, gemms)[0]
            side.synchronize()
            return ms
        ms = med(beside)
        out.append({"gemm_alone_ms": alone, "gemm_ms": ms, "gemm_slowdown": round(ms / alone, 4),
                    "grid": grid, "block": block})
    return out[0], out[1]


def request_batch(wl: Workload, steps: int, num_requests: int = 32, max_blocks: int = 128):
    """Requests of U{1..max_blocks} blocks with distinct random ids (seeded),
    moved one synchronous call per request and as one batched call, both
    directions, on the copy-engine and the zero-copy path; each path's
    batched D2H result is checked bit-exact, and its H2D into zeroed blocks
    restores them."""
    from flexkv_amd import c_ext
    L, kv = wl.w["layers"], wl.w["kv"]
    g = torch.Generator().manual_seed(1006)
    sizes = torch.randint(1, max_blocks + 1, (num_requests,), generator=g)
    total = int(sizes.sum())
    gids = torch.randperm(wl.w["ng"], generator=g)[:total].to(torch.int64)
    cids = torch.randperm(wl.w["nh"], generator=g)[:total].to(torch.int64)
    bounds = [0] + torch.cumsum(sizes, 0).tolist()
    reqs = [(gids[bounds[i]:bounds[i + 1]].clone(), cids[bounds[i]:bounds[i + 1]].clone())
            for i in range(num_requests)]
    nbytes = total * L * kv * wl.chunk

    def call(gi, ci, h2d, ce):
        c_ext.transfer_kv_blocks(gi, wl.ptrs, wl.gkv, wl.gblk, ci, wl.host, wl.ckv, wl.clay,
                                 wl.cblk, wl.chunk, 0, -1, h2d, ce, wl.mla)

    out = {"requests": num_requests, "blocks": total, "bytes": nbytes}
    saved = wl.gids, wl.cids
    wl.gids, wl.cids = gids, cids
    try:
        for path, ce in (("ce", True), ("kernel", False)):
            res = {}
            for h2d in (False, True):
                name = "h2d" if h2d else "d2h"
                per, _, _ = time_steps(lambda: [call(gi, ci, h2d, ce) for gi, ci in reqs],
                                       steps, 1)
                bat, _, _ = time_steps(lambda: call(gids, cids, h2d, ce), steps, 1)
                res[f"{name}_per_request_gbps"] = round(nbytes / per / 1e9, 2)
                res[f"{name}_batched_gbps"] = round(nbytes / bat / 1e9, 2)
            res["bit_exact"] = round_trip_bit_exact(wl, ce)
            out[path] = res
    finally:
        wl.gids, wl.cids = saved
    return out


def round_trip_bit_exact(wl: Workload, ce) -> bool:
    """D2H of the workload's blocks, the host rows checked against the GPU
    blocks; then the GPU blocks zeroed in place, H2D, and the blocks compared
    with a saved copy.  Both must hold bit for bit."""
    g = wl.gids.to(wl.dev)
    saved = [t.index_select(1, g) for t in wl.layers]
    gi = wl.gids.pin_memory()
    ci = wl.cids.pin_memory()
    from flexkv_amd import c_ext

    def move(h2d):
        c_ext.transfer_kv_blocks(gi, wl.ptrs, wl.gkv, wl.gblk, ci, wl.host, wl.ckv, wl.clay,
                                 wl.cblk, wl.chunk, 0, -1, h2d, ce, wl.mla)
    move(False)
    ok = wl.check()
    for t in wl.layers:
        t.index_fill_(1, g, 0)
    torch.cuda.synchronize()
    ok &= all(not t.index_select(1, g).any() for t in wl.layers)   # really cleared
    move(True)
    ok &= all(torch.equal(t.index_select(1, g), s) for t, s in zip(wl.layers, saved))
    del saved
    return bool(ok)


def path_rates(wl: Workload, steps: int, peaks: dict, paths=(("ce", True), ("kernel", False))):
    """D2H and H2D GB/s of the workload's step on each path, as fractions of
    the measured link and of the nominal PCIe Gen5 x16 rate; for the
    copy-engine path also the average rate of the gather and scatter pieces
    it launched (the library's event timing, HBM bytes = 2 x moved).  The
    rates come from a run without the library's profiling, which records
    events around every launch and costs small ops several percent; it runs
    at least 0.1 s (at 50 GB/s) so short ops are timed over many calls.  The
    piece rates come from a second, profiled run of `steps` transfers."""
    from flexkv_amd import _lib
    gb = wl.bytes_per_op / 1e9
    timed = max(steps, int(0.1 * 50e9 / wl.bytes_per_op) + 1)
    out = {}
    for name, ce in paths:
        res = {}
        for h2d in (False, True):
            d = "h2d" if h2d else "d2h"
            s, _, _ = time_steps(lambda: wl.transfer(h2d, ce), timed, 1)
            _lib.profile_enable(True)
            time_steps(lambda: wl.transfer(h2d, ce), steps, 0)
            prof = _lib.profile_read()
            _lib.profile_enable(False)
            rate = gb / s
            res[f"{d}_gbps"] = round(rate, 3)
            res[f"{d}_frac_link"] = round(rate / peaks[d], 4)
            res[f"{d}_frac_pcie_gen5_x16"] = round(rate / PCIE_GEN5_X16_GBS, 4)
            if ce and prof["dma_batches"] and prof["kernel_ms"] > 0:
                piece = 2 * prof["kernel_bytes"] / (prof["kernel_ms"] * 1e-3) / 1e9
                key = "scatter" if h2d else "gather"
                res[f"{key}_piece_gbps_hbm"] = round(piece, 1)
                res[f"{key}_piece_frac_hbm"] = round(piece / HBM_PEAK_GBS, 4)
                res[f"{key}_pieces_per_step"] = prof["kernel_launches"] // steps
            elif ce:
                res[f"{d}_moved_by"] = "zero-copy kernel (size or layout policy)"
        out[name] = res
    return out


def standalone_gather(wl: Workload, steps: int):
    """The device gather and scatter of the whole step in one launch each,
    into and out of one packed HBM buffer; rates from the library's events."""
    from flexkv_amd import _lib
    buf = torch.empty(wl.bytes_per_op, dtype=torch.uint8, device=wl.dev)
    out = {}
    for name, sc in (("gather", False), ("scatter", True)):
        _lib.profile_enable(True)
        time_steps(lambda: wl.gather(buf, scatter=sc), steps, 1)
        prof = _lib.profile_read()
        _lib.profile_enable(False)
        rate = 2 * prof["kernel_bytes"] / (prof["kernel_ms"] * 1e-3) / 1e9
        out[f"{name}_gbps_hbm"] = round(rate, 1)
        out[f"{name}_frac_hbm"] = round(rate / HBM_PEAK_GBS, 4)
    del buf
    release_device_memory()
    return out


def set_ids(wl: Workload, gids: torch.Tensor, cids: torch.Tensor) -> None:
    wl.gids, wl.cids = gids, cids
    wl.gids_p, wl.cids_p = gids.pin_memory(), cids.pin_memory()


def fragmentation_sweep(wl: Workload, steps: int, peaks: dict):
    """Config 2: the Llama-3-8B tensors with 1024 ids in contiguous runs of
    1, 8, 64 and 1024 (random non-overlapping run starts on both sides,
    seeded), both directions on both paths, each run length's D2H -> zeroed
    GPU blocks -> H2D round trip checked bit-exact."""
    saved = wl.gids, wl.cids
    w = wl.w
    out = {}
    try:
        for run in (1, 8, 64, 1024):
            gen = torch.Generator().manual_seed(wl.seed + 100 + run)
            set_ids(wl, _run_ids(gen, w["n"], w["ng"], run), _run_ids(gen, w["n"], w["nh"], run))
            res = path_rates(wl, steps, peaks)
            res["bit_exact"] = all(round_trip_bit_exact(wl, ce) for ce in (True, False))
            out[f"run_{run}"] = res
            log(f"cfg2 run {run}: {res}")
    finally:
        set_ids(wl, *saved)
    return out


def other_workload(name: str, args, peaks: dict, host_layout: str = "BLOCKWISE",
                   rect_copies: bool = False):
    """Configs 3 and 4, and config 1 on a layer-wise host cache: a workload of
    its own (allocated here, freed on return) through both paths, the device
    gather/scatter in one launch, bit-exact round trips; MLA adds the
    per-request / batched request mix."""
    import gc
    wl = Workload(name, args.seed, host_layout=host_layout)
    try:
        desc = WORKLOADS[name]["desc"]
        if host_layout != "BLOCKWISE":
            w = WORKLOADS[name]
            left, ids = desc.split(" <-> ")[0], desc.split("; ", 1)[1]
            desc = (f"{left} <-> pinned layer-wise host [{w['layers']},{w['kv']},{w['nh']},"
                    f"{w['tokens']},{w['heads']},{w['dim']}]; {ids}")
        out = {"workload": desc, "bytes_per_step": wl.bytes_per_op}
        steps = max(3, args.steps // 2)
        out.update(path_rates(wl, steps, peaks))
        if rect_copies:
            from flexkv_amd import c_ext
            c_ext.set_copy_engine_policy(layerwise_scattered="rect_copies")
            try:
                out["ce_rect_copies"] = path_rates(wl, steps, peaks, (("ce_rect", True),))["ce_rect"]
            finally:
                c_ext.set_copy_engine_policy(layerwise_scattered="unset")
            out["overlap_with_compute"] = overlap_with_compute(wl, 3, rect_copies=True,
                                                               resident_probe=False)
        out["device_gather"] = standalone_gather(wl, steps)
        out["bit_exact"] = all(round_trip_bit_exact(wl, ce) for ce in (True, False))
        if wl.mla:
            out["request_batch"] = request_batch(wl, steps)
            out["bit_exact"] &= all(out["request_batch"][p]["bit_exact"] for p in ("ce", "kernel"))
        return out
    finally:
        del wl
        gc.collect()
        release_device_memory()


def disk_ceilings(d: str, nbytes: int):
    """Sequential O_DIRECT rates of the file system under `d`: `nbytes` written
    to one preallocated file (timed to the end of an fsync), then read back,
    for a few (threads, request size) shapes; the best of each is the
    ceiling the SSD tier is measured against."""
    import mmap
    from concurrent.futures import ThreadPoolExecutor

    path = os.path.join(d, "ceiling.bin")
    shapes = ((16, 8 << 20), (32, 1 << 20), (64, 1 << 20))
    runs = []
    try:
        fd = os.open(path, os.O_RDWR | os.O_CREAT | os.O_DIRECT, 0o600)
    except OSError as e:
        return {"skipped": f"O_DIRECT open failed: {e}"}
    try:
        for threads, io in shapes:
            nio = max(1, nbytes // io)
            bufs = []
            for _ in range(threads):
                b = mmap.mmap(-1, io)          # page aligned, as O_DIRECT needs
                b.write(os.urandom(io))
                bufs.append(b)
            try:
                os.posix_fallocate(fd, 0, nio * io)
                with ThreadPoolExecutor(max_workers=threads) as ex:
                    t0 = time.perf_counter()
                    list(ex.map(lambda i: os.pwritev(fd, [bufs[i % threads]], i * io),
                                range(nio)))
                    os.fsync(fd)
                    t_w = time.perf_counter() - t0
                    t0 = time.perf_counter()
                    list(ex.map(lambda i: os.preadv(fd, [bufs[i % threads]], i * io),
                                range(nio)))
                    t_r = time.perf_counter() - t0
            finally:
                for b in bufs:
                    b.close()
            gb = nio * io / 1e9
            runs.append({"threads": threads, "request_mib": io >> 20,
                         "write_gbps_with_fsync": round(gb / t_w, 3),
                         "read_gbps": round(gb / t_r, 3)})
    except OSError as e:
        return {"skipped": f"O_DIRECT I/O failed: {e}"}
    finally:
        os.close(fd)
        os.unlink(path)
    return {"seq_write_gbps_with_fsync": max(r["write_gbps_with_fsync"] for r in runs),
            "seq_read_gbps": max(r["read_gbps"] for r in runs),
            "how": f"O_DIRECT over {nbytes / 1e9:.2f} GB, best of the shapes in runs",
            "runs": runs}


def ssd_tier(wl: Workload, max_bytes: int = 1 << 30):
    """Host cache <-> SSD files for about 1 GiB of blocks: the rows the last
    D2H left in the host cache are copied to host blocks [0, n), written to
    SSD slots [0, n) (buffered writes, then fsync), read back into n random
    host blocks (one request per block) and into host blocks [n, 2n)
    (consecutive blocks merge into large requests); both reads are compared
    with the written rows bit for bit.  Run once with the threads engine and
    once with a 256-deep io_uring ring.  O_DIRECT reads when the chunk is a
    multiple of 4 KiB.  Files go to a temporary directory on this host's file
    system and are removed after; the file system's sequential O_DIRECT
    rates are measured in the same directory."""
    import shutil
    import tempfile

    import numpy as np

    from flexkv_amd.common.config import CacheConfig
    from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType
    from flexkv_amd.common.transfer import TransferType
    from flexkv_amd.storage.allocator import SSDAllocator
    from flexkv_amd.transfer.worker import CPUSSDDiskTransferWorker

    w = wl.w
    L = w["layers"]
    row = L * w["kv"] * wl.chunk
    n = int(min(len(wl.cids), max(1, max_bytes // row), w["nh"] // 4))
    d = tempfile.mkdtemp(prefix="flexkv_ssd_bench_")
    try:
        free = SSDAllocator.get_file_size_limit(d)
        if free < 4 * n * row:
            return {"skipped": f"{free / 2**30:.1f} GiB free under {d}"}
        fs = "?"
        with open("/proc/mounts") as f:
            best = ""
            for line in f:
                parts = line.split()
                if len(parts) > 2 and d.startswith(parts[1]) and len(parts[1]) >= len(best):
                    best, fs = parts[1], parts[2]
        mk = lambda nb: KVCacheLayout(wl.cl.type, L, nb, w["tokens"],
                                      w["heads"], w["dim"], is_mla=wl.mla)
        ssd_lay = mk(n)
        h = SSDAllocator.allocate(ssd_lay, wl.dtype, cache_dir=[d], max_blocks_per_file=n)
        first = torch.arange(n)
        base = wl.host_rows(wl.cids[:n])
        src = np.arange(n, dtype=np.int64)
        sids = np.arange(n, dtype=np.int64)
        rnd = (2 * n + torch.randperm(w["nh"] - 2 * n,
                                      generator=torch.Generator().manual_seed(7))[:n]).numpy()
        rnd = rnd.astype(np.int64)
        run = np.arange(n, 2 * n, dtype=np.int64)
        gb = n * row / 1e9

        def engine(entries: int, salt: int):
            # each engine writes rows of its own and reads into cleared blocks,
            # so one engine's result cannot pass for another's
            written = base ^ salt
            wl.set_host_rows(first, written)
            wl.set_host_rows(torch.from_numpy(rnd), torch.zeros_like(written))
            wl.set_host_rows(torch.arange(n, 2 * n), torch.zeros_like(written))
            cfg = CacheConfig(ssd_cache_iouring_entries=entries)
            worker = CPUSSDDiskTransferWorker(0, None, None, wl.host, h.get_file_list(),
                                              mk(w["nh"]), ssd_lay, wl.dtype,
                                              h.num_blocks_per_file, cfg)
            depth = worker.ioctx.iouring_depth
            if entries and not depth:
                worker.close()
                return {"skipped": "the kernel refused an io_uring ring"}
            t0 = time.perf_counter()
            worker._transfer_impl(src, sids, TransferType.H2DISK, 0, L)
            t_write = time.perf_counter() - t0
            for paths in h.get_file_list().values():
                for pth in paths:
                    fd = os.open(pth, os.O_RDONLY)
                    os.fsync(fd)
                    os.close(fd)
            t_sync = time.perf_counter() - t0
            t0 = time.perf_counter()
            worker._transfer_impl(sids, rnd, TransferType.DISK2H, 0, L)
            t_rnd = time.perf_counter() - t0
            t0 = time.perf_counter()
            worker._transfer_impl(sids, run, TransferType.DISK2H, 0, L)
            t_run = time.perf_counter() - t0
            stats = worker.ioctx.stats()
            worker.close()
            ok = bool(torch.equal(wl.host_rows(torch.from_numpy(rnd)), written) and
                      torch.equal(wl.host_rows(torch.arange(n, 2 * n)), written))
            return {"write_gbps_buffered": round(gb / t_write, 3),
                    "write_gbps_with_fsync": round(gb / t_sync, 3),
                    "read_gbps_random_host_blocks": round(gb / t_rnd, 3),
                    "read_gbps_consecutive_host_blocks": round(gb / t_run, 3),
                    "bit_exact": ok,
                    "io_counters": stats,
                    **({"iouring_depth": depth} if depth else
                       {"threads_per_device": cfg.ssd_threads_per_device})}

        threads = engine(0, 0x1111)
        uring = engine(256, 0x2222)
        disk = disk_ceilings(d, n * row)
        out = {"blocks": n, "bytes": n * row, "fs": fs,
               "read_io": ("O_DIRECT into page-aligned bounce buffers, then copied to the "
                           "pinned host cache" if wl.chunk % 4096 == 0 else "buffered"),
               "threads": threads, "io_uring": uring, "disk": disk,
               "bit_exact": threads["bit_exact"] and uring.get("bit_exact", True)}
        if "seq_read_gbps" in disk:
            out["read_frac_of_disk_seq"] = {
                name: {k: round(r[f"read_gbps_{k}_host_blocks"] / disk["seq_read_gbps"], 4)
                       for k in ("random", "consecutive")}
                for name, r in (("threads", threads), ("io_uring", uring)) if "bit_exact" in r}
        return out
    finally:
        shutil.rmtree(d, ignore_errors=True)


def cpu_baseline(wl: Workload, budget_s: float):
    """The oracle's block-partitioned memcpy (oracle/kv_oracle.c) on this host's
    cores: D2H from host-resident copies of the selected GPU blocks into the
    pinned host cache, same ids and geometry."""
    import numpy as np

    import oracle

    oracle.build()
    threads = len(os.sched_getaffinity(0))
    n = len(wl.gids)
    # host-resident "GPU" layers holding exactly the moved blocks, in id order
    src = [t[:, wl.gids.to(wl.dev)].cpu().contiguous() for t in wl.layers]
    local = np.arange(n, dtype=np.int64)
    cids = wl.cids.numpy()
    gblk = wl.gblk
    gkv = wl.gblk * n

    def one(th):
        oracle.transfer_kv_blocks(local, src, gkv, gblk, cids, wl.host, wl.ckv, wl.clay, wl.cblk,
                                  wl.chunk, 0, False, use_ce_transfer=True, is_mla=wl.mla,
                                  num_threads=th)

    out = {}
    for th in (threads, 1):
        one(th)  # warm
        reps, t0 = 0, time.perf_counter()
        while True:
            one(th)
            reps += 1
            el = time.perf_counter() - t0
            if el > budget_s / 2 or reps >= 1000:
                break
        out[th] = (wl.bytes_per_op * reps / el / 1e9, reps, el)
    return threads, out


KERNEL_SOURCE = os.path.join(ROOT, "flexkv_amd", "csrc", "kv_transfer.hip")
# The kernel section of KERNEL_SOURCE ends where the next definition begins.
KERNEL_SECTION_END = b"// A system-scope acquire in every workgroup."


def kernel_section_sha16(path: str = KERNEL_SOURCE) -> str:
    """sha256 prefix of the transfer kernels' source: kv_transfer.hip from its
    start (build macros, CopyArgs, PackArgs) to the end of the data-moving
    kernels (kv_chunk_copy_kernel, kv_pack_kernel, kv_pack_span_kernel,
    stage_ids_kernel), the part that decides which bytes the kernels read and
    write.  Comments,
    blank lines and indentation are left out, so a change to a comment keeps
    the key and any change to the code changes it."""
    import hashlib
    import re
    with open(path, "rb") as fh:
        text = fh.read()
    end = text.find(KERNEL_SECTION_END)
    code = (text if end < 0 else text[:end]).decode()
    code = re.sub(r"/\*.*?\*/", " ", code, flags=re.S)
    lines = (re.sub(r"//.*", "", ln).strip() for ln in code.splitlines())
    code = "\n".join(ln for ln in lines if ln)
    return hashlib.sha256(code.encode()).hexdigest()[:16]


def measured_traffic(workload: str, run: int, alg_bytes: int) -> dict:
    """HBM bytes per gather launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes (calibrated against a plain 1 GiB copy), when they were
    taken on this workload, this launch size and this kernel source (the
    profile records the sha of the kernel section of kv_transfer.hip it was
    taken with); else null, with the reason."""
    path = os.path.join(ROOT, "profiles", f"kv_gather_{workload}_counters.json")
    rel = os.path.relpath(path, ROOT)
    if run or not os.path.exists(path):
        return {"bytes": None, "source": f"no counter profile for this workload ({rel})"}
    with open(path) as fh:
        prof = json.load(fh)
    g = prof["gather"]
    if g["algorithmic_bytes_per_launch"] != alg_bytes:
        return {"bytes": None, "source": f"{rel} was taken at another launch size"}
    want = kernel_section_sha16()
    if prof.get("kernel_sha16") != want:
        return {"bytes": None, "source": f"{rel} was taken with another transfer kernel "
                                         f"({prof.get('kernel_sha16')} != {want})"}
    return {"bytes": g["traffic_bytes_per_launch"],
            "source": f"{rel} (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes of "
                      f"bench.py --counters, transfer kernel sha {want})"}


def counters_pass(args) -> int:
    """Kernels for `rocprofv3 --pmc` passes: the calibration copy first, so the
    per-dispatch counter of a copy of known size scales the others; then 3
    gathers, 3 scatters, 3 zero-copy D2H and 3 zero-copy H2D transfers of the
    step's blocks, then one copy-engine D2H and one H2D (their gather and
    scatter pieces)."""
    wl = Workload(args.workload, args.seed, args.run, host=True)
    cal = torch.empty(1 << 30, dtype=torch.uint8, device=wl.dev)
    cal_dst = torch.empty_like(cal)
    torch.cuda.synchronize()
    cal_dst.copy_(cal)
    torch.cuda.synchronize()
    buf = torch.empty(wl.bytes_per_op, dtype=torch.uint8, device=wl.dev)
    for _ in range(3):
        wl.gather(buf)
    for _ in range(3):
        wl.gather(buf, scatter=True)
    del buf
    for h2d in (False, True):
        for _ in range(3):
            wl.transfer(h2d, False)
    # one copy-engine D2H and one H2D: their gather and scatter pieces
    for h2d in (False, True):
        wl.transfer(h2d, True)
    torch.cuda.synchronize()
    print(json.dumps({"calibration_copy_bytes": cal.numel(), "gather_launches": 3,
                      "scatter_launches": 3, "d2h_launches": 3, "h2d_launches": 3,
                      "copy_engine_transfers": 2,
                      "moved_bytes_per_launch": wl.bytes_per_op}), flush=True)
    return 0


def configs_on_step(args, wl: Workload, peaks: dict, result: dict) -> dict:
    """Configs 1 and 2 on the step's own tensors: both paths of the Llama-3-8B
    step and its fragmentation sweep."""
    cfg = {}
    steps = max(3, args.steps // 2)
    c1 = {"workload": WORKLOADS["llama3-8b"]["desc"], "bytes_per_step": wl.bytes_per_op}
    c1.update(path_rates(wl, steps, peaks))
    c1["device_gather"] = {"gather_gbps_hbm": result["roofline"]["achieved"],
                           "gather_frac_hbm": result["roofline"]["frac"],
                           "scatter_gbps_hbm": result["roofline"]["scatter"]["achieved"],
                           "scatter_frac_hbm": result["roofline"]["scatter"]["frac"]}
    c1["bit_exact"] = all(round_trip_bit_exact(wl, ce) for ce in (True, False))
    cfg["cfg1_llama3-8b"] = c1
    log(f"cfg1: {c1}")
    cfg["cfg2_llama3-8b_fragmentation"] = fragmentation_sweep(wl, steps, peaks)
    return cfg


def tp_group(peaks: dict, reps: int = 3, tp: int = 8, seed: int = 1003) -> dict:
    """The Llama-3-70B TP-8 shard's whole tensor-parallel group on this one
    GPU: eight ranks, each with its own K/V [8192,16,1,128] bf16 per layer
    (one KV head, 80 layers), sharing a pinned block-wise host cache whose
    chunk holds the eight ranks' chunks side by side ([4096,80,2,16,8,128]).
    One group transfer moves 2048 random blocks on every rank (10 GiB)
    through c_ext.TPTransferThreadGroup (a thread and a stream per rank, rank
    r at byte offset r * 4 KiB of each 32 KiB host chunk).  The ranks share
    this GPU's host link, which bounds the aggregate; across GPUs each rank
    has a link of its own.  Also: the same bytes as eight one-rank calls in
    turn (fkv_transfer_kv_blocks with the rank's offset), a round trip
    checked bit for bit, and 16 host blocks checked slot by slot."""
    import ctypes
    import gc
    from flexkv_amd import _lib, c_ext
    from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType
    from flexkv_amd.storage.allocator import CPUAllocator
    L, ng, nh, n, tokens, dim = 80, 8192, 4096, 2048, 16, 128
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(seed)
    ranks = []
    for _ in range(tp):
        layers = []
        for _ in range(L):
            t = torch.empty((2, ng, tokens, 1, dim), dtype=torch.bfloat16, device=dev)
            t.normal_(generator=gen)
            layers.append(t)
        ranks.append(layers)
    cl = KVCacheLayout(KVCacheLayoutType.BLOCKWISE, L, nh, tokens, tp, dim)
    host = CPUAllocator.allocate(cl, torch.bfloat16).get_tensor()
    cpu_gen = torch.Generator().manual_seed(seed + 1)
    gids = torch.randperm(ng, generator=cpu_gen)[:n].to(torch.int64)
    cids = torch.randperm(nh, generator=cpu_gen)[:n].to(torch.int64)
    chunk = tokens * dim * 2
    gkv, gblk = ng * chunk, chunk
    _, ckv, clay, cblk = cl.byte_strides(torch.bfloat16)
    nbytes = tp * n * L * 2 * chunk
    out = {"workload": f"Llama-3-70B at TP = 8 on one GPU: {tp} ranks x 80 layers, K/V "
                       f"[8192,16,1,128] bf16 each <-> pinned host [4096,80,2,16,8,128]; "
                       f"2048 random distinct ids on every rank",
           "ranks": tp, "bytes_per_op": nbytes}
    grp = c_ext.TPTransferThreadGroup(tp, ranks, host, 0)
    lib = _lib.load()
    try:
        def group_move(h2d):
            grp.tp_group_transfer(gids, gkv, gblk, chunk, cids, ckv, clay, cblk, tp * chunk, -1,
                                  h2d, False, 0, L, False)

        ptr_tables = [(ctypes.c_void_p * L)(*[t.data_ptr() for t in r]) for r in ranks]

        def ranks_in_turn(h2d):
            st = torch.cuda.current_stream().cuda_stream
            for r in range(tp):
                _lib.check(lib.fkv_transfer_kv_blocks(
                    n, 0, L, gids.data_ptr(), ptr_tables[r], gkv, gblk, cids.data_ptr(),
                    host.data_ptr(), ckv, clay, cblk, r * chunk, chunk, st, -1, int(h2d), 0, 0),
                    "fkv_transfer_kv_blocks")
        for name, fn in (("group", group_move), ("ranks_in_turn", ranks_in_turn)):
            for h2d in (False, True):
                d = "h2d" if h2d else "d2h"
                s, _, _ = time_steps(lambda: fn(h2d), reps, 1)
                out[f"{name}_{d}_gbps"] = round(nbytes / s / 1e9, 2)
                if name == "group":
                    out[f"group_{d}_frac_link"] = round(nbytes / s / 1e9 / peaks[d], 4)
        # round trip: D2H, rank blocks zeroed in place, H2D, compared
        g = gids.to(dev)
        group_move(False)
        torch.cuda.synchronize()
        rows = host.view(nh, L, 2, tp, chunk // 2)
        sample = torch.arange(16)
        ok = True
        for r in range(tp):
            for l in range(0, L, 7):
                want = ranks[r][l][:, g[sample]].reshape(2, 16, -1).transpose(0, 1).cpu()
                ok &= bool(torch.equal(rows[cids[sample], l, :, r].view(torch.int16),
                                       want.reshape(16, 2, -1).view(torch.int16)))
        saved = [[t.index_select(1, g) for t in r] for r in ranks]
        for r in ranks:
            for t in r:
                t.index_fill_(1, g, 0)
        torch.cuda.synchronize()    # the ranks run on streams of their own
        group_move(True)
        torch.cuda.synchronize()
        ok &= all(torch.equal(t.index_select(1, g), s)
                  for r, sr in zip(ranks, saved) for t, s in zip(r, sr))
        out["bit_exact"] = ok
        del saved
    finally:
        grp.close()
        del ranks, host
        gc.collect()
        release_device_memory()
    return out


def other_configs(args, peaks: dict, cfg: dict) -> dict:
    """The configurations with tensors of their own, each allocated and freed
    in turn: the CPU plumbing shape, Llama-3-8B on a layer-wise host cache,
    the Llama-3-70B TP-8 shard and the DeepSeek-V3 MLA latent cache with its
    request mix, and the 70B shard's whole eight-rank tensor-parallel group
    sharing this GPU (tp_group).  Every entry of the benchmark set (with configs_on_step's)
    gives GB/s on both paths with fractions of the measured link and of
    nominal PCIe Gen5 x16, the copy-engine path's gather/scatter piece rates,
    the device gather/scatter in one launch, and a bit-exact round trip."""
    t0 = time.perf_counter()
    for key, name, layout, rect in (("cfg0_plumbing", "plumbing", "BLOCKWISE", False),
                                    ("cfg1_llama3-8b_layerwise_host", "llama3-8b", "LAYERWISE",
                                     True),
                                    ("cfg3_llama3-70b-tp8", "llama3-70b-tp8", "BLOCKWISE", False),
                                    ("cfg4_mla-dsv3", "mla-dsv3", "BLOCKWISE", False)):
        cfg[key] = other_workload(name, args, peaks, layout, rect)
        log(f"{key}: {cfg[key]}")
    cfg["cfg3_llama3-70b-tp8_group"] = tp_group(peaks)
    log(f"cfg3_llama3-70b-tp8_group: {cfg['cfg3_llama3-70b-tp8_group']}")
    cfg["bit_exact"] = all(v.get("bit_exact", True) for v in cfg.values()
                           if isinstance(v, dict)) and all(
        r["bit_exact"] for r in cfg["cfg2_llama3-8b_fragmentation"].values())
    cfg["seconds"] = round(time.perf_counter() - t0, 1)
    return cfg


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="llama3-8b", choices=sorted(WORKLOADS))
    ap.add_argument("--run", type=int, default=0, help="contiguous id runs of this length")
    ap.add_argument("--host-layout", default="BLOCKWISE", choices=["BLOCKWISE", "LAYERWISE"],
                    help="host cache layout (the reference's CacheConfig default is LAYERWISE)")
    ap.add_argument("--path", default=None, choices=["kernel", "ce"],
                    help="D2H/H2D path reported as value (default: the product default)")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--quick", action="store_true", help="skip baselines (for profiling runs)")
    ap.add_argument("--layerwise-only", action="store_true",
                    help="run only the layer-wise H2D section (sync per layer, async handle, "
                         "overlap with per-layer GEMMs) and print its JSON (for profiling runs)")
    ap.add_argument("--tp-group-only", action="store_true",
                    help="run only the eight-rank tensor-parallel group section (the Llama-3-70B "
                         "TP-8 shard's whole group on this GPU) and print its JSON")
    ap.add_argument("--duplex-only", action="store_true",
                    help="run only the both-directions-at-once section and print its JSON")
    ap.add_argument("--worker-ops", action="store_true",
                    help="run only the worker-op section (thread and process workers, 16-block "
                         "and full-step ops, each inside a roctx range) and print its JSON "
                         "(for marker-trace profiling runs)")
    ap.add_argument("--overlap-only", action="store_true",
                    help="run only the overlap-with-compute section for --workload and "
                         "--host-layout (layer-wise: the rect-copy policy on the copy-engine "
                         "runs) and print its JSON (for kernel-trace profiling runs)")
    ap.add_argument("--seed", type=int, default=1001)
    ap.add_argument("--counters", action="store_true",
                    help="run only the kernels a PMC pass needs: a 1 GiB plain device copy "
                         "(calibration), then 3 gathers, 3 scatters, 3 zero-copy D2H and 3 "
                         "zero-copy H2D transfers of the step's blocks")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the transfer path is per-GPU (one PCIe link, one HBM); "
              "multi-GPU runs are out of scope for this package", file=sys.stderr)
        return 2
    full_run = not (args.quick or args.counters or args.layerwise_only or args.worker_ops
                    or args.duplex_only or args.overlap_only)
    ceilings = device_ceilings() if full_run else None
    abi_latency = c_abi_latency() if full_run else None
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2

    from flexkv_amd import _lib
    from flexkv_amd.common.config import CacheConfig

    _lib.load()
    if args.counters:
        return counters_pass(args)
    cfg = CacheConfig()
    default_ce = {"kernel": False, "ce": True}[args.path] if args.path else cfg.use_ce_transfer_d2h
    all_configs = (args.workload == "llama3-8b" and not args.run and args.host_layout == "BLOCKWISE"
                   and not (args.quick or args.layerwise_only or args.worker_ops
                            or args.duplex_only or args.overlap_only))
    wl = Workload(args.workload, args.seed, args.run, host_layout=args.host_layout)
    gb = wl.bytes_per_op / 1e9
    if args.layerwise_only:
        wl.transfer(False, default_ce)   # the host cache holds the blocks read back below
        print(json.dumps({"layerwise_h2d": layerwise_h2d(wl, args.steps)}), flush=True)
        return 0
    if args.worker_ops:
        print(json.dumps({"worker_ops": worker_ops(wl, reps=max(5, args.steps),
                                                   process=not args.quick)}), flush=True)
        return 0
    if args.tp_group_only:
        print(json.dumps({"tp_group": tp_group(link_peaks(wl))}), flush=True)
        return 0
    if args.duplex_only:
        pk = link_peaks(wl)
        d = duplex(wl, reps=max(3, args.steps))
        d["duplex_peak_gbps_measured"] = round(pk["duplex"], 2)
        d["one_way_peaks_gbps"] = [round(pk["d2h"], 2), round(pk["h2d"], 2)]
        print(json.dumps({"duplex": d}), flush=True)
        return 0
    if args.overlap_only:
        layerwise = args.host_layout == "LAYERWISE"
        print(json.dumps({"overlap_with_compute": overlap_with_compute(
            wl, 3, rect_copies=layerwise, resident_probe=True)}), flush=True)
        return 0

    # primary: D2H on the default path, library kernel timing on
    _lib.profile_enable(True)
    d2h_s, d2h_med, d2h_best = time_steps(lambda: wl.transfer(False, default_ce), args.steps,
                                          args.warmup)
    prof_d2h = _lib.profile_read()
    _lib.profile_enable(True)
    h2d_s, h2d_med, h2d_best = time_steps(lambda: wl.transfer(True, default_ce), args.steps,
                                          args.warmup)
    prof_h2d = _lib.profile_read()
    _lib.profile_enable(False)
    log(f"D2H {gb / d2h_s:.2f} GB/s, H2D {gb / h2d_s:.2f} GB/s "
        f"({'ce' if default_ce else 'kernel'} path)")

    # parity of the last D2H/H2D pair (H2D wrote back what D2H stored)
    wl.transfer(False, default_ce)
    parity = wl.check()
    log(f"bit-exact check of all {len(wl.gids)} blocks: {parity}")

    # Device-side gather/scatter (the HBM-bound kernel of the copy-engine path)
    # over the same blocks into one packed HBM buffer; its launches are timed
    # with HIP events on the launch stream by the library.
    buf = torch.empty(wl.bytes_per_op, dtype=torch.uint8, device=wl.dev)
    _lib.profile_enable(True)
    g_s, _, _ = time_steps(lambda: wl.gather(buf), args.steps, args.warmup)
    prof_g = _lib.profile_read()
    _lib.profile_enable(True)
    s_s, _, _ = time_steps(lambda: wl.gather(buf, scatter=True), args.steps, args.warmup)
    prof_s = _lib.profile_read()
    _lib.profile_enable(False)
    gather_ok = bool(torch.equal(buf.view(torch.int16), wl.packed_expected().view(torch.int16)))
    del buf
    release_device_memory()

    def kernel_rate(prof):
        launches = max(1, prof["kernel_launches"])
        avg_ms = prof["kernel_ms"] / launches
        hbm = 2 * prof["kernel_bytes"] / launches   # one read + one write per byte moved
        return avg_ms, hbm, (hbm / (avg_ms * 1e-3) / 1e9 if avg_ms > 0 else 0.0)

    g_ms, g_bytes, g_rate = kernel_rate(prof_g)
    s_ms, s_bytes, s_rate = kernel_rate(prof_s)
    traffic = measured_traffic(args.workload, args.run, int(g_bytes))
    # the gather and scatter pieces the copy-engine path itself launched in
    # the timed D2H / H2D steps (library event timing on the launch stream)
    in_path = {}
    if default_ce:
        for key, prof in (("gather", prof_d2h), ("scatter", prof_h2d)):
            if prof["dma_batches"] and prof["kernel_launches"]:
                p_ms, p_bytes, p_rate = kernel_rate(prof)
                in_path[key] = {"achieved": round(p_rate, 1),
                                "frac": round(p_rate / HBM_PEAK_GBS, 4),
                                "avg_piece_ms": round(p_ms, 4),
                                "algorithmic_bytes_per_piece": int(p_bytes),
                                "pieces_per_step": round(prof["kernel_launches"] /
                                                         (args.steps + args.warmup), 2)}
    z_ms = prof_d2h["kernel_ms"] / max(1, prof_d2h["kernel_launches"])
    log(f"device gather {g_rate:.0f} GB/s, scatter {s_rate:.0f} GB/s of HBM; packed bytes "
        f"bit-exact: {gather_ok}")

    result = {
        "metric": METRIC,
        "value": round(gb / d2h_s, 3),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(d2h_s * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",   # a byte copy: no arithmetic on the values, which are bf16
        "data": "synthetic: KV values ~N(0,1) bf16 from torch's seeded device generator; "
                "block ids from a seeded permutation",
        "config": {"workload": WORKLOADS[args.workload]["desc"] +
                   (f"; ids in contiguous runs of {args.run}" if args.run else "") +
                   ("; layer-wise host cache [32,2,16384,16,8,128]"
                    if args.host_layout == "LAYERWISE" and args.workload == "llama3-8b" else
                    f"; {args.host_layout.lower()} host cache"
                    if args.host_layout != "BLOCKWISE" else ""),
                   "direction": "D2H", "path": "ce" if default_ce else "kernel",
                   "element_dtype": "bf16",
                   "bytes_per_step": wl.bytes_per_op},
        "d2h": {"gbps": round(gb / d2h_s, 3), "median_ms": round(d2h_med * 1e3, 3),
                "best_ms": round(d2h_best * 1e3, 3),
                **({"gather_piece_avg_ms": round(z_ms, 4),
                    "sdma_copies": prof_d2h["dma_copies"], "sdma_bytes": prof_d2h["dma_bytes"]}
                   if default_ce else {"kernel_avg_ms": round(z_ms, 4)})},
        "h2d": {"gbps": round(gb / h2d_s, 3), "ms_per_step": round(h2d_s * 1e3, 3),
                "median_ms": round(h2d_med * 1e3, 3), "best_ms": round(h2d_best * 1e3, 3)},
        "bit_exact": parity and gather_ok,
        "roofline": {"bound": "hbm",
                     "kernel": "kv_chunk_copy_kernel<D2H, staging>: device-side gather of the "
                               "step's blocks into one packed HBM buffer",
                     "achieved": round(g_rate, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(g_rate / HBM_PEAK_GBS, 4),
                     "traffic": traffic["bytes"],
                     "traffic_source": traffic["source"],
                     "avg_launch_ms": round(g_ms, 4), "launches": prof_g["kernel_launches"],
                     "algorithmic_bytes_per_launch": int(g_bytes),
                     "bytes_rule": "2 x moved bytes (scattered 32 KiB reads + packed writes)",
                     "scatter": {"achieved": round(s_rate, 1), "frac": round(s_rate / HBM_PEAK_GBS, 4),
                                 "avg_launch_ms": round(s_ms, 4)},
                     **({"in_path": in_path} if in_path else {}),
                     **({"device_ceilings": {
                         "read_gbps": ceilings["read_gbps"], "write_gbps": ceilings["write_gbps"],
                         "copy_gbps": ceilings["copy_gbps"],
                         "gather_frac_of_copy": round(g_rate / ceilings["copy_gbps"], 4),
                         "scatter_frac_of_copy": round(s_rate / ceilings["copy_gbps"], 4),
                         "how": "flexkv_amd/hbm_ceiling: plain 16 B/lane read-only, write-only "
                                "and copy kernels over 4 GiB, launch shapes swept, best of 10 "
                                "launches each; rates count bytes read + bytes written"}}
                        if ceilings else {})},
        "library_profile": {"d2h": prof_d2h, "h2d": prof_h2d, "gather": prof_g,
                            "scatter": prof_s},
    }

    if not args.quick:
        peaks = link_peaks(wl)
        result["host_link"] = {
            "bound": "PCIe Gen5 x16 (host link); the zero-copy kernel is bound here, not by HBM",
            "d2h_peak_gbps_measured": round(peaks["d2h"], 2),
            "h2d_peak_gbps_measured": round(peaks["h2d"], 2),
            "d2h_frac": round((gb / d2h_s) / peaks["d2h"], 4),
            "h2d_frac": round((gb / h2d_s) / peaks["h2d"], 4),
            "pcie_gen5_x16_gbps_nominal": PCIE_GEN5_X16_GBS,
            "d2h_frac_pcie_gen5_x16": round((gb / d2h_s) / PCIE_GEN5_X16_GBS, 4),
            "h2d_frac_pcie_gen5_x16": round((gb / h2d_s) / PCIE_GEN5_X16_GBS, 4),
            **({} if default_ce else
               {"d2h_kernel_frac": round((gb / (z_ms * 1e-3)) / peaks["d2h"], 4)}),
            "d2d_copy_gbps_measured": round(peaks["d2d_copy_read_plus_write"], 1),
            "duplex_peak_gbps_measured": round(peaks["duplex"], 2),
            "how": "best of 8 hipMemcpyAsync over 1 GiB contiguous pinned host memory per "
                   "direction; duplex = a 1 GiB D2H and a 1 GiB H2D on two streams at once, "
                   "both directions' bytes over the wall time; D2D = 4 GiB device copy "
                   "counted read+write",
        }
        paths = {}
        for name, h2d, ce, cus in (("d2h_kernel", False, False, -1), ("d2h_ce", False, True, -1),
                                   ("h2d_kernel", True, False, -1), ("h2d_ce", True, True, -1),
                                   ("d2h_kernel_8cus", False, False, 8),
                                   ("h2d_kernel_8cus", True, False, 8)):
            s, med, best = time_steps(lambda: wl.transfer(h2d, ce, cus), args.steps, 1)
            paths[name] = round(gb / s, 3)
            log(f"path {name}: {gb / s:.2f} GB/s")
        result["paths_gbps"] = paths
        t0 = time.perf_counter()
        wl.transfer(False, 2)
        el = time.perf_counter() - t0
        result["ce_per_chunk_loop"] = {
            "gbps": round(gb / el, 3), "ms": round(el * 1e3, 1),
            "what": "reference copy-engine algorithm restated with HIP: one hipMemcpyAsync per "
                    "(layer, K|V, block) chunk (csrc/transfer.cu:97-121), D2H, one op"}
        log(f"CE per-chunk loop: {gb / el:.2f} GB/s")
        result["layerwise_h2d"] = layerwise_h2d(wl, args.steps)
        log(f"layer-wise H2D: {result['layerwise_h2d']}")
        result["engine_layerwise_read"] = engine_layerwise(wl, args.steps)
        log(f"engine layer-wise read: {result['engine_layerwise_read']}")
        result["engine_put_get"] = engine_put_get(wl, max(3, args.steps // 2))
        log(f"engine put and get: {result['engine_put_get']}")
        result["call_latency"] = call_latency(wl)
        log(f"call latency: {result['call_latency']}")
        result["call_latency_c_abi"] = abi_latency
        result["worker_ops"] = worker_ops(wl)
        log(f"worker ops: {result['worker_ops']}")
        result["overlap_with_compute"] = overlap_with_compute(wl)
        log(f"overlap with compute: {result['overlap_with_compute']}")
        result["duplex"] = duplex(wl)
        for name in ("ce", "kernel"):
            result["duplex"][f"{name}_frac_duplex_peak"] = round(
                result["duplex"][f"{name}_aggregate_gbps"] / peaks["duplex"], 4)
        log(f"duplex: {result['duplex']}")
        if wl.mla:
            result["request_batch"] = request_batch(wl, args.steps)
            log(f"request batch: {result['request_batch']}")
        wl.transfer(False, default_ce)     # host rows of the step's ids hold the GPU blocks
        result["ssd_tier"] = ssd_tier(wl)   # overwrites host blocks it stages through
        log(f"SSD tier: {result['ssd_tier']}")
        threads, cpu = cpu_baseline(wl, args.cpu_budget)
        v, reps, el = cpu[threads]
        v1, reps1, el1 = cpu[1]
        result["cpu_baseline"] = {
            "value": round(v, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"D2H of the same {len(wl.gids)} blocks x {WORKLOADS[args.workload]['layers']} "
                      f"layers ({gb:.2f} GB per op) from host-resident copies of the GPU blocks "
                      f"into the pinned host cache; {reps} ops in {el:.1f}s on {threads} threads",
            "single_thread_gbps": round(v1, 3),
        }
        log(f"CPU baseline: {v:.2f} GB/s on {threads} threads, {v1:.2f} GB/s on 1")
        if all_configs:
            import gc
            cfg = configs_on_step(args, wl, peaks, result)
            del wl
            gc.collect()
            release_device_memory()
            result["configs"] = other_configs(args, peaks, cfg)
            parity = parity and result["configs"]["bit_exact"]
            result["bit_exact"] = result["bit_exact"] and result["configs"]["bit_exact"]

    print(json.dumps(result), flush=True)
    return 0 if (parity and gather_ok) else 1


def end_helper_processes() -> None:
    """Leave no process behind: join (or, after 5 s, terminate) any worker
    process still alive, then stop the multiprocessing resource tracker that
    spawned workers and their semaphores started.  The tracker would exit on
    its own once this process has, but only after it notices."""
    import multiprocessing as mp
    from multiprocessing import resource_tracker
    for p in mp.active_children():
        p.join(timeout=5)
        if p.is_alive():
            p.terminate()
            p.join(timeout=5)
    tracker = resource_tracker._resource_tracker
    if not mp.active_children() and getattr(tracker, "_pid", None) is not None:
        tracker._stop()


if __name__ == "__main__":
    try:
        rc = main()
    finally:
        end_helper_processes()
    sys.exit(rc)
