"""Worker-level transfer benchmark with the reference's command line
(benchmarks/benchmark_workers.py:180-291 in FlexKV).

One transfer op over block ids 0..n-1 (or a random permutation of them with
--shuffle-ids) runs --warmup-round untimed and --benchmark-round timed times
through a transfer worker in its own process, each op submitted and waited for
on the finished-ops queue, as the reference does (:159-167, :232-240):

* H2D / D2H: a GPUCPUTransferWorker over per-layer device tensors of n blocks
  (the reference sizes the GPU cache to the op, :35) and a pinned host cache
  of CacheConfig.num_cpu_blocks blocks, with the transfer path and compute
  units the config names;
* H2DISK / DISK2H: a CPUSSDDiskTransferWorker over that host cache and SSD
  cache files of CacheConfig.num_ssd_blocks blocks under
  CacheConfig.ssd_cache_dir (DISK2H writes the blocks first, :226-231).

The reference's harness fixes the host layout to LAYERWISE and the transfer
path to its SM kernel with 8 SMs (:56-63, :87-100); here both come from the
config file.  The default, example_config.json beside this file, sets the
same; mi355x_config.json sets this package's defaults (block-wise host cache,
copy-engine path).  The printed "GB" figures follow the reference's arithmetic, bytes over
2^30 (:241-247); the final JSON line also gives 10^9-byte GB/s.

    python -m flexkv_amd.benchmarks.benchmark_workers --transfer-type D2H \\
        --num-blocks 1024 --shuffle-ids
"""
from __future__ import annotations

import argparse
import copy
import json
import multiprocessing as mp
import os
import sys
import tempfile
import time
from dataclasses import dataclass, fields
from typing import Any, Dict, Tuple

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from flexkv_amd.common.config import CacheConfig, ModelConfig  # noqa: E402
from flexkv_amd.common.debug import flexkv_logger  # noqa: E402
from flexkv_amd.common.memory_handle import TensorSharedHandle  # noqa: E402
from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType  # noqa: E402
from flexkv_amd.common.transfer import (TransferDescriptor, TransferOp,  # noqa: E402
                                        TransferType)
from flexkv_amd.storage.allocator import HostCacheSpec, SSDAllocator  # noqa: E402
from flexkv_amd.transfer.worker import (CPUSSDDiskTransferWorker,  # noqa: E402
                                        GPUCPUTransferWorker, tpGPUCPUTransferWorker)

DEFAULT_CONFIG = os.path.join(HERE, "example_config.json")


@dataclass
class BenchmarkConfig:
    transfer_type: TransferType = TransferType.H2D
    num_layers_to_transfer: int = -1
    num_blocks_to_transfer: int = 16
    shuffle_ids: bool = False
    warmup_round: int = 1
    benchmark_round: int = 10


def _pick(cls, d: Dict[str, Any]) -> Dict[str, Any]:
    """The keys of `d` that are fields of dataclass `cls`; the rest (remote
    cache, tracing, GDS: parts this package does not have) are reported and
    dropped."""
    names = {f.name for f in fields(cls)}
    extra = sorted(set(d) - names)
    if extra:
        flexkv_logger.info(f"{cls.__name__}: ignoring {', '.join(extra)}")
    return {k: v for k, v in d.items() if k in names}


def make_configs(args: argparse.Namespace) -> Tuple[ModelConfig, CacheConfig, BenchmarkConfig]:
    with open(args.config) as f:
        cfg = json.load(f)
    m = _pick(ModelConfig, cfg["ModelConfig"])
    if isinstance(m.get("dtype"), str):
        m["dtype"] = getattr(torch, m["dtype"])
    model = ModelConfig(**m)
    c = _pick(CacheConfig, cfg["CacheConfig"])
    for k in ("gpu_kv_layout_type", "cpu_kv_layout_type", "ssd_kv_layout_type"):
        if isinstance(c.get(k), str):
            c[k] = KVCacheLayoutType[c[k].upper()]
    cache = CacheConfig(**c)
    bench = BenchmarkConfig(transfer_type=TransferType(args.transfer_type),
                            num_layers_to_transfer=args.num_layers,
                            num_blocks_to_transfer=args.num_blocks,
                            shuffle_ids=args.shuffle_ids, warmup_round=args.warmup_round,
                            benchmark_round=args.benchmark_round)
    return model, cache, bench


def _layout(kind: KVCacheLayoutType, model: ModelConfig, cache: CacheConfig,
            num_blocks: int) -> KVCacheLayout:
    return KVCacheLayout(kind, model.num_layers, num_blocks, cache.tokens_per_block,
                         model.num_kv_heads, model.head_size, is_mla=model.use_mla)


def create_cpu_gpu_worker(model: ModelConfig, cache: CacheConfig, bench: BenchmarkConfig,
                          queue: Any):
    """The GPU<->CPU worker of the reference harness (:43-117): with tp_size
    > 1 a tpGPUCPUTransferWorker over tp_size ranks, each holding
    num_kv_heads / tp_size heads (all heads under MLA).  Every rank's cache
    is on cuda:0 (the reference puts rank r on GPU r and refuses a tp_size
    above the device count, :185-187); the ranks then share one GPU's link."""
    n = bench.num_blocks_to_transfer
    tp = model.tp_size
    gpu_layout = _layout(KVCacheLayoutType.LAYERWISE, model, cache, n)
    if tp > 1 and not model.use_mla:
        gpu_layout = gpu_layout.div_head(tp)
    cpu_layout = _layout(cache.cpu_kv_layout_type, model, cache, cache.num_cpu_blocks)
    per_layer = gpu_layout.get_total_elements() // model.num_layers
    ranks = [[torch.zeros(per_layer, dtype=model.dtype, device="cuda:0")
              for _ in range(model.num_layers)] for _ in range(tp)]
    common = dict(use_ce_transfer_h2d=cache.use_ce_transfer_h2d,
                  use_ce_transfer_d2h=cache.use_ce_transfer_d2h,
                  transfer_sms_h2d=cache.transfer_sms_h2d,
                  transfer_sms_d2h=cache.transfer_sms_d2h)
    spec = HostCacheSpec(cpu_layout, model.dtype)
    if tp == 1:
        handle = GPUCPUTransferWorker.create_worker(
            0, queue, [TensorSharedHandle(t) for t in ranks[0]], spec, gpu_layout, cpu_layout,
            model.dtype, 0, **common)
    else:
        handle = tpGPUCPUTransferWorker.create_worker(
            0, queue, [[TensorSharedHandle(t) for t in layers] for layers in ranks], spec,
            gpu_layout, cpu_layout, model.dtype, tp, 0, **common)
    return handle, ranks


def create_cpu_ssd_worker(model: ModelConfig, cache: CacheConfig, queue: Any, ssd_dir: str):
    cpu_layout = _layout(cache.cpu_kv_layout_type, model, cache, cache.num_cpu_blocks)
    ssd_layout = _layout(cache.ssd_kv_layout_type, model, cache, cache.num_ssd_blocks)
    ssd = SSDAllocator.allocate(ssd_layout, model.dtype, cache_dir=ssd_dir,
                                max_blocks_per_file=cache.max_blocks_per_file)
    spec = HostCacheSpec(cpu_layout, model.dtype, pinned=cache.use_pinned_memory)
    handle = CPUSSDDiskTransferWorker.create_worker(
        10, queue, spec, ssd.get_file_list(), cpu_layout,
        ssd_layout, model.dtype, ssd.num_blocks_per_file, cache)
    return handle, ssd


def launch_transfer(handle, queue, op: TransferOp) -> None:
    handle.submit_transfer(op)
    done = queue.get()
    if done != op.op_id:
        raise RuntimeError(f"worker finished op {done}, expected {op.op_id}")


def bench_worker(args: argparse.Namespace) -> Dict[str, Any]:
    model, cache, bench = make_configs(args)
    print(f"model_config: {model}")
    print(f"cache_config: {cache}")
    print(f"bench_config: {bench}")
    layers_moved = bench.num_layers_to_transfer
    if layers_moved == -1:
        layers_moved = model.num_layers
    n = bench.num_blocks_to_transfer
    kind = bench.transfer_type
    if n > cache.num_cpu_blocks or (kind in (TransferType.H2DISK, TransferType.DISK2H) and
                                    n > cache.num_ssd_blocks):
        raise ValueError(f"--num-blocks {n} exceeds the configured host or SSD block count")
    ctx = mp.get_context("spawn")
    queue = ctx.Queue()
    keep: Any = None
    tmp = None
    if kind in (TransferType.H2D, TransferType.D2H):
        handle, keep = create_cpu_gpu_worker(model, cache, bench, queue)
    elif kind in (TransferType.H2DISK, TransferType.DISK2H):
        ssd_dir = cache.ssd_cache_dir
        if ssd_dir is None:
            tmp = tempfile.TemporaryDirectory(prefix="flexkv_ssd_bench_")
            ssd_dir = tmp.name
        handle, keep = create_cpu_ssd_worker(model, cache, queue, ssd_dir)
    else:
        raise ValueError(f"Unsupported transfer type: {kind} for benchmark, currently only "
                         "support H2D, D2H, H2DISK, DISK2H")
    ids = torch.randperm(n) if bench.shuffle_ids else torch.arange(n)
    ids = ids.to(torch.int64)
    op = TransferOp(graph_id=0, transfer_type=kind, layer_id=0,
                    layer_granularity=layers_moved,
                    src_descriptor=TransferDescriptor(physical_block_ids=ids),
                    dst_descriptor=TransferDescriptor(physical_block_ids=ids))
    try:
        if kind == TransferType.DISK2H:
            first = copy.deepcopy(op)
            first.transfer_type = TransferType.H2DISK
            first.src_descriptor, first.dst_descriptor = op.dst_descriptor, op.src_descriptor
            launch_transfer(handle, queue, first)
        for _ in range(bench.warmup_round):
            launch_transfer(handle, queue, op)
        times = []
        for _ in range(bench.benchmark_round):
            t0 = time.perf_counter()
            launch_transfer(handle, queue, op)
            times.append(time.perf_counter() - t0)
    finally:
        handle.shutdown()
        if tmp is not None:
            tmp.cleanup()
    del keep
    nbytes = n * cache.tokens_per_block * model.token_size_in_bytes * layers_moved \
        // model.num_layers
    avg = sum(times) / len(times)
    print(f"Total data size: {nbytes / 2**30} GB")
    print(f"Avg Time taken: {avg} seconds")
    print(f"Avg Bandwidth: {nbytes / 2**30 / avg} GB/s")
    return {"transfer_type": kind.value, "num_blocks": n, "num_layers": layers_moved,
            "shuffle_ids": bench.shuffle_ids, "bytes": nbytes, "avg_s": avg,
            "best_s": min(times), "gib_per_s": nbytes / 2**30 / avg, "gb_per_s": nbytes / 1e9 / avg,
            "path": ("ce" if (cache.use_ce_transfer_h2d if kind == TransferType.H2D else
                              cache.use_ce_transfer_d2h) else "kernel")
            if kind in (TransferType.H2D, TransferType.D2H) else "ssd"}


def parse_args(argv=None) -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--transfer-type", type=str, default=TransferType.H2D.name)
    ap.add_argument("--num-layers", type=int, default=-1)
    ap.add_argument("--num-blocks", type=int, default=16)
    ap.add_argument("--config", type=str, default=DEFAULT_CONFIG)
    ap.add_argument("--shuffle-ids", action="store_true")
    ap.add_argument("--warmup-round", type=int, default=1)
    ap.add_argument("--benchmark-round", type=int, default=10)
    return ap.parse_args(argv)


if __name__ == "__main__":
    # quiet in this process and in the spawned worker, as the reference's
    # flexkv_logger.set_level("OFF") (:20)
    flexkv_logger.set_level("OFF")
    os.environ.setdefault("FLEXKV_LOG_LEVEL", "OFF")
    print(json.dumps(bench_worker(parse_args())), flush=True)
