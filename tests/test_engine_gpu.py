"""The reference's GPU<->CPU round trip through the engine stack
(tests/test_transfer_engine.py:55-161 with tests/test_utils.py:15-204):
StorageEngine + TransferEngine, a write graph (GPU->CPU), zeroed GPU blocks,
a read graph (CPU->GPU), then every layer compared with the ground truth."""
import time

import pytest
import torch

from flexkv_amd.cache.transfer_pattern import (convert_read_graph_to_layer_wise_graph,
                                               create_read_graph_cpu_storage,
                                               create_write_graph_cpu_storage)
from flexkv_amd.common.config import CacheConfig, ModelConfig
from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType
from flexkv_amd.common.transfer import DeviceType
from flexkv_amd.storage.storage_engine import StorageEngine
from flexkv_amd.transfer.transfer_engine import TransferEngine

pytestmark = pytest.mark.gpu

# the reference test's defaults (tests/test_utils.py:15-53)
MODEL = dict(num_layers=4, num_kv_heads=32, head_size=128, dtype=torch.float16)
CACHE = dict(tokens_per_block=16, num_cpu_blocks=128, use_ce_transfer_h2d=False,
             use_ce_transfer_d2h=True, transfer_sms_h2d=4, transfer_sms_d2h=4)


def _wait(engine, gid, limit=30.0):
    t0 = time.time()
    seen = []
    while time.time() - t0 < limit:
        seen += engine.get_completed_graphs_and_ops(timeout=0.1)
        if (gid, -1) in seen:
            return seen
    raise AssertionError(f"graph {gid} did not complete")


def _setup(use_mla, layout, worker_mode="thread", eager=True, num_gpu_blocks=128):
    mc = ModelConfig(use_mla=use_mla, **MODEL)
    cc = CacheConfig(cpu_kv_layout_type=layout, **CACHE)
    gl = KVCacheLayout(KVCacheLayoutType.LAYERWISE, mc.num_layers, num_gpu_blocks,
                       cc.tokens_per_block, mc.num_kv_heads, mc.head_size, is_mla=use_mla)
    gen = torch.Generator().manual_seed(17)
    gt = [torch.randn(tuple(gl.kv_shape[1:]), generator=gen).to(mc.dtype)
          for _ in range(mc.num_layers)]
    gpu = [t.cuda() for t in gt]
    se = StorageEngine(mc, cc)
    se.register_gpu_blocks(gpu, gl, device_id=0, dtype=mc.dtype)
    te = TransferEngine([se.get_storage_handle(DeviceType.GPU, 0)], mc, cc,
                        cpu_handle=se.get_storage_handle(DeviceType.CPU),
                        worker_mode=worker_mode, eager_dispatch=eager)
    te.start()
    return mc, gt, gpu, te


@pytest.mark.parametrize("use_mla", [False, True])
@pytest.mark.parametrize("layout", [KVCacheLayoutType.LAYERWISE, KVCacheLayoutType.BLOCKWISE])
def test_gpu_cpu_round_trip(use_mla, layout):
    mc, gt, gpu, te = _setup(use_mla, layout)
    try:
        gids = torch.arange(0, 16, dtype=torch.int64)
        cids = torch.arange(0, 16, dtype=torch.int64)
        wg, _ = create_write_graph_cpu_storage(gids, cids, torch.tensor([], dtype=torch.int64),
                                               gpu_device_id=0, layer_num=mc.num_layers)
        te.submit_transfer_graph(wg)
        _wait(te, wg.graph_id)
        for t in gpu:
            t[:, gids].zero_()
        torch.cuda.synchronize()
        rg, _ = create_read_graph_cpu_storage(gids, cids, torch.tensor([], dtype=torch.int64),
                                              gpu_device_id=0, layer_num=mc.num_layers)
        te.submit_transfer_graph(rg)
        _wait(te, rg.graph_id)
        for l in range(mc.num_layers):
            assert torch.equal(gpu[l].cpu(), gt[l]), f"layer {l}"
    finally:
        te.shutdown()


@pytest.mark.parametrize("eager", [False, True])
def test_layer_wise_read_graph(eager):
    """Read back one layer per op (convert_read_graph_to_layer_wise_graph);
    each tracked op is reported, in layer order, and the data arrives."""
    mc, gt, gpu, te = _setup(False, KVCacheLayoutType.BLOCKWISE, eager=eager)
    try:
        g = torch.Generator().manual_seed(3)
        gids = torch.randperm(128, generator=g)[:40]
        cids = torch.randperm(128, generator=g)[:40]
        wg, _ = create_write_graph_cpu_storage(gids, cids, torch.tensor([], dtype=torch.int64),
                                               layer_num=mc.num_layers)
        te.submit_transfer_graph(wg)
        _wait(te, wg.graph_id)
        for t in gpu:
            t[:, gids].zero_()
        torch.cuda.synchronize()
        rg, ends = create_read_graph_cpu_storage(gids, cids, torch.tensor([], dtype=torch.int64),
                                                 layer_num=mc.num_layers)
        lw, tracked = convert_read_graph_to_layer_wise_graph(rg, ends, mc.num_layers, 1)
        te.submit_transfer_graph(lw)
        seen = _wait(te, lw.graph_id)
        order = [op for gid, op in seen if gid == lw.graph_id and op >= 0]
        assert order == tracked
        for l in range(mc.num_layers):
            assert torch.equal(gpu[l].cpu(), gt[l]), f"layer {l}"
    finally:
        te.shutdown()


def test_process_workers_round_trip():
    """worker_mode='process': spawned worker, HIP IPC handles, a pinned host
    cache owned by the worker; the round trip restores the GPU blocks."""
    mc, gt, gpu, te = _setup(False, KVCacheLayoutType.BLOCKWISE, worker_mode="process")
    try:
        gids = torch.tensor([3, 9, 100, 42], dtype=torch.int64)
        cids = torch.tensor([7, 0, 55, 127], dtype=torch.int64)
        wg, _ = create_write_graph_cpu_storage(gids, cids, torch.tensor([], dtype=torch.int64),
                                               layer_num=mc.num_layers)
        te.submit_transfer_graph(wg)
        _wait(te, wg.graph_id, limit=120)
        for t in gpu:
            t[:, gids].zero_()
        torch.cuda.synchronize()
        rg, _ = create_read_graph_cpu_storage(gids, cids, torch.tensor([], dtype=torch.int64),
                                              layer_num=mc.num_layers)
        te.submit_transfer_graph(rg)
        _wait(te, rg.graph_id, limit=120)
        for l in range(mc.num_layers):
            assert torch.equal(gpu[l].cpu(), gt[l]), f"layer {l}"
    finally:
        te.shutdown()
