"""The reference's round trips through the engine stack
(tests/test_transfer_engine.py:55-410 with tests/test_utils.py:15-204):
StorageEngine + TransferEngine, a write graph (GPU->CPU[->SSD]), zeroed GPU
blocks (and, with an SSD tier, a zeroed host cache, so the data must come
back from the files), a read graph ([SSD->]CPU->GPU), then every layer
compared with the ground truth."""
import time

import pytest
import torch

from gpu_util import zero_blocks
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
SSD_BLOCKS = 512     # over two SSD directories, as tests/test_utils.py:31,40


def _wait(engine, gid, limit=30.0):
    t0 = time.time()
    seen = []
    while time.time() - t0 < limit:
        seen += engine.get_completed_graphs_and_ops(timeout=0.1)
        if (gid, -1) in seen:
            return seen
    raise AssertionError(f"graph {gid} did not complete")


def _setup(use_mla, layout, worker_mode="thread", eager=True, num_gpu_blocks=128,
           ssd_dirs=None, num_blocks=None):
    mc = ModelConfig(use_mla=use_mla, **MODEL)
    extra = dict(CACHE)
    if num_blocks is not None:
        extra["num_cpu_blocks"] = num_blocks
    if ssd_dirs is not None:
        extra.update(enable_ssd=True, ssd_kv_layout_type=layout, ssd_cache_dir=ssd_dirs,
                     num_ssd_blocks=SSD_BLOCKS if num_blocks is None else num_blocks)
    cc = CacheConfig(cpu_kv_layout_type=layout, **extra)
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
                        ssd_handle=se.get_storage_handle(DeviceType.SSD)
                        if ssd_dirs is not None else None,
                        worker_mode=worker_mode, eager_dispatch=eager)
    te.start()
    te._test_host = se.get_storage_handle(DeviceType.CPU).get_tensor()
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
            zero_blocks(t, gids)
        torch.cuda.synchronize()
        rg, _ = create_read_graph_cpu_storage(gids, cids, torch.tensor([], dtype=torch.int64),
                                              gpu_device_id=0, layer_num=mc.num_layers)
        te.submit_transfer_graph(rg)
        _wait(te, rg.graph_id)
        for l in range(mc.num_layers):
            assert torch.equal(gpu[l].cpu(), gt[l]), f"layer {l}"
    finally:
        te.shutdown()


@pytest.mark.parametrize("use_mla", [False, True])
@pytest.mark.parametrize("layout", [KVCacheLayoutType.LAYERWISE, KVCacheLayoutType.BLOCKWISE])
def test_write_graph_host_bytes(use_mla, layout):
    """Every byte of the host cache after a write graph through the engine,
    against tensor indexing on the host layout's own shape."""
    mc, gt, gpu, te = _setup(use_mla, layout)
    try:
        host = te._test_host
        host.view(torch.int16).fill_(0x5A5A)
        before = host.clone()
        g = torch.Generator().manual_seed(12)
        gids = torch.randperm(128, generator=g)[:33]
        cids = torch.randperm(CACHE["num_cpu_blocks"], generator=g)[:33]
        wg, _ = create_write_graph_cpu_storage(gids, cids, torch.tensor([], dtype=torch.int64),
                                               gpu_device_id=0, layer_num=mc.num_layers)
        te.submit_transfer_graph(wg)
        _wait(te, wg.graph_id)
        cl = KVCacheLayout(layout, mc.num_layers, CACHE["num_cpu_blocks"],
                           CACHE["tokens_per_block"], mc.num_kv_heads, mc.head_size,
                           is_mla=use_mla)
        exp = before.view(tuple(cl.kv_shape)).clone()
        for l, t in enumerate(gt):
            for k in range(t.shape[0]):
                if layout == KVCacheLayoutType.BLOCKWISE:
                    exp[cids, l, k] = t[k, gids]
                else:
                    exp[l, k, cids] = t[k, gids]
        assert torch.equal(host.view(torch.int16), exp.reshape(-1).view(torch.int16))
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
            zero_blocks(t, gids)
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
            zero_blocks(t, gids)
        torch.cuda.synchronize()
        rg, _ = create_read_graph_cpu_storage(gids, cids, torch.tensor([], dtype=torch.int64),
                                              layer_num=mc.num_layers)
        te.submit_transfer_graph(rg)
        _wait(te, rg.graph_id, limit=120)
        for l in range(mc.num_layers):
            assert torch.equal(gpu[l].cpu(), gt[l]), f"layer {l}"
    finally:
        te.shutdown()


def _ssd_dirs(tmp_path):
    return [str(tmp_path / "ssd_cache"), str(tmp_path / "ssd_cache2")]


@pytest.mark.parametrize("transfer_block_num", [8, 16])
@pytest.mark.parametrize("use_mla", [True, False])
@pytest.mark.parametrize("layout", [KVCacheLayoutType.LAYERWISE, KVCacheLayoutType.BLOCKWISE])
def test_ssd_round_trip(tmp_path, transfer_block_num, use_mla, layout):
    """GPU -> CPU -> SSD, then SSD -> CPU -> GPU (test_transfer_engine.py:165-265)."""
    mc, gt, gpu, te = _setup(use_mla, layout, ssd_dirs=_ssd_dirs(tmp_path))
    try:
        ids = torch.arange(0, transfer_block_num, dtype=torch.int64)
        wg, _ = create_write_graph_cpu_storage(ids, ids, ids, gpu_device_id=0,
                                               layer_num=mc.num_layers)
        wg.bind_to_dp_group(0)
        te.submit_transfer_graph(wg)
        _wait(te, wg.graph_id)
        for t in gpu:
            zero_blocks(t, ids)
        torch.cuda.synchronize()
        te._test_host.zero_()
        rg, _ = create_read_graph_cpu_storage(ids, ids, ids, gpu_device_id=0,
                                              layer_num=mc.num_layers)
        rg.bind_to_dp_group(0)
        te.submit_transfer_graph(rg)
        _wait(te, rg.graph_id)
        for l in range(mc.num_layers):
            assert torch.equal(gpu[l].cpu(), gt[l]), f"layer {l}"
    finally:
        te.shutdown()


@pytest.mark.parametrize("include_ssd", [True, False])
@pytest.mark.parametrize("use_mla", [True, False])
def test_concurrent_mixed_transfers(tmp_path, include_ssd, use_mla):
    """Four write graphs, then four read graphs, all in flight at once
    (test_transfer_engine.py:268-410; 16 blocks per transfer)."""
    n, per = 4, 16
    blocks = max(128, n * per * 2)
    mc, gt, gpu, te = _setup(use_mla, KVCacheLayoutType.BLOCKWISE, num_gpu_blocks=blocks,
                             ssd_dirs=_ssd_dirs(tmp_path) if include_ssd else None,
                             num_blocks=blocks)
    empty = torch.tensor([], dtype=torch.int64)
    try:
        graphs = []
        for i in range(n):
            ids = torch.arange(i * per, (i + 1) * per, dtype=torch.int64)
            g, _ = create_write_graph_cpu_storage(ids, ids, ids if include_ssd else empty,
                                                  gpu_device_id=0, layer_num=mc.num_layers)
            graphs.append(g)
        for g in graphs:
            te.submit_transfer_graph(g)
        seen = []
        for g in graphs:
            if (g.graph_id, -1) not in seen:
                seen += _wait(te, g.graph_id)
        cleared = torch.arange(0, (n + 1) * per, dtype=torch.int64)
        for t in gpu:
            zero_blocks(t, cleared)
        torch.cuda.synchronize()
        if include_ssd:
            te._test_host.zero_()
        graphs = []
        for i in range(n):
            ids = torch.arange(i * per, (i + 1) * per, dtype=torch.int64)
            g, _ = create_read_graph_cpu_storage(ids, ids, ids if include_ssd else empty,
                                                 gpu_device_id=0, layer_num=mc.num_layers)
            graphs.append(g)
        for g in graphs:
            te.submit_transfer_graph(g)
        seen = []
        for g in graphs:
            if (g.graph_id, -1) not in seen:
                seen += _wait(te, g.graph_id)
        for l in range(mc.num_layers):
            assert torch.equal(gpu[l][:, :(n + 1) * per].cpu(),
                               torch.cat([gt[l][:, :n * per],
                                          torch.zeros_like(gt[l][:, n * per:(n + 1) * per])],
                                         dim=1)), f"layer {l}"
    finally:
        te.shutdown()


@pytest.mark.parametrize("use_mla", [False, True])
def test_separate_kv_layers_round_trip(use_mla):
    """An engine whose layers are [K, V] pairs of separate [N, tokens, heads,
    dim] tensors (as SGLang allocates them) round-trips through the host cache."""
    mc = ModelConfig(use_mla=use_mla, **MODEL)
    cc = CacheConfig(cpu_kv_layout_type=KVCacheLayoutType.BLOCKWISE, **CACHE)
    gl = KVCacheLayout(KVCacheLayoutType.LAYERWISE, mc.num_layers, 128, cc.tokens_per_block,
                       mc.num_kv_heads, mc.head_size, is_mla=use_mla)
    gen = torch.Generator().manual_seed(23)
    gt = [torch.randn(tuple(gl.kv_shape[1:]), generator=gen).to(mc.dtype)
          for _ in range(mc.num_layers)]
    pairs = [[gt[l][k].cuda() for k in range(gl.kv_shape[1])] for l in range(mc.num_layers)]
    se = StorageEngine(mc, cc)
    se.register_gpu_blocks(pairs, gl, device_id=0, dtype=mc.dtype)
    te = TransferEngine([se.get_storage_handle(DeviceType.GPU, 0)], mc, cc,
                        cpu_handle=se.get_storage_handle(DeviceType.CPU))
    te.start()
    try:
        gids = torch.tensor([0, 7, 99, 127, 64], dtype=torch.int64)
        cids = torch.tensor([3, 1, 126, 40, 77], dtype=torch.int64)
        wg, _ = create_write_graph_cpu_storage(gids, cids, torch.tensor([], dtype=torch.int64),
                                               layer_num=mc.num_layers)
        te.submit_transfer_graph(wg)
        _wait(te, wg.graph_id)
        for pair in pairs:
            for t in pair:
                t.index_fill_(0, gids.cuda(), 0)
                assert not t.index_select(0, gids.cuda()).any()
        torch.cuda.synchronize()
        rg, _ = create_read_graph_cpu_storage(gids, cids, torch.tensor([], dtype=torch.int64),
                                              layer_num=mc.num_layers)
        te.submit_transfer_graph(rg)
        _wait(te, rg.graph_id)
        for l in range(mc.num_layers):
            for k, t in enumerate(pairs[l]):
                assert torch.equal(t.cpu(), gt[l][k]), f"layer {l} half {k}"
    finally:
        te.shutdown()
