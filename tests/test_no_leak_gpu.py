"""Repeated calls hold no memory: after a warm-up, hundreds more calls of
every transfer path (zero-copy kernel and copy engines, each direction, the
small-call kernel, the general kernel and the staged path) and of both
layer-wise handles leave the process's resident host memory and the device's
free memory where they were.  The library pools pinned id buffers, staging,
signals and events, so a call that dropped one of them would show here."""
import os

import psutil
import pytest
import torch

from oracle import inputs
from flexkv_amd import c_ext
from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType
from flexkv_amd.storage.allocator import pinned_empty

pytestmark = pytest.mark.gpu

L, NG, NH = 8, 256, 320


@pytest.fixture(scope="module")
def setup():
    dtype = torch.bfloat16
    gl = KVCacheLayout(KVCacheLayoutType.LAYERWISE, L, NG, 16, 8, 128)
    cl = KVCacheLayout(KVCacheLayoutType.BLOCKWISE, L, NH, 16, 8, 128)
    chunk, gkv, _, gblk = gl.div_layer(L).byte_strides(dtype)
    _, ckv, clay, cblk = cl.byte_strides(dtype)
    layers = [torch.randn(gl.kv_shape[1:], device="cuda").to(dtype) for _ in range(L)]
    ptrs = torch.tensor([t.data_ptr() for t in layers], dtype=torch.int64)
    host = pinned_empty(cl.get_total_elements(), dtype)
    return layers, ptrs, host, (gkv, gblk, ckv, clay, cblk, chunk)


def _snapshot():
    torch.cuda.synchronize()
    free, _ = torch.cuda.mem_get_info()
    return psutil.Process(os.getpid()).memory_info().rss, free


@pytest.mark.parametrize("n", [1, 40, 200])
def test_repeated_transfers_hold_no_memory(setup, monkeypatch, n):
    """1 block (small-call kernel), 40 blocks (general kernel) and 200
    blocks (100 MiB: the copy engines) per call, both modes and directions."""
    monkeypatch.setenv("FLEXKV_CE_MIN_BYTES", str(64 << 20))
    layers, ptrs, host, (gkv, gblk, ckv, clay, cblk, chunk) = setup
    gids = torch.from_numpy(inputs.distinct_ids(n, n, NG))
    cids = torch.from_numpy(inputs.distinct_ids(n + 1, n, NH))
    reps = 300 if n < 200 else 60

    def calls(k):
        for _ in range(k):
            for ce in (False, True):
                for h2d in (False, True):
                    c_ext.transfer_kv_blocks(gids, ptrs, gkv, gblk, cids, host, ckv, clay, cblk,
                                             chunk, 0, -1, h2d, ce, False)

    calls(20)
    rss0, free0 = _snapshot()
    calls(reps)
    rss1, free1 = _snapshot()
    assert rss1 - rss0 < (8 << 20), f"host memory grew {(rss1 - rss0) >> 10} KiB"
    assert free0 - free1 < (16 << 20), f"device memory fell {(free0 - free1) >> 20} MiB"


@pytest.mark.parametrize("ce", [False, True], ids=["kernel", "ce"])
def test_repeated_layerwise_handles_hold_no_memory(setup, ce):
    layers, ptrs, host, (gkv, gblk, ckv, clay, cblk, chunk) = setup
    gids = torch.from_numpy(inputs.distinct_ids(7, 64, NG))
    cids = torch.from_numpy(inputs.distinct_ids(8, 64, NH))

    def handles(k):
        for _ in range(k):
            h = c_ext.transfer_kv_blocks_layerwise(gids, ptrs, gkv, gblk, cids, host, ckv, clay,
                                                   cblk, chunk, start_layer_id=0,
                                                   layer_granularity=2, is_host_to_device=True,
                                                   use_ce_transfer=ce)
            h.release()

    handles(30)
    rss0, free0 = _snapshot()
    handles(200)
    rss1, free1 = _snapshot()
    assert rss1 - rss0 < (8 << 20), f"host memory grew {(rss1 - rss0) >> 10} KiB"
    assert free0 - free1 < (16 << 20), f"device memory fell {(free0 - free1) >> 20} MiB"


def test_tp_groups_release_threads_and_streams(setup):
    """Creating, using and closing TP groups leaves the process's thread
    count and the device's free memory where they were."""
    layers, ptrs, host, (gkv, gblk, ckv, clay, cblk, chunk) = setup
    gids = torch.from_numpy(inputs.distinct_ids(11, 16, NG))
    cids = torch.from_numpy(inputs.distinct_ids(12, 16, NH))
    ranks = [layers] * 2           # two ranks on one GPU, same caches (reads only)

    def groups(k):
        for _ in range(k):
            g = c_ext.TPTransferThreadGroup(2, ranks, host, 0)
            # D2H of half chunks: rank r into bytes [r * chunk / 2, ...) of each
            g.tp_group_transfer(gids, gkv, gblk, chunk // 2, cids, ckv, clay, cblk, chunk, -1,
                                False, False, 0, L, False)
            g.close()

    groups(3)
    proc = psutil.Process(os.getpid())
    threads0 = proc.num_threads()
    _, free0 = _snapshot()
    groups(30)
    _, free1 = _snapshot()
    assert proc.num_threads() <= threads0 + 2, (threads0, proc.num_threads())   # 2 rank threads each would add 60
    assert free0 - free1 < (16 << 20), f"device memory fell {(free0 - free1) >> 20} MiB"
