"""fkv_transfer_kv_blocks_noalloc, the entry point that allocates nothing,
against fkv_transfer_kv_blocks in kernel mode on the same inputs, bit for
bit: ids staged in the library's fixed device scratch (two calls in a row,
the second smaller, so the scratch keeps the first call's ids beyond the
second's), ids in the kernel arguments (32 blocks or fewer), the scratch's
capacity (65536 blocks) and its refusal above it."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_util import DeviceCase, abi_transfer
from kvcase import KVCase
from oracle import inputs

pytestmark = pytest.mark.gpu


def _noalloc(dc, gids, cids, h2d):
    from flexkv_amd import _lib
    case = dc.case
    s = case.strides()
    gids = np.ascontiguousarray(gids, dtype=np.int64)
    cids = np.ascontiguousarray(cids, dtype=np.int64)
    ptrs = (ctypes.c_void_p * len(dc.gpu))(*[t.data_ptr() for t in dc.gpu])
    rc = _lib.load().fkv_transfer_kv_blocks_noalloc(
        len(gids), case.start_layer, len(dc.gpu), gids.ctypes.data, ptrs, s["gpu_kv"],
        s["gpu_block"], cids.ctypes.data, dc.host.data_ptr(), s["cpu_kv"], s["cpu_layer"],
        s["cpu_block"], s["startoff"], s["chunk"], torch.cuda.current_stream().cuda_stream,
        -1, int(h2d), int(case.kv == 1))
    _lib.check(rc, "fkv_transfer_kv_blocks_noalloc")


def _same_both_ways(case, a, b, gids, cids, salt):
    """D2H on both entry points, host caches equal; then H2D of fresh host
    values into zeroed layers on both, layers equal."""
    _noalloc(a, gids, cids, False)
    abi_transfer(b, gids, cids, False, 0)
    torch.cuda.synchronize()
    assert np.array_equal(a.host_np(), b.host_np())
    fresh = a.host_np() ^ np.array(salt, dtype=case.dtype)
    for dc in (a, b):
        dc.set_host(fresh)
        dc.set_gpu([np.zeros_like(g) for g in case.gpu])
    _noalloc(a, gids, cids, True)
    abi_transfer(b, gids, cids, True, 0)
    torch.cuda.synchronize()
    for l, (x, y) in enumerate(zip(a.gpu_np(), b.gpu_np())):
        assert np.array_equal(x, y), f"layer {l}"


@pytest.mark.parametrize("layout,kv", [("BLOCKWISE", 2), ("LAYERWISE", 2), ("BLOCKWISE", 1)])
def test_noalloc_matches_transfer_kv_blocks(layout, kv):
    case = KVCase(layers_total=5, num_layers=4, start_layer=1, kv=kv, ng=512, nh=640, tokens=16,
                  heads=2, dim=64, layout=layout).fill(seed=80 + kv)
    a, b = DeviceCase(case), DeviceCase(case)
    for step, n in enumerate((300, 120, 7)):   # scratch, scratch (smaller), inline ids
        gids = inputs.distinct_ids(81 + step, n, case.ng)
        cids = inputs.distinct_ids(91 + step, n, case.nh)
        print(f"noalloc {layout} kv={kv} n={n}", flush=True)
        if step == 0:
            _noalloc(a, gids, cids, False)
            torch.cuda.synchronize()
            assert np.array_equal(a.host_np(), case.expect_d2h(gids, cids))   # the oracle
            a.set_host(case.host)
        _same_both_ways(case, a, b, gids, cids, 0x3C3C + step)


def test_noalloc_scratch_capacity():
    from flexkv_amd import _lib
    cap = 65536
    case = KVCase(layers_total=2, num_layers=2, start_layer=0, kv=2, ng=cap + 8, nh=cap + 8,
                  tokens=1, heads=1, dim=8).fill(seed=99)            # 16-byte chunks
    a, b = DeviceCase(case), DeviceCase(case)
    gids = inputs.distinct_ids(97, cap, case.ng)
    cids = inputs.distinct_ids(98, cap, case.nh)
    print("noalloc capacity", flush=True)
    _same_both_ways(case, a, b, gids, cids, 0x0F0F)
    over = inputs.distinct_ids(96, cap + 1, case.ng)
    with pytest.raises(RuntimeError, match="at most 65536 blocks"):
        _noalloc(a, over, inputs.distinct_ids(95, cap + 1, case.nh), False)
    assert "at most 65536 blocks" in _lib.last_error()
