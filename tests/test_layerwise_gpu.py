"""Asynchronous layer-grouped transfers (fkv_transfer_kv_blocks_layerwise)
against the oracle, and the ordering their per-group events give."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from oracle import inputs
from kvcase import KVCase

pytestmark = pytest.mark.gpu


def _abi_layerwise(dc, gids, cids, h2d, gran, stream=None, cus=-1, ce=False):
    from flexkv_amd import _lib
    from flexkv_amd.c_ext import LayerwiseTransfer
    case = dc.case
    s = case.strides()
    gids = np.ascontiguousarray(gids, dtype=np.int64)
    cids = np.ascontiguousarray(cids, dtype=np.int64)
    ptrs = (ctypes.c_void_p * len(dc.gpu))(*[t.data_ptr() for t in dc.gpu])
    st = (stream or torch.cuda.current_stream()).cuda_stream
    out = ctypes.c_void_p()
    lib = _lib.load()
    rc = lib.fkv_transfer_kv_blocks_layerwise(
        len(gids), case.start_layer, len(dc.gpu), gran, gids.ctypes.data, ptrs, s["gpu_kv"],
        s["gpu_block"], cids.ctypes.data, dc.host.data_ptr(), s["cpu_kv"], s["cpu_layer"],
        s["cpu_block"], s["startoff"], s["chunk"], st, cus, int(h2d), int(ce), int(case.kv == 1),
        ctypes.byref(out))
    _lib.check(rc, "fkv_transfer_kv_blocks_layerwise")
    # ids were copied by the call: overwrite ours to prove the handle kept its own
    gids[:] = -1
    cids[:] = -1
    return LayerwiseTransfer(out.value, ())


@pytest.mark.parametrize("ce", [False, True], ids=["kernel", "ce"])
@pytest.mark.parametrize("gran", [1, 3, 4, 200])
@pytest.mark.parametrize("geo", [(4, 2, 64, 96, 16, 8, 128, 40), (130, 2, 6, 8, 1, 1, 64, 5),
                                 (6, 1, 30, 40, 64, 1, 576, 9)], ids=["8b-like", "130-layers", "mla"])
def test_layerwise_matches_oracle(geo, gran, ce):
    from gpu_util import DeviceCase
    L, kv, ng, nh, t, h, d, n = geo
    case = KVCase(layers_total=L, num_layers=L, start_layer=0, kv=kv, ng=ng, nh=nh, tokens=t,
                  heads=h, dim=d).fill(seed=L * gran)
    gids = inputs.distinct_ids(gran, n, ng)
    cids = inputs.distinct_ids(gran + 1, n, nh)
    s = case.strides()
    dc = DeviceCase(case)
    hnd = _abi_layerwise(dc, gids.copy(), cids.copy(), False, gran)
    assert hnd.num_groups == -(-L // gran)
    hnd.release()
    want = case.host.copy()
    oracle.transfer_kv_blocks(gids, case.gpu, s["gpu_kv"], s["gpu_block"], cids, want, s["cpu_kv"],
                              s["cpu_layer"], s["cpu_block"], s["chunk"], 0, False, is_mla=kv == 1)
    assert np.array_equal(dc.host_np(), want)
    # H2D of fresh host values into zeroed layers
    fresh = want ^ np.uint16(0x3C3C)
    dc.set_host(fresh)
    zeros = [np.zeros_like(g) for g in case.gpu]
    dc.set_gpu(zeros)
    with _abi_layerwise(dc, gids.copy(), cids.copy(), True, gran, ce=ce) as hnd:
        for g in range(hnd.num_groups):
            hnd.wait(g)
            assert hnd.query(g)
    exp = [z.copy() for z in zeros]
    case.host = fresh
    oracle.transfer_kv_blocks(gids, exp, s["gpu_kv"], s["gpu_block"], cids, case.host,
                              s["cpu_kv"], s["cpu_layer"], s["cpu_block"], s["chunk"], 0, True,
                              is_mla=kv == 1)
    for got, e in zip(dc.gpu_np(), exp):
        assert np.array_equal(got, e)


@pytest.mark.parametrize("ce", [False, True], ids=["kernel", "ce"])
def test_stream_wait_orders_consumers(ce):
    """A consumer stream that waits on group g sees layer g's blocks (the
    kernel path: with no host synchronisation between the transfer and the
    consumer; the copy-engine path: the host waits for the group's event to
    exist, the consumer stream for it to complete)."""
    from gpu_util import DeviceCase
    L, n = 16, 256
    case = KVCase(layers_total=L, num_layers=L, start_layer=0, kv=2, ng=512, nh=1024, tokens=16,
                  heads=8, dim=128).fill(seed=5)
    gids = inputs.distinct_ids(1, n, 512)
    cids = inputs.distinct_ids(2, n, 1024)
    dc = DeviceCase(case)
    # host holds random values that must arrive; the device starts at zero
    src = KVCase(layers_total=L, num_layers=L, start_layer=0, kv=2, ng=512, nh=1024, tokens=16,
                 heads=8, dim=128)
    size = int(np.prod(src.host_shape()))
    src.host = (inputs.splitmix64(np.arange(size, dtype=np.uint64)) & np.uint64(0xFFFF)) \
        .astype(np.uint16).reshape(src.host_shape())
    dc.set_host(src.host)
    dc.set_gpu([np.zeros_like(g) for g in case.gpu])
    g_dev = torch.from_numpy(gids).to("cuda")
    torch.cuda.synchronize()
    xfer = torch.cuda.Stream()
    consumer = torch.cuda.Stream()
    outs = []
    with torch.cuda.stream(xfer):
        hnd = _abi_layerwise(dc, gids.copy(), cids.copy(), True, 1, stream=xfer, cus=1, ce=ce)
    with torch.cuda.stream(consumer):
        for l in range(L):
            hnd.stream_wait(l, consumer)
            outs.append(dc.gpu[l][:, g_dev].clone())
    consumer.synchronize()
    hnd.release()
    hv = src.host_view(src.host)
    for l in range(L):
        want = np.stack([hv[c, l, :, 0] for c in cids], axis=1)   # [kv, n, t, h, d]
        assert np.array_equal(outs[l].cpu().numpy().view(np.uint16), want), f"layer {l}"


def test_concurrent_handles_keep_their_ids():
    from gpu_util import DeviceCase
    a = KVCase(layers_total=8, num_layers=8, start_layer=0, kv=2, ng=128, nh=128, tokens=16,
               heads=4, dim=128).fill(seed=11)
    b = KVCase(layers_total=8, num_layers=8, start_layer=0, kv=2, ng=128, nh=128, tokens=16,
               heads=4, dim=128).fill(seed=12)
    da, db = DeviceCase(a), DeviceCase(b)
    ga, ca = inputs.distinct_ids(3, 100, 128), inputs.distinct_ids(4, 100, 128)
    gb, cb = inputs.distinct_ids(5, 60, 128), inputs.distinct_ids(6, 60, 128)
    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    ha = _abi_layerwise(da, ga.copy(), ca.copy(), False, 2, stream=sa)
    hb = _abi_layerwise(db, gb.copy(), cb.copy(), False, 3, stream=sb)
    hb.release()
    ha.release()
    for case, dc, g, c in ((a, da, ga, ca), (b, db, gb, cb)):
        assert np.array_equal(dc.host_np(), case.expect_d2h(g, c))


def test_empty_and_rejected():
    from flexkv_amd import c_ext
    from gpu_util import DeviceCase
    case = KVCase(layers_total=2, num_layers=2, start_layer=0, kv=2, ng=8, nh=8, tokens=16,
                  heads=2, dim=64).fill(seed=1)
    dc = DeviceCase(case)
    h = _abi_layerwise(dc, np.zeros(0, np.int64), np.zeros(0, np.int64), False, 1)
    assert h.num_groups == 0
    h.wait()
    h.release()
    h.release()
    with pytest.raises(RuntimeError):
        _abi_layerwise(dc, np.array([1, 1 << 22]), np.array([0, 1]), False, 1)
    with pytest.raises(RuntimeError, match="granularity"):
        _abi_layerwise(dc, np.array([1]), np.array([0]), False, 0)
    ptrs = torch.tensor([t.data_ptr() for t in dc.gpu], dtype=torch.int64)
    s = case.strides()
    ids = torch.tensor([1, 2], dtype=torch.int64)
    hnd = c_ext.transfer_kv_blocks_layerwise(ids, ptrs, s["gpu_kv"], s["gpu_block"], ids, dc.host,
                                             s["cpu_kv"], s["cpu_layer"], s["cpu_block"],
                                             s["chunk"], 0, 1, -1, False, False)
    assert hnd.num_groups == 2
    hnd.wait(1)
    with pytest.raises(IndexError):
        hnd.query(2)
    hnd.release()
    with pytest.raises(RuntimeError, match="released"):
        hnd.query(0)
    assert np.array_equal(dc.host_np(), case.expect_d2h(np.array([1, 2]), np.array([1, 2])))


@pytest.mark.parametrize("num_cus", [0, 8])
def test_transfer_stream_helper(num_cus):
    """fkv_stream_create: a transfer on a stream with its own hardware queue
    (optionally confined to num_cus compute units) moves the same bytes."""
    from flexkv_amd import c_ext, _lib
    from gpu_util import DeviceCase
    case = KVCase(layers_total=4, num_layers=4, start_layer=0, kv=2, ng=64, nh=64, tokens=16,
                  heads=4, dim=128).fill(seed=21 + num_cus)
    dc = DeviceCase(case)
    g, c = inputs.distinct_ids(7, 40, 64), inputs.distinct_ids(8, 40, 64)
    st = c_ext.transfer_stream(num_cus)
    torch.cuda.synchronize()
    with torch.cuda.stream(st):
        hnd = _abi_layerwise(dc, g.copy(), c.copy(), False, 1, stream=st)
    hnd.release()
    assert np.array_equal(dc.host_np(), case.expect_d2h(g, c))
    import ctypes
    out = ctypes.c_void_p()
    assert _lib.load().fkv_stream_create(100000, ctypes.byref(out)) == 1
    assert "num_cus" in _lib.last_error()


def _ce_copies_per_block(L, G, layer_row, half, min_copy, lpl=128, lead=0):
    """Engine copies per block the copy-engine layer-wise pipeline plans for a
    block-wise host cache: the first `lead` groups (at most all but one) move
    with the zero-copy kernel; then windows of whole layer groups, up to
    `min_copy` bytes per block, growing 1, 2, 4, ... groups and near the end
    holding at most half of the groups left; each cut into layer windows whose
    rows fit a staging half."""
    ngroups = -(-L // G)
    group_row = min(G, L) * layer_row
    gpw = 1
    if G <= lpl:
        gpw = max(1, min(-(-min_copy // group_row), lpl // G))
        while gpw > 1 and gpw * group_row > half:
            gpw -= 1
    copies, grp, ramp = 0, max(0, min(lead, ngroups - 1)), 1
    while grp < ngroups:
        take = min(gpw, ramp, max(1, (ngroups - grp) // 2))
        ramp = min(2 * ramp, gpw)
        l0 = grp * G
        nl = min(take * G, L - l0)
        grp += take
        win = min(nl, lpl)
        while win > 1 and win * layer_row > half:
            win = (win + 1) // 2
        copies += -(-nl // win)
    return copies


@pytest.mark.parametrize("staging_kib,gran,min_copy,lead",
                         [(0, 1, None, None), (256, 1, None, None), (256, 3, None, None),
                          (96, 2, None, None), (0, 1, 1, None), (0, 2, 64 << 10, None),
                          (0, 1, None, 1), (256, 1, None, 3), (0, 6, None, 1)])
def test_ce_pipeline_pieces_and_copies(staging_kib, gran, min_copy, lead, monkeypatch):
    """The copy-engine layer-wise pipeline with staging small enough that a
    group spans several pieces, or a group's rows are cut into layer windows,
    with several groups per engine copy, and with 0 (the default), 1 or 3
    leading groups on the zero-copy kernel (one group in all: none):
    each group's layers match the oracle as soon as that group alone is
    waited for, every group's event fires, and the engines moved the planned
    copies per block (the library's profile)."""
    from flexkv_amd import _lib
    from gpu_util import DeviceCase
    if min_copy is not None:
        monkeypatch.setenv("FLEXKV_LAYERWISE_CE_MIN_COPY_BYTES", str(min_copy))
    if lead is not None:
        monkeypatch.setenv("FLEXKV_LAYERWISE_CE_KERNEL_GROUPS", str(lead))
    L, n = 6, 37
    case = KVCase(layers_total=L, num_layers=L, start_layer=0, kv=2, ng=64, nh=96, tokens=16,
                  heads=4, dim=64).fill(seed=60 + gran)              # 8 KiB chunks
    s = case.strides()
    gids = inputs.distinct_ids(61, n, 64)
    cids = inputs.distinct_ids(62, n, 96)
    dc = DeviceCase(case)
    fresh = case.host ^ np.uint16(0x1E1E)
    dc.set_host(fresh)
    dc.set_gpu([np.zeros_like(g) for g in case.gpu])
    exp = [np.zeros_like(g) for g in case.gpu]
    oracle.transfer_kv_blocks(gids, exp, s["gpu_kv"], s["gpu_block"], cids, fresh, s["cpu_kv"],
                              s["cpu_layer"], s["cpu_block"], s["chunk"], 0, True)
    _lib.set_staging_bytes(staging_kib << 10)
    try:
        _lib.profile_enable(True)
        with _abi_layerwise(dc, gids.copy(), cids.copy(), True, gran, ce=True) as hnd:
            assert hnd.num_groups == -(-L // gran)
            for g in range(hnd.num_groups):
                hnd.wait(g)
                got = dc.gpu_np()
                for l in range(g * gran, min(L, (g + 1) * gran)):
                    assert np.array_equal(got[l], exp[l]), (g, l)
        prof = _lib.profile_read()
        _lib.profile_enable(False)
    finally:
        _lib.set_staging_bytes(0)
        _lib.release_staging()
    for got, e in zip(dc.gpu_np(), exp):
        assert np.array_equal(got, e)
    assert prof["dma_batches"] == 1, prof
    half = (staging_kib << 9) if staging_kib else 1 << 29
    per_block = _ce_copies_per_block(L, gran, 2 * s["chunk"], half,
                                     256 << 10 if min_copy is None else min_copy,
                                     lead=0 if lead is None else lead)
    assert prof["dma_copies"] == per_block * n, (prof, per_block)
    if min_copy == 1:
        assert per_block == L // gran       # one copy per block and group


def test_ce_handle_stream_wait_and_query_before_arrival():
    """query() reports a copy-engine group as pending until its copies land,
    then done; stream_wait() on a later group than the one waited for still
    orders the consumer; release() without waits drains the pipeline."""
    from gpu_util import DeviceCase
    L, n = 8, 200
    case = KVCase(layers_total=L, num_layers=L, start_layer=0, kv=2, ng=256, nh=256, tokens=16,
                  heads=8, dim=128).fill(seed=70)                  # 32 KiB chunks
    gids = inputs.distinct_ids(71, n, 256)
    cids = inputs.distinct_ids(72, n, 256)
    dc = DeviceCase(case)
    fresh = case.host ^ np.uint16(0x2D2D)
    dc.set_host(fresh)
    dc.set_gpu([np.zeros_like(g) for g in case.gpu])
    hnd = _abi_layerwise(dc, gids.copy(), cids.copy(), True, 1, ce=True)
    states = [hnd.query(g) for g in range(L)]           # some may still be pending
    consumer = torch.cuda.Stream()
    g_dev = torch.from_numpy(gids).cuda()
    with torch.cuda.stream(consumer):
        hnd.stream_wait(L - 1, consumer)
        last = dc.gpu[L - 1][:, g_dev].clone()
    consumer.synchronize()
    assert all(hnd.query(g) for g in range(L)), states
    hnd.release()
    hv = case.host_view(fresh)
    want = np.stack([hv[c, L - 1, :, 0] for c in cids], axis=1)
    assert np.array_equal(last.cpu().numpy().view(np.uint16), want)
    # a handle released at once
    dc.set_gpu([np.zeros_like(g) for g in case.gpu])
    _abi_layerwise(dc, gids.copy(), cids.copy(), True, 2, ce=True).release()
    for l, g in enumerate(dc.gpu_np()):
        assert np.array_equal(g[:, gids], np.stack([hv[c, l, :, 0] for c in cids], axis=1))


_NO_ENGINES_CHILD = r"""
import sys
sys.path.insert(0, {root!r}); sys.path.insert(0, {tests!r})
import numpy as np, torch
import oracle
from oracle import inputs
from kvcase import KVCase
from gpu_util import DeviceCase
from test_layerwise_gpu import _abi_layerwise
L, n = 6, 40
case = KVCase(layers_total=L, num_layers=L, start_layer=0, kv=2, ng=64, nh=96, tokens=16,
              heads=4, dim=64).fill(seed=31)
s = case.strides()
dc = DeviceCase(case)
for rnd in range(2):
    gids = inputs.distinct_ids(40 + rnd, n, 64)
    cids = inputs.distinct_ids(50 + rnd, n, 96)
    fresh = case.host ^ np.uint16(0x0F0F + rnd)
    dc.set_host(fresh)
    dc.set_gpu([np.zeros_like(g) for g in case.gpu])
    with _abi_layerwise(dc, gids.copy(), cids.copy(), True, 2, ce=True) as hnd:
        for g in range(hnd.num_groups):
            hnd.wait(g)
    exp = [np.zeros_like(g) for g in case.gpu]
    oracle.transfer_kv_blocks(gids, exp, s["gpu_kv"], s["gpu_block"], cids, fresh, s["cpu_kv"],
                              s["cpu_layer"], s["cpu_block"], s["chunk"], 0, True)
    assert all(np.array_equal(a, b) for a, b in zip(dc.gpu_np(), exp)), rnd
print("layer-wise copy-engine handles match the oracle", flush=True)
"""


def test_mixed_copy_engine_load():
    """Three threads at once on disjoint block sets, 40 rounds each: a
    copy-engine D2H loop, a copy-engine H2D loop (the two share engines 0-7
    through the duplex split) and copy-engine layer-wise handles (the H2D
    lane, taken in turn with the H2D loop).  Every set's bytes match at the
    end, and no call fails."""
    import threading
    from gpu_util import DeviceCase, abi_transfer
    L, n = 8, 150
    case = KVCase(layers_total=L, num_layers=L, start_layer=0, kv=2, ng=480, nh=480, tokens=16,
                  heads=8, dim=128).fill(seed=95)                 # 32 KiB chunks, 75 MiB per op
    g_all = inputs.distinct_ids(96, 3 * n, 480)
    c_all = inputs.distinct_ids(97, 3 * n, 480)
    sets = [(g_all[i * n:(i + 1) * n], c_all[i * n:(i + 1) * n]) for i in range(3)]
    dc = DeviceCase(case)
    fresh = case.host.copy()
    for g, c in sets[1:]:
        fresh[c] ^= np.asarray(0x6B6B, dtype=case.dtype)
    dc.set_host(fresh)
    errors = []

    def loop(i):
        try:
            g, c = sets[i]
            st = torch.cuda.Stream()
            for _ in range(40):
                if i < 2:
                    abi_transfer(dc, g, c, h2d=(i == 1), mode=1, stream=st)
                else:
                    with _abi_layerwise(dc, g.copy(), c.copy(), True, 1, stream=st, ce=True) as h:
                        for grp in range(L):
                            h.wait(grp)
            st.synchronize()
        except Exception as e:   # surfaced below
            errors.append((i, e))

    th = [threading.Thread(target=loop, args=(i,)) for i in range(3)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    host, gpu = dc.host_np(), dc.gpu_np()
    (ga, ca), (gb, cb), (gc, cc) = sets
    for l in range(L):
        for k in range(2):
            assert np.array_equal(host[ca, l, k][:, 0], case.gpu[l][k][ga]), ("D2H", l, k)
            assert np.array_equal(gpu[l][k][gb], fresh[cb, l, k][:, 0]), ("H2D", l, k)
            assert np.array_equal(gpu[l][k][gc], fresh[cc, l, k][:, 0]), ("layer-wise", l, k)


def test_ce_handle_without_staging_memory():
    """A copy-engine layer-wise handle whose staging cannot be allocated moves
    every group with the zero-copy kernel, events and bytes as the engines
    would have left them."""
    from flexkv_amd import _lib
    from gpu_util import DeviceCase
    L, n = 4, 64
    case = KVCase(layers_total=L, num_layers=L, start_layer=0, kv=2, ng=128, nh=128, tokens=16,
                  heads=8, dim=128).fill(seed=80)
    s = case.strides()
    gids = inputs.distinct_ids(81, n, 128)
    cids = inputs.distinct_ids(82, n, 128)
    dc = DeviceCase(case)
    fresh = case.host ^ np.uint16(0x3C3C)
    dc.set_host(fresh)
    dc.set_gpu([np.zeros_like(g) for g in case.gpu])
    exp = [np.zeros_like(g) for g in case.gpu]
    oracle.transfer_kv_blocks(gids, exp, s["gpu_kv"], s["gpu_block"], cids, fresh, s["cpu_kv"],
                              s["cpu_layer"], s["cpu_block"], s["chunk"], 0, True)
    _lib.release_staging()
    _lib.set_staging_bytes(1 << 40)
    try:
        _lib.profile_enable(True)
        with _abi_layerwise(dc, gids.copy(), cids.copy(), True, 1, ce=True) as hnd:
            for g in range(L):
                hnd.wait(g)
                assert np.array_equal(dc.gpu_np()[g], exp[g]), g
        prof = _lib.profile_read()
    finally:
        _lib.profile_enable(False)
        _lib.set_staging_bytes(0)
        _lib.release_staging()
    assert prof["dma_batches"] == 0 and prof["kernel_launches"] == L, prof


def test_ce_handle_without_engines():
    """With the library's engines turned off (FLEXKV_SDMA_ENGINES=0), the first
    copy-engine layer-wise handle finds the engines unavailable inside its
    pipeline and moves every group with the zero-copy kernel; the second takes
    the kernel path from the start.  Both match the oracle; the warning comes
    once.  Runs in a child process, as the engine state is per process."""
    import os
    import subprocess
    import sys
    tests = os.path.dirname(os.path.abspath(__file__))
    root = os.path.dirname(tests)
    code = _NO_ENGINES_CHILD.format(root=root, tests=tests)
    res = subprocess.run([sys.executable, "-c", code], cwd=root, capture_output=True, text=True,
                         env=dict(os.environ, FLEXKV_SDMA_ENGINES="0"), timeout=300)
    print(res.stdout[-2000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0, res.stderr[-2000:]
    assert "match the oracle" in res.stdout
    assert res.stderr.count("copy engines unavailable") == 1
