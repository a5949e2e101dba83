"""fkv_transfer_kv_blocks_noalloc, the entry point that allocates nothing,
against fkv_transfer_kv_blocks in kernel mode on the same inputs, bit for
bit: ids staged in the library's fixed device scratch (two calls in a row,
the second smaller, so the scratch keeps the first call's ids beyond the
second's), a call small enough for the small-transfer kernel, ids in the
kernel arguments (32 blocks or fewer, small kernel off), the scratch's
capacity (65536 blocks) and its refusal above it, calls from two threads at
once on two streams (they take turns on the scratch), and the refusal of a
stream under HIP graph capture."""
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
def test_noalloc_matches_transfer_kv_blocks(layout, kv, monkeypatch):
    case = KVCase(layers_total=5, num_layers=4, start_layer=1, kv=kv, ng=512, nh=640, tokens=16,
                  heads=2, dim=64, layout=layout).fill(seed=80 + kv)
    a, b = DeviceCase(case), DeviceCase(case)
    # scratch, scratch (smaller), the small-transfer kernel (at most 128
    # chunks), then the same 7 blocks with the small kernel off, so the
    # general kernel takes its ids from the kernel arguments
    steps = [(300, "1"), (120, "1"), (7, "1"), (7, "0")]
    for step, (n, small) in enumerate(steps):
        monkeypatch.setenv("FLEXKV_SMALL_KERNEL", small)
        gids = inputs.distinct_ids(81 + step, n, case.ng)
        cids = inputs.distinct_ids(91 + step, n, case.nh)
        print(f"noalloc {layout} kv={kv} n={n} small_kernel={small}", flush=True)
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


def test_noalloc_two_threads_take_turns():
    """Two threads on two streams issue noalloc calls at once on disjoint
    blocks, both directions, many times over; every call stages its ids in
    the same scratch array, so each must wait for the other's kernels.  The
    result equals fkv_transfer_kv_blocks moving the union."""
    import threading
    case = KVCase(layers_total=4, num_layers=4, start_layer=0, kv=2, ng=1024, nh=1024,
                  tokens=16, heads=1, dim=64).fill(seed=70)
    ids_g = inputs.distinct_ids(71, 800, case.ng)
    ids_c = inputs.distinct_ids(72, 800, case.nh)
    halves = [(ids_g[:400], ids_c[:400]), (ids_g[400:], ids_c[400:])]
    a, b = DeviceCase(case), DeviceCase(case)
    errors = []
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()

    def worker(i, h2d, reps):
        try:
            with torch.cuda.stream(streams[i]):
                g, c = halves[i]
                for r in range(reps):
                    # a different block order each time: a stale id list
                    # would move blocks to the wrong places
                    perm = np.roll(np.arange(len(g)), 37 * r + 11 * i)
                    _noalloc(a, g[perm], c[perm], h2d)
        except Exception as e:   # noqa: BLE001 - reported below
            errors.append(e)

    for h2d in (False, True):
        if h2d:
            fresh = a.host_np() ^ np.array(0x5A5A, dtype=case.dtype)
            for dc in (a, b):
                dc.set_host(fresh)
                dc.set_gpu([np.zeros_like(x) for x in case.gpu])
            torch.cuda.synchronize()
        print(f"noalloc two threads h2d={h2d}", flush=True)
        ths = [threading.Thread(target=worker, args=(i, h2d, 25)) for i in range(2)]
        for t in ths:
            t.start()
        for t in ths:
            t.join()
        assert not errors, errors
        abi_transfer(b, ids_g, ids_c, h2d, 0)
        torch.cuda.synchronize()
        if h2d:
            for l, (x, y) in enumerate(zip(a.gpu_np(), b.gpu_np())):
                assert np.array_equal(x, y), f"layer {l}"
        else:
            assert np.array_equal(a.host_np(), b.host_np())
            assert np.array_equal(a.host_np(), case.expect_d2h(ids_g, ids_c))   # numpy indexing


def test_noalloc_refuses_a_capturing_stream():
    """Under HIP graph capture the call is refused before anything is queued;
    the capture itself stays valid and ends with an empty graph."""
    from flexkv_amd import _lib
    hip = ctypes.CDLL("libamdhip64.so")   # the runtime torch loaded (same soname)
    case = KVCase(layers_total=2, num_layers=2, start_layer=0, kv=2, ng=64, nh=64, tokens=16,
                  heads=1, dim=64).fill(seed=60)
    a = DeviceCase(case)
    gids = inputs.distinct_ids(61, 40, case.ng)
    cids = inputs.distinct_ids(62, 40, case.nh)
    st = torch.cuda.Stream()
    torch.cuda.synchronize()
    relaxed = 2   # hipStreamCaptureModeRelaxed
    assert hip.hipStreamBeginCapture(ctypes.c_void_p(st.cuda_stream), relaxed) == 0
    graph = ctypes.c_void_p()
    try:
        with torch.cuda.stream(st):
            with pytest.raises(RuntimeError, match="graph capture"):
                _noalloc(a, gids, cids, False)
        assert "capture" in _lib.last_error()
    finally:
        assert hip.hipStreamEndCapture(ctypes.c_void_p(st.cuda_stream), ctypes.byref(graph)) == 0
        if graph.value:
            hip.hipGraphDestroy(graph)
    torch.cuda.synchronize()
    assert np.array_equal(a.host_np(), case.host), "a refused call moved bytes"
    # the stream works normally afterwards
    with torch.cuda.stream(st):
        _noalloc(a, gids, cids, False)
    st.synchronize()
    assert np.array_equal(a.host_np(), case.expect_d2h(gids, cids))
