"""GPU parity: the HIP transfer paths against the CPU oracle, byte for byte.

Each case runs the oracle (oracle/kv_oracle.c) and the device path on the same
inputs and compares every byte of the destination, including blocks that must
stay untouched.  Modes: 0 = zero-copy kernel, 1 = copy engines through HBM
staging, 2 = one DMA per chunk (the reference's CE loop).
"""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

import oracle
from oracle import inputs
from kvcase import KVCase

pytestmark = pytest.mark.gpu

MODES = [0, 1, 2]
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def dev():
    from flexkv_amd import _lib
    _lib.load()
    return torch.device("cuda:0")


def _oracle_d2h(case, gids, cids, mode):
    s = case.strides()
    host = case.host.copy()
    oracle.transfer_kv_blocks(gids, case.gpu, s["gpu_kv"], s["gpu_block"], cids, host,
                              s["cpu_kv"], s["cpu_layer"], s["cpu_block"], s["chunk"],
                              case.start_layer, False, use_ce_transfer=(mode != 0),
                              is_mla=case.kv == 1, cpu_startoff_inside_chunks=s["startoff"])
    return host


def _oracle_h2d(case, gids, cids, gpu_init, mode):
    s = case.strides()
    out = [g.copy() for g in gpu_init]
    oracle.transfer_kv_blocks(gids, out, s["gpu_kv"], s["gpu_block"], cids, case.host,
                              s["cpu_kv"], s["cpu_layer"], s["cpu_block"], s["chunk"],
                              case.start_layer, True, use_ce_transfer=(mode != 0),
                              is_mla=case.kv == 1, cpu_startoff_inside_chunks=s["startoff"])
    return out


def check_case(case, gids, cids, mode, transfer_cus=-1):
    from gpu_util import DeviceCase, abi_transfer
    print(f"case L={case.num_layers} kv={case.kv} n={len(gids)} chunk={case.strides()['chunk']} "
          f"layout={case.layout} mode={mode}", flush=True)
    dc = DeviceCase(case)
    abi_transfer(dc, gids, cids, h2d=False, mode=mode, transfer_cus=transfer_cus)
    torch.cuda.synchronize()
    want = _oracle_d2h(case, gids, cids, mode)
    got = dc.host_np()
    assert np.array_equal(got, want), "D2H differs from the oracle"
    # H2D from a host cache holding fresh values into a sentinel-filled GPU
    case2 = KVCase(**{k: getattr(case, k) for k in (
        "layers_total", "num_layers", "start_layer", "kv", "ng", "nh", "tokens", "heads", "dim",
        "dtype", "layout", "tp", "rank")})
    case2.fill(seed=99)
    flip = 0x1234 & ((1 << (8 * np.dtype(case.dtype).itemsize)) - 1)
    case2.host = want ^ np.asarray(flip, dtype=case.dtype)
    init = case2.gpu
    dc.set_host(case2.host)
    dc.set_gpu(init)
    abi_transfer(dc, gids, cids, h2d=True, mode=mode, transfer_cus=transfer_cus)
    torch.cuda.synchronize()
    want_g = _oracle_h2d(case2, gids, cids, init, mode)
    for l, (g, w) in enumerate(zip(dc.gpu_np(), want_g)):
        assert np.array_equal(g, w), f"H2D differs from the oracle at layer {l}"


@pytest.mark.parametrize("mode", MODES)
def test_tiny_fixture_vectors(dev, mode):
    fx = np.load(os.path.join(GOLDEN, "tiny_vectors.npz"), allow_pickle=False)
    meta = json.loads(str(fx["meta"]))
    from gpu_util import DeviceCase, abi_transfer
    for i, m in enumerate(meta):
        case = KVCase(**m["shape"])
        case.gpu = [fx[f"c{i}_gpu{l}"] for l in range(case.num_layers)]
        case.host = fx[f"c{i}_host"]
        gids, cids = fx[f"c{i}_gids"], fx[f"c{i}_cids"]
        dc = DeviceCase(case)
        abi_transfer(dc, gids, cids, h2d=False, mode=mode)
        torch.cuda.synchronize()
        assert np.array_equal(dc.host_np(), fx[f"c{i}_want_host"]), m
        dc.set_gpu([np.zeros_like(g) for g in case.gpu])
        abi_transfer(dc, gids, cids, h2d=True, mode=mode)
        torch.cuda.synchronize()
        for l, g in enumerate(dc.gpu_np()):
            assert np.array_equal(g, fx[f"c{i}_want_gpu{l}"]), m


@pytest.mark.parametrize("mode", MODES)
def test_config0_digests(dev, mode):
    """The CPU-plumbing configuration on the GPU reproduces the committed digests."""
    from golden.gen_golden import config0_case, config0_ids
    from gpu_util import DeviceCase, abi_transfer
    with open(os.path.join(GOLDEN, "config0_digests.json")) as fh:
        want = json.load(fh)
    case = config0_case()
    gids, cids = config0_ids()
    dc = DeviceCase(case)
    abi_transfer(dc, gids, cids, h2d=False, mode=mode)
    torch.cuda.synchronize()
    assert hashlib.sha256(dc.host_np().tobytes()).hexdigest() == want["d2h_host_sha256"]
    dc.set_gpu([np.zeros_like(g) for g in case.gpu])
    abi_transfer(dc, gids, cids, h2d=True, mode=mode)
    torch.cuda.synchronize()
    got = b"".join(g.tobytes() for g in dc.gpu_np())
    assert hashlib.sha256(got).hexdigest() == want["h2d_gpu_sha256"]


GEOMETRIES = [
    # (layers_total, num_layers, start, kv, ng, nh, tokens, heads, dim, dtype, layout, tp, rank, n)
    (4, 4, 0, 2, 64, 96, 16, 8, 128, np.uint16, "BLOCKWISE", 1, 0, 40),
    (4, 4, 0, 2, 64, 96, 16, 8, 128, np.uint16, "LAYERWISE", 1, 0, 40),
    (6, 3, 2, 2, 50, 70, 16, 1, 128, np.uint16, "BLOCKWISE", 1, 0, 33),   # 4 KiB chunks, layer window
    (5, 5, 0, 1, 30, 40, 64, 1, 576, np.uint16, "BLOCKWISE", 1, 0, 20),   # MLA latent, 72 KiB chunks
    (3, 3, 0, 2, 20, 20, 1, 1, 24, np.uint16, "BLOCKWISE", 1, 0, 7),      # 48 B chunk: partial row
    (3, 2, 1, 2, 20, 30, 1, 5, 104, np.uint16, "LAYERWISE", 1, 0, 9),     # 1040 B = 65 vectors
    (2, 2, 0, 2, 40, 40, 16, 2, 128, np.uint16, "BLOCKWISE", 4, 3, 25),   # TP host chunk, rank 3
    (130, 130, 0, 2, 6, 8, 1, 1, 64, np.uint16, "BLOCKWISE", 1, 0, 5),    # >128 layers: 2 launches
    (2, 2, 0, 2, 600, 700, 2, 2, 32, np.uint32, "BLOCKWISE", 1, 0, 520),  # many tiles
    (4, 4, 0, 2, 64, 96, 16, 8, 128, np.uint8, "LAYERWISE", 1, 0, 40),    # 1-byte (fp8) cache
    # Zero-copy D2H groups of 8 rows as two 4-row sub-groups: MLA 4 KiB chunks
    # over an odd number of chunks (a group's second sub-group past the end),
    # and 12 KiB chunks (groups across two chunks); both over 128 chunks, so
    # the general kernel takes them.
    (3, 3, 0, 1, 60, 80, 16, 1, 128, np.uint16, "BLOCKWISE", 1, 0, 45),
    (3, 3, 0, 1, 50, 60, 16, 3, 128, np.uint16, "BLOCKWISE", 1, 0, 43),
]


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("geo", GEOMETRIES, ids=[f"g{i}" for i in range(len(GEOMETRIES))])
def test_geometries_match_oracle(dev, geo, mode):
    lt, nl, st, kv, ng, nh, t, h, d, dt, layout, tp, rank, n = geo
    case = KVCase(layers_total=lt, num_layers=nl, start_layer=st, kv=kv, ng=ng, nh=nh, tokens=t,
                  heads=h, dim=d, dtype=dt, layout=layout, tp=tp, rank=rank).fill(seed=lt * 7 + n)
    gids = inputs.distinct_ids(n + 1, n, ng)
    cids = inputs.distinct_ids(n + 2, n, nh)
    check_case(case, gids, cids, mode)


@pytest.mark.parametrize("kv,layers,n", [(2, 8, 504), (2, 8, 520), (1, 9, 925), (1, 9, 939),
                                         (1, 9, 1851)],
                         ids=["kv-31.5MiB", "kv-32.5MiB", "mla-32.5MiB-odd", "mla-33MiB-odd",
                              "mla-65MiB-odd"])
def test_zero_copy_variants_at_the_size_policy_edges(dev, kv, layers, n):
    """Kernel-mode calls on either side of the sizes where the zero-copy
    kernel changes variant: host-to-device calls take the whole-group kernel
    from 32 MiB and the row-by-row one below, device-to-host calls the
    whole-group kernel of two 4-row sub-groups (4 CUs from 64 MiB).  4 KiB
    chunks; the MLA-shaped calls move an odd number of chunks (9 layers), so
    a group's second sub-group can lie past the end of a launch."""
    ng = max(1200, n + 200)
    case = KVCase(layers_total=layers, num_layers=layers, start_layer=0, kv=kv, ng=ng,
                  nh=ng + 100, tokens=16, heads=1, dim=128).fill(seed=kv * 1000 + n)
    gids = inputs.distinct_ids(n + 5, n, ng)
    cids = inputs.distinct_ids(n + 6, n, ng + 100)
    check_case(case, gids, cids, 0)


@pytest.mark.parametrize("h2d", [False, True])
@pytest.mark.parametrize("layout,heads", [("BLOCKWISE", 8), ("LAYERWISE", 8), ("BLOCKWISE", 1),
                                          ("LAYERWISE", 1)])
def test_copy_engine_size_policy(dev, h2d, layout, heads, monkeypatch):
    """Copy-engine mode sends transfers under FLEXKV_CE_MIN_BYTES, or whose
    engine copies would move under 128 KiB each, to the zero-copy kernel and
    the rest to the SDMA engines; 0 forces the engines.  An engine copy is a
    contiguous host run (block-wise host: a block's 4 layers) or one block's
    chunks as a rect copy (layer-wise host): 256 KiB with 32 KiB chunks, 32 KiB
    with 4 KiB chunks.  The bytes are the same either way.  The library's
    profile counts SDMA batches."""
    from flexkv_amd import _lib
    from gpu_util import DeviceCase, abi_transfer
    case = KVCase(layers_total=4, num_layers=4, start_layer=0, kv=2, ng=64, nh=96, tokens=16,
                  heads=heads, dim=128, layout=layout).fill(seed=31)   # 32 or 4 KiB chunks
    n = 20
    gids = inputs.distinct_ids(3, n, 64)
    cids = inputs.distinct_ids(4, n, 96)
    want = _oracle_d2h(case, gids, cids, 1)
    chunk = 16 * heads * 128 * 2
    total = n * 4 * 2 * chunk
    rows = 4 * 2 * chunk >= 128 << 10
    for env, engines in (("0", True), (None, False), (str(total), rows), (str(total + 1), False)):
        if env is None:
            monkeypatch.delenv("FLEXKV_CE_MIN_BYTES", raising=False)
        else:
            monkeypatch.setenv("FLEXKV_CE_MIN_BYTES", env)
        print(f"policy layout={layout} h2d={h2d} env={env}", flush=True)
        dc = DeviceCase(case)
        _lib.profile_enable(True)
        abi_transfer(dc, gids, cids, h2d=False, mode=1)
        if h2d:
            dc.set_gpu([np.zeros_like(g) for g in case.gpu])
            abi_transfer(dc, gids, cids, h2d=True, mode=1)
        prof = _lib.profile_read()
        _lib.profile_enable(False)
        torch.cuda.synchronize()
        assert (prof["dma_batches"] > 0) == engines, (env, prof)
        assert np.array_equal(dc.host_np(), want)
        if h2d:
            for l, g in enumerate(dc.gpu_np()):
                expect = np.zeros_like(case.gpu[l])
                expect[:, gids] = case.gpu[l][:, gids]
                assert np.array_equal(g, expect), f"layer {l}"


@pytest.mark.parametrize("mla,window", [(False, (0, 5)), (False, (2, 1)), (True, (0, 5)),
                                        (False, (1, 3))])
def test_layerwise_host_copy_engines_one_rect_per_block(dev, mla, window):
    """On a layer-wise host cache ([layer][K|V][block][chunk]) copy-engine
    mode moves each block's layer window with one rect copy: as many SDMA
    copies as blocks in both directions; the host cache equals the oracle's
    byte for byte and the round trip restores the blocks."""
    from flexkv_amd import _lib
    from gpu_util import DeviceCase, abi_transfer
    start, nl = window
    case = KVCase(layers_total=6, num_layers=nl, start_layer=start, kv=1 if mla else 2, ng=48,
                  nh=80, tokens=16, heads=4, dim=128, layout="LAYERWISE").fill(seed=37)
    n = 23
    gids = inputs.distinct_ids(7, n, 48)
    cids = inputs.distinct_ids(8, n, 80)
    print(f"rect mla={mla} window={window}", flush=True)
    dc = DeviceCase(case)
    _lib.profile_enable(True)
    abi_transfer(dc, gids, cids, h2d=False, mode=1)
    prof = _lib.profile_read()
    torch.cuda.synchronize()
    assert prof["dma_copies"] == n, prof
    assert np.array_equal(dc.host_np(), _oracle_d2h(case, gids, cids, 1))
    zero = [np.zeros_like(g) for g in case.gpu]
    dc.set_gpu(zero)
    _lib.profile_enable(True)
    abi_transfer(dc, gids, cids, h2d=True, mode=1)
    prof = _lib.profile_read()
    _lib.profile_enable(False)
    torch.cuda.synchronize()
    assert prof["dma_copies"] == n, prof
    # the round trip restores the moved blocks into the zeroed layers
    for l, g in enumerate(dc.gpu_np()):
        expect = np.zeros_like(case.gpu[l])
        expect[:, gids] = case.gpu[l][:, gids]
        assert np.array_equal(g, expect), f"layer {l}"


def test_rect_policy_default(dev, monkeypatch):
    """Without FLEXKV_CE_RECT_COPIES, copy-engine mode moves a layer-wise host
    cache with scattered ids with the zero-copy kernel (no SDMA batch), and
    one whose ids come in long runs with the engines (layer-major staging);
    the bytes match the oracle either way."""
    from flexkv_amd import _lib
    from gpu_util import DeviceCase, abi_transfer
    monkeypatch.delenv("FLEXKV_CE_RECT_COPIES", raising=False)
    monkeypatch.delenv("FLEXKV_CE_LAYER_RUN_BYTES", raising=False)
    case = KVCase(layers_total=4, num_layers=4, start_layer=0, kv=2, ng=64, nh=96, tokens=16,
                  heads=4, dim=128, layout="LAYERWISE").fill(seed=53)   # 16 KiB chunks
    runs = np.concatenate([np.arange(0, 32), np.arange(40, 72)])     # 512 KiB per run
    for name, cids, engines in (("scattered", inputs.distinct_ids(12, 32, 96), False),
                                ("runs", runs, True)):
        cids = np.ascontiguousarray(cids, dtype=np.int64)
        gids = inputs.distinct_ids(13, len(cids), 64)
        print(f"rect policy {name}", flush=True)
        dc = DeviceCase(case)
        for h2d in (False, True):
            if h2d:
                dc.set_gpu([np.zeros_like(g) for g in case.gpu])
            _lib.profile_enable(True)
            abi_transfer(dc, gids, cids, h2d=h2d, mode=1)
            prof = _lib.profile_read()
            _lib.profile_enable(False)
            torch.cuda.synchronize()
            assert (prof["dma_batches"] > 0) == engines, (name, h2d, prof)
        assert np.array_equal(dc.host_np(), _oracle_d2h(case, gids, cids, 1))
        for l, g in enumerate(dc.gpu_np()):
            expect = np.zeros_like(case.gpu[l])
            expect[:, gids] = case.gpu[l][:, gids]
            assert np.array_equal(g, expect), f"{name} layer {l}"


def test_copy_engine_policy_api_routes_transfers(dev, monkeypatch):
    """c_ext.set_copy_engine_policy overrides the FLEXKV_CE_* variables: a
    layer-wise host cache with scattered ids moves with rect copies under
    layerwise_scattered="rect_copies" and with the zero-copy kernel under
    "kernel"; a min_bytes above the transfer sends it to the kernel.  The
    bytes match the oracle every time; "unset" returns to the variables."""
    from flexkv_amd import _lib, c_ext
    from gpu_util import DeviceCase, abi_transfer
    monkeypatch.setenv("FLEXKV_CE_MIN_BYTES", "0")
    monkeypatch.setenv("FLEXKV_CE_RECT_COPIES", "1")
    case = KVCase(layers_total=4, num_layers=4, start_layer=0, kv=2, ng=64, nh=96, tokens=16,
                  heads=4, dim=128, layout="LAYERWISE").fill(seed=54)   # 16 KiB chunks
    gids = inputs.distinct_ids(14, 24, 64)
    cids = inputs.distinct_ids(15, 24, 96)
    total = 24 * 4 * 2 * 16384
    want = _oracle_d2h(case, gids, cids, 1)
    try:
        for policy, engines in (({"layerwise_scattered": "kernel"}, False),
                                ({"layerwise_scattered": "rect_copies"}, True),
                                ({"min_bytes": total + 1}, False),
                                ({"min_bytes": total}, True)):
            c_ext.set_copy_engine_policy(**policy)
            print(f"policy {policy}: {c_ext.copy_engine_policy()}", flush=True)
            dc = DeviceCase(case)
            _lib.profile_enable(True)
            abi_transfer(dc, gids, cids, h2d=False, mode=1)
            prof = _lib.profile_read()
            _lib.profile_enable(False)
            torch.cuda.synchronize()
            assert (prof["dma_batches"] > 0) == engines, (policy, prof)
            assert np.array_equal(dc.host_np(), want)
    finally:
        c_ext.set_copy_engine_policy(min_bytes="unset", layerwise_scattered="unset")
    assert c_ext.copy_engine_policy() == {"min_bytes": 0, "rect_copies": 1,
                                          "layerwise_scattered": "rect_copies"}


@pytest.mark.parametrize("mla", [False, True])
def test_layerwise_host_id_runs_stage_layer_major(dev, mla, monkeypatch):
    """On a layer-wise host cache whose ids come in runs of consecutive blocks
    (average run at least FLEXKV_CE_LAYER_RUN_BYTES), copy-engine mode stages
    the blocks layer-major and copies each run of each (layer, K|V) linearly:
    runs x layers x K|V SDMA copies instead of one rect copy per block.
    Bytes as the oracle's, and the round trip restores the blocks."""
    from flexkv_amd import _lib
    from gpu_util import DeviceCase, abi_transfer
    kv = 1 if mla else 2
    case = KVCase(layers_total=5, num_layers=4, start_layer=1, kv=kv, ng=64, nh=96, tokens=16,
                  heads=4, dim=128, layout="LAYERWISE").fill(seed=43)   # 16 KiB chunks
    chunk = 16 * 4 * 128 * 2
    cids = np.concatenate([np.arange(10, 18), np.arange(40, 52), np.arange(70, 75)])
    n = len(cids)                                     # 3 runs, 25 blocks
    gids = inputs.distinct_ids(9, n, 64)
    monkeypatch.setenv("FLEXKV_CE_LAYER_RUN_BYTES", str(4 * chunk))
    for order, ids, copies in (("layer-major", cids, 3 * 4 * kv),
                               ("rect", inputs.distinct_ids(10, n, 96), n)):
        print(f"runs mla={mla} order={order}", flush=True)
        ids = np.ascontiguousarray(ids, dtype=np.int64)
        dc = DeviceCase(case)
        _lib.profile_enable(True)
        abi_transfer(dc, gids, ids, h2d=False, mode=1)
        prof = _lib.profile_read()
        torch.cuda.synchronize()
        assert prof["dma_copies"] == copies, (order, prof)
        assert np.array_equal(dc.host_np(), _oracle_d2h(case, gids, ids, 1))
        zero = [np.zeros_like(g) for g in case.gpu]
        dc.set_gpu(zero)
        _lib.profile_enable(True)
        abi_transfer(dc, gids, ids, h2d=True, mode=1)
        prof = _lib.profile_read()
        _lib.profile_enable(False)
        torch.cuda.synchronize()
        assert prof["dma_copies"] == copies, (order, prof)
        for l, g in enumerate(dc.gpu_np()):
            expect = np.zeros_like(case.gpu[l])
            expect[:, gids] = case.gpu[l][:, gids]
            assert np.array_equal(g, expect), f"{order} layer {l}"


def test_layer_major_threshold_per_direction(dev, monkeypatch):
    """Default thresholds: runs of 256 KiB per (layer, K|V) are staged
    layer-major device-to-host (threshold 192 KiB) but move as one rect copy
    per block host-to-device (threshold 384 KiB); both round-trip exactly."""
    from flexkv_amd import _lib
    from gpu_util import DeviceCase, abi_transfer
    monkeypatch.delenv("FLEXKV_CE_LAYER_RUN_BYTES", raising=False)
    case = KVCase(layers_total=4, num_layers=4, start_layer=0, kv=2, ng=64, nh=96, tokens=16,
                  heads=4, dim=128, layout="LAYERWISE").fill(seed=47)   # 16 KiB chunks
    cids = np.concatenate([np.arange(0, 16), np.arange(30, 46), np.arange(60, 76)])
    n = len(cids)                                     # 3 runs of 16 blocks = 256 KiB
    gids = inputs.distinct_ids(11, n, 64)
    ids = np.ascontiguousarray(cids, dtype=np.int64)
    dc = DeviceCase(case)
    _lib.profile_enable(True)
    abi_transfer(dc, gids, ids, h2d=False, mode=1)
    prof = _lib.profile_read()
    torch.cuda.synchronize()
    assert prof["dma_copies"] == 3 * 4 * 2, prof      # runs x layers x K|V
    assert np.array_equal(dc.host_np(), _oracle_d2h(case, gids, ids, 1))
    dc.set_gpu([np.zeros_like(g) for g in case.gpu])
    _lib.profile_enable(True)
    abi_transfer(dc, gids, ids, h2d=True, mode=1)
    prof = _lib.profile_read()
    _lib.profile_enable(False)
    torch.cuda.synchronize()
    assert prof["dma_copies"] == n, prof              # one rect copy per block
    for l, g in enumerate(dc.gpu_np()):
        expect = np.zeros_like(case.gpu[l])
        expect[:, gids] = case.gpu[l][:, gids]
        assert np.array_equal(g, expect), f"layer {l}"


@pytest.mark.parametrize("mode", MODES)
def test_device_resident_cache_matches_oracle(dev, mode):
    """A "host" cache that lives in device memory (allowed by the API) moves
    the same bytes in every mode; copy-engine mode uses the kernel for it."""
    import ctypes
    from flexkv_amd import _lib
    from gpu_util import to_torch
    case = KVCase(layers_total=3, num_layers=3, start_layer=0, kv=2, ng=40, nh=50, tokens=16,
                  heads=2, dim=64).fill(seed=41)
    gids = inputs.distinct_ids(5, 17, 40)
    cids = inputs.distinct_ids(6, 17, 50)
    s = case.strides()
    gpu = [to_torch(g).to(dev) for g in case.gpu]
    host_dev = to_torch(case.host.reshape(-1)).to(dev)
    ptrs = (ctypes.c_void_p * 3)(*[t.data_ptr() for t in gpu])
    lib = _lib.load()
    rc = lib.fkv_transfer_kv_blocks(
        len(gids), 0, 3, gids.ctypes.data, ptrs, s["gpu_kv"], s["gpu_block"], cids.ctypes.data,
        host_dev.data_ptr(), s["cpu_kv"], s["cpu_layer"], s["cpu_block"], 0, s["chunk"],
        torch.cuda.current_stream().cuda_stream, -1, 0, mode, 0)
    _lib.check(rc, "fkv_transfer_kv_blocks")
    torch.cuda.synchronize()
    got = host_dev.cpu().numpy().view(case.dtype).reshape(case.host_shape())
    assert np.array_equal(got, _oracle_d2h(case, gids, cids, mode))


@pytest.mark.parametrize("layout", ["BLOCKWISE", "LAYERWISE"])
def test_concurrent_threads_mixed_paths(dev, layout):
    """Four host threads, each with its own stream, move disjoint block sets
    with different paths and directions at once (id buffers are per thread;
    copy-engine staging and SDMA state per direction, a D2H and an H2D
    copy-engine transfer running side by side; rect transfers of a
    layer-wise cache take both directions); every result is bit-exact."""
    import threading
    from gpu_util import DeviceCase, abi_transfer
    case = KVCase(layers_total=4, num_layers=4, start_layer=0, kv=2, ng=256, nh=256, tokens=16,
                  heads=8, dim=128, layout=layout).fill(seed=43)
    dc = DeviceCase(case)
    perm_g = inputs.distinct_ids(7, 240, 256)
    perm_c = inputs.distinct_ids(8, 240, 256)
    parts = [(perm_g[i * 60:(i + 1) * 60], perm_c[i * 60:(i + 1) * 60]) for i in range(4)]
    plan = [(False, 0), (False, 1), (True, 1), (True, 0)]   # (h2d, mode) per thread
    # H2D threads read host blocks that hold distinct fresh values first
    fresh = case.host.copy()

    def block(arr, c, l, k):      # host chunks [len(c), tp, tokens, heads, dim]
        return arr[c, l, k] if layout == "BLOCKWISE" else arr[l, k, c]

    for (h2d, _), (g, c) in zip(plan, parts):
        if h2d:
            if layout == "BLOCKWISE":
                fresh[c] ^= np.asarray(0x0F0F, dtype=case.dtype)
            else:
                fresh[:, :, c] ^= np.asarray(0x0F0F, dtype=case.dtype)
    dc.set_host(fresh)
    errors = []

    def run(i):
        try:
            h2d, mode = plan[i]
            g, c = parts[i]
            st = torch.cuda.Stream()
            with torch.cuda.stream(st):
                for _ in range(3):
                    abi_transfer(dc, g, c, h2d=h2d, mode=mode, stream=st)
            st.synchronize()
        except Exception as e:   # surfaced below
            errors.append(e)

    threads = [threading.Thread(target=run, args=(i,)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    host = dc.host_np()
    gpu = dc.gpu_np()
    for (h2d, mode), (g, c) in zip(plan, parts):
        if h2d:
            for l in range(4):
                for k in range(2):
                    assert np.array_equal(gpu[l][k][g], block(fresh, c, l, k)[:, 0]), (mode, l, k)
        else:
            for l in range(4):
                for k in range(2):
                    assert np.array_equal(block(host, c, l, k)[:, 0], case.gpu[l][k][g]), \
                        (mode, l, k)


def test_duplex_copy_engine_transfers(dev):
    """A copy-engine D2H and a copy-engine H2D of 128 MiB each, repeated from
    two threads so that they overlap over many staging halves: while both
    are in flight their copies take the duplex engine split, and halves
    issued before, during and after the overlap land on different engine
    sets.  Every byte matches."""
    import threading
    from gpu_util import DeviceCase, abi_transfer
    from flexkv_amd import _lib
    case = KVCase(layers_total=8, num_layers=8, start_layer=0, kv=2, ng=600, nh=600, tokens=16,
                  heads=8, dim=128).fill(seed=91)         # 32 KiB chunks
    dc = DeviceCase(case)
    g_all = inputs.distinct_ids(92, 512, 600)
    c_all = inputs.distinct_ids(93, 512, 600)
    (g_d, c_d), (g_h, c_h) = (g_all[:256], c_all[:256]), (g_all[256:], c_all[256:])
    fresh = case.host.copy()
    fresh[c_h] ^= np.asarray(0x5A5A, dtype=case.dtype)
    dc.set_host(fresh)
    _lib.set_staging_bytes(64 << 20)                       # 32 MiB halves: 4+ halves a call
    errors = []

    def run(h2d):
        try:
            st = torch.cuda.Stream()
            g, c = (g_h, c_h) if h2d else (g_d, c_d)
            for _ in range(6):
                abi_transfer(dc, g, c, h2d=h2d, mode=1, stream=st)
            st.synchronize()
        except Exception as e:   # surfaced below
            errors.append(e)
    try:
        th = [threading.Thread(target=run, args=(h,)) for h in (False, True)]
        for t in th:
            t.start()
        for t in th:
            t.join()
    finally:
        _lib.set_staging_bytes(0)
        _lib.release_staging()
    torch.cuda.synchronize()
    assert not errors, errors
    host, gpu = dc.host_np(), dc.gpu_np()
    for l in range(8):
        for k in range(2):
            assert np.array_equal(host[c_d, l, k][:, 0], case.gpu[l][k][g_d]), ("D2H", l, k)
            assert np.array_equal(gpu[l][k][g_h], fresh[c_h, l, k][:, 0]), ("H2D", l, k)


# Separate K and V allocations (fkv_transfer_kv_blocks_kv_ptrs): the same
# bytes must move as with K and V halves of one allocation, so the oracle of
# the combined layout is the expectation.  Geometry 7 (130 layers) needs three
# launches at 64 layers of K/V pointer pairs each.
@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("geo", [GEOMETRIES[i] for i in (0, 1, 2, 3, 5, 6, 7)],
                         ids=[f"g{i}" for i in (0, 1, 2, 3, 5, 6, 7)])
def test_separate_kv_allocations_match_oracle(dev, geo, mode):
    from gpu_util import DeviceCase, abi_transfer_kv_ptrs, split_kv_layers
    lt, nl, st, kv, ng, nh, t, h, d, dt, layout, tp, rank, n = geo
    print(f"kv_ptrs L={nl} kv={kv} n={n} layout={layout} mode={mode}", flush=True)
    case = KVCase(layers_total=lt, num_layers=nl, start_layer=st, kv=kv, ng=ng, nh=nh, tokens=t,
                  heads=h, dim=d, dtype=dt, layout=layout, tp=tp, rank=rank).fill(seed=lt * 5 + n)
    gids = inputs.distinct_ids(n + 3, n, ng)
    cids = inputs.distinct_ids(n + 4, n, nh)
    dc = DeviceCase(case)
    kvt = split_kv_layers(dc)
    abi_transfer_kv_ptrs(dc, kvt, gids, cids, h2d=False, mode=mode)
    torch.cuda.synchronize()
    assert np.array_equal(dc.host_np(), _oracle_d2h(case, gids, cids, mode)), "D2H"
    # H2D of fresh host values into sentinel-filled separate tensors
    fresh = KVCase(**{k: getattr(case, k) for k in (
        "layers_total", "num_layers", "start_layer", "kv", "ng", "nh", "tokens", "heads", "dim",
        "dtype", "layout", "tp", "rank")}).fill(seed=77)
    dc.set_host(fresh.host)
    for l, pair in enumerate(kvt):
        for k, tk in enumerate(pair):
            tk.copy_(to_torch_layer(fresh.gpu[l][k]))
    abi_transfer_kv_ptrs(dc, kvt, gids, cids, h2d=True, mode=mode)
    torch.cuda.synchronize()
    want = _oracle_h2d(fresh, gids, cids, fresh.gpu, mode)
    for l, pair in enumerate(kvt):
        for k, tk in enumerate(pair):
            got = tk.cpu().numpy().view(case.dtype)
            assert np.array_equal(got, want[l][k]), f"H2D layer {l} half {k}"


def to_torch_layer(a):
    from gpu_util import to_torch
    return to_torch(a)


def test_separate_kv_rejects_bad_pointers(dev):
    """A K/V pointer outside device memory, or ids past a separate tensor's
    end, are refused before any launch."""
    import ctypes
    from flexkv_amd import _lib
    from gpu_util import DeviceCase, abi_transfer_kv_ptrs, split_kv_layers
    case = KVCase(layers_total=2, num_layers=2, start_layer=0, kv=2, ng=8, nh=8, tokens=16,
                  heads=1, dim=64).fill(seed=5)
    dc = DeviceCase(case)
    kvt = split_kv_layers(dc)
    with pytest.raises(RuntimeError, match="outside the allocation"):
        abi_transfer_kv_ptrs(dc, kvt, np.array([1 << 22]), np.array([0]), h2d=False, mode=0)
    kvt[1][1] = torch.empty_like(kvt[1][1], device="cpu")     # host memory as a V pointer
    with pytest.raises(RuntimeError, match="not device memory"):
        abi_transfer_kv_ptrs(dc, kvt, np.array([0]), np.array([0]), h2d=False, mode=0)


@pytest.mark.parametrize("cus", [1, 3, 256])
def test_zero_copy_cu_limits(dev, cus):
    case = KVCase(layers_total=4, num_layers=4, start_layer=0, kv=2, ng=80, nh=80, tokens=16,
                  heads=2, dim=128).fill(seed=cus)
    check_case(case, inputs.distinct_ids(1, 64, 80), inputs.distinct_ids(2, 64, 80), 0, cus)


@pytest.mark.parametrize("heads", [2, 8])
@pytest.mark.parametrize("run", [1, 8, 64])
def test_staged_runs_and_small_staging(dev, run, heads):
    """Copy-engine path with a tiny staging buffer: many pieces, run merging
    across consecutive host ids, and a layer window split.  8 KiB chunks take
    the general gather; 32 KiB chunks (8 heads, host layers 2..9 of 10) the
    whole-group gather, with pieces that start past layer 0."""
    from flexkv_amd import _lib
    _lib.set_staging_bytes(1 << 20)
    try:
        start = 2 if heads == 8 else 0
        case = KVCase(layers_total=8 + start, num_layers=8, start_layer=start, kv=2, ng=256,
                      nh=512, tokens=16, heads=heads, dim=128).fill(seed=run)
        gids = inputs.run_ids(3, 128, 256, run)
        cids = inputs.run_ids(4, 128, 512, run)
        check_case(case, gids, cids, 1)
        # one block row (8*2*8 KiB = 128 KiB, or 512 KiB) per half would not
        # fit 64 KiB: the layer window splits
        _lib.release_staging()
        _lib.set_staging_bytes(128 << 10)
        check_case(case, gids, cids, 1)
    finally:
        _lib.release_staging()
        _lib.set_staging_bytes(0)


@pytest.mark.parametrize("scale", ["0", "1", "40"])
def test_held_engines_wait_for_the_scatter(dev, scale, monkeypatch):
    """Host-to-device copies shorter than 1 MiB spread over the six-engine set,
    and from the second piece on, the engines beyond the first four take their
    share only once the scatter of the previous piece is done (queued
    afterwards, counted as dma_held_copies).  64 KiB block rows in 512 KiB
    staging halves: 16 pieces of 8 copies.  Scale 0 holds nothing, 1 is the
    default, 40 defers the most the split allows; bytes match the oracle."""
    from flexkv_amd import _lib
    monkeypatch.setenv("FLEXKV_SDMA_HOLD_SCALE", scale)
    _lib.set_staging_bytes(1 << 20)
    try:
        case = KVCase(layers_total=8, num_layers=8, start_layer=0, kv=2, ng=256, nh=512,
                      tokens=16, heads=1, dim=128).fill(seed=int(scale) + 3)
        gids = inputs.distinct_ids(7, 128, 256)
        cids = inputs.distinct_ids(8, 128, 512)
        _lib.profile_enable(True)
        check_case(case, gids, cids, 1)
        prof = _lib.profile_read()
        _lib.profile_enable(False)
        assert prof["dma_copies"] == 2 * 128, prof
        if scale == "0":
            assert prof["dma_held_copies"] == 0, prof
        else:
            assert 15 <= prof["dma_held_copies"] <= 15 * 4, prof
    finally:
        _lib.profile_enable(False)
        _lib.release_staging()
        _lib.set_staging_bytes(0)


@pytest.mark.parametrize("blocks,launches", [(384, 2), (192, 2), (48, 1)])
def test_copy_engine_edge_piece(dev, blocks, launches):
    """A copy-engine transfer whose piece without engine copies beside it (the
    D2H's first gather, the H2D's last scatter) moves at least 128 MiB cuts
    an eighth of a staging half off it: 384 blocks of 512 KiB (192 MiB) in
    256 MiB halves go as 64 + 320 blocks (D2H) and 320 + 64 (H2D).  From
    32 MiB to 128 MiB it cuts a quarter of its blocks: 192 blocks (96 MiB)
    go as 48 + 144 and 144 + 48.  48 blocks (24 MiB) go as one piece.  Bytes
    match the oracle either way."""
    from flexkv_amd import _lib
    _lib.set_staging_bytes(512 << 20)
    try:
        case = KVCase(layers_total=8, num_layers=8, start_layer=0, kv=2, ng=512, nh=512,
                      tokens=16, heads=8, dim=128).fill(seed=blocks)
        gids = inputs.distinct_ids(5, blocks, 512)
        cids = inputs.distinct_ids(6, blocks, 512)
        _lib.profile_enable(True)
        check_case(case, gids, cids, 1)
        prof = _lib.profile_read()
        _lib.profile_enable(False)
        assert prof["dma_batches"] == 2, prof
        assert prof["kernel_launches"] == 2 * launches, prof   # gathers + scatters
        assert prof["kernel_bytes"] == 2 * blocks * 8 * 2 * 32768, prof
    finally:
        _lib.profile_enable(False)
        _lib.release_staging()
        _lib.set_staging_bytes(0)


@pytest.mark.parametrize("order", ["block-major", "layer-major", "rect"])
def test_copy_engine_small_edge_cut_every_staging_order(dev, order, monkeypatch):
    """With the small edge cut forced on (FLEXKV_CE_EDGE_MIN_BYTES = 1 MiB), a
    transfer of a few MiB splits its first gather (D2H) and its last scatter
    (H2D) into one more piece, in each staging order: contiguous block rows,
    layer-major runs of a layer-wise host cache, and one rect copy per block.
    Bytes as the oracle's both ways, with and without the cut."""
    from flexkv_amd import _lib
    from gpu_util import DeviceCase, abi_transfer
    layout = "BLOCKWISE" if order == "block-major" else "LAYERWISE"
    case = KVCase(layers_total=4, num_layers=4, start_layer=0, kv=2, ng=64, nh=96, tokens=16,
                  heads=4, dim=128, layout=layout).fill(seed=53)      # 16 KiB chunks
    if order == "layer-major":
        cids = np.concatenate([np.arange(8, 24), np.arange(50, 66)])  # 2 runs of 16 blocks
        monkeypatch.setenv("FLEXKV_CE_LAYER_RUN_BYTES", str(4 * 16384))
    else:
        cids = inputs.distinct_ids(12, 32, 96)
        monkeypatch.setenv("FLEXKV_CE_RECT_COPIES", "1")
    cids = np.ascontiguousarray(cids, dtype=np.int64)
    gids = inputs.distinct_ids(13, len(cids), 64)                     # 32 blocks, 4 MiB
    launches = {}
    for cut in (False, True):
        if cut:
            monkeypatch.setenv("FLEXKV_CE_EDGE_MIN_BYTES", str(1 << 20))
        else:
            monkeypatch.delenv("FLEXKV_CE_EDGE_MIN_BYTES", raising=False)
        print(f"edge cut order={order} cut={cut}", flush=True)
        dc = DeviceCase(case)
        _lib.profile_enable(True)
        abi_transfer(dc, gids, cids, h2d=False, mode=1)
        d2h = _lib.profile_read()["kernel_launches"]
        torch.cuda.synchronize()
        assert np.array_equal(dc.host_np(), _oracle_d2h(case, gids, cids, 1)), (order, cut)
        dc.set_gpu([np.zeros_like(g) for g in case.gpu])
        _lib.profile_enable(True)
        abi_transfer(dc, gids, cids, h2d=True, mode=1)
        h2d = _lib.profile_read()["kernel_launches"]
        _lib.profile_enable(False)
        torch.cuda.synchronize()
        for l, g in enumerate(dc.gpu_np()):
            expect = np.zeros_like(case.gpu[l])
            expect[:, gids] = case.gpu[l][:, gids]
            assert np.array_equal(g, expect), (order, cut, l)
        launches[cut] = (d2h, h2d)
    assert launches[True] == (launches[False][0] + 1, launches[False][1] + 1), launches


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("shape", [(1, 1, 32776, 1, 1), (3, 2, 32776, 1, 1),
                                   (1, 1, 128, 8, 16), (1, 1, 256, 16, 16)],
                         ids=["65-rows-1x1", "65-rows-3x2", "32KiB-1x1", "128KiB-1x1"])
def test_small_transfers_split_rows(dev, mode, shape):
    """Transfers with fewer (block, layer) tiles than grid slots split each
    tile's rows over several workgroups.  Chunks of 64 KiB + 16 B (65 rows,
    the last a single vector) put range boundaries inside chunks and partial
    rows at range ends; 32 KiB chunks split in the zero-copy kernels; 128 KiB
    chunks (256 rows per tile) split in the staging kernels too, through the
    whole-group gather in copy-engine mode."""
    n, nl, dim, heads, tokens = shape
    case = KVCase(layers_total=nl, num_layers=nl, start_layer=0, kv=2, ng=8, nh=12,
                  tokens=tokens, heads=heads, dim=dim).fill(seed=n * 10 + nl)
    check_case(case, inputs.distinct_ids(n + 40, n, 8), inputs.distinct_ids(n + 41, n, 12), mode)


SMALL_SHAPES = [
    # (blocks, layers, kv, tokens, heads, dim, layout, tp, rank); chunk = tokens*heads*dim*2 B
    (1, 1, 2, 16, 8, 128, "BLOCKWISE", 1, 0),   # 32 KiB chunks, two 16 KiB pieces each
    (16, 1, 2, 16, 8, 128, "BLOCKWISE", 1, 0),  # 64 pieces: the default grid cap decides
    (3, 2, 1, 1, 1, 8, "BLOCKWISE", 1, 0),      # MLA, 16 B chunks
    (5, 3, 2, 10, 8, 128, "BLOCKWISE", 1, 0),   # 20 KiB chunks: a 16 KiB and a 4 KiB piece
    (2, 1, 1, 64, 1, 576, "BLOCKWISE", 1, 0),   # 72 KiB MLA chunks: five pieces
    (4, 2, 2, 16, 2, 64, "LAYERWISE", 2, 1),    # layer-wise host, TP host chunk of rank 1
]


@pytest.mark.parametrize("small", ["1", "0"], ids=["small-kernel", "general-kernel"])
@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("shape", SMALL_SHAPES, ids=[f"s{i}" for i in range(len(SMALL_SHAPES))])
def test_small_kernel_matches_oracle(dev, monkeypatch, small, mode, shape):
    """Calls of at most 128 pieces of 16 KiB and 4 MiB take the small-transfer
    kernel (per-piece addresses in the kernel arguments); the same calls with
    FLEXKV_SMALL_KERNEL=0 take the general kernel.  Both match the oracle, in
    kernel mode and in copy-engine mode (which sends calls this small to the
    zero-copy kernels), with a start layer, MLA, partial pieces and a TP host
    chunk."""
    monkeypatch.setenv("FLEXKV_SMALL_KERNEL", small)
    n, nl, kv, tokens, heads, dim, layout, tp, rank = shape
    case = KVCase(layers_total=nl + 1, num_layers=nl, start_layer=1, kv=kv, ng=40, nh=48,
                  tokens=tokens, heads=heads, dim=dim, layout=layout, tp=tp,
                  rank=rank).fill(seed=n * 100 + nl * 10 + kv)
    check_case(case, inputs.distinct_ids(n + 70, n, 40), inputs.distinct_ids(n + 71, n, 48), mode)


@pytest.mark.parametrize("cus", [1, 2])
def test_small_kernel_grid_cap(dev, cus):
    """With few compute units allowed, a call whose pieces outnumber the
    workgroups those units hold takes the general kernel; both sides of that
    line match the oracle."""
    for n in (1, 4, 16):
        case = KVCase(layers_total=1, num_layers=1, start_layer=0, kv=2, ng=32, nh=32, tokens=16,
                      heads=8, dim=128).fill(seed=n + cus)
        check_case(case, inputs.distinct_ids(n + 5, n, 32), inputs.distinct_ids(n + 6, n, 32), 0,
                   transfer_cus=cus)


def test_prepare(dev):
    """fkv_prepare sets up staging, engines and signals ahead of the first
    transfer; it can run again, the transfers after it match the oracle, an
    out-of-range device is refused, and staging that cannot be allocated is
    not an error (transfers then fall back to the zero-copy kernel)."""
    from flexkv_amd import _lib
    _lib.release_staging()
    _lib.prepare(-1)
    _lib.prepare(0)
    with pytest.raises(RuntimeError, match="out of range"):
        _lib.prepare(4096)
    case = KVCase(layers_total=4, num_layers=4, start_layer=0, kv=2, ng=300, nh=300, tokens=16,
                  heads=8, dim=128).fill(seed=6)
    gids = inputs.distinct_ids(9, 256, 300)
    cids = inputs.distinct_ids(10, 256, 300)
    try:
        _lib.profile_enable(True)
        check_case(case, gids, cids, 1)
        assert _lib.profile_read()["dma_batches"] == 2
        _lib.release_staging()
        _lib.set_staging_bytes(1 << 40)
        _lib.prepare(0)
    finally:
        _lib.profile_enable(False)
        _lib.set_staging_bytes(0)
        _lib.release_staging()


def test_copy_engine_without_staging_memory(dev):
    """When the staging buffer cannot be allocated (here: asked for 1 TiB, more
    than the device holds), copy-engine transfers move with the zero-copy
    kernel instead of failing, and nothing reaches the engines; with staging
    back to its default the engines carry the same call again."""
    from flexkv_amd import _lib
    case = KVCase(layers_total=4, num_layers=4, start_layer=0, kv=2, ng=300, nh=300, tokens=16,
                  heads=8, dim=128).fill(seed=5)          # 32 KiB chunks, 64 MiB per call
    gids = inputs.distinct_ids(7, 256, 300)
    cids = inputs.distinct_ids(8, 256, 300)
    _lib.release_staging()
    _lib.set_staging_bytes(1 << 40)
    try:
        _lib.profile_enable(True)
        check_case(case, gids, cids, 1)
        prof = _lib.profile_read()
        assert prof["dma_batches"] == 0 and prof["kernel_launches"] >= 2, prof
        _lib.set_staging_bytes(0)
        _lib.profile_enable(True)
        check_case(case, gids, cids, 1)
        prof = _lib.profile_read()
        assert prof["dma_batches"] == 2, prof
    finally:
        _lib.profile_enable(False)
        _lib.set_staging_bytes(0)
        _lib.release_staging()


@pytest.mark.parametrize("mode", MODES)
def test_duplicate_sources_and_single_block(dev, mode):
    case = KVCase(layers_total=2, num_layers=2, start_layer=0, kv=2, ng=8, nh=16, tokens=16,
                  heads=2, dim=64).fill(seed=2)
    gids = np.array([3, 3, 5, 3], dtype=np.int64)
    cids = np.array([0, 9, 4, 15], dtype=np.int64)
    from gpu_util import DeviceCase, abi_transfer
    dc = DeviceCase(case)
    abi_transfer(dc, gids, cids, h2d=False, mode=mode)
    torch.cuda.synchronize()
    assert np.array_equal(dc.host_np(), _oracle_d2h(case, gids, cids, mode))
    check_case(case, gids[:1], cids[:1], mode)


@pytest.mark.parametrize("mode", MODES)
def test_empty_transfer_is_noop(dev, mode):
    case = KVCase(layers_total=2, num_layers=2, start_layer=0, kv=2, ng=8, nh=8, tokens=16,
                  heads=2, dim=64).fill(seed=1)
    from gpu_util import DeviceCase, abi_transfer
    dc = DeviceCase(case)
    empty = np.zeros(0, np.int64)
    abi_transfer(dc, empty, empty, h2d=False, mode=mode)
    abi_transfer(dc, empty, empty, h2d=True, mode=mode)
    torch.cuda.synchronize()
    assert np.array_equal(dc.host_np(), case.host)
    for g, w in zip(dc.gpu_np(), case.gpu):
        assert np.array_equal(g, w)


def test_rejected_arguments_launch_nothing(dev):
    """Bad geometry is refused on the host with RuntimeError; nothing moves."""
    from gpu_util import DeviceCase, abi_transfer
    case = KVCase(layers_total=2, num_layers=2, start_layer=0, kv=2, ng=8, nh=8, tokens=16,
                  heads=2, dim=64).fill(seed=1)
    dc = DeviceCase(case)
    ok = np.array([1, 2], np.int64)
    # Bounds are checked against the allocation holding each pointer (torch
    # may place small tensors inside one larger segment), so use ids far past it.
    far = 1 << 22
    bad_cases = [
        (np.array([1, far], np.int64), ok, {}),          # gpu id past the layer allocation
        (ok, np.array([far, 1], np.int64), {}),          # cpu id past the host cache
        (np.array([-1, 2], np.int64), ok, {}),           # negative id
    ]
    for mode in MODES:
        for g, c, ov in bad_cases:
            with pytest.raises(RuntimeError):
                abi_transfer(dc, g, c, h2d=False, mode=mode, **ov)
    # kernel mode only: copy-engine mode copies such chunks exactly
    with pytest.raises(RuntimeError, match="multiples of 16"):
        abi_transfer(dc, ok, ok, h2d=False, mode=0, chunk=24)
    with pytest.raises(RuntimeError, match="use_ce_transfer"):
        abi_transfer(dc, ok, ok, h2d=False, mode=7)
    with pytest.raises(RuntimeError):
        abi_transfer(dc, ok, ok, h2d=False, mode=0, start_layer=far)  # layer past host cache
    torch.cuda.synchronize()
    assert np.array_equal(dc.host_np(), case.host)


def test_pageable_host_cache_is_refused(dev):
    from flexkv_amd import c_ext
    gpu = torch.zeros(2, 4, 16, 2, 64, dtype=torch.int16, device=dev)
    ptrs = torch.tensor([gpu.data_ptr()], dtype=torch.int64)
    host = torch.zeros(4 * 2 * 16 * 2 * 64, dtype=torch.int16)  # pageable
    ids = torch.tensor([0, 1], dtype=torch.int64)
    with pytest.raises(RuntimeError, match="pinned"):
        c_ext.transfer_kv_blocks(ids, ptrs, gpu[0].numel() * 2, gpu[0, 0].numel() * 2, ids, host,
                                 16 * 2 * 64 * 2, 2 * 16 * 2 * 64 * 2, 2 * 16 * 2 * 64 * 2,
                                 16 * 2 * 64 * 2, 0, -1, False, False, False)


def test_unaligned_chunk_per_chunk_ce_matches_oracle(dev):
    """24-byte chunks: the per-chunk copy-engine loop copies them exactly,
    like the reference CE mode (csrc/transfer.cu:113-117)."""
    case = KVCase(layers_total=2, num_layers=2, start_layer=0, kv=2, ng=10, nh=12, tokens=1,
                  heads=1, dim=12).fill(seed=8)
    check_case(case, inputs.distinct_ids(1, 6, 10), inputs.distinct_ids(2, 6, 12), 2)


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("heads,dim", [(1, 12), (4, 131)])
def test_unaligned_chunk_ce_modes_match_oracle(dev, mode, heads, dim):
    """Chunks of 24 and 1048 bytes (block strides that are not multiples of
    16): both copy-engine modes copy them exactly, as the reference CE mode
    does (csrc/transfer.cu:97-121)."""
    case = KVCase(layers_total=3, num_layers=3, start_layer=0, kv=2, ng=10, nh=12, tokens=1,
                  heads=heads, dim=dim).fill(seed=9)
    assert case.strides()["chunk"] % 16 != 0
    check_case(case, inputs.distinct_ids(3, 7, 10), inputs.distinct_ids(4, 7, 12), mode)


@pytest.mark.parametrize("heads,dim", [(1, 12), (4, 131)])
def test_c_ext_ce_transfer_copies_any_chunk_size(dev, heads, dim):
    """The drop-in call with use_ce_transfer=True on chunks of 24 and 1048
    bytes, both directions, byte for byte against the oracle's CE mode."""
    from flexkv_amd import c_ext
    from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType
    from flexkv_amd.storage.allocator import CPUAllocator
    L, NG, NH, T = 3, 10, 12, 1
    dt = torch.float16
    gl = KVCacheLayout(KVCacheLayoutType.LAYERWISE, L, NG, T, heads, dim)
    cl = KVCacheLayout(KVCacheLayoutType.BLOCKWISE, L, NH, T, heads, dim)
    chunk, gkv, _, gblk = gl.div_layer(L).byte_strides(dt)
    _, ckv, clay, cblk = cl.byte_strides(dt)
    assert chunk in (24, 1048)
    gen = torch.Generator().manual_seed(11)
    src = [torch.randn(gl.kv_shape[1:], generator=gen).to(dt) for _ in range(L)]
    layers = [t.to(dev) for t in src]
    ptrs = torch.tensor([t.data_ptr() for t in layers], dtype=torch.int64).pin_memory()
    cache = CPUAllocator.allocate(cl, dt).get_tensor()
    cache.view(torch.int16).fill_(0x2B2B)
    gids = torch.tensor([7, 0, 9, 4, 2], dtype=torch.int64)
    cids = torch.tensor([11, 3, 0, 6, 8], dtype=torch.int64)
    want = cache.clone()
    oracle.transfer_kv_blocks(gids, src, gkv, gblk, cids, want, ckv, clay, cblk, chunk, 0,
                              False, use_ce_transfer=True)
    c_ext.transfer_kv_blocks(gids.pin_memory(), ptrs, gkv, gblk, cids.pin_memory(), cache, ckv,
                             clay, cblk, chunk, 0, -1, False, True, False)
    assert torch.equal(cache.view(torch.int16), want.view(torch.int16)), "D2H"
    # H2D of altered host blocks into sentinel-filled layers
    cache.view(torch.int16).bitwise_xor_(0x0F0F)
    init = [torch.full_like(t, 0).view(torch.int16).fill_(0x3C3C).view(dt) for t in src]
    back = [t.to(dev) for t in init]
    bptrs = torch.tensor([t.data_ptr() for t in back], dtype=torch.int64).pin_memory()
    c_ext.transfer_kv_blocks(gids.pin_memory(), bptrs, gkv, gblk, cids.pin_memory(), cache, ckv,
                             clay, cblk, chunk, 0, -1, True, True, False)
    want_g = [t.clone() for t in init]
    oracle.transfer_kv_blocks(gids, want_g, gkv, gblk, cids, cache, ckv, clay, cblk, chunk, 0,
                              True, use_ce_transfer=True)
    for l, (g, w) in enumerate(zip(back, want_g)):
        assert torch.equal(g.cpu().view(torch.int16), w.view(torch.int16)), f"H2D layer {l}"


@pytest.mark.parametrize("use_ce", [False, True])
def test_c_ext_dropin_on_side_stream(dev, use_ce, per_call_path):
    """The reference call shape: 15 positional args, pinned id tensors, on the
    current (non-default) stream; through the compiled per-call module and
    through its ctypes stand-in."""
    from flexkv_amd import c_ext
    from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType
    from flexkv_amd.storage.allocator import CPUAllocator
    L, NG, NH = 4, 32, 64
    gl = KVCacheLayout(KVCacheLayoutType.LAYERWISE, L, NG, 16, 8, 128)
    cl = KVCacheLayout(KVCacheLayoutType.BLOCKWISE, L, NH, 16, 8, 128)
    dt = torch.float16
    gen = torch.Generator().manual_seed(5)
    src = [torch.randn(gl.kv_shape[1:], generator=gen, dtype=torch.float32).to(dt) for _ in range(L)]
    layers = [s.to(dev) for s in src]
    cache = CPUAllocator.allocate(cl, dt).get_tensor()
    cache.zero_()
    chunk, gkv, _, gblk = gl.div_layer(L).byte_strides(dt)
    _, ckv, clay, cblk = cl.byte_strides(dt)
    gids = torch.tensor([5, 1, 30, 7], dtype=torch.int64).pin_memory()
    cids = torch.tensor([60, 2, 33, 0], dtype=torch.int64).pin_memory()
    ptrs = torch.tensor([t.data_ptr() for t in layers], dtype=torch.int64).pin_memory()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        c_ext.transfer_kv_blocks(gids, ptrs, gkv, gblk, cids, cache, ckv, clay, cblk, chunk, 0,
                                 8, False, use_ce, False)
    view = cache.view(NH, L, 2, 16, 8, 128)
    for i in range(4):
        for l in range(L):
            assert torch.equal(view[cids[i], l], src[l][:, gids[i]])
    assert torch.count_nonzero(view[torch.tensor([3, 4, 5])]) == 0
    for t in layers:
        t.zero_()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        c_ext.transfer_kv_blocks(gids, ptrs, gkv, gblk, cids, cache, ckv, clay, cblk, chunk, 0,
                                 8, True, use_ce, False)
    torch.cuda.synchronize()
    for l in range(L):
        assert torch.equal(layers[l][:, gids].cpu(), src[l][:, gids])


@pytest.mark.parametrize("use_ce", [False, True])
def test_c_ext_releases_the_gil(dev, use_ce):
    """Another Python thread runs while a transfer is in flight: the call
    releases the GIL for as long as the library works (a 256 MiB transfer,
    about 5 ms at the link's rate), so a thread of the serving engine or a
    second worker is not stalled by it."""
    import threading

    from flexkv_amd import c_ext
    from flexkv_amd.storage.allocator import pinned_empty
    L, NG, chunk = 8, 512, 32768
    layers = [torch.zeros(2 * NG * chunk, dtype=torch.uint8, device=dev) for _ in range(L)]
    host = pinned_empty(NG * L * 2 * chunk, torch.uint8)
    ids = torch.arange(NG, dtype=torch.int64)
    ptrs = torch.tensor([t.data_ptr() for t in layers], dtype=torch.int64)
    count = [0]
    stop = threading.Event()

    def spin():
        while not stop.is_set():
            count[0] += 1

    th = threading.Thread(target=spin)
    th.start()
    try:
        gained = []
        for _ in range(3):
            torch.cuda.synchronize()
            before = count[0]
            c_ext.transfer_kv_blocks(ids, ptrs, NG * chunk, chunk, ids, host, chunk, 2 * chunk,
                                     L * 2 * chunk, chunk, 0, -1, False, use_ce, False)
            gained.append(count[0] - before)
    finally:
        stop.set()
        th.join()
    # with the GIL held for the whole call the other thread could not count at all
    assert max(gained) > 1000, gained


@pytest.mark.parametrize("geo", [(4, 2, 64, 16, 8, 128, 37), (130, 2, 8, 1, 1, 64, 5),
                                 (5, 1, 30, 64, 1, 576, 11), (3, 2, 20, 1, 1, 24, 7),
                                 (3, 1, 24, 32, 1, 1024, 9), (4, 2, 40, 16, 1, 128, 19),
                                 (3, 2, 40, 16, 1, 128, 13), (5, 2, 32, 16, 2, 128, 12),
                                 (3, 2, 32, 16, 4, 128, 9), (4, 1, 30, 16, 6, 128, 7),
                                 (3, 2, 16, 4, 1, 128, 6), (3, 2, 20, 16, 10, 128, 7),
                                 (2, 1, 16, 33, 1, 512, 5), (3, 1, 20, 18, 1, 512, 7),
                                 (2, 2, 16, 12, 1, 512, 5), (3, 1, 16, 9, 1, 512, 5),
                                 (3, 1, 16, 16, 1, 512, 5)],
                         ids=["8b-like", "130-layers", "mla", "48B-chunk", "mla-64KiB",
                              "4KiB-8-chunk-groups", "4KiB-ragged", "8KiB", "16KiB", "24KiB-mla",
                              "1KiB", "40KiB", "33KiB-mla", "18KiB-mla", "12KiB", "9KiB-mla",
                              "16KiB-odd"])
@pytest.mark.parametrize("buffer_on_host", [False, True])
def test_gather_scatter_match_oracle(dev, geo, buffer_on_host):
    """fkv_gather/scatter_kv_blocks against the oracle with the contiguous
    buffer described as a block-wise cache [n, L, kv, chunk] and ids 0..n-1.
    Every packed-row kernel shape is here: 32-row span groups over chunks of
    72, 40 and 33 KiB (two bases), 18 and 16 KiB (three), 12 KiB (four), 9
    and 8 KiB (five), with groups that cross chunk edges and a short last
    group, and, scattering, over 32 / 64 KiB chunks; 24 KiB (24-row groups);
    16 / 8 / 4 KiB chunk counts that fill groups of 2 / 4 / 8 whole chunks;
    the tiled whole-group gather of 32 / 64 KiB chunks; and the row-by-row
    kernel's cases: partial rows (128 B, 48 B), 1 KiB chunks, 4 KiB chunks
    whose count is not a multiple of 8, more layers than one launch holds."""
    import ctypes
    from flexkv_amd import _lib
    from flexkv_amd.storage.allocator import pinned_empty
    from gpu_util import to_torch, to_numpy
    L, kv, ng, t, h, d, n = geo
    case = KVCase(layers_total=L, num_layers=L, start_layer=0, kv=kv, ng=ng, nh=n, tokens=t,
                  heads=h, dim=d).fill(seed=L + n)
    gids = inputs.distinct_ids(n + 9, n, ng)
    local = np.arange(n, dtype=np.int64)
    s = case.strides()
    want = case.host.copy()
    oracle.transfer_kv_blocks(gids, case.gpu, s["gpu_kv"], s["gpu_block"], local, want,
                              s["cpu_kv"], s["cpu_layer"], s["cpu_block"], s["chunk"], 0, False,
                              use_ce_transfer=True, is_mla=kv == 1)
    layers = [to_torch(g).to(dev) for g in case.gpu]
    ptrs = (ctypes.c_void_p * L)(*[x.data_ptr() for x in layers])
    nbytes = want.nbytes
    if buffer_on_host:
        buf = pinned_empty(nbytes // 2, torch.int16)
    else:
        buf = torch.empty(nbytes // 2, dtype=torch.int16, device=dev)
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.fkv_gather_kv_blocks(n, L, gids.ctypes.data, ptrs, s["gpu_kv"], s["gpu_block"],
                                        s["chunk"], buf.data_ptr(), nbytes, st, kv == 1),
               "gather")
    assert np.array_equal(to_numpy(buf, np.uint16).reshape(want.shape), want)
    # too small a buffer is refused
    with pytest.raises(RuntimeError, match="buffer holds"):
        _lib.check(lib.fkv_gather_kv_blocks(n, L, gids.ctypes.data, ptrs, s["gpu_kv"],
                                            s["gpu_block"], s["chunk"], buf.data_ptr(),
                                            nbytes - 16, st, kv == 1), "gather")
    # scatter fresh values back into sentinel-filled layers
    fresh = (want ^ np.uint16(0x0F0F)).reshape(-1)
    buf.copy_(to_torch(fresh))
    init = [np.full_like(g, 0x7777) for g in case.gpu]
    for x, i in zip(layers, init):
        x.copy_(to_torch(i))
    _lib.check(lib.fkv_scatter_kv_blocks(n, L, gids.ctypes.data, ptrs, s["gpu_kv"], s["gpu_block"],
                                         s["chunk"], buf.data_ptr(), nbytes, st, kv == 1),
               "scatter")
    exp = [i.copy() for i in init]
    host_case = KVCase(layers_total=L, num_layers=L, start_layer=0, kv=kv, ng=ng, nh=n, tokens=t,
                       heads=h, dim=d)
    host_case.host = fresh.reshape(want.shape)
    oracle.transfer_kv_blocks(gids, exp, s["gpu_kv"], s["gpu_block"], local, host_case.host,
                              s["cpu_kv"], s["cpu_layer"], s["cpu_block"], s["chunk"], 0, True,
                              use_ce_transfer=True, is_mla=kv == 1)
    for x, e in zip(layers, exp):
        assert np.array_equal(to_numpy(x, np.uint16), e)


from hypothesis import HealthCheck, given, settings, strategies as st  # noqa: E402


def _run_ids(g, n, universe, run):
    """n distinct ids in runs of `run` consecutive ids (the last run may be
    shorter), runs at random non-overlapping starts."""
    slots = g.permutation(universe // run)[: -(-n // run)]
    ids = (slots[:, None] * run + np.arange(run)[None, :]).reshape(-1)[:n]
    return np.ascontiguousarray(ids, dtype=np.int64)


@settings(max_examples=40, deadline=None, derandomize=True,
          suppress_health_check=[HealthCheck.function_scoped_fixture])
@given(layout=st.sampled_from(["BLOCKWISE", "LAYERWISE"]), kv=st.sampled_from([1, 2]),
       lt=st.integers(1, 6), tokens=st.sampled_from([1, 2, 16]), heads=st.sampled_from([1, 3]),
       dim=st.sampled_from([8, 64, 72, 128]), tp=st.sampled_from([1, 2]), mode=st.sampled_from(MODES),
       run=st.sampled_from([1, 3]), layer_major=st.booleans(), seed=st.integers(0, 10**6))
def test_random_geometries_match_oracle(dev, monkeypatch, layout, kv, lt, tokens, heads, dim, tp,
                                        mode, run, layer_major, seed):
    """Seeded random geometries (layouts, MLA, layer windows, TP host chunks,
    chunk sizes from 16 B up, block counts, ids scattered or in runs) in every
    mode, against the oracle; `layer_major` lowers FLEXKV_CE_LAYER_RUN_BYTES
    so that copy-engine transfers of layer-wise caches stage layer-major."""
    if layer_major:
        monkeypatch.setenv("FLEXKV_CE_LAYER_RUN_BYTES", "1")
    else:
        monkeypatch.delenv("FLEXKV_CE_LAYER_RUN_BYTES", raising=False)
    g = np.random.default_rng(seed)
    nl = int(g.integers(1, lt + 1))
    st_l = int(g.integers(0, lt - nl + 1))
    ng, nh = int(g.integers(4 * run, 60)), int(g.integers(4 * run, 60))
    n = int(g.integers(1, min(ng, nh) // run * run + 1))
    case = KVCase(layers_total=lt, num_layers=nl, start_layer=st_l, kv=kv, ng=ng, nh=nh,
                  tokens=tokens, heads=heads, dim=dim, layout=layout, tp=tp,
                  rank=int(g.integers(0, tp))).fill(seed=seed % 9973)
    if run == 1:
        gids = inputs.distinct_ids(seed % 7919 + 1, n, ng)
        cids = inputs.distinct_ids(seed % 7907 + 2, n, nh)
    else:
        gids, cids = _run_ids(g, n, ng, run), _run_ids(g, n, nh, run)
    check_case(case, gids, cids, mode)


@pytest.mark.parametrize("env,fallback", [({"HSA_ENABLE_SDMA": "0"}, None),
                                          ({"FLEXKV_SDMA_ENGINES": "0"}, True)])
def test_copy_engine_mode_without_sdma(dev, env, fallback):
    """Copy-engine mode with the engines unavailable still moves the right
    bytes.  With SDMA disabled in the HSA runtime (HSA_ENABLE_SDMA=0) the
    runtime may still report engines; with the library's engines turned off
    (FLEXKV_SDMA_ENGINES=0) the set-up fails and copy-engine transfers fall
    back to the zero-copy kernel after a one-time warning.  Each case runs in
    a child process, which runs the smoke check (kernel and copy-engine round
    trips against the oracle)."""
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = subprocess.run([sys.executable, "-c", "import __graft_entry__ as g; g.smoke()"],
                         cwd=root, env=dict(os.environ, FLEXKV_CE_MIN_BYTES="0", **env),
                         capture_output=True, text=True, timeout=300)
    print(res.stdout[-2000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0, res.stderr[-2000:]
    assert "match the oracle" in res.stdout
    if fallback:
        assert res.stderr.count("copy engines unavailable") == 1
