"""Pins for the CPU oracle (oracle/kv_oracle.c).

The reference ships no golden vectors for this path (its only check is the
GPU->CPU->GPU round trip, tests/test_transfer_engine.py:55-161), so the oracle
is pinned by:
  * element-by-element brute force on tiny shapes;
  * numpy fancy indexing on shaped arrays whose byte strides come from numpy;
  * the round trip and untouched-block invariants the reference relies on;
  * kernel mode == copy-engine mode, and the kernel's 16-byte tail rule
    (csrc/transfer.cu:35) where they differ;
  * a contiguous run reducing to one memcpy of a block-wise region;
  * committed fixtures (tests/golden/), and planted mistakes that each of the
    checks above must catch.
"""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle
from oracle import inputs
from kvcase import KVCase, brute_force_d2h

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def run_d2h(case, gids, cids, host=None, **kw):
    s = case.strides()
    host = case.host.copy() if host is None else host
    args = dict(cpu_startoff_inside_chunks=s["startoff"])
    args.update(kw)
    oracle.transfer_kv_blocks(gids, case.gpu, s["gpu_kv"], s["gpu_block"], cids, host,
                              s["cpu_kv"], s["cpu_layer"], s["cpu_block"], s["chunk"],
                              case.start_layer, False, is_mla=(case.kv == 1), **args)
    return host


def run_h2d(case, gids, cids, gpu=None, **kw):
    s = case.strides()
    gpu = [np.zeros_like(g) for g in case.gpu] if gpu is None else gpu
    args = dict(cpu_startoff_inside_chunks=s["startoff"])
    args.update(kw)
    oracle.transfer_kv_blocks(gids, gpu, s["gpu_kv"], s["gpu_block"], cids, case.host,
                              s["cpu_kv"], s["cpu_layer"], s["cpu_block"], s["chunk"],
                              case.start_layer, True, is_mla=(case.kv == 1), **args)
    return gpu


TINY = [
    dict(layers_total=3, num_layers=2, start_layer=1, kv=2, ng=5, nh=7, tokens=2, heads=2, dim=4),
    dict(layers_total=3, num_layers=3, start_layer=0, kv=1, ng=4, nh=6, tokens=2, heads=1, dim=8),
    dict(layers_total=2, num_layers=2, start_layer=0, kv=2, ng=4, nh=5, tokens=1, heads=2, dim=8,
         tp=2, rank=1),
]


@pytest.mark.parametrize("layout", ["BLOCKWISE", "LAYERWISE"])
@pytest.mark.parametrize("shape", TINY)
def test_brute_force_tiny(shape, layout):
    case = KVCase(layout=layout, **shape).fill(seed=3)
    gids = np.array([3, 0, 2], dtype=np.int64)
    cids = np.array([1, 4, 3], dtype=np.int64)
    want = brute_force_d2h(case, gids, cids)
    for ce in (False, True):
        got = run_d2h(case, gids, cids, use_ce_transfer=ce)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("layout", ["BLOCKWISE", "LAYERWISE"])
@pytest.mark.parametrize("mla", [False, True])
@pytest.mark.parametrize("dtype", [np.uint16, np.uint32])
def test_indexing_medium(layout, mla, dtype):
    case = KVCase(layers_total=6, num_layers=4, start_layer=2, kv=1 if mla else 2, ng=40, nh=64,
                  tokens=4, heads=2, dim=16, dtype=dtype, layout=layout).fill(seed=11)
    gids = inputs.distinct_ids(5, 17, case.ng)
    cids = inputs.distinct_ids(6, 17, case.nh)
    assert np.array_equal(run_d2h(case, gids, cids), case.expect_d2h(gids, cids))
    case.host = case.expect_d2h(gids, cids)
    init = [np.zeros_like(g) for g in case.gpu]
    got = run_h2d(case, gids, cids, [g.copy() for g in init])
    want = case.expect_h2d(gids, cids, init)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)


def test_round_trip_and_untouched_blocks():
    case = KVCase(layers_total=4, num_layers=4, start_layer=0, kv=2, ng=32, nh=48, tokens=4,
                  heads=2, dim=8).fill(seed=21)
    gids = inputs.distinct_ids(1, 12, case.ng)
    cids = inputs.distinct_ids(2, 12, case.nh)
    host = run_d2h(case, gids, cids)
    sel = np.zeros(case.nh, bool)
    sel[cids] = True
    assert np.all(host[~sel] == 0x5A5A), "blocks outside cpu_ids were written"
    case.host = host
    back = run_h2d(case, gids, cids)
    gsel = np.zeros(case.ng, bool)
    gsel[gids] = True
    for l in range(case.num_layers):
        assert np.array_equal(back[l][:, gsel], case.gpu[l][:, gsel])
        assert np.all(back[l][:, ~gsel] == 0)


def test_kernel_mode_drops_tail_below_16_bytes():
    # chunk = 1*1*12 uint16 = 24 bytes: the reference kernel copies one float4
    # (16 bytes) per chunk, the copy engine all 24.
    case = KVCase(layers_total=2, num_layers=2, start_layer=0, kv=2, ng=4, nh=4, tokens=1,
                  heads=1, dim=12).fill(seed=4)
    gids = np.array([2, 0], dtype=np.int64)
    cids = np.array([1, 3], dtype=np.int64)
    full = case.expect_d2h(gids, cids)
    ce = run_d2h(case, gids, cids, use_ce_transfer=True)
    assert np.array_equal(ce, full)
    kern = run_d2h(case, gids, cids, use_ce_transfer=False)
    hv, fv = case.host_view(kern), case.host_view(full)
    assert np.array_equal(hv[..., :8], fv[..., :8])
    assert np.all(hv[..., 8:] == 0x5A5A)


def test_contiguous_run_is_one_memcpy():
    case = KVCase(layers_total=3, num_layers=3, start_layer=0, kv=2, ng=16, nh=16, tokens=2,
                  heads=2, dim=8).fill(seed=9)
    n, c0 = 5, 7
    gids = np.arange(4, 4 + n, dtype=np.int64)
    cids = np.arange(c0, c0 + n, dtype=np.int64)
    host = run_d2h(case, gids, cids)
    row = host[0].nbytes
    flat = host.reshape(-1).view(np.uint8)
    # the selected GPU bytes in block -> layer -> kv order, as one contiguous buffer
    src = np.stack([np.stack([case.gpu[l][k, 4:4 + n] for k in range(2)], axis=1)
                    for l in range(3)], axis=1)
    assert np.array_equal(flat[c0 * row:(c0 + n) * row], src.reshape(-1).view(np.uint8))


def test_threads_match_sequential():
    case = KVCase(layers_total=4, num_layers=4, start_layer=0, kv=2, ng=64, nh=64, tokens=4,
                  heads=2, dim=16).fill(seed=13)
    gids = inputs.distinct_ids(3, 50, case.ng)
    cids = inputs.distinct_ids(4, 50, case.nh)
    one = run_d2h(case, gids, cids, num_threads=1)
    for t in (2, 3, 8, 64):
        assert np.array_equal(run_d2h(case, gids, cids, num_threads=t), one)


def test_empty_and_rejected_arguments():
    case = KVCase(layers_total=2, num_layers=2, start_layer=0, kv=2, ng=4, nh=4, tokens=1,
                  heads=1, dim=8).fill(seed=1)
    empty = np.zeros(0, dtype=np.int64)
    assert np.array_equal(run_d2h(case, empty, empty), case.host)
    with pytest.raises(ValueError):
        run_d2h(case, np.array([1], np.int64), np.array([1, 2], np.int64))
    with pytest.raises(ValueError):
        run_d2h(case, np.array([1], np.int64), np.array([1], np.int64), num_threads=0)


# ---- planted mistakes: each pin above must catch a plausible oracle bug ----

def test_planted_mistakes_are_caught():
    case = KVCase(layers_total=3, num_layers=2, start_layer=1, kv=2, ng=6, nh=8, tokens=2,
                  heads=2, dim=4, tp=2, rank=1).fill(seed=5)
    gids = np.array([5, 1, 3], dtype=np.int64)
    cids = np.array([2, 7, 0], dtype=np.int64)
    want = brute_force_d2h(case, gids, cids)
    s = case.strides()
    assert np.array_equal(run_d2h(case, gids, cids), want)
    # transposed operands: kv and layer strides swapped
    bad = case.host.copy()
    oracle.transfer_kv_blocks(gids, case.gpu, s["gpu_kv"], s["gpu_block"], cids, bad,
                              s["cpu_layer"], s["cpu_kv"], s["cpu_block"], s["chunk"],
                              case.start_layer, False, cpu_startoff_inside_chunks=s["startoff"])
    assert not np.array_equal(bad, want)
    # wrong index: gpu and cpu ids exchanged
    assert not np.array_equal(run_d2h(case, cids % case.ng, gids), want)
    # dropped term: start layer ignored
    bad = case.host.copy()
    oracle.transfer_kv_blocks(gids, case.gpu, s["gpu_kv"], s["gpu_block"], cids, bad,
                              s["cpu_kv"], s["cpu_layer"], s["cpu_block"], s["chunk"], 0, False,
                              cpu_startoff_inside_chunks=s["startoff"])
    assert not np.array_equal(bad, want)
    # dropped term: tensor-parallel start offset ignored
    assert not np.array_equal(run_d2h(case, gids, cids, cpu_startoff_inside_chunks=0), want)


# ---- committed fixtures --------------------------------------------------

def _load_tiny_fixture():
    path = os.path.join(GOLDEN, "tiny_vectors.npz")
    return np.load(path, allow_pickle=False)


def test_tiny_fixture_vectors():
    fx = _load_tiny_fixture()
    meta = json.loads(str(fx["meta"]))
    for i, m in enumerate(meta):
        case = KVCase(**m["shape"])
        case.gpu = [fx[f"c{i}_gpu{l}"] for l in range(case.num_layers)]
        case.host = fx[f"c{i}_host"]
        gids, cids = fx[f"c{i}_gids"], fx[f"c{i}_cids"]
        assert np.array_equal(run_d2h(case, gids, cids), fx[f"c{i}_want_host"]), m
        case.host = fx[f"c{i}_want_host"]
        back = run_h2d(case, gids, cids)
        for l in range(case.num_layers):
            assert np.array_equal(back[l], fx[f"c{i}_want_gpu{l}"]), m


def test_config0_digests():
    """Config 0 (4 layers, fp16 K/V [256,16,8,128] -> host [512,4,2,16,8,128],
    64 random distinct ids) reproduces the committed SHA-256 digests."""
    from golden.gen_golden import config0_case, config0_ids
    with open(os.path.join(GOLDEN, "config0_digests.json")) as fh:
        want = json.load(fh)
    case = config0_case()
    gids, cids = config0_ids()
    host = run_d2h(case, gids, cids)
    assert np.array_equal(host, case.expect_d2h(gids, cids))
    assert hashlib.sha256(host.tobytes()).hexdigest() == want["d2h_host_sha256"]
    case.host = host
    back = run_h2d(case, gids, cids)
    assert hashlib.sha256(b"".join(g.tobytes() for g in back)).hexdigest() == \
        want["h2d_gpu_sha256"]


def _tp_case(tp, layout, mla, seed, L=4, ng=6, nh=9, tokens=2, hpr=1, dim=4):
    """Tiny tensor-parallel case: rank r's per-layer caches [kv, ng, chunk]
    (uint16), a host cache whose chunk holds the tp ranks' chunks side by
    side ([tp][chunk], one chunk under MLA), and its byte strides."""
    rng = np.random.default_rng(seed)
    kv = 1 if mla else 2
    ce = tokens * hpr * dim
    width = 1 if mla else tp
    ranks = [[rng.integers(0, 65535, size=(kv, ng, ce), dtype=np.uint16) for _ in range(L)]
             for _ in range(tp)]
    if layout == "BLOCKWISE":
        host = np.zeros((nh, L, kv, width, ce), np.uint16)
        view = host
        cblk, clay, ckv = L * kv * width * ce * 2, kv * width * ce * 2, width * ce * 2
    else:
        host = np.zeros((L, kv, nh, width, ce), np.uint16)
        view = host.transpose(2, 0, 1, 3, 4)          # [nh, L, kv, width, ce]
        cblk, clay, ckv = width * ce * 2, kv * nh * width * ce * 2, nh * width * ce * 2
    strides = dict(gpu_kv_stride_in_bytes=ng * ce * 2, gpu_block_stride_in_bytes=ce * 2,
                   gpu_chunk_size_in_bytes=ce * 2, cpu_kv_stride_in_bytes=ckv,
                   cpu_layer_stride_in_bytes=clay, cpu_block_stride_in_bytes=cblk)
    return ranks, host, view, strides


@pytest.mark.parametrize("layout", ["BLOCKWISE", "LAYERWISE"])
@pytest.mark.parametrize("tp,mla", [(2, False), (3, False), (4, True)])
def test_tp_group_oracle_against_indexing(layout, tp, mla):
    """oracle.tp_group_transfer pinned by numpy indexing: after a D2H of a
    layer window, host chunk slot r of block cids[i], layer l, half k holds
    rank r's chunk gids[i] of that layer and half (under MLA, rank 0's in the
    one slot); every other host byte stays zero.  After an H2D into zeroed
    rank caches, each rank holds its slot (under MLA, every rank the one
    slot) in the window's layers and nothing else.  A planted mistake (every
    rank at offset 0) breaks the D2H check."""
    ranks, host, view, st = _tp_case(tp, layout, mla, seed=tp * 7 + mla)
    gids = np.array([4, 0, 5], np.int64)
    cids = np.array([2, 8, 5], np.int64)
    lid, gran = 1, 2
    oracle.tp_group_transfer(ranks, gids, st["gpu_kv_stride_in_bytes"],
                             st["gpu_block_stride_in_bytes"], st["gpu_chunk_size_in_bytes"],
                             cids, host, st["cpu_kv_stride_in_bytes"],
                             st["cpu_layer_stride_in_bytes"], st["cpu_block_stride_in_bytes"],
                             False, lid, gran, mla)
    want = np.zeros_like(view)
    for r in range(1 if mla else tp):
        for l in range(lid, lid + gran):
            want[cids, l, :, r] = ranks[r][l][:, gids].transpose(1, 0, 2)
    assert np.array_equal(view, want)
    # planted: every rank at offset 0
    bad = np.zeros_like(host)
    for r, layers in enumerate(ranks):
        oracle.transfer_kv_blocks(gids, layers[lid:lid + gran], st["gpu_kv_stride_in_bytes"],
                                  st["gpu_block_stride_in_bytes"], cids, bad,
                                  st["cpu_kv_stride_in_bytes"], st["cpu_layer_stride_in_bytes"],
                                  st["cpu_block_stride_in_bytes"], st["gpu_chunk_size_in_bytes"],
                                  lid, False, True, mla)
    bad_view = bad if layout == "BLOCKWISE" else bad.transpose(2, 0, 1, 3, 4)
    if not mla:
        assert not np.array_equal(bad_view, want)
    # H2D from a filled host cache into zeroed rank caches
    rng = np.random.default_rng(5)
    host[...] = rng.integers(0, 65535, size=host.shape, dtype=np.uint16)
    dst = [[np.zeros_like(a) for a in layers] for layers in ranks]
    oracle.tp_group_transfer(dst, gids, st["gpu_kv_stride_in_bytes"],
                             st["gpu_block_stride_in_bytes"], st["gpu_chunk_size_in_bytes"],
                             cids, host, st["cpu_kv_stride_in_bytes"],
                             st["cpu_layer_stride_in_bytes"], st["cpu_block_stride_in_bytes"],
                             True, lid, gran, mla)
    for r in range(tp):
        slot = 0 if mla else r
        for l in range(len(ranks[r])):
            exp = np.zeros_like(ranks[r][l])
            if lid <= l < lid + gran:
                exp[:, gids] = view[cids, l, :, slot].transpose(1, 0, 2)
            assert np.array_equal(dst[r][l], exp), (r, l)
