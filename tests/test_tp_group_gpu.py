"""Tensor-parallel transfer groups on one GPU: every rank's cache sits on
cuda:0, so the group's fan-out (a thread and a stream per rank, rank r at
byte offset r * chunk of each host chunk) runs as it would across GPUs, with
the ranks sharing one link.  Bytes are compared with oracle.tp_group_transfer
(the reference's per-rank calls, csrc/tp_transfer_thread_group.cpp:66-99)
over the whole host cache and every rank's whole cache; the engine tests are
the reference's TP round trips (tests/test_transfer_engine.py:55-161)."""
import time

import numpy as np
import pytest
import torch

import oracle
from gpu_util import pinned_empty, zero_blocks
from oracle import inputs
from flexkv_amd import c_ext
from flexkv_amd.cache.transfer_pattern import (create_read_graph_cpu_storage,
                                               create_write_graph_cpu_storage)
from flexkv_amd.common.config import CacheConfig, ModelConfig
from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType
from flexkv_amd.common.transfer import DeviceType
from flexkv_amd.storage.storage_engine import StorageEngine
from flexkv_amd.transfer.transfer_engine import TransferEngine

pytestmark = pytest.mark.gpu


class TpCase:
    """`tp` ranks of L layers, each layer [kv, ng, tokens, hpr, dim] fp16 on
    cuda:0 (rank r's head slice), and a pinned host cache whose chunk holds
    the ranks' chunks side by side (one chunk under MLA)."""

    def __init__(self, tp, layout, mla, L=6, ng=40, nh=64, tokens=16, hpr=2, dim=64, seed=0,
                 misaligned=()):
        self.tp, self.layout, self.mla, self.L = tp, layout, mla, L
        self.kv = 1 if mla else 2
        self.ce = tokens * hpr * dim
        width = 1 if mla else tp
        self.width = width
        rng = np.random.default_rng(seed)
        self.np_ranks = [[rng.integers(0, 65535, size=(self.kv, ng, self.ce), dtype=np.uint16)
                          for _ in range(L)] for r in range(tp)]

        def on_gpu(a, r):
            t = torch.from_numpy(a.view(np.float16)).reshape(self.kv, ng, tokens, hpr, dim)
            if r not in misaligned:
                return t.cuda()
            # 8 bytes into an allocation: not the 16-byte alignment kernels need
            buf = torch.empty(t.numel() + 4, dtype=torch.float16, device="cuda")
            v = buf[4:].view(t.shape)
            v.copy_(t)
            return v
        self.ranks = [[on_gpu(a, r) for a in layers] for r, layers in enumerate(self.np_ranks)]
        n = nh * L * self.kv * width * self.ce
        self.host = pinned_empty(n, torch.float16)
        self.host.zero_()
        es = 2
        if layout == "BLOCKWISE":
            self.shape = (nh, L, self.kv, width, self.ce)
            cblk, clay, ckv = L * self.kv * width * self.ce * es, self.kv * width * self.ce * es, \
                width * self.ce * es
        else:
            self.shape = (L, self.kv, nh, width, self.ce)
            cblk, clay, ckv = width * self.ce * es, self.kv * nh * width * self.ce * es, \
                nh * width * self.ce * es
        self.gpu_kv = ng * self.ce * es
        self.gpu_blk = self.ce * es
        self.chunk = self.ce * es
        self.ckv, self.clay, self.cblk = ckv, clay, cblk
        self.nh, self.ng = nh, ng

    def host_np(self):
        return self.host.view(torch.int16).numpy().view(np.uint16).copy()

    def set_host(self, arr):
        self.host.view(torch.int16).copy_(torch.from_numpy(arr.view(np.int16)))

    def group(self):
        return c_ext.TPTransferThreadGroup(self.tp, self.ranks, self.host, 0)

    def move(self, grp, gids, cids, h2d, ce, layer_id=0, gran=None, cus=-1):
        grp.tp_group_transfer(torch.from_numpy(gids), self.gpu_kv, self.gpu_blk, self.chunk,
                              torch.from_numpy(cids), self.ckv, self.clay, self.cblk,
                              self.width * self.chunk, cus, h2d, ce, layer_id,
                              gran or self.L, self.mla)
        torch.cuda.synchronize()

    def oracle(self, np_ranks, host, gids, cids, h2d, layer_id=0, gran=None):
        oracle.tp_group_transfer(np_ranks, gids, self.gpu_kv, self.gpu_blk, self.chunk, cids,
                                 host, self.ckv, self.clay, self.cblk, h2d, layer_id,
                                 gran or self.L, self.mla)


@pytest.mark.parametrize("layout", ["BLOCKWISE", "LAYERWISE"])
@pytest.mark.parametrize("tp,mla", [(2, False), (4, False), (8, False), (4, True)])
@pytest.mark.parametrize("ce", [False, True])
@pytest.mark.parametrize("window", [(0, None), (2, 3)])
def test_tp_group_matches_oracle(layout, tp, mla, ce, window):
    """D2H of a layer window into a zeroed host cache, then H2D of a fresh
    host cache into sentinel-filled rank caches: the whole host cache and
    every rank's every layer against the oracle.  The (2, 3) window is where
    the reference's rank pointer offset (r * layer_granularity) would read
    another rank's layers."""
    print(f"tp={tp} mla={mla} layout={layout} ce={ce} window={window}", flush=True)
    case = TpCase(tp, layout, mla, seed=tp * 11 + mla)
    gids = inputs.distinct_ids(tp + 1, 24, case.ng)
    cids = inputs.distinct_ids(tp + 2, 24, case.nh)
    lid, gran = window
    grp = case.group()
    try:
        case.move(grp, gids, cids, False, ce, lid, gran)
        want = np.zeros(case.shape, np.uint16)
        case.oracle([[a.copy() for a in r] for r in case.np_ranks], want, gids, cids, False,
                    lid, gran)
        assert np.array_equal(case.host_np().reshape(case.shape), want), "D2H"
        fresh = np.random.default_rng(3).integers(0, 65535, size=case.shape, dtype=np.uint16)
        case.set_host(fresh.reshape(-1))
        for layers in case.ranks:
            for t in layers:
                t.view(torch.int16).fill_(0x2323)
        torch.cuda.synchronize()
        case.move(grp, gids, cids, True, ce, lid, gran)
        exp = [[np.full(a.shape, 0x2323, np.uint16) for a in r] for r in case.np_ranks]
        case.oracle(exp, fresh.copy(), gids, cids, True, lid, gran)
        for r in range(tp):
            for l in range(case.L):
                got = case.ranks[r][l].cpu().view(torch.int16).numpy().view(np.uint16)
                assert np.array_equal(got.reshape(exp[r][l].shape), exp[r][l]), ("H2D", r, l)
    finally:
        grp.close()


def test_tp_group_error_names_the_rank():
    """Rank 1's layers start 8 bytes into their allocations: a zero-copy
    kernel transfer refuses them on the host, so the group's D2H raises
    naming rank 1 while rank 0's slots still land as the oracle's and rank
    1's stay untouched.  Copy-engine mode takes any alignment (the per-chunk
    engine loop), so the same D2H then moves both ranks.  After close() the
    group refuses to run."""
    case = TpCase(2, "BLOCKWISE", False, seed=5, misaligned=(1,))
    gids = inputs.distinct_ids(41, 12, case.ng)
    cids = inputs.distinct_ids(42, 12, case.nh)
    grp = case.group()
    try:
        with pytest.raises(RuntimeError, match="tp_group_transfer failed: TP rank 1"):
            case.move(grp, gids, cids, False, False)
        want = np.zeros(case.shape, np.uint16)
        case.oracle([[a.copy() for a in case.np_ranks[0]], [np.zeros_like(a) for a in
                                                             case.np_ranks[1]]],
                    want, gids, cids, False)
        want[:, :, :, 1] = 0
        assert np.array_equal(case.host_np().reshape(case.shape), want)
        case.move(grp, gids, cids, False, True)
        want = np.zeros(case.shape, np.uint16)
        case.oracle([[a.copy() for a in r] for r in case.np_ranks], want, gids, cids, False)
        assert np.array_equal(case.host_np().reshape(case.shape), want)
    finally:
        grp.close()
    with pytest.raises(RuntimeError, match="closed"):
        case.move(grp, gids, cids, False, False)


def test_close_from_another_thread_waits_for_the_transfer():
    """close() from a second thread while the first keeps transferring:
    every transfer that starts finishes whole (the group is freed only
    between transfers), the ones after close() raise, and the last D2H's host
    bytes match the oracle."""
    import threading

    case = TpCase(4, "BLOCKWISE", False, seed=9)
    gids = inputs.distinct_ids(41, 24, case.ng)
    cids = inputs.distinct_ids(42, 24, case.nh)
    grp = case.group()
    done, refused, errors = [], [], []

    def mover():
        for _ in range(200):
            try:
                case.move(grp, gids, cids, False, False)
                done.append(1)
            except RuntimeError as e:
                (refused if "closed" in str(e) else errors).append(str(e))
                return

    t = threading.Thread(target=mover)
    t.start()
    while not done:
        time.sleep(0.001)
    grp.close()
    t.join(timeout=60)
    assert not t.is_alive() and not errors, errors
    assert done and len(done) + len(refused) <= 200
    want = np.zeros(case.shape, np.uint16)
    case.oracle([[a.copy() for a in r] for r in case.np_ranks], want, gids, cids, False)
    assert np.array_equal(case.host_np().reshape(case.shape), want)
    with pytest.raises(RuntimeError, match="closed"):
        case.move(grp, gids, cids, False, False)


def test_two_groups_at_once():
    """Two data-parallel groups' transfers from two host threads at once,
    each group's ranks on their own host blocks (as dp groups own disjoint
    host blocks): both host caches match the oracle."""
    import threading
    cases = [TpCase(2, "BLOCKWISE", False, seed=s) for s in (21, 22)]
    groups = [c.group() for c in cases]
    gids = inputs.distinct_ids(31, 32, 40)
    cids = inputs.distinct_ids(32, 32, 64)
    errors = []

    def run(i):
        try:
            for ce in (False, True, False):
                cases[i].move(groups[i], gids, cids, False, ce)
        except Exception as e:   # surfaced below
            errors.append(e)
    try:
        th = [threading.Thread(target=run, args=(i,)) for i in range(2)]
        for t in th:
            t.start()
        for t in th:
            t.join()
        assert not errors, errors
        for c in cases:
            want = np.zeros(c.shape, np.uint16)
            c.oracle([[a.copy() for a in r] for r in c.np_ranks], want, gids, cids, False)
            assert np.array_equal(c.host_np().reshape(c.shape), want)
    finally:
        for g in groups:
            g.close()


# the engine round trips (tests/test_transfer_engine.py:55-161, TP/DP cases)
MODEL = dict(num_layers=4, num_kv_heads=32, head_size=128, dtype=torch.float16)
CACHE = dict(tokens_per_block=16, num_cpu_blocks=128, use_ce_transfer_h2d=False,
             use_ce_transfer_d2h=True, transfer_sms_h2d=4, transfer_sms_d2h=4)


def _wait(engine, gid, limit=120.0):
    t0 = time.time()
    seen = []
    while time.time() - t0 < limit:
        seen += engine.get_completed_graphs_and_ops(timeout=0.1)
        if (gid, -1) in seen:
            return
    raise AssertionError(f"graph {gid} did not complete")


@pytest.mark.parametrize("tp,dp,mode", [(2, 1, "thread"), (2, 2, "thread"), (4, 1, "thread"),
                                         (2, 1, "process")])
@pytest.mark.parametrize("use_mla", [False, True])
@pytest.mark.parametrize("layout", [KVCacheLayoutType.LAYERWISE, KVCacheLayoutType.BLOCKWISE])
def test_engine_tp_round_trip(tp, dp, mode, use_mla, layout):
    """GPU -> CPU -> GPU through StorageEngine + TransferEngine with tp ranks
    per data-parallel group, every rank's cache on cuda:0: each rank holds
    num_kv_heads / tp heads (all heads under MLA), dp group i writes host
    blocks [16 i, 16 i + 16), the rank caches are zeroed in place, and the
    read graph restores every rank's every layer.  In process mode the TP
    worker is a spawned process fed IPC handles of the rank caches, with a
    host cache of its own."""
    mc = ModelConfig(use_mla=use_mla, tp_size=tp, dp_size=dp, **MODEL)
    cc = CacheConfig(cpu_kv_layout_type=layout, **CACHE)
    heads = mc.num_kv_heads if use_mla else mc.num_kv_heads // tp
    gl = KVCacheLayout(KVCacheLayoutType.LAYERWISE, mc.num_layers, 64, cc.tokens_per_block,
                       heads, mc.head_size, is_mla=use_mla)
    gen = torch.Generator().manual_seed(tp * 10 + dp)
    se = StorageEngine(mc, cc)
    gts, gpus = [], []
    for j in range(tp * dp):
        # under MLA the ranks of a group hold the same latent
        src = j - j % tp if use_mla else j
        if src == j:
            gt = [torch.randn(tuple(gl.kv_shape[1:]), generator=gen).to(mc.dtype)
                  for _ in range(mc.num_layers)]
        else:
            gt = gts[src]
        gts.append(gt)
        gpu = [t.cuda() for t in gt]
        gpus.append(gpu)
        se.register_gpu_blocks(gpu, gl, device_id=j, dtype=mc.dtype)
    te = TransferEngine([se.get_storage_handle(DeviceType.GPU, j) for j in range(tp * dp)],
                        mc, cc, cpu_handle=se.get_storage_handle(DeviceType.CPU),
                        worker_mode=mode)
    te.start()
    try:
        for i in range(dp):
            gids = torch.arange(0, 16, dtype=torch.int64)
            cids = torch.arange(16 * i, 16 * i + 16, dtype=torch.int64)
            wg, _ = create_write_graph_cpu_storage(gids, cids,
                                                   torch.tensor([], dtype=torch.int64),
                                                   gpu_device_id=i * tp, layer_num=mc.num_layers)
            wg.bind_to_dp_group(i)
            te.submit_transfer_graph(wg)
            _wait(te, wg.graph_id)
            for j in range(i * tp, (i + 1) * tp):
                for t in gpus[j]:
                    zero_blocks(t, gids)
            torch.cuda.synchronize()
            rg, _ = create_read_graph_cpu_storage(gids, cids,
                                                  torch.tensor([], dtype=torch.int64),
                                                  gpu_device_id=i * tp, layer_num=mc.num_layers)
            rg.bind_to_dp_group(i)
            te.submit_transfer_graph(rg)
            _wait(te, rg.graph_id)
            for j in range(i * tp, (i + 1) * tp):
                for l in range(mc.num_layers):
                    assert torch.equal(gpus[j][l].cpu(), gts[j][l]), (i, j, l)
    finally:
        te.shutdown()
