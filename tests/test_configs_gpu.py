"""The measured configurations at full size, on the device.

Checks that hold at any size:
  * every moved block, bit for bit, against torch indexing of the source;
  * an oracle spot check: the C oracle run on a sample of the (gpu, cpu) id
    pairs, from host copies of those GPU blocks, must produce the same host
    block rows as the device path;
  * host block rows that no id names keep a sentinel pattern;
  * D2H then H2D into zeroed GPU blocks restores them exactly.
Configurations: Llama-3-8B (32 layers, K/V [4096,16,8,128] bf16, host
[16384,32,2,16,8,128], 1024 random ids; also with a layer-wise host cache
[32,2,16384,16,8,128]); the fragmentation sweep (runs of
1, 8, 64, 1024 ids); the Llama-3-70B TP-8 shard (80 layers, K/V
[8192,16,1,128], 2048 ids); the MLA latent cache (61 layers, [4096,64,576],
host [8192,61,64,576], 32 requests of 1-128 blocks, per request and batched).
"""
import gc

import numpy as np
import pytest
import torch

import oracle
from flexkv_amd import c_ext
from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType
from flexkv_amd.storage.allocator import CPUAllocator

pytestmark = pytest.mark.gpu

SENTINEL = 0x5A5A


class FullCase:
    def __init__(self, layers, kv, ng, nh, tokens, heads, dim, seed, host_layout="BLOCKWISE"):
        self.L, self.kv, self.ng, self.nh = layers, kv, ng, nh
        self.layout = host_layout
        self.dev = torch.device("cuda:0")
        mla = kv == 1
        gl = KVCacheLayout(KVCacheLayoutType.LAYERWISE, layers, ng, tokens, heads, dim, is_mla=mla)
        cl = KVCacheLayout(KVCacheLayoutType[host_layout], layers, nh, tokens, heads, dim,
                           is_mla=mla)
        self.chunk, self.gkv, _, self.gblk = gl.div_layer(layers).byte_strides(torch.bfloat16)
        _, self.ckv, self.clay, self.cblk = cl.byte_strides(torch.bfloat16)
        gen = torch.Generator(device=self.dev).manual_seed(seed)
        self.layers = [torch.empty(tuple(gl.kv_shape[1:]), dtype=torch.bfloat16,
                                   device=self.dev).normal_(generator=gen) for _ in range(layers)]
        self.host = CPUAllocator.allocate(cl, torch.bfloat16).get_tensor()
        self.row = layers * kv * self.chunk // 2            # elements per host block row
        self.ptrs = torch.tensor([t.data_ptr() for t in self.layers], dtype=torch.int64).pin_memory()
        self.mla = mla

    def xfer(self, gids, cids, h2d, ce):
        c_ext.transfer_kv_blocks(gids.pin_memory(), self.ptrs, self.gkv, self.gblk,
                                 cids.pin_memory(), self.host, self.ckv, self.clay, self.cblk,
                                 self.chunk, 0, -1, h2d, ce, self.mla)

    def get_rows(self, cids):
        """Host blocks `cids` as rows [n, layers * kv * chunk] (block-wise order)."""
        if self.layout == "BLOCKWISE":
            return self.host.view(self.nh, self.row)[cids]
        v = self.host.view(self.L, self.kv, self.nh, self.chunk // 2)[:, :, cids]
        return v.permute(2, 0, 1, 3).reshape(len(cids), self.row)

    def fill_rows(self, cids, value):
        if self.layout == "BLOCKWISE":
            self.host.view(self.nh, self.row)[cids] = value
        else:
            self.host.view(self.L, self.kv, self.nh, self.chunk // 2)[:, :, cids] = value

    def packed(self, gids):
        """Selected GPU blocks as host block rows [n, row], by indexing."""
        g = gids.to(self.dev)
        w = torch.stack([t[:, g] for t in self.layers], dim=1)   # [kv, L, n, ...]
        return w.permute(2, 1, 0, *range(3, w.dim())).reshape(len(gids), self.row)

    def check_rows(self, gids, cids, step=128):
        for s in range(0, len(gids), step):
            got = self.get_rows(cids[s:s + step]).to(self.dev)
            want = self.packed(gids[s:s + step])
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), \
                f"host rows differ in id slice {s}..{s + step}"

    def oracle_sample(self, gids, cids, k=12, seed=0):
        pick = torch.randperm(len(gids), generator=torch.Generator().manual_seed(seed))[:k]
        g, c = gids[pick], cids[pick]
        src = [t[:, g.to(self.dev)].cpu().contiguous() for t in self.layers]  # [kv, k, ...]
        small = torch.full((k, self.row), 0, dtype=torch.bfloat16)
        local = np.arange(k, dtype=np.int64)
        # the sample lands in a small block-wise buffer: [k][layer][K|V][chunk]
        oracle.transfer_kv_blocks(local, src, self.gblk * k, self.gblk, local, small, self.chunk,
                                  self.kv * self.chunk, self.row * 2, self.chunk, 0, False,
                                  use_ce_transfer=True, is_mla=self.mla)
        assert torch.equal(self.get_rows(c).view(torch.int16), small.view(torch.int16)), \
            "device path differs from the oracle on the sampled ids"

    def free(self):
        del self.layers, self.host
        gc.collect()
        torch.cuda.empty_cache()


def _untouched(nh, cids, count=64, seed=0):
    mask = torch.ones(nh, dtype=torch.bool)
    mask[cids] = False
    free = mask.nonzero().flatten()
    return free[torch.randperm(len(free), generator=torch.Generator().manual_seed(seed))[:count]]


def _round_trip(case, gids, cids, ce):
    print(f"round trip n={len(gids)} ce={ce}", flush=True)
    quiet = _untouched(case.nh, cids)
    case.fill_rows(quiet, torch.tensor(SENTINEL, dtype=torch.int16).view(torch.bfloat16))
    case.xfer(gids, cids, False, ce)
    case.check_rows(gids, cids)
    case.oracle_sample(gids, cids)
    assert torch.all(case.get_rows(quiet).view(torch.int16) == SENTINEL), "untouched rows changed"
    keep = case.packed(gids).clone()
    g = gids.to(case.dev)
    for t in case.layers:
        t[:, g] = 0
    torch.cuda.synchronize()
    case.xfer(gids, cids, True, ce)
    assert torch.equal(case.packed(gids).view(torch.int16), keep.view(torch.int16)), \
        "H2D did not restore the GPU blocks"


@pytest.fixture(scope="class")
def llama8b():
    # class scope: the 32 GiB pinned cache is freed before the other
    # configurations allocate theirs (pinned memory is limited per process)
    c = FullCase(32, 2, 4096, 16384, 16, 8, 128, seed=1001)
    yield c
    c.free()


class TestLlama3_8B:
    @pytest.mark.parametrize("ce", [False, True])
    def test_random_ids(self, llama8b, ce):
        g = torch.Generator().manual_seed(1002)
        gids = torch.randperm(4096, generator=g)[:1024]
        cids = torch.randperm(16384, generator=g)[:1024]
        _round_trip(llama8b, gids, cids, ce)

    @pytest.mark.parametrize("run", [1, 8, 64, 1024])
    @pytest.mark.parametrize("ce", [False, True])
    def test_fragmentation_sweep(self, llama8b, run, ce):
        g = torch.Generator().manual_seed(2000 + run)

        def runs(universe):
            slots = torch.randperm(universe // run, generator=g)[: 1024 // run]
            return (slots[:, None] * run + torch.arange(run)[None, :]).reshape(-1)

        _round_trip(llama8b, runs(4096), runs(16384), ce)


@pytest.mark.parametrize("run", [1, 8, 1024])
@pytest.mark.parametrize("ce", [False, True])
def test_llama3_8b_layerwise_host(ce, run):
    """1024 ids in runs of `run` consecutive blocks against a layer-wise host
    cache [32,2,16384,16,8,128] (the reference's default layout): the
    zero-copy kernel, and copy-engine mode (one SDMA rect copy per block for
    scattered ids, layer-major staging and one copy per (layer, K|V) run for
    runs of 8 and more)."""
    case = FullCase(32, 2, 4096, 16384, 16, 8, 128, seed=1003, host_layout="LAYERWISE")
    try:
        g = torch.Generator().manual_seed(1004 + run)

        def runs(universe):
            slots = torch.randperm(universe // run, generator=g)[: 1024 // run]
            return (slots[:, None] * run + torch.arange(run)[None, :]).reshape(-1)

        _round_trip(case, runs(4096), runs(16384), ce)
    finally:
        case.free()


def test_llama3_70b_tp8_shard():
    case = FullCase(80, 2, 8192, 16384, 16, 1, 128, seed=1003)
    try:
        g = torch.Generator().manual_seed(1004)
        gids = torch.randperm(8192, generator=g)[:2048]
        cids = torch.randperm(16384, generator=g)[:2048]
        for ce in (False, True):
            _round_trip(case, gids, cids, ce)
    finally:
        case.free()


def test_mla_latent_requests():
    """32 requests of U{1..128} blocks with distinct random ids, moved one
    call per request and as one batched call, both directions."""
    case = FullCase(61, 1, 4096, 8192, 64, 1, 576, seed=1005)
    try:
        g = torch.Generator().manual_seed(1006)
        sizes = torch.randint(1, 129, (32,), generator=g)
        total = int(sizes.sum())
        gids = torch.randperm(4096, generator=g)[:total]
        cids = torch.randperm(8192, generator=g)[:total]
        bounds = [0] + torch.cumsum(sizes, 0).tolist()
        for ce in (False, True):
            for i in range(32):
                case.xfer(gids[bounds[i]:bounds[i + 1]], cids[bounds[i]:bounds[i + 1]], False, ce)
            case.check_rows(gids, cids)
            case.oracle_sample(gids, cids)
            _round_trip(case, gids, cids, ce)
    finally:
        case.free()
