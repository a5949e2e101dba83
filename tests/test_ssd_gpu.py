"""The host cache <-> SSD tier on the GPU box, checked byte for byte.

Blocks move GPU -> host on the product path (copy engines), host -> SSD files
and back through CPUSSDDiskTransferWorker, then host -> GPU.  The host cache
is pinned (fkv_host_alloc), so O_DIRECT reads go through the library's bounce
buffers, as they do in service.  Every hop is compared with the oracle:
oracle.transfer_kv_blocks for the device hops and oracle.transfer_kv_blocks_ssd
(csrc/transfer_ssd.cpp:17-32,120-179 restated) over in-memory images of the
files for the SSD hops.  SSD ids and host ids are distinct random
permutations, so swapped id lists or a file offset that is wrong the same way
in both directions fail.
"""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import DeviceCase, abi_transfer
from kvcase import KVCase
from test_ssd_cpu import ENGINES, URING, _file_images, _oracle_mirror, _rng_bytes
from flexkv_amd import _lib
from flexkv_amd.common.config import CacheConfig
from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType
from flexkv_amd.common.transfer import TransferType
from flexkv_amd.storage.allocator import SSDAllocator
from flexkv_amd.transfer.worker import CPUSSDDiskTransferWorker

pytestmark = pytest.mark.gpu

GEOMS = [
    # (layout, mla, ssd devices, max blocks per file, layers, host blocks, ssd blocks,
    #  tokens, heads, dim): Llama-3-8B chunks (32 KiB) and MLA latent chunks (72 KiB)
    ("BLOCKWISE", False, 2, 20, 8, 48, 80, 16, 8, 128),
    ("LAYERWISE", False, 2, 20, 8, 48, 80, 16, 8, 128),
    ("BLOCKWISE", True, 1, 13, 6, 40, 60, 64, 1, 576),
    ("LAYERWISE", True, 3, 9, 6, 40, 60, 64, 1, 576),
]


@pytest.mark.parametrize("engine", ["threads", "uring64"])
@pytest.mark.parametrize("geom", GEOMS, ids=lambda g: f"{g[0]}-mla{int(g[1])}-d{g[2]}-f{g[3]}")
def test_gpu_host_ssd_chain_matches_oracle(tmp_path, geom, engine):
    if ENGINES[engine] and not URING:
        pytest.skip("this kernel refuses io_uring rings")
    layout, mla, n_dev, mbpf, L, nh, n_ssd, T, H, Dh = geom
    kv = 1 if mla else 2
    case = KVCase(layers_total=L, num_layers=L, start_layer=0, kv=kv, ng=64, nh=nh, tokens=T,
                  heads=H, dim=Dh, layout=layout).fill(seed=L * 7 + n_dev)
    s = case.strides()
    dc = DeviceCase(case)                       # pinned host cache from fkv_host_alloc
    g = np.random.default_rng(L * 100 + nh)
    n = 24
    gids = g.permutation(case.ng)[:n].astype(np.int64)
    cids = g.permutation(nh)[:n].astype(np.int64)
    sids = g.permutation(n_ssd)[:n].astype(np.int64)
    dst = g.permutation(nh)[:n].astype(np.int64)
    print(f"ssd chain {layout} mla={mla} engine={engine}", flush=True)

    # 1. GPU -> host on the copy-engine path
    abi_transfer(dc, gids, cids, False, _lib.FKV_XFER_CE)
    want_host = case.host.copy()
    oracle.transfer_kv_blocks(gids, case.gpu, s["gpu_kv"], s["gpu_block"], cids, want_host,
                              s["cpu_kv"], s["cpu_layer"], s["cpu_block"], s["chunk"], 0, False,
                              is_mla=mla)
    assert np.array_equal(dc.host_np(), want_host)

    # 2. host -> SSD files, against the oracle over images of the files
    lt = KVCacheLayoutType[layout]
    cpu_lay = KVCacheLayout(lt, L, nh, T, H, Dh, is_mla=mla)
    ssd_lay = KVCacheLayout(lt, L, n_ssd, T, H, Dh, is_mla=mla)
    dirs = [str(tmp_path / f"dev{d}") for d in range(n_dev)]
    sh = SSDAllocator.allocate(ssd_lay, torch.bfloat16, cache_dir=dirs, max_blocks_per_file=mbpf)
    files = sh.get_file_list()
    used = ssd_lay.div_block(sum(len(v) for v in files.values()), padding=True) \
        .get_total_elements() * 2
    for d, paths in files.items():
        for j, p in enumerate(paths):
            with open(p, "r+b") as f:
                f.write(_rng_bytes(used, 500 + 10 * d + j).tobytes())
    cfg = CacheConfig(ssd_threads_per_device=4, ssd_cache_iouring_entries=ENGINES[engine])
    w = CPUSSDDiskTransferWorker(0, None, None, dc.host, files, cpu_lay, ssd_lay, torch.bfloat16,
                                 sh.num_blocks_per_file, cfg)
    c = dict(worker=w, n_dev=n_dev, F=len(files[0]))
    host_bytes = dc.host.numpy().view(np.uint8)
    try:
        images = _file_images(files, used)
        _oracle_mirror(c, images, host_bytes.copy(), sids, cids, 0, L, is_read=False)
        w._transfer_impl(cids, sids, TransferType.H2DISK, 0, L)
        after = _file_images(files, used)
        for i, (a, b) in enumerate(zip(after, images)):
            assert np.array_equal(a, b), f"file image {i}"

        # 3. SSD -> zeroed host cache, into other host blocks
        dc.host.zero_()
        expect = np.zeros_like(host_bytes)
        _oracle_mirror(c, after, expect, sids, dst, 0, L, is_read=True)
        w._transfer_impl(sids, dst, TransferType.DISK2H, 0, L)
        assert np.array_equal(host_bytes, expect)
        if w.chunk_size_in_bytes % 4096 == 0:
            st = w.ioctx.stats()
            assert st["direct_read_bytes"] > 0, st   # the O_DIRECT bounce path ran
    finally:
        w.close()

    # 4. host -> zeroed GPU blocks; they hold the original blocks again
    for t in dc.gpu:
        t.index_fill_(1, torch.from_numpy(gids).cuda(), 0)
    abi_transfer(dc, gids, dst, True, _lib.FKV_XFER_CE)
    for l, t in enumerate(dc.gpu):
        got = t.cpu().numpy().view(case.dtype)
        assert np.array_equal(got[:, gids], case.gpu[l][:, gids]), f"layer {l}"
