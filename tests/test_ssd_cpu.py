"""The host cache <-> SSD tier, without a device.

The oracle (oracle_transfer_kv_blocks_ssd, restating
csrc/transfer_ssd.cpp:17-179) is pinned first by facts that do not restate
its formula: with one device and one file the SSD file is the host cache's
block array indexed by SSD id; the block -> (device, file, in-file block)
mapping is a bijection that stripes consecutive ids over devices, then files;
a per-file layer-wise file is the array [layers, K|V, blocks_per_file, chunk].
Then the product (fkv_transfer_kv_blocks_ssd through c_ext and
CPUSSDDiskTransferWorker, files made by SSDAllocator) is compared with the
oracle byte for byte, on both host layouts, MLA, layer windows, several
devices and files, O_DIRECT-sized and unaligned chunks, and the
reference's worker geometry (worker.py:482-602)."""
import os
import time

import numpy as np
import pytest
import torch

import oracle
from flexkv_amd import c_ext
from flexkv_amd.common.config import CacheConfig, ModelConfig
from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType
from flexkv_amd.common.transfer import (DeviceType, TransferDescriptor, TransferOp,
                                        TransferOpGraph, TransferType)
from flexkv_amd.storage.allocator import SSDAllocator
from flexkv_amd.transfer.worker import CPUSSDDiskTransferWorker

LW, BW = KVCacheLayoutType.LAYERWISE, KVCacheLayoutType.BLOCKWISE


def _uring_available():
    """Whether this kernel gives an unprivileged process an io_uring ring."""
    import ctypes
    import platform
    if platform.machine() != "x86_64":
        return False
    libc = ctypes.CDLL(None, use_errno=True)
    params = (ctypes.c_uint32 * 30)()          # struct io_uring_params is 120 bytes
    fd = libc.syscall(425, 4, ctypes.byref(params))   # __NR_io_uring_setup
    if fd < 0:
        return False
    os.close(fd)
    return True


URING = _uring_available()


def _rng_bytes(n, seed):
    return np.random.default_rng(seed).integers(0, 256, size=n, dtype=np.uint8)


def _mapping(b, rr, D, F):
    """Reference mapping in plain words: ids are cut into runs of rr; run r
    goes to device r % D as that device's run r // D; a device block x goes
    to file x % F at in-file slot x // F."""
    run, pos = divmod(b, rr)
    dev = run % D
    x = (run // D) * rr + pos
    return dev, x % F, x // F


# ---------------------------------------------------------------- oracle pins

def _oracle_roundtrip_case(layout_type, D, F, rr, mla, seed, start=0, nl=None):
    L, N_cpu, tpb, H, Dh = 3, 12, 2, 2, 8       # chunk = 2*2*8*2 = 64 bytes (fp16)
    es = 2
    n_ssd = D * F * 4
    cpu = KVCacheLayout(layout_type, L, N_cpu, tpb, H, Dh, is_mla=mla)
    ssd = KVCacheLayout(layout_type, L, n_ssd, tpb, H, Dh, is_mla=mla)
    per_file = ssd.div_block(D * F, padding=True)
    file_bytes = per_file.get_total_elements() * es
    files = [np.zeros(file_bytes, np.uint8) for _ in range(D * F)]
    host = _rng_bytes(cpu.get_total_elements() * es, seed)
    nl = L - start if nl is None else nl
    return dict(L=L, N_cpu=N_cpu, n_ssd=n_ssd, cpu=cpu, ssd=ssd, per_file=per_file, es=es,
                files=files, host=host, start=start, nl=nl, D=D, F=F, rr=rr, mla=mla)


def _oracle_call(c, host, sids, cids, is_read):
    es = c["es"]
    oracle.transfer_kv_blocks_ssd(
        c["files"], c["D"], c["F"], c["start"], c["nl"], host, sids, cids,
        c["cpu"].get_layer_stride() * es, c["cpu"].get_kv_stride() * es,
        c["per_file"].get_layer_stride() * es, c["per_file"].get_kv_stride() * es,
        c["cpu"].get_chunk_size() * es, c["cpu"].get_block_stride() * es, is_read,
        round_robin=c["rr"], is_mla=c["mla"])


def test_oracle_single_file_blockwise_is_block_array():
    c = _oracle_roundtrip_case(BW, 1, 1, 1, False, 1)
    sids = np.array([3, 0, 2], np.int64)
    cids = np.array([5, 11, 0], np.int64)
    _oracle_call(c, c["host"], sids, cids, is_read=False)
    blk = c["cpu"].get_elements_per_block() * c["es"]
    f = c["files"][0][:c["n_ssd"] * blk].reshape(c["n_ssd"], blk)
    h = c["host"].reshape(c["N_cpu"], blk)
    for s, ci in zip(sids, cids):
        assert np.array_equal(f[s], h[ci])
    untouched = [b for b in range(c["n_ssd"]) if b not in sids]
    assert not f[untouched].any()


@pytest.mark.parametrize("mla", [False, True])
def test_oracle_layerwise_file_is_layer_kv_block_array(mla):
    D, F = 2, 2
    c = _oracle_roundtrip_case(LW, D, F, 1, mla, 2)
    kv = 1 if mla else 2
    chunk = c["cpu"].get_chunk_size() * c["es"]
    nbf = c["per_file"].num_block
    sids = np.arange(c["n_ssd"], dtype=np.int64)[::-1].copy()
    cids = np.arange(c["n_ssd"], dtype=np.int64) % c["N_cpu"]
    sids, cids = sids[:c["N_cpu"]], cids[:c["N_cpu"]]
    _oracle_call(c, c["host"], sids, cids, is_read=False)
    h = c["host"].reshape(c["L"], kv, c["N_cpu"], chunk)
    for s, ci in zip(sids, cids):
        dev, fi, slot = _mapping(int(s), 1, D, F)
        f = c["files"][dev * F + fi].reshape(c["L"], kv, nbf, chunk)
        assert np.array_equal(f[:, :, slot], h[:, :, ci])


@pytest.mark.parametrize("D,F,rr", [(1, 1, 1), (2, 1, 1), (2, 3, 1), (3, 2, 2), (2, 2, 4)])
def test_oracle_mapping_is_a_striping_bijection(D, F, rr):
    """Every SSD id lands in a distinct (device, file, slot); ids stripe over
    devices in runs of rr, then over files; each file holds the first
    n/(D*F) slots.  Checked on the oracle's files by tagging each block."""
    c = _oracle_roundtrip_case(BW, D, F, rr, True, 3)
    n = c["n_ssd"]
    blk = c["cpu"].get_elements_per_block() * c["es"]
    L, kv = c["L"], 1
    # host block i is filled with the byte i+1 so that file slots name their id
    host = np.repeat(np.arange(1, n + 1, dtype=np.uint8), blk)
    c["cpu"] = KVCacheLayout(BW, L, n, 2, 2, 8, is_mla=True)
    _oracle_call(c, host, np.arange(n, dtype=np.int64), np.arange(n, dtype=np.int64), False)
    seen = {}
    for f_idx, img in enumerate(c["files"]):
        slots = img.reshape(-1, blk)
        for slot in range(slots.shape[0]):
            tag = int(slots[slot, 0])
            if tag:
                assert (slots[slot] == tag).all()
                seen[tag - 1] = (f_idx // F, f_idx % F, slot)
    assert sorted(seen) == list(range(n))
    assert len(set(seen.values())) == n
    for b in range(n):                       # stripe order
        dev = seen[b][0]
        assert dev == (b // rr) % D
    per_dev = [sorted(b for b in seen if seen[b][0] == d) for d in range(D)]
    assert all(len(p) == n // D for p in per_dev)
    for d in range(D):                       # device-local order walks files, then slots
        locs = [(seen[b][2], seen[b][1]) for b in per_dev[d]]
        assert locs == sorted(locs)


def _layerwise_view_ok(c, sids, cids):
    """The layer-wise pin: file (dev, file) slot `slot` of each written block
    holds the block's [layer][K|V] chunks, with the mapping of _mapping()."""
    kv = 1 if c["mla"] else 2
    chunk = c["cpu"].get_chunk_size() * c["es"]
    nbf = c["per_file"].num_block
    h = c["host"].reshape(c["L"], kv, c["N_cpu"], chunk)
    for sb, ci in zip(sids, cids):
        dev, fi, slot = _mapping(int(sb), 1, c["D"], c["F"])
        f = c["files"][dev * c["F"] + fi].reshape(c["L"], kv, nbf, chunk)
        if not np.array_equal(f[:, :, slot], h[:, :, ci]):
            return False
    return True


def test_oracle_planted_mistakes_are_caught():
    """Each plausible mistake, planted by calling the oracle with a wrong
    argument, breaks the layer-wise file view that pins the SSD oracle:
    layer and K|V strides transposed, a round-robin width other than the
    worker's, MLA taken for K/V, a dropped start layer."""
    def run(**wrong):
        c = _oracle_roundtrip_case(LW, 2, 2, 1, False, 6)
        sids = np.array([0, 5, 6, 11, 14, 3], np.int64)
        cids = np.array([2, 9, 4, 0, 7, 11], np.int64)
        es = c["es"]
        args = dict(cpu_layer=c["cpu"].get_layer_stride() * es,
                    cpu_kv=c["cpu"].get_kv_stride() * es,
                    ssd_layer=c["per_file"].get_layer_stride() * es,
                    ssd_kv=c["per_file"].get_kv_stride() * es, rr=1, mla=False, start=0)
        args.update(wrong)
        oracle.transfer_kv_blocks_ssd(
            c["files"], c["D"], c["F"], args["start"], c["L"] - args["start"], c["host"], sids,
            cids, args["cpu_layer"], args["cpu_kv"], args["ssd_layer"], args["ssd_kv"],
            c["cpu"].get_chunk_size() * es, c["cpu"].get_block_stride() * es, False,
            round_robin=args["rr"], is_mla=args["mla"])
        return _layerwise_view_ok(c, sids, cids)

    assert run()
    c0 = _oracle_roundtrip_case(LW, 2, 2, 1, False, 6)
    es = c0["es"]
    lay, kvs = c0["cpu"].get_layer_stride() * es, c0["cpu"].get_kv_stride() * es
    slay, skv = c0["per_file"].get_layer_stride() * es, c0["per_file"].get_kv_stride() * es
    assert not run(cpu_layer=kvs, cpu_kv=lay)            # transposed host strides
    assert not run(ssd_layer=skv, ssd_kv=slay)           # transposed file strides
    assert not run(rr=2)                                 # wrong round-robin width
    assert not run(mla=True)                             # V half dropped
    assert not run(start=1)                              # layer 0 skipped


@pytest.mark.parametrize("layout_type", [LW, BW])
@pytest.mark.parametrize("mla", [False, True])
def test_oracle_write_read_round_trip(layout_type, mla):
    c = _oracle_roundtrip_case(layout_type, 2, 2, 1, mla, 4, start=1, nl=2)
    g = np.random.default_rng(5)
    sids = g.permutation(c["n_ssd"])[:7].astype(np.int64)
    cids = g.permutation(c["N_cpu"])[:7].astype(np.int64)
    _oracle_call(c, c["host"], sids, cids, is_read=False)
    back = np.zeros_like(c["host"])
    dst = np.roll(cids, 3)
    _oracle_call(c, back, sids, dst, is_read=True)
    es = c["es"]
    kv = 1 if mla else 2
    chunk = c["cpu"].get_chunk_size() * es
    lay = c["cpu"]
    for s, a, b in zip(sids, cids, dst):
        for l in range(c["start"], c["start"] + c["nl"]):
            for k in range(kv):
                oa = a * lay.get_block_stride() * es + l * lay.get_layer_stride() * es + \
                    k * lay.get_kv_stride() * es
                ob = b * lay.get_block_stride() * es + l * lay.get_layer_stride() * es + \
                    k * lay.get_kv_stride() * es
                assert np.array_equal(back[ob:ob + chunk], c["host"][oa:oa + chunk])


# ----------------------------------------------------------- product vs oracle

ENGINES = {"threads": 0, "uring64": 64, "uring2": 2}


def _product_case(tmp_path, layout_type, mla, n_dev, max_blocks_per_file, tpb, H, Dh,
                  L=4, N_cpu=40, n_ssd=48, dtype=torch.float16, seed=0, engine="threads",
                  iouring_flags=0):
    dirs = [str(tmp_path / f"dev{d}") for d in range(n_dev)]
    cpu_lay = KVCacheLayout(layout_type, L, N_cpu, tpb, H, Dh, is_mla=mla)
    ssd_lay = KVCacheLayout(layout_type, L, n_ssd, tpb, H, Dh, is_mla=mla)
    h = SSDAllocator.allocate(ssd_lay, dtype, cache_dir=dirs,
                              max_blocks_per_file=max_blocks_per_file)
    files = h.get_file_list()
    es = dtype.itemsize
    # page-aligned host cache, as a pinned allocation would be
    nbytes = cpu_lay.get_total_elements() * es
    raw = np.zeros(nbytes + 4096, np.uint8)
    off = (-raw.ctypes.data) % 4096
    host = raw[off:off + nbytes]
    host[:] = _rng_bytes(nbytes, seed)
    # non-zero prior contents over the part of each file the per-file layout
    # addresses, so that untouched bytes are checked too (with no per-file
    # block limit a file is a sparse one as large as the free space)
    used = ssd_lay.div_block(sum(len(v) for v in files.values()), padding=True) \
        .get_total_elements() * es
    for d, paths in files.items():
        for j, p in enumerate(paths):
            with open(p, "r+b") as f:
                f.write(_rng_bytes(min(used, os.path.getsize(p)), 1000 + 10 * d + j).tobytes())
    cfg = CacheConfig(ssd_threads_per_device=4, ssd_cache_iouring_entries=ENGINES[engine],
                      ssd_cache_iouring_flags=iouring_flags)
    worker = CPUSSDDiskTransferWorker(0, None, None, torch.from_numpy(host), files, cpu_lay,
                                      ssd_lay, dtype, h.num_blocks_per_file, cfg)
    if ENGINES[engine] and iouring_flags == 0 and URING:
        # the ring this test asked for is the one that carries the transfers
        assert worker.ioctx.iouring_depth >= ENGINES[engine]
    return dict(host=host, files=files, worker=worker, cpu=cpu_lay, ssd=ssd_lay, es=es,
                n_dev=n_dev, F=len(files[0]), raw=raw, used=used)


def _file_images(files, nbytes=None):
    return [np.fromfile(p, dtype=np.uint8, count=-1 if nbytes is None else nbytes)
            for d in sorted(files) for p in files[d]]


def _oracle_mirror(c, images, host, sids, cids, start, nl, is_read):
    w = c["worker"]
    oracle.transfer_kv_blocks_ssd(
        images, c["n_dev"], c["F"], start, nl, host, sids, cids, w.cpu_layer_stride_in_bytes,
        w.cpu_kv_stride_in_bytes, w.ssd_layer_stride_in_bytes, w.ssd_kv_stride_in_bytes,
        w.chunk_size_in_bytes, w.block_stride_in_bytes, is_read, round_robin=1,
        is_mla=w.is_mla)


GEOMS = [
    # (layout, mla, devices, max_blocks_per_file, tpb, heads, head_dim)
    (BW, False, 2, -1, 16, 2, 64),     # chunk 4096: O_DIRECT-sized reads, one file per device
    (LW, False, 2, -1, 16, 2, 64),
    (BW, True, 1, 10, 4, 1, 72),       # chunk 576, 5 files
    (LW, True, 3, 7, 4, 1, 72),        # 3 devices x 3 files, padded per-file layout
    (LW, False, 2, 5, 3, 2, 40),       # chunk 480, 5 files per device
    (BW, False, 3, 6, 16, 4, 64),      # chunk 8192, 3 devices x 3 files
]


@pytest.mark.parametrize("geom", GEOMS, ids=lambda g: f"{g[0].name}-mla{int(g[1])}-d{g[2]}"
                         f"-f{g[3]}-{g[4]}x{g[5]}x{g[6]}")
@pytest.mark.parametrize("window", [(0, -1), (1, 2)], ids=["all", "l1+2"])
@pytest.mark.parametrize("engine", list(ENGINES))
def test_product_matches_oracle(tmp_path, geom, window, engine):
    layout, mla, n_dev, mbpf, tpb, H, Dh = geom
    c = _product_case(tmp_path, layout, mla, n_dev, mbpf, tpb, H, Dh, seed=hash(geom) & 0xffff,
                      engine=engine)
    start, nl = window
    nl = c["cpu"].num_layer if nl == -1 else nl
    g = np.random.default_rng(11)
    n = 17
    sids = g.permutation(c["ssd"].num_block)[:n].astype(np.int64)
    cids = g.permutation(c["cpu"].num_block)[:n].astype(np.int64)
    # write: host -> files
    images = _file_images(c["files"], c["used"])
    _oracle_mirror(c, images, c["host"], sids, cids, start, nl, is_read=False)
    c["worker"]._transfer_impl(cids, sids, TransferType.H2DISK, start, nl)
    after = _file_images(c["files"], c["used"])
    for a, b in zip(after, images):
        assert np.array_equal(a, b)
    # read: files -> another set of host blocks
    dst = g.permutation(c["cpu"].num_block)[:n].astype(np.int64)
    expect = c["host"].copy()
    _oracle_mirror(c, after, expect, sids, dst, start, nl, is_read=True)
    c["worker"]._transfer_impl(sids, dst, TransferType.DISK2H, start, nl)
    assert np.array_equal(c["host"], expect)
    c["worker"].close()


@pytest.mark.parametrize("geom", GEOMS, ids=lambda g: f"{g[0].name}-mla{int(g[1])}-d{g[2]}"
                         f"-f{g[3]}-{g[4]}x{g[5]}x{g[6]}")
@pytest.mark.parametrize("engine,max_request", [("threads", None), ("uring64", None),
                                                ("threads", 4096), ("uring2", 8192)])
def test_contiguous_runs_match_oracle(tmp_path, monkeypatch, geom, engine, max_request):
    """Runs of consecutive SSD and host ids, where neighbouring chunks merge
    into single requests: two runs plus a stray block, written then read.
    With a small FLEXKV_SSD_MAX_REQUEST_BYTES the merged runs (and chunks
    larger than the cap) are cut into several requests."""
    if max_request:
        monkeypatch.setenv("FLEXKV_SSD_MAX_REQUEST_BYTES", str(max_request))
    layout, mla, n_dev, mbpf, tpb, H, Dh = geom
    c = _product_case(tmp_path, layout, mla, n_dev, mbpf, tpb, H, Dh, seed=7, engine=engine)
    sids = np.concatenate([np.arange(3, 19), np.arange(30, 41), [1]]).astype(np.int64)
    cids = np.concatenate([np.arange(10, 26), np.arange(27, 38), [39]]).astype(np.int64)
    for start, nl in ((0, c["cpu"].num_layer), (1, 2)):
        images = _file_images(c["files"], c["used"])
        _oracle_mirror(c, images, c["host"], sids, cids, start, nl, is_read=False)
        c["worker"]._transfer_impl(cids, sids, TransferType.H2DISK, start, nl)
        assert all(np.array_equal(a, b) for a, b in zip(_file_images(c["files"], c["used"]),
                                                        images))
        dst = np.roll(cids, 5)
        expect = c["host"].copy()
        _oracle_mirror(c, images, expect, sids, dst, start, nl, is_read=True)
        c["worker"]._transfer_impl(sids, dst, TransferType.DISK2H, start, nl)
        assert np.array_equal(c["host"], expect)
    c["worker"].close()


def test_reference_worker_geometry(tmp_path):
    """The reference test's SSD setup (tests/test_utils.py:15-53): two
    devices, 512 SSD blocks, LAYERWISE, 16 tokens x head_size 128 fp16, 4
    layers, with 8 heads instead of 32 to keep the files small here (the GPU
    engine test runs the full size); written, then read back."""
    c = _product_case(tmp_path, LW, False, 2, 32000, 16, 8, 128, L=4, N_cpu=64, n_ssd=512)
    w = c["worker"]
    chunk = 16 * 8 * 128 * 2
    assert w.chunk_size_in_bytes == chunk
    assert w.ssd_kv_stride_in_bytes == 256 * chunk          # 512 blocks over 2 files
    assert w.ssd_layer_stride_in_bytes == 2 * 256 * chunk
    assert w.block_stride_in_bytes == chunk                 # LAYERWISE host block stride
    sids = np.arange(0, 16, dtype=np.int64)
    cids = np.arange(0, 16, dtype=np.int64)
    images = _file_images(c["files"], c["used"])
    _oracle_mirror(c, images, c["host"], sids, cids, 0, 4, False)
    w._transfer_impl(cids, sids, TransferType.H2DISK, 0, 4)
    assert all(np.array_equal(a, b) for a, b in zip(_file_images(c["files"], c["used"]), images))
    ref = c["host"].copy()
    c["host"][:] = 0
    w._transfer_impl(sids, cids, TransferType.DISK2H, 0, 4)
    # LAYERWISE host: blocks 0..15 of every layer and K/V restored, others zero
    h = c["host"].reshape(4, 2, 64, -1)
    r = ref.reshape(4, 2, 64, -1)
    assert np.array_equal(h[:, :, :16], r[:, :, :16]) and not h[:, :, 16:].any()
    w.close()


@pytest.mark.parametrize("engine", ["threads", "uring64"])
def test_unaligned_host_buffer_reads_exact(tmp_path, engine):
    """Direct reads land in page-aligned bounce buffers, so a host cache that
    is not page aligned reads the same bytes."""
    c = _product_case(tmp_path, BW, False, 1, -1, 16, 2, 64, engine=engine)
    w = c["worker"]
    sids = np.array([1, 2, 3], np.int64)
    cids = np.array([4, 5, 6], np.int64)
    w._transfer_impl(cids, sids, TransferType.H2DISK, 0, 4)
    # a host view shifted by 16 bytes: chunk addresses are no longer 4 KiB aligned
    shifted = c["raw"][16:16 + c["host"].size]
    shifted[:] = 0
    ioctx = w.ioctx
    c_ext.transfer_kv_blocks_ssd(
        ioctx, torch.arange(0, 4, dtype=torch.int32), shifted.ctypes.data,
        torch.from_numpy(sids), torch.from_numpy(cids), w.cpu_layer_stride_in_bytes,
        w.cpu_kv_stride_in_bytes, w.ssd_layer_stride_in_bytes, w.ssd_kv_stride_in_bytes,
        w.chunk_size_in_bytes, w.block_stride_in_bytes, True, w.num_blocks_per_file)
    blk = w.block_stride_in_bytes
    got = shifted.reshape(-1, blk)
    images = _file_images(c["files"], c["used"])
    f = images[0].reshape(-1, blk)
    for s, ci in zip(sids, cids):
        assert np.array_equal(got[ci], f[s])
    w.close()


# ------------------------------------------------------------ io_uring engine

def test_iouring_depth_reported(tmp_path):
    """iouring_entries = 0 keeps threads; a ring the kernel grants reports its
    depth (setup rounds entries up to a power of two)."""
    p = tmp_path / "f.bin"
    p.write_bytes(b"\0" * 8192)
    assert c_ext.SSDIOCTX({0: [str(p)]}, 1).iouring_depth == 0
    ctx = c_ext.SSDIOCTX({0: [str(p)]}, 1, iouring_entries=24)
    if URING:
        assert ctx.iouring_depth == 32
    else:
        assert ctx.iouring_depth == 0
    with pytest.raises(ValueError):
        c_ext.SSDIOCTX({0: [str(p)]}, 1, iouring_entries=-1)


def _o_direct_supported(path):
    try:
        fd = os.open(path, os.O_RDONLY | os.O_DIRECT)
    except OSError:
        return False
    os.close(fd)
    return True


@pytest.mark.parametrize("engine", ["threads", "uring64", "uring2"])
def test_stats_count_direct_reads(tmp_path, engine):
    """Page-multiple chunks are read with O_DIRECT (through the bounce
    buffers) wherever the file system allows it, with no page-cache retries;
    the counters account for every byte moved."""
    c = _product_case(tmp_path, BW, False, 2, -1, 16, 2, 64, engine=engine)
    w = c["worker"]
    # SSD ids 2, 4, 6 are consecutive slots of device 0's file (two devices,
    # round robin 1) and go to consecutive host blocks: one request each way
    # on the ring; the threads engine gives each of those blocks a thread of
    # its own (4 threads per device), one request each
    per_op = 2 if engine != "threads" and URING else 4
    sids = np.array([2, 4, 6, 3], np.int64)
    cids = np.array([10, 11, 12, 0], np.int64)
    w._transfer_impl(cids, sids, TransferType.H2DISK, 0, 4)
    moved = len(sids) * w.block_stride_in_bytes
    st = w.ioctx.stats()
    assert st["write_bytes"] == moved and st["fallbacks"] == 0
    assert st["requests"] == per_op
    w._transfer_impl(sids, cids + 13, TransferType.DISK2H, 0, 4)
    st = w.ioctx.stats()
    if _o_direct_supported(c["files"][0][0]):
        assert st["direct_read_bytes"] == moved and st["buffered_read_bytes"] == 0
    else:
        assert st["buffered_read_bytes"] == moved
    assert st["fallbacks"] == 0 and st["requests"] == 2 * per_op
    if engine != "threads" and URING:
        assert st["ring_entries"] >= st["requests"]
    w.close()


def test_iouring_refused_ring_falls_back_to_threads(tmp_path, capfd):
    """A ring the kernel refuses (here: an undefined setup flag) leaves the
    context on threads, with a warning, and transfers stay exact."""
    c = _product_case(tmp_path, BW, False, 2, -1, 16, 2, 64, engine="uring64",
                      iouring_flags=1 << 30)
    assert c["worker"].ioctx.iouring_depth == 0
    assert "io_uring setup" in capfd.readouterr().err
    sids = np.array([5, 0, 9, 2], np.int64)
    cids = np.array([1, 7, 3, 30], np.int64)
    images = _file_images(c["files"], c["used"])
    _oracle_mirror(c, images, c["host"], sids, cids, 0, 4, is_read=False)
    c["worker"]._transfer_impl(cids, sids, TransferType.H2DISK, 0, 4)
    assert all(np.array_equal(a, b) for a, b in zip(_file_images(c["files"], c["used"]), images))
    c["worker"].close()


@pytest.mark.skipif(not URING, reason="the kernel gives this process no io_uring ring")
@pytest.mark.parametrize("flags", [1, 2], ids=["IOPOLL", "SQPOLL"])
def test_iouring_setup_flags_match_oracle(tmp_path, flags):
    """Rings set up for polled completions (IORING_SETUP_IOPOLL: page-cache
    requests are refused by the kernel and redone with blocking I/O) and with
    a kernel submission thread (IORING_SETUP_SQPOLL) move the same bytes as
    the oracle, through writes and O_DIRECT-sized reads."""
    c = _product_case(tmp_path, BW, False, 2, -1, 16, 2, 64, engine="uring64",
                      iouring_flags=flags)
    g = np.random.default_rng(flags)
    sids = g.permutation(c["ssd"].num_block)[:13].astype(np.int64)
    cids = g.permutation(c["cpu"].num_block)[:13].astype(np.int64)
    images = _file_images(c["files"], c["used"])
    _oracle_mirror(c, images, c["host"], sids, cids, 0, 4, is_read=False)
    c["worker"]._transfer_impl(cids, sids, TransferType.H2DISK, 0, 4)
    after = _file_images(c["files"], c["used"])
    assert all(np.array_equal(a, b) for a, b in zip(after, images))
    dst = g.permutation(c["cpu"].num_block)[:13].astype(np.int64)
    expect = c["host"].copy()
    _oracle_mirror(c, after, expect, sids, dst, 0, 4, is_read=True)
    c["worker"]._transfer_impl(sids, dst, TransferType.DISK2H, 0, 4)
    assert np.array_equal(c["host"], expect)
    c["worker"].close()


def test_iouring_read_past_end_of_file_reports_error(tmp_path):
    """A ring read that meets the end of a file fails the call like the
    threaded read does."""
    p = tmp_path / "short.bin"
    p.write_bytes(b"\1" * 4096)
    ctx = c_ext.SSDIOCTX({0: [str(p)]}, 1, iouring_entries=8)
    host = np.zeros(4 * 4096 + 4096, np.uint8)
    with pytest.raises(RuntimeError, match="read failed|end of file"):
        c_ext.transfer_kv_blocks_ssd(
            ctx, torch.arange(0, 1, dtype=torch.int32), host.ctypes.data,
            torch.tensor([3], dtype=torch.int64), torch.tensor([0], dtype=torch.int64),
            4096, 4096, 4096, 4096, 4096, 4096, True, 4)
    ctx.close()


# ------------------------------------------------------------ error behaviour

def test_open_missing_file_raises(tmp_path):
    with pytest.raises(RuntimeError, match="open"):
        c_ext.SSDIOCTX({0: [str(tmp_path / "absent.bin")]}, 1)


def test_uneven_file_lists_rejected(tmp_path):
    p = tmp_path / "a.bin"
    p.write_bytes(b"\0" * 4096)
    with pytest.raises(ValueError):
        c_ext.SSDIOCTX({0: [str(p)], 1: [str(p), str(p)]}, 2)


def test_out_of_range_ids_rejected_by_worker(tmp_path):
    c = _product_case(tmp_path, BW, False, 1, -1, 4, 1, 64)
    w = c["worker"]
    with pytest.raises(ValueError, match="ssd block id"):
        w._transfer_impl(np.array([0], np.int64), np.array([c["ssd"].num_block], np.int64),
                         TransferType.H2DISK, 0, 4)
    with pytest.raises(ValueError, match="cpu block id"):
        w._transfer_impl(np.array([-1], np.int64), np.array([0], np.int64),
                         TransferType.H2DISK, 0, 4)
    with pytest.raises(ValueError, match="layer range"):
        w._transfer_impl(np.array([0], np.int64), np.array([0], np.int64),
                         TransferType.H2DISK, 3, 2)
    with pytest.raises(ValueError, match="Invalid transfer type"):
        w._transfer_impl(np.array([0], np.int64), np.array([0], np.int64),
                         TransferType.H2D, 0, 4)
    w.close()


def test_read_past_end_of_file_reports_error(tmp_path):
    """The C-ABI entry reports a short file instead of returning stale bytes."""
    p = tmp_path / "short.bin"
    p.write_bytes(b"\1" * 1000)
    ctx = c_ext.SSDIOCTX({0: [str(p)]}, 1)
    host = np.zeros(8192, np.uint8)
    with pytest.raises(RuntimeError, match="read failed"):
        c_ext.transfer_kv_blocks_ssd(ctx, torch.arange(0, 1, dtype=torch.int32), host.ctypes.data,
                                     torch.tensor([1]), torch.tensor([0]), 0, 512, 0, 512, 512,
                                     2048, True, 1, is_mla=False)
    ctx.close()


def test_layer_list_must_be_contiguous(tmp_path):
    p = tmp_path / "f.bin"
    p.write_bytes(b"\0" * 8192)
    ctx = c_ext.SSDIOCTX({0: [str(p)]}, 1)
    host = np.zeros(8192, np.uint8)
    with pytest.raises(ValueError):
        c_ext.transfer_kv_blocks_ssd(ctx, torch.tensor([0, 2], dtype=torch.int32),
                                     host.ctypes.data, torch.tensor([0]), torch.tensor([0]),
                                     1024, 512, 1024, 512, 512, 4096, True, 1)
    ctx.close()


# ------------------------------------------------------------ allocator/engine

def test_allocator_file_layout(tmp_path):
    lay = KVCacheLayout(LW, 2, 30, 4, 2, 8)
    dirs = [str(tmp_path / "a"), str(tmp_path / "b"), str(tmp_path / "c")]
    h = SSDAllocator.allocate(lay, torch.bfloat16, cache_dir=dirs, max_blocks_per_file=4)
    files = h.get_file_list()
    blk = lay.get_elements_per_block() * 2
    assert h.num_blocks_per_file == 4
    assert sorted(files) == [0, 1, 2]
    for d in range(3):
        assert len(files[d]) == 3            # ceil(10 / 4)
        for j, p in enumerate(files[d]):
            assert os.path.basename(p) == f"flexkv_ssd_cache_{d}_{j}.bin"
            assert os.path.getsize(p) == 4 * blk
    with pytest.raises(ValueError, match="multiple"):
        SSDAllocator.allocate(KVCacheLayout(LW, 2, 31, 4, 2, 8), torch.bfloat16, cache_dir=dirs)
    with pytest.raises(ValueError):
        SSDAllocator.allocate(lay, torch.bfloat16)


def test_engine_routes_ssd_ops(tmp_path, monkeypatch):
    """H2DISK then DISK2H graphs through TransferEngine's SSD workers move a
    host block to SSD and back into other host blocks (the GPU<->CPU worker is
    a recording stand-in: no device here)."""
    from _fake_worker import FakeGPUCPUWorker
    from flexkv_amd.storage.allocator import AccessHandleType, StorageHandle
    from flexkv_amd.transfer import transfer_engine as te
    monkeypatch.setattr(te, "GPUCPUTransferWorker", FakeGPUCPUWorker)
    mc = ModelConfig(num_layers=4, num_kv_heads=2, head_size=64, dtype=torch.float16)
    cc = CacheConfig(tokens_per_block=16, num_cpu_blocks=32, enable_ssd=True, num_ssd_blocks=64,
                     ssd_cache_dir=[str(tmp_path / "s0"), str(tmp_path / "s1")],
                     max_blocks_per_file=12)
    cpu_lay = KVCacheLayout(cc.cpu_kv_layout_type, 4, 32, 16, 2, 64)
    ssd_lay = KVCacheLayout(cc.ssd_kv_layout_type, 4, 64, 16, 2, 64)
    host = torch.from_numpy(_rng_bytes(cpu_lay.get_total_elements() * 2, 9)).view(torch.float16)
    ssd = SSDAllocator.allocate(ssd_lay, torch.float16, cache_dir=cc.ssd_cache_dir,
                                max_blocks_per_file=cc.max_blocks_per_file)
    cpu = StorageHandle(AccessHandleType.TENSOR, host, cpu_lay, torch.float16)
    gpu = StorageHandle(AccessHandleType.TENSOR, [torch.zeros(1)] * 4,
                        KVCacheLayout(LW, 4, 8, 16, 2, 64), torch.float16, gpu_device_id=0)
    eng = te.TransferEngine([gpu], mc, cc, cpu_handle=cpu, ssd_handle=ssd)
    eng.start()
    try:
        src = torch.tensor([0, 5, 9, 31], dtype=torch.int64)
        sids = torch.tensor([63, 2, 17, 40], dtype=torch.int64)
        dst = torch.tensor([1, 2, 3, 4], dtype=torch.int64)
        bits = host.view(torch.int16).view(32, -1)     # random bytes hold NaN patterns
        expect = bits[src].clone()
        g1 = TransferOpGraph()
        g1.add_transfer_op(TransferOp(g1.graph_id, TransferType.H2DISK, 0, 4,
                                      TransferDescriptor(DeviceType.CPU, 0, src),
                                      TransferDescriptor(DeviceType.SSD, 0, sids)))
        g2 = TransferOpGraph()
        g2.add_transfer_op(TransferOp(g2.graph_id, TransferType.DISK2H, 0, 4,
                                      TransferDescriptor(DeviceType.SSD, 0, sids),
                                      TransferDescriptor(DeviceType.CPU, 0, dst)))
        for g in (g1, g2):
            eng.submit_transfer_graph(g)
            t0 = time.time()
            seen = []
            while (g.graph_id, -1) not in seen:
                assert time.time() - t0 < 20, f"graph {g.graph_id} did not complete"
                seen += eng.get_completed_graphs_and_ops(timeout=0.05)
        assert torch.equal(bits[dst], expect)
    finally:
        eng.shutdown()


def test_engine_rejects_ssd_in_process_mode(tmp_path):
    from flexkv_amd.transfer.transfer_engine import TransferEngine
    from flexkv_amd.storage.allocator import AccessHandleType, StorageHandle
    lay = KVCacheLayout(BW, 1, 2, 1, 1, 8)
    h = StorageHandle(AccessHandleType.FILE, {0: []}, lay, torch.float16, num_blocks_per_file=1)
    with pytest.raises(NotImplementedError):
        TransferEngine([h], ModelConfig(1, 1, 8), CacheConfig(), cpu_handle=h, ssd_handle=h,
                       worker_mode="process")


# ------------------------------------------------------------ randomized

from hypothesis import HealthCheck, given, settings, strategies as st  # noqa: E402


@settings(max_examples=25, deadline=None, suppress_health_check=[HealthCheck.function_scoped_fixture])
@given(layout=st.sampled_from([LW, BW]), mla=st.booleans(), n_dev=st.integers(1, 3),
       mbpf=st.sampled_from([-1, 3, 5, 16]), tpb=st.sampled_from([1, 4, 16]),
       dh=st.sampled_from([8, 64, 72]), start=st.integers(0, 2), seed=st.integers(0, 10**6),
       engine=st.sampled_from(list(ENGINES)))
def test_random_geometries_match_oracle(tmp_path_factory, layout, mla, n_dev, mbpf, tpb, dh,
                                        start, seed, engine):
    """Random layouts, devices, files per device, chunk sizes (some not
    page multiples), layer windows and id lists: files and host cache equal
    the oracle's after a write and a read."""
    tmp = tmp_path_factory.mktemp("ssd")
    L = 3
    c = _product_case(tmp, layout, mla, n_dev, mbpf, tpb, 1, dh, L=L, N_cpu=24,
                      n_ssd=12 * n_dev, seed=seed % 997, engine=engine)
    g = np.random.default_rng(seed)
    n = int(g.integers(1, 12))
    sids = g.permutation(c["ssd"].num_block)[:n].astype(np.int64)
    cids = g.permutation(c["cpu"].num_block)[:n].astype(np.int64)
    nl = int(g.integers(1, L - start + 1))
    images = _file_images(c["files"], c["used"])
    _oracle_mirror(c, images, c["host"], sids, cids, start, nl, is_read=False)
    c["worker"]._transfer_impl(cids, sids, TransferType.H2DISK, start, nl)
    assert all(np.array_equal(a, b) for a, b in zip(_file_images(c["files"], c["used"]), images))
    dst = g.permutation(c["cpu"].num_block)[:n].astype(np.int64)
    expect = c["host"].copy()
    _oracle_mirror(c, images, expect, sids, dst, start, nl, is_read=True)
    c["worker"]._transfer_impl(sids, dst, TransferType.DISK2H, start, nl)
    assert np.array_equal(c["host"], expect)
    c["worker"].close()


@pytest.mark.parametrize("entries", [0, 8])
def test_contexts_release_their_files(tmp_path, entries):
    """Opening and closing contexts (threads, and a ring where the kernel
    allows one) leaves the process's open descriptors where they were."""
    import psutil
    paths = []
    for i in range(3):
        p = tmp_path / f"f{i}.bin"
        p.write_bytes(b"\0" * 8192)
        paths.append(str(p))
    proc = psutil.Process(os.getpid())
    c_ext.SSDIOCTX({0: paths[:2], 1: paths[1:]}, 2, iouring_entries=entries).close()
    before = proc.num_fds()
    for _ in range(100):
        ctx = c_ext.SSDIOCTX({0: paths[:2], 1: paths[1:]}, 2, iouring_entries=entries)
        ctx.close()
    assert proc.num_fds() == before
