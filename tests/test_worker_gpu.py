"""GPUCPUTransferWorker end to end on the device: the reference's round-trip
check (tests/test_transfer_engine.py:55-161 with tests/test_utils.py:133-204),
in process and through a spawned worker fed TensorSharedHandles."""
import multiprocessing as mp

import pytest
import torch

from gpu_util import zero_blocks
from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType
from flexkv_amd.common.transfer import TransferDescriptor, TransferOp, TransferType
from flexkv_amd.storage.allocator import CPUAllocator
from flexkv_amd.transfer.worker import GPUCPUTransferWorker, WorkerTransferOp

pytestmark = pytest.mark.gpu

L, NG, NH, T, H, D = 4, 128, 160, 16, 8, 128


def _ground_truth(mla, seed=0):
    gen = torch.Generator().manual_seed(seed)
    gl = KVCacheLayout(KVCacheLayoutType.LAYERWISE, L, NG, T, H, D, is_mla=mla)
    return gl, [torch.randn(tuple(gl.kv_shape[1:]), generator=gen).to(torch.float16)
                for _ in range(L)]


def _op(kind, src, dst, layer_id=-1, gran=-1):
    return TransferOp(graph_id=0, transfer_type=kind, layer_id=layer_id,
                      layer_granularity=gran,
                      src_descriptor=TransferDescriptor(physical_block_ids=src),
                      dst_descriptor=TransferDescriptor(physical_block_ids=dst))


@pytest.mark.parametrize("mla", [False, True])
@pytest.mark.parametrize("layout", [KVCacheLayoutType.LAYERWISE, KVCacheLayoutType.BLOCKWISE])
@pytest.mark.parametrize("ce", [False, True])
def test_in_process_round_trip(mla, layout, ce):
    gl, gt = _ground_truth(mla)
    gpu = [t.cuda() for t in gt]
    cl = KVCacheLayout(layout, L, NH, T, H, D, is_mla=mla)
    cpu = CPUAllocator.allocate(cl, torch.float16).get_tensor()
    w = GPUCPUTransferWorker(0, None, None, gpu, cpu, gl, cl, torch.float16, 0,
                             use_ce_transfer_h2d=ce, use_ce_transfer_d2h=not ce,
                             transfer_sms_h2d=4, transfer_sms_d2h=4)
    gids = torch.arange(0, 16, dtype=torch.int64)
    cids = torch.arange(40, 56, dtype=torch.int64)
    w.launch_transfer(WorkerTransferOp(_op(TransferType.D2H, gids, cids)))
    for t in gpu:
        zero_blocks(t, gids)
    torch.cuda.synchronize()
    w.launch_transfer(WorkerTransferOp(_op(TransferType.H2D, cids, gids)))
    for l in range(L):
        assert torch.equal(gpu[l].cpu(), gt[l]), f"layer {l}"
    assert w.failed_ops == []


def test_layer_wise_ops_and_random_ids():
    """Per-layer-group H2D ops, as the layer-wise read graph issues them
    (flexkv/cache/transfer_pattern.py:370-428, worker.py:293-295)."""
    gl, gt = _ground_truth(False, seed=3)
    gpu = [t.cuda() for t in gt]
    cl = KVCacheLayout(KVCacheLayoutType.BLOCKWISE, L, NH, T, H, D)
    cpu = CPUAllocator.allocate(cl, torch.float16).get_tensor()
    w = GPUCPUTransferWorker(0, None, None, gpu, cpu, gl, cl, torch.float16, 0)
    g = torch.Generator().manual_seed(1)
    gids = torch.randperm(NG, generator=g)[:37]
    cids = torch.randperm(NH, generator=g)[:37]
    w.launch_transfer(WorkerTransferOp(_op(TransferType.D2H, gids, cids)))
    for t in gpu:
        t.zero_()
    torch.cuda.synchronize()
    for layer_id in range(0, L, 2):
        w.launch_transfer(WorkerTransferOp(_op(TransferType.H2D, cids, gids, layer_id, 2)))
        for l in range(L):
            got = gpu[l][:, gids].cpu()
            if l < layer_id + 2:
                assert torch.equal(got, gt[l][:, gids])
            else:
                assert torch.count_nonzero(got) == 0
    host = cpu.view(NH, L, 2, T, H, D)
    assert torch.equal(host[cids, 1], torch.stack([gt[1][:, i] for i in gids]))


def test_failed_op_is_reported_and_recorded():
    gl, gt = _ground_truth(False)
    gpu = [t.cuda() for t in gt]
    cl = KVCacheLayout(KVCacheLayoutType.BLOCKWISE, L, NH, T, H, D)
    cpu = CPUAllocator.allocate(cl, torch.float16).get_tensor()
    w = GPUCPUTransferWorker(0, None, None, gpu, cpu, gl, cl, torch.float16, 0)
    bad = _op(TransferType.D2H, torch.tensor([1 << 30]), torch.tensor([0]))
    w._execute(WorkerTransferOp(bad))
    assert w.failed_ops == [bad.op_id]


def test_pageable_host_cache_rejected_at_worker_start():
    gl, gt = _ground_truth(False)
    gpu = [t.cuda() for t in gt]
    cl = KVCacheLayout(KVCacheLayoutType.BLOCKWISE, L, NH, T, H, D)
    cpu = CPUAllocator.allocate(cl, torch.float16, pin_memory=False).get_tensor()
    with pytest.raises(RuntimeError, match="pinned"):
        GPUCPUTransferWorker(0, None, None, gpu, cpu, gl, cl, torch.float16, 0)


def test_spawned_worker_with_shared_gpu_tensors():
    """create_worker in a spawned process; GPU layers reach it as
    TensorSharedHandles (HIP IPC); the worker allocates its pinned host cache
    from a HostCacheSpec.  Checked by the reference's round trip: D2H, zero
    the GPU blocks, H2D, compare with the ground truth."""
    from flexkv_amd.common.memory_handle import TensorSharedHandle
    from flexkv_amd.storage.allocator import HostCacheSpec
    gl, gt = _ground_truth(False, seed=9)
    gpu = [t.cuda() for t in gt]
    cl = KVCacheLayout(KVCacheLayoutType.BLOCKWISE, L, NH, T, H, D)
    ctx = mp.get_context("spawn")
    q = ctx.Queue()
    print("spawning worker", flush=True)
    handle = GPUCPUTransferWorker.create_worker(
        0, q, [TensorSharedHandle(t) for t in gpu], HostCacheSpec(cl, torch.float16), gl, cl,
        torch.float16, 0)
    try:
        assert handle.ready_event.wait(120), "worker did not start"
        gids = torch.tensor([3, 17, 64, 90], dtype=torch.int64)
        cids = torch.tensor([150, 2, 77, 8], dtype=torch.int64)
        op = _op(TransferType.D2H, gids, cids)
        handle.submit_transfer(op)
        assert q.get(timeout=120) == op.op_id
        for t in gpu:
            zero_blocks(t, gids)
        torch.cuda.synchronize()
        op2 = _op(TransferType.H2D, cids, gids)
        handle.submit_transfer(op2)
        assert q.get(timeout=120) == op2.op_id
        for l in range(L):
            assert torch.equal(gpu[l].cpu(), gt[l])
    finally:
        handle.shutdown()


def _host_expected(before, cl, gt, gids, cids):
    """The host cache after a D2H of GPU blocks `gids` into host blocks
    `cids`, by tensor indexing on the layout's own shape ([N, L, kv, ...]
    block-wise, [L, kv, N, ...] layer-wise), not by byte strides."""
    exp = before.clone().view(tuple(cl.kv_shape))
    for l, t in enumerate(gt):
        for k in range(t.shape[0]):
            if cl.type == KVCacheLayoutType.BLOCKWISE:
                exp[cids, l, k] = t[k, gids]
            else:
                exp[l, k, cids] = t[k, gids]
    return exp.reshape(-1)


@pytest.mark.parametrize("mla", [False, True])
@pytest.mark.parametrize("layout", [KVCacheLayoutType.LAYERWISE, KVCacheLayoutType.BLOCKWISE])
@pytest.mark.parametrize("ce", [False, True])
def test_worker_d2h_host_bytes(mla, layout, ce):
    """Every byte of the host cache after a D2H op through the worker,
    untouched blocks included (a layer-wise stride mistake that a round trip
    would undo shows up here)."""
    gl, gt = _ground_truth(mla, seed=11)
    gpu = [t.cuda() for t in gt]
    cl = KVCacheLayout(layout, L, NH, T, H, D, is_mla=mla)
    cpu = CPUAllocator.allocate(cl, torch.float16).get_tensor()
    cpu.view(torch.int16).fill_(0x5A5A)
    before = cpu.clone()
    w = GPUCPUTransferWorker(0, None, None, gpu, cpu, gl, cl, torch.float16, 0,
                             use_ce_transfer_h2d=ce, use_ce_transfer_d2h=ce)
    g = torch.Generator().manual_seed(5)
    gids = torch.randperm(NG, generator=g)[:45]
    cids = torch.randperm(NH, generator=g)[:45]
    w.launch_transfer(WorkerTransferOp(_op(TransferType.D2H, gids, cids)))
    assert w.failed_ops == []
    exp = _host_expected(before, cl, gt, gids, cids)
    assert torch.equal(cpu.view(torch.int16), exp.view(torch.int16))
    # one layer group (layers 1..2) of an H2D op lands in those layers only
    for t in gpu:
        t.zero_()
    torch.cuda.synchronize()
    w.launch_transfer(WorkerTransferOp(_op(TransferType.H2D, cids, gids, 1, 2)))
    for l in range(L):
        got = gpu[l].cpu()
        if l in (1, 2):
            assert torch.equal(got[:, gids], gt[l][:, gids]), f"layer {l}"
            rest = torch.ones(NG, dtype=torch.bool)
            rest[gids] = False
            assert not got[:, rest].any(), f"layer {l}: blocks outside the op were written"
        else:
            assert not got.any(), f"layer {l} outside the op's layer window was written"
