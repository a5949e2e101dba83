"""Worker host logic without a device: op records, the run loop, process
lifecycle, and GPUCPUTransferWorker's argument mapping
(flexkv/transfer/worker.py:49-342)."""
import multiprocessing as mp

import numpy as np
import pytest
import torch

from flexkv_amd.common.transfer import (DeviceType, TransferDescriptor, TransferOp,
                                        TransferType)
from flexkv_amd.transfer import worker as W
from _fake_worker import RecordingWorker


def make_op(kind=TransferType.D2H, src=(1, 2, 3), dst=(7, 8, 9), layer_id=-1, gran=-1):
    return TransferOp(graph_id=3, transfer_type=kind, layer_id=layer_id, layer_granularity=gran,
                      src_descriptor=TransferDescriptor(DeviceType.GPU, 0,
                                                        torch.tensor(src, dtype=torch.int64)),
                      dst_descriptor=TransferDescriptor(DeviceType.CPU, 0,
                                                        torch.tensor(dst, dtype=torch.int64)))


def test_transfer_op_checks_and_ids():
    a, b = make_op(), make_op()
    assert b.op_id > a.op_id
    with pytest.raises(ValueError):
        make_op(src=(1, 2), dst=(1,))
    v = TransferOp(graph_id=0, transfer_type=TransferType.VIRTUAL, layer_id=0,
                   layer_granularity=1,
                   src_descriptor=TransferDescriptor(physical_block_ids=torch.tensor([1])))
    assert v.transfer_type == TransferType.VIRTUAL
    with pytest.raises(ValueError):
        TransferDescriptor(physical_block_ids=torch.tensor([1], dtype=torch.int32))
    with pytest.raises(ValueError):
        TransferDescriptor(physical_block_ids=torch.zeros(2, 2, dtype=torch.int64))


def test_worker_transfer_op_record():
    op = make_op(layer_id=4, gran=2)
    w = W.WorkerTransferOp(op)
    assert w.transfer_op_id == op.op_id and w.transfer_graph_id == 3
    assert w.src_block_ids.dtype == np.int64 and list(w.dst_block_ids) == [7, 8, 9]
    assert (w.layer_id, w.layer_granularity) == (4, 2)


def test_run_loop_batches_reports_and_survives_failures():
    parent, child = mp.Pipe()
    q = mp.Queue()
    ops = [make_op() for _ in range(4)]
    w = RecordingWorker(0, child, q, fail_on={ops[1].op_id})
    for op in ops:
        parent.send(W.WorkerTransferOp(op))
    parent.send(None)
    w.run()
    assert w.seen == [op.op_id for op in ops]
    assert [q.get(timeout=5) for _ in ops] == [op.op_id for op in ops]
    assert w.failed_ops == [ops[1].op_id]


def test_spawned_worker_process_lifecycle():
    ctx = mp.get_context("spawn")
    q = ctx.Queue()
    handle = RecordingWorker.create_worker(5, q)
    assert handle.ready_event.wait(60)
    ops = [make_op() for _ in range(3)]
    for op in ops:
        handle.submit_transfer(op)
    got = [q.get(timeout=30) for _ in ops]
    assert got == [op.op_id for op in ops]
    handle.shutdown()
    assert not handle.process.is_alive()


class _Recorder:
    def __init__(self):
        self.calls = []
        self.streams = []

    def __call__(self, *args, stream=None):
        self.calls.append(args)
        self.streams.append(stream)


def _bare_gpu_worker(monkeypatch, mla=False):
    """A GPUCPUTransferWorker with its attributes set by hand (no device)."""
    rec = _Recorder()
    monkeypatch.setattr(W, "transfer_kv_blocks", rec)
    monkeypatch.setattr(torch.Tensor, "pin_memory", lambda self, *a, **k: self)
    w = object.__new__(W.GPUCPUTransferWorker)
    W.TransferWorkerBase.__init__(w, 0, None, None)
    w.gpu_layer_ptrs = torch.arange(100, 108, dtype=torch.int64)
    w.separate_kv = False
    w.num_layers = 8
    w.cpu_tensor = torch.zeros(4)
    w.is_mla = mla
    w.chunk_size_in_bytes = 32768
    w.gpu_kv_stride_in_bytes, w.gpu_block_stride_in_bytes = 1 << 27, 32768
    w.cpu_kv_stride_in_bytes, w.cpu_layer_stride_in_bytes = 32768, 65536
    w.cpu_block_stride_in_bytes = 1 << 20
    w.use_ce_transfer_h2d, w.use_ce_transfer_d2h = True, False
    w.transfer_sms_h2d, w.transfer_sms_d2h = 16, 8
    return w, rec


def test_direction_mapping(monkeypatch):
    w, rec = _bare_gpu_worker(monkeypatch)
    src, dst = np.array([1, 2], np.int64), np.array([30, 40], np.int64)
    w._transfer_impl(src, dst, TransferType.D2H, 0, 8)
    a = rec.calls[-1]
    assert list(a[0]) == [1, 2] and list(a[4]) == [30, 40]      # gpu = src for D2H
    assert a[11] == 8 and a[12] is False and a[13] is False       # sms, h2d, ce
    w._transfer_impl(src, dst, TransferType.H2D, 2, 3)
    a = rec.calls[-1]
    assert list(a[0]) == [30, 40] and list(a[4]) == [1, 2]      # gpu = dst for H2D
    assert list(a[1]) == [102, 103, 104] and a[10] == 2           # layer window, start layer
    assert a[11] == 16 and a[12] is True and a[13] is True


def test_separate_kv_pointer_window(monkeypatch):
    """Layers given as [K, V] pairs: the pointer table is [layer][K|V] and a
    layer window takes 2 entries per layer (1 for MLA)."""
    for mla, kv in ((False, 2), (True, 1)):
        w, rec = _bare_gpu_worker(monkeypatch, mla=mla)
        kvrec = _Recorder()
        monkeypatch.setattr(W, "transfer_kv_blocks_kv_ptrs", kvrec)
        w.separate_kv = True
        w.gpu_layer_ptrs = torch.arange(200, 200 + 8 * kv, dtype=torch.int64)
        src, dst = np.array([5], np.int64), np.array([6], np.int64)
        w._transfer_impl(src, dst, TransferType.H2D, 3, 2)
        a = kvrec.calls[-1]
        assert list(a[1]) == list(range(200 + 3 * kv, 200 + 5 * kv))
        assert list(a[0]) == [6] and list(a[3]) == [5] and a[9] == 3 and a[11] is True
        assert not rec.calls


def test_bad_type_empty_ids_and_layer_window(monkeypatch):
    w, rec = _bare_gpu_worker(monkeypatch)
    ids = np.array([1], np.int64)
    with pytest.raises(ValueError, match="Invalid transfer type"):
        w._transfer_impl(ids, ids, TransferType.H2DISK, 0, 8)
    empty = np.zeros(0, np.int64)
    w._transfer_impl(empty, empty, TransferType.D2H, 0, 8)
    assert rec.calls == []
    with pytest.raises(ValueError):
        w._transfer_impl(ids, ids, TransferType.D2H, 6, 4)
    with pytest.raises(AssertionError):
        w._transfer_impl(ids.astype(np.int32), ids, TransferType.D2H, 0, 8)


def test_launch_transfer_defaults(monkeypatch):
    w, rec = _bare_gpu_worker(monkeypatch, mla=True)
    monkeypatch.setattr(torch.cuda, "stream", lambda s: _NullCtx())
    w.transfer_stream = None
    w._stream_handle = 0x1234                                   # the worker's own stream
    op = W.WorkerTransferOp(make_op(TransferType.D2H, layer_id=-1, gran=-1))
    w.launch_transfer(op)
    a = rec.calls[-1]
    assert a[10] == 0 and len(a[1]) == 8 and a[14] is True       # all layers, is_mla
    assert rec.streams[-1] == 0x1234


class _NullCtx:
    def __enter__(self):
        return self

    def __exit__(self, *a):
        return False


def test_c_ext_argument_checks(per_call_path):
    from flexkv_amd import c_ext
    ids = torch.tensor([1, 2], dtype=torch.int64)
    ptrs = torch.tensor([0], dtype=torch.int64)
    cache = torch.zeros(16)
    with pytest.raises(TypeError):
        c_ext.transfer_kv_blocks(ids.int(), ptrs, 0, 0, ids, cache, 0, 0, 0, 16, 0)
    with pytest.raises(TypeError):
        c_ext.transfer_kv_blocks(ids, ptrs, 0, 0, ids, "cache", 0, 0, 0, 16, 0)
    with pytest.raises(RuntimeError, match="ids"):
        c_ext.transfer_kv_blocks(ids, ptrs, 0, 0, ids[:1], cache, 0, 0, 0, 16, 0)
    with pytest.raises(RuntimeError, match="contiguous"):
        c_ext.transfer_kv_blocks(torch.arange(4)[::2], ptrs, 0, 0, ids, cache, 0, 0, 0, 16, 0)
    if not torch.cuda.is_available():
        with pytest.raises(RuntimeError, match="HIP device"):
            c_ext.transfer_kv_blocks(ids, ptrs, 0, 0, ids, cache, 0, 0, 0, 16, 0)


def test_c_ext_kv_ptrs_and_scalar_checks(per_call_path):
    """The compiled per-call path refuses what the Python signature refuses,
    with the same error types, for both entry points."""
    from flexkv_amd import c_ext
    ids = torch.tensor([1, 2], dtype=torch.int64)
    cache = torch.zeros(16)
    three = torch.tensor([0, 0, 0], dtype=torch.int64)
    with pytest.raises(RuntimeError, match="not a multiple of 2"):
        c_ext.transfer_kv_blocks_kv_ptrs(ids, three, 0, ids, cache, 0, 0, 0, 16, 0)
    with pytest.raises(RuntimeError, match="ids"):
        c_ext.transfer_kv_blocks_kv_ptrs(ids, three[:2], 0, ids[:1], cache, 0, 0, 0, 16, 0)
    with pytest.raises(RuntimeError, match="host tensor"):
        c_ext.transfer_kv_blocks(ids.to("meta"), three, 0, 0, ids, cache, 0, 0, 0, 16, 0)
    with pytest.raises(TypeError):                      # strides are integers, as in bindings.cpp
        c_ext.transfer_kv_blocks(ids, three, 0.5, 0, ids, cache, 0, 0, 0, 16, 0)
    with pytest.raises(TypeError):
        c_ext.transfer_kv_blocks(ids, three, 0, 0, ids, cache, 0, 0, 0, 16, 0, -1, True, "ce")
    with pytest.raises(OverflowError):                  # start_layer_id is a C int
        c_ext.transfer_kv_blocks(ids, three, 0, 0, ids, cache, 0, 0, 0, 16, 1 << 31)
    if not torch.cuda.is_available():
        # integer-like scalars and an integer mode pass the checks; only the device is missing
        with pytest.raises(RuntimeError, match="HIP device"):
            c_ext.transfer_kv_blocks(ids, three, np.int64(0), 0, ids, cache, 0, 0, 0, 16, 0, -1,
                                     True, 2, False)
        with pytest.raises(RuntimeError, match="HIP device"):
            c_ext.transfer_kv_blocks_kv_ptrs(ids, three, 0, ids, cache, 0, 0, 0, 16, 0, -1, True,
                                             False, True)
        with pytest.raises(RuntimeError, match="HIP device"):   # numpy bools, as pybind takes them
            c_ext.transfer_kv_blocks(ids, three, 0, 0, ids, cache, 0, 0, 0, 16, 0, -1,
                                     np.True_, np.False_, np.False_)


def test_c_ext_fast_module_shares_the_library():
    """_fkv_py is bound to the functions of the library _lib loaded, and the
    process maps that library once."""
    import ctypes
    from flexkv_amd import _lib
    fast = _lib.fast()
    assert _lib.fast() is fast
    lib = _lib.load()
    assert ctypes.cast(lib.fkv_transfer_kv_blocks, ctypes.c_void_p).value
    paths = set()
    with open("/proc/self/maps") as fh:
        for line in fh:
            parts = line.split()
            if len(parts) >= 6 and parts[-1].endswith("libflexkv_hip.so"):
                paths.add(parts[-1])
    assert len(paths) == 1
    with pytest.raises(TypeError):
        fast.transfer_kv_blocks(1, 2, 3)


def test_idle_worker_waits_long_and_wakes_on_send():
    """The run loop waits POLL_IDLE_S per poll while idle, not the
    reference's 100 us, and a waiting poll returns as soon as an op is sent."""
    import threading
    import time
    ch = W.LocalChannel()
    assert ch.poll(0) is False
    got = []
    th = threading.Thread(target=lambda: got.append(ch.poll(30.0)))
    th.start()
    time.sleep(0.05)
    ch.send("op")
    th.join(timeout=10)
    assert not th.is_alive() and got == [True] and ch.recv() == "op"

    class Conn:
        def __init__(self):
            self.timeouts = []

        def poll(self, timeout=0.0):
            self.timeouts.append(timeout)
            return len(self.timeouts) > 1      # idle once, then the stop message

        def recv(self):
            return None

    w = RecordingWorker(0, Conn(), None)
    w.run()
    assert w.transfer_conn.timeouts[0] == W.TransferWorkerBase.POLL_IDLE_S >= 0.01


def test_layerwise_argument_checks():
    """The layer-wise entry refuses the same bad arguments before any device
    work: non-tensor host cache, ids of different lengths, non-int64 ids."""
    from flexkv_amd import c_ext
    ids = torch.tensor([1, 2], dtype=torch.int64)
    ptrs = torch.tensor([0], dtype=torch.int64)
    with pytest.raises(TypeError, match="cpu_tensor"):
        c_ext.transfer_kv_blocks_layerwise(ids, ptrs, 0, 0, ids, "cache", 0, 0, 0, 16, 0, 1)
    with pytest.raises(RuntimeError, match="differ in length"):
        c_ext.transfer_kv_blocks_layerwise(ids, ptrs, 0, 0, ids[:1], torch.zeros(4), 0, 0, 0,
                                           16, 0, 1)
    with pytest.raises(TypeError, match="int64"):
        c_ext.transfer_kv_blocks_layerwise(ids.int(), ptrs, 0, 0, ids, torch.zeros(4), 0, 0, 0,
                                           16, 0, 1)


def _put_ids(ch, ids):
    for i in ids:
        ch.put(i)


def test_finished_ops_channel_across_processes():
    """FinishedOpsChannel carries op ids from a spawned process in order, and
    follows queue.Queue's get: a timeout or get_nowait on an empty channel
    raises queue.Empty."""
    import queue
    ctx = mp.get_context("spawn")
    ch = W.FinishedOpsChannel(ctx)
    with pytest.raises(queue.Empty):
        ch.get_nowait()
    with pytest.raises(queue.Empty):
        ch.get(timeout=0.01)
    p = ctx.Process(target=_put_ids, args=(ch, list(range(200))))
    p.start()
    got = [ch.get(timeout=60) for _ in range(200)]
    p.join(60)
    assert got == list(range(200)) and p.exitcode == 0
    ch.put("local")
    assert ch.get() == "local"
