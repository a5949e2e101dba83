"""Transfer workers for the GPU<->CPU path and the CPU<->SSD tier.

Same API as the reference's worker module for the single-GPU case
(flexkv/transfer/worker.py:49-342 and :482-602): WorkerTransferOp,
TransferWorkerBase (create_worker spawns a process fed through a Pipe, run()
polls and batches ops, finished op ids go to a queue), WorkerHandle
(submit_transfer, shutdown), GPUCPUTransferWorker and CPUSSDDiskTransferWorker
(_transfer_impl, launch_transfer).  The transfers themselves are
flexkv_amd.c_ext.transfer_kv_blocks and transfer_kv_blocks_ssd.

Differences from the reference:
  * the host cache must already be pinned (CPUAllocator pin_memory=True);
    page-locking existing pageable memory is not supported, so host_register
    checks the buffer instead of registering it (worker.py:35-41 registers).
    A worker in a spawned process takes a HostCacheSpec and allocates its
    pinned cache itself;
  * an op that fails is still reported complete (worker.py:159-169), and is
    also recorded in ``failed_ops`` of the worker and logged at error level.
"""
from __future__ import annotations

import collections
import contextlib
import multiprocessing as mp
import queue
import threading
import time
from abc import ABC, abstractmethod
from multiprocessing.connection import Connection
from typing import Any, Dict, List, Optional, Sequence, Tuple, Union

import ctypes
import numpy as np
import torch

from .. import _lib
from ..c_ext import (SSDIOCTX, TPTransferThreadGroup, transfer_kv_blocks,
                     transfer_kv_blocks_kv_ptrs, transfer_kv_blocks_ssd)
from ..common import trace
from ..common.debug import flexkv_logger
from ..common.memory_handle import TensorSharedHandle
from ..common.storage import KVCacheLayout, KVCacheLayoutType
from ..common.transfer import TransferOp, TransferType
from ..storage.allocator import HostCacheSpec


def host_register(tensor: torch.Tensor) -> None:
    """Check that `tensor` is pinned host memory the device can address
    (the reference registers it with cudaHostRegister, worker.py:35-41)."""
    size = tensor.numel() * tensor.element_size()
    lib = _lib.load()
    _lib.check(lib.fkv_host_register(ctypes.c_void_p(tensor.data_ptr()), size, 1),
               "fkv_host_register")


def host_unregister(tensor: torch.Tensor) -> None:
    _lib.load().fkv_host_unregister(ctypes.c_void_p(tensor.data_ptr()))


class WorkerTransferOp:
    """Picklable op record sent to a worker (worker.py:49-68)."""

    def __init__(self, transfer_op: TransferOp) -> None:
        self.transfer_op_id = transfer_op.op_id
        self.transfer_graph_id = transfer_op.graph_id
        self.transfer_type = transfer_op.transfer_type
        self.src_block_ids = transfer_op.src_descriptor.physical_block_ids.numpy()
        self.dst_block_ids = transfer_op.dst_descriptor.physical_block_ids.numpy()
        self.layer_id = transfer_op.layer_id
        self.layer_granularity = transfer_op.layer_granularity

    def __repr__(self) -> str:
        return (f"WorkerTransferOp(id={self.transfer_op_id}, graph={self.transfer_graph_id}, "
                f"type={self.transfer_type.name}, blocks={len(self.src_block_ids)}, "
                f"layer_id={self.layer_id}, granularity={self.layer_granularity})")


class LocalChannel:
    """In-process stand-in for a multiprocessing Connection pair: send() from
    the engine, poll()/recv() in the worker thread; send() wakes a waiting
    poll() at once."""

    def __init__(self) -> None:
        self._items: "collections.deque" = collections.deque()
        self._cv = threading.Condition()

    def send(self, obj: Any) -> None:
        with self._cv:
            self._items.append(obj)
            self._cv.notify()

    def poll(self, timeout: float = 0.0) -> bool:
        with self._cv:
            if not self._items and timeout:
                self._cv.wait(timeout)
            return bool(self._items)

    def recv(self) -> Any:
        with self._cv:
            while not self._items:
                self._cv.wait()
            return self._items.popleft()

    def close(self) -> None:
        pass


class FinishedOpsChannel:
    """Finished-ops queue for worker processes over one pipe.  put() in the
    worker writes the op id straight into the pipe; a multiprocessing.Queue
    hands it to a feeder thread first, which adds about 50 us to each op's
    round trip (spawned processes, median of 3000 round trips: 114 us
    through a Queue, 60 us through a pipe).  get() and get_nowait() in the
    engine follow queue.Queue (queue.Empty on a timeout).  The engine reads
    it continuously, so the pipe's buffer does not fill."""

    def __init__(self, ctx: Any = None) -> None:
        ctx = ctx or mp.get_context("spawn")
        self._reader, self._writer = ctx.Pipe(duplex=False)
        self._write_lock = ctx.Lock()
        self._read_lock = threading.Lock()

    def __getstate__(self) -> dict:
        state = self.__dict__.copy()
        del state["_read_lock"]          # per process
        return state

    def __setstate__(self, state: dict) -> None:
        self.__dict__.update(state)
        self._read_lock = threading.Lock()

    def put(self, obj: Any) -> None:
        with self._write_lock:
            self._writer.send(obj)

    def get(self, block: bool = True, timeout: Optional[float] = None) -> Any:
        with self._read_lock:
            if not block:
                timeout = 0.0
            if timeout is not None and not self._reader.poll(timeout):
                raise queue.Empty
            return self._reader.recv()

    def get_nowait(self) -> Any:
        return self.get(block=False)

    def close(self) -> None:
        """Close this process's ends of the pipe (the engine, once every
        worker using the channel has stopped)."""
        for conn in (self._reader, self._writer):
            with contextlib.suppress(OSError):
                conn.close()


class TransferWorkerBase(ABC):
    def __init__(self, worker_id: int, transfer_conn: Optional[Connection],
                 finished_ops_queue: Optional[Any]) -> None:
        self.worker_id = worker_id
        self.transfer_conn = transfer_conn
        self.finished_ops_queue = finished_ops_queue
        self.failed_ops: List[int] = []
        # failed op id -> host block ids that copy engines may still write
        # (copies the library gave up waiting for); see _note_failure
        self.unsafe_host_blocks: Dict[int, np.ndarray] = {}

    @staticmethod
    def _get_layer_ptrs(layer_blocks: Union[Sequence[torch.Tensor], torch.Tensor]) -> torch.Tensor:
        """Pinned int64 table of per-layer base addresses (worker.py:79-90)."""
        if isinstance(layer_blocks, torch.Tensor):
            layer_blocks = [layer_blocks]
        ptrs = torch.tensor([t.data_ptr() for t in layer_blocks], dtype=torch.int64)
        return ptrs.pin_memory() if torch.cuda.is_available() else ptrs

    @classmethod
    def create_worker(cls, worker_id: int, finished_ops_queue: Any, *args: Any,
                      **kwargs: Any) -> "WorkerHandle":
        """Start the worker in a spawned process (worker.py:92-106)."""
        ctx = mp.get_context("spawn")
        parent_conn, child_conn = ctx.Pipe()
        ready_event = ctx.Event()
        process = ctx.Process(target=cls._worker_process,
                              args=(worker_id, child_conn, finished_ops_queue, ready_event, *args),
                              kwargs=kwargs, daemon=True)
        process.start()
        return WorkerHandle(worker_id, parent_conn, process, ready_event)

    @classmethod
    def create_worker_thread(cls, worker_id: int, finished_ops_queue: Any, *args: Any,
                             **kwargs: Any) -> "ThreadWorkerHandle":
        """Start the worker on a thread of this process.  The transfer call
        releases the GIL while it runs, and the worker shares this process's
        pinned host cache and device tensors directly, with no IPC."""
        conn = LocalChannel()
        ready_event = threading.Event()
        errors: List[BaseException] = []

        def body() -> None:
            try:
                worker = cls(worker_id, conn, finished_ops_queue, *args, **kwargs)
            except BaseException as e:  # surfaced by ThreadWorkerHandle.wait_ready
                errors.append(e)
                ready_event.set()
                return
            worker.serve(ready_event)

        thread = threading.Thread(target=body, name=f"flexkv-worker-{worker_id}", daemon=True)
        thread.start()
        return ThreadWorkerHandle(worker_id, conn, thread, ready_event, errors)

    @classmethod
    def _worker_process(cls, worker_id: int, transfer_conn: Connection, finished_ops_queue: Any,
                        ready_event: Any, *args: Any, **kwargs: Any) -> None:
        """Body of a spawned worker process.  Its end of the op pipe is closed
        whichever way it leaves, so the parent's next send fails at once
        instead of writing into a pipe nobody reads.  A worker that cannot
        be built never signals readiness; the parent's wait on ready_event
        times out and the exception is in this process's stderr."""
        with contextlib.closing(transfer_conn):
            cls(worker_id, transfer_conn, finished_ops_queue, *args, **kwargs).serve(ready_event)

    def serve(self, ready_event: Any) -> None:
        """Announce readiness, run the op loop until stopped, then release
        what the worker holds (close)."""
        ready_event.set()
        try:
            self.run()
        finally:
            self.close()

    def close(self) -> None:
        """Release the worker's own resources once its loop has ended."""

    @abstractmethod
    def _transfer_impl(self, src_block_ids: np.ndarray, dst_block_ids: np.ndarray,
                       transfer_type: TransferType, layer_id: int, layer_granularity: int,
                       **kwargs: Any) -> None:
        ...

    @abstractmethod
    def launch_transfer(self, transfer_op: WorkerTransferOp) -> None:
        ...

    def _log_transfer_performance(self, transfer_op: WorkerTransferOp, transfer_size: int,
                                  start_time: float, end_time: float) -> None:
        if not flexkv_logger.enabled("INFO"):
            return
        dt = max(end_time - start_time, 1e-12)
        flexkv_logger.info(
            f"{transfer_op.transfer_type.name} transfer request: {transfer_op.transfer_op_id} "
            f"finished transfer data size: {transfer_size / 2**30} GB "
            f"transfer time: {dt:.4f} s transfer bandwidth: {transfer_size / dt / 1e9:.2f} GB/s")

    def _execute(self, op: WorkerTransferOp) -> None:
        try:
            with trace.op_range(trace.op_message(op)):    # worker.py:160-165
                self.launch_transfer(op)
        except Exception as e:
            self.failed_ops.append(op.transfer_op_id)
            flexkv_logger.error(f"Error launching transfer: {e}\nFailed transfer op: {op}")
            self._note_failure(op)
        if self.finished_ops_queue is not None:
            self.finished_ops_queue.put(op.transfer_op_id)

    def _note_failure(self, op: WorkerTransferOp) -> None:
        """After a failed op: the host blocks whose rows a copy engine may
        still write, because the library gave up waiting for its copies
        (fkv_last_unsafe_host_blocks, read on the thread that made the
        call), are kept in unsafe_host_blocks under the op id and logged.
        The op is reported finished as any failed op is; those host blocks
        must not be read or reused until abandoned_copies_pending() reads 0."""
        ids = _lib.last_unsafe_host_blocks()
        if ids:
            self.unsafe_host_blocks[op.transfer_op_id] = np.asarray(ids, dtype=np.int64)
            flexkv_logger.error(
                f"transfer op {op.transfer_op_id}: copy engines may still write {len(ids)} host "
                f"blocks after the failure; they stay unsafe until the abandoned copies finish")

    # How long the main loop's poll waits for an op.  A poll returns as soon
    # as an op arrives, so this bounds only the wakeups of an idle worker.
    # The reference polls every 100 us (worker.py:148), which keeps an idle
    # worker process at about 4% of a host core (0.4% at 50 ms), per GPU
    # and per SSD worker.
    POLL_IDLE_S = 0.05

    def run(self) -> None:
        """Main loop: wait for an op, drain whatever else is queued, run the
        batch in order, report each op id (worker.py:144-177)."""
        while True:
            try:
                if not self.transfer_conn.poll(timeout=self.POLL_IDLE_S):
                    continue
                op = self.transfer_conn.recv()
                if op is None:
                    break
                batch = [op]
                stop = False
                while self.transfer_conn.poll(timeout=0):
                    nxt = self.transfer_conn.recv()
                    if nxt is None:
                        stop = True
                        break
                    batch.append(nxt)
                for item in batch:
                    self._execute(item)
                if stop:
                    break
            except EOFError:
                break
            except Exception as e:  # keep serving; the reference does the same
                flexkv_logger.error(f"Error in worker run loop: {e}")


class _WorkerHandleBase:
    """What the engine holds of a worker wherever it runs: ops go in through
    submit_transfer, and shutdown() stops it.  A stop puts the sentinel None
    behind the ops already sent (run() finishes those first), allows
    STOP_GRACE_S for the worker to end, then forces the end where that is
    possible.  Subclasses say how to wait for the worker and how to force it
    (the reference waits 5 s for its process, then terminates it,
    worker.py:189-198)."""

    STOP_GRACE_S = 5.0

    def __init__(self, worker_id: int, transfer_conn: Any, ready_event: Any) -> None:
        self.worker_id = worker_id
        self.transfer_conn = transfer_conn
        self.ready_event = ready_event

    def submit_transfer(self, op: TransferOp) -> None:
        self.transfer_conn.send(WorkerTransferOp(op))

    def shutdown(self) -> None:
        try:
            self.transfer_conn.send(None)
        except OSError:
            pass        # the worker's end is closed already: it has stopped or died
        self._after_stop_sent()
        if not self._ended_within(self.STOP_GRACE_S):
            self._force_end()

    def _after_stop_sent(self) -> None:
        pass

    def _ended_within(self, timeout: float) -> bool:
        raise NotImplementedError

    def _force_end(self) -> None:
        raise NotImplementedError


class WorkerHandle(_WorkerHandleBase):
    """Parent-side handle of a worker process started by create_worker."""

    def __init__(self, worker_id: int, transfer_conn: Connection, process: Any,
                 ready_event: Any) -> None:
        super().__init__(worker_id, transfer_conn, ready_event)
        self.process = process

    def _after_stop_sent(self) -> None:
        # nothing more is sent; the worker sees EOF after the sentinel
        with contextlib.suppress(OSError):
            self.transfer_conn.close()

    def _ended_within(self, timeout: float) -> bool:
        self.process.join(timeout)
        return not self.process.is_alive()

    def _force_end(self) -> None:
        flexkv_logger.warning(f"worker {self.worker_id} did not stop within "
                              f"{self.STOP_GRACE_S:.0f} s; terminating its process")
        self.process.terminate()
        self.process.join()

    def __del__(self) -> None:
        with contextlib.suppress(Exception):
            if self.process.is_alive():
                self.shutdown()


class ThreadWorkerHandle(_WorkerHandleBase):
    """Handle of a worker running on a thread of this process
    (create_worker_thread).  A thread cannot be forced to end: one that
    outlasts the grace period is left running (it is a daemon thread) and
    logged."""

    def __init__(self, worker_id: int, conn: LocalChannel, thread: threading.Thread,
                 ready_event: threading.Event, errors: List[BaseException]) -> None:
        super().__init__(worker_id, conn, ready_event)
        self.thread = thread
        self._errors = errors

    def wait_ready(self, timeout: float = 60.0) -> None:
        if not self.ready_event.wait(timeout):
            raise TimeoutError(f"worker {self.worker_id} did not start in {timeout}s")
        if self._errors:
            raise RuntimeError(f"worker {self.worker_id} failed to start: {self._errors[0]}") \
                from self._errors[0]

    def _ended_within(self, timeout: float) -> bool:
        self.thread.join(timeout)
        return not self.thread.is_alive()

    def _force_end(self) -> None:
        flexkv_logger.warning(f"worker thread {self.worker_id} did not stop within "
                              f"{self.STOP_GRACE_S:.0f} s; leaving it running")


def _op_ids(src_block_ids: np.ndarray, dst_block_ids: np.ndarray,
            transfer_type: TransferType, from_host: TransferType, to_host: TransferType,
            worker: str) -> Tuple[np.ndarray, np.ndarray]:
    """(ids on the worker's other tier, host cache ids) of one op: the host
    cache is the source of `from_host` ops and the destination of `to_host`
    ops (worker.py:272-283 for the GPU tier, :538-550 for SSD).  Ids are
    int64 and pair up one to one; another op type is a ValueError."""
    assert src_block_ids.dtype == np.int64 and dst_block_ids.dtype == np.int64, \
        "block ids must be int64"
    assert len(src_block_ids) == len(dst_block_ids), "source and destination ids must pair up"
    if transfer_type == from_host:
        return dst_block_ids, src_block_ids
    if transfer_type == to_host:
        return src_block_ids, dst_block_ids
    raise ValueError(f"Invalid transfer type: {transfer_type} for {worker}")


class GPUCPUTransferWorker(TransferWorkerBase):
    """Moves KV blocks between one GPU's per-layer cache and the host cache
    (worker.py:207-342; single GPU, no TP)."""

    def __init__(self, worker_id: int, transfer_conn: Optional[Connection],
                 finished_ops_queue: Optional[Any],
                 gpu_blocks: Sequence[Union[TensorSharedHandle, torch.Tensor]],
                 cpu_blocks: Union[torch.Tensor, HostCacheSpec], gpu_kv_layout: KVCacheLayout,
                 cpu_kv_layout: KVCacheLayout, dtype: torch.dtype, gpu_device_id: int,
                 use_ce_transfer_h2d: bool = False, use_ce_transfer_d2h: bool = False,
                 transfer_sms_h2d: int = 8, transfer_sms_d2h: int = 8) -> None:
        super().__init__(worker_id, transfer_conn, finished_ops_queue)
        if gpu_kv_layout.type != KVCacheLayoutType.LAYERWISE:
            raise ValueError("Only layerwise layout is supported for GPU")
        if gpu_device_id != -1:
            torch.cuda.set_device(gpu_device_id)
        if isinstance(cpu_blocks, HostCacheSpec):
            cpu_blocks = cpu_blocks.allocate()
        host_register(cpu_blocks)

        def tensor(h):
            return h.get_tensor() if isinstance(h, TensorSharedHandle) else h

        # A layer given as a [K, V] pair (K and V separate allocations, each
        # [blocks, tokens, heads, dim]) uses the separate-pointer entry point.
        self.separate_kv = isinstance(gpu_blocks[0], (list, tuple))
        kv = 1 if gpu_kv_layout.is_mla else 2
        if self.separate_kv:
            self.gpu_blocks = [[tensor(h) for h in pair] for pair in gpu_blocks]
            if any(len(pair) != kv for pair in self.gpu_blocks):
                raise ValueError(f"separate K/V layers need {kv} tensor(s) per layer")
            self.gpu_layer_ptrs = self._get_layer_ptrs(
                [t for pair in self.gpu_blocks for t in pair])
        else:
            self.gpu_blocks = [tensor(h) for h in gpu_blocks]
            self.gpu_layer_ptrs = self._get_layer_ptrs(self.gpu_blocks)
        self.cpu_tensor = cpu_blocks
        self.dtype = dtype
        self.is_mla = gpu_kv_layout.is_mla
        self.num_layers = gpu_kv_layout.num_layer
        per_layer = gpu_kv_layout.div_layer(self.num_layers)
        es = dtype.itemsize
        self.chunk_size_in_bytes = per_layer.get_chunk_size() * es
        self.gpu_kv_stride_in_bytes = per_layer.get_kv_stride() * es
        self.gpu_block_stride_in_bytes = per_layer.get_block_stride() * es
        self.cpu_layer_stride_in_bytes = cpu_kv_layout.get_layer_stride() * es
        self.cpu_kv_stride_in_bytes = cpu_kv_layout.get_kv_stride() * es
        self.cpu_block_stride_in_bytes = cpu_kv_layout.get_block_stride() * es
        self.transfer_stream = torch.cuda.Stream()
        self._stream_handle = self.transfer_stream.cuda_stream
        self.transfer_sms_h2d = transfer_sms_h2d
        self.transfer_sms_d2h = transfer_sms_d2h
        self.use_ce_transfer_h2d = use_ce_transfer_h2d
        self.use_ce_transfer_d2h = use_ce_transfer_d2h
        if use_ce_transfer_h2d or use_ce_transfer_d2h:
            # staging, copy engines and their signals set up now, not in the
            # first op (extension; the reference's worker has nothing to set up)
            _lib.prepare(torch.cuda.current_device())

    def _transfer_impl(self, src_block_ids: np.ndarray, dst_block_ids: np.ndarray,
                       transfer_type: TransferType, layer_id: int, layer_granularity: int,
                       **kwargs: Any) -> None:
        gpu_ids, cpu_ids = _op_ids(src_block_ids, dst_block_ids, transfer_type,
                                   TransferType.H2D, TransferType.D2H, "GPUCPUTransferWorker")
        if transfer_type == TransferType.H2D:
            use_ce, sms = self.use_ce_transfer_h2d, self.transfer_sms_h2d
        else:
            use_ce, sms = self.use_ce_transfer_d2h, self.transfer_sms_d2h
        if len(gpu_ids) == 0:
            return
        if layer_id < 0 or layer_granularity < 1 or layer_id + layer_granularity > self.num_layers:
            raise ValueError(f"layer range [{layer_id}, {layer_id + layer_granularity}) is outside "
                             f"[0, {self.num_layers})")
        # The library reads ids and layer pointers on the host and stages them
        # itself, so ordinary host tensors do (the reference pins them because
        # its kernel reads them, worker.py:285-295).
        gpu_id_t = torch.from_numpy(np.ascontiguousarray(gpu_ids))
        cpu_id_t = torch.from_numpy(np.ascontiguousarray(cpu_ids))
        if self.separate_kv:
            kv = 1 if self.is_mla else 2
            ptrs = self.gpu_layer_ptrs[layer_id * kv:(layer_id + layer_granularity) * kv]
            transfer_kv_blocks_kv_ptrs(
                gpu_id_t, ptrs, self.gpu_block_stride_in_bytes, cpu_id_t, self.cpu_tensor,
                self.cpu_kv_stride_in_bytes, self.cpu_layer_stride_in_bytes,
                self.cpu_block_stride_in_bytes, self.chunk_size_in_bytes, layer_id, sms,
                transfer_type == TransferType.H2D, use_ce, self.is_mla,
                stream=kwargs.get("stream"))
            return
        layer_ptrs = self.gpu_layer_ptrs[layer_id:layer_id + layer_granularity]
        transfer_kv_blocks(gpu_id_t, layer_ptrs, self.gpu_kv_stride_in_bytes,
                           self.gpu_block_stride_in_bytes, cpu_id_t, self.cpu_tensor,
                           self.cpu_kv_stride_in_bytes, self.cpu_layer_stride_in_bytes,
                           self.cpu_block_stride_in_bytes, self.chunk_size_in_bytes, layer_id,
                           sms, transfer_type == TransferType.H2D, use_ce, self.is_mla,
                           stream=kwargs.get("stream"))

    def launch_transfer(self, transfer_op: WorkerTransferOp) -> None:
        layer_id = 0 if transfer_op.layer_id == -1 else transfer_op.layer_id
        granularity = self.num_layers if transfer_op.layer_granularity == -1 \
            else transfer_op.layer_granularity
        # the transfer runs on the worker's own stream (worker.py:323), passed
        # to the call instead of made current for it
        start = time.time()
        self._transfer_impl(transfer_op.src_block_ids, transfer_op.dst_block_ids,
                            transfer_op.transfer_type, layer_id, granularity,
                            stream=self._stream_handle)
        end = time.time()
        kv_dim = 1 if self.is_mla else 2
        size = self.chunk_size_in_bytes * granularity * len(transfer_op.src_block_ids) * kv_dim
        self._log_transfer_performance(transfer_op, size, start, end)


class tpGPUCPUTransferWorker(TransferWorkerBase):
    """Moves KV blocks between the GPU caches of one tensor-parallel group
    and the host cache (worker.py:344-480): ``gpu_blocks[r]`` is rank r's
    per-layer cache (its head slice), and every op moves the same blocks on
    all ranks at once through a c_ext.TPTransferThreadGroup, rank r into bytes
    [r * chunk, (r + 1) * chunk) of each host chunk.  Ranks may share a GPU."""

    def __init__(self, worker_id: int, transfer_conn: Optional[Connection],
                 finished_ops_queue: Optional[Any],
                 gpu_blocks: Sequence[Sequence[Union[TensorSharedHandle, torch.Tensor]]],
                 cpu_blocks: Union[torch.Tensor, HostCacheSpec], gpu_kv_layout: KVCacheLayout,
                 cpu_kv_layout: KVCacheLayout, dtype: torch.dtype, tp_group_size: int,
                 dp_group_id: int, use_ce_transfer_h2d: bool = False,
                 use_ce_transfer_d2h: bool = False, transfer_sms_h2d: int = 8,
                 transfer_sms_d2h: int = 8) -> None:
        super().__init__(worker_id, transfer_conn, finished_ops_queue)
        if len(gpu_blocks) != tp_group_size:
            raise ValueError(f"gpu_blocks holds {len(gpu_blocks)} ranks, the TP group "
                             f"{tp_group_size}")
        if gpu_kv_layout.type != KVCacheLayoutType.LAYERWISE:
            raise ValueError("Only layerwise layout is supported for GPU")
        if isinstance(cpu_blocks, HostCacheSpec):
            cpu_blocks = cpu_blocks.allocate()
        host_register(cpu_blocks)

        def tensor(h):
            return h.get_tensor() if isinstance(h, TensorSharedHandle) else h

        self.gpu_blocks = [[tensor(h) for h in rank] for rank in gpu_blocks]
        self.cpu_tensor = cpu_blocks
        self.dtype = dtype
        self.is_mla = gpu_kv_layout.is_mla
        self.num_gpus = len(self.gpu_blocks)
        self.tp_group_size = tp_group_size
        self.dp_group_id = dp_group_id
        self.num_layers = gpu_kv_layout.num_layer
        per_layer = gpu_kv_layout.div_layer(self.num_layers)
        es = dtype.itemsize
        self.gpu_chunk_size_in_bytes = per_layer.get_chunk_size() * es
        self.gpu_kv_stride_in_bytes = per_layer.get_kv_stride() * es
        self.gpu_block_stride_in_bytes = per_layer.get_block_stride() * es
        self.cpu_chunk_size_in_bytes = cpu_kv_layout.get_chunk_size() * es
        self.cpu_layer_stride_in_bytes = cpu_kv_layout.get_layer_stride() * es
        self.cpu_kv_stride_in_bytes = cpu_kv_layout.get_kv_stride() * es
        self.cpu_block_stride_in_bytes = cpu_kv_layout.get_block_stride() * es
        width = 1 if self.is_mla else tp_group_size
        if self.cpu_chunk_size_in_bytes != width * self.gpu_chunk_size_in_bytes:
            raise ValueError(f"the host chunk ({self.cpu_chunk_size_in_bytes} B) must hold "
                             f"{width} rank chunk(s) of {self.gpu_chunk_size_in_bytes} B")
        self.transfer_sms_h2d = transfer_sms_h2d
        self.transfer_sms_d2h = transfer_sms_d2h
        self.use_ce_transfer_h2d = use_ce_transfer_h2d
        self.use_ce_transfer_d2h = use_ce_transfer_d2h
        if use_ce_transfer_h2d or use_ce_transfer_d2h:
            for dev in sorted({b[0].device.index for b in self.gpu_blocks}):
                _lib.prepare(dev)
        self.tp_transfer_thread_group = TPTransferThreadGroup(
            self.num_gpus, self.gpu_blocks, cpu_blocks, dp_group_id)

    def _transfer_impl(self, src_block_ids: np.ndarray, dst_block_ids: np.ndarray,
                       transfer_type: TransferType, layer_id: int, layer_granularity: int,
                       **kwargs: Any) -> None:
        gpu_ids, cpu_ids = _op_ids(src_block_ids, dst_block_ids, transfer_type,
                                   TransferType.H2D, TransferType.D2H, "tpGPUCPUTransferWorker")
        if transfer_type == TransferType.H2D:
            use_ce, sms = self.use_ce_transfer_h2d, self.transfer_sms_h2d
        else:
            use_ce, sms = self.use_ce_transfer_d2h, self.transfer_sms_d2h
        if len(gpu_ids) == 0:
            return
        self.tp_transfer_thread_group.tp_group_transfer(
            torch.from_numpy(np.ascontiguousarray(gpu_ids)), self.gpu_kv_stride_in_bytes,
            self.gpu_block_stride_in_bytes, self.gpu_chunk_size_in_bytes,
            torch.from_numpy(np.ascontiguousarray(cpu_ids)), self.cpu_kv_stride_in_bytes,
            self.cpu_layer_stride_in_bytes, self.cpu_block_stride_in_bytes,
            self.cpu_chunk_size_in_bytes, sms, transfer_type == TransferType.H2D, use_ce,
            layer_id, layer_granularity, self.is_mla)

    def launch_transfer(self, transfer_op: WorkerTransferOp) -> None:
        layer_id = 0 if transfer_op.layer_id == -1 else transfer_op.layer_id
        granularity = self.num_layers if transfer_op.layer_granularity == -1 \
            else transfer_op.layer_granularity
        start = time.time()
        self._transfer_impl(transfer_op.src_block_ids, transfer_op.dst_block_ids,
                            transfer_op.transfer_type, layer_id, granularity)
        end = time.time()
        kv_dim = 1 if self.is_mla else 2
        size = self.cpu_chunk_size_in_bytes * granularity * len(transfer_op.src_block_ids) * kv_dim
        self._log_transfer_performance(transfer_op, size, start, end)

    def close(self) -> None:
        self.tp_transfer_thread_group.close()


class CPUSSDDiskTransferWorker(TransferWorkerBase):
    """Moves KV blocks between the host cache and the SSD cache files
    (worker.py:482-602): H2DISK writes host blocks to SSD blocks, DISK2H
    reads them back.  The SSD layout is split over all files
    (div_block(num_files, padding=True)) for its layer and K/V strides; the
    block stride is the host layout's, so both layouts must be the same
    type.  Host code only: it needs no device."""

    def __init__(self, worker_id: int, transfer_conn: Optional[Connection],
                 finished_ops_queue: Optional[Any],
                 cpu_blocks: Union[torch.Tensor, HostCacheSpec],
                 ssd_files: Dict[int, List[str]], cpu_kv_layout: KVCacheLayout,
                 ssd_kv_layout: KVCacheLayout, dtype: torch.dtype, num_blocks_per_file: int,
                 cache_config: Any = None) -> None:
        super().__init__(worker_id, transfer_conn, finished_ops_queue)
        if cpu_kv_layout.type != ssd_kv_layout.type:
            raise ValueError("no support for different CPU and SSD KV cache layout type")
        if isinstance(cpu_blocks, HostCacheSpec):   # a worker in its own process
            cpu_blocks = cpu_blocks.allocate()
        self.ssd_files = ssd_files
        self.num_blocks_per_file = num_blocks_per_file
        self.num_files = sum(len(v) for v in ssd_files.values())
        self.num_layers = cpu_kv_layout.num_layer
        self.num_cpu_blocks = cpu_kv_layout.num_block
        self.num_ssd_blocks = ssd_kv_layout.num_block
        self.round_robin = 1
        self.dtype = dtype
        self.cpu_tensor = cpu_blocks
        self.is_mla = cpu_kv_layout.is_mla
        per_file = ssd_kv_layout.div_block(self.num_files, padding=True)
        es = dtype.itemsize
        self.chunk_size_in_bytes = cpu_kv_layout.get_chunk_size() * es
        self.block_stride_in_bytes = cpu_kv_layout.get_block_stride() * es
        self.cpu_kv_stride_in_bytes = cpu_kv_layout.get_kv_stride() * es
        self.cpu_layer_stride_in_bytes = cpu_kv_layout.get_layer_stride() * es
        self.ssd_kv_stride_in_bytes = per_file.get_kv_stride() * es
        self.ssd_layer_stride_in_bytes = per_file.get_layer_stride() * es
        self.num_threads_per_device = getattr(cache_config, "ssd_threads_per_device", 32)
        try:
            self.ioctx = SSDIOCTX(ssd_files, len(ssd_files),
                                  getattr(cache_config, "ssd_cache_iouring_entries", 0),
                                  getattr(cache_config, "ssd_cache_iouring_flags", 0))
        except Exception as e:
            flexkv_logger.error(f"Error setting ssd ioctx: {e}")
            raise RuntimeError("SSD Worker init failed") from e

    def _transfer_impl(self, src_block_ids: np.ndarray, dst_block_ids: np.ndarray,
                       transfer_type: TransferType, layer_id: int, layer_granularity: int,
                       **kwargs: Any) -> None:
        ssd_ids, cpu_ids = _op_ids(src_block_ids, dst_block_ids, transfer_type,
                                   TransferType.H2DISK, TransferType.DISK2H,
                                   "CPUSSDDiskTransferWorker")
        if len(ssd_ids) == 0:
            return
        if layer_id < 0 or layer_granularity < 1 or layer_id + layer_granularity > self.num_layers:
            raise ValueError(f"layer range [{layer_id}, {layer_id + layer_granularity}) is outside "
                             f"[0, {self.num_layers})")
        # a write past a file's end would grow the file, a read past it fails:
        # reject ids outside either cache up front
        for name, ids, limit in (("ssd", ssd_ids, self.num_ssd_blocks),
                                 ("cpu", cpu_ids, self.num_cpu_blocks)):
            if ids.min() < 0 or ids.max() >= limit:
                raise ValueError(f"{name} block id out of range [0, {limit})")
        transfer_kv_blocks_ssd(
            ioctx=self.ioctx,
            cpu_layer_id_list=torch.arange(layer_id, layer_id + layer_granularity,
                                           dtype=torch.int32),
            cpu_tensor_ptr=self.cpu_tensor.data_ptr(),
            ssd_block_ids=torch.from_numpy(np.ascontiguousarray(ssd_ids)),
            cpu_block_ids=torch.from_numpy(np.ascontiguousarray(cpu_ids)),
            cpu_layer_stride_in_bytes=self.cpu_layer_stride_in_bytes,
            cpu_kv_stride_in_bytes=self.cpu_kv_stride_in_bytes,
            ssd_layer_stride_in_bytes=self.ssd_layer_stride_in_bytes,
            ssd_kv_stride_in_bytes=self.ssd_kv_stride_in_bytes,
            chunk_size_in_bytes=self.chunk_size_in_bytes,
            block_stride_in_bytes=self.block_stride_in_bytes,
            is_read=transfer_type == TransferType.DISK2H,
            num_blocks_per_file=self.num_blocks_per_file,
            round_robin=self.round_robin,
            num_threads_per_device=self.num_threads_per_device,
            is_mla=self.is_mla)

    def launch_transfer(self, transfer_op: WorkerTransferOp) -> None:
        layer_id = 0 if transfer_op.layer_id == -1 else transfer_op.layer_id
        granularity = self.num_layers if transfer_op.layer_granularity == -1 \
            else transfer_op.layer_granularity
        start = time.time()
        self._transfer_impl(transfer_op.src_block_ids, transfer_op.dst_block_ids,
                            transfer_op.transfer_type, layer_id, granularity)
        end = time.time()
        kv_dim = 1 if self.is_mla else 2
        size = self.chunk_size_in_bytes * granularity * len(transfer_op.src_block_ids) * kv_dim
        self._log_transfer_performance(transfer_op, size, start, end)

    def close(self) -> None:
        self.ioctx.close()
