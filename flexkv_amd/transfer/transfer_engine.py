"""Transfer engine: runs transfer graphs on workers (role of
flexkv/transfer/transfer_engine.py:42-307, GPU<->CPU and CPU<->SSD tiers).

Same interface as the reference: TransferEngine(gpu_handles, model_config,
cache_config, cpu_handle, ssd_handle, ...), start(),
submit_transfer_graph(graph), get_completed_graphs_and_ops(timeout) ->
[(graph_id, op_id)] with op_id -1 for a finished graph, shutdown().  The
GPU<->CPU ops of a data-parallel group (op.dp_id) go to that group's worker;
with an SSD handle, one CPU<->SSD worker takes the DISK2H ops and another the
H2DISK ops (transfer_engine.py:129-153).

Differences:
  * workers run on threads of this process by default (worker_mode="thread"):
    the transfer releases the GIL, and the pinned host cache needs no
    inter-process sharing; worker_mode="process" spawns them as the
    reference does, each allocating its own pinned host cache;
  * thread mode gives each group two GPU<->CPU workers, one for H2D and one
    for D2H, so that a get and a put overlap on the full-duplex link (the
    reference's single worker runs them in turn); a process worker owns its
    host cache, so process mode keeps one per group;
  * the scheduler thread blocks on one event queue (new graphs and finished
    ops) instead of polling every millisecond;
  * eager_dispatch: an op whose unfinished predecessors are all already
    queued on the same worker is handed to that worker at once; the worker
    runs its ops in submission order on one stream, so the dependency holds
    without a scheduler round trip between layer groups;
  * the SSD workers share the engine process's host cache, so an SSD tier
    needs worker_mode="thread".
"""
from __future__ import annotations

import queue
import threading
from typing import Dict, List, Optional, Tuple

import torch

from ..common.config import CacheConfig, ModelConfig
from ..common.debug import flexkv_logger
from ..common.transfer import TransferOp, TransferOpGraph, TransferType
from ..storage.allocator import HostCacheSpec, StorageHandle
from .scheduler import TransferScheduler
from .worker import (CPUSSDDiskTransferWorker, FinishedOpsChannel, GPUCPUTransferWorker,
                     tpGPUCPUTransferWorker)

_GPU_CPU = (TransferType.H2D, TransferType.D2H)
_CPU_SSD = (TransferType.DISK2H, TransferType.H2DISK)


class TransferEngine:
    def __init__(self, gpu_handles: List[StorageHandle], model_config: ModelConfig,
                 cache_config: CacheConfig, cpu_handle: Optional[StorageHandle] = None,
                 ssd_handle: Optional[StorageHandle] = None,
                 remote_handle: Optional[StorageHandle] = None,
                 worker_mode: str = "thread", eager_dispatch: bool = True) -> None:
        if worker_mode not in ("thread", "process"):
            raise ValueError(f"worker_mode must be 'thread' or 'process', got {worker_mode!r}")
        if remote_handle is not None:
            raise NotImplementedError("the remote tier is not provided")
        if ssd_handle is not None and worker_mode != "thread":
            raise NotImplementedError("the SSD tier shares the engine's host cache and needs "
                                      "worker_mode='thread'")
        assert len(gpu_handles) == model_config.dp_size * model_config.tp_size
        self.model_config = model_config
        self.cache_config = cache_config
        self.gpu_handles = gpu_handles
        self._cpu_handle = cpu_handle
        self._ssd_handle = ssd_handle
        self._ssd_workers: Dict[TransferType, object] = {}
        self.worker_mode = worker_mode
        self.eager_dispatch = eager_dispatch
        self.scheduler = TransferScheduler(self._same_worker if eager_dispatch else None)
        self._events: "queue.Queue" = queue.Queue()
        self.completed_queue: "queue.Queue[Tuple[int, int]]" = queue.Queue()
        self.op_id_to_op: Dict[int, TransferOp] = {}
        self._running = False
        self._workers: List = []
        self._gpu_workers: Dict[tuple, object] = {}
        self._mp_finished = None
        self._forwarder: Optional[threading.Thread] = None

    # -- worker routing ---------------------------------------------------
    def _worker_key(self, op: TransferOp):
        if op.transfer_type in _GPU_CPU:
            # thread workers: one per GPU and direction, so that a put (D2H)
            # and a get (H2D) on one GPU overlap (PCIe is full duplex); a
            # worker process owns its host cache, so there is one per GPU
            split = self.worker_mode == "thread"
            return ("gpucpu", op.dp_id, op.transfer_type if split else None)
        return (op.transfer_type, 0)

    def _same_worker(self, op: TransferOp, pending_predecessors: List[TransferOp]) -> bool:
        if op.transfer_type == TransferType.VIRTUAL:
            return False
        key = self._worker_key(op)
        return all(p.transfer_type != TransferType.VIRTUAL and self._worker_key(p) == key
                   for p in pending_predecessors)

    # -- lifecycle ----------------------------------------------------------
    def _init_workers(self) -> None:
        if self._running:
            return
        if self._cpu_handle is None:
            raise ValueError("a CPU storage handle is required")
        cfg = self.cache_config
        tp = self.model_config.tp_size
        for i in range(self.model_config.dp_size):
            # a data-parallel group's ranks are handles [i * tp, (i + 1) * tp)
            # (transfer_engine.py:105-122)
            group = self.gpu_handles[i * tp:(i + 1) * tp]
            g = group[0]
            common = dict(gpu_kv_layout=g.kv_layout, cpu_kv_layout=self._cpu_handle.kv_layout,
                          dtype=g.dtype,
                          use_ce_transfer_h2d=cfg.use_ce_transfer_h2d,
                          use_ce_transfer_d2h=cfg.use_ce_transfer_d2h,
                          transfer_sms_h2d=cfg.transfer_sms_h2d,
                          transfer_sms_d2h=cfg.transfer_sms_d2h)
            if tp == 1:
                cls = GPUCPUTransferWorker
                common["gpu_device_id"] = g.gpu_device_id if g.gpu_device_id is not None else i
            else:
                cls = tpGPUCPUTransferWorker
                common.update(tp_group_size=tp, dp_group_id=i)

            def blocks(thread: bool):
                lists = [h.get_tensor_list() if thread else h.get_tensor_handle_list()
                         for h in group]
                return lists[0] if tp == 1 else lists
            if self.worker_mode == "thread":
                for kind in (TransferType.H2D, TransferType.D2H):
                    w = cls.create_worker_thread(
                        i, self._events, gpu_blocks=blocks(True),
                        cpu_blocks=self._cpu_handle.get_tensor(), **common)
                    w.wait_ready(60)
                    self._gpu_workers[("gpucpu", i, kind)] = w
                    self._workers.append(w)
            else:
                if self._mp_finished is None:
                    self._mp_finished = FinishedOpsChannel()
                w = cls.create_worker(
                    i, self._mp_finished, gpu_blocks=blocks(False),
                    cpu_blocks=HostCacheSpec(self._cpu_handle.kv_layout, self._cpu_handle.dtype),
                    **common)
                if not w.ready_event.wait(120):
                    raise TimeoutError(f"worker {i} did not start")
                self._gpu_workers[("gpucpu", i, None)] = w
                self._workers.append(w)
        if self._ssd_handle is not None:
            common = dict(cpu_blocks=self._cpu_handle.get_tensor(),
                          ssd_files=self._ssd_handle.get_file_list(),
                          cpu_kv_layout=self._cpu_handle.kv_layout,
                          ssd_kv_layout=self._ssd_handle.kv_layout,
                          dtype=self._cpu_handle.dtype,
                          num_blocks_per_file=self._ssd_handle.num_blocks_per_file,
                          cache_config=cfg)
            for wid, kind in ((10, TransferType.DISK2H), (11, TransferType.H2DISK)):
                w = CPUSSDDiskTransferWorker.create_worker_thread(wid, self._events, **common)
                w.wait_ready(60)
                self._ssd_workers[kind] = w
        self._running = True
        if self._mp_finished is not None:
            self._forwarder = threading.Thread(target=self._forward_finished, daemon=True)
            self._forwarder.start()
        self._scheduler_thread = threading.Thread(target=self._scheduler_loop, daemon=True,
                                                  name="flexkv-scheduler")
        self._scheduler_thread.start()
        flexkv_logger.info(f"TransferEngine running with {len(self._workers)} "
                           f"{self.worker_mode} worker(s)")

    def start(self) -> None:
        self._init_workers()

    def _forward_finished(self) -> None:
        while self._running:
            try:
                op_id = self._mp_finished.get(timeout=0.05)
            except queue.Empty:
                continue
            self._events.put(op_id)

    def _scheduler_loop(self) -> None:
        while self._running:
            try:
                self._schedule_once()
            except Exception as e:  # keep scheduling other graphs
                flexkv_logger.error(f"Error in scheduler loop: {e}")

    def _schedule_once(self) -> None:
        """Take every pending event (new graphs, finished op ids), schedule, dispatch."""
        try:
            first = self._events.get(timeout=0.05)
        except queue.Empty:
            return
        items = [first]
        while True:
            try:
                items.append(self._events.get_nowait())
            except queue.Empty:
                break
        finished: List[TransferOp] = []
        for item in items:
            if isinstance(item, TransferOpGraph):
                self.scheduler.add_transfer_graph(item)
            elif item is None:
                continue
            else:
                op = self.op_id_to_op.pop(item)
                self.completed_queue.put((op.graph_id, op.op_id))
                finished.append(op)
        done_graphs, next_ops = self.scheduler.schedule(finished)
        for op in next_ops:
            if op.transfer_type == TransferType.VIRTUAL:
                self.completed_queue.put((op.graph_id, op.op_id))
            else:
                self.op_id_to_op[op.op_id] = op
                self._assign_op_to_worker(op)
        for gid in done_graphs:
            self.completed_queue.put((gid, -1))

    def _assign_op_to_worker(self, op: TransferOp) -> None:
        if op.transfer_type in _GPU_CPU:
            self._gpu_workers[self._worker_key(op)].submit_transfer(op)
        elif op.transfer_type in _CPU_SSD and op.transfer_type in self._ssd_workers:
            self._ssd_workers[op.transfer_type].submit_transfer(op)
        else:
            raise ValueError(f"Unsupported transfer type: {op.transfer_type}")

    # -- public API ------------------------------------------------------------
    def submit_transfer_graph(self, transfer_graph: TransferOpGraph) -> None:
        self._events.put(transfer_graph)

    def get_completed_graphs_and_ops(self, timeout: Optional[float] = None
                                     ) -> List[Tuple[int, int]]:
        """Every (graph_id, op_id) completed so far; op_id -1 marks a finished
        graph.  Waits up to `timeout` for the first one."""
        out: List[Tuple[int, int]] = []
        try:
            out.append(self.completed_queue.get(timeout=timeout) if timeout
                       else self.completed_queue.get_nowait())
        except queue.Empty:
            return out
        while True:
            try:
                out.append(self.completed_queue.get_nowait())
            except queue.Empty:
                return out

    def shutdown(self) -> None:
        self._running = False
        self._events.put(None)
        if hasattr(self, "_scheduler_thread"):
            self._scheduler_thread.join(timeout=5)
        for w in self._workers + list(self._ssd_workers.values()):
            try:
                w.shutdown()
            except Exception as e:
                flexkv_logger.error(f"Error during worker shutdown: {e}")
        self._workers = []
        self._gpu_workers = {}
        self._ssd_workers = {}
        if self._forwarder is not None:
            self._forwarder.join(timeout=5)
        if self._mp_finished is not None and (self._forwarder is None
                                              or not self._forwarder.is_alive()):
            self._mp_finished.close()
            self._mp_finished = None
        if torch.cuda.is_available():
            torch.cuda.synchronize()
