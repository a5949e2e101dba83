"""Transfer op records and graphs.

Same names, fields and checks as the reference's op types
(flexkv/common/transfer.py:9-236): TransferType, DeviceType, TransferDescriptor
(1-D int64 physical block ids), TransferOp (globally numbered; src and dst
id lists must have equal length except for VIRTUAL ops) and TransferOpGraph.
"""
from __future__ import annotations

import itertools
import threading
from dataclasses import dataclass, field
from enum import Enum
from typing import ClassVar, Dict, List, Set

import torch


class DeviceType(Enum):
    CPU = 0
    GPU = 1
    SSD = 2
    REMOTE = 3


class TransferType(Enum):
    H2D = "H2D"
    D2H = "D2H"
    DISK2H = "DISK2H"
    H2DISK = "H2DISK"
    DISK2D = "DISK2D"
    D2DISK = "D2DISK"
    REMOTE2H = "REMOTE2H"
    H2REMOTE = "H2REMOTE"
    VIRTUAL = "Virtual"


class TransferOpStatus(Enum):
    PENDING = 0
    RUNNING = 1
    COMPLETED = 2


def _empty_ids() -> torch.Tensor:
    return torch.empty(0, dtype=torch.int64)


@dataclass
class TransferDescriptor:
    device_type: DeviceType = DeviceType.CPU
    device_id: int = 0
    physical_block_ids: torch.Tensor = field(default_factory=_empty_ids)

    def __post_init__(self) -> None:
        ids = self.physical_block_ids
        if ids.ndim != 1:
            raise ValueError(f"physical_block_ids must be 1-D, got shape {tuple(ids.shape)}")
        if ids.dtype != torch.int64:
            raise ValueError(f"physical_block_ids must be int64, got {ids.dtype}")


@dataclass
class TransferOp:
    _ids: ClassVar = itertools.count()
    _lock: ClassVar[threading.Lock] = threading.Lock()

    graph_id: int
    transfer_type: TransferType
    layer_id: int
    layer_granularity: int
    src_descriptor: TransferDescriptor = field(default_factory=TransferDescriptor)
    dst_descriptor: TransferDescriptor = field(default_factory=TransferDescriptor)
    predecessors: Set[int] = field(default_factory=set)
    successors: Set[int] = field(default_factory=set)
    status: TransferOpStatus = TransferOpStatus.PENDING
    dp_id: int = 0
    op_id: int = field(init=False)

    def __post_init__(self) -> None:
        if self.transfer_type != TransferType.VIRTUAL and \
                self.src_descriptor.physical_block_ids.numel() != \
                self.dst_descriptor.physical_block_ids.numel():
            raise ValueError("src_descriptor and dst_descriptor must have the same number "
                             "of physical blocks")
        with TransferOp._lock:
            self.op_id = next(TransferOp._ids)


class TransferOpGraph:
    """A DAG of TransferOps for one request (flexkv/common/transfer.py:77-236).

    Same interface as the reference: ops are added with add_transfer_op /
    add_virtual_op, ordered with add_dependency(successor, predecessor),
    handed out by take_ready_ops (which marks them RUNNING) and retired by
    mark_completed.  Virtual ops carry no data; one added with
    need_trigger=True completes only when trigger_op is called.  Internally
    each op keeps the set of predecessors that have not completed yet.
    """

    _ids = itertools.count()
    _lock = threading.Lock()

    def __init__(self) -> None:
        with TransferOpGraph._lock:
            self.graph_id = next(TransferOpGraph._ids)
        self._op_map: Dict[int, TransferOp] = {}
        self._waiting_trigger: Set[int] = set()

    def set_graph_id(self, graph_id: int) -> None:
        self.graph_id = graph_id
        for op in self._op_map.values():
            op.graph_id = graph_id

    @classmethod
    def create_empty_graph(cls) -> "TransferOpGraph":
        return cls()

    def add_transfer_op(self, op: TransferOp) -> None:
        op.graph_id = self.graph_id
        self._op_map[op.op_id] = op

    def add_virtual_op(self, op: TransferOp, need_trigger: bool = False) -> None:
        op.graph_id = self.graph_id
        op.transfer_type = TransferType.VIRTUAL
        self._op_map[op.op_id] = op
        if need_trigger:
            self._waiting_trigger.add(op.op_id)

    def trigger_op(self, op_id: int) -> None:
        """Complete a virtual op that was waiting for an external trigger."""
        self._waiting_trigger.remove(op_id)
        op = self._op_map[op_id]
        op.status = TransferOpStatus.RUNNING
        self.mark_completed(op_id)

    def add_dependency(self, successor_op_id: int, predecessor_op_id: int) -> None:
        """`successor_op_id` may start only after `predecessor_op_id` completed."""
        assert successor_op_id in self._op_map and predecessor_op_id in self._op_map
        self._op_map[successor_op_id].predecessors.add(predecessor_op_id)
        self._op_map[predecessor_op_id].successors.add(successor_op_id)

    def mark_completed(self, op_id: int) -> None:
        op = self._op_map.get(op_id)
        if op is None:
            return
        assert op.status == TransferOpStatus.RUNNING, \
            f"op {op_id} completed while {op.status.name}"
        op.status = TransferOpStatus.COMPLETED
        for succ in op.successors:
            self._op_map[succ].predecessors.discard(op_id)

    def take_ready_ops(self, can_start_early=None) -> List[int]:
        """Ids of PENDING ops with no incomplete predecessor, now RUNNING.

        `can_start_early(op, pending_predecessors)` may also admit an op whose
        remaining predecessors are all RUNNING (e.g. queued on the same
        in-order worker); the reference has no such hook."""
        ready = []
        for op_id, op in self._op_map.items():
            if op.status != TransferOpStatus.PENDING or op_id in self._waiting_trigger:
                continue
            if not op.predecessors or (can_start_early is not None and all(
                    self._op_map[p].status == TransferOpStatus.RUNNING for p in op.predecessors)
                    and can_start_early(op, [self._op_map[p] for p in op.predecessors])):
                op.status = TransferOpStatus.RUNNING
                ready.append(op_id)
        return ready

    def all_transfer_ops_completed(self) -> bool:
        return all(op.status == TransferOpStatus.COMPLETED for op in self._op_map.values())

    @property
    def num_ops(self) -> int:
        return len(self._op_map)

    def bind_to_dp_group(self, dp_id: int) -> None:
        for op in self._op_map.values():
            op.dp_id = dp_id

    def print_op_map(self) -> None:
        print(f"Transfer Graph {self.graph_id}:")
        ids = sorted(self._op_map)
        for n, op_id in enumerate(ids):
            op = self._op_map[op_id]
            last = n == len(ids) - 1
            print(f"{'└── ' if last else '├── '}Op {op_id} ({op.transfer_type.name}) "
                  f"[{op.status.name.capitalize()}]")
            if op.transfer_type == TransferType.VIRTUAL:
                continue
            pad = "    " if last else "│   "
            succ = ", ".join(str(s) for s in sorted(op.successors)) or "none"
            print(f"{pad}└── successors: {succ}; layers {op.layer_id} - "
                  f"{op.layer_id + op.layer_granularity}; "
                  f"{op.src_descriptor.device_type.name} -> {op.dst_descriptor.device_type.name}, "
                  f"{op.src_descriptor.physical_block_ids.numel()} blocks")
