"""Transfer op records for the GPU<->CPU path.

Same names, fields and checks as the reference's op types
(flexkv/common/transfer.py:9-75): TransferType, DeviceType, TransferDescriptor
(1-D int64 physical block ids) and TransferOp (globally numbered; src and dst
id lists must have equal length except for VIRTUAL ops).
"""
from __future__ import annotations

import itertools
import threading
from dataclasses import dataclass, field
from enum import Enum
from typing import ClassVar, Set

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
