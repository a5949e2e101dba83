"""Transfer-graph builders for a CPU-backed cache.

Same functions and graph shapes as the reference's
flexkv/cache/transfer_pattern.py:9-428 for the CPU tiers (the remote-storage
variants belong to a tier this package does not implement):

  read  (get):  [DISK2H ->] H2D, blocks split so that SSD-resident blocks
                are staged into the tail of the CPU block list first;
  write (put):  D2H [-> H2DISK];
  layer-wise:   every op split into layer groups, group i of an op after
                group i-1 of the same op, original dependencies kept per
                group.
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from ..common.transfer import (DeviceType, TransferDescriptor, TransferOp, TransferOpGraph,
                               TransferType)


def _op(graph: TransferOpGraph, kind: TransferType, src_dev: DeviceType, src_ids: torch.Tensor,
        dst_dev: DeviceType, dst_ids: torch.Tensor, layer_num: int, gpu_device_id: int = 0,
        layer_id: int = 0) -> TransferOp:
    op = TransferOp(
        graph_id=graph.graph_id, transfer_type=kind, layer_id=layer_id,
        layer_granularity=layer_num,
        src_descriptor=TransferDescriptor(src_dev, gpu_device_id if src_dev == DeviceType.GPU else 0,
                                          src_ids),
        dst_descriptor=TransferDescriptor(dst_dev, gpu_device_id if dst_dev == DeviceType.GPU else 0,
                                          dst_ids))
    graph.add_transfer_op(op)
    return op


def add_virtual_op_for_multiple_finished_ops(
        graph: TransferOpGraph, finished_ops_ids: List[int]) -> Tuple[TransferOpGraph, List[int]]:
    """With several end ops, add one VIRTUAL op after all of them and track
    that instead (transfer_pattern.py:9-25)."""
    if len(finished_ops_ids) <= 1:
        return graph, finished_ops_ids
    v = TransferOp(graph_id=graph.graph_id, transfer_type=TransferType.VIRTUAL, layer_id=-1,
                   layer_granularity=-1)
    graph.add_transfer_op(v)
    for op_id in finished_ops_ids:
        graph.add_dependency(v.op_id, op_id)
    return graph, [v.op_id]


# the reference's spelling, kept for callers that import it by that name
add_virtal_op_for_mutiple_finished_ops = add_virtual_op_for_multiple_finished_ops


def create_read_graph_cpu_storage(gpu_blocks: torch.Tensor, cpu_blocks: torch.Tensor,
                                  ssd_blocks: torch.Tensor, gpu_device_id: int = 0,
                                  layer_num: int = 1, graph: Optional[TransferOpGraph] = None
                                  ) -> Tuple[TransferOpGraph, List[int]]:
    """Graph for (SSD ->) CPU -> GPU.  The last len(ssd_blocks) CPU blocks
    are filled from SSD before their H2D; the rest go to the GPU directly
    (transfer_pattern.py:27-152).  Returns the graph and the op ids whose
    completion means the data is on the GPU."""
    assert len(gpu_blocks) == len(cpu_blocks) and len(gpu_blocks) > 0
    graph = TransferOpGraph() if graph is None else graph
    n, ns = len(cpu_blocks), len(ssd_blocks)
    if ns == 0:
        op = _op(graph, TransferType.H2D, DeviceType.CPU, cpu_blocks, DeviceType.GPU, gpu_blocks,
                 layer_num, gpu_device_id)
        return graph, [op.op_id]
    if ns >= n:
        disk = _op(graph, TransferType.DISK2H, DeviceType.SSD, ssd_blocks, DeviceType.CPU,
                   cpu_blocks, layer_num)
        h2d = _op(graph, TransferType.H2D, DeviceType.CPU, cpu_blocks, DeviceType.GPU, gpu_blocks,
                  layer_num, gpu_device_id)
        graph.add_dependency(h2d.op_id, disk.op_id)
        return graph, [h2d.op_id]
    ends = []
    disk = _op(graph, TransferType.DISK2H, DeviceType.SSD, ssd_blocks, DeviceType.CPU,
               cpu_blocks[n - ns:], layer_num)
    tail = _op(graph, TransferType.H2D, DeviceType.CPU, cpu_blocks[n - ns:], DeviceType.GPU,
               gpu_blocks[n - ns:], layer_num, gpu_device_id)
    graph.add_dependency(tail.op_id, disk.op_id)
    ends.append(tail.op_id)
    head = _op(graph, TransferType.H2D, DeviceType.CPU, cpu_blocks[:n - ns], DeviceType.GPU,
               gpu_blocks[:n - ns], layer_num, gpu_device_id)
    ends.append(head.op_id)
    return graph, ends


def create_write_graph_cpu_storage(gpu_blocks: torch.Tensor, cpu_blocks: torch.Tensor,
                                   ssd_blocks: torch.Tensor, gpu_device_id: int = 0,
                                   layer_num: int = 1, graph: Optional[TransferOpGraph] = None
                                   ) -> Tuple[TransferOpGraph, List[int]]:
    """Graph for GPU -> CPU (-> SSD): D2H into the last len(gpu_blocks) CPU
    blocks, then optionally H2DISK of the last len(ssd_blocks) CPU blocks
    (transfer_pattern.py:245-287).  Returns the graph and [D2H op id]."""
    graph = TransferOpGraph() if graph is None else graph
    n = len(gpu_blocks)
    d2h = _op(graph, TransferType.D2H, DeviceType.GPU, gpu_blocks, DeviceType.CPU,
              cpu_blocks[len(cpu_blocks) - n:], layer_num, gpu_device_id)
    if len(ssd_blocks) > 0:
        ns = len(ssd_blocks)
        disk = _op(graph, TransferType.H2DISK, DeviceType.CPU, cpu_blocks[len(cpu_blocks) - ns:],
                   DeviceType.SSD, ssd_blocks, layer_num)
        graph.add_dependency(disk.op_id, d2h.op_id)
    return graph, [d2h.op_id]


def convert_read_graph_to_layer_wise_graph(transfer_graph: TransferOpGraph,
                                           finished_ops_ids: List[int], layer_num: int,
                                           layer_granularity: int
                                           ) -> Tuple[TransferOpGraph, List[int]]:
    """Split every op into layer_num / layer_granularity ops over consecutive
    layer groups (transfer_pattern.py:370-428).  Group i of an op depends on
    group i-1 of the same op (VIRTUAL ops excepted) and on group i of each
    original predecessor.  Returns the new graph (same graph id) and, per
    group, the split of the first tracked op."""
    assert layer_num % layer_granularity == 0
    groups = layer_num // layer_granularity
    new = TransferOpGraph()
    new.set_graph_id(transfer_graph.graph_id)
    split = {}
    for op_id, op in transfer_graph._op_map.items():
        ids = []
        for g in range(groups):
            cp = TransferOp(graph_id=new.graph_id, transfer_type=op.transfer_type,
                            layer_id=g * layer_granularity, layer_granularity=layer_granularity,
                            src_descriptor=op.src_descriptor, dst_descriptor=op.dst_descriptor,
                            dp_id=op.dp_id)
            new.add_transfer_op(cp)
            ids.append(cp.op_id)
        split[op_id] = ids
    for op_id, op in transfer_graph._op_map.items():
        for succ in op.successors:
            for g in range(groups):
                new.add_dependency(split[succ][g], split[op_id][g])
        if op.transfer_type != TransferType.VIRTUAL:
            for g in range(1, groups):
                new.add_dependency(split[op_id][g], split[op_id][g - 1])
    return new, [split[finished_ops_ids[0]][g] for g in range(groups)]
