"""Transfer-graph scheduler (role of flexkv/transfer/scheduler.py:7-55).

schedule(finished_ops) retires finished ops and returns
(completed_graph_ids, next_ops).  Unlike the reference it iterates to a fixed
point, so a VIRTUAL op that completes inside one call also releases its
successors in that call, and it accepts an optional `can_start_early` hook
(see TransferOpGraph.take_ready_ops) to hand out ops whose remaining
predecessors are already queued on the same in-order worker.
"""
from __future__ import annotations

from collections import OrderedDict
from typing import Callable, List, Optional, Tuple

from ..common.transfer import TransferOp, TransferOpGraph, TransferType


class TransferScheduler:
    def __init__(self, can_start_early: Optional[Callable] = None) -> None:
        self._transfer_graphs: "OrderedDict[int, TransferOpGraph]" = OrderedDict()
        self._can_start_early = can_start_early

    def add_transfer_graph(self, graph: TransferOpGraph) -> None:
        self._transfer_graphs[graph.graph_id] = graph

    @property
    def num_graphs(self) -> int:
        return len(self._transfer_graphs)

    def schedule(self, finished_ops: List[TransferOp]) -> Tuple[List[int], List[TransferOp]]:
        for op in finished_ops:
            g = self._transfer_graphs.get(op.graph_id)
            if g is not None:
                g.mark_completed(op.op_id)
        next_ops: List[TransferOp] = []
        progress = True
        while progress:
            progress = False
            for g in self._transfer_graphs.values():
                for op_id in g.take_ready_ops(self._can_start_early):
                    op = g._op_map[op_id]
                    next_ops.append(op)
                    if op.transfer_type == TransferType.VIRTUAL:
                        g.mark_completed(op_id)
                        progress = True
        done = [gid for gid, g in self._transfer_graphs.items() if g.all_transfer_ops_completed()]
        for gid in done:
            del self._transfer_graphs[gid]
        return done, next_ops
