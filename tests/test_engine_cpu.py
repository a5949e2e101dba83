"""Transfer graphs, scheduler, graph builders and the engine's scheduling,
without a device (flexkv/common/transfer.py:77-236, transfer/scheduler.py,
transfer/transfer_engine.py, cache/transfer_pattern.py)."""
import time

import pytest
import torch

from flexkv_amd.cache.transfer_pattern import (add_virtual_op_for_multiple_finished_ops,
                                               convert_read_graph_to_layer_wise_graph,
                                               create_read_graph_cpu_storage,
                                               create_write_graph_cpu_storage)
from flexkv_amd.common.transfer import TransferOp, TransferOpGraph, TransferType
from flexkv_amd.transfer.scheduler import TransferScheduler


def ids(*v):
    return torch.tensor(v, dtype=torch.int64)


def _op(g, kind=TransferType.H2D, layer=0):
    op = TransferOp(graph_id=g.graph_id, transfer_type=kind, layer_id=layer, layer_granularity=1)
    g.add_transfer_op(op)
    return op


def test_graph_dependencies_and_completion():
    g = TransferOpGraph()
    a, b, c = _op(g), _op(g), _op(g)
    g.add_dependency(c.op_id, a.op_id)
    g.add_dependency(c.op_id, b.op_id)
    assert sorted(g.take_ready_ops()) == sorted([a.op_id, b.op_id])
    assert g.take_ready_ops() == []
    g.mark_completed(a.op_id)
    assert g.take_ready_ops() == []
    g.mark_completed(b.op_id)
    assert g.take_ready_ops() == [c.op_id]
    assert not g.all_transfer_ops_completed()
    g.mark_completed(c.op_id)
    assert g.all_transfer_ops_completed() and g.num_ops == 3
    with pytest.raises(AssertionError):
        g.mark_completed(c.op_id)


def test_virtual_and_trigger_ops():
    g = TransferOpGraph()
    a = _op(g)
    v = TransferOp(graph_id=0, transfer_type=TransferType.VIRTUAL, layer_id=-1, layer_granularity=-1)
    g.add_virtual_op(v, need_trigger=True)
    b = _op(g)
    g.add_dependency(b.op_id, v.op_id)
    s = TransferScheduler()
    s.add_transfer_graph(g)
    done, nxt = s.schedule([])
    assert [o.op_id for o in nxt] == [a.op_id] and done == []
    a.status  # running
    done, nxt = s.schedule([a])
    assert nxt == [] and done == []
    g.trigger_op(v.op_id)
    done, nxt = s.schedule([])
    assert [o.op_id for o in nxt] == [b.op_id]
    done, nxt = s.schedule([b])
    assert done == [g.graph_id] and s.num_graphs == 0


def test_scheduler_resolves_virtual_chains_in_one_call():
    g = TransferOpGraph()
    a = _op(g)
    v = TransferOp(graph_id=0, transfer_type=TransferType.VIRTUAL, layer_id=-1, layer_granularity=-1)
    g.add_transfer_op(v)
    b = _op(g)
    g.add_dependency(v.op_id, a.op_id)
    g.add_dependency(b.op_id, v.op_id)
    s = TransferScheduler()
    s.add_transfer_graph(g)
    _, nxt = s.schedule([])
    assert [o.op_id for o in nxt] == [a.op_id]
    _, nxt = s.schedule([a])
    assert [o.op_id for o in nxt] == [v.op_id, b.op_id]


def test_eager_hook_releases_same_worker_chains():
    g = TransferOpGraph()
    ops = [_op(g, layer=i) for i in range(4)]
    for i in range(1, 4):
        g.add_dependency(ops[i].op_id, ops[i - 1].op_id)
    plain = TransferScheduler()
    plain.add_transfer_graph(g)
    _, nxt = plain.schedule([])
    assert [o.op_id for o in nxt] == [ops[0].op_id]
    g2 = TransferOpGraph()
    ops2 = [_op(g2, layer=i) for i in range(4)]
    for i in range(1, 4):
        g2.add_dependency(ops2[i].op_id, ops2[i - 1].op_id)
    eager = TransferScheduler(lambda op, preds: True)
    eager.add_transfer_graph(g2)
    _, nxt = eager.schedule([])
    assert [o.op_id for o in nxt] == [o.op_id for o in ops2]
    done, _ = eager.schedule(ops2)
    assert done == [g2.graph_id]


def test_read_write_graph_shapes():
    g, ends = create_read_graph_cpu_storage(ids(0, 1, 2), ids(5, 6, 7), ids(), layer_num=4)
    assert g.num_ops == 1
    op = g._op_map[ends[0]]
    assert op.transfer_type == TransferType.H2D and op.layer_granularity == 4
    assert op.src_descriptor.physical_block_ids.tolist() == [5, 6, 7]
    g, ends = create_read_graph_cpu_storage(ids(0, 1, 2, 3), ids(4, 5, 6, 7), ids(9, 8))
    kinds = sorted(o.transfer_type.name for o in g._op_map.values())
    assert kinds == ["DISK2H", "H2D", "H2D"] and len(ends) == 2
    disk = [o for o in g._op_map.values() if o.transfer_type == TransferType.DISK2H][0]
    assert disk.dst_descriptor.physical_block_ids.tolist() == [6, 7]
    tail = [o for o in g._op_map.values() if disk.op_id in o.predecessors][0]
    assert tail.dst_descriptor.physical_block_ids.tolist() == [2, 3]
    g, ends = create_read_graph_cpu_storage(ids(0, 1), ids(4, 5), ids(9, 8))
    assert g.num_ops == 2 and len(ends) == 1
    g, ends = create_write_graph_cpu_storage(ids(3, 4), ids(7, 8, 9), ids(1))
    d2h = g._op_map[ends[0]]
    assert d2h.transfer_type == TransferType.D2H
    assert d2h.dst_descriptor.physical_block_ids.tolist() == [8, 9]
    h2disk = [o for o in g._op_map.values() if o.transfer_type == TransferType.H2DISK][0]
    assert h2disk.src_descriptor.physical_block_ids.tolist() == [9]
    assert d2h.op_id in h2disk.predecessors
    g, ends = add_virtual_op_for_multiple_finished_ops(*create_read_graph_cpu_storage(
        ids(0, 1, 2, 3), ids(4, 5, 6, 7), ids(9)))
    assert g._op_map[ends[0]].transfer_type == TransferType.VIRTUAL


def test_layer_wise_conversion():
    g, ends = create_read_graph_cpu_storage(ids(0, 1), ids(4, 5), ids(9), layer_num=8)
    new, tracked = convert_read_graph_to_layer_wise_graph(g, ends, 8, 2)
    assert new.graph_id == g.graph_id and new.num_ops == 3 * 4 and len(tracked) == 4
    layers = sorted(new._op_map[t].layer_id for t in tracked)
    assert layers == [0, 2, 4, 6]
    for t in tracked:
        op = new._op_map[t]
        assert op.layer_granularity == 2
        if op.layer_id > 0:   # previous layer group of the same op, and this group's DISK2H
            kinds = sorted(new._op_map[p].transfer_type.name for p in op.predecessors)
            layer_ids = sorted(new._op_map[p].layer_id for p in op.predecessors)
            assert kinds == ["DISK2H", "H2D"] and layer_ids == [op.layer_id - 2, op.layer_id]


@pytest.fixture
def fake_engine(monkeypatch):
    from _fake_worker import FakeGPUCPUWorker
    from flexkv_amd.common.config import CacheConfig, ModelConfig
    from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType
    from flexkv_amd.storage.allocator import AccessHandleType, StorageHandle
    from flexkv_amd.transfer import transfer_engine as te
    monkeypatch.setattr(te, "GPUCPUTransferWorker", FakeGPUCPUWorker)
    FakeGPUCPUWorker.log = []
    lay = KVCacheLayout(KVCacheLayoutType.LAYERWISE, 4, 8, 1, 1, 8)
    gpu = StorageHandle(AccessHandleType.TENSOR, [torch.zeros(1)] * 4, lay, torch.float16,
                        gpu_device_id=0)
    cpu = StorageHandle(AccessHandleType.TENSOR, torch.zeros(4), lay, torch.float16)

    def make(eager):
        e = te.TransferEngine([gpu], ModelConfig(4, 1, 8), CacheConfig(), cpu_handle=cpu,
                              eager_dispatch=eager)
        e.start()
        return e
    yield make, FakeGPUCPUWorker


def _wait_graph(engine, gid, limit=10.0):
    """Completion records seen so far (kept on the engine across calls)."""
    seen = engine.__dict__.setdefault("_test_seen", [])
    t0 = time.time()
    while (gid, -1) not in seen:
        if time.time() - t0 > limit:
            raise AssertionError(f"graph {gid} did not complete; saw {seen}")
        seen.extend(engine.get_completed_graphs_and_ops(timeout=0.05))
    return [item for item in seen if item[0] == gid]


@pytest.mark.parametrize("eager", [False, True])
def test_engine_runs_layer_wise_graph_in_order(fake_engine, eager):
    make, worker = fake_engine
    eng = make(eager)
    try:
        g, ends = create_read_graph_cpu_storage(ids(0, 1), ids(4, 5), ids(), layer_num=4)
        new, tracked = convert_read_graph_to_layer_wise_graph(g, ends, 4, 1)
        eng.submit_transfer_graph(new)
        seen = _wait_graph(eng, new.graph_id)
        assert [layer for _, _, layer in worker.log] == [0, 1, 2, 3]
        assert {op for _, op in seen if op >= 0} == set(tracked)
    finally:
        eng.shutdown()


def test_engine_multiple_graphs_and_virtual(fake_engine):
    make, worker = fake_engine
    eng = make(True)
    try:
        gw, _ = create_write_graph_cpu_storage(ids(0, 1), ids(2, 3), ids())
        gr, ends = add_virtual_op_for_multiple_finished_ops(
            *create_read_graph_cpu_storage(ids(0, 1), ids(2, 3), ids()))
        gr2 = TransferOpGraph()
        v = TransferOp(graph_id=0, transfer_type=TransferType.VIRTUAL, layer_id=-1,
                       layer_granularity=-1)
        gr2.add_virtual_op(v)
        for g in (gw, gr, gr2):
            eng.submit_transfer_graph(g)
        for g in (gw, gr, gr2):
            _wait_graph(eng, g.graph_id)
        assert sorted(k for _, k, _ in worker.log) == ["D2H", "H2D"]
    finally:
        eng.shutdown()


def test_engine_shutdown_leaves_no_threads(fake_engine):
    """Engines started and shut down one after another (thread-mode workers
    and the scheduler) leave the process's threads where they were."""
    import threading
    make, _ = fake_engine
    eng = make(True)
    eng.shutdown()
    before = {t.ident for t in threading.enumerate()}
    for _ in range(5):
        eng = make(True)
        eng.shutdown()
    left = [t.name for t in threading.enumerate() if t.ident not in before and t.is_alive()]
    assert not left, left
