"""Op trace ranges: the reference's range name for a worker op
(flexkv/transfer/worker.py:160-162), ranges that nest and unwind on errors,
and no-ops where roctx is switched off."""
import pytest
import torch

from flexkv_amd.common import trace
from flexkv_amd.common.transfer import TransferDescriptor, TransferOp, TransferType
from flexkv_amd.transfer.worker import WorkerTransferOp


def _op():
    ids = torch.arange(7, dtype=torch.int64)
    return WorkerTransferOp(TransferOp(graph_id=3, transfer_type=TransferType.D2H, layer_id=0,
                                       layer_granularity=-1,
                                       src_descriptor=TransferDescriptor(physical_block_ids=ids),
                                       dst_descriptor=TransferDescriptor(physical_block_ids=ids)))


def test_op_message_is_the_references():
    op = _op()
    assert trace.op_message(op) == (f"launch D2H op_id: {op.transfer_op_id}, graph_id: 3, "
                                    "num_blocks: 7")


def test_ranges_nest_and_unwind():
    with trace.op_range("outer"):
        with trace.op_range("inner"):
            pass
    with pytest.raises(ValueError):
        with trace.op_range("failing"):
            raise ValueError("op failed")
    with trace.op_range("after"):
        pass


def test_switched_off(monkeypatch):
    monkeypatch.setattr(trace, "_loaded", False)
    monkeypatch.setattr(trace, "_lib", None)
    monkeypatch.setenv("FLEXKV_ROCTX", "0")
    assert not trace.available()
    with trace.op_range("ignored"):
        pass
