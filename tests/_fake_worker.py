"""A TransferWorkerBase subclass that records ops instead of moving data,
importable by spawned worker processes in CPU tests."""
from flexkv_amd.transfer.worker import TransferWorkerBase


class RecordingWorker(TransferWorkerBase):
    def __init__(self, worker_id, transfer_conn, finished_ops_queue, fail_on=()):
        super().__init__(worker_id, transfer_conn, finished_ops_queue)
        self.fail_on = set(fail_on)
        self.seen = []

    def _transfer_impl(self, src_block_ids, dst_block_ids, transfer_type, layer_id,
                       layer_granularity, **kwargs):
        raise NotImplementedError

    def launch_transfer(self, transfer_op):
        self.seen.append(transfer_op.transfer_op_id)
        if transfer_op.transfer_op_id in self.fail_on:
            raise RuntimeError("planted failure")


class FakeGPUCPUWorker(TransferWorkerBase):
    """Stands in for GPUCPUTransferWorker in engine tests without a device:
    records (op id, type, layer_id) in execution order."""
    log = []

    def __init__(self, worker_id, transfer_conn, finished_ops_queue, gpu_blocks=None,
                 cpu_blocks=None, gpu_kv_layout=None, cpu_kv_layout=None, dtype=None,
                 gpu_device_id=0, **kwargs):
        super().__init__(worker_id, transfer_conn, finished_ops_queue)

    def _transfer_impl(self, *a, **k):
        raise NotImplementedError

    def launch_transfer(self, transfer_op):
        import time
        time.sleep(0.002)
        FakeGPUCPUWorker.log.append((transfer_op.transfer_op_id, transfer_op.transfer_type.name,
                                     transfer_op.layer_id))
