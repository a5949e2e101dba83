"""The bounded copy-engine wait on the device path.  A child process runs
with FLEXKV_SDMA_TIMEOUT_MS=1, so the host stops waiting for copies that are
still in flight (the copies themselves finish normally): the worker reports
the op as finished, records it in failed_ops and logs the timeout; the
device's later copy-engine transfers move with the zero-copy kernel and are
bit-exact.  The worker records the host blocks the given-up copies may still write
with the failed op (unsafe_host_blocks, from fkv_last_unsafe_host_blocks),
and fkv_abandoned_copies_pending reads 0 once those copies have finished.
The child sleeps before it exits, so the given-up copies end inside the
process (their staging and signals are never freed or reused)."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

_CHILD = r"""
import os, sys, time, queue
sys.path.insert(0, {root!r})
import torch
from flexkv_amd.common.storage import KVCacheLayout, KVCacheLayoutType
from flexkv_amd.common.transfer import TransferDescriptor, TransferOp, TransferType
from flexkv_amd.storage.allocator import CPUAllocator
from flexkv_amd.transfer.worker import GPUCPUTransferWorker, WorkerTransferOp
L, NG, NH = 4, 2048, 2048
gl = KVCacheLayout(KVCacheLayoutType.LAYERWISE, L, NG, 16, 8, 128)
cl = KVCacheLayout(KVCacheLayoutType.BLOCKWISE, L, NH, 16, 8, 128)
gen = torch.Generator(device="cuda").manual_seed(3)
gpu = [torch.randint(-30000, 30000, tuple(gl.kv_shape[1:]), dtype=torch.int16, device="cuda",
                     generator=gen).view(torch.bfloat16) for _ in range(L)]
cpu = CPUAllocator.allocate(cl, torch.bfloat16).get_tensor()
w = GPUCPUTransferWorker(0, None, None, gpu, cpu, gl, cl, torch.bfloat16, 0,
                         use_ce_transfer_h2d=True, use_ce_transfer_d2h=True)
g = torch.Generator().manual_seed(4)
gids = torch.randperm(NG, generator=g)[:1024]
cids = torch.randperm(NH, generator=g)[:1024]
def op(kind, src, dst):
    return TransferOp(graph_id=0, transfer_type=kind, layer_id=-1, layer_granularity=-1,
                      src_descriptor=TransferDescriptor(physical_block_ids=src),
                      dst_descriptor=TransferDescriptor(physical_block_ids=dst))
q = queue.Queue()
w.finished_ops_queue = q
bad = op(TransferType.D2H, gids, cids)         # 256 MiB: the engines need ~4.5 ms
w._execute(WorkerTransferOp(bad))
assert q.get(timeout=60) == bad.op_id
assert w.failed_ops == [bad.op_id], w.failed_ops
print("child: op failed and was reported", flush=True)
from flexkv_amd import _lib
unsafe = w.unsafe_host_blocks[bad.op_id]
assert len(unsafe) > 0 and set(unsafe.tolist()) <= set(cids.tolist()), unsafe
assert len(set(unsafe.tolist())) == len(unsafe)
print(f"child: {{len(unsafe)}} host blocks reported unsafe", flush=True)
time.sleep(1.0)                                 # the given-up copies finish
assert _lib.abandoned_copies_pending(0) == 0
print("child: the abandoned copies have finished", flush=True)
cpu.view(torch.int16).zero_()
good = op(TransferType.D2H, gids, cids)         # the zero-copy kernel from now on
w._execute(WorkerTransferOp(good))
assert q.get(timeout=60) == good.op_id and w.failed_ops == [bad.op_id]
host = cpu.view(torch.int16).view(NH, L, 2, -1)
g_dev = gids.cuda()
for l, t in enumerate(gpu):
    want = t.view(torch.int16).view(2, NG, -1)[:, g_dev].transpose(0, 1).cpu()
    assert torch.equal(host[cids, l], want), l
print("child: the fallback transfer is bit-exact", flush=True)
"""


def test_copy_engine_wait_timeout_fails_the_op_and_falls_back(tmp_path):
    script = tmp_path / "child.py"
    script.write_text(_CHILD.format(root=ROOT))
    env = dict(os.environ, FLEXKV_SDMA_TIMEOUT_MS="1", FLEXKV_CE_MIN_BYTES="0",
               FLEXKV_LOG_LEVEL="ERROR")
    res = subprocess.run([sys.executable, str(script)], capture_output=True, text=True,
                         timeout=180, env=env)
    out = res.stdout + res.stderr
    assert res.returncode == 0, out[-3000:]
    assert "child: op failed and was reported" in res.stdout, out[-3000:]
    assert "host blocks reported unsafe" in res.stdout, out[-3000:]
    assert "child: the abandoned copies have finished" in res.stdout, out[-3000:]
    assert "child: the fallback transfer is bit-exact" in res.stdout, out[-3000:]
    assert "did not finish within 1 ms" in res.stderr, res.stderr[-3000:]
