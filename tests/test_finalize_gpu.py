"""fkv_finalize: every process-lifetime object of the library (layer-wise
handles left unreleased, streams from fkv_stream_create, copy-engine signals,
events and staging, pinned id buffers) is released before the runtimes'
exit-time finalizers run, and the library works again afterwards."""
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

import oracle
from gpu_util import DeviceCase, abi_transfer
from kvcase import KVCase
from oracle import inputs

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _case(seed):
    return KVCase(layers_total=4, num_layers=4, start_layer=0, kv=2, ng=64, nh=96, tokens=16,
                  heads=8, dim=128).fill(seed=seed)


def _d2h_expected(case, gids, cids):
    s = case.strides()
    want = case.host.copy()
    oracle.transfer_kv_blocks(gids, case.gpu, s["gpu_kv"], s["gpu_block"], cids, want,
                              s["cpu_kv"], s["cpu_layer"], s["cpu_block"], s["chunk"], 0, False)
    return want


def _layerwise(dc, gids, cids):
    from flexkv_amd import c_ext
    s = dc.case.strides()
    ptrs = torch.tensor([t.data_ptr() for t in dc.gpu], dtype=torch.int64)
    return c_ext.transfer_kv_blocks_layerwise(
        torch.from_numpy(gids), ptrs, s["gpu_kv"], s["gpu_block"], torch.from_numpy(cids),
        dc.host, s["cpu_kv"], s["cpu_layer"], s["cpu_block"], s["chunk"], 0, 1, -1, False)


def test_finalize_then_library_works_again():
    from flexkv_amd import _lib, c_ext
    case = _case(21)
    dc = DeviceCase(case)
    gids = inputs.distinct_ids(3, 20, case.ng)
    cids = inputs.distinct_ids(4, 20, case.nh)
    abi_transfer(dc, gids, cids, False, _lib.FKV_XFER_CE)     # staging, signals, events
    stream = c_ext.transfer_stream()
    with torch.cuda.stream(stream):
        hnd = _layerwise(dc, gids, cids)                       # left unreleased
    group = c_ext.TPTransferThreadGroup(2, [dc.gpu, dc.gpu], dc.host, 0)   # left open
    _lib.finalize()
    hnd.release()                                               # already released: no call
    c_ext.release_transfer_stream(stream)                       # already destroyed: no call
    group.close()                                               # already destroyed: no call
    assert np.array_equal(dc.host_np(), _d2h_expected(case, gids, cids))
    # everything is made again on demand
    dc.set_host(case.host)
    abi_transfer(dc, gids, cids, False, _lib.FKV_XFER_CE)
    assert np.array_equal(dc.host_np(), _d2h_expected(case, gids, cids))
    s2 = c_ext.transfer_stream()
    with torch.cuda.stream(s2):
        h2 = _layerwise(dc, gids, cids)
    h2.release()
    c_ext.release_transfer_stream(s2)


_CHILD = r"""
import os, sys
sys.path.insert(0, {root!r})
sys.path.insert(0, os.path.join({root!r}, "tests"))
os.environ["FLEXKV_CE_MIN_BYTES"] = "0"
import numpy as np
import torch
from gpu_util import DeviceCase, abi_transfer
from kvcase import KVCase
from oracle import inputs
from flexkv_amd import _lib, c_ext
case = KVCase(layers_total=4, num_layers=4, start_layer=0, kv=2, ng=64, nh=96, tokens=16,
              heads=8, dim=128).fill(seed=5)
dc = DeviceCase(case)
gids = inputs.distinct_ids(1, 16, 64)
cids = inputs.distinct_ids(2, 16, 96)
for h2d in (False, True):
    abi_transfer(dc, gids, cids, h2d, _lib.FKV_XFER_CE)
s = case.strides()
stream = c_ext.transfer_stream()
ptrs = torch.tensor([t.data_ptr() for t in dc.gpu], dtype=torch.int64)
with torch.cuda.stream(stream):
    keep = c_ext.transfer_kv_blocks_layerwise(
        torch.from_numpy(gids), ptrs, s["gpu_kv"], s["gpu_block"], torch.from_numpy(cids),
        dc.host, s["cpu_kv"], s["cpu_layer"], s["cpu_block"], s["chunk"], 0, 1, -1, True)
group = c_ext.TPTransferThreadGroup(2, [dc.gpu, dc.gpu], dc.host, 0)
print("child: exiting with a stream, a handle, a TP group and copy-engine state alive",
      flush=True)
"""


def test_process_exits_cleanly_with_library_objects_alive(tmp_path):
    script = tmp_path / "child.py"
    script.write_text(_CHILD.format(root=ROOT))
    res = subprocess.run([sys.executable, str(script)], capture_output=True, text=True,
                         timeout=180)
    assert "child: exiting" in res.stdout, res.stdout + res.stderr
    assert res.returncode == 0, res.stderr[-2000:]
