"""Op trace ranges for profiler timelines (roctx).

The reference wraps every worker op in an NVTX range named after the op's
type, id, graph id and block count (flexkv/transfer/worker.py:160-165).  Here
the same range is a roctx range, so ``rocprofv3 --marker-trace`` puts it on
the timeline next to the op's kernels and copy-engine copies.  roctx comes
from ROCm's librocprofiler-sdk-roctx; where it is absent the ranges are
no-ops.  FLEXKV_ROCTX=0 turns them off.
"""
from __future__ import annotations

import ctypes
import os
from contextlib import contextmanager
from typing import Iterator, Optional

_lib: Optional[ctypes.CDLL] = None
_loaded = False


def _roctx() -> Optional[ctypes.CDLL]:
    global _lib, _loaded
    if _loaded:
        return _lib
    _loaded = True
    if os.environ.get("FLEXKV_ROCTX", "1") == "0":
        return None
    names = ["librocprofiler-sdk-roctx.so.1", "librocprofiler-sdk-roctx.so"]
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    names += [os.path.join(rocm, "lib", n) for n in list(names)]
    for name in names:
        try:
            lib = ctypes.CDLL(name)
        except OSError:
            continue
        lib.roctxRangePushA.restype = ctypes.c_int
        lib.roctxRangePushA.argtypes = [ctypes.c_char_p]
        lib.roctxRangePop.restype = ctypes.c_int
        lib.roctxRangePop.argtypes = []
        _lib = lib
        break
    return _lib


def available() -> bool:
    return _roctx() is not None


@contextmanager
def op_range(message: str) -> Iterator[None]:
    """A roctx range around the body (nested ranges nest on the timeline)."""
    lib = _roctx()
    if lib is None:
        yield
        return
    lib.roctxRangePushA(message.encode())
    try:
        yield
    finally:
        lib.roctxRangePop()


def op_message(op) -> str:
    """The reference's range name for a worker op (worker.py:160-162)."""
    return (f"launch {op.transfer_type.name} op_id: {op.transfer_op_id}, "
            f"graph_id: {op.transfer_graph_id}, num_blocks: {len(op.src_block_ids)}")
