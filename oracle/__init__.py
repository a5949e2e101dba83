"""CPU oracle for the GPU<->CPU KV-block transfer.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``, as the parity oracle and the CPU
baseline.
The product package ``flexkv_amd`` never imports it.

``transfer_kv_blocks`` calls the C restatement in ``kv_oracle.c`` (built into
``liboracle.so`` by the Makefile beside it).  Its arguments mirror the
reference binding ``transfer_kv_blocks`` (csrc/bindings.cpp:25-32) with the
"GPU" side given as host arrays.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Sequence, Union

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

ArrayLike = Union[np.ndarray, "torch.Tensor"]  # noqa: F821


def build(force: bool = False) -> str:
    """Compile liboracle.so with gcc (make) and return its path."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "all"], cwd=_HERE, check=True)
    return _LIB_PATH


def _load():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        lib = ctypes.CDLL(_LIB_PATH)
        f = lib.oracle_transfer_kv_blocks
        f.restype = ctypes.c_int
        f.argtypes = [
            ctypes.c_int, ctypes.c_int, ctypes.c_int,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
            ctypes.c_int64, ctypes.c_int64,
            ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ]
        g = lib.oracle_transfer_kv_blocks_ssd
        g.restype = ctypes.c_int
        g.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                      ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64,
                      ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        _lib = lib
    return _lib


def _addr(x) -> int:
    """Host address of a C-contiguous numpy array or CPU torch tensor."""
    if isinstance(x, np.ndarray):
        if not x.flags["C_CONTIGUOUS"]:
            raise ValueError("oracle needs C-contiguous arrays")
        return x.ctypes.data
    if hasattr(x, "data_ptr"):
        if x.device.type != "cpu":
            raise ValueError("oracle works on host memory only")
        if not x.is_contiguous():
            raise ValueError("oracle needs contiguous tensors")
        return x.data_ptr()
    raise TypeError(f"unsupported buffer type {type(x)!r}")


def _ids(x) -> np.ndarray:
    if hasattr(x, "numpy"):
        x = x.numpy()
    a = np.ascontiguousarray(np.asarray(x, dtype=np.int64))
    if a.ndim != 1:
        raise ValueError("block ids must be 1-D")
    return a


def transfer_kv_blocks(gpu_block_ids, gpu_layers: Sequence, gpu_kv_stride_in_bytes: int,
                       gpu_block_stride_in_bytes: int, cpu_block_ids, cpu_buffer,
                       cpu_kv_stride_in_bytes: int, cpu_layer_stride_in_bytes: int,
                       cpu_block_stride_in_bytes: int, chunk_size_in_bytes: int,
                       start_layer_id: int, is_host_to_device: bool,
                       use_ce_transfer: bool = False, is_mla: bool = False,
                       cpu_startoff_inside_chunks: int = 0, num_threads: int = 1) -> None:
    """Oracle transfer, in place.  ``gpu_layers`` is one host buffer per layer
    (the slice [start_layer_id, start_layer_id + len) of the engine's layers,
    as in worker.py:293-295); ``cpu_buffer`` is the flat host cache."""
    gids = _ids(gpu_block_ids)
    cids = _ids(cpu_block_ids)
    if gids.shape != cids.shape:
        raise ValueError("gpu and cpu block id lists differ in length")
    ptrs = np.array([_addr(t) for t in gpu_layers], dtype=np.uint64)
    rc = _load().oracle_transfer_kv_blocks(
        int(gids.size), int(start_layer_id), int(len(gpu_layers)),
        gids.ctypes.data, ptrs.ctypes.data, int(gpu_kv_stride_in_bytes),
        int(gpu_block_stride_in_bytes), cids.ctypes.data, _addr(cpu_buffer),
        int(cpu_kv_stride_in_bytes), int(cpu_layer_stride_in_bytes),
        int(cpu_block_stride_in_bytes), int(cpu_startoff_inside_chunks),
        int(chunk_size_in_bytes), int(bool(is_host_to_device)), int(use_ce_transfer),
        int(bool(is_mla)), int(num_threads))
    if rc != 0:
        raise ValueError(f"oracle rejected arguments (rc={rc})")


def tp_group_transfer(rank_layers: Sequence[Sequence], gpu_block_ids,
                      gpu_kv_stride_in_bytes: int, gpu_block_stride_in_bytes: int,
                      gpu_chunk_size_in_bytes: int, cpu_block_ids, cpu_buffer,
                      cpu_kv_stride_in_bytes: int, cpu_layer_stride_in_bytes: int,
                      cpu_block_stride_in_bytes: int, is_host_to_device: bool,
                      layer_id: int, layer_granularity: int, is_mla: bool = False) -> None:
    """Oracle of a tensor-parallel group transfer, in place: rank r (its
    per-layer host buffers ``rank_layers[r]``, all layers) moves host layers
    [layer_id, layer_id + layer_granularity) from its own layers of that
    window, at byte offset r * gpu_chunk inside each host chunk, as each
    thread of csrc/tp_transfer_thread_group.cpp:66-99 calls transfer_kv_blocks
    (startoff :79-80).  Rank r's window is rank_layers[r][layer_id:...]; the
    reference's pointer arithmetic (:76-77) differs from that when the window
    is not every layer, which the product does not follow.  Under MLA every
    rank holds the same latent: device-to-host is rank 0's move (the
    reference has every rank write the same bytes at offset 0), host-to-device
    is every rank's."""
    for r, layers in enumerate(rank_layers):
        if is_mla and not is_host_to_device and r != 0:
            continue
        transfer_kv_blocks(gpu_block_ids, list(layers[layer_id:layer_id + layer_granularity]),
                           gpu_kv_stride_in_bytes, gpu_block_stride_in_bytes, cpu_block_ids,
                           cpu_buffer, cpu_kv_stride_in_bytes, cpu_layer_stride_in_bytes,
                           cpu_block_stride_in_bytes, gpu_chunk_size_in_bytes, layer_id,
                           is_host_to_device, use_ce_transfer=True, is_mla=is_mla,
                           cpu_startoff_inside_chunks=0 if is_mla else r * gpu_chunk_size_in_bytes)


def transfer_kv_blocks_ssd(files: Sequence, num_devices: int, files_per_device: int,
                           start_layer: int, num_layers: int, cpu_buffer, ssd_block_ids,
                           cpu_block_ids, cpu_layer_stride: int, cpu_kv_stride: int,
                           ssd_layer_stride: int, ssd_kv_stride: int, chunk_size: int,
                           block_stride: int, is_read: bool, round_robin: int = 1,
                           is_mla: bool = False) -> None:
    """Oracle SSD transfer over in-memory file images (`files`, device-major,
    num_devices * files_per_device writable byte arrays), in place."""
    sids = _ids(ssd_block_ids)
    cids = _ids(cpu_block_ids)
    if sids.shape != cids.shape:
        raise ValueError("ssd and cpu block id lists differ in length")
    if len(files) != num_devices * files_per_device:
        raise ValueError("need num_devices * files_per_device file images")
    ptrs = np.array([_addr(f) for f in files], dtype=np.uint64)
    rc = _load().oracle_transfer_kv_blocks_ssd(
        ptrs.ctypes.data, int(num_devices), int(files_per_device), int(start_layer),
        int(num_layers), _addr(cpu_buffer), sids.ctypes.data, cids.ctypes.data, int(sids.size),
        int(cpu_layer_stride), int(cpu_kv_stride), int(ssd_layer_stride), int(ssd_kv_stride),
        int(chunk_size), int(block_stride), int(bool(is_read)), int(round_robin),
        int(bool(is_mla)))
    if rc != 0:
        raise ValueError(f"oracle rejected arguments (rc={rc})")
