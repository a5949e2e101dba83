"""Helpers for GPU parity tests: put a KVCase on the device and call the C-ABI."""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from flexkv_amd import _lib
from flexkv_amd.storage.allocator import pinned_empty

_TORCH_OF = {np.uint16: torch.int16, np.uint32: torch.int32, np.uint8: torch.uint8}
_SIGNED = {np.uint16: np.int16, np.uint32: np.int32, np.uint8: np.uint8}


def to_torch(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(_SIGNED[a.dtype.type]))


def to_numpy(t: torch.Tensor, dtype) -> np.ndarray:
    return t.cpu().numpy().view(dtype)


class DeviceCase:
    """Device layers + pinned host cache mirroring a KVCase."""

    def __init__(self, case, device="cuda:0", host_coherence=_lib.FKV_HOST_DEFAULT):
        self.case = case
        self.dtype = case.dtype
        self.gpu = [to_torch(g).to(device) for g in case.gpu]
        flat = to_torch(case.host.reshape(-1))
        self.host = pinned_empty(flat.numel(), flat.dtype, host_coherence)
        self.host.copy_(flat)

    def host_np(self) -> np.ndarray:
        return self.host.numpy().view(self.dtype).reshape(self.case.host_shape())

    def gpu_np(self):
        return [to_numpy(g, self.dtype) for g in self.gpu]

    def set_gpu(self, arrays):
        for t, a in zip(self.gpu, arrays):
            t.copy_(to_torch(a))

    def set_host(self, a: np.ndarray):
        self.host.copy_(to_torch(a.reshape(-1)))


def abi_transfer(dc: DeviceCase, gids, cids, h2d: bool, mode: int, transfer_cus: int = -1,
                 stream=None, layers=None, start_layer=None, **override) -> None:
    """fkv_transfer_kv_blocks over the case's geometry; raises RuntimeError."""
    case = dc.case
    s = case.strides()
    s.update(override)
    layers = dc.gpu if layers is None else layers
    start = case.start_layer if start_layer is None else start_layer
    gids = np.ascontiguousarray(gids, dtype=np.int64)
    cids = np.ascontiguousarray(cids, dtype=np.int64)
    ptrs = (ctypes.c_void_p * max(1, len(layers)))(*[t.data_ptr() for t in layers])
    st = torch.cuda.current_stream() if stream is None else stream
    lib = _lib.load()
    rc = lib.fkv_transfer_kv_blocks(
        len(gids), start, len(layers), gids.ctypes.data, ptrs, s["gpu_kv"], s["gpu_block"],
        cids.ctypes.data, dc.host.data_ptr(), s["cpu_kv"], s["cpu_layer"], s["cpu_block"],
        s["startoff"], s["chunk"], st.cuda_stream, transfer_cus, 1 if h2d else 0, mode,
        1 if case.kv == 1 else 0)
    _lib.check(rc, "fkv_transfer_kv_blocks")


def zero_blocks(t: torch.Tensor, ids: torch.Tensor) -> None:
    """Zero blocks `ids` (axis 1) of a per-layer [kv, blocks, ...] tensor in
    place and check that they are zero (``t[:, ids].zero_()`` would only
    zero a gathered copy)."""
    idx = ids.to(t.device)
    t.index_fill_(1, idx, 0)
    assert not t.index_select(1, idx).any(), "blocks were not cleared"


def split_kv_layers(dc: DeviceCase):
    """The case's device layers as separate allocations, [layer][K|V], each
    [ng, tokens, heads, dim] (one per layer for MLA)."""
    return [[dc.gpu[l][k].clone() for k in range(dc.case.kv)] for l in range(len(dc.gpu))]


def abi_transfer_kv_ptrs(dc: DeviceCase, kv_tensors, gids, cids, h2d: bool, mode: int,
                         transfer_cus: int = -1) -> None:
    """fkv_transfer_kv_blocks_kv_ptrs over the case's host geometry with the
    device side given as separate K/V tensors; raises RuntimeError."""
    case = dc.case
    s = case.strides()
    flat = [t for pair in kv_tensors for t in pair]
    gids = np.ascontiguousarray(gids, dtype=np.int64)
    cids = np.ascontiguousarray(cids, dtype=np.int64)
    ptrs = (ctypes.c_void_p * max(1, len(flat)))(*[t.data_ptr() for t in flat])
    lib = _lib.load()
    rc = lib.fkv_transfer_kv_blocks_kv_ptrs(
        len(gids), case.start_layer, len(kv_tensors), gids.ctypes.data, ptrs, s["gpu_block"],
        cids.ctypes.data, dc.host.data_ptr(), s["cpu_kv"], s["cpu_layer"], s["cpu_block"],
        s["startoff"], s["chunk"], torch.cuda.current_stream().cuda_stream, transfer_cus,
        1 if h2d else 0, mode, 1 if case.kv == 1 else 0)
    _lib.check(rc, "fkv_transfer_kv_blocks_kv_ptrs")
