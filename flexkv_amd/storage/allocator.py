"""Host and GPU cache allocation for the transfer path.

Role of flexkv/storage/allocator.py:41-130.  The host cache is one flat 1-D
tensor of layout.get_total_elements() elements (allocator.py:99-107).  Pinned
host caches come from fkv_host_alloc (hipHostMalloc, mapped into the device
address space) rather than torch's caching host allocator, which rounds
requests up to powers of two (34 GiB would pin 64 GiB).  The pinned tensor
owns its allocation: the memory is freed when the last view of it dies.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from enum import Enum, auto
from typing import Any, List, Optional, Union

import numpy as np
import torch

from .. import _lib
from ..common.debug import flexkv_logger
from ..common.memory_handle import TensorSharedHandle
from ..common.storage import KVCacheLayout


class AccessHandleType(Enum):
    TENSOR = auto()
    FILE = auto()
    TENSOR_HANDLE = auto()


@dataclass
class StorageHandle:
    """Same fields and accessors as the reference (common/storage.py:158-217)
    for the tensor-backed handle types."""
    handle_type: AccessHandleType
    data: Any
    kv_layout: KVCacheLayout
    dtype: torch.dtype
    num_blocks_per_file: Optional[int] = None
    gpu_device_id: Optional[int] = None

    def get_tensor(self) -> torch.Tensor:
        if self.handle_type != AccessHandleType.TENSOR or not isinstance(self.data, torch.Tensor):
            raise ValueError(f"Invalid handle type: {self.handle_type}, expected TENSOR")
        return self.data

    def get_tensor_list(self) -> List[torch.Tensor]:
        if self.handle_type == AccessHandleType.TENSOR:
            return list(self.data)
        if self.handle_type == AccessHandleType.TENSOR_HANDLE:
            return [h.get_tensor() for h in self.data]
        raise ValueError(f"Invalid handle type: {self.handle_type}, expected TENSOR or TENSOR_HANDLE")

    def get_tensor_handle_list(self) -> List[TensorSharedHandle]:
        if self.handle_type == AccessHandleType.TENSOR_HANDLE:
            return list(self.data)
        if self.handle_type == AccessHandleType.TENSOR:
            return [TensorSharedHandle(t) for t in self.data]
        raise ValueError(f"Invalid handle type: {self.handle_type}, expected TENSOR_HANDLE or TENSOR")


def _owned_host_array(ptr: int, nbytes: int):
    """ctypes byte array over [ptr, ptr+nbytes) whose collection frees ptr."""
    base = ctypes.c_uint8 * nbytes
    # Bound now: module globals may already be gone when the last view dies
    # during interpreter shutdown.
    free_fn = _lib.load().fkv_host_free
    void_p = ctypes.c_void_p

    class _PinnedBytes(base):  # type: ignore[valid-type, misc]
        _fkv_ptr = 0

        def __del__(self, _free=free_fn, _vp=void_p) -> None:
            p, self._fkv_ptr = self._fkv_ptr, 0
            if p:
                try:
                    _free(_vp(p))
                except Exception:
                    pass

    arr = _PinnedBytes.from_address(ptr)
    arr._fkv_ptr = ptr
    return arr


def pinned_empty(numel: int, dtype: torch.dtype, coherence: int = _lib.FKV_HOST_DEFAULT) -> torch.Tensor:
    """A 1-D pinned host tensor of `numel` elements (uninitialised)."""
    es = torch.empty((), dtype=dtype).element_size()
    nbytes = int(numel) * es
    if nbytes <= 0:
        raise ValueError("pinned_empty needs a positive size")
    lib = _lib.load()
    p = ctypes.c_void_p()
    _lib.check(lib.fkv_host_alloc(ctypes.byref(p), nbytes, coherence), "fkv_host_alloc")
    raw = _owned_host_array(p.value, nbytes)
    flat = torch.from_numpy(np.frombuffer(raw, dtype=np.uint8))
    return flat.view(dtype)


@dataclass
class HostCacheSpec:
    """A host cache to be allocated, pinned, by the process that uses it.

    Pinned host memory cannot be handed to a spawned worker by pickling (the
    copy the child would receive is ordinary shared memory, and this library
    does not page-lock existing memory), so a worker in its own process is
    given this spec and allocates the cache itself."""
    layout: KVCacheLayout
    dtype: torch.dtype
    coherence: int = _lib.FKV_HOST_DEFAULT

    def allocate(self) -> torch.Tensor:
        return pinned_empty(self.layout.get_total_elements(), self.dtype, self.coherence)


class GPUAllocator:
    @classmethod
    def allocate(cls, layout: KVCacheLayout, dtype: torch.dtype, **kwargs: Any) -> StorageHandle:
        """num_chunks flat device tensors splitting layout's elements evenly
        (allocator.py:43-68); num_chunks = num_layer gives per-layer tensors."""
        device_id = kwargs.get("device_id", torch.cuda.current_device())
        num_chunks = kwargs.get("num_chunks", 1)
        per = layout.get_total_elements() // num_chunks
        chunks = [torch.empty(per, dtype=dtype, device=f"cuda:{device_id}") for _ in range(num_chunks)]
        return StorageHandle(AccessHandleType.TENSOR, chunks, layout, dtype, gpu_device_id=device_id)

    @classmethod
    def free(cls, handle: StorageHandle) -> None:
        pass

    @classmethod
    def from_raw_data(cls, data: Union[List[TensorSharedHandle], List[torch.Tensor]],
                      layout: KVCacheLayout, dtype: torch.dtype, **kwargs: Any) -> StorageHandle:
        device_id = kwargs.get("device_id")
        if device_id is None:
            raise ValueError("device_id is required for GPU allocator")
        kind = AccessHandleType.TENSOR if isinstance(data[0], torch.Tensor) else AccessHandleType.TENSOR_HANDLE
        return StorageHandle(kind, data, layout, dtype, gpu_device_id=device_id)


class CPUAllocator:
    @classmethod
    def allocate(cls, layout: KVCacheLayout, dtype: torch.dtype, **kwargs: Any) -> StorageHandle:
        """Flat host cache; pinned (default) through fkv_host_alloc."""
        pin_memory = kwargs.get("pin_memory", True)
        coherence = kwargs.get("coherence", _lib.FKV_HOST_DEFAULT)
        total = layout.get_total_elements()
        es = torch.empty((), dtype=dtype).element_size()
        flexkv_logger.info(f"CPU allocate total_size: {total * es / 2**30:.3f} GiB "
                           f"({'pinned' if pin_memory else 'pageable'})")
        t = pinned_empty(total, dtype, coherence) if pin_memory else torch.empty(total, dtype=dtype)
        return StorageHandle(AccessHandleType.TENSOR, t, layout, dtype)

    @classmethod
    def free(cls, handle: StorageHandle) -> None:
        pass

    @classmethod
    def from_raw_data(cls, data: torch.Tensor, layout: KVCacheLayout, dtype: torch.dtype,
                      **kwargs: Any) -> StorageHandle:
        return StorageHandle(AccessHandleType.TENSOR, data, layout, dtype)
