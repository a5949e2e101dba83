"""Host, GPU and SSD cache allocation for the transfer path.

Role of flexkv/storage/allocator.py:41-206.  The host cache is one flat 1-D
tensor of layout.get_total_elements() elements (allocator.py:99-107).  Pinned
host caches come from fkv_host_alloc (hipHostMalloc, mapped into the device
address space) rather than torch's caching host allocator, which rounds
requests up to powers of two (34 GiB would pin 64 GiB).  The pinned tensor
owns its allocation: the memory is freed when the last view of it dies.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from enum import Enum, auto
from typing import Any, BinaryIO, Dict, List, Optional, Union

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
        """Per-layer tensors; a layer whose K and V are separate allocations
        is a [K, V] list."""
        if self.handle_type == AccessHandleType.TENSOR:
            return list(self.data)
        if self.handle_type == AccessHandleType.TENSOR_HANDLE:
            return [_map_layer(h, lambda x: x.get_tensor()) for h in self.data]
        raise ValueError(f"Invalid handle type: {self.handle_type}, expected TENSOR or TENSOR_HANDLE")

    def get_file_list(self) -> Union[List[str], Dict[int, List[str]]]:
        if self.handle_type != AccessHandleType.FILE:
            raise ValueError(f"Invalid handle type: {self.handle_type}, expected FILE")
        return self.data

    def get_tensor_handle_list(self) -> List[TensorSharedHandle]:
        if self.handle_type == AccessHandleType.TENSOR_HANDLE:
            return list(self.data)
        if self.handle_type == AccessHandleType.TENSOR:
            return [_map_layer(t, TensorSharedHandle) for t in self.data]
        raise ValueError(f"Invalid handle type: {self.handle_type}, expected TENSOR_HANDLE or TENSOR")


def _map_layer(layer, fn):
    """Apply fn to a layer entry: one tensor/handle, or a [K, V] sequence."""
    if isinstance(layer, (list, tuple)):
        return [fn(x) for x in layer]
    return fn(layer)


def _first_leaf(layers):
    x = layers[0]
    return x[0] if isinstance(x, (list, tuple)) else x


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
    # False: ordinary pageable memory (enough for a worker that only does file I/O)
    pinned: bool = True

    def allocate(self) -> torch.Tensor:
        if not self.pinned:
            return torch.empty(self.layout.get_total_elements(), dtype=self.dtype)
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
        kind = AccessHandleType.TENSOR if isinstance(_first_leaf(data), torch.Tensor) \
            else AccessHandleType.TENSOR_HANDLE
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


class SSDAllocator:
    """SSD cache files (allocator.py:132-206).  The blocks of `layout` are
    split evenly over the directories of `cache_dir` (one per device); each
    device holds ceil(blocks_per_device / num_blocks_per_file) files named
    ``{file_prefix}_{device}_{file}.bin``, each truncated to
    num_blocks_per_file * block bytes, where num_blocks_per_file is the
    smaller of max_blocks_per_file and what the first directory's free space
    holds.  The handle's data is {device: [paths]}."""

    @classmethod
    def allocate(cls, layout: KVCacheLayout, dtype: torch.dtype, **kwargs: Any) -> StorageHandle:
        cache_dir = kwargs.get("cache_dir")
        file_prefix = kwargs.get("file_prefix", "flexkv_ssd_cache")
        cfg_max = kwargs.get("max_blocks_per_file", -1)
        if cfg_max == -1:
            cfg_max = int(1e9)
        if cache_dir is None:
            raise ValueError("cache_dir is required for SSD allocator")
        if isinstance(cache_dir, str):
            cache_dir = [cache_dir]
        for d in cache_dir:
            os.makedirs(d, exist_ok=True)
            if not os.path.isdir(d):
                raise ValueError("cache_dir must be a directory")
        if not isinstance(file_prefix, str):
            raise ValueError("file_prefix must be a string")
        num_devices = len(cache_dir)
        if layout.num_block % num_devices != 0:
            raise ValueError(f"num_ssd_blocks ({layout.num_block}) must be a multiple of "
                             f"num_ssd_devices ({num_devices})")
        per_device = layout.num_block // num_devices
        block_size = layout.get_elements_per_block() * dtype.itemsize
        num_blocks_per_file = min(cls.get_file_size_limit(cache_dir[0]) // block_size, cfg_max)
        if num_blocks_per_file <= 0:
            raise ValueError(f"no room for one {block_size}-byte block in {cache_dir[0]}")
        files_per_device = (per_device + num_blocks_per_file - 1) // num_blocks_per_file
        file_size = num_blocks_per_file * block_size
        ssd_files: Dict[int, List[str]] = {}
        for i, d in enumerate(cache_dir):
            ssd_files[i] = []
            for j in range(files_per_device):
                path = os.path.join(d, f"{file_prefix}_{i}_{j}.bin")
                with open(path, "wb+", buffering=0) as f:
                    cls._create_file(f, file_size)
                ssd_files[i].append(path)
        flexkv_logger.info(f"SSD allocate {num_devices} device(s) x {files_per_device} file(s) "
                           f"of {file_size / 2**30:.3f} GiB")
        return StorageHandle(AccessHandleType.FILE, ssd_files, layout, dtype,
                             num_blocks_per_file=num_blocks_per_file)

    @classmethod
    def _create_file(cls, file: BinaryIO, size: int) -> None:
        try:
            os.truncate(file.fileno(), size)
        except OSError as e:
            raise RuntimeError(f"Failed to initialize file: {e}") from e
        file.flush()
        os.fsync(file.fileno())

    @classmethod
    def from_raw_data(cls, data: Union[str, List[str]], layout: KVCacheLayout,
                      dtype: torch.dtype, **kwargs: Any) -> StorageHandle:
        raise NotImplementedError

    @classmethod
    def free(cls, handle: StorageHandle) -> None:
        pass

    @staticmethod
    def get_file_size_limit(path: str) -> int:
        st = os.statvfs(path)
        return st.f_frsize * st.f_bavail
