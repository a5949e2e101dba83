"""Storage handles for the GPU, host and SSD caches (role of
flexkv/storage/storage_engine.py:15-190, CPU, GPU and SSD tiers).

The host cache is allocated pinned (CacheConfig.use_pinned_memory, default
True here; pageable memory cannot be used by the device path)."""
from __future__ import annotations

from typing import Any, Dict, List, Optional, Tuple, Union

import torch

from ..common.config import CacheConfig, ModelConfig
from ..common.memory_handle import TensorSharedHandle
from ..common.storage import KVCacheLayout, KVCacheLayoutType
from ..common.transfer import DeviceType
from .allocator import CPUAllocator, GPUAllocator, SSDAllocator, StorageHandle


class StorageEngine:
    def __init__(self, model_config: ModelConfig, cache_config: CacheConfig) -> None:
        self._storage_handles: Dict[Tuple[DeviceType, int], StorageHandle] = {}
        self._model_config = model_config
        self._cache_config = cache_config
        if cache_config.gpu_kv_layout_type != KVCacheLayoutType.LAYERWISE:
            raise ValueError("Only layerwise layout is supported for GPU")
        self._cpu_layout: Optional[KVCacheLayout] = None
        if cache_config.enable_cpu:
            self._cpu_layout = KVCacheLayout(
                type=cache_config.cpu_kv_layout_type, num_layer=model_config.num_layers,
                num_block=cache_config.num_cpu_blocks,
                tokens_per_block=cache_config.tokens_per_block,
                num_head=model_config.num_kv_heads, head_size=model_config.head_size,
                is_mla=model_config.use_mla)
            self.allocate(DeviceType.CPU, self._cpu_layout, model_config.dtype,
                          pin_memory=cache_config.use_pinned_memory)
        self._ssd_layout: Optional[KVCacheLayout] = None
        if cache_config.enable_ssd:
            if self._cpu_layout is None or cache_config.ssd_kv_layout_type != self._cpu_layout.type:
                raise ValueError("SSD layout type must be the same as CPU layout type: "
                                 f"{None if self._cpu_layout is None else self._cpu_layout.type}")
            self._ssd_layout = KVCacheLayout(
                type=cache_config.ssd_kv_layout_type, num_layer=model_config.num_layers,
                num_block=cache_config.num_ssd_blocks,
                tokens_per_block=cache_config.tokens_per_block,
                num_head=model_config.num_kv_heads, head_size=model_config.head_size,
                is_mla=model_config.use_mla)
            self.allocate(DeviceType.SSD, self._ssd_layout, model_config.dtype,
                          cache_dir=cache_config.ssd_cache_dir,
                          max_blocks_per_file=cache_config.max_blocks_per_file)

    def register_gpu_blocks(self, gpu_blocks: List[Union[TensorSharedHandle, torch.Tensor]],
                            gpu_layout: KVCacheLayout, device_id: int = 0,
                            dtype: torch.dtype = torch.float16) -> None:
        self.allocate(DeviceType.GPU, gpu_layout, dtype, device_id=device_id, raw_data=gpu_blocks)

    def allocate(self, device_type: DeviceType, layout: KVCacheLayout, dtype: torch.dtype,
                 device_id: int = 0, raw_data: Optional[Any] = None, **kwargs: Any) -> bool:
        key = (device_type, device_id)
        if key in self._storage_handles:
            return False
        if device_type == DeviceType.CPU:
            handle = CPUAllocator.from_raw_data(raw_data, layout, dtype) if raw_data is not None \
                else CPUAllocator.allocate(layout, dtype, pin_memory=kwargs.get("pin_memory", True))
        elif device_type == DeviceType.GPU:
            handle = GPUAllocator.from_raw_data(raw_data, layout, dtype, device_id=device_id) \
                if raw_data is not None else \
                GPUAllocator.allocate(layout, dtype, device_id=device_id,
                                      num_chunks=kwargs.get("num_chunks", layout.num_layer))
        elif device_type == DeviceType.SSD:
            if raw_data is not None:
                handle = SSDAllocator.from_raw_data(raw_data, layout, dtype)
            else:
                if not kwargs.get("cache_dir"):
                    raise ValueError("cache_dir is required for SSD allocator")
                handle = SSDAllocator.allocate(layout, dtype, cache_dir=kwargs["cache_dir"],
                                               file_prefix="flexkv_ssd_cache",
                                               max_blocks_per_file=kwargs.get(
                                                   "max_blocks_per_file", -1))
        else:
            raise ValueError(f"storage tier {device_type.name} is not provided by this package")
        self._storage_handles[key] = handle
        return True

    def get_storage_handle(self, device_type: DeviceType, device_id: int = 0) -> StorageHandle:
        key = (device_type, device_id)
        if key not in self._storage_handles:
            raise ValueError(f"no storage handle for {device_type.name}:{device_id}")
        return self._storage_handles[key]

    def has_storage(self, device_type: DeviceType, device_id: int = 0) -> bool:
        return (device_type, device_id) in self._storage_handles
