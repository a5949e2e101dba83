"""Model and cache configuration for the GPU<->CPU transfer path.

ModelConfig matches the reference (flexkv/common/config.py:10-25).  CacheConfig
keeps the fields that shape this path (config.py:27-51): block size, host
layout and pinning, host block count, and the per-direction transfer knobs.
The SSD, remote and trace fields belong to tiers this package does not
implement and are not present.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .storage import KVCacheLayoutType


@dataclass
class ModelConfig:
    num_layers: int
    num_kv_heads: int
    head_size: int
    use_mla: bool = False
    dtype: torch.dtype = torch.bfloat16
    tp_size: int = 1
    dp_size: int = 1

    @property
    def token_size_in_bytes(self) -> int:
        kv_dim = 1 if self.use_mla else 2
        return self.num_layers * self.num_kv_heads * self.head_size * kv_dim * self.dtype.itemsize


@dataclass
class CacheConfig:
    tokens_per_block: int = 16
    enable_cpu: bool = True
    use_pinned_memory: bool = True
    gpu_kv_layout_type: KVCacheLayoutType = KVCacheLayoutType.LAYERWISE
    cpu_kv_layout_type: KVCacheLayoutType = KVCacheLayoutType.BLOCKWISE
    num_cpu_blocks: int = 1000000
    # False = zero-copy kernel, True = copy engines via on-device staging
    use_ce_transfer_h2d: bool = False
    use_ce_transfer_d2h: bool = False
    # compute units the zero-copy kernel may occupy (-1 = automatic)
    transfer_sms_h2d: int = 8
    transfer_sms_d2h: int = 8
