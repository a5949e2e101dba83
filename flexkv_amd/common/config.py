"""Model and cache configuration for the GPU<->CPU transfer path.

ModelConfig matches the reference (flexkv/common/config.py:10-25).  CacheConfig
keeps the fields that shape this path and its SSD tier (config.py:27-57):
block size, host layout and pinning, host block count, the per-direction
transfer knobs, and the SSD cache (enable_ssd, layout, block count, files).
The remote and trace fields belong to parts this package does not implement
and are not present.  Defaults that differ from the reference: the host and
SSD layouts are BLOCKWISE (one block's layers contiguous, which the device
path and the SSD path both move as single runs), the host cache is pinned, and
both directions use the copy-engine path: on MI355X it moves whole-block
transfers as fast as the zero-copy kernel (56.4 / 56.7 GB/s against 56.5 /
57.2) while leaving the compute units to the model (GEMMs beside a 2 GiB D2H
slow down 7% instead of 120%), and it hands small or fine-grained transfers to
the zero-copy kernel by itself.  With a LAYERWISE host cache the copy engines
move one rect copy per block at about 47 GB/s.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Union

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
    enable_ssd: bool = False
    use_pinned_memory: bool = True
    gpu_kv_layout_type: KVCacheLayoutType = KVCacheLayoutType.LAYERWISE
    cpu_kv_layout_type: KVCacheLayoutType = KVCacheLayoutType.BLOCKWISE
    ssd_kv_layout_type: KVCacheLayoutType = KVCacheLayoutType.BLOCKWISE
    num_cpu_blocks: int = 1000000
    num_ssd_blocks: int = 10000000
    # False = zero-copy kernel, True = SDMA engines via on-device staging
    use_ce_transfer_h2d: bool = True
    use_ce_transfer_d2h: bool = True
    # compute units the zero-copy kernel may occupy (-1 = automatic)
    transfer_sms_h2d: int = 8
    transfer_sms_d2h: int = 8
    # SSD cache: one directory per device; -1 = no per-file block limit
    max_blocks_per_file: int = 32000
    ssd_cache_dir: Optional[Union[str, List[str]]] = None
    # io_uring ring depth for SSD transfers (0 = pread/pwrite threads) and
    # the ring's io_uring_setup flags
    ssd_cache_iouring_entries: int = 0
    ssd_cache_iouring_flags: int = 0
    # threads per SSD device for one transfer (worker.py:573 uses 32)
    ssd_threads_per_device: int = 32
