"""KV-cache layouts and their element strides.

Same public interface and results as the reference's KVCacheLayout
(flexkv/common/storage.py:18-155):
  LAYERWISE shape [layer, kv, block, token, head, dim]
  BLOCKWISE shape [block, layer, kv, token, head, dim]
with kv = 1 for MLA.  Strides are in elements.  A stride is derived here as
the product of the extents after that axis in the layout's axis order, which
gives the reference's formulas (storage.py:124-149):
  LAYERWISE layer = kv*N*t*h*d, kv = N*t*h*d, block = t*h*d
  BLOCKWISE layer = kv*t*h*d,   kv = t*h*d,   block = L*kv*t*h*d
"""
from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum
from math import prod
from typing import Dict, Optional, Tuple

import torch


class KVCacheLayoutType(Enum):
    LAYERWISE = "LAYERWISE"
    BLOCKWISE = "BLOCKWISE"


_AXES = {
    KVCacheLayoutType.LAYERWISE: ("layer", "kv", "block", "token", "head", "dim"),
    KVCacheLayoutType.BLOCKWISE: ("block", "layer", "kv", "token", "head", "dim"),
}


@dataclass
class KVCacheLayout:
    type: KVCacheLayoutType
    num_layer: int
    num_block: int
    tokens_per_block: int
    num_head: int
    head_size: int
    is_mla: bool = False
    _kv_shape: Optional[torch.Size] = field(default=None, repr=False, compare=False)

    def __post_init__(self) -> None:
        if self.type not in _AXES:
            raise ValueError(f"Invalid KVCacheLayoutType: {self.type}")
        self._kv_shape = torch.Size(self._extents()[a] for a in _AXES[self.type])

    @property
    def _kv_dim(self) -> int:
        return 1 if self.is_mla else 2

    def _extents(self) -> Dict[str, int]:
        return {"layer": self.num_layer, "kv": self._kv_dim, "block": self.num_block,
                "token": self.tokens_per_block, "head": self.num_head, "dim": self.head_size}

    def _stride(self, axis: str) -> int:
        order = _AXES[self.type]
        ext = self._extents()
        return prod(ext[a] for a in order[order.index(axis) + 1:])

    @property
    def kv_shape(self) -> torch.Size:
        return self._kv_shape

    def __eq__(self, other: object) -> bool:
        if not isinstance(other, KVCacheLayout):
            return NotImplemented
        return (self.type, self.num_layer, self.num_block, self.tokens_per_block,
                self.num_head, self.head_size, self.is_mla) == \
               (other.type, other.num_layer, other.num_block, other.tokens_per_block,
                other.num_head, other.head_size, other.is_mla)

    def _replace(self, **kw) -> "KVCacheLayout":
        args = dict(type=self.type, num_layer=self.num_layer, num_block=self.num_block,
                    tokens_per_block=self.tokens_per_block, num_head=self.num_head,
                    head_size=self.head_size, is_mla=self.is_mla)
        args.update(kw)
        return KVCacheLayout(**args)

    def div_block(self, num_chunks: int, padding: bool = False) -> "KVCacheLayout":
        if padding:
            return self._replace(num_block=-(-self.num_block // num_chunks))
        assert self.num_block % num_chunks == 0, \
            f"num_block {self.num_block} must be divisible by num_chunks {num_chunks}"
        return self._replace(num_block=self.num_block // num_chunks)

    def div_layer(self, num_chunks: int) -> "KVCacheLayout":
        assert self.num_layer % num_chunks == 0, \
            f"num_layer {self.num_layer} must be divisible by num_chunks {num_chunks}"
        return self._replace(num_layer=self.num_layer // num_chunks)

    def div_head(self, num_chunks: int) -> "KVCacheLayout":
        assert self.num_head % num_chunks == 0, \
            f"num_head {self.num_head} must be divisible by num_chunks {num_chunks}"
        return self._replace(num_head=self.num_head // num_chunks)

    def get_chunk_size(self) -> int:
        return self.tokens_per_block * self.num_head * self.head_size

    def get_layer_stride(self) -> int:
        return self._stride("layer")

    def get_block_stride(self) -> int:
        return self._stride("block")

    def get_kv_stride(self) -> int:
        return self._stride("kv")

    def get_total_elements(self) -> int:
        return prod(self.kv_shape)

    def get_elements_per_block(self) -> int:
        return self.get_total_elements() // self.num_block

    def byte_strides(self, dtype: torch.dtype) -> Tuple[int, int, int, int]:
        """(chunk, kv, layer, block) strides in bytes for element type dtype."""
        es = torch.empty((), dtype=dtype).element_size()
        return (self.get_chunk_size() * es, self.get_kv_stride() * es,
                self.get_layer_stride() * es, self.get_block_stride() * es)
