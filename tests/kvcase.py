"""KV transfer problems for tests, described as multi-dimensional arrays.

Byte strides come from numpy's own ``.strides`` of the shaped arrays and the
expected result of a transfer comes from numpy fancy indexing on those shapes,
so neither shares code with the stride arithmetic under test.

GPU side: one array per layer of the call, shape [kv, NG, T, H, D] (vLLM's
per-layer [2, N, tpb, H, D] tensor, worker.py:236-246 strides).  Host side:
BLOCKWISE [NH, LT, kv, tp, T, H, D] or LAYERWISE [LT, kv, NH, tp, T, H, D]
where tp > 1 gives the tensor-parallel host chunk in which a GPU chunk lands
at byte offset rank*chunk (csrc/tp_transfer_thread_group.cpp:79-80).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List

import numpy as np

from oracle import inputs


@dataclass
class KVCase:
    layers_total: int
    num_layers: int          # layers moved by the call
    start_layer: int
    kv: int                  # 2, or 1 for MLA
    ng: int
    nh: int
    tokens: int
    heads: int
    dim: int
    dtype: type = np.uint16
    layout: str = "BLOCKWISE"
    tp: int = 1
    rank: int = 0
    gpu: List[np.ndarray] = field(default_factory=list)
    host: np.ndarray = None

    # ---- shapes -------------------------------------------------------
    def gpu_shape(self):
        return (self.kv, self.ng, self.tokens, self.heads, self.dim)

    def host_shape(self):
        tail = (self.tp, self.tokens, self.heads, self.dim)
        if self.layout == "BLOCKWISE":
            return (self.nh, self.layers_total, self.kv) + tail
        return (self.layers_total, self.kv, self.nh) + tail

    # ---- byte strides, from numpy --------------------------------------
    def strides(self):
        g = np.empty(self.gpu_shape(), self.dtype).strides
        h = np.empty(self.host_shape(), self.dtype).strides
        if self.layout == "BLOCKWISE":
            cblk, clay, ckv, crank = h[0], h[1], h[2], h[3]
        else:
            clay, ckv, cblk, crank = h[0], h[1], h[2], h[3]
        chunk = self.tokens * self.heads * self.dim * np.dtype(self.dtype).itemsize
        return dict(gpu_kv=g[0], gpu_block=g[1], cpu_kv=ckv, cpu_layer=clay, cpu_block=cblk,
                    chunk=chunk, startoff=self.rank * crank)

    # ---- data -----------------------------------------------------------
    def fill(self, seed: int, sentinel: int = 0x5A5A) -> "KVCase":
        bits = np.dtype(self.dtype).itemsize * 8
        n = int(np.prod(self.gpu_shape()))
        self.gpu = []
        for l in range(self.num_layers):
            raw = inputs.splitmix64(np.arange(n, dtype=np.uint64) +
                                    np.uint64((seed * 1000 + l) << 32))
            self.gpu.append((raw & np.uint64((1 << bits) - 1)).astype(self.dtype)
                            .reshape(self.gpu_shape()))
        self.host = np.full(self.host_shape(), sentinel & ((1 << bits) - 1), dtype=self.dtype)
        return self

    # ---- expected results by indexing ------------------------------------
    def host_view(self, host: np.ndarray) -> np.ndarray:
        """[NH, LT, kv, tp, T, H, D] view regardless of layout."""
        return host if self.layout == "BLOCKWISE" else host.transpose(2, 0, 1, 3, 4, 5, 6)

    def expect_d2h(self, gids, cids) -> np.ndarray:
        out = self.host.copy()
        hv = self.host_view(out)
        for l in range(self.num_layers):
            for k in range(self.kv):
                hv[cids, self.start_layer + l, k, self.rank] = self.gpu[l][k, gids]
        return out

    def expect_h2d(self, gids, cids, gpu_init: List[np.ndarray]) -> List[np.ndarray]:
        out = [g.copy() for g in gpu_init]
        hv = self.host_view(self.host)
        for l in range(self.num_layers):
            for k in range(self.kv):
                out[l][k, gids] = hv[cids, self.start_layer + l, k, self.rank]
        return out


def brute_force_d2h(case: KVCase, gids, cids) -> np.ndarray:
    """Element-by-element loop over (block, layer, kv, token, head, dim):
    for tiny cases only."""
    out = case.host.copy()
    hv = case.host_view(out)
    for i in range(len(gids)):
        for l in range(case.num_layers):
            for k in range(case.kv):
                for t in range(case.tokens):
                    for h in range(case.heads):
                        for d in range(case.dim):
                            hv[cids[i], case.start_layer + l, k, case.rank, t, h, d] = \
                                case.gpu[l][k, gids[i], t, h, d]
    return out
