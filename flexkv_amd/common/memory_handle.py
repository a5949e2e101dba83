"""Cross-process GPU tensor handles (role of flexkv/common/memory_handle.py:16-53).

A handle carries torch's IPC reduction of a device tensor (HIP IPC through
torch.multiprocessing.reductions) and rebuilds the tensor in another process.
Unlike the reference, a failed import raises instead of returning an empty
tensor, so a worker cannot start on a half-imported cache.
"""
from __future__ import annotations

from typing import Any, Callable, List

import torch
import torch.multiprocessing.reductions as reductions


class TensorSharedHandle:
    def __init__(self, tensor: torch.Tensor) -> None:
        if not tensor.is_cuda:
            raise ValueError("Only support device (HIP) tensor sharing")
        self.device: torch.device = tensor.device
        self.rebuild_func: Callable
        self.rebuild_args: List[Any]
        self.rebuild_func, self.rebuild_args = reductions.reduce_tensor(tensor)

    def get_tensor(self) -> torch.Tensor:
        try:
            tensor = self.rebuild_func(*self.rebuild_args)
        except Exception as e:  # pragma: no cover - exercised only with a GPU
            raise RuntimeError(f"importing shared device tensor failed: {e}") from e
        if not isinstance(tensor, torch.Tensor):
            raise RuntimeError("shared handle did not rebuild a tensor")
        if tensor.device != self.device:
            tensor = tensor.to(self.device)
        return tensor
