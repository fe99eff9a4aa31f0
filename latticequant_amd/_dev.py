"""Device plumbing shared by the API modules: run on the current ROCm device,
hand results back on the caller's device."""
from __future__ import annotations

import torch

from . import _lib as L


def to_gpu(t: torch.Tensor, dtype=None) -> torch.Tensor:
    L.lib()   # verifies the kernel library and the GPU
    if dtype is not None:
        t = t.to(dtype)
    if not t.is_cuda:
        t = t.to(torch.device("cuda", torch.cuda.current_device()))
    return t.contiguous()


def back(t: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    return t if like.is_cuda else t.to(like.device)
