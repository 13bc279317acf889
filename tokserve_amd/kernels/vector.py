"""Drop-in one-dimensional vector addition (tokserve/kernels/vector.py).

Same checks and messages as the reference wrapper (vector.py:6-41); the sum
runs in the tks_vector_add HIP kernel. Importing this module does not load the
HIP library.
"""

from __future__ import annotations

import torch

from tokserve_amd.kernels import ops

__all__ = ["vector_add"]


def vector_add(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """Add matching one-dimensional HIP vectors."""

    if x.ndim != 1 or y.ndim != 1:
        raise ValueError("x and y must be one-dimensional")
    if x.shape != y.shape:
        raise ValueError("x and y must have matching shapes")
    if x.device.type != "cuda" or y.device.type != "cuda":
        raise ValueError("x and y must be CUDA tensors")
    if x.device != y.device:
        raise ValueError("x and y must use the same CUDA device")
    if x.dtype != y.dtype:
        raise ValueError("x and y must have the same dtype")
    if x.dtype not in (torch.float32, torch.float16):
        raise TypeError("vector_add supports float32 and float16")
    if not x.is_contiguous() or not y.is_contiguous():
        raise ValueError("x and y must be contiguous")
    if x.numel() == 0:
        return torch.empty_like(x)
    return ops.vector_add(x, y)
