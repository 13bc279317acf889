"""Rotary position embeddings under the reference's module path (tokserve/engine/rope.py).

Same functions, signatures, checks and messages as the reference's
(rope.py:6-153). The table math (`inverse_frequencies`, `rotary_cos_sin`) is
torch arithmetic on the positions' device, exactly the reference's (fp32
inverse frequencies from torch's pow, fp32 angles from one outer product, the
halves duplicated, cast to the dtype); `apply_rope` rotates through the HIP
RoPE kernel, which reads those same cos/sin values from a cached table and
rounds each product to the dtype before the add, as the reference's torch
expression does (bit-identical; the kernel runs on HIP tensors only).
"""

from __future__ import annotations

import torch

from tokserve_amd.kernels.rope import hip_apply_rope

__all__ = ["positions_for_sequence", "inverse_frequencies", "rotary_cos_sin", "rotate_half",
           "apply_rope"]


def positions_for_sequence(sequence_length: int, *, offset: int,
                           device: torch.device) -> torch.Tensor:
    """Absolute positions offset .. offset + sequence_length - 1 (int64)."""

    if sequence_length < 1:
        raise ValueError("sequence_length must be positive")
    if offset < 0:
        raise ValueError("offset must be nonnegative")
    return torch.arange(offset, offset + sequence_length, dtype=torch.int64, device=device)


def inverse_frequencies(head_dim: int, *, theta: float, device: torch.device) -> torch.Tensor:
    """theta ** (-(0, 2, 4, ...) / head_dim) in fp32 on `device`."""

    if head_dim < 2 or head_dim % 2 != 0:
        raise ValueError("head_dim must be a positive even integer")
    if theta <= 0.0:
        raise ValueError("theta must be positive")
    even = torch.arange(0, head_dim, 2, dtype=torch.float32, device=device)
    return theta ** (-even / head_dim)


def rotary_cos_sin(positions: torch.Tensor, head_dim: int, *, theta: float,
                   dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """(T, Dh) cosine and sine of the fp32 angles positions x inverse_frequencies."""

    if positions.ndim != 1:
        raise ValueError("positions must have shape (T,)")
    if positions.dtype not in (torch.int32, torch.int64):
        raise TypeError("positions must contain integers")
    if torch.any(positions < 0):
        raise ValueError("positions must be nonnegative")
    angles = torch.outer(positions.to(torch.float32),
                         inverse_frequencies(head_dim, theta=theta, device=positions.device))
    both = torch.cat((angles, angles), dim=-1)
    return both.cos().to(dtype), both.sin().to(dtype)


def rotate_half(inputs: torch.Tensor) -> torch.Tensor:
    """(x1, x2) -> (-x2, x1) on the last dimension."""

    if inputs.ndim < 1:
        raise ValueError("inputs must have at least one dimension")
    width = inputs.shape[-1]
    if width < 2 or width % 2 != 0:
        raise ValueError("final dimension must be a positive even integer")
    first, second = inputs.split(width // 2, dim=-1)
    return torch.cat((-second, first), dim=-1)


def apply_rope(query: torch.Tensor, key: torch.Tensor, positions: torch.Tensor, *,
               theta: float) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotate Q (B, Hq, T, Dh) and K (B, Hkv, T, Dh) at positions (T,) on the GPU."""

    if query.ndim != 4 or key.ndim != 4:
        raise ValueError("query and key must have shape (B, H, T, Dh)")
    if query.device != key.device:
        raise ValueError("query and key must use the same device")
    if positions.device != query.device:
        raise ValueError("positions must use the same device as query and key")
    if query.shape[0] != key.shape[0]:
        raise ValueError("query and key batch sizes must match")
    if query.shape[-2:] != key.shape[-2:]:
        raise ValueError("query and key sequence and head dimensions must match")
    if positions.shape != (query.shape[-2],):
        raise ValueError("positions must have shape (T,)")
    return hip_apply_rope(query, key, positions, theta=theta)
