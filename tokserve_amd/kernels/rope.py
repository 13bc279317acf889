"""Drop-in RoPE (tokserve/kernels/rope.py).

`hip_apply_rope` keeps the reference operator's signature, checks and messages
(tokserve/kernels/rope.py:8-63) and returns new rotated Q and K. The cos/sin
rows come from a per-(head_dim, theta, dtype, device) RotaryTable (the values
rotary_cos_sin computes, tokserve/engine/rope.py:52-87) grown to the largest
position seen; the kernel gathers rows by position. `triton_apply_rope` is the
same function under the reference's name.
"""

from __future__ import annotations

import torch

from tokserve_amd.kernels import ops

__all__ = ["hip_apply_rope", "triton_apply_rope", "rotary_table"]

_TABLES: dict[tuple, ops.RotaryTable] = {}


def rotary_table(
    head_dim: int, *, theta: float, dtype: torch.dtype, device: torch.device, length: int
) -> ops.RotaryTable:
    """The shared table for (head_dim, theta, dtype, device), covering [0, length)."""

    key = (head_dim, float(theta), dtype, torch.device(device))
    table = _TABLES.get(key)
    if table is None:
        table = ops.RotaryTable(
            head_dim, theta=theta, max_position=max(length, 1), dtype=dtype, device=device
        )
        _TABLES[key] = table
    else:
        table.ensure(length)
    return table


def hip_apply_rope(
    query: torch.Tensor,
    key: torch.Tensor,
    positions: torch.Tensor,
    *,
    theta: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Apply the half-rotation RoPE to Q (B, Hq, T, Dh) and K (B, Hkv, T, Dh)."""

    if query.ndim != 4 or key.ndim != 4:
        raise ValueError("query and key must have shape (B, H, T, Dh)")
    if query.shape[0] != key.shape[0]:
        raise ValueError("query and key batch sizes must match")
    if query.shape[-2:] != key.shape[-2:]:
        raise ValueError("query and key sequence and head dimensions must match")
    if query.dtype != key.dtype:
        raise ValueError("query and key must use the same dtype")
    if query.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise TypeError("query and key must use a supported floating dtype")
    if not query.is_cuda or not key.is_cuda or not positions.is_cuda:
        raise ValueError("query, key, and positions must be CUDA tensors")
    if query.device != key.device or positions.device != query.device:
        raise ValueError("query, key, and positions must use the same device")
    sequence_length = query.shape[-2]
    head_dim = query.shape[-1]
    if positions.shape != (sequence_length,):
        raise ValueError("positions must have shape (T,)")
    if positions.dtype not in (torch.int32, torch.int64):
        raise TypeError("positions must contain integers")
    if head_dim < 2 or head_dim % 2 != 0:
        raise ValueError("head_dim must be a positive even integer")
    if theta <= 0.0:
        raise ValueError("theta must be positive")
    if sequence_length == 0 or query.numel() == 0:
        return query.clone(), key.clone()
    lowest, highest = (int(v) for v in torch.aminmax(positions))
    if lowest < 0:
        raise ValueError("positions must be nonnegative")
    table = rotary_table(head_dim, theta=theta, dtype=query.dtype, device=query.device,
                         length=highest + 1)
    return ops.rope(query, key, positions, table)


triton_apply_rope = hip_apply_rope
