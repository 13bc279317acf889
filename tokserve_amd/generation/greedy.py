"""Greedy token selection (tokserve/generation/greedy.py:6-18).

The first index of each row's maximum, NaN counting as the maximum, as
torch.argmax(dim=-1, keepdim=True) gives it; computed by the tks_argmax kernel
(one launch over the whole (B, V) block of logits).
"""

from __future__ import annotations

import torch

from tokserve_amd.kernels import ops

__all__ = ["select_greedy"]


def select_greedy(logits: torch.Tensor) -> torch.Tensor:
    """(B, V) logits -> (B, 1) int64 indices of the first row maximum."""

    if logits.ndim != 2:
        raise ValueError("logits must have shape (B, V)")
    if logits.shape[0] < 1:
        raise ValueError("logits must contain at least one batch row")
    if logits.shape[1] < 1:
        raise ValueError("vocabulary size must be positive")
    return ops.greedy_argmax(logits)
