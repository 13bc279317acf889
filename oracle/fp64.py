"""float64 NumPy closed forms used to pin the torch-path restatement.

These are textbook formulas written independently of the reference's torch
code: the reference's own NumPy model (tokserve/reference/llama/rope.py:8-121,
tokserve/reference/llama/layers.py:8-33) and the test suite's
independent_attention (tests/unit/engine/test_attention_contract.py:15-59).
"""

from __future__ import annotations

import numpy as np


def attention(
    query: np.ndarray, key: np.ndarray, value: np.ndarray, *, query_position_offset: int
) -> np.ndarray:
    """Causal GQA softmax attention, one (query, key) pair at a time in float64.

    query (B, Hq, Tq, Dh), key/value (B, Hkv, Tk, Dh); head h reads KV head h // G.
    """

    q = np.asarray(query, dtype=np.float64)
    k = np.asarray(key, dtype=np.float64)
    v = np.asarray(value, dtype=np.float64)
    batch, num_q_heads, tq, dh = q.shape
    groups = num_q_heads // k.shape[1]
    out = np.zeros_like(q)
    for b in range(batch):
        for h in range(num_q_heads):
            kh = h // groups
            for i in range(tq):
                visible = query_position_offset + i + 1
                scores = k[b, kh, :visible] @ q[b, h, i] / np.sqrt(dh)
                weights = np.exp(scores - scores.max())
                weights /= weights.sum()
                out[b, h, i] = weights @ v[b, kh, :visible]
    return out


def rope(query: np.ndarray, key: np.ndarray, positions: np.ndarray, *, theta: float):
    """Half-rotation RoPE in float64: x*cos + rotate_half(x)*sin."""

    dh = query.shape[-1]
    inv_freq = theta ** (-np.arange(0, dh, 2, dtype=np.float64) / dh)
    angles = np.outer(np.asarray(positions, dtype=np.float64), inv_freq)
    angles = np.concatenate((angles, angles), axis=-1)
    cos, sin = np.cos(angles), np.sin(angles)

    def rotate(x: np.ndarray) -> np.ndarray:
        x = np.asarray(x, dtype=np.float64)
        half = x.shape[-1] // 2
        rotated = np.concatenate((-x[..., half:], x[..., :half]), axis=-1)
        return x * cos + rotated * sin

    return rotate(query), rotate(key)


def rms_norm(inputs: np.ndarray, weight: np.ndarray, epsilon: float) -> np.ndarray:
    """weight * x / sqrt(mean(x^2) + eps) in float64."""

    x = np.asarray(inputs, dtype=np.float64)
    return np.asarray(weight, dtype=np.float64) * x / np.sqrt(
        np.mean(x * x, axis=-1, keepdims=True) + epsilon
    )
