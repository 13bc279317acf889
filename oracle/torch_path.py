"""The reference's torch-backend float math, restated op for op (CPU).

Each function performs the same torch operations in the same order and dtype
as the reference, so the roundings (bf16 after every op, fp32 reductions in
RMSNorm, fp32 RoPE angles) are the reference's own. Inputs are CPU tensors.
"""

from __future__ import annotations

from math import sqrt

import torch


def inverse_frequencies(head_dim: int, *, theta: float) -> torch.Tensor:
    """theta ** (-arange(0, Dh, 2) / Dh) in fp32 (tokserve/engine/rope.py:28-49)."""

    if head_dim < 2 or head_dim % 2 != 0:
        raise ValueError("head_dim must be a positive even integer")
    indices = torch.arange(0, head_dim, 2, dtype=torch.float32)
    return theta ** (-indices / head_dim)


def rotary_cos_sin(
    positions: torch.Tensor, head_dim: int, *, theta: float, dtype: torch.dtype
) -> tuple[torch.Tensor, torch.Tensor]:
    """(T, Dh) cos/sin: fp32 outer(pos, inv_freq), duplicated, cast to dtype.

    tokserve/engine/rope.py:52-87.
    """

    if torch.any(positions < 0):
        raise ValueError("positions must be nonnegative")
    frequencies = inverse_frequencies(head_dim, theta=theta)
    angles = torch.outer(positions.to(torch.float32), frequencies)
    duplicated = torch.cat((angles, angles), dim=-1)
    return duplicated.cos().to(dtype), duplicated.sin().to(dtype)


def rotate_half(inputs: torch.Tensor) -> torch.Tensor:
    """cat(-x2, x1) on the last dimension (tokserve/engine/rope.py:90-103)."""

    half = inputs.shape[-1] // 2
    return torch.cat((-inputs[..., half:], inputs[..., :half]), dim=-1)


def apply_rope(
    query: torch.Tensor, key: torch.Tensor, positions: torch.Tensor, *, theta: float
) -> tuple[torch.Tensor, torch.Tensor]:
    """q*cos + rotate_half(q)*sin for (B, H, T, Dh) Q and K (tokserve/engine/rope.py:106-153)."""

    cosine, sine = rotary_cos_sin(positions, query.shape[-1], theta=theta, dtype=query.dtype)
    cosine = cosine[None, None, :, :]
    sine = sine[None, None, :, :]
    return (
        query * cosine + rotate_half(query) * sine,
        key * cosine + rotate_half(key) * sine,
    )


def rms_norm(inputs: torch.Tensor, weight: torch.Tensor, epsilon: float) -> torch.Tensor:
    """weight * to_in(x32 * rsqrt(mean(x32^2) + eps)) (tokserve/engine/layers.py:29-42)."""

    input_dtype = inputs.dtype
    float_inputs = inputs.to(torch.float32)
    mean_square = float_inputs.pow(2).mean(dim=-1, keepdim=True)
    normalized = float_inputs * torch.rsqrt(mean_square + epsilon)
    return weight * normalized.to(input_dtype)


def repeat_key_value(inputs: torch.Tensor, *, num_groups: int) -> torch.Tensor:
    """(B, Hkv, T, Dh) -> (B, Hkv*G, T, Dh) (tokserve/engine/attention.py:42-55)."""

    return inputs.repeat_interleave(num_groups, dim=1)


def causal_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    query_position_offset: int = 0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """softmax(q k^T / sqrt(Dh), mask k <= offset + i) v in the input dtype.

    tokserve/engine/attention.py:58-127.
    """

    query_length = query.shape[-2]
    key_length = key.shape[-2]
    head_dim = query.shape[-1]
    if query_position_offset + query_length > key_length:
        raise ValueError("query positions cannot exceed the key sequence length")
    scores = torch.matmul(query, key.transpose(-1, -2)) / sqrt(head_dim)
    query_positions = torch.arange(query_position_offset, query_position_offset + query_length)
    key_positions = torch.arange(key_length)
    causal_mask = key_positions.unsqueeze(0) <= query_positions.unsqueeze(1)
    scores = scores.masked_fill(~causal_mask[None, None, :, :], float("-inf"))
    weights = torch.softmax(scores, dim=-1)
    return torch.matmul(weights, value), weights


def gqa_attention(
    query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, *, query_position_offset: int
) -> torch.Tensor:
    """The torch backend's attention step: repeat K/V to Hq heads, then causal_attention.

    tokserve/engine/attention.py:341-356.
    """

    groups = query.shape[1] // key.shape[1]
    output, _ = causal_attention(
        query,
        repeat_key_value(key, num_groups=groups),
        repeat_key_value(value, num_groups=groups),
        query_position_offset=query_position_offset,
    )
    return output


def online_softmax_update(
    running_max: torch.Tensor,
    running_sum: torch.Tensor,
    accumulator: torch.Tensor,
    scores: torch.Tensor,
    values: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """One tile of the online softmax (tokserve/engine/tiled_attention.py:122-166)."""

    tile_max = scores.max(dim=-1, keepdim=True).values
    new_max = torch.maximum(running_max, tile_max)
    previous_scale = torch.exp(running_max - new_max)
    probabilities = torch.exp(scores - new_max)
    new_sum = previous_scale * running_sum + probabilities.sum(dim=-1, keepdim=True)
    new_accumulator = previous_scale * accumulator + torch.matmul(probabilities, values)
    return new_max, new_sum, new_accumulator


def tiled_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    query_position_offset: int = 0,
    query_block_size: int = 16,
    key_block_size: int = 16,
) -> torch.Tensor:
    """Causal GQA by online-softmax tiles in fp32 (tokserve/engine/tiled_attention.py:8-119)."""

    batch, num_q_heads, query_length, head_dim = query.shape
    key_length = key.shape[2]
    groups = num_q_heads // key.shape[1]
    kv_index = torch.arange(num_q_heads) // groups
    grouped_key = key.index_select(1, kv_index)
    grouped_value = value.index_select(1, kv_index)
    output = torch.empty_like(query)
    scale = 1.0 / sqrt(head_dim)
    for q0 in range(0, query_length, query_block_size):
        q1 = min(q0 + query_block_size, query_length)
        q_tile = query[:, :, q0:q1, :].to(torch.float32)
        running_max = torch.full((batch, num_q_heads, q1 - q0, 1), float("-inf"))
        running_sum = torch.zeros_like(running_max)
        accumulator = torch.zeros((batch, num_q_heads, q1 - q0, head_dim))
        positions = torch.arange(query_position_offset + q0, query_position_offset + q1)
        for k0 in range(0, key_length, key_block_size):
            k1 = min(k0 + key_block_size, key_length)
            k_tile = grouped_key[:, :, k0:k1, :].to(torch.float32)
            v_tile = grouped_value[:, :, k0:k1, :].to(torch.float32)
            scores = torch.matmul(q_tile, k_tile.transpose(-1, -2)) * scale
            allowed = torch.arange(k0, k1)[None, :] <= positions[:, None]
            scores = scores.masked_fill(~allowed[None, None, :, :], float("-inf"))
            running_max, running_sum, accumulator = online_softmax_update(
                running_max, running_sum, accumulator, scores, v_tile
            )
        output[:, :, q0:q1, :] = (accumulator / running_sum).to(query.dtype)
    return output


def select_greedy(logits: torch.Tensor) -> torch.Tensor:
    """argmax(dim=-1, keepdim=True), first index on ties (tokserve/generation/greedy.py:6-18)."""

    return torch.argmax(logits, dim=-1, keepdim=True)
