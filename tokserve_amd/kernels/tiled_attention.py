"""Drop-in causal tiled GQA over contiguous Q/K/V (tokserve/kernels/tiled_attention.py).

`hip_tiled_attention` keeps the reference operator's signature, checks and
messages (tokserve/kernels/tiled_attention.py:9-58). K and V of shape
(B, Hkv, Tk, Dh) are exactly a one-layer paged pool [1, NB=B, Hkv, BS=Tk, Dh]
with one block per batch row, so the operator runs the chunked-prefill kernel
with block table [[0], [1], ..., [B-1]]: query i of row b sits at position
query_position_offset + i and sees keys 0 .. query_position_offset + i.
`triton_tiled_attention` is the same function under the reference's name.
"""

from __future__ import annotations

import torch

from tokserve_amd.kernels import ops

__all__ = ["hip_tiled_attention", "triton_tiled_attention"]

# Query heads per KV head the kernels take in one launch.
MAX_GROUP = 16


def hip_tiled_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    query_position_offset: int = 0,
) -> torch.Tensor:
    """Apply causal tiled GQA to Q (B, Hq, Tq, Dh) and K/V (B, Hkv, Tk, Dh)."""

    if query.ndim != 4 or key.ndim != 4 or value.ndim != 4:
        raise ValueError("query, key, and value must have shape (B, H, T, Dh)")
    if key.shape != value.shape:
        raise ValueError("key and value shapes must match")
    if query.shape[0] != key.shape[0]:
        raise ValueError("query and key batch sizes must match")
    if query.shape[1] % key.shape[1] != 0:
        raise ValueError("query head count must be divisible by KV head count")
    if query.shape[-1] != key.shape[-1]:
        raise ValueError("query and key head dimensions must match")
    if query.shape[2] < 1 or key.shape[2] < 1:
        raise ValueError("sequence lengths must be positive")
    if query.shape[-1] < 1 or query.shape[-1] > 128:
        raise ValueError("head_dim must be in the interval [1, 128]")
    if query_position_offset < 0:
        raise ValueError("query_position_offset must be nonnegative")
    if query_position_offset + query.shape[2] > key.shape[2]:
        raise ValueError("query positions cannot exceed key sequence length")
    if not query.is_cuda or not key.is_cuda or not value.is_cuda:
        raise ValueError("query, key, and value must be CUDA tensors")
    if query.device != key.device or key.device != value.device:
        raise ValueError("query, key, and value must use the same device")
    if query.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise TypeError("query, key, and value must use float32, float16, or bfloat16")
    if key.dtype != query.dtype or value.dtype != query.dtype:
        raise ValueError("query, key, and value must use the same dtype")
    batch, num_q_heads, query_length, head_dim = query.shape
    num_kv_heads, key_length = key.shape[1], key.shape[2]
    if num_q_heads // num_kv_heads > MAX_GROUP:
        raise ValueError(f"at most {MAX_GROUP} query heads per KV head are supported")

    key_pool = key.contiguous().unsqueeze(0)
    value_pool = value.contiguous().unsqueeze(0)
    # Packed (B*Tq, Hq, Dh) query and output rows, sequence-major.
    packed_query = query.transpose(1, 2).reshape(batch * query_length, num_q_heads, head_dim)
    packed_out = torch.empty_like(packed_query, memory_format=torch.contiguous_format)
    visible = query_position_offset + query_length
    meta = torch.cat(
        (
            torch.arange(batch, dtype=torch.int32),
            torch.full((batch,), visible, dtype=torch.int32),
            torch.arange(0, (batch + 1) * query_length, query_length, dtype=torch.int32),
        )
    ).to(query.device)
    block_tables = meta[:batch].view(batch, 1)
    seq_lens = meta[batch : 2 * batch]
    cu_seqlens_q = meta[2 * batch :]
    ops.paged_attention_prefill(
        packed_query, key_pool, value_pool, block_tables, seq_lens, cu_seqlens_q,
        layer_index=0, max_query_len=query_length, max_seq_len=visible, out=packed_out,
    )
    return packed_out.view(batch, query_length, num_q_heads, head_dim).transpose(1, 2).contiguous()


triton_tiled_attention = hip_tiled_attention
