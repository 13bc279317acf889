"""Drop-in paged attention over a PagedKVStorage (tokserve/kernels/paged_attention.py).

`hip_paged_attention` keeps the reference operator's signature, argument
meaning, checks and messages (tokserve/kernels/paged_attention.py:11-65) and
runs the gfx950 kernels: a one-token query goes to the split-K decode kernel,
longer queries to the chunked-prefill kernel. `triton_paged_attention` is the
same function under the reference's name.

Reference semantics: query (1, Hq, Tq, Dh) holds positions
query_position_offset + i, keys 0 .. key_length-1 are read through block_ids,
and key k is visible to query i when k <= query_position_offset + i
(_triton_paged_attention.py:118-123). Keys past query_position_offset + Tq - 1
are never visible, so the kernels get that key count.
"""

from __future__ import annotations

import torch

from tokserve_amd.engine.paged.storage import PagedKVStorage
from tokserve_amd.kernels import ops

__all__ = ["hip_paged_attention", "triton_paged_attention"]


def hip_paged_attention(
    query: torch.Tensor,
    storage: PagedKVStorage,
    block_ids: tuple[int, ...],
    *,
    layer_index: int,
    key_length: int,
    query_position_offset: int,
) -> torch.Tensor:
    """Apply causal attention while reading K/V through a block table."""

    if query.ndim != 4 or query.shape[0] != 1:
        raise ValueError("paged query must have shape (1, Hq, Tq, Dh)")
    if not query.is_cuda or storage.device.type != "cuda":
        raise ValueError("paged HIP attention requires CUDA (HIP) tensors")
    if query.device != storage.device:
        raise ValueError("query and paged storage must use the same device")
    if query.dtype != storage.dtype:
        raise ValueError("query and paged storage must use the same dtype")
    if query.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise TypeError("paged attention requires a supported floating dtype")
    if query.shape[1] % storage.num_key_value_heads != 0:
        raise ValueError("query head count must be divisible by KV head count")
    if query.shape[-1] != storage.head_dim:
        raise ValueError("query head_dim must match paged storage")
    if query.shape[-1] > 128:
        raise ValueError("head_dim must not exceed 128")
    if layer_index < 0 or layer_index >= storage.num_layers:
        raise IndexError("layer_index is out of range")
    if key_length < 1:
        raise ValueError("key_length must be positive")
    if query_position_offset < 0:
        raise ValueError("query_position_offset must be nonnegative")
    query_length = query.shape[2]
    if query_position_offset + query_length > key_length:
        raise ValueError("query positions cannot exceed key length")
    required_blocks = (key_length + storage.block_size - 1) // storage.block_size
    if len(block_ids) < required_blocks:
        raise ValueError("block table does not cover the valid key length")

    out = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    if query_length == 0:
        return out
    visible = query_position_offset + query_length
    # Block table, key count and query offsets travel in one host -> device copy.
    meta = torch.tensor(
        [*block_ids[:required_blocks], visible, 0, query_length], dtype=torch.int32
    ).to(query.device)
    block_table = meta[:required_blocks].view(1, required_blocks)
    seq_lens = meta[required_blocks : required_blocks + 1]
    cu_seqlens_q = meta[required_blocks + 1 :]
    # (Tq, Hq, Dh) views of the (1, Hq, Tq, Dh) query and output.
    packed_query = query[0].transpose(0, 1)
    packed_out = out[0].transpose(0, 1)
    if query_length == 1:
        ops.paged_attention_decode(
            packed_query, storage.key_storage, storage.value_storage, block_table, seq_lens,
            layer_index=layer_index, max_seq_len=visible, out=packed_out, **storage.scales,
        )
    else:
        ops.paged_attention_prefill(
            packed_query, storage.key_storage, storage.value_storage, block_table, seq_lens,
            cu_seqlens_q, layer_index=layer_index, max_query_len=query_length,
            max_seq_len=visible, out=packed_out, **storage.scales,
        )
    return out


triton_paged_attention = hip_paged_attention
