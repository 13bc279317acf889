"""Llama grouped-query attention module (tokserve/engine/attention.py:130-368).

Same projections (q_proj, k_proj, v_proj, o_proj, created in that order) and
the same op order as the reference: project, RoPE, write K/V into the paged
cache, attend over cache_len + T keys with query offset cache_len, merge
heads, o_proj (attention.py:241-368). Two entry points:

  forward         one sequence, (1, T, D), through the drop-in operators
                  (hip_apply_rope, SequencePagedKVCache.write_layer,
                  hip_paged_attention; hip_tiled_attention without a cache);
  forward_packed  a packed ragged batch (N, D) through one fused QKV GEMM,
                  one RoPE launch, one KV-append launch and the paged
                  prefill / decode kernels.
"""

from __future__ import annotations

from typing import TYPE_CHECKING

import torch
from torch import nn
from torch.nn import functional

from tokserve_amd.engine.config import LlamaConfig
from tokserve_amd.engine.kernel_backend import KernelBackend, check_backend
from tokserve_amd.engine.layers import fused_weight
from tokserve_amd.kernels import ops
from tokserve_amd.kernels.paged_attention import hip_paged_attention
from tokserve_amd.kernels.rope import hip_apply_rope
from tokserve_amd.kernels.tiled_attention import hip_tiled_attention

if TYPE_CHECKING:
    from tokserve_amd.batching.metadata import PackedBatch
    from tokserve_amd.engine.paged.sequence_cache import SequencePagedKVCache
    from tokserve_amd.engine.paged.storage import PagedKVStorage

__all__ = ["GroupedQueryAttention", "reject_contiguous_cache"]


def reject_contiguous_cache(cache: object, paged_cache: object) -> None:
    """The `cache=` keyword of the reference's forwards (model.py:50,124,
    attention.py:181) takes its contiguous per-sequence KV cache (engine/cache.py),
    which this library does not provide: None is accepted, as the reference's default,
    and any other value raises ValueError (with the reference's message when a paged
    cache is given too)."""

    if cache is None:
        return
    if paged_cache is not None:
        raise ValueError("choose either contiguous or paged cache")
    raise ValueError("contiguous KV caches are not supported; pass paged_cache instead")


class GroupedQueryAttention(nn.Module):
    """Llama grouped-query self-attention over paged K/V."""

    def __init__(self, config: LlamaConfig, *, backend: KernelBackend = "torch") -> None:
        super().__init__()
        self.backend = check_backend(backend)
        self.hidden_size = config.hidden_size
        self.num_attention_heads = config.num_attention_heads
        self.num_key_value_heads = config.num_key_value_heads
        self.num_key_value_groups = config.num_key_value_groups
        self.head_dim = config.head_dim
        self.rope_theta = config.rope_theta
        kv_size = self.num_key_value_heads * self.head_dim
        self.q_proj = nn.Linear(self.hidden_size, self.hidden_size, bias=False)
        self.k_proj = nn.Linear(self.hidden_size, kv_size, bias=False)
        self.v_proj = nn.Linear(self.hidden_size, kv_size, bias=False)
        self.o_proj = nn.Linear(self.hidden_size, self.hidden_size, bias=False)

    # ------------------------------------------------------------ one sequence

    def forward(
        self,
        inputs: torch.Tensor,
        positions: torch.Tensor,
        *,
        cache: None = None,
        paged_cache: SequencePagedKVCache | None = None,
        layer_index: int | None = None,
    ) -> torch.Tensor:
        """(1, T, D) -> (1, T, D) attention output for one sequence. `cache` must be
        None (see reject_contiguous_cache)."""

        if inputs.ndim != 3:
            raise ValueError("inputs must have shape (B, T, D)")
        reject_contiguous_cache(cache, paged_cache)
        if inputs.shape[0] < 1 or inputs.shape[1] < 1:
            raise ValueError("batch and sequence dimensions must be positive")
        if inputs.shape[-1] != self.hidden_size:
            raise ValueError("inputs must use the configured hidden_size")
        batch, length, _ = inputs.shape
        if paged_cache is not None:
            if batch != 1:
                raise ValueError("paged attention currently supports batch size 1")
            if layer_index is None:
                raise ValueError("layer_index is required for paged attention")
        elif layer_index is not None:
            raise ValueError("layer_index requires a paged cache")
        cache_length = 0 if paged_cache is None else paged_cache.current_length
        if positions.shape != (length,):
            raise ValueError("positions must have shape (T,)")

        def heads(projection: torch.Tensor, count: int) -> torch.Tensor:
            return projection.view(batch, length, count, self.head_dim).transpose(1, 2)

        query = heads(self.q_proj(inputs), self.num_attention_heads)
        key = heads(self.k_proj(inputs), self.num_key_value_heads)
        value = heads(self.v_proj(inputs), self.num_key_value_heads)
        query, key = hip_apply_rope(query, key, positions, theta=self.rope_theta)
        if paged_cache is not None:
            paged_cache.write_layer(layer_index, key[0], value[0])
            attended = hip_paged_attention(
                query, paged_cache.storage, paged_cache.block_ids, layer_index=layer_index,
                key_length=cache_length + length, query_position_offset=cache_length,
            )
        else:
            attended = hip_tiled_attention(query, key, value, query_position_offset=0)
        merged = attended.transpose(1, 2).reshape(batch, length, self.hidden_size)
        return self.o_proj(merged)

    # ----------------------------------------------------------- packed batch

    def qkv_weight(self) -> torch.Tensor:
        return fused_weight(self, [self.q_proj, self.k_proj, self.v_proj], "_qkv")

    def forward_packed(
        self,
        inputs: torch.Tensor,
        batch: PackedBatch,
        storage: PagedKVStorage,
        layer_index: int,
        rotary: ops.RotaryTable,
    ) -> torch.Tensor:
        """(N, D) packed tokens of a ragged batch -> (N, D) attention output.

        Rows [0, batch.num_prefill_tokens) are prefill chunks (causal within
        each chunk, after the sequence's cached keys); the remaining rows are
        one decode token per sequence.
        """

        tokens = inputs.shape[0]
        hq, hkv, dh = self.num_attention_heads, self.num_key_value_heads, self.head_dim
        qkv = functional.linear(inputs, self.qkv_weight())  # (N, (Hq + 2 Hkv) Dh)
        query = qkv[:, : hq * dh].view(tokens, hq, dh)
        key = qkv[:, hq * dh : (hq + hkv) * dh].view(tokens, hkv, dh)
        value = qkv[:, (hq + hkv) * dh :].view(tokens, hkv, dh)
        split = batch.num_prefill_tokens
        if layer_index < 0 or layer_index >= storage.num_layers:
            raise IndexError("layer_index is out of range")
        if split == 0:
            # Decode-only iteration: RoPE, the KV append and the attention in one call.
            attended = ops.rope_append_paged_decode(
                query, key, value, batch.positions, rotary, storage.key_storage,
                storage.value_storage, batch.slot_mapping, batch.decode_block_tables,
                batch.decode_seq_lens, layer_index=layer_index,
                max_seq_len=batch.decode_max_seq_len, seq_order=batch.decode_seq_order,
                **storage.scales)
            return self.o_proj(attended.view(tokens, self.hidden_size))
        # Q rotated in place; rotated K and V go straight to the pool slots (quantized
        # with the pool scales over fp8 pools).
        ops.rope_kv_append(query, key, value, batch.positions, rotary, storage.key_storage,
                           storage.value_storage, batch.slot_mapping, layer_index,
                           **storage.scales)
        attended = torch.empty((tokens, hq, dh), dtype=inputs.dtype, device=inputs.device)
        if split > 0:
            ops.paged_attention_prefill(
                query[:split], storage.key_storage, storage.value_storage,
                batch.prefill_block_tables, batch.prefill_seq_lens, batch.prefill_cu_seqlens_q,
                layer_index=layer_index, max_query_len=batch.prefill_max_query_len,
                max_seq_len=batch.prefill_max_seq_len, out=attended[:split],
                seq_order=batch.prefill_seq_order, **storage.scales,
            )
        if split < tokens:
            ops.paged_attention_decode(
                query[split:], storage.key_storage, storage.value_storage,
                batch.decode_block_tables, batch.decode_seq_lens, layer_index=layer_index,
                max_seq_len=batch.decode_max_seq_len, out=attended[split:],
                seq_order=batch.decode_seq_order, **storage.scales,
            )
        return self.o_proj(attended.view(tokens, self.hidden_size))
