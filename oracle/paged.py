"""Paged-KV attention as the reference's torch backend computes it (CPU).

The torch backend writes the new K/V into the pool, rebuilds the layer's K/V in
logical order through the block table (read_layer, include_pending=True) and
runs repeat_kv + causal_attention over cache_len + T keys with offset
cache_len (tokserve/engine/attention.py:298-356). The batched functions below
are the per-request loop of tokserve/batching/execution.py:33-131 applied to a
packed batch.

Two arithmetics of the same attention exist in the reference, and both are
available here:
  compute_dtype=None     the torch backend: every op in the input dtype, so bf16
                         rounds after the matmul, the scale, the softmax and the
                         second matmul (tokserve/engine/attention.py:58-127);
  compute_dtype=float32  the reference's GPU kernel: Q, K and V loaded as fp32,
                         scores, online softmax and the accumulator in fp32, one
                         rounding to the output dtype on the store
                         (tokserve/kernels/_triton_paged_attention.py:60-66,101-149).
The reference's own GPU tests bound the gap between the two at 4e-2 for bf16
(tests/gpu/test_tiled_attention_prefill.py:50-59).
"""

from __future__ import annotations

import torch

from oracle.torch_path import gqa_attention


def read_layer(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_ids: list[int] | torch.Tensor,
    layer: int,
    length: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(1, Hkv, S, Dh) K/V of positions 0..length-1 in logical order.

    Position p lives at block_ids[p // BS], offset p % BS
    (tokserve/engine/paged/sequence_cache.py:157-193, block_table.py:53-67).
    """

    block_size = key_cache.shape[3]
    table = torch.as_tensor(block_ids, dtype=torch.int64)
    positions = torch.arange(length)
    blocks = table[positions // block_size]
    offsets = positions % block_size
    keys = key_cache[layer, blocks, :, offsets, :]  # (S, Hkv, Dh)
    values = value_cache[layer, blocks, :, offsets, :]
    return keys.permute(1, 0, 2).unsqueeze(0), values.permute(1, 0, 2).unsqueeze(0)


def paged_attention(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_ids: list[int] | torch.Tensor,
    *,
    layer: int,
    key_length: int,
    query_position_offset: int,
    compute_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """query (1, Hq, Tq, Dh) -> (1, Hq, Tq, Dh) through the block table."""

    keys, values = read_layer(key_cache, value_cache, block_ids, layer, key_length)
    if compute_dtype is None:
        return gqa_attention(query, keys, values, query_position_offset=query_position_offset)
    out = gqa_attention(query.to(compute_dtype), keys.to(compute_dtype), values.to(compute_dtype),
                        query_position_offset=query_position_offset)
    return out.to(query.dtype)


def decode_batch(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    layer: int,
    compute_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """One query per sequence: (B, Hq, Dh) -> (B, Hq, Dh); sequence b sees seq_lens[b] keys."""

    out = torch.empty_like(query)
    for b in range(query.shape[0]):
        length = int(seq_lens[b])
        if length == 0:
            out[b] = 0
            continue
        q = query[b][None, :, None, :]
        o = paged_attention(
            q, key_cache, value_cache, block_tables[b], layer=layer, key_length=length,
            query_position_offset=length - 1, compute_dtype=compute_dtype,
        )
        out[b] = o[0, :, 0, :]
    return out


def prefill_batch(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    layer: int,
    compute_dtype: torch.dtype | None = None,
) -> torch.Tensor:
    """Packed query chunks (N, Hq, Dh): sequence b's chunk sits at the end of its seq_lens[b] keys."""

    out = torch.empty_like(query)
    for b in range(seq_lens.shape[0]):
        q0, q1 = int(cu_seqlens_q[b]), int(cu_seqlens_q[b + 1])
        if q1 == q0:
            continue
        length = int(seq_lens[b])
        q = query[q0:q1].permute(1, 0, 2).unsqueeze(0)  # (1, Hq, Tq, Dh)
        o = paged_attention(
            q, key_cache, value_cache, block_tables[b], layer=layer, key_length=length,
            query_position_offset=length - (q1 - q0), compute_dtype=compute_dtype,
        )
        out[q0:q1] = o[0].permute(1, 0, 2)
    return out


# fp8 pools (the build's pool variant; the reference keeps pools in the model
# dtype, tokserve/engine/paged/storage.py:40-56). One fp32 scale per pool.
FP8_MAX = 448.0


def quantize_e4m3(x: torch.Tensor, scale: float) -> torch.Tensor:
    """e4m3(clamp(x / scale, -448, 448)) as torch.float8_e4m3fn (round to nearest even)."""

    return (x.to(torch.float32) / scale).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)


def dequantize_e4m3(codes: torch.Tensor, scale: float, dtype: torch.dtype) -> torch.Tensor:
    """float(code) * scale in fp32, rounded once to dtype."""

    return (codes.to(torch.float32) * scale).to(dtype)


# fp8 pools with one scale per pool row (per token and KV head), the second pool
# variant: the scales sit beside the pools as float32 [L, NB, Hkv, BS].


def row_scales_e4m3(x: torch.Tensor) -> torch.Tensor:
    """float32 scale of each row of x (..., Dh): max|x| / 448, 1 where that is 0, NaN or
    infinite (a NaN anywhere in the row makes the maximum NaN)."""

    amax = x.to(torch.float32).abs().amax(dim=-1)
    s = amax / FP8_MAX
    return torch.where((s > 0) & torch.isfinite(s), s, torch.ones_like(s))


def quantize_e4m3_rows(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(e4m3(clamp(x / s, -448, 448)) as torch.float8_e4m3fn, s) with s = row_scales_e4m3(x)."""

    s = row_scales_e4m3(x)
    codes = (x.to(torch.float32) / s.unsqueeze(-1)).clamp(-FP8_MAX, FP8_MAX)
    return codes.to(torch.float8_e4m3fn), s


def dequantize_e4m3_rows(codes: torch.Tensor, scales: torch.Tensor,
                         dtype: torch.dtype) -> torch.Tensor:
    """float(code) * s (s per row, the scales shaped like codes without the last axis) in
    fp32, rounded once to dtype."""

    return (codes.to(torch.float32) * scales.unsqueeze(-1)).to(dtype)
