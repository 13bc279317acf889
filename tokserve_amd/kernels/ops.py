"""Batched device operators of the hot path.

These take the packed ragged-batch metadata (`cu_seqlens`, `block_tables`,
`seq_lens`, `slot_mapping`, `positions`) that tokserve/batching lacks (it runs
one request at a time, tokserve/batching/execution.py:33,81). Every function
validates shapes and devices with the reference's exception types, allocates
the outputs the caller did not pass, and calls one PyTorch operator
(`torch.ops.tokserve_amd.*`, registered in torch_ops.py), whose device kernel
enqueues one C-ABI entry point on the current torch stream. Tensors must live
on a HIP device: there is no CPU path.
"""

from __future__ import annotations

from math import sqrt

import torch

from tokserve_amd.kernels import torch_ops

_ops = torch.ops.tokserve_amd


def require_hip(operation: str, *tensors: torch.Tensor) -> torch.device:
    """All tensors on one HIP device (torch reports HIP tensors as is_cuda)."""

    device = tensors[0].device
    for tensor in tensors:
        if not tensor.is_cuda:
            raise ValueError(f"{operation} requires HIP device tensors")
        if tensor.device != device:
            raise ValueError(f"{operation}: tensors must use the same device")
    return device


def _pool_shape(key_cache: torch.Tensor, value_cache: torch.Tensor) -> tuple[int, ...]:
    if key_cache.ndim != 5 or key_cache.shape != value_cache.shape:
        raise ValueError("KV pools must both have shape (L, NB, Hkv, BS, Dh)")
    if key_cache.dtype != value_cache.dtype:
        raise ValueError("KV pools must use the same dtype")
    if not key_cache.is_contiguous() or not value_cache.is_contiguous():
        raise ValueError("KV pools must be contiguous")
    return tuple(key_cache.shape)


# K/V pools may hold OCP fp8 e4m3 with one fp32 scale per pool (stored =
# e4m3(clamp(x / scale, -448, 448)), decoded = float(stored) * scale); every
# other tensor of the call keeps a float dtype.
FP8_POOL_DTYPE = torch.float8_e4m3fn


def is_fp8_pool(pool: torch.Tensor) -> bool:
    return pool.dtype == FP8_POOL_DTYPE


def _pool_scales(pool: torch.Tensor, k_scale: float, v_scale: float) -> tuple[float, float]:
    k_scale, v_scale = float(k_scale), float(v_scale)
    if not is_fp8_pool(pool):
        if k_scale != 1.0 or v_scale != 1.0:
            raise ValueError("k_scale and v_scale apply to fp8 KV pools only")
        return k_scale, v_scale
    for name, value in (("k_scale", k_scale), ("v_scale", v_scale)):
        if not (0.0 < value < float("inf")):
            raise ValueError(f"{name} must be a positive finite float")
    return k_scale, v_scale


def _row_scales(
    operation: str,
    key_cache: torch.Tensor,
    k_scales: torch.Tensor | None,
    v_scales: torch.Tensor | None,
    k_scale: float,
    v_scale: float,
) -> tuple[torch.Tensor | None, torch.Tensor | None]:
    """Per-row scales of fp8 pools: float32 (L, NB, Hkv, BS) each, on the pools'
    device, contiguous, or both None (per-pool scales k_scale / v_scale apply).

    Row (l, b, h, r) of a pool holds e4m3(clamp(x / s, -448, 448)) with
    s = k_scales[l, b, h, r] (v_scales for the value pool), decoded as code * s;
    the pool scales must then stay 1.
    """

    if k_scales is None and v_scales is None:
        return None, None
    if k_scales is None or v_scales is None:
        raise ValueError(f"{operation}: k_scales and v_scales go together")
    if not is_fp8_pool(key_cache):
        raise ValueError("per-row scales apply to fp8 KV pools only")
    if k_scale != 1.0 or v_scale != 1.0:
        raise ValueError("per-row scales replace k_scale and v_scale, which must stay 1")
    require_hip(operation, key_cache, k_scales, v_scales)
    for name, scales in (("k_scales", k_scales), ("v_scales", v_scales)):
        if scales.dtype != torch.float32:
            raise TypeError(f"{name} must be float32")
        if scales.shape != key_cache.shape[:4] or not scales.is_contiguous():
            raise ValueError(f"{name} must be a contiguous (L, NB, Hkv, BS) tensor")
    return k_scales, v_scales


def _last_dim_contiguous(tensor: torch.Tensor, name: str) -> torch.Tensor:
    return tensor if tensor.stride(-1) == 1 else tensor.contiguous()


def _int_tensor(tensor: torch.Tensor, dtype: torch.dtype, name: str) -> torch.Tensor:
    if tensor.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}")
    return tensor if tensor.is_contiguous() else tensor.contiguous()


# ----------------------------------------------------------------------------
# KV cache


def kv_append(
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    layer_index: int,
    *,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    k_scales: torch.Tensor | None = None,
    v_scales: torch.Tensor | None = None,
) -> None:
    """Scatter K/V rows (N, Hkv, Dh) into the pools at slot_mapping (int64, N).

    fp8 pools quantize the rows with the pool scales (k_scale, v_scale), or, given
    k_scales / v_scales (float32 (L, NB, Hkv, BS)), each row with a scale of its
    own, s = max|row| / 448 (1 for an all-zero or non-finite maximum), written to
    the row's entry of k_scales / v_scales. Pools in a float dtype take rows of
    that dtype, copied bit for bit.
    """

    require_hip("kv_append", key, value, key_cache, value_cache, slot_mapping)
    num_layers, num_blocks, num_kv_heads, block_size, head_dim = _pool_shape(
        key_cache, value_cache
    )
    if key.ndim != 3 or key.shape != value.shape:
        raise ValueError("key and value must have shape (N, Hkv, Dh)")
    if key.shape[1:] != (num_kv_heads, head_dim):
        raise ValueError("key rows must match the pool's (Hkv, Dh)")
    fp8 = is_fp8_pool(key_cache)
    k_scale, v_scale = _pool_scales(key_cache, k_scale, v_scale)
    k_scales, v_scales = _row_scales("kv_append", key_cache, k_scales, v_scales, k_scale, v_scale)
    if value.dtype != key.dtype or (not fp8 and key.dtype != key_cache.dtype):
        raise ValueError("keys and values must match the storage dtype")
    if slot_mapping.shape != (key.shape[0],):
        raise ValueError("slot_mapping must have shape (N,)")
    slots = _int_tensor(slot_mapping, torch.int64, "slot_mapping")
    key = _last_dim_contiguous(key, "key")
    value = _last_dim_contiguous(value, "value")
    _ops.kv_append(key, value, key_cache, value_cache, slots, layer_index, k_scale, v_scale,
                   k_scales, v_scales)


def paged_gather(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    cu_seqlens: torch.Tensor,
    layer_index: int,
    max_seq_len: int,
    key_out: torch.Tensor,
    value_out: torch.Tensor,
    *,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    k_scales: torch.Tensor | None = None,
    v_scales: torch.Tensor | None = None,
) -> None:
    """Copy each sequence's K/V in logical order into key_out/value_out.

    key_out/value_out are (S_total, Hkv, Dh) views (any token/head strides, Dh
    contiguous); sequence b fills rows cu_seqlens[b] .. cu_seqlens[b]+seq_lens[b]-1.
    fp8 pools are decoded with their scales (per pool, or per row with
    k_scales / v_scales) into the outputs' float dtype.
    """

    require_hip(
        "paged_gather", key_cache, value_cache, block_tables, seq_lens, cu_seqlens,
        key_out, value_out,
    )
    num_layers, num_blocks, num_kv_heads, block_size, head_dim = _pool_shape(
        key_cache, value_cache
    )
    if block_tables.ndim != 2:
        raise ValueError("block_tables must have shape (B, max_blocks)")
    tables = _int_tensor(block_tables, torch.int32, "block_tables")
    lens = _int_tensor(seq_lens, torch.int32, "seq_lens")
    cu = _int_tensor(cu_seqlens, torch.int32, "cu_seqlens")
    if key_out.ndim != 3 or key_out.shape[1:] != (num_kv_heads, head_dim):
        raise ValueError("outputs must have shape (S, Hkv, Dh)")
    if value_out.shape != key_out.shape or value_out.stride() != key_out.stride():
        raise ValueError("key_out and value_out must share shape and strides")
    if key_out.stride(-1) != 1:
        raise ValueError("outputs must be contiguous in head_dim")
    fp8 = is_fp8_pool(key_cache)
    k_scale, v_scale = _pool_scales(key_cache, k_scale, v_scale)
    k_scales, v_scales = _row_scales("paged_gather", key_cache, k_scales, v_scales, k_scale,
                                     v_scale)
    if value_out.dtype != key_out.dtype or (not fp8 and key_out.dtype != key_cache.dtype):
        raise ValueError("outputs must match the storage dtype")
    _ops.paged_gather(key_cache, value_cache, tables, lens, cu, layer_index, max_seq_len,
                      key_out, value_out, k_scale, v_scale, k_scales, v_scales)


# ----------------------------------------------------------------------------
# Attention


def decode_workspace_bytes(
    num_seqs: int,
    num_q_heads: int,
    num_kv_heads: int,
    head_dim: int,
    block_size: int,
    max_seq_len: int,
    pages_per_split: int = 0,
) -> int:
    """Bytes of split-K scratch the decode kernel needs for this batch."""

    return torch_ops.decode_workspace_bytes(num_seqs, num_q_heads, num_kv_heads, head_dim,
                                            block_size, max_seq_len, pages_per_split)


def longest_first(seq_lens: list[int], device: torch.device | str) -> torch.Tensor:
    """Host-side launch plan: sequence indices by decreasing length (int32, on device).

    Built from the lengths the scheduler already holds on the host; ties keep
    batch order so the plan is deterministic.
    """

    order = sorted(range(len(seq_lens)), key=lambda b: (-seq_lens[b], b))
    return torch.tensor(order, dtype=torch.int32).to(device)


def _seq_order(operation: str, like: torch.Tensor,
               seq_order: torch.Tensor | None) -> torch.Tensor | None:
    """A launch's sequence order: int32 (B,) on the device of `like` (B = like.shape[0],
    the decode query or the seq_lens), or None."""

    if seq_order is None:
        return None
    require_hip(operation, like, seq_order)
    order = _int_tensor(seq_order, torch.int32, "seq_order")
    if order.shape != (like.shape[0],):
        raise ValueError("seq_order must have shape (B,)")
    return order


def _check_workspace(operation: str, query: torch.Tensor, workspace: torch.Tensor | None) -> None:
    """A caller's split workspace: contiguous uint8 on the query's device (its size is
    checked against the launch's partials by the library)."""

    if workspace is None:
        return
    require_hip(operation, query, workspace)
    if workspace.dtype != torch.uint8 or not workspace.is_contiguous():
        raise ValueError("workspace must be a contiguous uint8 tensor")


def paged_attention_decode(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    *,
    layer_index: int,
    max_seq_len: int,
    scale: float | None = None,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    pages_per_split: int = 0,
    seq_order: torch.Tensor | None = None,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    k_scales: torch.Tensor | None = None,
    v_scales: torch.Tensor | None = None,
) -> torch.Tensor:
    """One query token per sequence: query (B, Hq, Dh) -> out (B, Hq, Dh).

    Sequence b attends to its seq_lens[b] keys through block_tables[b]
    (int32, (B, max_blocks)); max_seq_len is a host bound on seq_lens.
    `workspace` (uint8, >= decode_workspace_bytes) holds split partials when a
    sequence is split across workgroups; it defaults to a per-device buffer.
    Launches that share a workspace must be ordered on one stream.
    `seq_order` (int32 permutation of 0..B-1, see longest_first) is the order in
    which sequences reach workgroups; longest-first avoids a tail of long
    sequences. Results do not depend on it. fp8 pools are decoded with
    (k_scale, v_scale), or per row with k_scales / v_scales.
    """

    require_hip("paged_attention_decode", query, key_cache, value_cache, block_tables, seq_lens)
    num_layers, num_blocks, num_kv_heads, block_size, head_dim = _pool_shape(
        key_cache, value_cache
    )
    if query.ndim != 3 or query.shape[2] != head_dim:
        raise ValueError("query must have shape (B, Hq, Dh) with the pool's Dh")
    fp8 = is_fp8_pool(key_cache)
    k_scale, v_scale = _pool_scales(key_cache, k_scale, v_scale)
    k_scales, v_scales = _row_scales("paged_attention_decode", key_cache, k_scales, v_scales,
                                     k_scale, v_scale)
    if not fp8 and query.dtype != key_cache.dtype:
        raise ValueError("query and paged storage must use the same dtype")
    num_seqs, num_q_heads, _ = query.shape
    if num_q_heads % num_kv_heads != 0:
        raise ValueError("query head count must be divisible by KV head count")
    tables = _int_tensor(block_tables, torch.int32, "block_tables")
    lens = _int_tensor(seq_lens, torch.int32, "seq_lens")
    if tables.ndim != 2 or tables.shape[0] != num_seqs or lens.shape != (num_seqs,):
        raise ValueError("block_tables (B, max_blocks) and seq_lens (B,) must match query")
    query = _last_dim_contiguous(query, "query")
    if out is None:
        out = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    if scale is None:
        scale = 1.0 / sqrt(head_dim)
    order = _seq_order("paged_attention_decode", query, seq_order)
    _check_workspace("paged_attention_decode", query, workspace)
    _ops.paged_attention_decode(query, key_cache, value_cache, tables, lens, order, layer_index,
                                max_seq_len, float(scale), pages_per_split, k_scale, v_scale, out,
                                workspace, k_scales, v_scales)
    return out


def paged_attention_decode_noalloc(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    *,
    layer_index: int,
    max_seq_len: int,
    out: torch.Tensor,
    scale: float | None = None,
    pages_per_split: int = 0,
    seq_order: torch.Tensor | None = None,
) -> torch.Tensor:
    """paged_attention_decode with the split partials in the library's static per-GPU
    buffer: no device memory is allocated (the output comes from the caller). Batches
    whose partials exceed the buffer raise ValueError; calls that can overlap on one GPU
    race on the buffer. Pools in the query dtype."""

    require_hip("paged_attention_decode", query, key_cache, value_cache, block_tables, seq_lens,
                out)
    _, _, num_kv_heads, _, head_dim = _pool_shape(key_cache, value_cache)
    if query.ndim != 3 or query.shape[2] != head_dim or query.stride(-1) != 1:
        raise ValueError("query must have shape (B, Hq, Dh) with the pool's Dh, Dh contiguous")
    if query.dtype != key_cache.dtype:
        raise ValueError("query and paged storage must use the same dtype")
    if query.shape[1] % num_kv_heads != 0:
        raise ValueError("query head count must be divisible by KV head count")
    if out.shape != query.shape or out.dtype != query.dtype or out.stride(-1) != 1:
        raise ValueError("out must match the query")
    tables = _int_tensor(block_tables, torch.int32, "block_tables")
    lens = _int_tensor(seq_lens, torch.int32, "seq_lens")
    if tables.ndim != 2 or tables.shape[0] != query.shape[0] or lens.shape != (query.shape[0],):
        raise ValueError("block_tables (B, max_blocks) and seq_lens (B,) must match query")
    order = _seq_order("paged_attention_decode", query, seq_order)
    _ops.paged_attention_decode_noalloc(
        query, key_cache, value_cache, tables, lens, order, layer_index, max_seq_len,
        float(1.0 / sqrt(head_dim) if scale is None else scale), pages_per_split, out)
    return out


def paged_attention_prefill(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    *,
    layer_index: int,
    max_query_len: int,
    max_seq_len: int,
    scale: float | None = None,
    out: torch.Tensor | None = None,
    seq_order: torch.Tensor | None = None,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    k_scales: torch.Tensor | None = None,
    v_scales: torch.Tensor | None = None,
) -> torch.Tensor:
    """Causal attention of packed query chunks (N, Hq, Dh) over their paged KV.

    Sequence b owns query rows cu_seqlens_q[b] .. cu_seqlens_q[b+1]-1; its
    seq_lens[b] keys already include those rows, so query i sits at absolute
    position seq_lens[b] - q_len_b + i. `seq_order` (int32 permutation of 0..B-1,
    e.g. longest_first of seq_lens) is the order in which sequences reach
    workgroups; results do not depend on it. fp8 pools are decoded with
    (k_scale, v_scale), or per row with k_scales / v_scales.
    """

    require_hip(
        "paged_attention_prefill", query, key_cache, value_cache, block_tables, seq_lens,
        cu_seqlens_q,
    )
    num_layers, num_blocks, num_kv_heads, block_size, head_dim = _pool_shape(
        key_cache, value_cache
    )
    if query.ndim != 3 or query.shape[2] != head_dim:
        raise ValueError("query must have shape (N, Hq, Dh) with the pool's Dh")
    fp8 = is_fp8_pool(key_cache)
    k_scale, v_scale = _pool_scales(key_cache, k_scale, v_scale)
    k_scales, v_scales = _row_scales("paged_attention_prefill", key_cache, k_scales, v_scales,
                                     k_scale, v_scale)
    if not fp8 and query.dtype != key_cache.dtype:
        raise ValueError("query and paged storage must use the same dtype")
    num_q_heads = query.shape[1]
    if num_q_heads % num_kv_heads != 0:
        raise ValueError("query head count must be divisible by KV head count")
    tables = _int_tensor(block_tables, torch.int32, "block_tables")
    lens = _int_tensor(seq_lens, torch.int32, "seq_lens")
    cu = _int_tensor(cu_seqlens_q, torch.int32, "cu_seqlens_q")
    num_seqs = lens.shape[0]
    if tables.ndim != 2 or tables.shape[0] != num_seqs or cu.shape != (num_seqs + 1,):
        raise ValueError("block_tables (B, max_blocks), seq_lens (B,), cu_seqlens_q (B+1,)")
    query = _last_dim_contiguous(query, "query")
    if out is None:
        out = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    if scale is None:
        scale = 1.0 / sqrt(head_dim)
    order = _seq_order("paged_attention_prefill", lens, seq_order)
    _ops.paged_attention_prefill(query, key_cache, value_cache, tables, lens, cu, order,
                                 layer_index, max_query_len, max_seq_len, float(scale), k_scale,
                                 v_scale, out, k_scales, v_scales)
    return out


# ----------------------------------------------------------------------------
# RMSNorm


def rms_norm(
    inputs: torch.Tensor,
    weight: torch.Tensor,
    epsilon: float,
    *,
    residual: torch.Tensor | None = None,
    residual_out: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """weight * to_in(x * rsqrt(mean(x^2) + eps)) over the last dimension.

    With `residual`, x = to_in(inputs + residual) is first written to
    `residual_out` (defaults to a new tensor, returned via the second slot of
    the tuple when residual is given).
    """

    require_hip("rms_norm", inputs, weight)
    hidden = inputs.shape[-1]
    if weight.shape != (hidden,):
        raise ValueError("weight must have shape (D,)")
    out_dtype = torch.promote_types(weight.dtype, inputs.dtype)
    rows_in = inputs.reshape(-1, hidden)
    if rows_in.stride(-1) != 1:
        rows_in = rows_in.contiguous()
    weight = weight.contiguous()
    if out is None:
        out = torch.empty(inputs.shape, dtype=out_dtype, device=inputs.device)
    rows_out = out.view(-1, hidden)
    res_rows = res_out_rows = None
    if residual is not None:
        require_hip("rms_norm", residual)
        if residual.shape != inputs.shape or residual.dtype != inputs.dtype:
            raise ValueError("residual must match inputs")
        res_rows = residual.reshape(-1, hidden)
        if res_rows.stride(-1) != 1:
            res_rows = res_rows.contiguous()
        if residual_out is None:
            residual_out = torch.empty_like(inputs)
        res_out_rows = residual_out.view(-1, hidden)
    _ops.rms_norm(rows_in, weight, float(epsilon), res_rows, rows_out, res_out_rows)
    return out


# ----------------------------------------------------------------------------
# RoPE


class RotaryTable:
    """Per-position cos/sin rows, (cache_len, Dh/2) each, in the model dtype.

    Row p holds cos/sin(fp32(p) * inv_freq) cast to dtype, with
    inv_freq = theta ** (-arange(0, Dh, 2) / Dh) in fp32: the values
    rotary_cos_sin computes (tokserve/engine/rope.py:28-87). The table is
    computed once with torch on the host and copied to the device; the kernel
    only gathers rows by position.
    """

    def __init__(
        self,
        head_dim: int,
        *,
        theta: float,
        max_position: int,
        dtype: torch.dtype,
        device: torch.device,
    ) -> None:
        if head_dim < 2 or head_dim % 2 != 0:
            raise ValueError("head_dim must be a positive even integer")
        if theta <= 0.0:
            raise ValueError("theta must be positive")
        if max_position < 1:
            raise ValueError("max_position must be positive")
        self.head_dim = head_dim
        self.theta = theta
        self.dtype = dtype
        self.device = torch.device(device)
        self.length = 0
        self.cos = torch.empty(0)
        self.sin = torch.empty(0)
        self.ensure(max_position)

    def ensure(self, max_position: int) -> None:
        """Grow the table to cover positions [0, max_position)."""

        if max_position <= self.length:
            return
        length = max(max_position, 2 * self.length)
        indices = torch.arange(0, self.head_dim, 2, dtype=torch.float32)
        inv_freq = self.theta ** (-indices / self.head_dim)
        positions = torch.arange(length, dtype=torch.int64).to(torch.float32)
        angles = torch.outer(positions, inv_freq)
        self.cos = angles.cos().to(self.dtype).to(self.device).contiguous()
        self.sin = angles.sin().to(self.dtype).to(self.device).contiguous()
        self.length = length


def rope(
    query: torch.Tensor,
    key: torch.Tensor,
    positions: torch.Tensor,
    table: RotaryTable,
    *,
    query_out: torch.Tensor | None = None,
    key_out: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotate Q (B, Hq, T, Dh) and K (B, Hkv, T, Dh) at positions (T,) in one launch.

    Packed streams pass (1, H, N, Dh) views of (N, H, Dh) tensors. Outputs may
    alias the inputs (in-place rotation). Positions must lie in [0, table.length).
    """

    require_hip("rope", query, key, positions)
    if query.ndim != 4 or key.ndim != 4:
        raise ValueError("query and key must have shape (B, H, T, Dh)")
    if query.shape[0] != key.shape[0] or query.shape[2:] != key.shape[2:]:
        raise ValueError("query and key batch, sequence and head dimensions must match")
    if query.dtype != key.dtype or query.dtype != table.dtype:
        raise ValueError("query, key and the rotary table must use the same dtype")
    if query.shape[-1] != table.head_dim:
        raise ValueError("head_dim must match the rotary table")
    if positions.shape != (query.shape[2],):
        raise ValueError("positions must have shape (T,)")
    pos = positions if positions.dtype == torch.int64 else positions.to(torch.int64)
    pos = pos.contiguous()
    query = _last_dim_contiguous(query, "query")
    key = _last_dim_contiguous(key, "key")
    if query_out is None:
        query_out = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    if key_out is None:
        key_out = torch.empty(key.shape, dtype=key.dtype, device=key.device)
    if query_out.stride(-1) != 1 or key_out.stride(-1) != 1:
        raise ValueError("rope outputs must be contiguous in head_dim")
    if query_out is query and key_out is key:
        _ops.rope_(query, key, pos, table.cos, table.sin)
    else:
        _ops.rope(query, key, pos, table.cos, table.sin, query_out, key_out)
    return query_out, key_out


def rope_kv_append(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    positions: torch.Tensor,
    table: RotaryTable,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    layer_index: int,
    *,
    query_out: torch.Tensor | None = None,
    key_out: torch.Tensor | None = None,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    k_scales: torch.Tensor | None = None,
    v_scales: torch.Tensor | None = None,
) -> torch.Tensor:
    """Packed step: rotate query (N, Hq, Dh) into query_out (in place by default), rotate
    key (N, Hkv, Dh) and append it with value (N, Hkv, Dh) to the pools at slot_mapping.

    One launch, bit-identical to rope() followed by kv_append() of the rotated keys.
    key_out, when given, also receives the rotated keys. Pools in the rows' dtype, or
    fp8 pools quantized with k_scale / v_scale, or per row into k_scales / v_scales, as
    kv_append() does.
    """

    require_hip("rope_kv_append", query, key, value, positions, key_cache, value_cache,
                slot_mapping)
    num_layers, num_blocks, num_kv_heads, block_size, head_dim = _pool_shape(
        key_cache, value_cache
    )
    if query.ndim != 3 or key.ndim != 3 or value.shape != key.shape:
        raise ValueError("query (N, Hq, Dh), key and value (N, Hkv, Dh) expected")
    tokens = query.shape[0]
    if key.shape != (tokens, num_kv_heads, head_dim) or query.shape[2] != head_dim:
        raise ValueError("key and value rows must match the pool's (Hkv, Dh)")
    k_scale, v_scale = _pool_scales(key_cache, k_scale, v_scale)
    k_scales, v_scales = _row_scales("rope_kv_append", key_cache, k_scales, v_scales, k_scale,
                                     v_scale)
    pool_dtype = query.dtype if is_fp8_pool(key_cache) else key_cache.dtype
    if len({query.dtype, key.dtype, value.dtype, pool_dtype, table.dtype}) != 1:
        raise ValueError("query, key, value, pools and the rotary table must share a dtype")
    if head_dim != table.head_dim:
        raise ValueError("head_dim must match the rotary table")
    if positions.shape != (tokens,) or slot_mapping.shape != (tokens,):
        raise ValueError("positions and slot_mapping must have shape (N,)")
    pos = positions if positions.dtype == torch.int64 else positions.to(torch.int64)
    pos = pos.contiguous()
    slots = _int_tensor(slot_mapping, torch.int64, "slot_mapping")
    for name, t in (("query", query), ("key", key), ("value", value)):
        if t.stride(-1) != 1:
            raise ValueError(f"{name} must be contiguous in head_dim")
    if query_out is None:
        query_out = query
    if query_out.shape != query.shape or query_out.stride(-1) != 1:
        raise ValueError("query_out must match query and be contiguous in head_dim")
    if key_out is not None and (key_out.shape != key.shape or key_out.stride(-1) != 1):
        raise ValueError("key_out must match key and be contiguous in head_dim")
    if query_out is query:
        _ops.rope_kv_append_(query, key, value, pos, table.cos, table.sin, key_cache,
                             value_cache, slots, layer_index, key_out, k_scale, v_scale,
                             k_scales, v_scales)
    else:
        _ops.rope_kv_append(query, key, value, pos, table.cos, table.sin, key_cache, value_cache,
                            slots, layer_index, query_out, key_out, k_scale, v_scale, k_scales,
                            v_scales)
    return query_out


def rope_append_paged_decode(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    positions: torch.Tensor,
    table: RotaryTable,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    *,
    layer_index: int,
    max_seq_len: int,
    scale: float | None = None,
    out: torch.Tensor | None = None,
    workspace: torch.Tensor | None = None,
    pages_per_split: int = 0,
    seq_order: torch.Tensor | None = None,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    k_scales: torch.Tensor | None = None,
    v_scales: torch.Tensor | None = None,
) -> torch.Tensor:
    """A decode step's RoPE, KV append and attention in one call: query (B, Hq, Dh) is
    rotated at positions (B,) (read only), the rotated key and the value rows (B, Hkv, Dh)
    go to pool slots slot_mapping (B,), which must address position seq_lens[b] - 1, and
    out (B, Hq, Dh) receives the attention over seq_lens[b] keys.

    Bit-identical to rope_kv_append() followed by paged_attention_decode() with the
    same arguments (one launch on the MFMA decode kernel; with per-row scales the append
    is a launch of its own ahead of the attention). Pools in the rows' dtype, or fp8
    pools with their scales (per pool, or per row with k_scales / v_scales).
    """

    require_hip("rope_append_paged_decode", query, key, value, positions, key_cache,
                value_cache, slot_mapping, block_tables, seq_lens)
    num_layers, num_blocks, num_kv_heads, block_size, head_dim = _pool_shape(
        key_cache, value_cache
    )
    k_scale, v_scale = _pool_scales(key_cache, k_scale, v_scale)
    k_scales, v_scales = _row_scales("rope_append_paged_decode", key_cache, k_scales, v_scales,
                                     k_scale, v_scale)
    if query.ndim != 3 or key.ndim != 3 or value.shape != key.shape:
        raise ValueError("query (B, Hq, Dh), key and value (B, Hkv, Dh) expected")
    num_seqs, num_q_heads, _ = query.shape
    if key.shape != (num_seqs, num_kv_heads, head_dim) or query.shape[2] != head_dim:
        raise ValueError("key and value rows must match the pool's (Hkv, Dh)")
    pool_dtype = query.dtype if is_fp8_pool(key_cache) else key_cache.dtype
    if len({query.dtype, key.dtype, value.dtype, pool_dtype, table.dtype}) != 1:
        raise ValueError("query, key, value, pools and the rotary table must share a dtype")
    if head_dim != table.head_dim:
        raise ValueError("head_dim must match the rotary table")
    if num_q_heads % num_kv_heads != 0:
        raise ValueError("query head count must be divisible by KV head count")
    if positions.shape != (num_seqs,) or slot_mapping.shape != (num_seqs,):
        raise ValueError("positions and slot_mapping must have shape (B,)")
    pos = positions if positions.dtype == torch.int64 else positions.to(torch.int64)
    pos = pos.contiguous()
    slots = _int_tensor(slot_mapping, torch.int64, "slot_mapping")
    for name, t in (("query", query), ("key", key), ("value", value)):
        if t.stride(-1) != 1:
            raise ValueError(f"{name} must be contiguous in head_dim")
    tables = _int_tensor(block_tables, torch.int32, "block_tables")
    lens = _int_tensor(seq_lens, torch.int32, "seq_lens")
    if tables.ndim != 2 or tables.shape[0] != num_seqs or lens.shape != (num_seqs,):
        raise ValueError("block_tables (B, max_blocks) and seq_lens (B,) must match query")
    if out is None:
        out = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    if out.shape != query.shape or out.dtype != query.dtype or out.stride(-1) != 1:
        raise ValueError("out must match query and be contiguous in head_dim")
    if scale is None:
        scale = 1.0 / sqrt(head_dim)
    order = _seq_order("rope_append_paged_decode", query, seq_order)
    _check_workspace("rope_append_paged_decode", query, workspace)
    _ops.rope_append_paged_decode(query, key, value, pos, table.cos, table.sin, slots, key_cache,
                                  value_cache, tables, lens, order, layer_index, max_seq_len,
                                  float(scale), pages_per_split, out, workspace, k_scale, v_scale,
                                  k_scales, v_scales)
    return out


# ----------------------------------------------------------------------------
# Greedy selection


def greedy_argmax(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """(B, V) logits -> (B, 1) int64 first-maximum indices (torch.argmax rules)."""

    require_hip("greedy_argmax", logits)
    if logits.ndim != 2:
        raise ValueError("logits must have shape (B, V)")
    if logits.shape[0] < 1:
        raise ValueError("logits must contain at least one batch row")
    if logits.shape[1] < 1:
        raise ValueError("vocabulary size must be positive")
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    if out is None:
        out = torch.empty((logits.shape[0], 1), dtype=torch.int64, device=logits.device)
    _ops.greedy_argmax(logits, out)
    return out


# ----------------------------------------------------------------------------
# Elementwise


def vector_add(x: torch.Tensor, y: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """out = x + y for contiguous 1-D fp32/fp16 HIP vectors of one shape."""

    require_hip("vector_add", x, y)
    if x.ndim != 1 or x.shape != y.shape or x.dtype != y.dtype:
        raise ValueError("x and y must be matching one-dimensional vectors")
    if not x.is_contiguous() or not y.is_contiguous():
        raise ValueError("x and y must be contiguous")
    if out is None:
        out = torch.empty_like(x)
    _ops.vector_add(x, y, out)
    return out


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """SwiGLU activation: (..., 2I) stacked gate/up rows -> (..., I) silu(gate) * up,
    rounded as functional.silu(gate) * up in the input dtype."""

    require_hip("silu_mul", gate_up)
    if gate_up.ndim < 1 or gate_up.shape[-1] % 2 != 0:
        raise ValueError("gate_up must have an even last dimension (gate then up)")
    inter = gate_up.shape[-1] // 2
    rows = gate_up.reshape(-1, 2 * inter)
    if rows.stride(-1) != 1:
        rows = rows.contiguous()
    if out is None:
        out = torch.empty((*gate_up.shape[:-1], inter), dtype=gate_up.dtype, device=gate_up.device)
    out_rows = out.view(-1, inter)
    _ops.silu_mul(rows, out_rows)
    return out
