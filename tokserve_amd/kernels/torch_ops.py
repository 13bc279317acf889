"""PyTorch operator registrations of the C-ABI kernels (`torch.ops.tokserve_amd.*`).

Each operator is declared with a schema that marks every tensor it writes
(`Tensor(a!)`: KV pools, outputs, in-place rotations), has a CUDA-key kernel
(HIP tensors dispatch as CUDA on ROCm) that hands the tensors' addresses,
strides and the current stream to one `libtokserve_hip.so` entry point through
the ctypes binding, and a fake (meta) kernel for tracing, so `torch.compile`,
FakeTensor propagation and HIP-graph capture all see the same operators. Every
operator writes into tensors the caller passes (the validated wrappers in
`ops.py` allocate them), so the fake kernels return nothing and the schemas need
no aliasing annotations beyond the writes.

The operators are defined with schema strings (`torch.library.define` / `impl`
/ `register_fake`) rather than the `custom_op` decorator: both register through
torch.library and both are traced by `torch.compile`, but the decorator's Python
wrapper costs ~30 us per eager call against ~9 us for a schema-defined operator
with a device kernel, and an eager prefill forward makes ~180 of these calls.

A CPU tensor reaching an operator directly finds no CPU kernel and fails with
torch's dispatch error: there is no host fallback.

Reference interfaces, by operator (the reference has no compiled code; its
kernels are Triton functions behind tokserve/kernels/<op>.py):
  kv_append                 SequencePagedKVCache.write_layer (engine/paged/sequence_cache.py:86-131)
  paged_gather              SequencePagedKVCache.read_layer (engine/paged/sequence_cache.py:133-193)
  paged_attention_decode    triton_paged_attention, Tq == 1 (kernels/paged_attention.py:11-88)
  paged_attention_prefill   triton_paged_attention / triton_tiled_attention (kernels/tiled_attention.py:9-73)
  rms_norm                  triton_rms_norm (kernels/rmsnorm.py:6-45)
  rope, rope_               triton_apply_rope (kernels/rope.py:8-63)
  rope_kv_append(_)         apply_rope then write_layer (engine/attention.py:247-265)
  greedy_argmax             select_greedy (generation/greedy.py:6-18)
  silu_mul                  SwiGLU's silu(gate) * up (engine/layers.py:84-91)
  vector_add                vector_add (kernels/vector.py:6-41)
"""

from __future__ import annotations

import torch

from tokserve_amd.kernels import _lib

NAMESPACE = "tokserve_amd"

FP8_POOL_DTYPE = torch.float8_e4m3fn

SCHEMAS = {
    "kv_append": (
        "kv_append(Tensor key, Tensor value, Tensor(a!) key_cache, Tensor(b!) value_cache, "
        "Tensor slot_mapping, int layer_index, float k_scale, float v_scale, "
        "Tensor(c!)? k_scales=None, Tensor(d!)? v_scales=None) -> ()"
    ),
    "paged_gather": (
        "paged_gather(Tensor key_cache, Tensor value_cache, Tensor block_tables, "
        "Tensor seq_lens, Tensor cu_seqlens, int layer_index, int max_seq_len, "
        "Tensor(a!) key_out, Tensor(b!) value_out, float k_scale, float v_scale, "
        "Tensor? k_scales=None, Tensor? v_scales=None) -> ()"
    ),
    "paged_attention_decode": (
        "paged_attention_decode(Tensor query, Tensor key_cache, Tensor value_cache, "
        "Tensor block_tables, Tensor seq_lens, Tensor? seq_order, int layer_index, "
        "int max_seq_len, float scale, int pages_per_split, float k_scale, float v_scale, "
        "Tensor(a!) out, Tensor(b!)? workspace, Tensor? k_scales=None, "
        "Tensor? v_scales=None) -> ()"
    ),
    "paged_attention_decode_noalloc": (
        "paged_attention_decode_noalloc(Tensor query, Tensor key_cache, Tensor value_cache, "
        "Tensor block_tables, Tensor seq_lens, Tensor? seq_order, int layer_index, "
        "int max_seq_len, float scale, int pages_per_split, Tensor(a!) out) -> ()"
    ),
    "paged_attention_prefill": (
        "paged_attention_prefill(Tensor query, Tensor key_cache, Tensor value_cache, "
        "Tensor block_tables, Tensor seq_lens, Tensor cu_seqlens_q, Tensor? seq_order, "
        "int layer_index, "
        "int max_query_len, int max_seq_len, float scale, float k_scale, float v_scale, "
        "Tensor(a!) out, Tensor? k_scales=None, Tensor? v_scales=None) -> ()"
    ),
    "rms_norm": (
        "rms_norm(Tensor input, Tensor weight, float epsilon, Tensor? residual, "
        "Tensor(a!) out, Tensor(b!)? residual_out) -> ()"
    ),
    "rope": (
        "rope(Tensor query, Tensor key, Tensor positions, Tensor cos, Tensor sin, "
        "Tensor(a!) query_out, Tensor(b!) key_out) -> ()"
    ),
    "rope_": (
        "rope_(Tensor(a!) query, Tensor(b!) key, Tensor positions, Tensor cos, Tensor sin) -> ()"
    ),
    "rope_kv_append": (
        "rope_kv_append(Tensor query, Tensor key, Tensor value, Tensor positions, Tensor cos, "
        "Tensor sin, Tensor(a!) key_cache, Tensor(b!) value_cache, Tensor slot_mapping, "
        "int layer_index, Tensor(c!) query_out, Tensor(d!)? key_out, float k_scale=1.0, "
        "float v_scale=1.0, Tensor(e!)? k_scales=None, Tensor(f!)? v_scales=None) -> ()"
    ),
    "rope_kv_append_": (
        "rope_kv_append_(Tensor(a!) query, Tensor key, Tensor value, Tensor positions, "
        "Tensor cos, Tensor sin, Tensor(b!) key_cache, Tensor(c!) value_cache, "
        "Tensor slot_mapping, int layer_index, Tensor(d!)? key_out, float k_scale=1.0, "
        "float v_scale=1.0, Tensor(e!)? k_scales=None, Tensor(f!)? v_scales=None) -> ()"
    ),
    "rope_append_paged_decode": (
        "rope_append_paged_decode(Tensor query, Tensor key, Tensor value, Tensor positions, "
        "Tensor cos, Tensor sin, Tensor slot_mapping, Tensor(a!) key_cache, "
        "Tensor(b!) value_cache, Tensor block_tables, Tensor seq_lens, Tensor? seq_order, "
        "int layer_index, int max_seq_len, float scale, int pages_per_split, Tensor(c!) out, "
        "Tensor(d!)? workspace, float k_scale=1.0, float v_scale=1.0, "
        "Tensor(e!)? k_scales=None, Tensor(f!)? v_scales=None) -> ()"
    ),
    "greedy_argmax": "greedy_argmax(Tensor logits, Tensor(a!) out) -> ()",
    "silu_mul": "silu_mul(Tensor gate_up, Tensor(a!) out) -> ()",
    "vector_add": "vector_add(Tensor x, Tensor y, Tensor(a!) out) -> ()",
}

# Entry points behind each operator (the *_fp8 ones serve e4m3 pools with one scale per
# pool, the *_fp8_rows ones e4m3 pools with one scale per pool row).
ENTRY_POINTS = {
    "kv_append": ("tks_kv_append", "tks_kv_append_fp8", "tks_kv_append_fp8_rows"),
    "paged_gather": ("tks_paged_gather", "tks_paged_gather_fp8", "tks_paged_gather_fp8_rows"),
    "paged_attention_decode": ("tks_paged_attention_decode_workspace_bytes",
                               "tks_paged_attention_decode", "tks_paged_attention_decode_fp8",
                               "tks_paged_attention_decode_fp8_rows"),
    "paged_attention_decode_noalloc": ("tks_paged_attention_decode_noalloc",
                                       "tks_paged_attention_decode_noalloc_max_workspace_bytes"),
    "paged_attention_prefill": ("tks_paged_attention_prefill",
                                "tks_paged_attention_prefill_fp8_workspace_bytes",
                                "tks_paged_attention_prefill_fp8",
                                "tks_paged_attention_prefill_fp8_rows"),
    "rms_norm": ("tks_rms_norm",),
    "rope": ("tks_rope",),
    "rope_": ("tks_rope",),
    "rope_kv_append": ("tks_rope_kv_append", "tks_rope_kv_append_fp8",
                       "tks_rope_kv_append_fp8_rows"),
    "rope_kv_append_": ("tks_rope_kv_append", "tks_rope_kv_append_fp8",
                        "tks_rope_kv_append_fp8_rows"),
    "rope_append_paged_decode": ("tks_rope_append_paged_decode",
                                 "tks_rope_append_paged_decode_fp8",
                                 "tks_rope_append_paged_decode_fp8_rows",
                                 "tks_paged_attention_decode_workspace_bytes"),
    "greedy_argmax": ("tks_argmax",),
    "silu_mul": ("tks_silu_mul",),
    "vector_add": ("tks_vector_add",),
}


def _code(tensor: torch.Tensor) -> int:
    return _lib.dtype_code(tensor.dtype)


def _stream(tensor: torch.Tensor) -> int:
    return _lib.stream_of(tensor)


def _pool_dims(pool: torch.Tensor) -> tuple[int, int, int, int, int]:
    num_layers, num_blocks, num_kv_heads, block_size, head_dim = pool.shape
    return num_layers, num_blocks, num_kv_heads, block_size, head_dim


# Per-(device, use) scratch buffers of the kernels that need one. They only grow;
# a replaced buffer stays allocated, since a captured HIP graph keeps the device
# address it was recorded with. Calls that share a buffer are ordered on one
# stream, as the kernels require.
_workspaces: dict[tuple[torch.device, str], torch.Tensor] = {}
_retired: list[torch.Tensor] = []


def workspace(device: torch.device, nbytes: int, use: str) -> torch.Tensor | None:
    """A scratch buffer of at least nbytes for `use` on `device` (None for 0 bytes)."""

    if nbytes == 0:
        return None
    slot = (torch.device(device), use)
    buffer = _workspaces.get(slot)
    if buffer is None or buffer.numel() < nbytes:
        size = max(nbytes, 1 << 20, 0 if buffer is None else 2 * buffer.numel())
        if buffer is not None:
            _retired.append(buffer)
        buffer = torch.empty(size, dtype=torch.uint8, device=device)
        _workspaces[slot] = buffer
    return buffer


def decode_workspace_bytes(num_seqs: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                           block_size: int, max_seq_len: int, pages_per_split: int) -> int:
    size = _lib.load().tks_paged_attention_decode_workspace_bytes(
        num_seqs, num_q_heads, num_kv_heads, head_dim, block_size, max_seq_len, pages_per_split)
    if size < 0:
        raise ValueError("invalid decode workspace query")
    return int(size)


# ----------------------------------------------------------------------------
# Device kernels


def _kv_append(key, value, key_cache, value_cache, slot_mapping, layer_index, k_scale, v_scale,
               k_scales=None, v_scales=None):
    dims = _pool_dims(key_cache)
    rows = (key.data_ptr(), key.stride(0), key.stride(1),
            value.data_ptr(), value.stride(0), value.stride(1), key.shape[0],
            key_cache.data_ptr(), value_cache.data_ptr())
    common = (*rows, *dims, layer_index, slot_mapping.data_ptr())
    library = _lib.load()
    if k_scales is not None:
        status = library.tks_kv_append_fp8_rows(*rows, k_scales.data_ptr(), v_scales.data_ptr(),
                                                *dims, layer_index, slot_mapping.data_ptr(),
                                                _code(key), _stream(key))
    elif key_cache.dtype == FP8_POOL_DTYPE:
        status = library.tks_kv_append_fp8(*common, k_scale, v_scale, _code(key), _stream(key))
    else:
        status = library.tks_kv_append(*common, _code(key), _stream(key))
    _lib.check(status, "kv_append")


def _paged_gather(key_cache, value_cache, block_tables, seq_lens, cu_seqlens, layer_index,
                  max_seq_len, key_out, value_out, k_scale, v_scale, k_scales=None,
                  v_scales=None):
    rest = (*_pool_dims(key_cache), layer_index,
            block_tables.data_ptr(), block_tables.shape[1], seq_lens.data_ptr(),
            cu_seqlens.data_ptr(), block_tables.shape[0], max_seq_len,
            key_out.data_ptr(), value_out.data_ptr(), key_out.stride(0), key_out.stride(1))
    common = (key_cache.data_ptr(), value_cache.data_ptr(), *rest)
    library = _lib.load()
    if k_scales is not None:
        status = library.tks_paged_gather_fp8_rows(
            key_cache.data_ptr(), value_cache.data_ptr(), k_scales.data_ptr(),
            v_scales.data_ptr(), *rest, _code(key_out), _stream(key_cache))
    elif key_cache.dtype == FP8_POOL_DTYPE:
        status = library.tks_paged_gather_fp8(*common, k_scale, v_scale, _code(key_out),
                                              _stream(key_cache))
    else:
        status = library.tks_paged_gather(*common, _code(key_out), _stream(key_cache))
    _lib.check(status, "paged_gather")


def _decode_common(query, key_cache, value_cache, block_tables, seq_lens, seq_order,
                   layer_index, max_seq_len, scale, pages_per_split, out):
    return (query.data_ptr(), query.stride(0), query.stride(1),
            key_cache.data_ptr(), value_cache.data_ptr(), *_pool_dims(key_cache), layer_index,
            block_tables.data_ptr(), block_tables.shape[1], seq_lens.data_ptr(),
            _lib.ptr(seq_order), query.shape[0], query.shape[1], max_seq_len, scale,
            pages_per_split, out.data_ptr(), out.stride(0), out.stride(1))


def _paged_attention_decode(query, key_cache, value_cache, block_tables, seq_lens, seq_order,
                            layer_index, max_seq_len, scale, pages_per_split, k_scale, v_scale,
                            out, workspace_tensor, k_scales=None, v_scales=None):
    _, _, num_kv_heads, block_size, head_dim = _pool_dims(key_cache)
    if workspace_tensor is None:
        nbytes = decode_workspace_bytes(query.shape[0], query.shape[1], num_kv_heads, head_dim,
                                        block_size, max_seq_len, pages_per_split)
        workspace_tensor = workspace(query.device, nbytes, "decode")
    common = _decode_common(query, key_cache, value_cache, block_tables, seq_lens, seq_order,
                            layer_index, max_seq_len, scale, pages_per_split, out)
    ws = (_lib.ptr(workspace_tensor), 0 if workspace_tensor is None else workspace_tensor.numel())
    library = _lib.load()
    if k_scales is not None:
        # The row entry takes the scale arrays right after the pools.
        status = library.tks_paged_attention_decode_fp8_rows(
            *common[:5], k_scales.data_ptr(), v_scales.data_ptr(), *common[5:], *ws,
            _code(query), _stream(query))
    elif key_cache.dtype == FP8_POOL_DTYPE:
        status = library.tks_paged_attention_decode_fp8(*common, *ws, k_scale, v_scale,
                                                        _code(query), _stream(query))
    else:
        status = library.tks_paged_attention_decode(*common, *ws, _code(query), _stream(query))
    _lib.check(status, "paged_attention_decode")


def _paged_attention_decode_noalloc(query, key_cache, value_cache, block_tables, seq_lens,
                                    seq_order, layer_index, max_seq_len, scale, pages_per_split,
                                    out):
    common = _decode_common(query, key_cache, value_cache, block_tables, seq_lens, seq_order,
                            layer_index, max_seq_len, scale, pages_per_split, out)
    status = _lib.load().tks_paged_attention_decode_noalloc(*common, _code(query),
                                                            _stream(query))
    _lib.check(status, "paged_attention_decode_noalloc")


def _paged_attention_prefill(query, key_cache, value_cache, block_tables, seq_lens,
                             cu_seqlens_q, seq_order, layer_index, max_query_len, max_seq_len,
                             scale, k_scale, v_scale, out, k_scales=None, v_scales=None):
    dims = _pool_dims(key_cache)
    num_seqs = seq_lens.shape[0]
    common = (query.data_ptr(), query.stride(0), query.stride(1),
              key_cache.data_ptr(), value_cache.data_ptr(), *dims, layer_index,
              block_tables.data_ptr(), block_tables.shape[1], seq_lens.data_ptr(),
              cu_seqlens_q.data_ptr(), _lib.ptr(seq_order), num_seqs, query.shape[0],
              query.shape[1],
              max_query_len, max_seq_len, scale, out.data_ptr(), out.stride(0), out.stride(1))
    library = _lib.load()
    if key_cache.dtype == FP8_POOL_DTYPE:
        _, _, num_kv_heads, block_size, head_dim = dims
        nbytes = library.tks_paged_attention_prefill_fp8_workspace_bytes(
            num_seqs, query.shape[1], num_kv_heads, head_dim, block_size, block_tables.shape[1],
            max_seq_len, _code(query))
        if nbytes < 0:
            raise ValueError("invalid fp8 prefill workspace query")
        scratch = workspace(query.device, nbytes, "prefill_fp8_pages")
        ws = (_lib.ptr(scratch), 0 if scratch is None else scratch.numel())
        if k_scales is not None:
            # The row entry takes the scale arrays right after the pools.
            status = library.tks_paged_attention_prefill_fp8_rows(
                *common[:5], k_scales.data_ptr(), v_scales.data_ptr(), *common[5:], *ws,
                _code(query), _stream(query))
        else:
            status = library.tks_paged_attention_prefill_fp8(
                *common, *ws, k_scale, v_scale, _code(query), _stream(query))
    else:
        status = library.tks_paged_attention_prefill(*common, _code(query), _stream(query))
    _lib.check(status, "paged_attention_prefill")


def _rms_norm(inputs, weight, epsilon, residual, out, residual_out):
    status = _lib.load().tks_rms_norm(
        inputs.data_ptr(), inputs.stride(0),
        _lib.ptr(residual), 0 if residual is None else residual.stride(0),
        _lib.ptr(residual_out), 0 if residual_out is None else residual_out.stride(0),
        weight.data_ptr(), out.data_ptr(), out.stride(0), inputs.shape[0], inputs.shape[1],
        epsilon, _code(inputs), _code(weight), _code(out), _stream(inputs))
    _lib.check(status, "rms_norm")


def _rope_launch(query, key, positions, cos, sin, query_out, key_out):
    batch, num_q_heads, tokens, head_dim = query.shape
    status = _lib.load().tks_rope(
        query.data_ptr(), query_out.data_ptr(),
        query.stride(0), query.stride(1), query.stride(2),
        query_out.stride(0), query_out.stride(1), query_out.stride(2), num_q_heads,
        key.data_ptr(), key_out.data_ptr(), key.stride(0), key.stride(1), key.stride(2),
        key_out.stride(0), key_out.stride(1), key_out.stride(2), key.shape[1],
        batch, tokens, head_dim, positions.data_ptr(), cos.data_ptr(), sin.data_ptr(),
        cos.shape[0], _code(query), _stream(query))
    _lib.check(status, "rope")


def _rope(query, key, positions, cos, sin, query_out, key_out):
    _rope_launch(query, key, positions, cos, sin, query_out, key_out)


def _rope_inplace(query, key, positions, cos, sin):
    _rope_launch(query, key, positions, cos, sin, query, key)


def _rope_kv_append_launch(query, query_out, key, value, positions, cos, sin, key_cache,
                           value_cache, slot_mapping, layer_index, key_out, k_scale, v_scale,
                           k_scales, v_scales):
    num_layers, num_blocks, num_kv_heads, block_size, head_dim = _pool_dims(key_cache)
    library = _lib.load()
    fp8 = key_cache.dtype == FP8_POOL_DTYPE
    pools = (key_cache.data_ptr(), value_cache.data_ptr())
    if k_scales is not None:
        entry, scales = library.tks_rope_kv_append_fp8_rows, ()
        pools += (k_scales.data_ptr(), v_scales.data_ptr())
    elif fp8:
        entry, scales = library.tks_rope_kv_append_fp8, (k_scale, v_scale)
    else:
        entry, scales = library.tks_rope_kv_append, ()
    status = entry(
        query.data_ptr(), query_out.data_ptr(), query.stride(0), query.stride(1),
        query_out.stride(0), query_out.stride(1), query.shape[1],
        key.data_ptr(), _lib.ptr(key_out), key.stride(0), key.stride(1),
        0 if key_out is None else key_out.stride(0), 0 if key_out is None else key_out.stride(1),
        value.data_ptr(), value.stride(0), value.stride(1), num_kv_heads, query.shape[0],
        head_dim, positions.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.shape[0],
        *pools, num_layers, num_blocks, block_size,
        layer_index, slot_mapping.data_ptr(), *scales, _code(query), _stream(query))
    _lib.check(status, "rope_kv_append")


def _rope_kv_append(query, key, value, positions, cos, sin, key_cache, value_cache,
                    slot_mapping, layer_index, query_out, key_out, k_scale=1.0, v_scale=1.0,
                    k_scales=None, v_scales=None):
    _rope_kv_append_launch(query, query_out, key, value, positions, cos, sin, key_cache,
                           value_cache, slot_mapping, layer_index, key_out, k_scale, v_scale,
                           k_scales, v_scales)


def _rope_kv_append_inplace(query, key, value, positions, cos, sin, key_cache, value_cache,
                            slot_mapping, layer_index, key_out, k_scale=1.0, v_scale=1.0,
                            k_scales=None, v_scales=None):
    _rope_kv_append_launch(query, query, key, value, positions, cos, sin, key_cache,
                           value_cache, slot_mapping, layer_index, key_out, k_scale, v_scale,
                           k_scales, v_scales)


def _rope_append_paged_decode(query, key, value, positions, cos, sin, slot_mapping, key_cache,
                              value_cache, block_tables, seq_lens, seq_order, layer_index,
                              max_seq_len, scale, pages_per_split, out, workspace_tensor,
                              k_scale=1.0, v_scale=1.0, k_scales=None, v_scales=None):
    num_layers, num_blocks, num_kv_heads, block_size, head_dim = _pool_dims(key_cache)
    if workspace_tensor is None:
        nbytes = decode_workspace_bytes(query.shape[0], query.shape[1], num_kv_heads, head_dim,
                                        block_size, max_seq_len, pages_per_split)
        workspace_tensor = workspace(query.device, nbytes, "decode")
    library = _lib.load()
    fp8 = key_cache.dtype == FP8_POOL_DTYPE
    pools = (key_cache.data_ptr(), value_cache.data_ptr())
    if k_scales is not None:
        entry, scales = library.tks_rope_append_paged_decode_fp8_rows, ()
        pools += (k_scales.data_ptr(), v_scales.data_ptr())
    elif fp8:
        entry, scales = library.tks_rope_append_paged_decode_fp8, (k_scale, v_scale)
    else:
        entry, scales = library.tks_rope_append_paged_decode, ()
    status = entry(
        query.data_ptr(), query.stride(0), query.stride(1),
        key.data_ptr(), key.stride(0), key.stride(1),
        value.data_ptr(), value.stride(0), value.stride(1),
        positions.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.shape[0],
        slot_mapping.data_ptr(), *pools,
        num_layers, num_blocks, num_kv_heads, block_size, head_dim, layer_index,
        block_tables.data_ptr(), block_tables.shape[1], seq_lens.data_ptr(), _lib.ptr(seq_order),
        query.shape[0], query.shape[1], max_seq_len, scale, pages_per_split,
        out.data_ptr(), out.stride(0), out.stride(1),
        _lib.ptr(workspace_tensor), 0 if workspace_tensor is None else workspace_tensor.numel(),
        *scales, _code(query), _stream(query))
    _lib.check(status, "rope_append_paged_decode")


def _greedy_argmax(logits, out):
    status = _lib.load().tks_argmax(logits.data_ptr(), logits.stride(0), logits.shape[0],
                                    logits.shape[1], out.data_ptr(), _code(logits),
                                    _stream(logits))
    _lib.check(status, "greedy_argmax")


def _silu_mul(gate_up, out):
    status = _lib.load().tks_silu_mul(gate_up.data_ptr(), gate_up.stride(0), gate_up.shape[0],
                                      gate_up.shape[1] // 2, out.data_ptr(), out.stride(0),
                                      _code(gate_up), _stream(gate_up))
    _lib.check(status, "silu_mul")


def _vector_add(x, y, out):
    status = _lib.load().tks_vector_add(x.data_ptr(), y.data_ptr(), out.data_ptr(), x.numel(),
                                        _code(x), _stream(x))
    _lib.check(status, "vector_add")


KERNELS = {
    "kv_append": _kv_append,
    "paged_gather": _paged_gather,
    "paged_attention_decode": _paged_attention_decode,
    "paged_attention_decode_noalloc": _paged_attention_decode_noalloc,
    "paged_attention_prefill": _paged_attention_prefill,
    "rms_norm": _rms_norm,
    "rope": _rope,
    "rope_": _rope_inplace,
    "rope_kv_append": _rope_kv_append,
    "rope_kv_append_": _rope_kv_append_inplace,
    "rope_append_paged_decode": _rope_append_paged_decode,
    "greedy_argmax": _greedy_argmax,
    "silu_mul": _silu_mul,
    "vector_add": _vector_add,
}


def _fake(*args, **kwargs) -> None:
    """Every operator writes only into tensors it is given: nothing to propagate."""

    return None


def _register() -> None:
    library = torch.library.Library(NAMESPACE, "DEF")
    for name, schema in SCHEMAS.items():
        library.define(schema)
        library.impl(name, KERNELS[name], "CUDA")
        torch.library.register_fake(f"{NAMESPACE}::{name}", _fake, lib=library)
    # Kept for the life of the process: dropping the handle would deregister the ops.
    globals()["_LIBRARY"] = library


if not hasattr(torch.ops, NAMESPACE) or not hasattr(getattr(torch.ops, NAMESPACE), "kv_append"):
    _register()
