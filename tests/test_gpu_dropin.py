"""The drop-in operators (tokserve.kernels.* names) and the paged-KV mirror on the GPU.

Cases follow the reference's own GPU tests: tests/gpu/test_paged_tiled_attention.py
(sentinel-filled pool read through non-contiguous pages (3, 1, 2)),
tests/gpu/test_tiled_attention.py (query/key length and offset grid, GQA
ratios, head-distinct values), tests/gpu/test_rmsnorm.py, test_triton_rope.py,
test_vector.py, and tests/integration/test_paged_kv_cache_parity.py (values
K = v + 100 * layer, V = K + 1000 that make every layer and slot distinct).
Expected values come from the oracle. fp32 within rtol 1e-5 / atol 1e-6 unless
a test says otherwise; bf16/fp16 within 2e-2 absolute.
"""

import pytest
import torch
from torch.testing import assert_close

from oracle import torch_path
from tokserve_amd.engine.paged.manager import PagedKVCacheManager
from tokserve_amd.engine.paged.storage import PagedKVStorage
from tokserve_amd.kernels.paged_attention import triton_paged_attention
from tokserve_amd.kernels.rmsnorm import triton_rms_norm
from tokserve_amd.kernels.rope import triton_apply_rope
from tokserve_amd.kernels.tiled_attention import triton_tiled_attention
from tokserve_amd.kernels.vector import vector_add

pytestmark = pytest.mark.gpu

FP32 = dict(rtol=1e-5, atol=1e-6)
HALF = dict(rtol=0, atol=2e-2)


def _assert_half_parity(actual, query, key, value, offset) -> None:
    """bf16/fp16 attention: within 2e-2 of the reference kernel's fp32 arithmetic and within
    the reference's own 4e-2 of its torch backend (tests/gpu/test_tiled_attention_prefill.py:50-59)."""

    actual = actual.cpu()
    kernel = torch_path.gqa_attention(query.float(), key.float(), value.float(),
                                      query_position_offset=offset).to(query.dtype)
    assert_close(actual, kernel, **HALF)
    backend = torch_path.gqa_attention(query, key, value, query_position_offset=offset)
    assert_close(actual, backend, rtol=0, atol=4e-2)


def _randn(*shape, seed, dtype=torch.float32):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)).to(dtype)


# ----------------------------------------------------------- paged attention

def _sentinel_storage(device, dtype, *, layers=1, blocks=4, hkv=2, bs=2, dh=8):
    storage = PagedKVStorage(num_layers=layers, num_blocks=blocks, num_key_value_heads=hkv,
                             block_size=bs, head_dim=dh, device=device, dtype=dtype)
    storage.key_storage.fill_(50_000.0)
    storage.value_storage.fill_(-50_000.0)
    return storage


@pytest.mark.parametrize(("query_length", "key_length", "offset"), [(1, 5, 4), (3, 5, 2),
                                                                    (5, 5, 0), (2, 6, 3)])
def test_paged_attention_reads_noncontiguous_pages(device, query_length, key_length, offset) -> None:
    storage = _sentinel_storage(device, torch.float32)
    block_ids = (3, 1, 2)
    query = _randn(1, 4, query_length, 8, seed=700)
    keys = _randn(1, 2, key_length, 8, seed=701)
    values = _randn(1, 2, key_length, 8, seed=702)
    for position in range(key_length):
        storage.write_token(layer_index=0, block_id=block_ids[position // 2], offset=position % 2,
                            keys=keys[0, :, position].to(device),
                            values=values[0, :, position].to(device))
    expected = torch_path.gqa_attention(query, keys, values, query_position_offset=offset)
    actual = triton_paged_attention(query.to(device), storage, block_ids, layer_index=0,
                                    key_length=key_length, query_position_offset=offset)
    torch.cuda.synchronize()
    assert actual.shape == query.shape and actual.dtype == query.dtype
    assert_close(actual.cpu(), expected, **FP32)


@pytest.mark.parametrize(("query_length", "offset"), [(1, 299), (64, 236), (300, 0)])
def test_paged_attention_bf16_model_shape(device, query_length, offset) -> None:
    """Llama-3-8B heads (32/8, Dh 128), block size 16: the MFMA decode and prefill kernels."""

    key_length = 300
    storage = _sentinel_storage(device, torch.bfloat16, blocks=24, hkv=8, bs=16, dh=128)
    block_ids = tuple(int(b) for b in torch.randperm(24, generator=torch.Generator().manual_seed(3)))
    keys = _randn(1, 8, key_length, 128, seed=710, dtype=torch.bfloat16)
    values = _randn(1, 8, key_length, 128, seed=711, dtype=torch.bfloat16)
    cache = storage
    for position in range(key_length):
        cache.write_token(layer_index=0, block_id=block_ids[position // 16], offset=position % 16,
                          keys=keys[0, :, position].to(device), values=values[0, :, position].to(device))
    query = _randn(1, 32, query_length, 128, seed=712, dtype=torch.bfloat16)
    actual = triton_paged_attention(query.to(device), storage, block_ids, layer_index=0,
                                    key_length=key_length, query_position_offset=offset)
    torch.cuda.synchronize()
    _assert_half_parity(actual, query, keys, values, offset)


def test_paged_attention_argument_errors(device) -> None:
    storage = _sentinel_storage(device, torch.float32)
    query = torch.zeros(1, 4, 1, 8, device=device)
    with pytest.raises(ValueError, match="cannot exceed key length"):
        triton_paged_attention(query, storage, (0,), layer_index=0, key_length=1,
                               query_position_offset=1)
    with pytest.raises(ValueError, match="does not cover the valid key length"):
        triton_paged_attention(query, storage, (0,), layer_index=0, key_length=3,
                               query_position_offset=2)
    with pytest.raises(IndexError, match="layer_index is out of range"):
        triton_paged_attention(query, storage, (0,), layer_index=1, key_length=1,
                               query_position_offset=0)
    with pytest.raises(ValueError, match="divisible by KV head count"):
        triton_paged_attention(torch.zeros(1, 3, 1, 8, device=device), storage, (0,),
                               layer_index=0, key_length=1, query_position_offset=0)
    with pytest.raises(ValueError, match="same dtype"):
        triton_paged_attention(query.half(), storage, (0,), layer_index=0, key_length=1,
                               query_position_offset=0)


# ----------------------------------------------------------- tiled attention

@pytest.mark.parametrize(("query_length", "key_length", "offset", "head_dim"), [
    (1, 1, 0, 8), (7, 7, 0, 8), (16, 16, 0, 16), (17, 17, 0, 16), (1, 35, 34, 8), (3, 19, 16, 8),
])
def test_tiled_attention_grid(device, query_length, key_length, offset, head_dim) -> None:
    query = _randn(2, 2, query_length, head_dim, seed=400)
    key = _randn(2, 2, key_length, head_dim, seed=401)
    value = _randn(2, 2, key_length, head_dim, seed=402)
    expected, _ = torch_path.causal_attention(query, key, value, query_position_offset=offset)
    actual = triton_tiled_attention(query.to(device), key.to(device), value.to(device),
                                    query_position_offset=offset)
    torch.cuda.synchronize()
    assert actual.shape == query.shape and actual.dtype == query.dtype and actual.is_cuda
    assert_close(actual.cpu(), expected, **FP32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize(("hq", "hkv", "dh", "tq", "tk", "offset"), [
    (8, 2, 128, 40, 64, 24), (8, 8, 64, 32, 32, 0), (32, 8, 128, 1, 96, 95), (4, 1, 128, 20, 48, 3),
    (8, 2, 64, 10, 30, 5),
])
def test_tiled_attention_half_precision(device, dtype, hq, hkv, dh, tq, tk, offset) -> None:
    """Key lengths that are multiples of 16 run the MFMA kernel (the batch is a pool of
    one Tk-key block per row); others, like 30, the generic one."""

    query = _randn(2, hq, tq, dh, seed=403, dtype=dtype)
    key = _randn(2, hkv, tk, dh, seed=404, dtype=dtype)
    value = _randn(2, hkv, tk, dh, seed=405, dtype=dtype)
    actual = triton_tiled_attention(query.to(device), key.to(device), value.to(device),
                                    query_position_offset=offset)
    torch.cuda.synchronize()
    _assert_half_parity(actual, query, key, value, offset)


def test_tiled_attention_noncontiguous_views(device) -> None:
    sources = [_randn(1, 2, 9, 16, seed=410 + i).to(device) for i in range(3)]
    query, key, value = (s[..., ::2] for s in sources)
    assert not query.is_contiguous()
    expected, _ = torch_path.causal_attention(query.cpu(), key.cpu(), value.cpu())
    actual = triton_tiled_attention(query, key, value)
    torch.cuda.synchronize()
    assert_close(actual.cpu(), expected, **FP32)


@pytest.mark.parametrize(("hq", "hkv"), [(2, 2), (4, 2), (8, 2), (8, 1)])
def test_tiled_attention_gqa(device, hq, hkv) -> None:
    query = _randn(1, hq, 19, 8, seed=420)
    key = _randn(1, hkv, 19, 8, seed=421)
    value = _randn(1, hkv, 19, 8, seed=422)
    expected = torch_path.gqa_attention(query, key, value, query_position_offset=0)
    actual = triton_tiled_attention(query.to(device), key.to(device), value.to(device))
    torch.cuda.synchronize()
    assert_close(actual.cpu(), expected, **FP32)


def test_tiled_attention_gqa_mapping_known_answer(device) -> None:
    """Query head h reads KV head h // G: zero scores average V of that head exactly."""

    query = torch.zeros(1, 4, 1, 8, device=device)
    key = torch.zeros(1, 2, 1, 8, device=device)
    value = torch.empty(1, 2, 1, 8, device=device)
    value[:, 0] = 10.0
    value[:, 1] = 20.0
    actual = triton_tiled_attention(query, key, value).cpu()
    for head, expected in enumerate((10.0, 10.0, 20.0, 20.0)):
        assert torch.equal(actual[:, head], torch.full_like(actual[:, head], expected))


def test_tiled_attention_rejects_bad_gqa_ratio(device) -> None:
    with pytest.raises(ValueError, match="query head count must be divisible"):
        triton_tiled_attention(torch.zeros(1, 3, 7, 8, device=device),
                               torch.zeros(1, 2, 7, 8, device=device),
                               torch.zeros(1, 2, 7, 8, device=device))


# ------------------------------------------------------------- RMSNorm / RoPE

@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", [(1, 8), (2, 3, 512), (5, 4096), (3, 1000)])
def test_rms_norm_float32_contract(device, dtype, shape) -> None:
    inputs = _randn(*shape, seed=800, dtype=dtype)
    weight = 1.0 + 0.02 * _randn(shape[-1], seed=801)
    expected = torch_path.rms_norm(inputs, weight, 1e-6)
    actual = triton_rms_norm(inputs.to(device), weight.to(device))
    torch.cuda.synchronize()
    assert actual.dtype == torch.float32 and actual.shape == inputs.shape
    # Both sides round the normalized value to the input dtype; a last-bit
    # difference in the fp32 mean can move that rounding by one input ulp.
    ulp = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 1.6e-2}[dtype]
    assert_close(actual.cpu(), expected, rtol=ulp, atol=1e-5)


def test_rms_norm_contract_errors(device) -> None:
    inputs = torch.zeros(2, 8, device=device)
    with pytest.raises(TypeError, match="weight must use float32"):
        triton_rms_norm(inputs, torch.ones(8, device=device, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match=r"weight must have shape \(D,\)"):
        triton_rms_norm(inputs, torch.ones(7, device=device))
    with pytest.raises(ValueError, match="epsilon must be positive"):
        triton_rms_norm(inputs, torch.ones(8, device=device), epsilon=0.0)
    empty = triton_rms_norm(torch.zeros(0, 8, device=device), torch.ones(8, device=device))
    assert empty.shape == (0, 8) and empty.dtype == torch.float32


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("position_dtype", [torch.int32, torch.int64])
def test_apply_rope_matches_oracle(device, dtype, position_dtype) -> None:
    query = _randn(2, 8, 11, 64, seed=900, dtype=dtype)
    key = _randn(2, 2, 11, 64, seed=901, dtype=dtype)
    positions = torch.tensor([0, 1, 2, 7, 100, 511, 4095, 4096, 9000, 3, 3], dtype=position_dtype)
    expected_q, expected_k = torch_path.apply_rope(query, key, positions, theta=10_000.0)
    actual_q, actual_k = triton_apply_rope(query.to(device), key.to(device), positions.to(device),
                                           theta=10_000.0)
    torch.cuda.synchronize()
    tol = FP32 if dtype == torch.float32 else dict(rtol=0, atol=1e-2)
    assert_close(actual_q.cpu(), expected_q, **tol)
    assert_close(actual_k.cpu(), expected_k, **tol)


def test_apply_rope_position_zero_is_identity_and_errors(device) -> None:
    query = _randn(1, 2, 3, 16, seed=902).to(device)
    key = _randn(1, 1, 3, 16, seed=903).to(device)
    zeros = torch.zeros(3, dtype=torch.int64, device=device)
    q, k = triton_apply_rope(query, key, zeros, theta=500_000.0)
    assert torch.equal(q, query) and torch.equal(k, key)
    with pytest.raises(ValueError, match="positions must be nonnegative"):
        triton_apply_rope(query, key, torch.tensor([0, -1, 2], device=device), theta=1e4)
    with pytest.raises(TypeError, match="positions must contain integers"):
        triton_apply_rope(query, key, torch.zeros(3, device=device), theta=1e4)


# ------------------------------------------------------------------- vector

@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("n", [1, 7, 1024, 1_000_003])
def test_vector_add(device, dtype, n) -> None:
    x = _randn(n + 1, seed=60, dtype=dtype)
    y = _randn(n + 1, seed=61, dtype=dtype)
    for sl in (slice(0, n), slice(1, n + 1)):  # 16-byte aligned and misaligned starts
        out = vector_add(x[sl].to(device), y[sl].to(device))
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), x[sl] + y[sl])


def test_vector_add_contract(device) -> None:
    x = torch.ones(4, device=device)
    assert vector_add(x[:0], x[:0]).numel() == 0
    with pytest.raises(TypeError, match="float32 and float16"):
        vector_add(x.bfloat16(), x.bfloat16())
    with pytest.raises(ValueError, match="contiguous"):
        vector_add(torch.ones(8, device=device)[::2], x)
    with pytest.raises(ValueError, match="matching shapes"):
        vector_add(x, torch.ones(5, device=device))


# ------------------------------------------------------------ paged KV mirror

def _distinct(layer, hkv, length, dh, start=0):
    v = torch.arange(start * hkv * dh, (start + length) * hkv * dh, dtype=torch.float32)
    keys = v.view(length, hkv, dh).transpose(0, 1) + 100.0 * layer  # (Hkv, T, Dh)
    return keys, keys + 1000.0


def test_storage_token_round_trip_and_isolation(device) -> None:
    storage = _sentinel_storage(device, torch.float32, layers=2, blocks=3, hkv=2, bs=4, dh=8)
    keys = _randn(2, 8, seed=30).to(device)
    storage.write_token(layer_index=1, block_id=2, offset=3, keys=keys, values=keys + 1)
    k, v = storage.read_token(layer_index=1, block_id=2, offset=3)
    assert torch.equal(k, keys) and torch.equal(v, keys + 1)
    k0, _ = storage.read_token(layer_index=0, block_id=2, offset=3)
    assert torch.equal(k0, torch.full_like(k0, 50_000.0))
    written = keys.clone()
    keys.add_(5.0)  # the storage holds a copy
    assert torch.equal(storage.read_token(layer_index=1, block_id=2, offset=3)[0], written)


def test_sequence_cache_reads_logical_order_per_layer(device) -> None:
    manager = PagedKVCacheManager(num_layers=2, num_blocks=10, num_key_value_heads=2, block_size=3,
                                  head_dim=4, device=device, dtype=torch.float32)
    other = manager.create_sequence("other", max_sequence_length=32)
    cache = manager.create_sequence("s", max_sequence_length=32)
    length = 0
    for step, (owner, count) in enumerate([(cache, 5), (other, 4), (cache, 1), (cache, 4)]):
        start = owner.current_length
        owner.begin_append(count)
        for layer in range(2):
            keys, values = _distinct(layer, 2, count, 4, start)
            if owner is cache and layer == 0 and step == 2:
                # Positions stay hidden until written, and include_pending shows them.
                assert owner.read_layer(0)[0].shape == (1, 2, length, 4)
            owner.write_layer(layer, keys.to(device), values.to(device))
        assert owner.read_layer(1, include_pending=True)[0].shape[2] == start + count
        owner.finish_append()
        if owner is cache:
            length += count
    for layer in range(2):
        keys, values = _distinct(layer, 2, length, 4)
        k, v = cache.read_layer(layer)
        assert torch.equal(k.cpu(), keys.unsqueeze(0)) and torch.equal(v.cpu(), values.unsqueeze(0))
    # The interleaved appends gave the sequences disjoint, lowest-first blocks.
    assert cache.block_ids == (0, 1, 4, 5) and other.block_ids == (2, 3)


def test_released_blocks_are_reused_without_exposing_stale_values(device) -> None:
    manager = PagedKVCacheManager(num_layers=1, num_blocks=4, num_key_value_heads=1, block_size=2,
                                  head_dim=4, device=device, dtype=torch.float32)
    first = manager.create_sequence("a", max_sequence_length=8)
    first.begin_append(4)
    first.write_layer(0, torch.ones(1, 4, 4, device=device), torch.ones(1, 4, 4, device=device))
    first.finish_append()
    kept = manager.create_sequence("b", max_sequence_length=8)
    kept.begin_append(2)
    kept.write_layer(0, torch.full((1, 2, 4), 7.0, device=device),
                     torch.full((1, 2, 4), 8.0, device=device))
    kept.finish_append()
    manager.release_sequence("a")
    fresh = manager.create_sequence("c", max_sequence_length=8)
    fresh.begin_append(1)
    assert fresh.block_ids == (0,)
    fresh.write_layer(0, torch.full((1, 1, 4), 3.0, device=device),
                      torch.full((1, 1, 4), 4.0, device=device))
    fresh.finish_append()
    k, v = fresh.read_layer(0)
    assert k.shape == (1, 1, 1, 4) and torch.equal(k.cpu(), torch.full((1, 1, 1, 4), 3.0))
    kk, kv = kept.read_layer(0)
    assert torch.equal(kk.cpu(), torch.full((1, 1, 2, 4), 7.0))
    assert torch.equal(kv.cpu(), torch.full((1, 1, 2, 4), 8.0))
