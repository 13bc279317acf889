"""fp8 (OCP e4m3) K/V pools on the GPU against the CPU oracle.

The pool variant stores e4m3(clamp(x / scale, -448, 448)) with one fp32 scale
per pool and decodes float(code) * scale. Encoding (KV append) and decoding
(gather) are bit-exact against the oracle (oracle/paged.py quantize_e4m3 /
dequantize_e4m3, pinned by oracle/e4m3.c in tests/test_oracle_pins.py).
Attention over fp8 pools is the attention of the decoded pools: compared with
the oracle's fp32 arithmetic on those decoded values, fp32 within rtol 1e-5 /
atol 1e-6 and bf16/fp16 within 2e-2 absolute (the tolerances of the pools in
the model dtype).
"""

import pytest
import torch
from torch.testing import assert_close

from oracle import kvslots, paged
from tokserve_amd import workloads
from tokserve_amd.engine.paged.storage import PagedKVStorage
from tokserve_amd.kernels import ops

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn
TOL = {torch.float32: dict(rtol=1e-5, atol=1e-6), torch.float16: dict(rtol=0, atol=2e-2),
       torch.bfloat16: dict(rtol=0, atol=2e-2)}


def _rows(n, hkv, dh, dtype, seed):
    """Rows over many magnitudes plus the encoder's edge cases (ties, saturation, NaN)."""

    g = torch.Generator().manual_seed(seed)
    scale = 2.0 ** torch.randint(-12, 10, (n, hkv, 1), generator=g).float()
    x = torch.randn(n, hkv, dh, generator=g) * scale
    special = torch.tensor([0.0, -0.0, 1.0625, 1.1875, 2.0 ** -10, 3 * 2.0 ** -10, 440.0, 464.0,
                            1e30, -1e30, float("inf"), float("nan"), -float("nan"),
                            2.0 ** -6 - 2.0 ** -10])
    flat = x.view(-1)
    flat[: special.numel()] = special
    return x.to(dtype)


def _same_bits(a: torch.Tensor, b: torch.Tensor) -> None:
    assert a.shape == b.shape and a.dtype == b.dtype
    nan_a, nan_b = torch.isnan(a.float()), torch.isnan(b.float())
    assert torch.equal(nan_a, nan_b)
    assert torch.equal(a[~nan_a], b[~nan_b])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [128, 64, 24])
@pytest.mark.parametrize("scales", [(1.0, 1.0), (0.37, 2.5)])
def test_fp8_kv_append_bit_exact(device, dtype, head_dim, scales) -> None:
    """Quantizing append into fp8 pools equals the oracle's encoding scattered by the C
    restatement, byte for byte (16-byte path at Dh 64/128, element path at Dh 24)."""

    layers, blocks, hkv, bs, n = 2, 12, 4, 16, 70
    g = torch.Generator().manual_seed(head_dim)
    slots = torch.randperm(blocks * bs, generator=g)[:n].to(torch.int64)
    slots[5] = -1  # padding row: skipped
    keys, values = _rows(n, hkv, head_dim, dtype, 1), _rows(n, hkv, head_dim, dtype, 2)
    kc = torch.zeros(layers, blocks, hkv, bs, head_dim, dtype=FP8, device=device)
    vc = torch.zeros_like(kc)
    ops.kv_append(keys.to(device), values.to(device), kc, vc, slots.to(device), 1,
                  k_scale=scales[0], v_scale=scales[1])
    torch.cuda.synchronize()
    ek = torch.zeros(kc.shape, dtype=FP8)
    ev = torch.zeros_like(ek)
    kvslots.kv_append(paged.quantize_e4m3(keys, scales[0]), paged.quantize_e4m3(values, scales[1]),
                      ek, ev, slots, 1)
    assert torch.equal(kc.cpu().view(torch.uint8), ek.view(torch.uint8))
    assert torch.equal(vc.cpu().view(torch.uint8), ev.view(torch.uint8))


def test_fp8_decode_of_every_code(device) -> None:
    """All 256 codes through the gather's decoder (scale 1, fp32 out) equal torch's table."""

    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    pool = codes.view(FP8).view(1, 1, 1, 16, 16).to(device)
    table = torch.zeros(1, 1, dtype=torch.int32, device=device)
    lens = torch.tensor([16], dtype=torch.int32, device=device)
    cu = torch.tensor([0, 16], dtype=torch.int32, device=device)
    k = torch.empty(16, 1, 16, dtype=torch.float32, device=device)
    v = torch.empty_like(k)
    ops.paged_gather(pool, pool, table, lens, cu, 0, 16, k, v)
    torch.cuda.synchronize()
    _same_bits(k.cpu().view(-1), codes.view(FP8).float())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [128, 24])
def test_fp8_gather_bit_exact(device, dtype, head_dim) -> None:
    """Decoding gather into fp32/bf16/fp16 equals the oracle's decode of the C gather.
    The scales put fp16 outputs in the subnormal range (K, 2^-12) and past the largest
    finite fp16 (V, 600: codes above 109 overflow to infinity)."""

    blocks, hkv, bs = 20, 2, 16
    g = torch.Generator().manual_seed(3)
    codes = torch.randint(0, 256, (1, blocks, hkv, bs, head_dim), generator=g, dtype=torch.int32)
    kc = codes.to(torch.uint8).view(FP8)
    vc = torch.flip(kc.view(torch.uint8), dims=[4]).view(FP8).contiguous()
    contexts = [1, 17, 60, 33]
    tables = torch.randperm(blocks, generator=g)[:16].view(4, 4).to(torch.int32)
    lens = torch.tensor(contexts, dtype=torch.int32)
    cu = torch.zeros(5, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0)
    total = int(cu[-1])
    k = torch.empty(total, hkv, head_dim, dtype=dtype, device=device)
    v = torch.empty_like(k)
    ops.paged_gather(kc.to(device), vc.to(device), tables.to(device), lens.to(device),
                     cu.to(device), 0, max(contexts), k, v, k_scale=2.0 ** -12, v_scale=600.0)
    torch.cuda.synchronize()
    ek, ev = kvslots.paged_gather(kc, vc, tables, lens, 0)
    _same_bits(k.cpu(), paged.dequantize_e4m3(ek, 2.0 ** -12, dtype))
    _same_bits(v.cpu(), paged.dequantize_e4m3(ev, 600.0, dtype))


def _decoded(batch):
    """CPU fp32 pools holding the decoded values of the batch's fp8 pools."""

    return (paged.dequantize_e4m3(batch.key_cache.cpu(), batch.k_scale, torch.float32),
            paged.dequantize_e4m3(batch.value_cache.cpu(), batch.v_scale, torch.float32))


def _decode_expected(batch):
    kc, vc = _decoded(batch)
    return paged.decode_batch(batch.query.cpu(), kc, vc, batch.block_tables.cpu(),
                              batch.seq_lens.cpu(), 0, torch.float32)


def _prefill_expected(batch):
    kc, vc = _decoded(batch)
    return paged.prefill_batch(batch.query.cpu(), kc, vc, batch.block_tables.cpu(),
                               batch.seq_lens.cpu(), batch.cu_seqlens_q.cpu(), 0, torch.float32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(("hq", "hkv", "dh"), [(32, 8, 128), (32, 4, 64), (8, 2, 64),
                                               (16, 1, 128), (4, 2, 16)])
@pytest.mark.parametrize("scales", [(1.0, 1.0), (0.05, 3.0)])
def test_fp8_decode_matches_decoded_pool_oracle(device, dtype, hq, hkv, dh, scales) -> None:
    contexts = [1, 15, 16, 17, 100, 513, 1300]
    batch = workloads.paged_batch(contexts, [1] * len(contexts), num_q_heads=hq,
                                  num_kv_heads=hkv, head_dim=dh, block_size=16, dtype=dtype,
                                  device=device, seed=hq + dh, kv_dtype=FP8,
                                  k_scale=scales[0], v_scale=scales[1])
    out = ops.paged_attention_decode(
        batch.query, batch.key_cache, batch.value_cache, batch.block_tables, batch.seq_lens,
        layer_index=0, max_seq_len=batch.max_seq_len, k_scale=batch.k_scale,
        v_scale=batch.v_scale)
    torch.cuda.synchronize()
    assert_close(out.cpu(), _decode_expected(batch), **TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("pages_per_split", [1, 3, 64])
def test_fp8_decode_split_k(device, dtype, pages_per_split) -> None:
    """Split partials carry the V scale into the merge."""

    contexts = [5, 160, 2049, 700]
    batch = workloads.paged_batch(contexts, [1] * 4, num_q_heads=32, num_kv_heads=8,
                                  head_dim=128, block_size=16, dtype=dtype, device=device,
                                  seed=pages_per_split, kv_dtype=FP8, k_scale=0.5, v_scale=2.0)
    out = ops.paged_attention_decode(
        batch.query, batch.key_cache, batch.value_cache, batch.block_tables, batch.seq_lens,
        layer_index=0, max_seq_len=batch.max_seq_len, pages_per_split=pages_per_split,
        k_scale=batch.k_scale, v_scale=batch.v_scale)
    torch.cuda.synchronize()
    assert_close(out.cpu(), _decode_expected(batch), **TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(("hq", "hkv", "dh", "bs"), [(32, 8, 128, 16), (8, 2, 64, 32),
                                                     (4, 4, 16, 5)])
def test_fp8_prefill_matches_decoded_pool_oracle(device, dtype, hq, hkv, dh, bs) -> None:
    """bf16/fp16 at Dh 64/128 with block sizes 16 and 32: pages decoded into the scratch
    pool, then the MFMA kernel; the rest (fp32, Dh 16, block size 5): the VALU kernel on
    the fp8 pool."""
    contexts = [7, 64, 300, 33]
    query_lens = [7, 20, 128, 1]
    batch = workloads.paged_batch(contexts, query_lens, num_q_heads=hq, num_kv_heads=hkv,
                                  head_dim=dh, block_size=bs, dtype=dtype, device=device,
                                  seed=bs, kv_dtype=FP8, k_scale=0.25, v_scale=1.5)
    out = ops.paged_attention_prefill(
        batch.query, batch.key_cache, batch.value_cache, batch.block_tables, batch.seq_lens,
        batch.cu_seqlens_q, layer_index=0, max_query_len=batch.max_query_len,
        max_seq_len=batch.max_seq_len, k_scale=batch.k_scale, v_scale=batch.v_scale)
    torch.cuda.synchronize()
    assert_close(out.cpu(), _prefill_expected(batch), **TOL[dtype])


def test_fp8_storage_round_trip_and_scale_checks(device) -> None:
    storage = PagedKVStorage(num_layers=2, num_blocks=4, num_key_value_heads=2, block_size=4,
                             head_dim=32, device=device, dtype=torch.bfloat16, kv_dtype=FP8,
                             k_scale=0.5, v_scale=4.0)
    assert storage.key_storage.dtype == FP8 and storage.dtype == torch.bfloat16
    g = torch.Generator().manual_seed(11)
    keys = torch.randn(2, 32, generator=g).to(torch.bfloat16)
    values = torch.randn(2, 32, generator=g).to(torch.bfloat16)
    storage.write_token(layer_index=1, block_id=3, offset=2, keys=keys.to(device),
                        values=values.to(device))
    k, v = storage.read_token(layer_index=1, block_id=3, offset=2)
    torch.cuda.synchronize()
    assert k.dtype == torch.bfloat16
    _same_bits(k.cpu(), paged.dequantize_e4m3(paged.quantize_e4m3(keys, 0.5), 0.5, torch.bfloat16))
    _same_bits(v.cpu(), paged.dequantize_e4m3(paged.quantize_e4m3(values, 4.0), 4.0,
                                              torch.bfloat16))
    with pytest.raises(ValueError):
        PagedKVStorage(num_layers=1, num_blocks=1, num_key_value_heads=1, block_size=1,
                       head_dim=8, device=device, dtype=torch.bfloat16, k_scale=2.0)
    with pytest.raises(ValueError):
        PagedKVStorage(num_layers=1, num_blocks=1, num_key_value_heads=1, block_size=1,
                       head_dim=8, device=device, dtype=torch.bfloat16, kv_dtype=FP8,
                       v_scale=0.0)
    with pytest.raises(ValueError):
        ops.kv_append(keys.view(1, 2, 32).to(device), values.view(1, 2, 32).to(device),
                      torch.empty(1, 1, 2, 4, 32, dtype=torch.bfloat16, device=device),
                      torch.empty(1, 1, 2, 4, 32, dtype=torch.bfloat16, device=device),
                      torch.zeros(1, dtype=torch.int64, device=device), 0, k_scale=2.0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fp8_nan_codes_in_unwritten_rows_are_never_read(device, dtype) -> None:
    """Tail rows of the last pages hold the e4m3 NaN code: decode (MFMA and split) and
    prefill stay finite and equal the decoded-pool oracle on the written rows."""

    contexts, query_lens = [1, 17, 35, 100], [1, 5, 35, 16]
    batch = workloads.paged_batch(contexts, query_lens, num_q_heads=32, num_kv_heads=8,
                                  head_dim=128, block_size=16, dtype=dtype, device=device,
                                  seed=5, kv_dtype=FP8, k_scale=0.5, v_scale=2.0)
    tables = batch.block_tables.cpu()
    valid = torch.zeros(batch.key_cache.shape[1], 16, dtype=torch.bool)
    for b, ctx in enumerate(contexts):
        for pos in range(ctx):
            valid[int(tables[b, pos // 16]), pos % 16] = True
    mask = valid.view(1, -1, 1, 16, 1).to(device)
    for pool in (batch.key_cache, batch.value_cache):
        raw = pool.view(torch.uint8)
        raw.copy_(torch.where(mask, raw, torch.tensor(0x7F, dtype=torch.uint8, device=device)))
    q_rows = torch.tensor([sum(query_lens[: b + 1]) - 1 for b in range(4)], device=device)
    outs = [ops.paged_attention_decode(
        batch.query[q_rows], batch.key_cache, batch.value_cache, batch.block_tables,
        batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len, pages_per_split=pps,
        k_scale=batch.k_scale, v_scale=batch.v_scale) for pps in (0, 1)]
    prefill = ops.paged_attention_prefill(
        batch.query, batch.key_cache, batch.value_cache, batch.block_tables, batch.seq_lens,
        batch.cu_seqlens_q, layer_index=0, max_query_len=batch.max_query_len,
        max_seq_len=batch.max_seq_len, k_scale=batch.k_scale, v_scale=batch.v_scale)
    torch.cuda.synchronize()
    kc, vc = _decoded(batch)
    q = batch.query.cpu()
    expected = paged.decode_batch(q[q_rows.cpu()], kc, vc, batch.block_tables.cpu(),
                                  batch.seq_lens.cpu(), 0, torch.float32)
    for out in outs:
        assert torch.isfinite(out.float()).all()
        assert_close(out.cpu(), expected, **TOL[dtype])
    assert torch.isfinite(prefill.float()).all()
    assert_close(prefill.cpu(), _prefill_expected(batch), **TOL[dtype])
