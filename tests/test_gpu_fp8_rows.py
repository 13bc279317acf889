"""fp8 (OCP e4m3) K/V pools with one scale per pool row, on the GPU against the oracle.

Each pool row (one token of one KV head) is stored as e4m3(clamp(x / s, -448, 448))
with s = max|row| / 448 (1 when that is 0, NaN or infinite), s kept in a float32
[L, NB, Hkv, BS] array beside the pool. Appends (plain and with RoPE fused in) and
the decoding gather are bit-exact against the oracle (oracle/e4m3.c
oracle_e4m3_encode_rows, scattered by the C slot restatement; dequantize_e4m3_rows).
Attention over such pools is the attention of the decoded pools: compared with the
oracle's fp32 arithmetic on the decoded values, fp32 within rtol 1e-5 / atol 1e-6 and
bf16/fp16 within 2e-2 absolute (the tolerances of pools in the model dtype).
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
    """Rows over many magnitudes, plus whole rows that exercise the scale rule: all zero,
    one NaN, one infinity, the largest magnitude negative, subnormal and huge values."""

    g = torch.Generator().manual_seed(seed)
    magnitude = 2.0 ** torch.randint(-20, 20, (n, hkv, 1), generator=g).float()
    x = torch.randn(n, hkv, dh, generator=g) * magnitude
    x[0, 0] = 0.0
    x[1, 0, 3] = float("nan")
    x[2, 0, 5] = float("inf")
    x[3, 0] = -x[3, 0].abs()
    x[3, 0, 1] = -1e4
    x[4, 0] = torch.randn(dh, generator=g) * 1e-40   # fp32 / bf16 subnormals
    x[5, 0] = torch.randn(dh, generator=g) * 1e30
    x[6, 0] = 448.0                                   # every element equal
    return x.to(dtype)


def _same_bits(a: torch.Tensor, b: torch.Tensor) -> None:
    assert a.shape == b.shape and a.dtype == b.dtype
    nan_a, nan_b = torch.isnan(a.float()), torch.isnan(b.float())
    assert torch.equal(nan_a, nan_b)
    assert torch.equal(a[~nan_a], b[~nan_b])


def _expected_append(keys, values, slots, shape, layer):
    """Oracle pools and scale arrays after appending rows (N, Hkv, Dh) at slots."""

    ek = torch.zeros(shape, dtype=torch.uint8)
    ev = torch.zeros_like(ek)
    eks = torch.ones((*shape[:4], 1), dtype=torch.float32)
    evs = torch.ones_like(eks)
    kcodes, kscales = kvslots.e4m3_encode_rows(keys)
    vcodes, vscales = kvslots.e4m3_encode_rows(values)
    kvslots.kv_append(kcodes, vcodes, ek, ev, slots, layer)
    kvslots.kv_append(kscales.unsqueeze(-1), vscales.unsqueeze(-1), eks, evs, slots, layer)
    return ek, ev, eks.squeeze(-1), evs.squeeze(-1)


def _pools(device, shape):
    kc = torch.zeros(shape, dtype=FP8, device=device)
    ks = torch.ones(shape[:4], dtype=torch.float32, device=device)
    return kc, torch.zeros_like(kc), ks, torch.ones_like(ks)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [128, 64, 24, 256])
def test_fp8_rows_append_bit_exact(device, dtype, head_dim) -> None:
    """Codes and scales written by the row-scaled append equal the C encoder's, scattered
    by the C slot restatement, byte for byte; a padding slot (-1) writes nothing."""

    layers, blocks, hkv, bs, n = 2, 12, 4, 16, 70
    g = torch.Generator().manual_seed(head_dim)
    slots = torch.randperm(blocks * bs, generator=g)[:n].to(torch.int64)
    slots[9] = -1
    keys, values = _rows(n, hkv, head_dim, dtype, 1), _rows(n, hkv, head_dim, dtype, 2)
    shape = (layers, blocks, hkv, bs, head_dim)
    kc, vc, ks, vs = _pools(device, shape)
    ops.kv_append(keys.to(device), values.to(device), kc, vc, slots.to(device), 1,
                  k_scales=ks, v_scales=vs)
    torch.cuda.synchronize()
    ek, ev, eks, evs = _expected_append(keys, values, slots, shape, 1)
    assert torch.equal(kc.cpu().view(torch.uint8), ek)
    assert torch.equal(vc.cpu().view(torch.uint8), ev)
    assert torch.equal(ks.cpu(), eks)
    assert torch.equal(vs.cpu(), evs)


def test_fp8_rows_scale_rule_known_answers(device) -> None:
    """Closed forms on the GPU's output: a row's largest magnitude becomes code 448 (0x7E
    or 0xFE), an all-zero row keeps scale 1 and zero codes, a NaN row scale 1 with its
    NaN kept, a row with an infinity scale 1 and saturated codes."""

    hkv, dh = 1, 64
    rows = torch.randn(4, hkv, dh, generator=torch.Generator().manual_seed(5)) * 3.0
    rows[1] = 0.0
    rows[2, 0, 7] = float("nan")
    rows[3, 0, 9] = -float("inf")
    kc, vc, ks, vs = _pools(device, (1, 1, hkv, 16, dh))
    slots = torch.arange(4, dtype=torch.int64, device=device)
    ops.kv_append(rows.to(device), rows.to(device), kc, vc, slots, 0, k_scales=ks, v_scales=vs)
    torch.cuda.synchronize()
    codes, scales = kc.cpu().view(torch.uint8)[0, 0, 0], ks.cpu()[0, 0, 0]
    top = int(rows[0, 0].abs().argmax())
    assert int(codes[0, top]) & 0x7F == 0x7E
    assert torch.equal(scales[0], rows[0, 0].abs().max() / 448.0)  # fp32 quotient
    assert float(scales[1]) == 1.0 and int(codes[1].max()) == 0
    assert float(scales[2]) == 1.0 and int(codes[2, 7]) & 0x7F == 0x7F
    assert float(scales[3]) == 1.0 and int(codes[3, 9]) == 0xFE


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [128, 24])
def test_fp8_rows_gather_bit_exact(device, dtype, head_dim) -> None:
    """Decoding gather: float(code) * the row's scale, rounded once, equals the oracle's
    decode of the C gather of codes and scales."""

    blocks, hkv, bs = 20, 2, 16
    g = torch.Generator().manual_seed(3)
    codes = torch.randint(0, 256, (1, blocks, hkv, bs, head_dim), generator=g,
                          dtype=torch.int32).to(torch.uint8)
    kc = codes.view(FP8)
    vc = torch.flip(codes, dims=[4]).contiguous().view(FP8)
    ks = torch.exp(torch.randn(1, blocks, hkv, bs, generator=g) * 4.0)
    vs = torch.exp(torch.randn(1, blocks, hkv, bs, generator=g) * 4.0)
    contexts = [1, 17, 60, 33]
    tables = torch.randperm(blocks, generator=g)[:16].view(4, 4).to(torch.int32)
    lens = torch.tensor(contexts, dtype=torch.int32)
    cu = torch.zeros(5, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0)
    total = int(cu[-1])
    k = torch.empty(total, hkv, head_dim, dtype=dtype, device=device)
    v = torch.empty_like(k)
    ops.paged_gather(kc.to(device), vc.to(device), tables.to(device), lens.to(device),
                     cu.to(device), 0, max(contexts), k, v, k_scales=ks.to(device),
                     v_scales=vs.to(device))
    torch.cuda.synchronize()
    ek, ev = kvslots.paged_gather(kc, vc, tables, lens, 0)
    eks, evs = kvslots.paged_gather(ks.unsqueeze(-1), vs.unsqueeze(-1), tables, lens, 0)
    _same_bits(k.cpu(), paged.dequantize_e4m3_rows(ek, eks.squeeze(-1), dtype))
    _same_bits(v.cpu(), paged.dequantize_e4m3_rows(ev, evs.squeeze(-1), dtype))


def _decoded(batch):
    """CPU fp32 pools holding the decoded values of the batch's row-scaled fp8 pools."""

    return (paged.dequantize_e4m3_rows(batch.key_cache.cpu(), batch.k_scales.cpu(),
                                       torch.float32),
            paged.dequantize_e4m3_rows(batch.value_cache.cpu(), batch.v_scales.cpu(),
                                       torch.float32))


def _decode_expected(batch, query=None):
    kc, vc = _decoded(batch)
    q = batch.query.cpu() if query is None else query.cpu()
    return paged.decode_batch(q, kc, vc, batch.block_tables.cpu(), batch.seq_lens.cpu(), 0,
                              torch.float32)


def _prefill_expected(batch):
    kc, vc = _decoded(batch)
    return paged.prefill_batch(batch.query.cpu(), kc, vc, batch.block_tables.cpu(),
                               batch.seq_lens.cpu(), batch.cu_seqlens_q.cpu(), 0, torch.float32)


def _batch(device, contexts, query_lens, hq, hkv, dh, dtype, seed, bs=16):
    batch = workloads.paged_batch(contexts, query_lens, num_q_heads=hq, num_kv_heads=hkv,
                                  head_dim=dh, block_size=bs, dtype=dtype, device=device,
                                  seed=seed, kv_dtype=FP8, scale_granularity="row")
    assert batch.k_scales is not None and batch.k_scales.shape == batch.key_cache.shape[:4]
    return batch


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(("hq", "hkv", "dh"), [(32, 8, 128), (32, 4, 64), (8, 2, 64),
                                               (16, 1, 128), (4, 2, 16)])
def test_fp8_rows_decode_matches_decoded_pool_oracle(device, dtype, hq, hkv, dh) -> None:
    """bf16/fp16 at Dh 64/128 run the MFMA decode kernel, the rest the VALU kernel."""

    contexts = [1, 15, 16, 17, 100, 513, 1300]
    batch = _batch(device, contexts, [1] * len(contexts), hq, hkv, dh, dtype, hq + dh)
    out = ops.paged_attention_decode(
        batch.query, batch.key_cache, batch.value_cache, batch.block_tables, batch.seq_lens,
        layer_index=0, max_seq_len=batch.max_seq_len, **batch.scale_kwargs)
    torch.cuda.synchronize()
    assert_close(out.cpu(), _decode_expected(batch), **TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("pages_per_split", [1, 3, 64])
def test_fp8_rows_decode_split_k(device, dtype, pages_per_split) -> None:
    contexts = [5, 160, 2049, 700]
    batch = _batch(device, contexts, [1] * 4, 32, 8, 128, dtype, pages_per_split)
    order = ops.longest_first(contexts, device)
    out = ops.paged_attention_decode(
        batch.query, batch.key_cache, batch.value_cache, batch.block_tables, batch.seq_lens,
        layer_index=0, max_seq_len=batch.max_seq_len, pages_per_split=pages_per_split,
        seq_order=order, **batch.scale_kwargs)
    torch.cuda.synchronize()
    assert_close(out.cpu(), _decode_expected(batch), **TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(("hq", "hkv", "dh", "bs"), [(32, 8, 128, 16), (8, 2, 64, 32),
                                                     (4, 4, 16, 5)])
def test_fp8_rows_prefill_matches_decoded_pool_oracle(device, dtype, hq, hkv, dh, bs) -> None:
    """bf16/fp16 at Dh 64/128: pages decoded with their row scales into the scratch pool,
    then the MFMA kernel; the rest: the VALU kernel on the fp8 pool and its scales."""

    contexts = [7, 64, 300, 33]
    query_lens = [7, 20, 128, 1]
    batch = _batch(device, contexts, query_lens, hq, hkv, dh, dtype, bs, bs=bs)
    out = ops.paged_attention_prefill(
        batch.query, batch.key_cache, batch.value_cache, batch.block_tables, batch.seq_lens,
        batch.cu_seqlens_q, layer_index=0, max_query_len=batch.max_query_len,
        max_seq_len=batch.max_seq_len, seq_order=ops.longest_first(contexts, device),
        **batch.scale_kwargs)
    torch.cuda.synchronize()
    assert_close(out.cpu(), _prefill_expected(batch), **TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fp8_rows_unwritten_rows_are_never_read(device, dtype) -> None:
    """Rows past each sequence's keys hold the e4m3 NaN code and a NaN scale: decode
    (one launch and split) and prefill stay finite and equal the decoded-pool oracle."""

    contexts, query_lens = [1, 17, 35, 100], [1, 5, 35, 16]
    batch = _batch(device, contexts, query_lens, 32, 8, 128, dtype, 5)
    tables = batch.block_tables.cpu()
    valid = torch.zeros(batch.key_cache.shape[1], 16, dtype=torch.bool)
    for b, ctx in enumerate(contexts):
        for pos in range(ctx):
            valid[int(tables[b, pos // 16]), pos % 16] = True
    mask = valid.view(1, -1, 1, 16).to(device)
    for pool, scales in ((batch.key_cache, batch.k_scales), (batch.value_cache, batch.v_scales)):
        raw = pool.view(torch.uint8)
        raw.copy_(torch.where(mask.unsqueeze(-1), raw,
                              torch.tensor(0x7F, dtype=torch.uint8, device=device)))
        scales.copy_(torch.where(mask, scales, torch.tensor(float("nan"), device=device)))
    q_rows = torch.tensor([sum(query_lens[: b + 1]) - 1 for b in range(4)], device=device)
    outs = [ops.paged_attention_decode(
        batch.query[q_rows], batch.key_cache, batch.value_cache, batch.block_tables,
        batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len, pages_per_split=pps,
        **batch.scale_kwargs) for pps in (0, 1)]
    prefill = ops.paged_attention_prefill(
        batch.query, batch.key_cache, batch.value_cache, batch.block_tables, batch.seq_lens,
        batch.cu_seqlens_q, layer_index=0, max_query_len=batch.max_query_len,
        max_seq_len=batch.max_seq_len, **batch.scale_kwargs)
    torch.cuda.synchronize()
    expected = _decode_expected(batch, batch.query[q_rows])
    for out in outs:
        assert torch.isfinite(out.float()).all()
        assert_close(out.cpu(), expected, **TOL[dtype])
    assert torch.isfinite(prefill.float()).all()
    assert_close(prefill.cpu(), _prefill_expected(batch), **TOL[dtype])


def _step_inputs(device, dtype, n, hq, hkv, dh, seed):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(n, hq, dh, generator=g) * 2.0).to(dtype).to(device)
    k = (torch.randn(n, hkv, dh, generator=g) * 3.0).to(dtype).to(device)
    v = torch.randn(n, hkv, dh, generator=g).to(dtype).to(device)
    positions = torch.randint(0, 300, (n,), generator=g).to(device)
    return q, k, v, positions


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("dh", [128, 64])
def test_fp8_rows_rope_kv_append_equals_rope_then_append(device, dtype, dh) -> None:
    """The fused rotation + row-scaled append equals rope() followed by kv_append() of the
    rotated keys, bit for bit (query out, key_out, codes and scales)."""

    n, hq, hkv, blocks, bs = 37, 8, 2, 8, 16
    table = ops.RotaryTable(dh, theta=10_000.0, max_position=512, dtype=dtype, device=device)
    q, k, v, positions = _step_inputs(device, dtype, n, hq, hkv, dh, dh)
    slots = torch.randperm(blocks * bs, generator=torch.Generator().manual_seed(1))[:n]
    slots = slots.to(device)
    shape = (2, blocks, hkv, bs, dh)
    kc, vc, ks, vs = _pools(device, shape)
    qf, kf = q.clone(), torch.empty_like(k)
    ops.rope_kv_append(qf, k, v, positions, table, kc, vc, slots, 1, key_out=kf,
                       k_scales=ks, v_scales=vs)
    kc2, vc2, ks2, vs2 = _pools(device, shape)
    q2, k2 = ops.rope(q.unsqueeze(0).transpose(1, 2), k.unsqueeze(0).transpose(1, 2),
                      positions, table)
    q2, k2 = q2.transpose(1, 2)[0], k2.transpose(1, 2)[0]
    ops.kv_append(k2, v, kc2, vc2, slots, 1, k_scales=ks2, v_scales=vs2)
    torch.cuda.synchronize()
    assert torch.equal(qf, q2) and torch.equal(kf, k2)
    assert torch.equal(kc.view(torch.uint8), kc2.view(torch.uint8))
    assert torch.equal(vc.view(torch.uint8), vc2.view(torch.uint8))
    assert torch.equal(ks, ks2) and torch.equal(vs, vs2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_fp8_rows_fused_decode_step_equals_two_calls(device, dtype) -> None:
    """rope_append_paged_decode over row-scaled pools equals rope_kv_append() followed by
    paged_attention_decode(), bit for bit, and leaves the same pools and scales."""

    contexts = [3, 16, 17, 250, 1000]
    batch = _batch(device, contexts, [1] * len(contexts), 32, 8, 128, dtype, 9)
    hkv, dh = 8, 128
    table = ops.RotaryTable(dh, theta=500_000.0, max_position=2048, dtype=dtype, device=device)
    _, k, v, _ = _step_inputs(device, dtype, len(contexts), 32, hkv, dh, 4)
    positions = (batch.seq_lens - 1).to(torch.int64)
    tables = batch.block_tables
    last = positions // 16
    slots = (tables.gather(1, last.view(-1, 1)).view(-1).to(torch.int64) * 16 + positions % 16)
    pools = [t.clone() for t in (batch.key_cache, batch.value_cache, batch.k_scales,
                                 batch.v_scales)]
    fused = ops.rope_append_paged_decode(
        batch.query, k, v, positions, table, pools[0], pools[1], slots, tables, batch.seq_lens,
        layer_index=0, max_seq_len=batch.max_seq_len, k_scales=pools[2], v_scales=pools[3])
    q2 = batch.query.clone()
    ops.rope_kv_append(q2, k, v, positions, table, batch.key_cache, batch.value_cache, slots, 0,
                       **batch.scale_kwargs)
    two = ops.paged_attention_decode(q2, batch.key_cache, batch.value_cache, tables,
                                     batch.seq_lens, layer_index=0,
                                     max_seq_len=batch.max_seq_len, **batch.scale_kwargs)
    torch.cuda.synchronize()
    assert torch.equal(fused, two)
    assert torch.equal(pools[0].view(torch.uint8), batch.key_cache.view(torch.uint8))
    assert torch.equal(pools[1].view(torch.uint8), batch.value_cache.view(torch.uint8))
    assert torch.equal(pools[2], batch.k_scales) and torch.equal(pools[3], batch.v_scales)
    assert_close(two.cpu(), _decode_expected(batch, q2), **TOL[dtype])


def test_fp8_rows_storage_round_trip_and_checks(device) -> None:
    storage = PagedKVStorage(num_layers=2, num_blocks=4, num_key_value_heads=2, block_size=4,
                             head_dim=32, device=device, dtype=torch.bfloat16, kv_dtype=FP8,
                             scale_granularity="row")
    assert storage.key_scales.shape == (2, 4, 2, 4) and storage.key_scales.dtype == torch.float32
    assert set(storage.scales) == {"k_scales", "v_scales"}
    g = torch.Generator().manual_seed(11)
    keys = (torch.randn(2, 32, generator=g) * torch.tensor([[1e-3], [50.0]])).to(torch.bfloat16)
    values = torch.randn(2, 32, generator=g).to(torch.bfloat16)
    storage.write_token(layer_index=1, block_id=3, offset=2, keys=keys.to(device),
                        values=values.to(device))
    k, v = storage.read_token(layer_index=1, block_id=3, offset=2)
    torch.cuda.synchronize()
    for got, rows in ((k, keys), (v, values)):
        assert got.dtype == torch.bfloat16
        _same_bits(got.cpu(), paged.dequantize_e4m3_rows(*paged.quantize_e4m3_rows(rows),
                                                         torch.bfloat16))
    for bad in (dict(kv_dtype=None), dict(kv_dtype=FP8, k_scale=2.0),
                dict(kv_dtype=FP8, scale_granularity="block")):
        granularity = bad.pop("scale_granularity", "row")
        with pytest.raises(ValueError):
            PagedKVStorage(num_layers=1, num_blocks=1, num_key_value_heads=1, block_size=1,
                           head_dim=8, device=device, dtype=torch.bfloat16,
                           scale_granularity=granularity, **bad)
