"""A decode step's RoPE + KV append + attention in one call (tks_rope_append_paged_decode)
against the two calls it replaces, tks_rope_kv_append then tks_paged_attention_decode,
on the same inputs: the pools after the call and the outputs are bit-identical, the
query is left as it was. Covered: the fused MFMA launch (bf16 / fp16, Dh 64 and 128,
several GQA groups, with and without key splits, partly filled and exactly full last
pages, a new token that opens a page), the two-launch path the entry takes elsewhere
(fp32, Dh 32 and block size 8 on the generic kernel, new rows not in 16-byte chunks), a
negative slot (nothing appended) and an empty
sequence (its row is appended, its output is zero). Over fp8 (e4m3) pools the same
against tks_rope_kv_append_fp8 then tks_paged_attention_decode_fp8, and the fp8
RoPE + append launch against tks_rope then the quantizing tks_kv_append_fp8. Over fp8
pools with one scale per pool row, the fused launch against the per-row
tks_rope_kv_append_fp8_rows then the decode: outputs, codes and scales bit-identical.
"""

import pytest
import torch

from tokserve_amd import workloads
from tokserve_amd.kernels import ops

pytestmark = pytest.mark.gpu

FP8 = torch.float8_e4m3fn

CASES = [
    # dtype, Hq, Hkv, Dh, contexts
    (torch.bfloat16, 32, 4, 64, [64 + 37 * i for i in range(24)]),
    (torch.bfloat16, 32, 8, 128, [1, 16, 17, 31, 32, 33, 200, 1025, 4096, 4097]),
    (torch.float16, 16, 8, 128, [5, 48, 49, 700]),
    (torch.bfloat16, 16, 16, 128, [300, 17, 1]),
    (torch.bfloat16, 32, 4, 128, [90, 900]),       # G 8 at Dh 128
    (torch.float32, 8, 2, 64, [16, 17, 513, 100]),  # fp32: generic kernel, two launches
    (torch.float32, 16, 4, 128, [1, 64, 65, 300]),  # fp32, Dh 128: likewise
    (torch.bfloat16, 8, 2, 32, [17, 40, 3, 64]),    # Dh 32: likewise
]


@pytest.mark.parametrize("dh", [64, 128])
@pytest.mark.parametrize("group", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("dtype, kv_dtype", [(torch.bfloat16, None), (torch.float16, FP8)])
def test_fused_decode_step_every_mfma_group(device, dh, group, dtype, kv_dtype) -> None:
    hkv = 2
    contexts = [1, 15, 16, 17, 130, 700]
    batch, query, key, value, positions, slots, table = _inputs(
        device, dtype, hkv * group, hkv, dh, contexts, seed=70 + group + dh, kv_dtype=kv_dtype)
    kw = dict(k_scale=0.75, v_scale=1.25) if kv_dtype is not None else {}
    kc_ref, vc_ref = batch.key_cache.clone(), batch.value_cache.clone()
    q_ref = query.clone()
    ops.rope_kv_append(q_ref, key, value, positions, table, kc_ref, vc_ref, slots, 0, **kw)
    expected = ops.paged_attention_decode(q_ref, kc_ref, vc_ref, batch.block_tables,
                                          batch.seq_lens, layer_index=0,
                                          max_seq_len=batch.max_seq_len, **kw)
    actual = ops.rope_append_paged_decode(
        query, key, value, positions, table, batch.key_cache, batch.value_cache, slots,
        batch.block_tables, batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len, **kw)
    torch.cuda.synchronize()
    assert torch.equal(actual.cpu().view(torch.int16), expected.cpu().view(torch.int16))
    assert torch.equal(batch.key_cache.view(torch.uint8), kc_ref.view(torch.uint8))
    assert torch.equal(batch.value_cache.view(torch.uint8), vc_ref.view(torch.uint8))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("kv_dtype", [None, torch.float8_e4m3fn])
def test_fused_decode_step_block_size_8_takes_two_launches(device, dtype, kv_dtype) -> None:
    hq, hkv, dh, contexts = 8, 2, 64, [7, 8, 9, 300, 1]
    batch, query, key, value, positions, slots, table = _inputs(
        device, dtype, hq, hkv, dh, contexts, seed=51, kv_dtype=kv_dtype, block_size=8)
    kw = dict(k_scale=0.5, v_scale=2.0) if kv_dtype is not None else {}
    kc_ref, vc_ref = batch.key_cache.clone(), batch.value_cache.clone()
    q_ref = query.clone()
    ops.rope_kv_append(q_ref, key, value, positions, table, kc_ref, vc_ref, slots, 0, **kw)
    for pages_per_split in (0, 3):
        kc, vc = batch.key_cache.clone(), batch.value_cache.clone()
        expected = ops.paged_attention_decode(
            q_ref, kc_ref, vc_ref, batch.block_tables, batch.seq_lens, layer_index=0,
            max_seq_len=batch.max_seq_len, pages_per_split=pages_per_split, **kw)
        actual = ops.rope_append_paged_decode(
            query, key, value, positions, table, kc, vc, slots, batch.block_tables,
            batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len,
            pages_per_split=pages_per_split, **kw)
        torch.cuda.synchronize()
        bits = torch.int32 if dtype == torch.float32 else torch.int16
        assert torch.equal(actual.cpu().view(bits), expected.cpu().view(bits))
        assert torch.equal(kc.view(torch.uint8), kc_ref.view(torch.uint8))
        assert torch.equal(vc.view(torch.uint8), vc_ref.view(torch.uint8))


def _inputs(device, dtype, hq, hkv, dh, contexts, seed, kv_dtype=None, scales=(1.0, 1.0),
            block_size=16):
    batch = workloads.paged_batch(contexts, [1] * len(contexts), num_q_heads=hq,
                                  num_kv_heads=hkv, head_dim=dh, block_size=block_size,
                                  dtype=dtype, device=device, seed=seed, kv_dtype=kv_dtype,
                                  k_scale=scales[0], v_scale=scales[1])
    b = len(contexts)
    g = torch.Generator().manual_seed(seed + 3)
    qkv = torch.randn(b, (hq + 2 * hkv) * dh, generator=g).to(dtype).to(device)
    query = qkv[:, : hq * dh].view(b, hq, dh)
    key = qkv[:, hq * dh : (hq + hkv) * dh].view(b, hkv, dh)
    value = qkv[:, (hq + hkv) * dh :].view(b, hkv, dh)
    lens = torch.tensor(contexts, dtype=torch.int64)
    positions = (lens - 1).to(device)
    tables = batch.block_tables.to(torch.int64).cpu()
    pos = lens - 1
    slots = (tables[torch.arange(b), pos // block_size] * block_size + pos % block_size)
    slots = slots.to(device)
    table = ops.RotaryTable(dh, theta=10_000.0, max_position=8192, dtype=dtype, device=device)
    return batch, query, key, value, positions, slots, table


@pytest.mark.parametrize("case", range(len(CASES)))
@pytest.mark.parametrize("pages_per_split", [0, 2])
def test_fused_decode_step_equals_rope_append_then_decode(device, case, pages_per_split) -> None:
    dtype, hq, hkv, dh, contexts = CASES[case]
    batch, query, key, value, positions, slots, table = _inputs(device, dtype, hq, hkv, dh,
                                                                contexts, seed=case)
    order = ops.longest_first(batch.contexts, device)
    query_before = query.clone()
    kc_ref, vc_ref = batch.key_cache.clone(), batch.value_cache.clone()
    q_ref = query.clone()
    ops.rope_kv_append(q_ref, key, value, positions, table, kc_ref, vc_ref, slots, 0)
    expected = ops.paged_attention_decode(
        q_ref, kc_ref, vc_ref, batch.block_tables, batch.seq_lens, layer_index=0,
        max_seq_len=batch.max_seq_len, pages_per_split=pages_per_split, seq_order=order)

    actual = ops.rope_append_paged_decode(
        query, key, value, positions, table, batch.key_cache, batch.value_cache, slots,
        batch.block_tables, batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len,
        pages_per_split=pages_per_split, seq_order=order)
    torch.cuda.synchronize()
    assert torch.equal(actual.cpu().view(torch.int8 if dtype != torch.float32 else torch.int32),
                       expected.cpu().view(torch.int8 if dtype != torch.float32 else torch.int32))
    assert torch.equal(batch.key_cache, kc_ref) and torch.equal(batch.value_cache, vc_ref)
    assert torch.equal(query, query_before)


def test_fused_decode_step_negative_slot_appends_nothing(device) -> None:
    dtype, hq, hkv, dh, contexts = CASES[0]
    batch, query, key, value, positions, slots, table = _inputs(device, dtype, hq, hkv, dh,
                                                                contexts, seed=11)
    slots[3] = -1
    kc_ref, vc_ref = batch.key_cache.clone(), batch.value_cache.clone()
    q_ref = query.clone()
    ops.rope_kv_append(q_ref, key, value, positions, table, kc_ref, vc_ref, slots, 0)
    expected = ops.paged_attention_decode(q_ref, kc_ref, vc_ref, batch.block_tables,
                                          batch.seq_lens, layer_index=0,
                                          max_seq_len=batch.max_seq_len)
    actual = ops.rope_append_paged_decode(
        query, key, value, positions, table, batch.key_cache, batch.value_cache, slots,
        batch.block_tables, batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len)
    torch.cuda.synchronize()
    assert torch.equal(actual.cpu().view(torch.int16), expected.cpu().view(torch.int16))
    assert torch.equal(batch.key_cache, kc_ref) and torch.equal(batch.value_cache, vc_ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_fused_decode_step_empty_sequence_still_appends(device, dtype) -> None:
    contexts = [0, 40, 17, 0]
    hq, hkv, dh = 16, 4, 128
    batch = workloads.paged_batch(contexts, [1] * 4, num_q_heads=hq, num_kv_heads=hkv,
                                  head_dim=dh, block_size=16, dtype=dtype, device=device,
                                  seed=21, num_blocks=8)
    _, query, key, value, positions, slots, table = _inputs(device, dtype, hq, hkv, dh,
                                                            [1, 40, 17, 1], seed=21)
    tables = batch.block_tables.cpu()
    used = {int(tables[b, p]) for b in (1, 2) for p in range((contexts[b] + 15) // 16)}
    free = [blk for blk in range(8) if blk not in used]
    slots[0], slots[3] = free[0] * 16 + 5, free[1] * 16 + 15
    for b in (1, 2):
        slots[b] = int(tables[b, (contexts[b] - 1) // 16]) * 16 + (contexts[b] - 1) % 16
    positions[0], positions[3] = 0, 7
    kc_ref, vc_ref = batch.key_cache.clone(), batch.value_cache.clone()
    q_ref = query.clone()
    ops.rope_kv_append(q_ref, key, value, positions, table, kc_ref, vc_ref, slots, 0)
    expected = ops.paged_attention_decode(q_ref, kc_ref, vc_ref, batch.block_tables,
                                          batch.seq_lens, layer_index=0,
                                          max_seq_len=batch.max_seq_len)
    actual = ops.rope_append_paged_decode(
        query, key, value, positions, table, batch.key_cache, batch.value_cache, slots,
        batch.block_tables, batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len)
    torch.cuda.synchronize()
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    assert torch.equal(actual.cpu().view(bits), expected.cpu().view(bits))
    assert not actual[0].any() and not actual[3].any()
    assert torch.equal(batch.key_cache, kc_ref) and torch.equal(batch.value_cache, vc_ref)


FP8_CASES = [
    # dtype, Hq, Hkv, Dh, contexts, (k_scale, v_scale)
    (torch.bfloat16, 32, 4, 64, [64 + 37 * i for i in range(24)], (0.5, 0.25)),
    (torch.bfloat16, 32, 8, 128, [1, 16, 17, 31, 32, 33, 200, 1025, 4096, 4097], (1.0, 1.0)),
    (torch.float16, 16, 8, 128, [5, 48, 49, 700], (2.0, 0.75)),
    (torch.bfloat16, 32, 4, 128, [90, 900, 33], (0.125, 4.0)),   # G 8 at Dh 128
    (torch.float32, 8, 2, 64, [16, 17, 513, 100], (0.5, 2.0)),   # fp32: two launches
]


@pytest.mark.parametrize("case", range(len(FP8_CASES)))
@pytest.mark.parametrize("pages_per_split", [0, 2])
def test_fused_decode_step_over_fp8_pools(device, case, pages_per_split) -> None:
    dtype, hq, hkv, dh, contexts, scales = FP8_CASES[case]
    batch, query, key, value, positions, slots, table = _inputs(
        device, dtype, hq, hkv, dh, contexts, seed=40 + case, kv_dtype=FP8, scales=scales)
    kw = dict(k_scale=scales[0], v_scale=scales[1])
    order = ops.longest_first(batch.contexts, device)
    query_before = query.clone()
    kc_ref, vc_ref = batch.key_cache.clone(), batch.value_cache.clone()
    q_ref = query.clone()
    ops.rope_kv_append(q_ref, key, value, positions, table, kc_ref, vc_ref, slots, 0, **kw)
    expected = ops.paged_attention_decode(
        q_ref, kc_ref, vc_ref, batch.block_tables, batch.seq_lens, layer_index=0,
        max_seq_len=batch.max_seq_len, pages_per_split=pages_per_split, seq_order=order, **kw)
    actual = ops.rope_append_paged_decode(
        query, key, value, positions, table, batch.key_cache, batch.value_cache, slots,
        batch.block_tables, batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len,
        pages_per_split=pages_per_split, seq_order=order, **kw)
    torch.cuda.synchronize()
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    assert torch.equal(actual.cpu().view(bits), expected.cpu().view(bits))
    assert torch.equal(batch.key_cache.view(torch.uint8), kc_ref.view(torch.uint8))
    assert torch.equal(batch.value_cache.view(torch.uint8), vc_ref.view(torch.uint8))
    assert torch.equal(query, query_before)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("dh", [64, 128, 40])
def test_rope_kv_append_over_fp8_pools_equals_rope_then_quantizing_append(device, dtype,
                                                                          dh) -> None:
    n, hq, hkv, scales = 37, 8, 2, (0.375, 1.5)
    g = torch.Generator().manual_seed(dh)
    pool_shape = (2, 8, hkv, 16, dh)
    kc = (torch.randn(pool_shape, generator=g) * 3).to(FP8).to(device)
    vc = (torch.randn(pool_shape, generator=g) * 3).to(FP8).to(device)
    q = (torch.randn(n, hq, dh, generator=g) * 4).to(dtype).to(device)
    k = (torch.randn(n, hkv, dh, generator=g) * 4).to(dtype).to(device)
    v = (torch.randn(n, hkv, dh, generator=g) * 4).to(dtype).to(device)
    k[3, 1, 5] = float("nan")
    v[4, 0, 7] = -float("nan")
    k[5, 0, 0] = 1e4                                   # past the e4m3 range after scaling
    pos = torch.randint(0, 500, (n,), generator=g).to(device)
    slots = torch.randperm(8 * 16, generator=g)[:n].to(torch.int64)
    slots[6] = -1
    slots = slots.to(device)
    table = ops.RotaryTable(dh, theta=10_000.0, max_position=512, dtype=dtype, device=device)
    kw = dict(k_scale=scales[0], v_scale=scales[1])

    q_ref, k_ref = q.clone(), k.clone()
    ops.rope(q_ref.transpose(0, 1).unsqueeze(0), k_ref.transpose(0, 1).unsqueeze(0), pos,
             table, query_out=q_ref.transpose(0, 1).unsqueeze(0),
             key_out=k_ref.transpose(0, 1).unsqueeze(0))
    kc_ref, vc_ref = kc.clone(), vc.clone()
    ops.kv_append(k_ref, v, kc_ref, vc_ref, slots, 1, **kw)

    q_out = torch.empty_like(q)
    k_out = torch.empty_like(k)
    ops.rope_kv_append(q, k, v, pos, table, kc, vc, slots, 1, query_out=q_out, key_out=k_out,
                       **kw)
    torch.cuda.synchronize()
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    assert torch.equal(q_out.cpu().view(bits), q_ref.cpu().view(bits))
    assert torch.equal(k_out.cpu().view(bits), k_ref.cpu().view(bits))
    assert torch.equal(kc.view(torch.uint8), kc_ref.view(torch.uint8))
    assert torch.equal(vc.view(torch.uint8), vc_ref.view(torch.uint8))


@pytest.mark.parametrize("kv_dtype", [None, FP8])
def test_fused_decode_step_unaligned_new_rows_take_two_launches(device, kv_dtype) -> None:
    hq, hkv, dh, contexts = 16, 4, 64, [70, 5, 300]
    batch, query, _, _, positions, slots, table = _inputs(
        device, torch.bfloat16, hq, hkv, dh, contexts, seed=31, kv_dtype=kv_dtype)
    b = len(contexts)
    rows = torch.randn(b, 2 * hkv * dh + 1, generator=torch.Generator().manual_seed(5))
    rows = rows.to(torch.bfloat16).to(device)
    key = rows[:, 1 : 1 + hkv * dh].view(b, hkv, dh)   # 2-byte aligned only
    value = rows[:, 1 + hkv * dh :].view(b, hkv, dh)
    kw = dict(k_scale=0.5, v_scale=2.0) if kv_dtype is not None else {}
    kc_ref, vc_ref = batch.key_cache.clone(), batch.value_cache.clone()
    q_ref = query.clone()
    ops.rope_kv_append(q_ref, key, value, positions, table, kc_ref, vc_ref, slots, 0, **kw)
    expected = ops.paged_attention_decode(q_ref, kc_ref, vc_ref, batch.block_tables,
                                          batch.seq_lens, layer_index=0,
                                          max_seq_len=batch.max_seq_len, **kw)
    actual = ops.rope_append_paged_decode(
        query, key, value, positions, table, batch.key_cache, batch.value_cache, slots,
        batch.block_tables, batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len, **kw)
    torch.cuda.synchronize()
    assert torch.equal(actual.cpu().view(torch.int16), expected.cpu().view(torch.int16))
    assert torch.equal(batch.key_cache.view(torch.uint8), kc_ref.view(torch.uint8))
    assert torch.equal(batch.value_cache.view(torch.uint8), vc_ref.view(torch.uint8))


@pytest.mark.parametrize("kv_dtype", [None, FP8])
def test_fused_decode_step_lengths_past_the_host_bound(device, kv_dtype) -> None:
    """A length above max_seq_len is clamped to the bound, as the decode alone clamps it:
    the new rows still go to their slot, and the attention covers the clamped keys."""
    hq, hkv, dh, contexts = 32, 8, 128, [100, 40, 64, 65]
    batch, query, key, value, positions, slots, table = _inputs(
        device, torch.bfloat16, hq, hkv, dh, contexts, seed=61, kv_dtype=kv_dtype)
    kw = dict(k_scale=0.5, v_scale=2.0) if kv_dtype is not None else {}
    kc_ref, vc_ref = batch.key_cache.clone(), batch.value_cache.clone()
    q_ref = query.clone()
    ops.rope_kv_append(q_ref, key, value, positions, table, kc_ref, vc_ref, slots, 0, **kw)
    expected = ops.paged_attention_decode(q_ref, kc_ref, vc_ref, batch.block_tables,
                                          batch.seq_lens, layer_index=0, max_seq_len=64, **kw)
    actual = ops.rope_append_paged_decode(
        query, key, value, positions, table, batch.key_cache, batch.value_cache, slots,
        batch.block_tables, batch.seq_lens, layer_index=0, max_seq_len=64, **kw)
    torch.cuda.synchronize()
    assert torch.equal(actual.cpu().view(torch.int16), expected.cpu().view(torch.int16))
    assert torch.equal(batch.key_cache.view(torch.uint8), kc_ref.view(torch.uint8))
    assert torch.equal(batch.value_cache.view(torch.uint8), vc_ref.view(torch.uint8))


@pytest.mark.parametrize("fp8", [False, True])
def test_fused_decode_step_at_the_full_llama3_8b_decode_size(device, fp8) -> None:
    """The 256-sequence Llama-3-8B decode batch (contexts log-uniform in [128, 8192]): the
    fused step equals the two launches bit for bit at full size."""
    batch = (workloads.decode_llama3_8b_fp8 if fp8 else workloads.decode_llama3_8b)(device)
    n, hq, hkv, dh = batch.num_seqs, 32, 8, 128
    g = torch.Generator(device=device).manual_seed(3)
    qkv = torch.randn(n, (hq + 2 * hkv) * dh, generator=g, device=device).to(torch.bfloat16)
    query = qkv[:, : hq * dh].view(n, hq, dh)
    key = qkv[:, hq * dh : (hq + hkv) * dh].view(n, hkv, dh)
    value = qkv[:, (hq + hkv) * dh :].view(n, hkv, dh)
    positions = batch.seq_lens.to(torch.int64) - 1
    tables = batch.block_tables.to(torch.int64)
    slots = tables[torch.arange(n, device=device), positions // 16] * 16 + positions % 16
    table = ops.RotaryTable(dh, theta=500_000.0, max_position=8192, dtype=torch.bfloat16,
                            device=device)
    order = ops.longest_first(batch.contexts, device)
    kc_ref, vc_ref = batch.key_cache.clone(), batch.value_cache.clone()
    q_ref = query.clone()
    ops.rope_kv_append(q_ref, key, value, positions, table, kc_ref, vc_ref, slots, 0)
    expected = ops.paged_attention_decode(q_ref, kc_ref, vc_ref, batch.block_tables,
                                          batch.seq_lens, layer_index=0,
                                          max_seq_len=batch.max_seq_len, seq_order=order)
    del kc_ref, vc_ref
    actual = ops.rope_append_paged_decode(
        query, key, value, positions, table, batch.key_cache, batch.value_cache, slots,
        batch.block_tables, batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len,
        seq_order=order)
    torch.cuda.synchronize()
    assert torch.equal(actual.view(torch.int16), expected.view(torch.int16))
    # The appended rows: each sequence's slot holds the rotated key and the value.
    rows = slots // 16, slots % 16
    q4 = query.clone().transpose(0, 1).unsqueeze(0)
    k4 = key.clone().transpose(0, 1).unsqueeze(0)
    ops.rope(q4, k4, positions, table, query_out=q4, key_out=k4)
    k_rot = k4[0].transpose(0, 1)
    stored_k = batch.key_cache[0, rows[0], :, rows[1], :]
    stored_v = batch.value_cache[0, rows[0], :, rows[1], :]
    if fp8:
        k_rot = k_rot.float().clamp(-448, 448).to(torch.float8_e4m3fn)
        value = value.float().clamp(-448, 448).to(torch.float8_e4m3fn)
    assert torch.equal(stored_k.view(torch.uint8), k_rot.view(torch.uint8))
    assert torch.equal(stored_v.view(torch.uint8), value.view(torch.uint8))


def test_fused_decode_step_argument_errors(device) -> None:
    dtype, hq, hkv, dh, contexts = CASES[0]
    batch, query, key, value, positions, slots, table = _inputs(device, dtype, hq, hkv, dh,
                                                                contexts, seed=12)
    common = dict(layer_index=0, max_seq_len=batch.max_seq_len)
    with pytest.raises(ValueError):
        ops.rope_append_paged_decode(query, key[:, :2], value[:, :2], positions, table,
                                     batch.key_cache, batch.value_cache, slots,
                                     batch.block_tables, batch.seq_lens, **common)
    with pytest.raises(ValueError):
        ops.rope_append_paged_decode(query, key, value, positions[:-1], table, batch.key_cache,
                                     batch.value_cache, slots, batch.block_tables,
                                     batch.seq_lens, **common)
    with pytest.raises(IndexError):
        ops.rope_append_paged_decode(query, key, value, positions, table, batch.key_cache,
                                     batch.value_cache, slots, batch.block_tables,
                                     batch.seq_lens, layer_index=1,
                                     max_seq_len=batch.max_seq_len)


ROWS_CASES = [
    # dtype, Hq, Hkv, Dh, contexts
    (torch.bfloat16, 32, 4, 64, [64 + 37 * i for i in range(24)]),  # the e2e shape, G 8
    (torch.bfloat16, 32, 8, 128, [1, 16, 17, 31, 32, 33, 200, 1025, 4096, 4097]),
    (torch.float16, 16, 8, 128, [5, 48, 49, 700]),
    (torch.bfloat16, 32, 4, 128, [90, 900, 33]),     # G 8 at Dh 128
    (torch.bfloat16, 32, 2, 64, [300, 17, 1]),       # G 16 at Dh 64
    (torch.float32, 8, 2, 64, [16, 17, 513, 100]),   # fp32: two launches
]


def _rows_inputs(device, dtype, hq, hkv, dh, contexts, seed):
    batch = workloads.paged_batch(contexts, [1] * len(contexts), num_q_heads=hq,
                                  num_kv_heads=hkv, head_dim=dh, block_size=16, dtype=dtype,
                                  device=device, seed=seed, kv_dtype=FP8,
                                  scale_granularity="row")
    _, query, key, value, positions, slots, table = _inputs(device, dtype, hq, hkv, dh,
                                                            contexts, seed)
    return batch, query, key, value, positions, slots, table


def _rows_two_calls(batch, query, key, value, positions, table, slots, **kw):
    """The reference: the per-row RoPE + quantizing append, then the decode, on copies
    of the pools and scales."""
    pools = [t.clone() for t in (batch.key_cache, batch.value_cache, batch.k_scales,
                                 batch.v_scales)]
    q_ref = query.clone()
    ops.rope_kv_append(q_ref, key, value, positions, table, pools[0], pools[1], slots, 0,
                       k_scales=pools[2], v_scales=pools[3])
    out = ops.paged_attention_decode(q_ref, pools[0], pools[1], batch.block_tables,
                                     batch.seq_lens, layer_index=0,
                                     max_seq_len=kw.pop("max_seq_len", batch.max_seq_len),
                                     k_scales=pools[2], v_scales=pools[3], **kw)
    return out, pools


def _assert_rows_equal(batch, actual, expected, pools, dtype) -> None:
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    assert torch.equal(actual.cpu().view(bits), expected.cpu().view(bits))
    assert torch.equal(batch.key_cache.view(torch.uint8), pools[0].view(torch.uint8))
    assert torch.equal(batch.value_cache.view(torch.uint8), pools[1].view(torch.uint8))
    assert torch.equal(batch.k_scales.view(torch.int32), pools[2].view(torch.int32))
    assert torch.equal(batch.v_scales.view(torch.int32), pools[3].view(torch.int32))


@pytest.mark.parametrize("case", range(len(ROWS_CASES)))
@pytest.mark.parametrize("pages_per_split", [0, 2])
def test_fused_decode_step_over_row_scaled_fp8_pools(device, case, pages_per_split) -> None:
    """One scale per pool row: the fused launch quantizes the new rows with scales of
    their own (amax / 448), attends with them in place of what their slot held, and
    writes codes and scales; all of it bit for bit as the per-row append followed by the
    decode. New rows include a NaN key element, an all-zero value row and large keys."""
    dtype, hq, hkv, dh, contexts = ROWS_CASES[case]
    batch, query, key, value, positions, slots, table = _rows_inputs(
        device, dtype, hq, hkv, dh, contexts, seed=80 + case)
    key[min(2, len(contexts) - 1), 0, 5] = float("nan")
    value[min(1, len(contexts) - 1)] = 0.0
    key[0] *= 300.0
    order = ops.longest_first(batch.contexts, device)
    query_before = query.clone()
    expected, pools = _rows_two_calls(batch, query, key, value, positions, table, slots,
                                      pages_per_split=pages_per_split, seq_order=order)
    actual = ops.rope_append_paged_decode(
        query, key, value, positions, table, batch.key_cache, batch.value_cache, slots,
        batch.block_tables, batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len,
        pages_per_split=pages_per_split, seq_order=order, k_scales=batch.k_scales,
        v_scales=batch.v_scales)
    torch.cuda.synchronize()
    _assert_rows_equal(batch, actual, expected, pools, dtype)
    assert torch.equal(query, query_before)


def test_fused_decode_step_over_row_scaled_pools_empty_and_negative_slots(device) -> None:
    """Row scales: an empty sequence still appends its rows (codes and scales) and gets a
    zero output; a negative slot appends nothing; both as the two calls do."""
    dtype, hq, hkv, dh = torch.bfloat16, 32, 4, 64
    contexts = [0, 40, 17, 0, 33]
    batch = workloads.paged_batch(contexts, [1] * 5, num_q_heads=hq, num_kv_heads=hkv,
                                  head_dim=dh, block_size=16, dtype=dtype, device=device,
                                  seed=23, num_blocks=12, kv_dtype=FP8,
                                  scale_granularity="row")
    _, query, key, value, positions, slots, table = _inputs(device, dtype, hq, hkv, dh,
                                                            [1, 40, 17, 1, 33], seed=23)
    tables = batch.block_tables.cpu()
    used = {int(tables[b, p]) for b in (1, 2, 4) for p in range((contexts[b] + 15) // 16)}
    free = [blk for blk in range(12) if blk not in used]
    slots[0], slots[3] = free[0] * 16 + 5, free[1] * 16 + 15
    for b in (1, 2, 4):
        slots[b] = int(tables[b, (contexts[b] - 1) // 16]) * 16 + (contexts[b] - 1) % 16
    slots[4] = -1
    positions[0], positions[3] = 0, 7
    expected, pools = _rows_two_calls(batch, query, key, value, positions, table, slots)
    actual = ops.rope_append_paged_decode(
        query, key, value, positions, table, batch.key_cache, batch.value_cache, slots,
        batch.block_tables, batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len,
        k_scales=batch.k_scales, v_scales=batch.v_scales)
    torch.cuda.synchronize()
    _assert_rows_equal(batch, actual, expected, pools, dtype)
    assert not actual[0].any() and not actual[3].any()


@pytest.mark.parametrize("dh", [64, 128])
@pytest.mark.parametrize("group", [1, 2, 4, 8, 16])
def test_fused_decode_step_every_mfma_group_over_row_scaled_pools(device, dh, group) -> None:
    hkv = 2
    contexts = [1, 15, 16, 17, 130, 700]
    batch, query, key, value, positions, slots, table = _rows_inputs(
        device, torch.float16, hkv * group, hkv, dh, contexts, seed=90 + group + dh)
    expected, pools = _rows_two_calls(batch, query, key, value, positions, table, slots)
    actual = ops.rope_append_paged_decode(
        query, key, value, positions, table, batch.key_cache, batch.value_cache, slots,
        batch.block_tables, batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len,
        k_scales=batch.k_scales, v_scales=batch.v_scales)
    torch.cuda.synchronize()
    _assert_rows_equal(batch, actual, expected, pools, torch.float16)
