"""A decode step's RoPE + KV append + attention in one call (tks_rope_append_paged_decode)
against the two calls it replaces, tks_rope_kv_append then tks_paged_attention_decode,
on the same inputs: the pools after the call and the outputs are bit-identical, the
query is left as it was. Covered: the fused MFMA launch (bf16 / fp16, Dh 64 and 128,
several GQA groups, with and without key splits, partly filled and exactly full last
pages, a new token that opens a page), the two-call path it takes elsewhere (fp32 on the
generic kernel, Dh 128 with G 8), a negative slot (nothing appended) and an empty
sequence (its row is appended, its output is zero).
"""

import pytest
import torch

from tokserve_amd import workloads
from tokserve_amd.kernels import ops

pytestmark = pytest.mark.gpu

CASES = [
    # dtype, Hq, Hkv, Dh, contexts
    (torch.bfloat16, 32, 4, 64, [64 + 37 * i for i in range(24)]),
    (torch.bfloat16, 32, 8, 128, [1, 16, 17, 31, 32, 33, 200, 1025, 4096, 4097]),
    (torch.float16, 16, 8, 128, [5, 48, 49, 700]),
    (torch.bfloat16, 16, 16, 128, [300, 17, 1]),
    (torch.bfloat16, 32, 4, 128, [90, 900]),       # G 8 at Dh 128: the two-call path
    (torch.float32, 8, 2, 64, [16, 17, 513, 100]),  # fp32: generic kernel, two calls
]


def _inputs(device, dtype, hq, hkv, dh, contexts, seed):
    batch = workloads.paged_batch(contexts, [1] * len(contexts), num_q_heads=hq,
                                  num_kv_heads=hkv, head_dim=dh, block_size=16, dtype=dtype,
                                  device=device, seed=seed)
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
    slots = (tables[torch.arange(b), pos // 16] * 16 + pos % 16).to(device)
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


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
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
    assert torch.equal(actual.cpu().view(torch.int16), expected.cpu().view(torch.int16))
    assert not actual[0].any() and not actual[3].any()
    assert torch.equal(batch.key_cache, kc_ref) and torch.equal(batch.value_cache, vc_ref)


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
