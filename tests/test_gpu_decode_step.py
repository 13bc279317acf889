"""The CPU-runnable fp32 decode step as one composed step on the GPU against the oracle.

8 sequences with contexts U[16, 512] (+1 appended token), 8 query / 2 KV heads,
head_dim 64, block size 16, a 512-block pool with disjoint random block tables,
seed 0. The step is what the model layer runs for one decode token per sequence:
RMSNorm (hidden 512, eps 1e-5, weight N(1, 0.02)), RoPE (theta 1e4) of the new
query and key at each sequence's next position with the K/V append through
slot_mapping in the same launch, then split-K decode attention over the appended
pools. Bar: RMSNorm and attention within 1e-5 relative, RoPE and the pools bit-exact.
"""

import pytest
import torch
from torch.testing import assert_close

from oracle import kvslots, paged, torch_path
from tokserve_amd import workloads
from tokserve_amd.kernels import ops

pytestmark = pytest.mark.gpu

FP32 = dict(rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("pages_per_split", [0, 1, 4])
def test_fp32_decode_step_composed_matches_oracle(device, pages_per_split) -> None:
    batch = workloads.decode_fp32_small(device, seed=0)
    g = torch.Generator().manual_seed(1)
    hidden = torch.randn(8, 512, generator=g)
    weight = 1.0 + 0.02 * torch.randn(512, generator=g)
    new_k = torch.randn(8, 2, 64, generator=g)
    new_v = torch.randn(8, 2, 64, generator=g)
    tables = batch.block_tables.cpu()
    positions = torch.tensor([c - 1 for c in batch.contexts], dtype=torch.int64)
    slots = kvslots.slot_mapping(tables, positions, torch.ones(8, dtype=torch.int64), 16)
    k_pool, v_pool = batch.key_cache.cpu(), batch.value_cache.cpu()

    table = ops.RotaryTable(64, theta=10_000.0, max_position=1024, dtype=torch.float32,
                            device=device)
    normed = ops.rms_norm(hidden.to(device), weight.to(device), 1e-5)
    q_rot = torch.empty_like(batch.query)
    k_rot = torch.empty((8, 2, 64), device=device)
    ops.rope_kv_append(batch.query, new_k.to(device), new_v.to(device), positions.to(device),
                       table, batch.key_cache, batch.value_cache, slots.to(device), 0,
                       query_out=q_rot, key_out=k_rot)
    out = ops.paged_attention_decode(q_rot, batch.key_cache, batch.value_cache,
                                     batch.block_tables, batch.seq_lens, layer_index=0,
                                     max_seq_len=batch.max_seq_len,
                                     pages_per_split=pages_per_split)
    torch.cuda.synchronize()

    expected_norm = torch_path.rms_norm(hidden, weight, 1e-5)
    # Packed (N, H, Dh) rows as one (1, H, N, Dh) sequence: every token has its own position.
    eq, ek = torch_path.apply_rope(batch.query.cpu().transpose(0, 1).unsqueeze(0),
                                   new_k.transpose(0, 1).unsqueeze(0), positions, theta=10_000.0)
    eq = eq.squeeze(0).transpose(0, 1)
    ek = ek.squeeze(0).transpose(0, 1)
    kvslots.kv_append(ek.contiguous(), new_v, k_pool, v_pool, slots, 0)
    expected_out = paged.decode_batch(eq.contiguous(), k_pool, v_pool, tables,
                                      batch.seq_lens.cpu(), 0)

    assert_close(normed.cpu(), expected_norm, **FP32)
    assert torch.equal(q_rot.cpu(), eq)
    assert torch.equal(k_rot.cpu(), ek)
    assert torch.equal(batch.key_cache.cpu(), k_pool)
    assert torch.equal(batch.value_cache.cpu(), v_pool)
    assert_close(out.cpu(), expected_out, **FP32)
