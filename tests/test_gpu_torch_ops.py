"""The kernels as PyTorch operators (torch.ops.tokserve_amd.*) under torch.compile.

A packed decode step of the Llama-3-8B layer shape (RMSNorm -> QKV GEMM -> RoPE with
the K/V append into the pools -> split-K decode attention, as two operators or as the
fused one) compiles with
fullgraph=True (no graph break: every kernel call is an operator that tracing sees,
with a fake kernel for shapes and its writes declared in its schema) and gives
results bit-identical to eager execution: outputs and the written pools. The
`aot_eager` backend runs the traced, functionalized graph without generating code
(Inductor would emit Triton for the copies functionalization adds).
"""

import pytest
import torch

from tokserve_amd import workloads
from tokserve_amd.kernels import ops

pytestmark = pytest.mark.gpu


def _step_inputs(device, seed):
    contexts = [300, 17, 1500, 64, 9, 800, 2100, 128]
    batch = workloads.paged_batch(contexts, [1] * len(contexts), num_q_heads=32, num_kv_heads=8,
                                  head_dim=128, block_size=16, dtype=torch.bfloat16,
                                  device=device, seed=seed)
    g = torch.Generator().manual_seed(seed + 1)
    hidden = torch.randn(len(contexts), 4096, generator=g).to(torch.bfloat16).to(device)
    weight = (1 + 0.02 * torch.randn(4096, generator=g)).to(torch.bfloat16).to(device)
    qkv_weight = (torch.randn(48 * 128, 4096, generator=g) / 64).to(torch.bfloat16).to(device)
    tables = batch.block_tables.cpu()
    positions = torch.tensor([c - 1 for c in contexts], dtype=torch.int64)
    slots = torch.tensor([int(tables[b, p // 16]) * 16 + p % 16
                          for b, p in enumerate(positions.tolist())], dtype=torch.int64)
    return batch, hidden, weight, qkv_weight, positions.to(device), slots.to(device)


def _make_step(table, max_seq_len, pages_per_split, fused):
    def step(hidden, weight, qkv_weight, positions, slots, key_cache, value_cache, tables, lens):
        normed = ops.rms_norm(hidden, weight, 1e-5)
        qkv = normed @ qkv_weight.t()
        tokens = qkv.shape[0]
        query = qkv[:, : 32 * 128].view(tokens, 32, 128)
        key = qkv[:, 32 * 128 : 40 * 128].view(tokens, 8, 128)
        value = qkv[:, 40 * 128 :].view(tokens, 8, 128)
        if fused:
            return ops.rope_append_paged_decode(
                query, key, value, positions, table, key_cache, value_cache, slots, tables,
                lens, layer_index=0, max_seq_len=max_seq_len, pages_per_split=pages_per_split)
        ops.rope_kv_append(query, key, value, positions, table, key_cache, value_cache, slots, 0)
        return ops.paged_attention_decode(query, key_cache, value_cache, tables, lens,
                                          layer_index=0, max_seq_len=max_seq_len,
                                          pages_per_split=pages_per_split)

    return step


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("pages_per_split", [0, 8])
def test_compiled_packed_decode_step_is_bit_identical_to_eager(device, pages_per_split,
                                                               fused) -> None:
    batch, hidden, weight, qkv_weight, positions, slots = _step_inputs(device, seed=5)
    table = ops.RotaryTable(128, theta=500_000.0, max_position=4096, dtype=torch.bfloat16,
                            device=device)
    step = _make_step(table, batch.max_seq_len, pages_per_split, fused)
    compiled = torch.compile(step, fullgraph=True, backend="aot_eager", dynamic=False)
    pools = []
    outs = []
    for fn in (step, compiled):
        key_cache, value_cache = batch.key_cache.clone(), batch.value_cache.clone()
        with torch.no_grad():
            outs.append(fn(hidden, weight, qkv_weight, positions, slots, key_cache, value_cache,
                           batch.block_tables, batch.seq_lens))
        pools.append((key_cache, value_cache))
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(pools[0][0], pools[1][0]) and torch.equal(pools[0][1], pools[1][1])
    assert not torch.equal(pools[0][0], batch.key_cache)  # the step did append


def test_compiled_prefill_and_norm_with_residual(device) -> None:
    """Chunked prefill attention and the fused residual RMSNorm under torch.compile."""

    batch = workloads.paged_batch([40, 300, 7], [40, 100, 7], num_q_heads=32, num_kv_heads=8,
                                  head_dim=128, block_size=16, dtype=torch.bfloat16,
                                  device=device, seed=9)
    g = torch.Generator().manual_seed(10)
    hidden = torch.randn(147, 4096, generator=g).to(torch.bfloat16).to(device)
    residual = torch.randn(147, 4096, generator=g).to(torch.bfloat16).to(device)
    weight = (1 + 0.02 * torch.randn(4096, generator=g)).to(torch.bfloat16).to(device)

    def step(query, hidden, residual):
        attended = ops.paged_attention_prefill(
            query, batch.key_cache, batch.value_cache, batch.block_tables, batch.seq_lens,
            batch.cu_seqlens_q, layer_index=0, max_query_len=100, max_seq_len=300)
        summed = torch.empty_like(hidden)
        normed = ops.rms_norm(hidden, weight, 1e-5, residual=residual, residual_out=summed)
        return attended, normed, summed

    compiled = torch.compile(step, fullgraph=True, backend="aot_eager", dynamic=False)
    with torch.no_grad():
        eager = step(batch.query, hidden, residual)
        traced = compiled(batch.query, hidden, residual)
    torch.cuda.synchronize()
    for a, b in zip(eager, traced):
        assert torch.equal(a, b)
