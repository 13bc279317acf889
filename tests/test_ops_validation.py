"""Host-side validation of the operators: CPU tensors and bad shapes are rejected
before anything reaches the HIP library (tokserve/kernels/paged_attention.py:22-65
and tokserve/kernels/rmsnorm.py:26-27 raise ValueError for non-device tensors)."""

import pytest
import torch

from tokserve_amd.kernels import ops


def test_cpu_tensors_are_rejected() -> None:
    kc = torch.zeros(1, 4, 2, 16, 8)
    with pytest.raises(ValueError, match="requires HIP device tensors"):
        ops.kv_append(torch.zeros(1, 2, 8), torch.zeros(1, 2, 8), kc, kc.clone(),
                      torch.zeros(1, dtype=torch.int64), 0)
    with pytest.raises(ValueError, match="requires HIP device tensors"):
        ops.paged_attention_decode(torch.zeros(1, 4, 8), kc, kc.clone(),
                                   torch.zeros(1, 1, dtype=torch.int32),
                                   torch.ones(1, dtype=torch.int32), layer_index=0,
                                   max_seq_len=1)
    with pytest.raises(ValueError, match="requires HIP device tensors"):
        ops.rms_norm(torch.ones(2, 7), torch.ones(7), 1e-6)
    with pytest.raises(ValueError, match="requires HIP device tensors"):
        ops.greedy_argmax(torch.ones(2, 7))


def test_rotary_table_matches_reference_formula() -> None:
    """The table rows are the fp32 angles' cos/sin cast to the dtype
    (tokserve/engine/rope.py:52-87): position 0 row is exactly (1, 0)."""

    table = ops.RotaryTable(8, theta=10_000.0, max_position=5, dtype=torch.float32,
                            device=torch.device("cpu"))
    assert table.cos.shape == (5, 4)
    assert torch.equal(table.cos[0], torch.ones(4))
    assert torch.equal(table.sin[0], torch.zeros(4))
    inv = 10_000.0 ** (-torch.arange(0, 8, 2, dtype=torch.float32) / 8)
    assert torch.equal(table.cos[3], (3.0 * inv).cos())
    table.ensure(12)
    assert table.length >= 12


def test_workspace_growth_keeps_replaced_buffers_alive() -> None:
    """A grown workspace never frees the old buffer (a captured graph may still hold its
    address), and different uses do not share one buffer."""

    cpu = torch.device("cpu")
    key = "test-growth"
    first = ops._workspace(cpu, 100, key)
    assert first is not None and first.numel() >= 100
    assert ops._workspace(cpu, 50, key) is first
    grown = ops._workspace(cpu, first.numel() + 1, key)
    assert grown is not first and grown.numel() >= 2 * first.numel()
    assert any(t is first for t in ops._retired)
    other = ops._workspace(cpu, 10, key + "-other")
    assert other is not grown
    assert ops._workspace(cpu, 0, key) is None
