"""Host-side validation of the operators: CPU tensors and bad shapes are rejected
before anything reaches the HIP library (tokserve/kernels/paged_attention.py:22-65
and tokserve/kernels/rmsnorm.py:26-27 raise ValueError for non-device tensors)."""

import pytest
import torch

from tokserve_amd.kernels import ops, torch_ops


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
    table = ops.RotaryTable(8, theta=10_000.0, max_position=16, dtype=torch.float32,
                            device=torch.device("cpu"))
    with pytest.raises(ValueError, match="requires HIP device tensors"):
        ops.rope_append_paged_decode(
            torch.zeros(1, 4, 8), torch.zeros(1, 2, 8), torch.zeros(1, 2, 8),
            torch.zeros(1, dtype=torch.int64), table, kc, kc.clone(),
            torch.zeros(1, dtype=torch.int64), torch.zeros(1, 1, dtype=torch.int32),
            torch.ones(1, dtype=torch.int32), layer_index=0, max_seq_len=1)


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
    first = torch_ops.workspace(cpu, 100, key)
    assert first is not None and first.numel() >= 100
    assert torch_ops.workspace(cpu, 50, key) is first
    grown = torch_ops.workspace(cpu, first.numel() + 1, key)
    assert grown is not first and grown.numel() >= 2 * first.numel()
    assert any(t is first for t in torch_ops._retired)
    other = torch_ops.workspace(cpu, 10, key + "-other")
    assert other is not grown
    assert torch_ops.workspace(cpu, 0, key) is None


def test_every_operator_is_registered_with_its_writes_marked() -> None:
    """Each C-ABI kernel family is a torch.library operator; the tensors it writes (KV
    pools and their per-row scales, outputs, in-place rotations) are marked mutable in
    its schema, and nothing else is."""

    writes = {
        "kv_append": {"key_cache", "value_cache", "k_scales", "v_scales"},
        "paged_gather": {"key_out", "value_out"},
        "paged_attention_decode": {"out", "workspace"},
        "paged_attention_decode_noalloc": {"out"},
        "paged_attention_prefill": {"out"},
        "rms_norm": {"out", "residual_out"},
        "rope": {"query_out", "key_out"},
        "rope_": {"query", "key"},
        "rope_kv_append": {"key_cache", "value_cache", "query_out", "key_out", "k_scales", "v_scales"},
        "rope_kv_append_": {"query", "key_cache", "value_cache", "key_out", "k_scales", "v_scales"},
        "rope_append_paged_decode": {"key_cache", "value_cache", "out", "workspace", "k_scales", "v_scales"},
        "greedy_argmax": {"out"},
        "silu_mul": {"out"},
        "vector_add": {"out"},
    }
    assert set(torch_ops.SCHEMAS) == set(writes)
    for name, expected in writes.items():
        schema = getattr(torch.ops.tokserve_amd, name).default._schema
        mutated = {a.name for a in schema.arguments if a.alias_info is not None
                   and a.alias_info.is_write}
        assert mutated == expected, name
        assert not schema.returns, name


def test_entry_points_behind_the_operators_cover_the_c_abi() -> None:
    from tokserve_amd.kernels import _lib

    covered = {entry for entries in torch_ops.ENTRY_POINTS.values() for entry in entries}
    infrastructure = {"tks_abi_version", "tks_status_string", "tks_last_hip_error"}
    assert covered | infrastructure == set(_lib.SIGNATURES)


def test_operators_have_no_cpu_kernel() -> None:
    with pytest.raises(NotImplementedError):
        torch.ops.tokserve_amd.vector_add(torch.ones(3), torch.ones(3), torch.empty(3))


def test_operators_trace_with_fake_tensors() -> None:
    """FakeTensor propagation runs the fake kernels (no device, no library call)."""

    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q = torch.empty(4, 8, 64, dtype=torch.bfloat16, device="cuda")
        pool = torch.empty(1, 16, 2, 16, 64, dtype=torch.bfloat16, device="cuda")
        tables = torch.zeros(4, 4, dtype=torch.int32, device="cuda")
        lens = torch.ones(4, dtype=torch.int32, device="cuda")
        out = torch.empty_like(q)
        torch.ops.tokserve_amd.paged_attention_decode(q, pool, pool, tables, lens, None, 0, 64,
                                                      0.125, 0, 1.0, 1.0, out, None)
        assert out.shape == q.shape
        kv = torch.empty(4, 2, 64, dtype=torch.bfloat16, device="cuda")
        pos = torch.zeros(4, dtype=torch.int64, device="cuda")
        cos = torch.empty(16, 32, dtype=torch.bfloat16, device="cuda")
        torch.ops.tokserve_amd.rope_append_paged_decode(q, kv, kv, pos, cos, cos, pos, pool,
                                                        pool, tables, lens, None, 0, 64, 0.125,
                                                        0, out, None)


@pytest.fixture
def meta_as_device(monkeypatch):
    """Tensors on the meta device stand in for HIP tensors (CPU tensors stay host
    tensors), and the library's operators only record that they were reached."""

    reached: list[str] = []

    def require(operation, *tensors):
        for tensor in tensors:
            if tensor.device.type != "meta":
                raise ValueError(f"{operation} requires HIP device tensors")
        return tensors[0].device

    class Library:
        def __getattr__(self, name):
            return lambda *args, **kwargs: reached.append(name)

    monkeypatch.setattr(ops, "require_hip", require)
    monkeypatch.setattr(ops, "_ops", Library())
    return reached


def _decode_args(device):
    kc = torch.zeros(1, 4, 2, 16, 8, device=device)
    return (torch.zeros(3, 4, 8, device=device), kc, torch.zeros_like(kc),
            torch.zeros(3, 1, dtype=torch.int32, device=device),
            torch.ones(3, dtype=torch.int32, device=device))


def test_decode_sequence_order_and_workspace_must_be_device_tensors(meta_as_device) -> None:
    """A host seq_order or workspace beside device tensors would hand a host address to the
    kernel: every decode entry point rejects it, and a seq_order of the wrong length,
    before anything is launched."""

    meta = torch.device("meta")
    args = _decode_args(meta)
    good_order = torch.arange(3, dtype=torch.int32, device=meta)
    ops.paged_attention_decode(*args, layer_index=0, max_seq_len=1, seq_order=good_order,
                               workspace=torch.zeros(64, dtype=torch.uint8, device=meta))
    ops.paged_attention_decode_noalloc(*args, layer_index=0, max_seq_len=1,
                                       out=torch.zeros_like(args[0]), seq_order=good_order)
    assert meta_as_device == ["paged_attention_decode", "paged_attention_decode_noalloc"]
    meta_as_device.clear()
    host_order = torch.arange(3, dtype=torch.int32)
    for order, message in ((host_order, "requires HIP device tensors"),
                           (torch.arange(4, dtype=torch.int32, device=meta),
                            r"seq_order must have shape \(B,\)")):
        with pytest.raises(ValueError, match=message):
            ops.paged_attention_decode(*args, layer_index=0, max_seq_len=1, seq_order=order)
        with pytest.raises(ValueError, match=message):
            ops.paged_attention_decode_noalloc(*args, layer_index=0, max_seq_len=1,
                                               out=torch.zeros_like(args[0]), seq_order=order)
    for workspace, message in ((torch.zeros(64, dtype=torch.uint8), "requires HIP device"),
                               (torch.zeros(16, device=meta), "contiguous uint8")):
        with pytest.raises(ValueError, match=message):
            ops.paged_attention_decode(*args, layer_index=0, max_seq_len=1, workspace=workspace)
    assert meta_as_device == []


def test_fused_decode_sequence_order_and_workspace_must_be_device_tensors(
        meta_as_device) -> None:
    meta = torch.device("meta")
    query, kc, vc, tables, lens = _decode_args(meta)
    table = ops.RotaryTable(8, theta=10_000.0, max_position=16, dtype=torch.float32,
                            device=meta)
    rows = (torch.zeros(3, 2, 8, device=meta), torch.zeros(3, 2, 8, device=meta),
            torch.zeros(3, dtype=torch.int64, device=meta))

    def call(**kwargs):
        ops.rope_append_paged_decode(query, *rows[:2], rows[2], table, kc, vc,
                                     torch.zeros(3, dtype=torch.int64, device=meta), tables,
                                     lens, layer_index=0, max_seq_len=1, **kwargs)

    call(seq_order=torch.arange(3, dtype=torch.int32, device=meta))
    assert meta_as_device == ["rope_append_paged_decode"]
    meta_as_device.clear()
    with pytest.raises(ValueError, match="requires HIP device tensors"):
        call(seq_order=torch.arange(3, dtype=torch.int32))
    with pytest.raises(ValueError, match="requires HIP device tensors"):
        call(workspace=torch.zeros(64, dtype=torch.uint8))
    with pytest.raises(ValueError, match="contiguous uint8"):
        call(workspace=torch.zeros(64, dtype=torch.int32, device=meta))
    assert meta_as_device == []


def test_row_scales_are_checked_before_launch(meta_as_device) -> None:
    """Per-row scale arrays: both or neither, fp8 pools only, float32 (L, NB, Hkv, BS)
    contiguous on the pools' device, and no pool scales beside them."""

    meta = torch.device("meta")
    query, _, _, tables, lens = _decode_args(meta)
    kc = torch.zeros(1, 4, 2, 16, 8, dtype=ops.FP8_POOL_DTYPE, device=meta)
    vc = torch.zeros_like(kc)
    ks = torch.ones(1, 4, 2, 16, device=meta)

    def call(pool=kc, **kwargs):
        ops.paged_attention_decode(query, pool, pool if pool is not kc else vc, tables, lens,
                                   layer_index=0, max_seq_len=1, **kwargs)

    call(k_scales=ks, v_scales=ks.clone())
    assert meta_as_device == ["paged_attention_decode"]
    meta_as_device.clear()
    for kwargs, error, message in (
        (dict(k_scales=ks), ValueError, "go together"),
        (dict(k_scales=ks, v_scales=ks.double()), TypeError, "float32"),
        (dict(k_scales=ks, v_scales=ks[..., :8]), ValueError, "contiguous"),
        (dict(k_scales=ks, v_scales=ks.transpose(2, 3).contiguous().transpose(2, 3)), ValueError,
         "contiguous"),
        (dict(k_scales=ks, v_scales=torch.ones(1, 4, 2, 16)), ValueError, "HIP device"),
        (dict(k_scales=ks, v_scales=ks, k_scale=2.0), ValueError, "must stay 1"),
        (dict(pool=torch.zeros(1, 4, 2, 16, 8, device=meta), k_scales=ks, v_scales=ks),
         ValueError, "fp8 KV pools only"),
    ):
        with pytest.raises(error, match=message):
            call(**kwargs)
    assert meta_as_device == []
