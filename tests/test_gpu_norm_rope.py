"""RMSNorm, RoPE and greedy argmax on the GPU against the CPU oracle.

RoPE is expected to be bit-exact: the kernel reads the same fp32-angle cos/sin
table (cast to the dtype) and rounds each product to the dtype before the add,
as the reference does. RMSNorm differs from the oracle only by the order of the
fp32 sum of squares: fp32 is held to the parity contract's 1e-5 relative (atol
1e-6 for outputs at zero), fp16 and bf16 to the reference's own tolerances (2e-3,
1e-2; tests/gpu/test_rmsnorm.py:57-68) and the packed bf16 shape to 2e-2 absolute.
"""

from math import prod

import pytest
import torch
from torch.testing import assert_close

from oracle import torch_path
from tokserve_amd import workloads
from tokserve_amd.kernels import ops

pytestmark = pytest.mark.gpu

NORM_TOL = {torch.float32: dict(rtol=1e-5, atol=1e-6), torch.float16: dict(rtol=2e-3, atol=2e-3),
            torch.bfloat16: dict(rtol=1e-2, atol=1e-2)}


@pytest.mark.parametrize(("shape", "epsilon"), [((2, 7), 1e-6), ((2, 3, 13), 1e-3),
                                                ((4, 128), 1e-6), ((3, 4096), 1e-5),
                                                ((5, 2048), 1e-5), ((2, 9000), 1e-6)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_rmsnorm_matches_oracle(device, shape, epsilon, dtype) -> None:
    """Inputs of tests/gpu/test_rmsnorm.py:27-68 (arange/7 - 1, linspace weights)."""

    hidden = shape[-1]
    x = (torch.arange(prod(shape), dtype=torch.float32).reshape(shape) / 7.0 - 1.0).to(dtype)
    w = torch.linspace(0.5, 1.5, hidden, dtype=torch.float32)
    expected = torch_path.rms_norm(x, w, epsilon)
    actual = ops.rms_norm(x.to(device), w.to(device), epsilon)
    torch.cuda.synchronize()
    assert actual.dtype == expected.dtype == torch.float32
    assert_close(actual.cpu(), expected, **NORM_TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rmsnorm_model_dtype_weight(device, dtype) -> None:
    """A weight of the model dtype gives an output of that dtype (torch promotion)."""

    g = torch.Generator().manual_seed(8)
    x = torch.randn(33, 2048, generator=g).to(dtype)
    w = (1 + 0.02 * torch.randn(2048, generator=g)).to(dtype)
    expected = torch_path.rms_norm(x, w, 1e-5)
    actual = ops.rms_norm(x.to(device), w.to(device), 1e-5)
    torch.cuda.synchronize()
    assert actual.dtype == dtype
    assert_close(actual.cpu(), expected, **NORM_TOL[dtype])


def test_rmsnorm_fused_residual(device) -> None:
    """x = to_bf16(h + r) is written back, then normalised (tokserve/engine/model.py:73-82)."""

    g = torch.Generator().manual_seed(9)
    h = torch.randn(17, 2048, generator=g).to(torch.bfloat16)
    r = torch.randn(17, 2048, generator=g).to(torch.bfloat16)
    w = (1 + 0.02 * torch.randn(2048, generator=g)).to(torch.bfloat16)
    summed = h + r
    expected = torch_path.rms_norm(summed, w, 1e-5)
    res_out = torch.empty(17, 2048, dtype=torch.bfloat16, device=device)
    actual = ops.rms_norm(h.to(device), w.to(device), 1e-5, residual=r.to(device),
                          residual_out=res_out)
    torch.cuda.synchronize()
    assert torch.equal(res_out.cpu(), summed)
    assert_close(actual.cpu(), expected, rtol=1e-2, atol=1e-2)


def test_rmsnorm_noncontiguous_input(device) -> None:
    x = torch.randn(2, 3, 13).transpose(0, 1)
    w = torch.linspace(0.5, 1.5, 13)
    expected = torch_path.rms_norm(x, w, 1e-6)
    actual = ops.rms_norm(x.to(device), w.to(device), 1e-6)
    torch.cuda.synchronize()
    assert_close(actual.cpu(), expected, **NORM_TOL[torch.float32])


def test_packed_norm_rope_full_shape(device) -> None:
    """64 sequences, lengths U[1,256] (~8.2k tokens), hidden 4096, 32/8 x 128, theta 5e5, bf16."""

    data = workloads.norm_rope_packed(device, seed=0)
    normed = ops.rms_norm(data.hidden, data.weight, data.epsilon)
    table = ops.RotaryTable(128, theta=data.theta, max_position=4096 + 257,
                            dtype=torch.bfloat16, device=device)
    q4 = data.query.permute(1, 0, 2).unsqueeze(0)  # (1, Hq, N, Dh) view
    k4 = data.key.permute(1, 0, 2).unsqueeze(0)
    rq, rk = ops.rope(q4, k4, data.positions, table)
    torch.cuda.synchronize()
    expected_norm = torch_path.rms_norm(data.hidden.cpu(), data.weight.cpu(), data.epsilon)
    assert_close(normed.cpu(), expected_norm, rtol=0, atol=2e-2)
    assert (normed.cpu() == expected_norm).float().mean() > 0.99
    eq, ek = torch_path.apply_rope(q4.cpu(), k4.cpu(), data.positions.cpu(), theta=data.theta)
    assert torch.equal(rq.cpu(), eq)
    assert torch.equal(rk.cpu(), ek)


@pytest.mark.parametrize(("batch", "hq", "hkv", "length", "dh"), [(1, 4, 2, 3, 8),
                                                                   (2, 6, 2, 5, 16),
                                                                   (1, 32, 4, 7, 64)])
@pytest.mark.parametrize("start", [0, 11])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_rope_bit_exact(device, batch, hq, hkv, length, dh, start, dtype) -> None:
    """Shapes of tests/gpu/test_triton_rope.py:30-70; the oracle is matched bit for bit."""

    g = torch.Generator().manual_seed(7)
    q = torch.randn(batch, hq, length, dh, generator=g).to(dtype)
    k = torch.randn(batch, hkv, length, dh, generator=g).to(dtype)
    pos = torch.arange(start, start + length, dtype=torch.int64)
    eq, ek = torch_path.apply_rope(q, k, pos, theta=10_000.0)
    table = ops.RotaryTable(dh, theta=10_000.0, max_position=64, dtype=dtype, device=device)
    aq, ak = ops.rope(q.to(device), k.to(device), pos.to(device), table)
    torch.cuda.synchronize()
    assert torch.equal(aq.cpu(), eq)
    assert torch.equal(ak.cpu(), ek)


def test_rope_noncontiguous_and_in_place(device) -> None:
    """tests/gpu/test_triton_rope.py:73-92 layout, then an in-place packed rotation."""

    q = torch.randn(1, 3, 4, 8).transpose(1, 2)
    k = torch.randn(1, 3, 2, 8).transpose(1, 2)
    pos = torch.tensor([5, 6, 7])
    eq, ek = torch_path.apply_rope(q, k, pos, theta=10_000.0)
    table = ops.RotaryTable(8, theta=10_000.0, max_position=16, dtype=torch.float32,
                            device=device)
    aq, ak = ops.rope(q.to(device), k.to(device), pos.to(device), table)
    torch.cuda.synchronize()
    assert torch.equal(aq.cpu(), eq)
    assert torch.equal(ak.cpu(), ek)
    packed_q = q[0].transpose(0, 1).contiguous().to(device)  # (T, H, Dh)
    packed_k = k[0].transpose(0, 1).contiguous().to(device)
    q4 = packed_q.permute(1, 0, 2).unsqueeze(0)
    k4 = packed_k.permute(1, 0, 2).unsqueeze(0)
    ops.rope(q4, k4, pos.to(device), table, query_out=q4, key_out=k4)
    torch.cuda.synchronize()
    assert torch.equal(packed_q.cpu(), eq[0].transpose(0, 1))
    assert torch.equal(packed_k.cpu(), ek[0].transpose(0, 1))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_greedy_argmax_matches_torch(device, dtype) -> None:
    g = torch.Generator().manual_seed(12)
    logits = torch.randn(128, 32000, generator=g).to(dtype)
    logits[3, 100] = logits[3, 7] = 50.0  # tie: first index wins
    logits[5, 9] = float("nan")
    logits[5, 2] = float("nan")
    expected = torch_path.select_greedy(logits)
    actual = ops.greedy_argmax(logits.to(device))
    torch.cuda.synchronize()
    assert torch.equal(actual.cpu(), expected)
    assert int(actual[3]) == 7 and int(actual[5]) == 2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(("vocab", "width"), [(32003, 32003), (32000, 32005), (9, 9), (2049, 2056),
                                            (40000, 40000)])
def test_greedy_argmax_chunked_and_element_paths(device, dtype, vocab, width) -> None:
    """Rows read in 16-byte chunks (aligned starts and strides) and element by element
    (any other stride), a vocabulary tail past the last whole chunk, ties between
    entries that different threads and chunks read, NaN in the tail."""

    g = torch.Generator().manual_seed(vocab + width)
    base = torch.randn(6, width, generator=g).to(dtype)
    logits = base.to(device)[:, :vocab]
    host = base[:, :vocab]
    host[0, vocab - 1] = host[0, 1] = 60.0                      # tie: first index wins
    if vocab > 48:
        host[1, 48] = host[1, 8] = 70.0                         # tie across threads' chunks
    if vocab > 36000:
        host[5, 35000] = host[5, 30] = 80.0                     # tie across load batches
    host[2, vocab - 1] = float("nan")                           # NaN in the tail
    host[3, 0] = float("nan")
    host[3, vocab - 1] = float("nan")                           # first NaN wins
    host[4, :] = float("-inf")                                  # all -inf: index 0
    logits.copy_(host.to(device))
    expected = torch_path.select_greedy(host)
    actual = ops.greedy_argmax(logits)
    torch.cuda.synchronize()
    assert torch.equal(actual.cpu(), expected)
    assert int(actual[0]) == 1 and int(actual[2]) == vocab - 1
    assert int(actual[3]) == 0 and int(actual[4]) == 0
    if vocab > 48:
        assert int(actual[1]) == 8
    if vocab > 36000:
        assert int(actual[5]) == 30


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(("hq", "hkv", "dh", "bs"), [(32, 8, 128, 16), (32, 4, 64, 16),
                                                     (4, 2, 10, 3)])
def test_rope_kv_append_equals_rope_then_append(device, dtype, hq, hkv, dh, bs) -> None:
    """The fused launch on the model's packed QKV rows: rotated Q in place, rotated K and V
    in the pools, bit-identical to rope() then kv_append() and to the oracle (torch
    apply_rope, the C append); a negative slot rotates Q and appends nothing
    (Dh 10: the element path)."""

    from oracle import kvslots

    n, layers, blocks = 37, 2, 40
    g = torch.Generator().manual_seed(dh + hq)
    qkv = torch.randn(n, (hq + 2 * hkv) * dh, generator=g).to(dtype)
    pos = torch.randint(0, 200, (n,), generator=g)
    slots = torch.randperm(blocks * bs, generator=g)[:n].to(torch.int64)
    slots[3] = -1
    table = ops.RotaryTable(dh, theta=10_000.0, max_position=256, dtype=dtype, device=device)

    def views(t):
        return (t[:, : hq * dh].view(n, hq, dh), t[:, hq * dh : (hq + hkv) * dh].view(n, hkv, dh),
                t[:, (hq + hkv) * dh :].view(n, hkv, dh))

    shape = (layers, blocks, hkv, bs, dh)
    fused_rows = qkv.to(device)
    q, k, v = views(fused_rows)
    kc, vc = torch.zeros(shape, dtype=dtype, device=device), torch.zeros(shape, dtype=dtype, device=device)
    k_rot = torch.empty(n, hkv, dh, dtype=dtype, device=device)
    ops.rope_kv_append(q, k, v, pos.to(device), table, kc, vc, slots.to(device), 1, key_out=k_rot)

    split_rows = qkv.to(device)
    q2, k2, v2 = views(split_rows)
    q4, k4 = q2.transpose(0, 1).unsqueeze(0), k2.transpose(0, 1).unsqueeze(0)
    ops.rope(q4, k4, pos.to(device), table, query_out=q4, key_out=k4)
    kc2, vc2 = torch.zeros_like(kc), torch.zeros_like(vc)
    ops.kv_append(k2, v2, kc2, vc2, slots.to(device), 1)
    torch.cuda.synchronize()

    assert torch.equal(q.cpu(), q2.cpu())
    assert torch.equal(k_rot.cpu(), k2.cpu())
    assert torch.equal(kc.cpu(), kc2.cpu()) and torch.equal(vc.cpu(), vc2.cpu())
    assert torch.equal(k.cpu(), views(qkv)[1])  # the K rows themselves are left as they were

    qc, kcpu, vcpu = views(qkv)
    eq, ek = torch_path.apply_rope(qc.transpose(0, 1).unsqueeze(0), kcpu.transpose(0, 1).unsqueeze(0),
                                   pos, theta=10_000.0)
    assert torch.equal(q.cpu(), eq[0].transpose(0, 1))
    ekc, evc = torch.zeros(shape, dtype=dtype), torch.zeros(shape, dtype=dtype)
    kvslots.kv_append(ek[0].transpose(0, 1).contiguous(), vcpu.contiguous(), ekc, evc, slots, 1)
    assert torch.equal(kc.cpu(), ekc) and torch.equal(vc.cpu(), evc)
