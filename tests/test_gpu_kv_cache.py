"""KV append and block-table gather on the GPU: bit-exact against the C oracle."""

import pytest
import torch

from oracle import kvslots
from tokserve_amd.kernels import ops

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _pool(layers, nb, hkv, bs, dh, dtype, fill):
    return torch.full((layers, nb, hkv, bs, dh), fill, dtype=dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("hkv", "bs", "dh"), [(2, 16, 64), (8, 16, 128), (2, 2, 8), (3, 5, 12)])
def test_kv_append_bit_exact(device, dtype, hkv, bs, dh) -> None:
    g = torch.Generator().manual_seed(31)
    lens = torch.tensor([7, 1, 33, 16])
    starts = torch.tensor([0, 5, 10, 16])
    width = (int((starts + lens).max()) + bs - 1) // bs
    layers, nb = 2, 4 * width + 8
    tables = torch.randperm(nb, generator=g)[:4 * width].view(4, width).to(torch.int32)
    slots = kvslots.slot_mapping(tables, starts, lens, bs)
    slots[3] = -1  # a padding token is skipped
    n = slots.shape[0]
    # Source rows as the (Hkv, T, Dh) transposed view the model produces.
    src_k = torch.randn(hkv, n, dh, generator=g).to(dtype).transpose(0, 1)
    src_v = torch.randn(hkv, n, dh, generator=g).to(dtype).transpose(0, 1)
    kc_ref = _pool(layers, nb, hkv, bs, dh, dtype, 7.0)
    vc_ref = _pool(layers, nb, hkv, bs, dh, dtype, -7.0)
    kvslots.kv_append(src_k, src_v, kc_ref, vc_ref, slots, 1)
    kc = kc_ref.new_full(kc_ref.shape, 7.0).to(device)
    vc = vc_ref.new_full(vc_ref.shape, -7.0).to(device)
    ops.kv_append(src_k.to(device), src_v.to(device), kc, vc, slots.to(device), 1)
    torch.cuda.synchronize()
    assert torch.equal(kc.cpu(), kc_ref)
    assert torch.equal(vc.cpu(), vc_ref)


def test_kv_append_mixed_step_size(device) -> None:
    """Append of the mixed-step shape: 16 x 512 prefill tokens + 240 decodes, 8 x 128 bf16."""

    g = torch.Generator().manual_seed(32)
    hkv, bs, dh = 8, 16, 128
    n = 16 * 512 + 240
    nb = (n + bs - 1) // bs + 64
    slots = torch.randperm(nb * bs, generator=g)[:n].to(torch.int64)
    k = torch.randn(n, hkv, dh, generator=g).to(torch.bfloat16)
    v = torch.randn(n, hkv, dh, generator=g).to(torch.bfloat16)
    kc_ref = torch.zeros(1, nb, hkv, bs, dh, dtype=torch.bfloat16)
    vc_ref = torch.zeros_like(kc_ref)
    kvslots.kv_append(k, v, kc_ref, vc_ref, slots, 0)
    kc = torch.zeros_like(kc_ref, device=device)
    vc = torch.zeros_like(vc_ref, device=device)
    ops.kv_append(k.to(device), v.to(device), kc, vc, slots.to(device), 0)
    torch.cuda.synchronize()
    assert torch.equal(kc.cpu(), kc_ref)
    assert torch.equal(vc.cpu(), vc_ref)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("hkv", "bs", "dh"), [(2, 16, 64), (8, 16, 128), (2, 2, 8), (3, 5, 12)])
def test_paged_gather_bit_exact(device, dtype, hkv, bs, dh) -> None:
    g = torch.Generator().manual_seed(33)
    layers, nb = 2, 48
    kc = torch.randn(layers, nb, hkv, bs, dh, generator=g).to(dtype)
    vc = torch.randn(layers, nb, hkv, bs, dh, generator=g).to(dtype)
    tables = torch.randperm(nb, generator=g)[:5 * 9].view(5, 9).to(torch.int32)
    lens = torch.tensor([1, 9 * bs, 0, bs + 1, 2 * bs - 1], dtype=torch.int32)
    k_ref, v_ref = kvslots.paged_gather(kc, vc, tables, lens, 1)
    cu = torch.zeros(6, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0)
    total = int(cu[-1])
    k_out = torch.full((total, hkv, dh), 3.0, dtype=dtype, device=device)
    v_out = torch.full_like(k_out, 3.0)
    ops.paged_gather(kc.to(device), vc.to(device), tables.to(device), lens.to(device),
                     cu.to(device), 1, int(lens.max()), k_out, v_out)
    torch.cuda.synchronize()
    assert torch.equal(k_out.cpu(), k_ref)
    assert torch.equal(v_out.cpu(), v_ref)
