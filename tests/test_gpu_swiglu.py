"""SwiGLU activation kernel (tks_silu_mul) against the reference's
functional.silu(gate) * up in the input dtype (tokserve/engine/layers.py:84-91),
computed by torch on the CPU, and against the fp64 closed form g / (1 + e^-g) * u.

Tolerance: fp32 rtol 1e-6; bf16/fp16 one unit in the last place of the dtype
(exp may differ from the CPU's by an fp32 ulp, which can move one rounding).
"""

import pytest
import torch
from torch.nn import functional
from torch.testing import assert_close

from tokserve_amd.kernels import ops

pytestmark = pytest.mark.gpu

ULP = {torch.float32: 1e-6, torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize(("rows", "inter"), [(1, 8), (3, 5632), (128, 5632), (7, 13), (2, 4)])
def test_silu_mul_matches_torch(device, dtype, rows, inter) -> None:
    g = torch.Generator().manual_seed(rows * 1000 + inter)
    gate_up = (3 * torch.randn(rows, 2 * inter, generator=g)).to(dtype)
    gate, up = gate_up.split(inter, dim=-1)
    expected = functional.silu(gate) * up
    actual = ops.silu_mul(gate_up.to(device))
    torch.cuda.synchronize()
    assert actual.shape == (rows, inter) and actual.dtype == dtype
    assert_close(actual.cpu(), expected, rtol=ULP[dtype], atol=1e-6)
    exact = (gate.double() / (1 + torch.exp(-gate.double()))) * up.double()
    assert_close(actual.cpu().double(), exact, rtol=3 * ULP[dtype], atol=1e-6)


def test_silu_mul_strided_rows_and_special_values(device) -> None:
    base = torch.randn(4, 40, dtype=torch.bfloat16)
    base[0, 0], base[0, 1], base[0, 2] = float("inf"), float("-inf"), 0.0
    gate_up = base.to(device)[:, :32]  # row stride 40, width 32 (I = 16)
    actual = ops.silu_mul(gate_up)
    gate, up = base[:, :32].split(16, dim=-1)
    torch.cuda.synchronize()
    assert_close(actual.cpu(), functional.silu(gate) * up, rtol=2.0 ** -7, atol=1e-6,
                 equal_nan=True)
    out = torch.empty(4, 24, dtype=torch.bfloat16, device=device)
    ops.silu_mul(gate_up, out=out[:, :16])
    torch.cuda.synchronize()
    assert_close(out[:, :16].cpu(), actual.cpu(), rtol=0, atol=0, equal_nan=True)
