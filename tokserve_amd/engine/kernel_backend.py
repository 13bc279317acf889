"""Backend selection under the reference's module path (tokserve/engine/kernel_backend.py).

The reference chooses between its torch ops and its Triton kernels
(`KernelBackend = Literal["torch", "triton"]`, kernel_backend.py:10-34). Here
both names run the HIP kernels: "torch" through the RMSNorm module (the
torch backend's contract: output dtype promote(weight, input)), "triton" with
the Triton wrapper's contract and checks (a device tensor, fp32 weights, fp32
output).
"""

from __future__ import annotations

from typing import Literal

import torch

from tokserve_amd.engine.layers import RMSNorm
from tokserve_amd.kernels.rmsnorm import triton_rms_norm

__all__ = ["KernelBackend", "BACKENDS", "check_backend", "apply_rms_norm"]

KernelBackend = Literal["torch", "triton"]
BACKENDS = ("torch", "triton")


def check_backend(backend: str) -> str:
    """The reference's constructor check (engine/model.py:26-27,96-97; attention.py:141-142)."""

    if backend not in BACKENDS:
        raise ValueError("backend must be 'torch' or 'triton'")
    return backend


def apply_rms_norm(norm: RMSNorm, inputs: torch.Tensor, backend: KernelBackend) -> torch.Tensor:
    """RMSNorm of `inputs` with `norm`'s weight under the backend's contract."""

    if backend == "torch":
        return norm(inputs)
    if not inputs.is_cuda:
        raise ValueError("Triton backend requires CUDA")
    if norm.weight.dtype != torch.float32:
        raise TypeError("Triton backend requires float32 RMSNorm weights")
    return triton_rms_norm(inputs, norm.weight, epsilon=norm.epsilon)
