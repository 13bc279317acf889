"""Drop-in RMSNorm (tokserve/kernels/rmsnorm.py).

`hip_rms_norm` keeps the reference operator's contract: float32 weight,
float32 output, y = w * to_in_dtype(x * rsqrt(mean(x^2) + eps)) with the
normalized value rounded to the input dtype before the weight multiply
(tokserve/kernels/_triton_rmsnorm.py:30-36). `triton_rms_norm` is the same
function under the reference's name.
"""

from __future__ import annotations

import torch

from tokserve_amd.kernels import ops

__all__ = ["hip_rms_norm", "triton_rms_norm"]


def hip_rms_norm(
    inputs: torch.Tensor,
    weight: torch.Tensor,
    *,
    epsilon: float = 1e-6,
) -> torch.Tensor:
    """Apply RMSNorm across the final dimension of HIP inputs."""

    if inputs.ndim < 1:
        raise ValueError("inputs must have at least one dimension")
    hidden_size = inputs.shape[-1]
    if hidden_size < 1:
        raise ValueError("hidden size must be positive")
    if weight.shape != (hidden_size,):
        raise ValueError("weight must have shape (D,)")
    if epsilon <= 0.0:
        raise ValueError("epsilon must be positive")
    if not inputs.is_cuda or not weight.is_cuda:
        raise ValueError("inputs and weight must be CUDA tensors")
    if inputs.device != weight.device:
        raise ValueError("inputs and weight must use the same device")
    if inputs.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        raise TypeError("inputs must use float32, float16, or bfloat16")
    if weight.dtype != torch.float32:
        raise TypeError("weight must use float32")
    if inputs.numel() == 0:
        return torch.empty(inputs.shape, dtype=torch.float32, device=inputs.device)
    return ops.rms_norm(inputs, weight, epsilon)


triton_rms_norm = hip_rms_norm
