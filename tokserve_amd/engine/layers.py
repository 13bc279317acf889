"""RMSNorm and SwiGLU modules (tokserve/engine/layers.py).

Parameters, their names, shapes and creation order match the reference
modules, so a state dict moves between the two and a seeded random
initialisation produces the same weights. The forward passes run on HIP
tensors only: RMSNorm through the tks_rms_norm kernel (the reference's
rounding: normalised value rounded to the input dtype, then times the weight,
output dtype = promote(weight, input)), SwiGLU as one library GEMM over the
stacked gate/up weights, the tks_silu_mul kernel, and the down GEMM.
"""

from __future__ import annotations

import torch
from torch import nn
from torch.nn import functional

from tokserve_amd.kernels import ops

__all__ = ["RMSNorm", "SwiGLU", "fused_weight"]


class RMSNorm(nn.Module):
    """Llama RMSNorm with a learned scale."""

    def __init__(self, hidden_size: int, *, epsilon: float = 1e-6) -> None:
        super().__init__()
        if hidden_size < 1:
            raise ValueError("hidden_size must be positive")
        if epsilon <= 0.0:
            raise ValueError("epsilon must be positive")
        self.hidden_size = hidden_size
        self.epsilon = epsilon
        self.weight = nn.Parameter(torch.ones(hidden_size))

    def forward(
        self, inputs: torch.Tensor, residual: torch.Tensor | None = None
    ) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor]:
        """weight * to_in(x * rsqrt(mean(x^2) + eps)); with `residual`, x = to_in(inputs +
        residual) is formed first and (normalised, x) returned."""

        if inputs.ndim < 1:
            raise ValueError("inputs must have at least one dimension")
        if inputs.shape[-1] != self.hidden_size:
            raise ValueError("inputs must use the configured hidden_size")
        if residual is None:
            return ops.rms_norm(inputs, self.weight, self.epsilon)
        summed = torch.empty_like(inputs)
        normalized = ops.rms_norm(inputs, self.weight, self.epsilon, residual=residual,
                                  residual_out=summed)
        return normalized, summed


def fused_weight(owner: nn.Module, linears: list[nn.Linear], cache_name: str) -> torch.Tensor:
    """One weight matrix stacking the rows of `linears`, which then view into it.

    The first call (and any call after .to() or load_state_dict gave a
    parameter new storage) concatenates the weights and rebinds each
    parameter's data to its row range of the result, so the fused matrix costs
    no extra memory and stays the modules' own storage.
    """

    fused = getattr(owner, cache_name, None)
    if fused is not None:
        offset = 0
        intact = True
        for linear in linears:
            rows = linear.weight.shape[0]
            view = fused[offset : offset + rows]
            if (linear.weight.data_ptr() != view.data_ptr() or linear.weight.dtype != fused.dtype
                    or linear.weight.device != fused.device):
                intact = False
                break
            offset += rows
        if intact:
            return fused
    # Built outside inference mode, so the parameters stay ordinary tensors that
    # .to() and load_state_dict may later update in place.
    with torch.inference_mode(False), torch.no_grad():
        fused = torch.cat([linear.weight.detach() for linear in linears], dim=0).contiguous()
        offset = 0
        for linear in linears:
            rows = linear.weight.shape[0]
            linear.weight.data = fused[offset : offset + rows]
            offset += rows
    object.__setattr__(owner, cache_name, fused)
    return fused


class SwiGLU(nn.Module):
    """Bias-free Llama SwiGLU feed-forward network."""

    def __init__(self, hidden_size: int, intermediate_size: int) -> None:
        super().__init__()
        if hidden_size < 1:
            raise ValueError("hidden_size must be positive")
        if intermediate_size < 1:
            raise ValueError("intermediate_size must be positive")
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.gate_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.up_proj = nn.Linear(hidden_size, intermediate_size, bias=False)
        self.down_proj = nn.Linear(intermediate_size, hidden_size, bias=False)

    def forward(self, inputs: torch.Tensor) -> torch.Tensor:
        """down(silu(gate(x)) * up(x))."""

        if inputs.ndim < 1:
            raise ValueError("inputs must have at least one dimension")
        if inputs.shape[-1] != self.hidden_size:
            raise ValueError("inputs must use the configured hidden_size")
        gate_up = functional.linear(
            inputs, fused_weight(self, [self.gate_proj, self.up_proj], "_gate_up")
        )
        return self.down_proj(ops.silu_mul(gate_up))
