"""Next-token selection (tokserve/generation/{sampling,temperature,top_k,top_p}.py).

Greedy selection, the hot path's, is generation.greedy.select_greedy (the
tks_argmax kernel). Sampling
(temperature, top-k, top-p, multinomial with the request's own generator) uses
torch's device ops in the reference's order; it is outside the measured path.
"""

from __future__ import annotations

import torch

from tokserve_amd.generation.greedy import select_greedy
from tokserve_amd.generation.types import GenerationConfig

__all__ = ["select_greedy", "scale_temperature", "filter_top_k", "filter_top_p",
           "sample_from_logits", "select_next_token"]


def scale_temperature(logits: torch.Tensor, temperature: float) -> torch.Tensor:
    if logits.ndim != 2:
        raise ValueError("logits must have shape (B, V)")
    if temperature <= 0.0:
        raise ValueError("temperature must be positive")
    return logits / temperature


def filter_top_k(logits: torch.Tensor, top_k: int | None) -> torch.Tensor:
    if logits.ndim != 2:
        raise ValueError("logits must have shape (B, V)")
    if top_k is None or top_k >= logits.shape[-1]:
        return logits.clone()
    if top_k < 1:
        raise ValueError("top_k must be positive")
    threshold = torch.topk(logits, top_k, dim=-1).values[..., -1:]
    return logits.masked_fill(logits < threshold, -torch.inf)


def filter_top_p(logits: torch.Tensor, top_p: float | None) -> torch.Tensor:
    """Keep the smallest high-probability prefix whose mass reaches top_p (the first
    token always stays)."""

    if logits.ndim != 2:
        raise ValueError("logits must have shape (B, V)")
    if top_p is None or top_p == 1.0:
        return logits.clone()
    if not 0.0 < top_p <= 1.0:
        raise ValueError("top_p must be in the interval (0, 1]")
    ordered, order = torch.sort(logits, descending=True, dim=-1)
    mass = torch.cumsum(torch.softmax(ordered, dim=-1), dim=-1)
    drop_sorted = torch.zeros_like(mass, dtype=torch.bool)
    drop_sorted[..., 1:] = mass[..., :-1] > top_p
    drop = torch.zeros_like(drop_sorted).scatter_(-1, order, drop_sorted)
    return logits.masked_fill(drop, -torch.inf)


def sample_from_logits(
    logits: torch.Tensor, *, generator: torch.Generator | None = None
) -> torch.Tensor:
    if logits.ndim != 2:
        raise ValueError("logits must have shape (B, V)")
    if logits.shape[0] < 1 or logits.shape[1] < 1:
        raise ValueError("logits dimensions must be positive")
    if not torch.isfinite(logits).any(dim=-1).all():
        raise ValueError("each logits row must contain a finite value")
    return torch.multinomial(torch.softmax(logits, dim=-1), num_samples=1, generator=generator)


def select_next_token(
    logits: torch.Tensor, config: GenerationConfig, *, generator: torch.Generator | None = None
) -> torch.Tensor:
    """(B, V) -> (B, 1) next tokens under `config`."""

    if not config.do_sample:
        return select_greedy(logits)
    filtered = filter_top_p(filter_top_k(scale_temperature(logits, config.temperature),
                                         config.top_k), config.top_p)
    return sample_from_logits(filtered, generator=generator)
