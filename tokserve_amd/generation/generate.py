"""One-sequence generation without a cache (tokserve/generation/generate.py).

`generate` recomputes the whole sequence every step; the prompt checks and the
seeded sampling generator are shared with generation.paged_generate.
"""

from __future__ import annotations

import torch

from tokserve_amd.engine.model import LlamaModel
from tokserve_amd.generation.sampling import select_next_token
from tokserve_amd.generation.types import GenerationConfig, GenerationResult, StopReason

__all__ = ["generate"]

_INTEGER_DTYPES = (torch.int8, torch.int16, torch.int32, torch.int64, torch.uint8)


def _check_prompt(input_ids: torch.Tensor) -> None:
    if input_ids.ndim != 2:
        raise ValueError("input_ids must have shape (1, T)")
    if input_ids.shape[0] != 1:
        raise ValueError("generation currently supports batch size 1")
    if input_ids.shape[1] < 1:
        raise ValueError("input_ids must contain at least one token")
    if input_ids.dtype not in _INTEGER_DTYPES:
        raise TypeError("input_ids must contain integers")


def _generator(input_ids: torch.Tensor, config: GenerationConfig) -> torch.Generator | None:
    if config.do_sample and config.seed is not None:
        generator = torch.Generator(device=input_ids.device)
        generator.manual_seed(config.seed)
        return generator
    return None


@torch.inference_mode()
def generate(model: LlamaModel, input_ids: torch.Tensor,
             config: GenerationConfig) -> GenerationResult:
    _check_prompt(input_ids)
    generator = _generator(input_ids, config)
    sequence = input_ids.clone()
    new_tokens: list[torch.Tensor] = []
    stop: StopReason = "max_new_tokens"
    for _ in range(config.max_new_tokens):
        logits = model(sequence)
        token = select_next_token(logits[:, -1, :], config, generator=generator).to(sequence.dtype)
        sequence = torch.cat((sequence, token), dim=1)
        new_tokens.append(token)
        if config.eos_token_id is not None and int(token.item()) == config.eos_token_id:
            stop = "eos"
            break
    generated = torch.cat(new_tokens, dim=1) if new_tokens else input_ids.new_empty((1, 0))
    return GenerationResult(token_ids=sequence, generated_token_ids=generated, stop_reason=stop)
