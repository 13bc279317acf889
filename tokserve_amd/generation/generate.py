"""One-sequence generation loops (tokserve/generation/generate.py, paged_generate.py).

`generate` recomputes the whole sequence every step (no cache);
`generate_with_paged_cache` prefills into a paged sequence and decodes one
token at a time, releasing the sequence's blocks at the end.
"""

from __future__ import annotations

import torch

from tokserve_amd.engine.model import LlamaModel
from tokserve_amd.engine.paged.inference import decode_paged, prefill_paged
from tokserve_amd.engine.paged.manager import PagedKVCacheManager
from tokserve_amd.generation.sampling import select_next_token
from tokserve_amd.generation.types import GenerationConfig, GenerationResult, StopReason

__all__ = ["generate", "generate_with_paged_cache"]

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


@torch.inference_mode()
def generate_with_paged_cache(model: LlamaModel, input_ids: torch.Tensor, config: GenerationConfig,
                              manager: PagedKVCacheManager, *, sequence_id: str) -> GenerationResult:
    _check_prompt(input_ids)
    if config.max_new_tokens == 0:
        return GenerationResult(token_ids=input_ids.clone(),
                                generated_token_ids=input_ids.new_empty((1, 0)),
                                stop_reason="max_new_tokens")
    if input_ids.shape[1] + config.max_new_tokens > model.config.max_position_embeddings:
        raise ValueError("prompt and generated tokens exceed max_position_embeddings")
    generator = _generator(input_ids, config)
    prefill = None
    try:
        prefill = prefill_paged(model, input_ids, manager, sequence_id=sequence_id)
        logits = prefill.logits
        sequence = input_ids.clone()
        new_tokens: list[torch.Tensor] = []
        stop: StopReason = "max_new_tokens"
        for step in range(config.max_new_tokens):
            token = select_next_token(logits[:, -1, :], config,
                                      generator=generator).to(sequence.dtype)
            sequence = torch.cat((sequence, token), dim=1)
            new_tokens.append(token)
            if config.eos_token_id is not None and int(token.item()) == config.eos_token_id:
                stop = "eos"
                break
            if step + 1 < config.max_new_tokens:
                logits = decode_paged(model, token, prefill.cache)
        return GenerationResult(token_ids=sequence, generated_token_ids=torch.cat(new_tokens, dim=1),
                                stop_reason=stop)
    finally:
        if prefill is not None:
            manager.release_sequence(sequence_id)
