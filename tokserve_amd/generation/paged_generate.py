"""One-sequence generation over a paged KV cache (tokserve/generation/paged_generate.py:18).

The prompt goes through prefill_paged into a new sequence of the cache manager,
each further token through decode_paged (one query over the sequence's pages),
and the sequence's physical blocks go back to the pool when generation ends.
"""

from __future__ import annotations

import torch

from tokserve_amd.engine.model import LlamaModel
from tokserve_amd.engine.paged.inference import decode_paged, prefill_paged
from tokserve_amd.engine.paged.manager import PagedKVCacheManager
from tokserve_amd.generation.generate import _check_prompt, _generator
from tokserve_amd.generation.sampling import select_next_token
from tokserve_amd.generation.types import GenerationConfig, GenerationResult, StopReason

__all__ = ["generate_with_paged_cache"]


@torch.inference_mode()
def generate_with_paged_cache(model: LlamaModel, input_ids: torch.Tensor,
                              config: GenerationConfig, manager: PagedKVCacheManager, *,
                              sequence_id: str) -> GenerationResult:
    """Generate one sequence through a paged sequence of `manager`: prefill the prompt,
    then decode one token at a time; the sequence's blocks are released at the end,
    also when a step raises."""

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
        return GenerationResult(token_ids=sequence,
                                generated_token_ids=torch.cat(new_tokens, dim=1),
                                stop_reason=stop)
    finally:
        if prefill is not None:
            manager.release_sequence(sequence_id)
