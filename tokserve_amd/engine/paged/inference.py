"""One-sequence paged prefill and decode (tokserve/engine/paged/inference.py)."""

from __future__ import annotations

from dataclasses import dataclass

import torch

from tokserve_amd.engine.model import LlamaModel
from tokserve_amd.engine.paged.manager import PagedKVCacheManager
from tokserve_amd.engine.paged.sequence_cache import SequencePagedKVCache

__all__ = ["PagedPrefillResult", "validate_manager", "prefill_paged", "decode_paged"]


@dataclass(frozen=True)
class PagedPrefillResult:
    logits: torch.Tensor
    cache: SequencePagedKVCache


def validate_manager(model: LlamaModel, manager: PagedKVCacheManager) -> None:
    model.validate_storage(manager.storage)


@torch.inference_mode()
def prefill_paged(model: LlamaModel, prompt_ids: torch.Tensor, manager: PagedKVCacheManager, *,
                  sequence_id: str) -> PagedPrefillResult:
    """Run a (1, T) prompt into a newly registered sequence; logits (1, T, V)."""

    if prompt_ids.ndim != 2:
        raise ValueError("prompt_ids must have shape (1, T)")
    if prompt_ids.shape[0] != 1:
        raise ValueError("paged prefill currently supports batch size 1")
    if prompt_ids.shape[1] < 1:
        raise ValueError("prompt must contain at least one token")
    validate_manager(model, manager)
    cache = manager.create_sequence(sequence_id,
                                    max_sequence_length=model.config.max_position_embeddings)
    try:
        logits = model(prompt_ids, paged_cache=cache)
        if cache.current_length != prompt_ids.shape[1]:
            raise RuntimeError("paged prefill length does not match prompt length")
        return PagedPrefillResult(logits=logits, cache=cache)
    except Exception:
        manager.release_sequence(sequence_id)
        raise


@torch.inference_mode()
def decode_paged(model: LlamaModel, token_ids: torch.Tensor,
                 cache: SequencePagedKVCache) -> torch.Tensor:
    """Append exactly one token (1, 1) to a populated sequence; logits (1, 1, V)."""

    if token_ids.ndim != 2 or token_ids.shape != (1, 1):
        raise ValueError("paged decode requires token_ids shaped (1, 1)")
    if cache.current_length < 1:
        raise ValueError("paged decode requires a populated cache")
    if cache.current_length >= cache.max_sequence_length:
        raise ValueError("paged cache capacity exceeded")
    previous = cache.current_length
    logits = model(token_ids, paged_cache=cache)
    if cache.current_length != previous + 1:
        raise RuntimeError("paged decode must increase length by one")
    return logits
