"""One-sequence paged prefill and decode (tokserve/engine/paged/inference.py).

These are the reference's single-request entry points: a prompt (1, T) into a
newly registered sequence, or one token (1, 1) onto a populated one, each a
`LlamaModel.forward` with the sequence's paged cache (begin/finish append
bracket the layers, each layer's K/V written with one KV-append launch). The
serving engine uses the batched executor instead (batching/execution.py); these
remain for callers of the reference API and for the paged generation loop.
A prefill that fails for any reason takes its new sequence with it, as the
reference's does (inference.py:71-79).
"""

from __future__ import annotations

from contextlib import contextmanager
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
    """The manager's pool fits the model (layers, KV heads, head_dim, device, dtype)."""

    model.validate_storage(manager.storage)


@contextmanager
def _sequence_released_on_error(manager: PagedKVCacheManager, sequence_id: str):
    try:
        yield
    except Exception:
        manager.release_sequence(sequence_id)
        raise


def _check_tokens(tokens: torch.Tensor, rules: tuple[tuple[bool, str], ...]) -> None:
    for failed, message in rules:
        if failed:
            raise ValueError(message)


@torch.inference_mode()
def prefill_paged(model: LlamaModel, prompt_ids: torch.Tensor, manager: PagedKVCacheManager, *,
                  sequence_id: str) -> PagedPrefillResult:
    """Run a (1, T) prompt into a newly registered sequence; logits (1, T, V)."""

    _check_tokens(prompt_ids, (
        (prompt_ids.ndim != 2, "prompt_ids must have shape (1, T)"),
        (prompt_ids.ndim == 2 and prompt_ids.shape[0] != 1,
         "paged prefill currently supports batch size 1"),
        (prompt_ids.ndim == 2 and prompt_ids.shape[1] < 1,
         "prompt must contain at least one token"),
    ))
    validate_manager(model, manager)
    limit = model.config.max_position_embeddings
    cache = manager.create_sequence(sequence_id, max_sequence_length=limit)
    with _sequence_released_on_error(manager, sequence_id):
        logits = model(prompt_ids, paged_cache=cache)
        if cache.current_length != prompt_ids.shape[1]:
            raise RuntimeError("paged prefill length does not match prompt length")
    return PagedPrefillResult(logits=logits, cache=cache)


@torch.inference_mode()
def decode_paged(model: LlamaModel, token_ids: torch.Tensor,
                 cache: SequencePagedKVCache) -> torch.Tensor:
    """Append exactly one token (1, 1) to a populated sequence; logits (1, 1, V)."""

    before = cache.current_length if token_ids.shape == (1, 1) else 0
    _check_tokens(token_ids, (
        (token_ids.shape != (1, 1), "paged decode requires token_ids shaped (1, 1)"),
        (before < 1, "paged decode requires a populated cache"),
        (before >= cache.max_sequence_length, "paged cache capacity exceeded"),
    ))
    logits = model(token_ids, paged_cache=cache)
    if cache.current_length != before + 1:
        raise RuntimeError("paged decode must increase length by one")
    if logits.shape[:2] != token_ids.shape:
        raise RuntimeError("paged decode logits must match token_ids dimensions")
    return logits
