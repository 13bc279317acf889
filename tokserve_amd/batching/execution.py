"""Batched execution of one continuous-batching iteration.

The reference runs each planned request as its own batch-1 forward: prefills
first, in plan order, then decodes (tokserve/batching/execution.py:21-101).
Here the whole iteration is one packed forward (LlamaModel.forward_packed):
every prefill chunk and every decode token in one token stream, one launch
per kernel per layer, logits for the B last tokens only, greedy tokens for
all B sequences from one argmax launch and one device -> host copy.

What stays identical to the reference: block allocation happens in the same
order (each prefill's begin_append in plan order, then each decode's), so
every block id matches; each sequence's positions, causal masking and cached
keys are its own, so its tokens match; requests with max_new_tokens == 0
complete at prefill without a forward; the state transitions and their
checks are the same.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

from tokserve_amd.batching.graphs import DecodeGraphs
from tokserve_amd.batching.metadata import PackedBatchBuilder, SequenceWork
from tokserve_amd.engine.model import LlamaModel
from tokserve_amd.engine.paged.manager import PagedKVCacheManager
from tokserve_amd.generation.sampling import select_next_token
from tokserve_amd.kernels import ops
from tokserve_amd.scheduler.request import RequestState, ScheduledRequest

__all__ = ["BatchExecutor", "execute_prefill", "execute_decode"]


class BatchExecutor:
    """Runs planned prefill and decode requests of one iteration as one packed forward."""

    def __init__(self, model: LlamaModel, manager: PagedKVCacheManager, *,
                 use_graphs: bool = True) -> None:
        model.validate_storage(manager.storage)
        self.model = model
        self.manager = manager
        self.builder = PackedBatchBuilder(manager.storage.device, manager.storage.block_size)
        graphs = DecodeGraphs(model, manager.storage)
        self.graphs = graphs if use_graphs and graphs.supported() else None

    def execute(
        self, prefill: Sequence[ScheduledRequest], decode: Sequence[ScheduledRequest]
    ) -> tuple[str, ...]:
        """Advance every request by one step; returns ids that reached completion."""

        _check_group(prefill, "prefill")
        _check_group(decode, "decode")
        for request in prefill:
            if request.prefill_complete:
                raise ValueError("request prefill is already complete")
            if request.completion_reason is not None:
                raise ValueError("completed request cannot be prefetched")
        for request in decode:
            if not request.decode_ready:
                raise ValueError("decode requests must be decode-ready")

        completed: list[str] = []
        limit = self.model.config.max_position_embeddings
        pre_work: list[tuple[ScheduledRequest, SequenceWork]] = []
        for request in prefill:
            if request.generation_config.max_new_tokens == 0:
                request.mark_prefill_complete()
                completed.append(request.request_id)
                continue
            prompt = request.prompt_tokens
            if len(prompt) > limit:
                raise ValueError("sequence length exceeds max_position_embeddings")
            cache = self.manager.create_sequence(request.request_id, max_sequence_length=limit)
            blocks = cache.reserve(len(prompt))
            pre_work.append((request, SequenceWork(request.prompt_array, 0, blocks)))
        dec_work: list[tuple[ScheduledRequest, SequenceWork]] = []
        caches = []
        for request in decode:
            cache = self.manager.get_sequence(request.request_id)
            length = cache.current_length
            if length < 1:
                raise ValueError("paged decode requires a populated cache")
            if length >= cache.max_sequence_length:
                raise ValueError("paged cache capacity exceeded")
            blocks = cache.reserve(1)
            dec_work.append((request, SequenceWork((request.last_token,), length, blocks)))
            caches.append(cache)
        work = pre_work + dec_work
        if not work:
            return tuple(completed)

        tokens = self._forward([w for _, w in pre_work], [w for _, w in dec_work],
                               [r for r, _ in work])
        for request, _ in pre_work:
            self.manager.get_sequence(request.request_id).commit()
        for cache in caches:
            cache.commit()
        for index, (request, _) in enumerate(work):
            if index < len(pre_work):
                request.mark_prefill_complete()
            request.append_generated_token(tokens[index])
            if request.completion_reason is not None:
                completed.append(request.request_id)
        return tuple(completed)

    def _forward(self, prefill: list[SequenceWork], decode: list[SequenceWork],
                 requests: list[ScheduledRequest]) -> list[int]:
        """One packed forward of the iteration; the next token of every sequence."""

        if self.graphs is not None and not prefill:
            logits, greedy = self.graphs.run(decode)
            return self._select(logits, requests, greedy)
        batch = self.builder.build(prefill, decode)
        logits = self.model.forward_packed(batch, self.manager.storage)
        return self._select(logits, requests)

    @staticmethod
    def _select(logits: torch.Tensor, requests: list[ScheduledRequest],
                greedy: torch.Tensor | None = None) -> list[int]:
        """Greedy rows from one argmax launch; sampled rows one by one with their
        own generators; one device -> host copy."""

        chosen = ops.greedy_argmax(logits).view(-1) if greedy is None else greedy.clone()
        for row, request in enumerate(requests):
            config = request.generation_config
            if config.do_sample:
                chosen[row] = select_next_token(logits[row : row + 1], config,
                                                generator=request.sampling_generator).view(())
        return chosen.tolist()


def _check_group(requests: Sequence[ScheduledRequest], kind: str) -> None:
    seen: set[str] = set()
    for request in requests:
        if request.request_id in seen:
            raise ValueError(f"{kind} batch contains a duplicate request_id")
        seen.add(request.request_id)
        if request.state is not RequestState.RUNNING:
            raise ValueError(f"{kind} requests must be running")


def execute_prefill(model: LlamaModel, manager: PagedKVCacheManager,
                    requests: Sequence[ScheduledRequest]) -> tuple[str, ...]:
    """Prefill `requests` and select their first tokens (one packed forward)."""

    return BatchExecutor(model, manager).execute(requests, ())


def execute_decode(model: LlamaModel, manager: PagedKVCacheManager,
                   requests: Sequence[ScheduledRequest]) -> tuple[str, ...]:
    """Advance decode-ready `requests` by one token (one packed forward)."""

    return BatchExecutor(model, manager).execute((), requests)
