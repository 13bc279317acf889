"""Batched execution of one continuous-batching iteration.

The reference runs each planned request as its own batch-1 forward: prefills
first, in plan order, then decodes (tokserve/batching/execution.py:21-101).
Here the whole iteration is one packed forward (LlamaModel.forward_packed):
every prefill chunk and every decode token in one token stream, one launch
per kernel per layer, logits for the B last tokens only, greedy tokens for
all B sequences from one argmax launch and one device -> host copy.

An iteration runs in three phases:
  1. check   every request and every sequence the iteration will touch is
             checked (states, duplicates, lengths against the model and the
             caches) before anything changes;
  2. reserve inside one StepReservation of the cache manager, prefills open
             their sequences and every sequence begins its append, in plan
             order (prefills, then decodes), so blocks come out of the pool in
             the reference's order and every block id matches its; then the
             packed forward runs and the reservation commits. Any failure in
             this phase (an exhausted pool, a failed launch) rolls the
             reservation back: the pool and every sequence are as before the
             call, and no request has changed;
  3. apply   tokens are appended and the metrics hooks fire, per request in
             the reference's order: for each prefill, prefill_finished and
             token_produced; then token_produced for each decode.
The prefill hooks bracket the forward that serves the prefill, as the
reference's do (execution.py:39-50): prefill_started fires for every prefill
of the iteration, in plan order, just before the packed forward, and
prefill_finished once it has run, so a collector's prefill duration is the
forward's (one forward serves them all, so their starts come together).
Requests with max_new_tokens == 0 complete at prefill without a forward or
hooks, as in the reference.

A decode-only iteration of greedy requests can also run split in two
(launch_decode, then finish): launch checks, reserves and queues the graph
replay with an asynchronous copy of the greedy tokens to pinned host memory,
and keeps the reservation open; commit makes the reserved positions valid;
finish waits for the copy and applies phase 3. Between launch and finish the
host is free, and a launch may take its token ids from the previous launch's
device tokens, so the engine can queue iteration i+1 before it reads back
iteration i.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import torch

from tokserve_amd.batching.graphs import DecodeGraphs
from tokserve_amd.batching.metadata import PackedBatchBuilder, SequenceWork
from tokserve_amd.engine.model import LlamaModel
from tokserve_amd.engine.paged.manager import PagedKVCacheManager, StepReservation
from tokserve_amd.generation.sampling import select_next_token
from tokserve_amd.kernels import ops
from tokserve_amd.scheduler.request import RequestState, ScheduledRequest

__all__ = ["BatchExecutor", "LaunchedDecode", "execute_prefill", "execute_decode"]


@dataclass(frozen=True)
class _Checked:
    """Phase 1's outcome: who runs the forward and who completes without one."""

    no_tokens: tuple[ScheduledRequest, ...]   # prefills with max_new_tokens == 0
    prefill: tuple[ScheduledRequest, ...]
    decode: tuple[ScheduledRequest, ...]
    decode_caches: tuple                       # each decode request's sequence cache
    decode_lengths: tuple[int, ...]            # cached positions of each decode sequence


@dataclass
class LaunchedDecode:
    """A decode-only iteration queued on the GPU whose tokens are not read yet."""

    checked: _Checked
    reservation: StepReservation
    tokens: torch.Tensor         # (B,) int64 greedy tokens, on the device
    host: torch.Tensor           # pinned (>= B,) int64: their copy, valid once `ready` is
    ready: torch.cuda.Event

    @property
    def requests(self) -> tuple[ScheduledRequest, ...]:
        return self.checked.decode


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
        self._token_host: list[torch.Tensor | None] = [None, None]
        self._token_turn = 0

    def execute(self, prefill: Sequence[ScheduledRequest], decode: Sequence[ScheduledRequest],
                *, metrics=None) -> tuple[str, ...]:
        """Advance every request by one step; returns the ids that reached completion."""

        checked = self._check(prefill, decode)
        tokens: list[int] = []
        if checked.prefill or checked.decode:
            with self.manager.reservation() as reservation:
                pre_work, dec_work = self._reserve(reservation, checked)
                if metrics is not None:
                    for request in checked.prefill:
                        metrics.prefill_started(request.request_id)
                tokens = self._forward(pre_work, dec_work, [*checked.prefill, *checked.decode])
                reservation.commit()
        return self._apply(prefill, checked, tokens, metrics)

    # ------------------------------------------------- split decode iteration

    def can_launch(self, decode: Sequence[ScheduledRequest]) -> bool:
        """Whether these decode requests can run as launch_decode / finish."""

        return (self.graphs is not None and bool(decode)
                and not any(r.generation_config.do_sample for r in decode))

    def launch_decode(self, decode: Sequence[ScheduledRequest], *,
                      token_source: torch.Tensor | None = None) -> LaunchedDecode:
        """Phases 1 and 2 of a decode-only iteration up to the queued replay; the
        reservation stays open (commit or discard it). token_source: the (B,) device
        tokens to feed, in `decode` order, instead of each request's last token."""

        checked = self._check((), decode)
        reservation = self.manager.reservation()
        try:
            _, dec_work = self._reserve(reservation, checked)
            _, greedy = self.graphs.run(dec_work, token_source=token_source)
            b = len(dec_work)
            turn = self._token_turn
            self._token_turn ^= 1
            host = self._token_host[turn]
            if host is None or host.numel() < b:
                host = torch.empty(max(b, 256), dtype=torch.int64, pin_memory=True)
                self._token_host[turn] = host
            host[:b].copy_(greedy.view(-1), non_blocking=True)
            ready = torch.cuda.Event()
            ready.record()
        except BaseException:
            reservation.rollback()
            raise
        return LaunchedDecode(checked, reservation, greedy.view(-1), host, ready)

    @staticmethod
    def commit(launched: LaunchedDecode) -> None:
        launched.reservation.commit()

    @staticmethod
    def discard(launched: LaunchedDecode) -> None:
        """Undo a launch that will not be finished: its positions and blocks go back
        (the K/V it writes lands past every sequence's valid length)."""

        launched.reservation.rollback()

    def finish(self, launched: LaunchedDecode, *, metrics=None) -> tuple[str, ...]:
        """Phase 3 of a launched iteration (after commit): its tokens and hooks."""

        launched.ready.synchronize()
        tokens = launched.host[: len(launched.checked.decode)].tolist()
        return self._apply((), launched.checked, tokens, metrics)

    # ----------------------------------------------------------- phase 1

    def _check(self, prefill: Sequence[ScheduledRequest],
               decode: Sequence[ScheduledRequest]) -> _Checked:
        _check_group(prefill, "prefill")
        for request in prefill:
            if request.prefill_complete:
                raise ValueError("request prefill is already complete")
            if request.completion_reason is not None:
                raise ValueError("completed request cannot be prefetched")
        _check_group(decode, "decode")
        for request in decode:
            if not request.decode_ready:
                raise ValueError("decode requests must be decode-ready")
        limit = self.model.config.max_position_embeddings
        runs = tuple(r for r in prefill if r.generation_config.max_new_tokens)
        for request in runs:
            if request.sequence_length > limit:
                raise ValueError("sequence length exceeds max_position_embeddings")
        caches, lengths = [], []
        get = self.manager.get_sequence
        for request in decode:
            cache = get(request.request_id)
            length = cache.current_length
            if length < 1:
                raise ValueError("paged decode requires a populated cache")
            if length >= cache.max_sequence_length:
                raise ValueError("paged cache capacity exceeded")
            caches.append(cache)
            lengths.append(length)
        return _Checked(
            no_tokens=tuple(r for r in prefill if not r.generation_config.max_new_tokens),
            prefill=runs, decode=tuple(decode), decode_caches=tuple(caches),
            decode_lengths=tuple(lengths))

    # ----------------------------------------------------------- phase 2

    def _reserve(self, reservation: StepReservation, checked: _Checked):
        limit = self.model.config.max_position_embeddings
        appends = [(reservation.open(request.request_id, max_sequence_length=limit),
                    request.prompt_array.size) for request in checked.prefill]
        appends.extend((cache, 1) for cache in checked.decode_caches)
        tables = reservation.extend_all(appends)
        n_pre = len(checked.prefill)
        pre_work = [SequenceWork(request.prompt_array, 0, table)
                    for request, table in zip(checked.prefill, tables)]
        dec_work = [SequenceWork((request.last_token,), length, table)
                    for request, length, table in zip(checked.decode, checked.decode_lengths,
                                                      tables[n_pre:])]
        return pre_work, dec_work

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

    # ----------------------------------------------------------- phase 3

    @staticmethod
    def _apply(prefill: Sequence[ScheduledRequest], checked: _Checked, tokens: list[int],
               metrics) -> tuple[str, ...]:
        served = iter(tokens)
        completed: list[str] = []
        for request in prefill:
            if not request.generation_config.max_new_tokens:
                request.mark_prefill_complete()
                completed.append(request.request_id)
                continue
            if metrics is not None:
                metrics.prefill_finished(request.request_id)
            request.mark_prefill_complete()
            _take(request, next(served), metrics, completed)
        for request in checked.decode:
            _take(request, next(served), metrics, completed)
        return tuple(completed)


def _take(request: ScheduledRequest, token: int, metrics, completed: list[str]) -> None:
    request.append_generated_token(token)
    if metrics is not None:
        metrics.token_produced(request.request_id)
    if request.completion_reason is not None:
        completed.append(request.request_id)


def _check_group(requests: Sequence[ScheduledRequest], kind: str) -> None:
    seen: set[str] = set()
    for request in requests:
        if request.request_id in seen:
            raise ValueError(f"{kind} batch contains a duplicate request_id")
        seen.add(request.request_id)
        if request.state is not RequestState.RUNNING:
            raise ValueError(f"{kind} requests must be running")


def _executor_for(model: LlamaModel, manager: PagedKVCacheManager) -> BatchExecutor:
    """The executor of (model, manager), so that callers looping over execute_decode
    reuse its staging buffers and decode graphs. It is kept on the manager itself: the
    two refer to each other, and the cycle (with the pools and graphs it holds) is
    collected once the caller lets go of the manager."""

    executor = getattr(manager, "_batch_executor", None)
    if executor is None or executor.model is not model:
        executor = BatchExecutor(model, manager)
        manager._batch_executor = executor
    return executor


def execute_prefill(model: LlamaModel, manager: PagedKVCacheManager,
                    requests: Sequence[ScheduledRequest], *, metrics=None) -> tuple[str, ...]:
    """Prefill `requests` and select their first tokens (one packed forward)."""

    return _executor_for(model, manager).execute(requests, (), metrics=metrics)


def execute_decode(model: LlamaModel, manager: PagedKVCacheManager,
                   requests: Sequence[ScheduledRequest], *, metrics=None) -> tuple[str, ...]:
    """Advance decode-ready `requests` by one token (one packed forward)."""

    return _executor_for(model, manager).execute((), requests, metrics=metrics)
