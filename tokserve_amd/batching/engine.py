"""Iteration-level continuous batching (tokserve/batching/engine.py).

Each step: the scheduler admits waiting requests (FIFO under the slot and
block limits), the running requests are planned into prefill and decode
work, the BatchExecutor runs all of it as one packed forward, and requests
that reached EOS or max_new_tokens are completed (their blocks released).
The IterationRecord of every step (admitted, prefill, decode, completed and
still-active ids) is the reference's.
"""

from __future__ import annotations

from dataclasses import dataclass

from tokserve_amd.batching.execution import BatchExecutor
from tokserve_amd.batching.plan import build_iteration_plan
from tokserve_amd.engine.model import LlamaModel
from tokserve_amd.engine.paged.manager import PagedKVCacheManager
from tokserve_amd.generation.types import GenerationResult
from tokserve_amd.scheduler.scheduler import RequestScheduler

__all__ = ["IterationRecord", "ContinuousBatchEngine"]


@dataclass(frozen=True)
class IterationRecord:
    iteration: int
    admitted_ids: tuple[str, ...]
    prefill_ids: tuple[str, ...]
    decode_ids: tuple[str, ...]
    completed_ids: tuple[str, ...]
    active_ids: tuple[str, ...]


class ContinuousBatchEngine:
    """Advances dynamically changing requests one iteration at a time."""

    def __init__(self, model: LlamaModel, scheduler: RequestScheduler,
                 cache_manager: PagedKVCacheManager) -> None:
        if scheduler.cache_manager is not cache_manager:
            raise ValueError("scheduler and engine must share the cache manager")
        self.model = model
        self.scheduler = scheduler
        self.cache_manager = cache_manager
        self.executor = BatchExecutor(model, cache_manager)
        self._iteration = 0
        self._history: list[IterationRecord] = []
        self._results: list[GenerationResult] = []

    @property
    def history(self) -> tuple[IterationRecord, ...]:
        return tuple(self._history)

    @property
    def results(self) -> tuple[GenerationResult, ...]:
        return tuple(self._results)

    def step(self) -> IterationRecord:
        admitted = self.scheduler.schedule().admitted_requests
        plan = build_iteration_plan(self.scheduler.running_requests)
        self.executor.execute(plan.prefill_requests, plan.decode_requests)
        completed: list[str] = []
        for request in self.scheduler.running_requests:
            if request.completion_reason is None:
                continue
            result = request.build_result()
            self.scheduler.complete(request.request_id, result)
            self._results.append(result)
            completed.append(request.request_id)
        record = IterationRecord(
            iteration=self._iteration,
            admitted_ids=tuple(r.request_id for r in admitted),
            prefill_ids=tuple(r.request_id for r in plan.prefill_requests),
            decode_ids=tuple(r.request_id for r in plan.decode_requests),
            completed_ids=tuple(completed),
            active_ids=tuple(r.request_id for r in self.scheduler.running_requests),
        )
        self._history.append(record)
        self._iteration += 1
        return record

    def run_until_idle(self, *, max_iterations: int = 1_000) -> tuple[GenerationResult, ...]:
        if max_iterations < 1:
            raise ValueError("max_iterations must be positive")
        iterations = 0
        while self.scheduler.waiting_count or self.scheduler.running_count:
            if iterations >= max_iterations:
                raise RuntimeError("continuous batching exceeded max_iterations")
            record = self.step()
            iterations += 1
            if not (record.admitted_ids or record.prefill_ids or record.decode_ids
                    or record.completed_ids):
                raise RuntimeError("continuous batching cannot make progress")
        return self.results
