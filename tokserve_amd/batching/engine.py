"""Iteration-level continuous batching (tokserve/batching/engine.py).

One step is four phases: admit (the scheduler's FIFO admission under the slot
and block limits), plan (running requests split into prefill and decode
work), run (the BatchExecutor's single packed forward) and retire (requests
that reached EOS or max_new_tokens complete and give their blocks back). The
step's IterationRecord (admitted, prefill, decode, completed and still-active
ids) and the metrics hooks are the reference's: request_admitted per admitted
request, the executor's prefill/token hooks, complete_request per completed
request and record_iteration per step (engine.py:65-131).

With overlap_decode=True, decode-only iterations of greedy requests run as a
launch and a finish (BatchExecutor.launch_decode / finish), and when the
next iteration is already known at launch time, it is queued on the GPU
before this one's tokens are read back: the next plan is this plan again
when nothing waits for admission, every running request decodes, none has
an EOS token and none reaches max_new_tokens in this iteration. Its token
ids come straight from this iteration's device tokens, so the host's
bookkeeping of iteration i (token readback, hooks, retirement, record) runs
while the GPU computes iteration i+1. Records, hooks, tokens and block ids
are those of the sequential engine; what differs is only visible between
two step() calls: the queued iteration's positions are reserved (an open
append per sequence, and any new block it needed). A step that finds the
scheduler changed since (a submission, a cancellation) discards the queued
iteration, returning those positions and blocks, and runs sequentially.
"""

from __future__ import annotations

from dataclasses import dataclass

from tokserve_amd.batching.execution import BatchExecutor, LaunchedDecode
from tokserve_amd.batching.plan import IterationPlan, build_iteration_plan
from tokserve_amd.engine.model import LlamaModel
from tokserve_amd.engine.paged.manager import PagedKVCacheManager
from tokserve_amd.generation.types import GenerationResult
from tokserve_amd.scheduler.request import ScheduledRequest
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

    @property
    def made_progress(self) -> bool:
        return bool(self.admitted_ids or self.prefill_ids or self.decode_ids
                    or self.completed_ids)


def _ids(requests: tuple[ScheduledRequest, ...] | list[ScheduledRequest]) -> tuple[str, ...]:
    return tuple(request.request_id for request in requests)


class ContinuousBatchEngine:
    """Advances dynamically changing requests one iteration at a time."""

    def __init__(self, model: LlamaModel, scheduler: RequestScheduler,
                 cache_manager: PagedKVCacheManager, *, metrics=None,
                 overlap_decode: bool = False) -> None:
        if scheduler.cache_manager is not cache_manager:
            raise ValueError("scheduler and engine must share the cache manager")
        self.model = model
        self.scheduler = scheduler
        self.cache_manager = cache_manager
        self.metrics = metrics
        self.overlap_decode = overlap_decode
        self.executor = BatchExecutor(model, cache_manager)
        self._history: list[IterationRecord] = []
        self._results: list[GenerationResult] = []
        self._queued: LaunchedDecode | None = None

    @property
    def history(self) -> tuple[IterationRecord, ...]:
        return tuple(self._history)

    @property
    def results(self) -> tuple[GenerationResult, ...]:
        return tuple(self._results)

    def step(self) -> IterationRecord:
        admitted = self._admit()
        plan = build_iteration_plan(self.scheduler.running_requests)
        launched = self._take_queued(admitted, plan)
        if launched is None and self.overlap_decode and not plan.prefill_requests \
                and self.executor.can_launch(plan.decode_requests):
            launched = self.executor.launch_decode(plan.decode_requests)
        if launched is None:
            completed = self.executor.execute(plan.prefill_requests, plan.decode_requests,
                                              metrics=self.metrics)
        else:
            self.executor.commit(launched)
            if self._next_plan_is(plan):
                try:
                    self._queued = self.executor.launch_decode(plan.decode_requests,
                                                               token_source=launched.tokens)
                except Exception:  # the next step runs it again and raises there
                    self._queued = None
            completed = self.executor.finish(launched, metrics=self.metrics)
        retired = self._retire(completed)
        return self._record(admitted, plan, retired)

    def _take_queued(self, admitted, plan: IterationPlan) -> LaunchedDecode | None:
        """The iteration queued by the previous step, if it is still this step's plan."""

        queued, self._queued = self._queued, None
        if queued is None:
            return None
        same = (not admitted and not plan.prefill_requests
                and len(queued.requests) == len(plan.decode_requests)
                and all(a is b for a, b in zip(queued.requests, plan.decode_requests)))
        if same:
            return queued
        self.executor.discard(queued)
        return None

    def _next_plan_is(self, plan: IterationPlan) -> bool:
        """Whether the iteration after this one is this plan again (see the module
        docstring), so that it can be queued now."""

        decode = plan.decode_requests
        if self.scheduler.waiting_count or len(decode) != self.scheduler.running_count:
            return False
        for request in decode:
            config = request.generation_config
            if config.eos_token_id is not None or \
                    request.num_generated_tokens + 1 >= config.max_new_tokens:
                return False
        return True

    def _admit(self) -> tuple[ScheduledRequest, ...]:
        admitted = self.scheduler.schedule().admitted_requests
        if self.metrics is not None:
            for request in admitted:
                self.metrics.request_admitted(request.request_id)
        return admitted

    def _retire(self, completed: tuple[str, ...]) -> list[ScheduledRequest]:
        """Complete, in running order, the requests the iteration finished."""

        if not completed:
            return []
        done = set(completed)
        finished = [r for r in self.scheduler.running_requests if r.request_id in done]
        for request in finished:
            result = request.build_result()
            self.scheduler.complete(request.request_id, result)
            if self.metrics is not None:
                self.metrics.complete_request(request.request_id, result.stop_reason)
            self._results.append(result)
        return finished

    def _record(self, admitted, plan: IterationPlan, retired) -> IterationRecord:
        record = IterationRecord(
            iteration=len(self._history), admitted_ids=_ids(admitted),
            prefill_ids=_ids(plan.prefill_requests), decode_ids=_ids(plan.decode_requests),
            completed_ids=_ids(retired), active_ids=_ids(self.scheduler.running_requests))
        self._history.append(record)
        if self.metrics is not None:
            self.metrics.record_iteration(prefill_requests=len(plan.prefill_requests),
                                          decode_requests=len(plan.decode_requests))
        return record

    def run_until_idle(self, *, max_iterations: int = 1_000) -> tuple[GenerationResult, ...]:
        """Step until nothing waits or runs; stalls and runaway loops raise."""

        if max_iterations < 1:
            raise ValueError("max_iterations must be positive")
        for _ in range(max_iterations):
            if not (self.scheduler.waiting_count or self.scheduler.running_count):
                return self.results
            if not self.step().made_progress:
                raise RuntimeError("continuous batching cannot make progress")
        if self.scheduler.waiting_count or self.scheduler.running_count:
            raise RuntimeError("continuous batching exceeded max_iterations")
        return self.results
