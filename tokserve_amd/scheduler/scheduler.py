"""Deterministic FIFO request scheduler (tokserve/scheduler/scheduler.py).

Admission is first-in first-out under two limits: free running slots
(max_running_requests) and the paged pool's unreserved blocks, against which
every admitted request reserves ceil((prompt + max_new_tokens) / block_size)
blocks until it leaves (scheduler.py:75-104,146-168). Here one admission
decision is a prefix computation over the head of the queue: the block needs
of the first `free slots` waiting requests, their running sum, and the first
position where that sum passes the unreserved blocks; everything before it is
admitted in queue order, nothing after it (a blocked head request holds back
the queue, as in the reference). Admission order, and with it every block id
the engine allocates, is a function of the submission order only.

The waiting queue is an insertion-ordered dict (FIFO order, O(1) cancellation
by id); reservations are a dict plus their running total.
"""

from __future__ import annotations

from dataclasses import dataclass
from itertools import islice

import numpy as np

from tokserve_amd.engine.paged.manager import PagedKVCacheManager
from tokserve_amd.generation.types import GenerationResult
from tokserve_amd.scheduler.request import RequestState, ScheduledRequest

__all__ = ["ScheduleResult", "RequestScheduler"]


@dataclass(frozen=True)
class ScheduleResult:
    admitted_requests: tuple[ScheduledRequest, ...]
    waiting_count: int
    running_count: int


class RequestScheduler:
    """Waiting and running requests in FIFO order."""

    def __init__(self, *, max_running_requests: int,
                 cache_manager: PagedKVCacheManager | None = None) -> None:
        if max_running_requests < 1:
            raise ValueError("max_running_requests must be positive")
        self.max_running_requests = max_running_requests
        self.cache_manager = cache_manager
        self._known: dict[str, ScheduledRequest] = {}
        self._queue: dict[str, ScheduledRequest] = {}
        self._running: dict[str, ScheduledRequest] = {}
        self._holds: dict[str, int] = {}
        self._held = 0

    # ------------------------------------------------------------ views

    @property
    def waiting_requests(self) -> tuple[ScheduledRequest, ...]:
        return tuple(self._queue.values())

    @property
    def running_requests(self) -> tuple[ScheduledRequest, ...]:
        return tuple(self._running.values())

    @property
    def waiting_count(self) -> int:
        return len(self._queue)

    @property
    def running_count(self) -> int:
        return len(self._running)

    def get_request(self, request_id: str) -> ScheduledRequest:
        request = self._known.get(request_id)
        if request is None:
            raise KeyError("unknown request_id")
        return request

    # ------------------------------------------------------- admission

    def submit(self, request: ScheduledRequest) -> None:
        if request.request_id in self._known:
            raise ValueError("request_id is already registered")
        if request.state is not RequestState.WAITING:
            raise ValueError("submitted request must be waiting")
        self._known[request.request_id] = request
        self._queue[request.request_id] = request

    def schedule(self) -> ScheduleResult:
        """Admit the longest FIFO prefix of the queue that fits the free slots and blocks."""

        slots = self.max_running_requests - len(self._running)
        if slots <= 0 or not self._queue:
            return ScheduleResult((), len(self._queue), len(self._running))
        head = list(islice(self._queue.values(), slots))
        needs = np.fromiter((self._block_need(r) for r in head), dtype=np.int64, count=len(head))
        fits = int(np.searchsorted(np.cumsum(needs), self._unheld_blocks(), side="right"))
        admitted = head[:fits]
        for request, need in zip(admitted, needs[:fits].tolist()):
            del self._queue[request.request_id]
            request.mark_running()
            self._running[request.request_id] = request
            if need:
                self._holds[request.request_id] = need
                self._held += need
        return ScheduleResult(tuple(admitted), len(self._queue), len(self._running))

    def _block_need(self, request: ScheduledRequest) -> int:
        new_tokens = request.generation_config.max_new_tokens
        if self.cache_manager is None or new_tokens == 0:
            return 0
        size = self.cache_manager.storage.block_size
        return -(-(request.sequence_length + new_tokens) // size)

    def _unheld_blocks(self) -> int:
        if self.cache_manager is None:
            return 0
        return max(0, self.cache_manager.allocator.num_blocks - self._held)

    # ---------------------------------------------------------- leaving

    def complete(self, request_id: str, result: GenerationResult | None = None) -> None:
        request = self._running.get(request_id)
        if request is None:
            raise RuntimeError("request is not running")
        self._leave(request_id)
        request.mark_finished(result)

    def cancel(self, request_id: str) -> None:
        request = self.get_request(request_id)
        if request.state is RequestState.WAITING:
            del self._queue[request_id]
        elif request.state is RequestState.RUNNING:
            self._leave(request_id)
        else:
            raise RuntimeError(f"cannot cancel request in state {request.state.value}")
        request.cancel()

    def _leave(self, request_id: str) -> None:
        """A running request stops running: its hold and its cache go back to the pool."""

        self._held -= self._holds.pop(request_id, 0)
        del self._running[request_id]
        manager = self.cache_manager
        if manager is not None and request_id in manager.active_sequence_ids:
            manager.release_sequence(request_id)
