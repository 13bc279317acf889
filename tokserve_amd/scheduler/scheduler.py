"""Deterministic FIFO request scheduler (tokserve/scheduler/scheduler.py).

Admission is first-in first-out under two limits: max_running_requests, and
the paged pool's block count, against which every admitted request reserves
ceil((prompt + max_new_tokens) / block_size) blocks until it completes
(scheduler.py:58-89,136-159). The admission order, and with it every block id
the engine allocates, is therefore a function of the submission order only.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass

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
        self._requests: dict[str, ScheduledRequest] = {}
        self._waiting: deque[ScheduledRequest] = deque()
        self._running: dict[str, ScheduledRequest] = {}
        self._reserved: dict[str, int] = {}

    @property
    def waiting_requests(self) -> tuple[ScheduledRequest, ...]:
        return tuple(self._waiting)

    @property
    def running_requests(self) -> tuple[ScheduledRequest, ...]:
        return tuple(self._running.values())

    @property
    def waiting_count(self) -> int:
        return len(self._waiting)

    @property
    def running_count(self) -> int:
        return len(self._running)

    def submit(self, request: ScheduledRequest) -> None:
        if request.request_id in self._requests:
            raise ValueError("request_id is already registered")
        if request.state is not RequestState.WAITING:
            raise ValueError("submitted request must be waiting")
        self._requests[request.request_id] = request
        self._waiting.append(request)

    def schedule(self) -> ScheduleResult:
        """Admit waiting requests in FIFO order while slots and blocks remain."""

        slots = self.max_running_requests - len(self._running)
        blocks = self._unreserved_blocks()
        admitted: list[ScheduledRequest] = []
        while slots > 0 and self._waiting:
            request = self._waiting[0]
            needed = self._required_blocks(request)
            if needed > blocks:
                break
            self._waiting.popleft()
            request.mark_running()
            self._running[request.request_id] = request
            if needed:
                self._reserved[request.request_id] = needed
                blocks -= needed
            admitted.append(request)
            slots -= 1
        return ScheduleResult(tuple(admitted), len(self._waiting), len(self._running))

    def complete(self, request_id: str, result: GenerationResult | None = None) -> None:
        request = self._get_running(request_id)
        self._release(request_id)
        del self._running[request_id]
        request.mark_finished(result)

    def cancel(self, request_id: str) -> None:
        request = self.get_request(request_id)
        if request.state is RequestState.WAITING:
            self._waiting = deque(r for r in self._waiting if r.request_id != request_id)
            request.cancel()
            return
        if request.state is RequestState.RUNNING:
            self._release(request_id)
            del self._running[request_id]
            request.cancel()
            return
        raise RuntimeError(f"cannot cancel request in state {request.state.value}")

    def get_request(self, request_id: str) -> ScheduledRequest:
        try:
            return self._requests[request_id]
        except KeyError as error:
            raise KeyError("unknown request_id") from error

    def _get_running(self, request_id: str) -> ScheduledRequest:
        try:
            return self._running[request_id]
        except KeyError as error:
            raise RuntimeError("request is not running") from error

    def _required_blocks(self, request: ScheduledRequest) -> int:
        if self.cache_manager is None or request.generation_config.max_new_tokens == 0:
            return 0
        total = len(request.prompt_tokens) + request.generation_config.max_new_tokens
        size = self.cache_manager.storage.block_size
        return (total + size - 1) // size

    def _unreserved_blocks(self) -> int:
        if self.cache_manager is None:
            return 0
        return max(0, self.cache_manager.allocator.num_blocks - sum(self._reserved.values()))

    def _release(self, request_id: str) -> None:
        self._reserved.pop(request_id, None)
        manager = self.cache_manager
        if manager is not None and request_id in manager.active_sequence_ids:
            manager.release_sequence(request_id)
