"""Split the running requests into prefill and decode work (tokserve/batching/plan.py)."""

from __future__ import annotations

from collections.abc import Iterable
from dataclasses import dataclass

from tokserve_amd.scheduler.request import RequestState, ScheduledRequest

__all__ = ["IterationPlan", "build_iteration_plan"]


@dataclass(frozen=True)
class IterationPlan:
    prefill_requests: tuple[ScheduledRequest, ...]
    decode_requests: tuple[ScheduledRequest, ...]

    @property
    def is_empty(self) -> bool:
        return not self.prefill_requests and not self.decode_requests

    @property
    def request_ids(self) -> tuple[str, ...]:
        return tuple(r.request_id for r in (*self.prefill_requests, *self.decode_requests))


def build_iteration_plan(requests: Iterable[ScheduledRequest]) -> IterationPlan:
    """Running, unfinished requests: prefill if their prompt is not cached yet,
    decode if they are decode-ready; order preserved."""

    seen: set[str] = set()
    prefill: list[ScheduledRequest] = []
    decode: list[ScheduledRequest] = []
    for request in requests:
        if request.request_id in seen:
            raise ValueError("iteration plan contains a duplicate request_id")
        seen.add(request.request_id)
        if request.state is not RequestState.RUNNING or request.completion_reason is not None:
            continue
        if not request.prefill_complete:
            prefill.append(request)
        elif request.decode_ready:
            decode.append(request)
    return IterationPlan(tuple(prefill), tuple(decode))
