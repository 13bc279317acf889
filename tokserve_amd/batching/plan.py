"""Prefill and decode work of one iteration (tokserve/batching/plan.py).

Each running request that has not completed is in exactly one phase: PREFILL
(its prompt is not in the cache yet) or DECODE (prefilled, with a token to
feed); anything else sits the iteration out. The plan keeps the given order
within each phase, so the batched forward packs prefill chunks first, in
admission order, then the decode rows.
"""

from __future__ import annotations

from collections.abc import Iterable
from dataclasses import dataclass
from enum import Enum

from tokserve_amd.scheduler.request import RequestState, ScheduledRequest

__all__ = ["IterationPlan", "build_iteration_plan"]


class _Phase(Enum):
    IDLE = 0
    PREFILL = 1
    DECODE = 2


def _phase(request: ScheduledRequest) -> _Phase:
    if request.state is not RequestState.RUNNING or request.completion_reason is not None:
        return _Phase.IDLE
    if not request.prefill_complete:
        return _Phase.PREFILL
    return _Phase.DECODE if request.decode_ready else _Phase.IDLE


@dataclass(frozen=True)
class IterationPlan:
    prefill_requests: tuple[ScheduledRequest, ...]
    decode_requests: tuple[ScheduledRequest, ...]

    @property
    def is_empty(self) -> bool:
        return not (self.prefill_requests or self.decode_requests)

    @property
    def request_ids(self) -> tuple[str, ...]:
        """Every planned id: prefill work first, then decode work."""

        return tuple(r.request_id for r in self.prefill_requests + self.decode_requests)


def build_iteration_plan(requests: Iterable[ScheduledRequest]) -> IterationPlan:
    """Group the running requests by phase, keeping their order within a phase."""

    groups: dict[_Phase, list[ScheduledRequest]] = {phase: [] for phase in _Phase}
    ids: set[str] = set()
    for request in requests:
        if request.request_id in ids:
            raise ValueError("iteration plan contains a duplicate request_id")
        ids.add(request.request_id)
        groups[_phase(request)].append(request)
    return IterationPlan(tuple(groups[_Phase.PREFILL]), tuple(groups[_Phase.DECODE]))
