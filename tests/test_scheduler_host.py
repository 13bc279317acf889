"""Request lifecycle, FIFO scheduler and iteration plan (CPU): the behaviour the reference's
unit tests fix, restated against this package's classes. Sources:
tests/unit/scheduler/test_{request,iterative_request,scheduler_queue,scheduler_admission,
scheduler_lifecycle,scheduler_pressure}.py and tests/unit/batching/test_plan.py.
"""

import pytest
import torch
from torch.testing import assert_close

from tokserve_amd.batching.plan import build_iteration_plan
from tokserve_amd.engine.paged.manager import PagedKVCacheManager
from tokserve_amd.generation.types import GenerationConfig
from tokserve_amd.scheduler.request import RequestState, ScheduledRequest
from tokserve_amd.scheduler.scheduler import RequestScheduler


def _request(rid="request", prompt=(1, 2), max_new_tokens=3, eos=None):
    return ScheduledRequest(rid, torch.tensor([list(prompt)], dtype=torch.int64),
                            GenerationConfig(max_new_tokens=max_new_tokens, eos_token_id=eos))


def _manager(num_blocks):
    return PagedKVCacheManager(num_layers=1, num_blocks=num_blocks, num_key_value_heads=1,
                               block_size=2, head_dim=2, device=torch.device("cpu"),
                               dtype=torch.float32)


def _ids(requests):
    return tuple(r.request_id for r in requests)


# Request (test_request.py, test_iterative_request.py)

def test_request_lifecycle_transitions() -> None:
    request = _request("request-1", (1, 2, 3), 2)
    assert request.state is RequestState.WAITING and request.generated_token_ids.shape == (1, 0)
    with pytest.raises(RuntimeError, match="must be running"):
        request.mark_finished()
    request.mark_running()
    assert (request.prefill_complete, request.decode_ready) == (False, False)
    assert request.sequence_length == 3 and request.num_generated_tokens == 0
    with pytest.raises(RuntimeError, match="prefill must complete"):
        request.append_generated_token(torch.tensor([[4]]))
    request.mark_prefill_complete()
    with pytest.raises(RuntimeError, match="already complete"):
        request.mark_prefill_complete()
    request.append_generated_token(torch.tensor([[4]], dtype=torch.int64))
    assert request.decode_ready and request.sequence_length == 4
    assert_close(request.next_input_token, torch.tensor([[4]]))
    request.mark_finished()
    assert request.state is RequestState.FINISHED
    assert_close(request.generated_token_ids, torch.tensor([[4]]))
    with pytest.raises(RuntimeError, match="must be waiting"):
        request.mark_running()
    with pytest.raises(RuntimeError, match="not decode-ready"):
        _request().next_input_token


def test_completion_reasons_and_results() -> None:
    by_count = _request(max_new_tokens=2)
    by_count.mark_running()
    by_count.mark_prefill_complete()
    by_count.append_generated_token(torch.tensor([[3]]))
    by_count.append_generated_token(torch.tensor([[4]]))
    assert by_count.completion_reason == "max_new_tokens" and not by_count.decode_ready
    result = by_count.build_result()
    assert_close(result.token_ids, torch.tensor([[1, 2, 3, 4]]))
    assert result.stop_reason == "max_new_tokens"
    by_eos = _request(max_new_tokens=5, eos=3)
    by_eos.mark_running()
    by_eos.mark_prefill_complete()
    by_eos.append_generated_token(torch.tensor([[3]]))
    assert by_eos.completion_reason == "eos" and by_eos.num_generated_tokens == 1
    assert by_eos.build_result().stop_reason == "eos"
    zero = _request(max_new_tokens=0)
    zero.mark_running()
    zero.mark_prefill_complete()
    assert zero.completion_reason == "max_new_tokens" and zero.generated_token_ids.shape == (1, 0)
    first, second = _request("A"), _request("B")
    for r, token in ((first, 5), (second, 7)):
        r.mark_running()
        r.mark_prefill_complete()
        r.append_generated_token(torch.tensor([[token]]))
    assert first.generated_token_ids.tolist() == [[5]] and second.generated_token_ids.tolist() == [[7]]


def test_waiting_and_running_requests_can_be_cancelled() -> None:
    waiting, running = _request("w"), _request("r")
    waiting.cancel()
    running.mark_running()
    running.cancel()
    assert waiting.state is RequestState.CANCELLED and running.state is RequestState.CANCELLED


@pytest.mark.parametrize(("rid", "ids", "message"), [
    ("", torch.tensor([[1]]), "request_id must be nonempty"),
    ("bad-rank", torch.tensor([1]), r"input_ids must have shape \(1, T\)"),
    ("empty", torch.empty((1, 0), dtype=torch.int64), "input_ids must contain at least one token"),
    ("float", torch.tensor([[1.0]]), "input_ids must contain integers"),
])
def test_invalid_requests_are_rejected(rid, ids, message) -> None:
    with pytest.raises((TypeError, ValueError), match=message):
        ScheduledRequest(rid, ids, GenerationConfig(max_new_tokens=1))


# Scheduler queue and admission (test_scheduler_queue.py, test_scheduler_admission.py)

def test_queue_order_duplicates_and_snapshots() -> None:
    scheduler = RequestScheduler(max_running_requests=2)
    assert scheduler.waiting_requests == () and scheduler.running_requests == ()
    with pytest.raises(KeyError, match="unknown request_id"):
        scheduler.get_request("missing")
    for rid in "ABC":
        scheduler.submit(_request(rid, (1,), 1))
    assert _ids(scheduler.waiting_requests) == ("A", "B", "C")
    assert isinstance(scheduler.waiting_requests, tuple)
    assert (scheduler.waiting_count, scheduler.running_count) == (3, 0)
    with pytest.raises(ValueError, match="already registered"):
        scheduler.submit(_request("A", (1,), 1))
    assert scheduler.waiting_count == 3
    with pytest.raises(ValueError, match="must be positive"):
        RequestScheduler(max_running_requests=0)


@pytest.mark.parametrize(("capacity", "submitted", "admitted"), [
    (1, "AB", "A"), (2, "ABC", "AB"), (3, "A", "A")])
def test_fifo_admission_up_to_capacity(capacity, submitted, admitted) -> None:
    scheduler = RequestScheduler(max_running_requests=capacity)
    for rid in submitted:
        scheduler.submit(_request(rid, (1,), 1))
    result = scheduler.schedule()
    assert _ids(result.admitted_requests) == tuple(admitted)
    assert result.running_count == len(admitted)
    assert result.waiting_count == len(submitted) - len(admitted)
    assert all(scheduler.get_request(r).state is RequestState.RUNNING for r in admitted)


def test_empty_and_repeated_scheduling_are_safe() -> None:
    scheduler = RequestScheduler(max_running_requests=1)
    assert scheduler.schedule().admitted_requests == ()
    scheduler.submit(_request("A", (1,), 1))
    scheduler.submit(_request("B", (1,), 1))
    scheduler.schedule()
    repeated = scheduler.schedule()
    assert repeated.admitted_requests == ()
    assert (repeated.running_count, repeated.waiting_count) == (1, 1)


# Lifecycle (test_scheduler_lifecycle.py)

def test_completion_restores_capacity_and_releases_the_cache() -> None:
    scheduler = RequestScheduler(max_running_requests=1)
    scheduler.submit(_request("A", (1, 2), 2))
    scheduler.submit(_request("B", (1, 2), 2))
    scheduler.schedule()
    scheduler.complete("A")
    assert _ids(scheduler.schedule().admitted_requests) == ("B",)
    assert scheduler.get_request("A").state is RequestState.FINISHED
    with pytest.raises(RuntimeError, match="not running"):
        scheduler.complete("A")
    with pytest.raises(KeyError, match="unknown request_id"):
        scheduler.cancel("missing")

    manager = _manager(4)
    scheduler = RequestScheduler(max_running_requests=1, cache_manager=manager)
    scheduler.submit(_request("A", (1, 2), 2))
    scheduler.schedule()
    manager.create_sequence("A", max_sequence_length=4).begin_append(2)
    assert manager.allocator.allocated_count == 1
    scheduler.complete("A")
    assert manager.active_sequence_ids == () and manager.allocator.allocated_count == 0


def test_waiting_and_running_cancellation() -> None:
    scheduler = RequestScheduler(max_running_requests=1)
    scheduler.submit(_request("A", (1, 2), 2))
    scheduler.submit(_request("B", (1, 2), 2))
    scheduler.schedule()
    scheduler.cancel("B")
    scheduler.cancel("A")
    assert scheduler.get_request("A").state is RequestState.CANCELLED
    assert scheduler.get_request("B").state is RequestState.CANCELLED
    assert (scheduler.running_count, scheduler.waiting_count) == (0, 0)


# Cache pressure (test_scheduler_pressure.py; blocks of 2, reservations of
# ceil((prompt + max_new_tokens) / 2) blocks)

def test_resource_pressure_keeps_request_waiting_atomically() -> None:
    manager = _manager(2)
    scheduler = RequestScheduler(max_running_requests=2, cache_manager=manager)
    large = _request("large", range(3), 2)  # 3 blocks > 2
    scheduler.submit(large)
    assert scheduler.schedule().admitted_requests == ()
    assert large.state is RequestState.WAITING
    assert (scheduler.waiting_count, scheduler.running_count) == (1, 0)
    assert manager.allocator.allocated_count == 0


def test_fifo_does_not_bypass_blocked_earlier_request() -> None:
    scheduler = RequestScheduler(max_running_requests=2, cache_manager=_manager(2))
    scheduler.submit(_request("A", range(3), 2))
    scheduler.submit(_request("B", range(1), 1))
    assert scheduler.schedule().admitted_requests == ()
    assert _ids(scheduler.waiting_requests) == ("A", "B")


def test_completion_allows_next_fifo_request_to_run() -> None:
    scheduler = RequestScheduler(max_running_requests=1, cache_manager=_manager(3))
    scheduler.submit(_request("A", range(2), 2))
    scheduler.submit(_request("B", range(1), 1))
    scheduler.submit(_request("C", range(1), 1))
    first = scheduler.schedule()
    scheduler.complete("A")
    second = scheduler.schedule()
    scheduler.complete("B")
    third = scheduler.schedule()
    assert [_ids(r.admitted_requests) for r in (first, second, third)] == [("A",), ("B",), ("C",)]
    assert [scheduler.get_request(r).state for r in "ABC"] == [
        RequestState.FINISHED, RequestState.FINISHED, RequestState.RUNNING]


# Iteration plan (tests/unit/batching/test_plan.py)

def _running(rid, decode_token=None):
    request = _request(rid)
    request.mark_running()
    if decode_token is not None:
        request.mark_prefill_complete()
        request.append_generated_token(torch.tensor([[decode_token]]))
    return request


def test_iteration_plan_splits_and_orders_requests() -> None:
    empty = build_iteration_plan(())
    assert (empty.prefill_requests, empty.decode_requests, empty.request_ids) == ((), (), ())
    assert empty.is_empty
    prefills = build_iteration_plan([_running(r) for r in "ABC"])
    assert _ids(prefills.prefill_requests) == ("A", "B", "C") and prefills.decode_requests == ()
    decodes = build_iteration_plan([_running("A", 3), _running("B", 4)])
    assert decodes.prefill_requests == () and _ids(decodes.decode_requests) == ("A", "B")
    mixed = build_iteration_plan([_running("prefill"), _running("decode", 3)])
    assert _ids(mixed.prefill_requests) == ("prefill",)
    assert _ids(mixed.decode_requests) == ("decode",)
    assert mixed.request_ids == ("prefill", "decode")


def test_iteration_plan_excludes_inactive_and_complete_requests() -> None:
    waiting = _request("waiting")
    finished = _running("finished", 3)
    finished.mark_finished()
    cancelled = _running("cancelled")
    cancelled.cancel()
    assert build_iteration_plan((waiting, finished, cancelled)).is_empty
    done = _request("complete", (1,), 1)
    done.mark_running()
    done.mark_prefill_complete()
    done.append_generated_token(torch.tensor([[2]]))
    assert done.completion_reason == "max_new_tokens"
    assert build_iteration_plan((done,)).is_empty
    request = _running("A")
    with pytest.raises(ValueError, match="duplicate request_id"):
        build_iteration_plan((request, request))
