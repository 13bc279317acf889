"""The batched executor's host logic on the CPU: metrics hooks in the reference's order,
all-or-nothing reservations, the reference keyword interfaces and module paths.

The GPU forward is replaced by a stub that returns token 0 for every sequence, so
what is checked is bookkeeping only: hook sequences, block ids, sequence and
allocator state.
"""

import pytest
import torch

from oracle import engine as oracle_engine
from tokserve_amd.batching import execution
from tokserve_amd.batching.engine import ContinuousBatchEngine
from tokserve_amd.batching.execution import BatchExecutor, execute_decode, execute_prefill
from tokserve_amd.batching.plan import build_iteration_plan
from tokserve_amd.engine.config import LlamaConfig
from tokserve_amd.engine.model import LlamaModel
from tokserve_amd.engine.paged.allocator import BlockExhaustedError
from tokserve_amd.engine.paged.manager import PagedKVCacheManager
from tokserve_amd.generation.types import GenerationConfig
from tokserve_amd.scheduler.request import ScheduledRequest
from tokserve_amd.scheduler.scheduler import RequestScheduler

CONFIG = dict(vocab_size=32, hidden_size=16, intermediate_size=32, num_hidden_layers=2,
              num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=16,
              rms_norm_eps=1e-6, rope_theta=10_000.0)


class Recorder:
    """A metrics collector that records each hook call (the reference's hook names)."""

    def __init__(self) -> None:
        self.events: list[tuple] = []

    def request_admitted(self, request_id):
        self.events.append(("request_admitted", request_id))

    def prefill_started(self, request_id):
        self.events.append(("prefill_started", request_id))

    def prefill_finished(self, request_id):
        self.events.append(("prefill_finished", request_id))

    def token_produced(self, request_id):
        self.events.append(("token_produced", request_id))

    def complete_request(self, request_id, completion_reason):
        self.events.append(("complete_request", request_id, completion_reason))

    def record_iteration(self, *, prefill_requests, decode_requests):
        self.events.append(("record_iteration", prefill_requests, decode_requests))


class StubExecutor(BatchExecutor):
    """Token 0 for everyone instead of the GPU forward; optionally fails on a call."""

    fail_on_call: int | None = None

    def _forward(self, prefill, decode, requests):
        self.calls = getattr(self, "calls", 0) + 1
        if self.fail_on_call == self.calls:
            raise RuntimeError("forward failed")
        self.builder.build(prefill, decode)
        return [0] * len(requests)


def _model():
    torch.manual_seed(0)
    return LlamaModel(LlamaConfig(**CONFIG))


def _manager(num_blocks, block_size):
    return PagedKVCacheManager(num_layers=2, num_blocks=num_blocks, num_key_value_heads=2,
                               block_size=block_size, head_dim=4, device=torch.device("cpu"),
                               dtype=torch.float32)


def _engine(max_running, num_blocks, block_size, metrics=None):
    model = _model()
    manager = _manager(num_blocks, block_size)
    scheduler = RequestScheduler(max_running_requests=max_running, cache_manager=manager)
    engine = ContinuousBatchEngine(model, scheduler, manager, metrics=metrics)
    engine.executor = StubExecutor(model, manager)
    return engine, scheduler, manager


def _submit(scheduler, specs, eos=None):
    for rid, prompt, n in specs:
        scheduler.submit(ScheduledRequest(rid, torch.tensor([prompt]),
                                          GenerationConfig(max_new_tokens=n, eos_token_id=eos)))


RAGGED = (("A", [1, 2, 3], 3), ("B", [4, 5, 6, 7], 2), ("C", [8, 9, 10, 11, 12, 13, 14], 1),
          ("D", [15], 2))


def _oracle_events(specs, max_running, num_blocks, block_size, eos=None):
    reference = oracle_engine.Engine({}, CONFIG, num_blocks=num_blocks, block_size=block_size,
                                     max_running=max_running)
    reference._next_token = lambda request, tokens: 0
    for rid, prompt, n in specs:
        reference.submit(oracle_engine.Request(rid, list(prompt), n, eos_token_id=eos))
    records = reference.run()
    return _one_forward_per_iteration(reference.events), records


def _one_forward_per_iteration(events: list[tuple]) -> list[tuple]:
    """The reference's hook sequence (each prefill's started / finished around its own
    forward) as an engine that serves an iteration's prefills with one forward emits it:
    within each iteration, every prefill_started moves, in order, to where the first one
    was; everything else keeps its place."""

    out: list[tuple] = []
    group: list[tuple] = []
    for event in events + [("record_iteration",)]:
        group.append(event)
        if event[0] != "record_iteration":
            continue
        starts = [e for e in group if e[0] == "prefill_started"]
        rest = [e for e in group if e[0] != "prefill_started"]
        if starts:
            first = next(i for i, e in enumerate(group) if e[0] == "prefill_started")
            rest[first:first] = starts
        out.extend(rest)
        group = []
    return out[:-1]


def test_one_forward_order_moves_only_the_starts() -> None:
    events = [("request_admitted", "a"), ("request_admitted", "b"),
              ("prefill_started", "a"), ("prefill_finished", "a"), ("token_produced", "a"),
              ("prefill_started", "b"), ("prefill_finished", "b"), ("token_produced", "b"),
              ("record_iteration", 2, 0), ("token_produced", "a"), ("record_iteration", 0, 1)]
    assert _one_forward_per_iteration(events) == [
        ("request_admitted", "a"), ("request_admitted", "b"),
        ("prefill_started", "a"), ("prefill_started", "b"),
        ("prefill_finished", "a"), ("token_produced", "a"),
        ("prefill_finished", "b"), ("token_produced", "b"),
        ("record_iteration", 2, 0), ("token_produced", "a"), ("record_iteration", 0, 1)]


@pytest.mark.parametrize(("specs", "max_running", "num_blocks", "block_size"), [
    (RAGGED, 3, 8, 4),
    ((("A", [1, 2], 3), ("Z", [3], 0), ("B", [3, 4, 5], 1), ("C", [6], 2)), 2, 16, 2),
])
def test_metrics_hooks_follow_the_reference_order(specs, max_running, num_blocks,
                                                  block_size) -> None:
    """The ragged scenario (tests/integration/test_continuous_batch_ragged.py:57-169) and a
    mix with a zero-token request: the same hook calls, in the same order, as the
    reference's per-request loop (restated in oracle/engine.py), except that an
    iteration's prefill_started calls all come before its one packed forward."""

    recorder = Recorder()
    engine, scheduler, _ = _engine(max_running, num_blocks, block_size, metrics=recorder)
    _submit(scheduler, specs)
    engine.run_until_idle()
    expected_events, expected_records = _oracle_events(specs, max_running, num_blocks,
                                                       block_size)
    assert recorder.events == expected_events
    assert [tuple(r.__dict__.values()) for r in engine.history] == \
        [tuple(r.__dict__.values()) for r in expected_records]


def test_hook_counts_of_the_reference_lifecycle_tests() -> None:
    """tests/integration/test_metrics_lifecycle.py:95-121: one request of 3 tokens is one
    prefill request and two decode requests over the iterations, 3 tokens; an EOS first
    token (:142-160) completes once with reason "eos" after 1 token."""

    recorder = Recorder()
    engine, scheduler, _ = _engine(4, 24, 2, metrics=recorder)
    _submit(scheduler, [("r", [1, 2], 3)])
    engine.run_until_idle()
    iterations = [e for e in recorder.events if e[0] == "record_iteration"]
    assert sum(e[1] for e in iterations) == 1 and sum(e[2] for e in iterations) == 2
    assert sum(e[0] == "token_produced" for e in recorder.events) == 3
    assert [e for e in recorder.events if e[0] == "complete_request"] == [
        ("complete_request", "r", "max_new_tokens")]

    recorder = Recorder()
    engine, scheduler, _ = _engine(4, 24, 2, metrics=recorder)
    _submit(scheduler, [("e", [1], 4)], eos=0)
    engine.run_until_idle()
    assert sum(e[0] == "token_produced" for e in recorder.events) == 1
    assert [e for e in recorder.events if e[0] == "complete_request"] == [
        ("complete_request", "e", "eos")]
    assert recorder.events == _oracle_events([("e", [1], 4)], 4, 24, 2, eos=0)[0]


def _state(manager):
    return (manager.active_sequence_ids, manager.allocator.free_count,
            manager.allocator.allocated_blocks,
            {sid: (manager.get_sequence(sid).block_ids, manager.get_sequence(sid).current_length,
                   manager.get_sequence(sid).pending_length)
             for sid in manager.active_sequence_ids})


def _running(specs):
    requests = []
    for rid, prompt, n in specs:
        request = ScheduledRequest(rid, torch.tensor([prompt]), GenerationConfig(max_new_tokens=n))
        request.mark_running()
        requests.append(request)
    return requests


def test_failed_batch_leaves_manager_and_allocator_unchanged() -> None:
    """[ok, too long]: the second prompt exceeds max_position_embeddings. Nothing is
    created or reserved, no request changes, and the same batch without it then runs."""

    model, manager = _model(), _manager(16, 2)
    executor = StubExecutor(model, manager)
    first = _running([("warm", [1, 2, 3], 4)])
    executor.execute(first, ())
    before = _state(manager)
    ok, too_long = _running([("ok", [1, 2], 2), ("long", list(range(17)), 2)])
    with pytest.raises(ValueError, match="sequence length exceeds max_position_embeddings"):
        executor.execute([ok, too_long], first)
    assert _state(manager) == before
    assert not ok.prefill_complete and first[0].num_generated_tokens == 1
    assert executor.execute([ok], first) == ()
    assert manager.get_sequence("ok").block_ids == (2,)


def test_exhausted_pool_mid_batch_rolls_back_every_reservation() -> None:
    """Three prefills and a decode need more blocks than the pool holds: the iteration's
    one allocation fails after the prefills opened their sequences; they are dropped and
    the pool and the existing sequence are untouched."""

    model, manager = _model(), _manager(6, 2)
    executor = StubExecutor(model, manager)
    old = _running([("old", [1, 2], 4)])
    executor.execute(old, ())
    before = _state(manager)
    fresh = _running([("a", [1, 2, 3], 1), ("b", [4, 5, 6], 1), ("c", [7, 8, 9], 1)])
    with pytest.raises(BlockExhaustedError):
        executor.execute(fresh, old)
    assert _state(manager) == before
    assert all(not r.prefill_complete for r in fresh)


def test_failed_forward_rolls_back_and_changes_no_request() -> None:
    model, manager = _model(), _manager(12, 2)
    executor = StubExecutor(model, manager)
    old = _running([("old", [1, 2], 4)])
    executor.execute(old, ())
    before = _state(manager)
    executor.fail_on_call = 2
    fresh = _running([("a", [1, 2, 3], 2)])
    with pytest.raises(RuntimeError, match="forward failed"):
        executor.execute(fresh, old)
    assert _state(manager) == before
    assert old[0].num_generated_tokens == 1 and not fresh[0].prefill_complete
    executor.fail_on_call = None
    assert executor.execute(fresh, old) == ()
    assert (old[0].num_generated_tokens, fresh[0].num_generated_tokens) == (2, 1)


def test_abort_append_returns_only_the_blocks_it_took() -> None:
    manager = _manager(8, 2)
    cache = manager.create_sequence("s", max_sequence_length=16)
    cache.begin_append(3)
    cache.commit()
    assert cache.block_ids == (0, 1)
    cache.begin_append(4)  # positions 3..6: block 1 (kept) + blocks 2, 3
    assert cache.block_ids == (0, 1, 2, 3)
    cache.abort_append()
    assert (cache.block_ids, cache.current_length, cache.pending_length) == ((0, 1), 3, 0)
    assert manager.allocator.free_count == 6
    cache.begin_append(1)
    assert cache.block_ids == (0, 1)  # position 3 fits block 1


def test_module_level_execution_reuses_one_executor_per_manager() -> None:
    model, manager = _model(), _manager(16, 2)
    requests = _running([("a", [1, 2], 3)])
    original = execution.BatchExecutor
    execution.BatchExecutor = StubExecutor
    try:
        execute_prefill(model, manager, requests)
        first = manager._batch_executor
        execute_decode(model, manager, requests, metrics=Recorder())
        assert manager._batch_executor is first
    finally:
        execution.BatchExecutor = original
    assert requests[0].num_generated_tokens == 2


def test_module_level_execution_lets_the_manager_go() -> None:
    """The executor execute_prefill / execute_decode keep for a manager (with its pools and
    decode graphs) is collected with the manager once the caller drops it."""

    import gc
    import weakref

    model, manager = _model(), _manager(16, 2)
    requests = _running([("a", [1, 2], 3)])
    original = execution.BatchExecutor
    execution.BatchExecutor = StubExecutor
    try:
        execute_prefill(model, manager, requests)
        execute_decode(model, manager, requests)
    finally:
        execution.BatchExecutor = original
    assert requests[0].num_generated_tokens == 2
    alive = weakref.ref(manager)
    executor = weakref.ref(manager._batch_executor)
    assert executor().manager is manager
    del manager, requests
    gc.collect()
    assert alive() is None and executor() is None


def test_reference_keyword_interfaces_and_module_paths() -> None:
    from tokserve_amd.engine import kernel_backend, rope
    from tokserve_amd.generation.greedy import select_greedy
    from oracle import torch_path

    config = LlamaConfig(**CONFIG)
    for backend in ("torch", "triton"):
        model = LlamaModel(config, backend=backend)
        assert model.backend == backend and model.layers[0].self_attention.backend == backend
    with pytest.raises(ValueError, match="backend must be 'torch' or 'triton'"):
        LlamaModel(config, backend="cuda")
    with pytest.raises(ValueError, match="Triton backend requires CUDA"):
        kernel_backend.apply_rms_norm(LlamaModel(config).final_norm, torch.ones(2, 16), "triton")
    with pytest.raises(ValueError, match="logits must have shape"):
        select_greedy(torch.ones(3))
    positions = rope.positions_for_sequence(5, offset=7, device=torch.device("cpu"))
    assert positions.tolist() == [7, 8, 9, 10, 11]
    cos, sin = rope.rotary_cos_sin(positions, 8, theta=10_000.0, dtype=torch.float32)
    expected_cos, expected_sin = torch_path.rotary_cos_sin(positions, 8, theta=10_000.0,
                                                           dtype=torch.float32)
    assert torch.equal(cos, expected_cos) and torch.equal(sin, expected_sin)
    x = torch.arange(8.0)
    assert torch.equal(rope.rotate_half(x), torch_path.rotate_half(x))
    with pytest.raises(ValueError, match="offset must be nonnegative"):
        rope.positions_for_sequence(2, offset=-1, device=torch.device("cpu"))
    with pytest.raises(ValueError, match="CUDA tensors"):
        rope.apply_rope(torch.ones(1, 2, 3, 8), torch.ones(1, 1, 3, 8), positions[:3],
                        theta=10_000.0)
    assert build_iteration_plan([]).is_empty


def test_reference_cache_keyword_and_paged_generate_module() -> None:
    """tokserve/engine/model.py:50,124 and attention.py:181 take cache= beside paged_cache=;
    generate_with_paged_cache lives at tokserve/generation/paged_generate.py:18. cache=None
    is accepted (the call goes on, here to the device check), a contiguous cache raises
    ValueError, with the reference's message when a paged cache comes too."""

    import inspect

    from tokserve_amd.generation import paged_generate

    assert list(inspect.signature(paged_generate.generate_with_paged_cache).parameters) == [
        "model", "input_ids", "config", "manager", "sequence_id"]
    model = LlamaModel(LlamaConfig(**CONFIG))
    ids = torch.ones(1, 3, dtype=torch.int64)
    block, attention = model.layers[0], model.layers[0].self_attention
    hidden, positions = torch.ones(1, 3, CONFIG["hidden_size"]), torch.arange(3)
    for call in (lambda **kw: model(ids, **kw), lambda **kw: block(hidden, positions, **kw),
                 lambda **kw: attention(hidden, positions, **kw)):
        with pytest.raises(ValueError, match="requires HIP device tensors|CUDA"):
            call(cache=None)
        with pytest.raises(ValueError, match="contiguous KV caches are not supported"):
            call(cache=object())
        with pytest.raises(ValueError, match="choose either contiguous or paged cache"):
            call(cache=object(), paged_cache=object())


class _Ready:
    def synchronize(self) -> None:
        pass


class LengthTokens(StubExecutor):
    """Token = (sequence length after the append) % 5, through both the packed forward and
    the split launch (launch_decode / finish) that the engine's overlap_decode uses, which
    runs here on the CPU with the same reservations as on the GPU."""

    def _forward(self, prefill, decode, requests):
        self.builder.build(prefill, decode)
        return [(w.start + len(w.tokens)) % 5 for w in (*prefill, *decode)]

    def can_launch(self, decode) -> bool:
        return bool(decode)

    def launch_decode(self, decode, *, token_source=None):
        self.queued_launches = getattr(self, "queued_launches", 0) + (token_source is not None)
        checked = self._check((), decode)
        reservation = self.manager.reservation()
        try:
            self._reserve(reservation, checked)
        except BaseException:
            reservation.rollback()
            raise
        tokens = torch.tensor([(length + 1) % 5 for length in checked.decode_lengths])
        return execution.LaunchedDecode(checked, reservation, tokens, tokens, _Ready())


def _overlap_run(overlap, specs, *, max_running, num_blocks, block_size, eos=None,
                 between=None, ids=None):
    recorder = Recorder()
    model = _model()
    manager = _manager(num_blocks, block_size)
    scheduler = RequestScheduler(max_running_requests=max_running, cache_manager=manager)
    engine = ContinuousBatchEngine(model, scheduler, manager, metrics=recorder,
                                   overlap_decode=overlap)
    engine.executor = LengthTokens(model, manager)
    released = {}
    original = manager.release_sequence

    def record(sequence_id):
        released[sequence_id] = manager.get_sequence(sequence_id).block_ids
        original(sequence_id)

    manager.release_sequence = record
    _submit(scheduler, specs, eos=eos)
    step = 0
    while scheduler.waiting_count or scheduler.running_count:
        engine.step()
        step += 1
        if between is not None:
            between(step, scheduler)
    ids = [rid for rid, _, _ in specs] if ids is None else ids
    tokens = {rid: (scheduler.get_request(rid).state.value,
                    scheduler.get_request(rid).generated_tokens) for rid in ids}
    outcome = ([tuple(r.__dict__.values()) for r in engine.history], recorder.events,
               released, tokens, manager.allocator.free_count)
    return outcome, getattr(engine.executor, "queued_launches", 0)


LONG = (("A", [1, 2, 3], 9), ("B", [4, 5, 6, 7], 6), ("C", [8], 12), ("D", [9, 10], 4))


@pytest.mark.parametrize(("max_running", "eos"), [(4, None), (2, None), (4, 3)])
def test_overlapped_decode_keeps_records_hooks_and_blocks(max_running, eos) -> None:
    """overlap_decode queues iteration i+1 before finishing iteration i wherever the next
    plan is fixed; records, hook order, tokens, released block ids and the final pool
    equal the one-at-a-time engine's. With an EOS token nothing is queued."""

    sequential, queued_off = _overlap_run(False, LONG, max_running=max_running, num_blocks=24,
                                          block_size=2, eos=eos)
    overlapped, queued_on = _overlap_run(True, LONG, max_running=max_running, num_blocks=24,
                                         block_size=2, eos=eos)
    assert overlapped == sequential
    assert queued_off == 0
    assert (queued_on > 0) == (eos is None)


def test_overlapped_decode_discards_on_submission_and_cancellation() -> None:
    """A submission and then a cancellation between steps while an iteration is queued."""

    def between(step, scheduler):
        if step == 3:
            scheduler.submit(ScheduledRequest("E", torch.tensor([[11, 12]]),
                                              GenerationConfig(max_new_tokens=3)))
        if step == 6 and scheduler.get_request("C").state.value == "running":
            scheduler.cancel("C")

    ids = [rid for rid, _, _ in LONG] + ["E"]
    sequential, _ = _overlap_run(False, LONG, max_running=4, num_blocks=30, block_size=2,
                                 between=between, ids=ids)
    overlapped, queued = _overlap_run(True, LONG, max_running=4, num_blocks=30, block_size=2,
                                      between=between, ids=ids)
    assert overlapped == sequential
    assert queued > 0
    assert overlapped[3]["C"][0] == "cancelled" and overlapped[3]["E"][0] == "finished"
    assert overlapped[4] == 30
