"""Model construction, the e2e oracle, and the continuous-batching host logic (CPU).

The golden fixture tests/golden/tiny_llama_fp32.pt comes from the reference's
own LlamaModel (tests/golden/make_tiny_llama_fixture.py): its weights pin the
module creation order, its logits and greedy tokens pin oracle/model.py, and
the block ids pin the paged allocation order. The engine cases are the known
answers of tests/integration/test_continuous_batch_ragged.py:57-169.
"""

from pathlib import Path

import pytest
import torch
from torch.testing import assert_close

from oracle import engine as oracle_engine
from oracle import model as oracle_model
from tokserve_amd.batching.engine import ContinuousBatchEngine
from tokserve_amd.batching.execution import BatchExecutor
from tokserve_amd.batching.plan import build_iteration_plan
from tokserve_amd.engine.config import LlamaConfig
from tokserve_amd.engine.model import LlamaModel
from tokserve_amd.engine.paged.manager import PagedKVCacheManager
from tokserve_amd.generation.types import GenerationConfig
from tokserve_amd.scheduler.request import RequestState, ScheduledRequest
from tokserve_amd.scheduler.scheduler import RequestScheduler

FIXTURE = torch.load(Path(__file__).parent / "golden" / "tiny_llama_fp32.pt", weights_only=True)


def test_seeded_init_matches_the_reference_weights() -> None:
    torch.manual_seed(FIXTURE["seed"])
    model = LlamaModel(LlamaConfig(**FIXTURE["config"]))
    ours = model.state_dict()
    assert list(ours) == list(FIXTURE["state_dict"])
    for name, value in FIXTURE["state_dict"].items():
        assert torch.equal(ours[name], value), name


def test_oracle_forward_reproduces_reference_logits() -> None:
    prompt = torch.tensor([FIXTURE["prompt"]])
    logits = oracle_model.forward(FIXTURE["state_dict"], FIXTURE["config"], prompt)
    assert_close(logits, FIXTURE["prompt_logits"], rtol=1e-6, atol=1e-6)


def test_oracle_incremental_decode_reproduces_reference_tokens() -> None:
    kv = oracle_model.SequenceKV()
    state, config = FIXTURE["state_dict"], FIXTURE["config"]
    logits = oracle_model.forward(state, config, torch.tensor([FIXTURE["prompt"]]), kv)[0, -1]
    steps = [logits]
    tokens = []
    for _ in FIXTURE["decode_tokens"]:
        token = int(torch.argmax(logits))
        tokens.append(token)
        logits = oracle_model.forward(state, config, torch.tensor([[token]]), kv)[0, -1]
        steps.append(logits)
    assert tokens == FIXTURE["decode_tokens"]
    assert_close(torch.stack(steps), FIXTURE["decode_logits"], rtol=1e-5, atol=1e-5)
    assert kv.length == len(FIXTURE["prompt"]) + len(tokens)


def _abcd():
    return (("A", [1, 2, 3], 3), ("B", [4, 5, 6, 7], 2), ("C", [8, 9, 10, 11, 12, 13, 14], 1),
            ("D", [15], 2))


def test_oracle_engine_ragged_known_answers() -> None:
    engine = oracle_engine.Engine(FIXTURE["state_dict"], FIXTURE["config"], num_blocks=8,
                                  block_size=4, max_running=3)
    for rid, prompt, n in _abcd():
        engine.submit(oracle_engine.Request(rid, prompt, n))
    first, second, third = engine.step(), engine.step(), engine.step()
    assert (first.prefill_ids, first.completed_ids) == (("A", "B", "C"), ("C",))
    assert (second.admitted_ids, second.prefill_ids, second.decode_ids, second.completed_ids) == (
        ("D",), ("D",), ("A", "B"), ("B",))
    assert (third.prefill_ids, third.decode_ids, third.completed_ids, third.active_ids) == (
        (), ("A", "D"), ("A", "D"), ())
    released = {rid: r.released_blocks for rid, r in engine.finished.items()}
    assert released["C"] == (2, 3) and released["D"] == (2,)
    assert len(released["A"]) == 2 and len(released["B"]) == 2
    # Paged-engine tokens equal independent full-recompute generation.
    for rid, prompt, n in _abcd():
        tokens = list(prompt)
        for _ in range(n):
            logits = oracle_model.forward(FIXTURE["state_dict"], FIXTURE["config"],
                                          torch.tensor([tokens]))
            tokens.append(int(torch.argmax(logits[0, -1])))
        assert engine.finished[rid].generated == tokens[len(prompt):]


class _HostExecutor(BatchExecutor):
    """The batched executor with its GPU forward replaced by token 0 for everyone."""

    def _forward(self, prefill, decode, requests):
        self.calls.append((len(prefill), len(decode)))
        batch = self.builder.build(prefill, decode)
        self.batches.append(batch)
        return [0] * len(requests)


def _host_engine(max_running: int, num_blocks: int, block_size: int):
    torch.manual_seed(0)
    model = LlamaModel(LlamaConfig(vocab_size=32, hidden_size=16, intermediate_size=32,
                                   num_hidden_layers=2, num_attention_heads=4,
                                   num_key_value_heads=2, max_position_embeddings=64))
    manager = PagedKVCacheManager(num_layers=2, num_blocks=num_blocks, num_key_value_heads=2,
                                  block_size=block_size, head_dim=4, device=torch.device("cpu"),
                                  dtype=torch.float32)
    scheduler = RequestScheduler(max_running_requests=max_running, cache_manager=manager)
    engine = ContinuousBatchEngine(model, scheduler, manager)
    engine.executor = _HostExecutor(model, manager)
    engine.executor.calls, engine.executor.batches = [], []
    released = {}
    original = manager.release_sequence

    def record(sequence_id):
        released[sequence_id] = manager.get_sequence(sequence_id).block_ids
        original(sequence_id)

    manager.release_sequence = record
    return engine, scheduler, manager, released


def test_engine_ragged_known_answers_and_packed_metadata() -> None:
    engine, scheduler, manager, released = _host_engine(3, 8, 4)
    for rid, prompt, n in _abcd():
        scheduler.submit(ScheduledRequest(rid, torch.tensor([prompt]),
                                          GenerationConfig(max_new_tokens=n)))
    first = engine.step()
    assert first.prefill_ids == ("A", "B", "C") and first.completed_ids == ("C",)
    assert scheduler.get_request("D").state is RequestState.WAITING
    assert released["C"] == (2, 3)
    assert manager.get_sequence("A").block_ids == (0,) and manager.get_sequence("B").block_ids == (1,)
    batch = engine.executor.batches[0]
    assert batch.num_prefill_tokens == 14 and batch.logits_rows.tolist() == [2, 6, 13]
    assert batch.slot_mapping.tolist() == [0, 1, 2, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14]
    second = engine.step()
    assert (second.admitted_ids, second.prefill_ids, second.decode_ids, second.completed_ids) == (
        ("D",), ("D",), ("A", "B"), ("B",))
    assert manager.get_sequence("D").block_ids == (2,)
    batch = engine.executor.batches[1]
    # D's prompt, then A at position 3 (block 0) and B at position 4 (its new block 3).
    assert batch.positions.tolist() == [0, 3, 4]
    assert batch.slot_mapping.tolist() == [8, 3, 12]
    assert batch.decode_seq_lens.tolist() == [4, 5] and batch.decode_seq_order.tolist() == [1, 0]
    third = engine.step()
    assert (third.prefill_ids, third.decode_ids, third.completed_ids, third.active_ids) == (
        (), ("A", "D"), ("A", "D"), ())
    assert released == {"C": (2, 3), "B": (1, 3), "A": (0, 1), "D": (2,)}
    assert manager.allocator.allocated_count == 0
    assert engine.executor.calls == [(3, 0), (1, 2), (0, 2)]
    for rid, prompt, n in _abcd():
        result = scheduler.get_request(rid).result
        assert result.generated_token_ids.tolist() == [[0] * n]
        assert result.token_ids.tolist() == [prompt + [0] * n]


def test_engine_records_match_the_oracle_loop_on_a_ragged_workload() -> None:
    g = torch.Generator().manual_seed(5)
    specs = [(f"r{i}", torch.randint(0, 32, (int(torch.randint(1, 14, (1,), generator=g)),),
                                     generator=g).tolist(),
              int(torch.randint(0, 6, (1,), generator=g))) for i in range(14)]
    engine, scheduler, manager, released = _host_engine(4, 12, 4)
    reference = oracle_engine.Engine(FIXTURE["state_dict"], FIXTURE["config"], num_blocks=12,
                                     block_size=4, max_running=4)
    reference._next_token = lambda request, tokens: 0
    for rid, prompt, n in specs:
        scheduler.submit(ScheduledRequest(rid, torch.tensor([prompt]),
                                          GenerationConfig(max_new_tokens=n)))
        reference.submit(oracle_engine.Request(rid, prompt, n))
    engine.run_until_idle()
    expected = reference.run()
    assert [tuple(r.__dict__.values()) for r in engine.history] == \
        [tuple(r.__dict__.values()) for r in expected]
    for rid, request in reference.finished.items():
        if request.max_new_tokens:
            assert released[rid] == request.released_blocks


def test_plan_and_request_lifecycle_checks() -> None:
    request = ScheduledRequest("x", torch.tensor([[1, 2]]), GenerationConfig(max_new_tokens=2))
    with pytest.raises(RuntimeError, match="request must be running, not waiting"):
        request.mark_prefill_complete()
    request.mark_running()
    assert build_iteration_plan([request]).prefill_requests == (request,)
    request.mark_prefill_complete()
    assert build_iteration_plan([request]).is_empty
    request.append_generated_token(torch.tensor([[7]]))
    assert request.decode_ready and request.next_input_token.tolist() == [[7]]
    with pytest.raises(TypeError, match="match the prompt dtype"):
        request.append_generated_token(torch.tensor([[7]], dtype=torch.int32))
    request.append_generated_token(9)
    assert request.completion_reason == "max_new_tokens" and not request.decode_ready
    with pytest.raises(RuntimeError, match="already completed"):
        request.append_generated_token(1)
    with pytest.raises(ValueError, match="duplicate request_id"):
        build_iteration_plan([request, request])
    eos = ScheduledRequest("e", torch.tensor([[1]]), GenerationConfig(max_new_tokens=5,
                                                                      eos_token_id=3))
    eos.mark_running()
    eos.mark_prefill_complete()
    eos.append_generated_token(3)
    assert eos.completion_reason == "eos"
    assert eos.build_result().token_ids.tolist() == [[1, 3]]


# The scheduling scenarios of tests/integration/test_continuous_batch_pressure.py:60-244 and
# tests/integration/test_continuous_batch_engine.py:57-233 (block size 2), with the GPU
# forward replaced by token 0: admission, FIFO order, cache pressure and membership do not
# depend on the token values (every request ends by max_new_tokens).

def _submit(scheduler, rid, prompt, n):
    request = ScheduledRequest(rid, torch.tensor([prompt]), GenerationConfig(max_new_tokens=n))
    scheduler.submit(request)
    return request


def _ids(record):
    return (record.admitted_ids, record.prefill_ids, record.decode_ids, record.completed_ids)


def test_arrivals_preserve_fifo_across_iteration_boundaries() -> None:
    engine, scheduler, _, _ = _host_engine(2, 16, 2)
    a = _submit(scheduler, "A", [1, 2], 4)
    b = _submit(scheduler, "B", [3], 2)
    zero = engine.step()
    assert zero.admitted_ids == ("A", "B") and zero.prefill_ids == ("A", "B")
    c = _submit(scheduler, "C", [4, 5, 6], 2)
    one = engine.step()
    assert (one.admitted_ids, one.decode_ids, one.completed_ids) == ((), ("A", "B"), ("B",))
    assert c.state is RequestState.WAITING
    d = _submit(scheduler, "D", [7], 1)
    two = engine.step()
    assert (two.admitted_ids, two.prefill_ids, two.decode_ids) == (("C",), ("C",), ("A",))
    assert d.state is RequestState.WAITING
    three = engine.step()
    assert (three.decode_ids, three.completed_ids) == (("A", "C"), ("A", "C"))
    assert d.state is RequestState.WAITING
    four = engine.step()
    assert (four.admitted_ids, four.prefill_ids, four.completed_ids) == (("D",), ("D",), ("D",))
    assert scheduler.waiting_count == 0 and scheduler.running_count == 0
    assert all(r.state is RequestState.FINISHED for r in (a, b, c, d))


def test_cache_pressure_keeps_request_waiting_until_capacity_returns() -> None:
    engine, scheduler, manager, _ = _host_engine(2, 3, 2)
    _submit(scheduler, "A", [1, 2], 3)  # ceil((2 + 3) / 2) = 3 blocks: the whole pool
    b = _submit(scheduler, "B", [3], 1)
    zero = engine.step()
    assert (zero.admitted_ids, zero.prefill_ids) == (("A",), ("A",))
    assert b.state is RequestState.WAITING and scheduler.waiting_count == 1
    one = engine.step()
    assert (one.admitted_ids, one.decode_ids) == ((), ("A",)) and b.state is RequestState.WAITING
    two = engine.step()
    assert (two.decode_ids, two.completed_ids) == (("A",), ("A",))
    assert b.state is RequestState.WAITING and manager.allocator.allocated_count == 0
    three = engine.step()
    assert (three.admitted_ids, three.prefill_ids, three.completed_ids) == (("B",),) * 3
    assert b.state is RequestState.FINISHED
    assert scheduler.waiting_count == 0 and scheduler.running_count == 0
    assert manager.active_sequence_ids == ()
    assert manager.allocator.allocated_count == 0 and manager.allocator.free_count == 3


def test_waiting_order_is_unchanged_during_resource_pressure() -> None:
    engine, scheduler, _, _ = _host_engine(3, 3, 2)
    _submit(scheduler, "A", [1, 2], 3)
    _submit(scheduler, "B", [3], 1)
    _submit(scheduler, "C", [4], 1)
    engine.step()
    assert tuple(r.request_id for r in scheduler.waiting_requests) == ("B", "C")
    engine.step()
    assert tuple(r.request_id for r in scheduler.waiting_requests) == ("B", "C")
    engine.step()
    last = engine.step()
    assert (last.admitted_ids, last.prefill_ids, last.completed_ids) == (("B", "C"),) * 3


def test_batch_membership_changes_between_iterations() -> None:
    engine, scheduler, _, _ = _host_engine(2, 16, 2)
    _submit(scheduler, "A", [1, 2], 3)
    _submit(scheduler, "B", [3, 4, 5], 1)
    c = _submit(scheduler, "C", [6], 2)
    first = engine.step()
    assert _ids(first) == (("A", "B"), ("A", "B"), (), ("B",)) and first.active_ids == ("A",)
    assert scheduler.get_request("B").state is RequestState.FINISHED
    assert c.state is RequestState.WAITING
    second = engine.step()
    assert _ids(second) == (("C",), ("C",), ("A",), ()) and second.active_ids == ("A", "C")
    assert c.num_generated_tokens == 1
    third = engine.step()
    assert _ids(third) == ((), (), ("A", "C"), ("A", "C")) and third.active_ids == ()
    assert scheduler.waiting_count == 0 and scheduler.running_count == 0


def test_newly_prefilled_request_waits_until_next_decode_iteration() -> None:
    engine, scheduler, _, _ = _host_engine(1, 16, 2)
    request = _submit(scheduler, "A", [1, 2], 3)
    first = engine.step()
    assert (first.prefill_ids, first.decode_ids) == (("A",), ()) and request.num_generated_tokens == 1
    second = engine.step()
    assert (second.prefill_ids, second.decode_ids) == ((), ("A",))
    assert request.num_generated_tokens == 2


def test_completed_requests_never_execute_again() -> None:
    engine, scheduler, _, _ = _host_engine(1, 16, 2)
    _submit(scheduler, "A", [1], 1)
    first = engine.step()
    second = engine.step()
    assert first.completed_ids == ("A",)
    assert (second.prefill_ids, second.decode_ids, second.completed_ids) == ((), (), ())
    assert engine.executor.calls == [(1, 0)]


def test_engine_rejects_different_cache_manager() -> None:
    engine, scheduler, _, _ = _host_engine(1, 16, 2)
    other = PagedKVCacheManager(num_layers=2, num_blocks=16, num_key_value_heads=2, block_size=2,
                                head_dim=4, device=torch.device("cpu"), dtype=torch.float32)
    with pytest.raises(ValueError, match="share the cache manager"):
        ContinuousBatchEngine(engine.model, scheduler, other)


def test_continuous_batching_end_to_end_records() -> None:
    """tests/integration/test_continuous_batch_end_to_end.py:58-188 (8 blocks of 2): C and D
    arrive mid-run."""

    engine, scheduler, manager, released = _host_engine(2, 8, 2)
    requests = {"A": _submit(scheduler, "A", [1, 2], 4), "B": _submit(scheduler, "B", [3, 4, 5], 2)}
    zero = engine.step()
    assert (zero.iteration, *_ids(zero), zero.active_ids) == (
        0, ("A", "B"), ("A", "B"), (), (), ("A", "B"))
    one = engine.step()
    assert (one.iteration, *_ids(one), one.active_ids) == (1, (), (), ("A", "B"), ("B",), ("A",))
    requests["C"] = _submit(scheduler, "C", [6], 3)
    two = engine.step()
    assert (two.iteration, *_ids(two), two.active_ids) == (
        2, ("C",), ("C",), ("A",), (), ("A", "C"))
    requests["D"] = _submit(scheduler, "D", [7, 8, 9, 10], 1)
    three = engine.step()
    assert (three.iteration, *_ids(three), three.active_ids) == (
        3, (), (), ("A", "C"), ("A",), ("C",))
    assert requests["D"].state is RequestState.WAITING
    four = engine.step()
    assert (four.iteration, *_ids(four), four.active_ids) == (
        4, ("D",), ("D",), ("C",), ("C", "D"), ())
    assert engine.history == (zero, one, two, three, four)
    assert all(r.state is RequestState.FINISHED for r in requests.values())
    assert set(released) == {"A", "B", "C", "D"}
    assert set(released["D"]) & set(released["A"] + released["B"])  # freed blocks are reused
    assert manager.active_sequence_ids == () and manager.allocator.allocated_count == 0
    assert manager.allocator.free_count == manager.allocator.num_blocks
    assert scheduler.waiting_count == 0 and scheduler.running_count == 0


def test_run_until_idle_records_every_iteration() -> None:
    engine, scheduler, manager, _ = _host_engine(2, 16, 2)
    _submit(scheduler, "A", [1], 2)
    _submit(scheduler, "B", [2, 3], 3)
    results = engine.run_until_idle()
    assert len(results) == 2 and len(engine.history) == 3
    assert engine.history[0].prefill_ids == ("A", "B")
    assert (engine.history[1].decode_ids, engine.history[1].completed_ids) == (("A", "B"), ("A",))
    assert (engine.history[2].decode_ids, engine.history[2].completed_ids) == (("B",), ("B",))
    assert scheduler.waiting_count == 0 and scheduler.running_count == 0
    assert manager.allocator.allocated_count == 0
