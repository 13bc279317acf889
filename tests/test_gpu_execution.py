"""Batched prefill and decode execution (execute_prefill / execute_decode) on the GPU:
the behaviour of the reference's tests/unit/batching/test_prefill.py and test_decode.py,
with the fixture model (fp32): greedy tokens equal to independent full-recompute
generation, independent per-request caches, completion by max_new_tokens and EOS, and
invalid groups rejected before anything runs.
"""

from pathlib import Path

import pytest
import torch

from tokserve_amd.batching.execution import execute_decode, execute_prefill
from tokserve_amd.engine.config import LlamaConfig
from tokserve_amd.engine.model import LlamaModel
from tokserve_amd.engine.paged.manager import PagedKVCacheManager
from tokserve_amd.generation.generate import generate
from tokserve_amd.generation.types import GenerationConfig
from tokserve_amd.scheduler.request import ScheduledRequest

pytestmark = pytest.mark.gpu

FIXTURE = torch.load(Path(__file__).parent / "golden" / "tiny_llama_fp32.pt", weights_only=True)


@pytest.fixture()
def model(device):
    m = LlamaModel(LlamaConfig(**FIXTURE["config"]))
    m.load_state_dict(FIXTURE["state_dict"])
    return m.to(device).eval()


def _manager(model):
    c = model.config
    return PagedKVCacheManager(num_layers=c.num_hidden_layers, num_blocks=16,
                               num_key_value_heads=c.num_key_value_heads, block_size=2,
                               head_dim=c.head_dim, device=model.embed_tokens.weight.device,
                               dtype=torch.float32)


def _running(rid, prompt, device, max_new_tokens=3, eos=None):
    request = ScheduledRequest(rid, torch.tensor([prompt], device=device),
                               GenerationConfig(max_new_tokens=max_new_tokens, eos_token_id=eos))
    request.mark_running()
    return request


def _alone(model, prompt, n, device):
    return generate(model, torch.tensor([prompt], device=device),
                    GenerationConfig(max_new_tokens=n)).generated_token_ids.tolist()


def test_prefills_match_independent_generation_and_keep_separate_caches(model, device) -> None:
    manager = _manager(model)
    prompts = ([1, 2], [3, 4, 5, 6])
    a, b = (_running(rid, p, device) for rid, p in zip("AB", prompts))
    assert execute_prefill(model, manager, (a, b)) == ()
    for request, prompt in zip((a, b), prompts):
        assert request.generated_token_ids.tolist() == _alone(model, prompt, 1, device)
        assert request.prefill_complete and request.decode_ready
    first, second = manager.get_sequence("A"), manager.get_sequence("B")
    assert manager.active_sequence_ids == ("A", "B")
    assert (first.current_length, second.current_length) == (2, 4)
    assert set(first.block_ids).isdisjoint(second.block_ids)
    assert (a.sequence_length, b.sequence_length) == (3, 5)


def test_prefill_completions(model, device) -> None:
    manager = _manager(model)
    one = _running("A", [1, 2], device, max_new_tokens=1)
    assert execute_prefill(model, manager, (one,)) == ("A",)
    assert one.completion_reason == "max_new_tokens" and one.num_generated_tokens == 1
    assert not one.decode_ready
    manager = _manager(model)
    zero = _running("zero", [1, 2], device, max_new_tokens=0)
    assert execute_prefill(model, manager, (zero,)) == ("zero",)
    assert zero.completion_reason == "max_new_tokens" and zero.generated_token_ids.shape == (1, 0)
    assert manager.active_sequence_ids == () and manager.allocator.allocated_count == 0
    first = _alone(model, [1], 1, device)[0][0]
    eos = _running("eos", [1], device, max_new_tokens=4, eos=first)
    assert execute_prefill(model, _manager(model), (eos,)) == ("eos",)
    assert eos.completion_reason == "eos" and eos.generated_token_ids.tolist() == [[first]]


def test_invalid_prefill_group_is_rejected_before_execution(model, device) -> None:
    manager = _manager(model)
    waiting = ScheduledRequest("waiting", torch.tensor([[1]], device=device),
                               GenerationConfig(max_new_tokens=1))
    with pytest.raises(ValueError, match="must be running"):
        execute_prefill(model, manager, (waiting,))
    running = _running("duplicate", [1], device)
    with pytest.raises(ValueError, match="duplicate request_id"):
        execute_prefill(model, manager, (running, running))
    assert manager.active_sequence_ids == ()


def test_decode_step_matches_independent_generation(model, device) -> None:
    manager = _manager(model)
    prompts = ([1, 2], [3, 4, 5])
    a, b = (_running(rid, p, device) for rid, p in zip("AB", prompts))
    execute_prefill(model, manager, (a, b))
    before = {rid: manager.get_sequence(rid).block_ids for rid in "AB"}
    assert execute_decode(model, manager, (a, b)) == ()
    for request, prompt in zip((a, b), prompts):
        assert request.generated_token_ids.tolist() == _alone(model, prompt, 2, device)
        assert request.num_generated_tokens == 2 and request.decode_ready
    first, second = manager.get_sequence("A"), manager.get_sequence("B")
    assert (first.current_length, second.current_length) == (3, 4)
    assert set(first.block_ids).isdisjoint(second.block_ids)
    assert set(before["A"]) <= set(first.block_ids) and set(before["B"]) <= set(second.block_ids)


def test_one_request_finishes_while_another_continues(model, device) -> None:
    manager = _manager(model)
    a = _running("A", [1], device, max_new_tokens=2)
    b = _running("B", [2], device, max_new_tokens=3)
    execute_prefill(model, manager, (a, b))
    assert execute_decode(model, manager, (a, b)) == ("A",)
    assert a.completion_reason == "max_new_tokens" and not a.decode_ready
    assert b.completion_reason is None and b.decode_ready
    # EOS: A's second greedy token (30 then 23 for prompt [1]) ends it early; B goes on.
    first, second = _alone(model, [1], 2, device)[0]
    assert first != second
    manager = _manager(model)
    a = _running("A", [1], device, max_new_tokens=4, eos=second)
    b = _running("B", [2], device, max_new_tokens=4)
    assert execute_prefill(model, manager, (a, b)) == ()
    assert execute_decode(model, manager, (a, b)) == ("A",)
    assert a.completion_reason == "eos" and not a.decode_ready
    assert b.completion_reason is None and b.decode_ready


def test_adding_a_request_does_not_change_the_first_greedy_output(model, device) -> None:
    solo_manager, batch_manager = _manager(model), _manager(model)
    solo = _running("solo", [1, 2], device)
    execute_prefill(model, solo_manager, (solo,))
    execute_decode(model, solo_manager, (solo,))
    batched = _running("A", [1, 2], device)
    companion = _running("B", [7, 8, 9], device)
    execute_prefill(model, batch_manager, (batched, companion))
    execute_decode(model, batch_manager, (batched, companion))
    assert batched.generated_token_ids.tolist() == solo.generated_token_ids.tolist()


def test_invalid_decode_group_is_rejected_before_execution(model, device) -> None:
    manager = _manager(model)
    request = _running("A", [1], device)
    with pytest.raises(ValueError, match="decode-ready"):
        execute_decode(model, manager, (request,))
    execute_prefill(model, manager, (request,))
    with pytest.raises(ValueError, match="duplicate request_id"):
        execute_decode(model, manager, (request, request))
    assert manager.get_sequence("A").current_length == 1
