"""The model runs on this library's kernels: operator-call counts of one packed prefill
iteration and one decode iteration of the batched executor, and of the reference-API
per-sequence forward, recorded with a dispatch mode (the analogue of the reference's
call-count check that its custom kernels ran, tests/gpu/test_tiled_attention_end_to_end.py:237-290).

Over pools in the model dtype and over fp8 pools alike, per layer a packed iteration makes
two RMSNorm launches (the first layer's input norm without a residual), one SiLU*mul, and
either one RoPE + KV append and one prefill attention launch (an iteration with prefill
tokens) or one fused RoPE + KV append + decode attention call (a decode-only iteration);
the final norm and one greedy argmax close it. No softmax, matmul-based attention or
gather of the pools runs in torch.
"""

from collections import Counter

import pytest
import torch
from torch.utils._python_dispatch import TorchDispatchMode

from tokserve_amd.batching.execution import BatchExecutor
from tokserve_amd.engine.config import LlamaConfig
from tokserve_amd.engine.model import LlamaModel
from tokserve_amd.engine.paged.manager import PagedKVCacheManager
from tokserve_amd.generation.types import GenerationConfig
from tokserve_amd.scheduler.request import ScheduledRequest
from tokserve_amd.scheduler.scheduler import RequestScheduler

pytestmark = pytest.mark.gpu

LAYERS = 3
# Operators whose presence would mean attention or normalisation ran in torch.
TORCH_FALLBACKS = ("aten::_softmax", "aten::softmax", "aten::bmm", "aten::baddbmm",
                   "aten::rsqrt", "aten::masked_fill", "aten::repeat_interleave")


class _Calls(TorchDispatchMode):
    def __init__(self) -> None:
        super().__init__()
        self.count: Counter = Counter()

    def __torch_dispatch__(self, func, types, args=(), kwargs=None):
        self.count[func._schema.name] += 1
        return func(*args, **(kwargs or {}))


def _ours(count: Counter) -> Counter:
    return Counter({name.split("::", 1)[1]: n for name, n in count.items()
                    if name.startswith("tokserve_amd::")})


def _model(device, dtype) -> LlamaModel:
    torch.manual_seed(0)
    config = LlamaConfig(vocab_size=512, hidden_size=256, intermediate_size=512,
                         num_hidden_layers=LAYERS, num_attention_heads=4, num_key_value_heads=2,
                         max_position_embeddings=256)
    with torch.device(device):
        model = LlamaModel(config)
    return model.to(dtype).eval()


@pytest.mark.parametrize("dtype, kv_dtype", [(torch.bfloat16, None), (torch.float32, None),
                                             (torch.bfloat16, torch.float8_e4m3fn)])
def test_packed_iterations_launch_only_library_kernels(device, dtype, kv_dtype) -> None:
    model = _model(device, dtype)
    config = model.config
    scales = dict(k_scale=0.5, v_scale=0.25) if kv_dtype is not None else {}
    manager = PagedKVCacheManager(num_layers=LAYERS, num_blocks=64,
                                  num_key_value_heads=config.num_key_value_heads, block_size=16,
                                  head_dim=config.head_dim, device=device, dtype=dtype,
                                  kv_dtype=kv_dtype, **scales)
    scheduler = RequestScheduler(max_running_requests=8, cache_manager=manager)
    executor = BatchExecutor(model, manager, use_graphs=False)
    for index, length in enumerate((37, 5, 64)):
        prompt = torch.randint(0, config.vocab_size, (1, length), device=device)
        scheduler.submit(ScheduledRequest(f"r{index}", prompt,
                                          GenerationConfig(max_new_tokens=4)))
    running = scheduler.schedule().admitted_requests
    assert len(running) == 3

    with _Calls() as prefill:
        executor.execute(running, ())
    with _Calls() as decode:
        executor.execute((), running)
    torch.cuda.synchronize()

    pre, dec = _ours(prefill.count), _ours(decode.count)
    assert pre["rope_kv_append_"] + pre["rope_kv_append"] == LAYERS, pre
    assert pre["rope"] + pre["rope_"] + pre["kv_append"] == 0, pre
    assert pre["paged_attention_prefill"] == LAYERS, pre
    assert pre["paged_attention_decode"] + pre["rope_append_paged_decode"] == 0, pre
    assert dec["rope_append_paged_decode"] == LAYERS, dec
    assert dec["rope_kv_append_"] + dec["rope_kv_append"] == 0, dec
    assert dec["rope"] + dec["rope_"] + dec["kv_append"] == 0, dec
    assert dec["paged_attention_prefill"] + dec["paged_attention_decode"] == 0, dec
    for calls in (prefill, decode):
        ours = _ours(calls.count)
        assert ours["rms_norm"] == 2 * LAYERS + 1, ours
        assert ours["silu_mul"] == LAYERS, ours
        assert ours["greedy_argmax"] == 1, ours
        assert ours["paged_gather"] == 0, ours
        assert not [name for name in calls.count if name in TORCH_FALLBACKS], calls.count


def test_reference_api_forward_launches_library_kernels(device) -> None:
    model = _model(device, torch.float32)
    prompt = torch.randint(0, model.config.vocab_size, (1, 21), device=device)
    with _Calls() as calls:
        logits = model(prompt)
    torch.cuda.synchronize()
    assert logits.shape == (1, 21, model.config.vocab_size)
    ours = _ours(calls.count)
    assert ours["rms_norm"] >= 2 * LAYERS + 1, ours
    assert ours["rope"] + ours["rope_"] == LAYERS, ours
    assert ours["paged_attention_prefill"] + ours["paged_attention_decode"] == LAYERS, ours
    assert ours["silu_mul"] == LAYERS, ours
    assert not [name for name in calls.count if name in TORCH_FALLBACKS], calls.count
