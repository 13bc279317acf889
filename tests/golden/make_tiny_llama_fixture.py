"""Writes tests/golden/tiny_llama_fp32.pt from the reference's own LlamaModel.

Run in a container that holds the reference checkout (default path below):
    python tests/golden/make_tiny_llama_fixture.py [/path/to/reference]

What the fixture pins, and why an import is needed for it: the random weights
LlamaModel(config) draws under torch.manual_seed depend on the order in which
the reference creates its modules (tokserve/engine/model.py:101-117,
attention.py:154-173, layers.py:27,63-77), and the logits depend on the order of
its ops; no closed form fixes either. The fixture holds, for a tiny fp32
config on the CPU (torch backend):
  state_dict       every parameter after torch.manual_seed(1234); LlamaModel(config)
  prompt_logits    model(prompt) without a cache, (1, 7, 64)
  decode_tokens    greedy tokens of prefill_paged + decode_paged over a paged pool
  decode_logits    the last-position logits of each of those steps
  block_ids        the sequence's physical blocks at the end
Only data is written; no reference source is copied.
"""

from __future__ import annotations

import sys
from pathlib import Path

import torch

CONFIG = dict(vocab_size=64, hidden_size=32, intermediate_size=64, num_hidden_layers=2,
              num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64,
              rms_norm_eps=1e-6, rope_theta=10_000.0)
SEED = 1234
PROMPT = [3, 14, 15, 9, 2, 6, 5]
STEPS = 6
BLOCK_SIZE = 4
NUM_BLOCKS = 8


def main() -> None:
    reference = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, reference)
    from tokserve.engine.model import LlamaModel
    from tokserve.engine.paged.inference import decode_paged, prefill_paged
    from tokserve.engine.paged.manager import PagedKVCacheManager
    from tokserve.reference.llama.config import LlamaConfig

    config = LlamaConfig(**CONFIG)
    torch.manual_seed(SEED)
    model = LlamaModel(config).eval()
    prompt = torch.tensor([PROMPT], dtype=torch.int64)
    with torch.inference_mode():
        prompt_logits = model(prompt)
        manager = PagedKVCacheManager(num_layers=config.num_hidden_layers, num_blocks=NUM_BLOCKS,
                                      num_key_value_heads=config.num_key_value_heads,
                                      block_size=BLOCK_SIZE, head_dim=config.head_dim,
                                      device=torch.device("cpu"), dtype=torch.float32)
        result = prefill_paged(model, prompt, manager, sequence_id="s")
        last = result.logits[:, -1, :]
        tokens, step_logits = [], [last[0].clone()]
        for _ in range(STEPS):
            token = torch.argmax(last, dim=-1, keepdim=True)
            tokens.append(int(token))
            last = decode_paged(model, token, result.cache)[:, -1, :]
            step_logits.append(last[0].clone())
        block_ids = list(result.cache.block_ids)
    fixture = {
        "config": CONFIG, "seed": SEED, "prompt": PROMPT, "block_size": BLOCK_SIZE,
        "num_blocks": NUM_BLOCKS,
        "state_dict": {k: v.detach().clone() for k, v in model.state_dict().items()},
        "prompt_logits": prompt_logits.detach().clone(),
        "decode_tokens": tokens, "decode_logits": torch.stack(step_logits),
        "block_ids": block_ids,
    }
    out = Path(__file__).with_name("tiny_llama_fp32.pt")
    torch.save(fixture, out)
    print(f"wrote {out} ({out.stat().st_size} bytes); tokens {tokens}; blocks {block_ids}")


if __name__ == "__main__":
    main()
