"""Writes tests/golden/e2e_tinyllama_fp32_tokens.pt: the greedy tokens the reference's
torch backend produces for the end-to-end serving workload in fp32.

Run on the CPU (about an hour on 8 cores; no GPU and no reference checkout needed):
    python tests/golden/make_e2e_fp32_tokens.py [--max-new-tokens 128] [--threads N]
(--num-requests and --out make a smaller file elsewhere, for a quick check of the script.)

Workload: TinyLlama-1.1B shape (22 layers, hidden 2048, 32 query / 4 KV heads of 64,
MLP 5632, vocabulary 32000, eps 1e-5, theta 1e4), random init on the CPU under
torch.manual_seed(0) -- LlamaModel's parameter order is the reference's, so these are
the weights tokserve/engine/model.py:101-117 draws under that seed -- served in fp32 to
the 128 requests of workloads.tinyllama_requests(seed=0) (prompts U[64, 1024] of random
token ids), block size 16, max 128 running, 128 greedy tokens each.

The tokens come from oracle/engine.py, the reference's continuous-batching loop
(tokserve/batching/engine.py:65-131, scheduler/scheduler.py:58-159,
batching/execution.py:21-101) driving the reference's torch-backend forward
(oracle/model.py) request by request. The fixture holds only data:
  config, seed, weights_sha256   the model and a digest of its fp32 parameters (in
                                 state_dict order), so a loader can check it rebuilt
                                 the same weights
  request_ids, prompt_lengths    the workload
  tokens        (R, T) int32     greedy token ids per request
  margins       (R, T) float32   top-1 minus top-2 logit of the step that chose each token
  records       list of dicts    each iteration's admitted / prefill / decode /
                                 completed / active request ids
  released_blocks                each request's physical block ids when it completed
"""

from __future__ import annotations

import argparse
import hashlib
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import engine as oracle_engine  # noqa: E402
from oracle import model as oracle_model  # noqa: E402
from tokserve_amd import workloads  # noqa: E402
from tokserve_amd.engine.config import tinyllama_1_1b  # noqa: E402
from tokserve_amd.engine.model import LlamaModel  # noqa: E402

OUT = Path(__file__).with_name("e2e_tinyllama_fp32_tokens.pt")
SEED = 0
BLOCK_SIZE = 16
MAX_RUNNING = 128
CONFIG_KEYS = ("vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers",
               "num_attention_heads", "num_key_value_heads", "max_position_embeddings",
               "rms_norm_eps", "rope_theta")


def build_model() -> LlamaModel:
    """The fp32 model of the workload, drawn on the CPU under torch.manual_seed(SEED)."""

    torch.manual_seed(SEED)
    return LlamaModel(tinyllama_1_1b(max_position_embeddings=2048)).eval()


def weights_sha256(model: LlamaModel) -> str:
    """Digest of every parameter's fp32 bytes, in state_dict order (CPU tensors)."""

    digest = hashlib.sha256()
    for name, tensor in model.state_dict().items():
        digest.update(name.encode())
        digest.update(tensor.detach().to("cpu", torch.float32).contiguous().numpy().tobytes())
    return digest.hexdigest()


class MarginEngine(oracle_engine.Engine):
    """The oracle engine, also keeping the top-1 minus top-2 logit of every chosen token."""

    def __init__(self, *args, **kwargs) -> None:
        super().__init__(*args, **kwargs)
        self.margins: dict[str, list[float]] = {}

    def _next_token(self, request, tokens):
        ids = torch.tensor([tokens], dtype=torch.int64)
        logits = oracle_model.forward(self.state, self.config, ids, request.kv, self.kv_quant)
        top = torch.topk(logits[0, -1], 2)
        self.margins.setdefault(request.request_id, []).append(
            float(top.values[0] - top.values[1]))
        return int(torch.argmax(logits[0, -1]))


def main() -> None:
    parser = argparse.ArgumentParser()
    parser.add_argument("--max-new-tokens", type=int, default=128)
    parser.add_argument("--threads", type=int, default=0)
    parser.add_argument("--num-requests", type=int, default=128)
    parser.add_argument("--out", type=Path, default=OUT)
    args = parser.parse_args()
    if args.threads:
        torch.set_num_threads(args.threads)

    model = build_model()
    config = {k: getattr(model.config, k) for k in CONFIG_KEYS}
    state = {k: v.detach() for k, v in model.state_dict().items()}
    specs = workloads.tinyllama_requests(seed=SEED, max_new_tokens=args.max_new_tokens)
    specs = specs[: args.num_requests]
    engine = MarginEngine(state, config, num_blocks=workloads.pool_blocks(specs, BLOCK_SIZE),
                          block_size=BLOCK_SIZE, max_running=MAX_RUNNING)
    for spec in specs:
        engine.submit(oracle_engine.Request(spec.request_id, list(spec.prompt),
                                            spec.max_new_tokens))
    start = time.perf_counter()
    with torch.inference_mode():
        while engine.waiting or engine.running:
            record = engine.step()
            print(f"iteration {record.iteration}: {len(record.prefill_ids)} prefills, "
                  f"{len(record.decode_ids)} decodes, {time.perf_counter() - start:.0f} s",
                  flush=True)
    ids = [s.request_id for s in specs]
    finished = engine.finished
    torch.save({
        "config": config,
        "seed": SEED,
        "weights_sha256": weights_sha256(model),
        "block_size": BLOCK_SIZE,
        "max_running": MAX_RUNNING,
        "num_blocks": engine.num_blocks,
        "max_new_tokens": args.max_new_tokens,
        "request_ids": ids,
        "prompt_lengths": [len(s.prompt) for s in specs],
        "tokens": torch.tensor([finished[r].generated for r in ids], dtype=torch.int32),
        "margins": torch.tensor([engine.margins[r] for r in ids], dtype=torch.float32),
        "records": [{"admitted": list(r.admitted_ids), "prefill": list(r.prefill_ids),
                     "decode": list(r.decode_ids), "completed": list(r.completed_ids),
                     "active": list(r.active_ids)} for r in engine.records],
        "released_blocks": {r: list(finished[r].released_blocks) for r in ids},
    }, args.out)
    print(f"wrote {args.out} ({time.perf_counter() - start:.0f} s)", flush=True)


if __name__ == "__main__":
    main()
