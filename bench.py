"""Benchmark of the paged-attention decode step at the Llama-3-8B layer shape.

Workload: 256 sequences, context lengths log-uniform in [128, 8192], 32 query /
8 KV heads, head_dim 128, block_size 16, bf16, random block tables over a pool
sized to the total block count, Q/K/V ~ N(0, 1) (seed 0). One step is one
split-K decode launch over the whole batch (one layer).

Prints one JSON line. `value` is achieved HBM GB/s of algorithmic bytes
(every visible K/V byte once + Q + O + block tables + lengths) over the mean
kernel time measured with HIP events on the launch stream; `roofline` rates it
against MI355X's 8 TB/s; `cpu_baseline` times the oracle's per-request torch
path (the reference's torch backend) on the host for a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "paged-attn decode HBM GB/s (% of peak); decode tokens/sec on 1 MI355X"
PEAK_HBM_GBPS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "decode_llama3_8b_traffic.txt"


def algorithmic_bytes(batch) -> int:
    _, _, hkv, _, dh = batch.key_cache.shape
    elem = batch.key_cache.element_size()
    kv = sum(batch.contexts) * hkv * dh * 2 * elem
    qo = 2 * batch.query.numel() * elem
    tables = sum((c + 15) // 16 for c in batch.contexts) * 4
    return kv + qo + tables + 4 * batch.num_seqs


def measured_traffic() -> float | None:
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if present."""

    if not TRAFFIC_FILE.is_file():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        if line.startswith("hbm_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def cpu_baseline(batch, target_seconds: float) -> dict:
    """Time the oracle's per-request decode (gather + repeat_kv + causal_attention, bf16)
    on the host over the sequences of the same workload, in batch order, repeating whole
    passes until target_seconds of CPU work (at least one full pass)."""

    import torch

    from oracle import paged

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    _, _, hkv, bs, dh = batch.key_cache.shape
    elem = batch.key_cache.element_size()
    requests = []
    for b in range(batch.num_seqs):  # compact CPU pool per sequence (copy not timed)
        ctx = batch.contexts[b]
        nblk = (ctx + bs - 1) // bs
        ids = batch.block_tables[b, :nblk].long()
        requests.append((batch.query[b : b + 1].cpu(), batch.key_cache[:, ids].cpu(),
                         batch.value_cache[:, ids].cpu(),
                         torch.arange(nblk, dtype=torch.int32).unsqueeze(0),
                         torch.tensor([ctx], dtype=torch.int32)))
    per_pass = sum(c * hkv * dh * 2 * elem for c in batch.contexts) + 2 * batch.query.numel() * elem
    elapsed = 0.0
    passes = 0
    while passes == 0 or elapsed < target_seconds:
        start = time.perf_counter()
        for q, kc, vc, table, lens in requests:
            paged.decode_batch(q, kc, vc, table, lens, 0)
        elapsed += time.perf_counter() - start
        passes += 1
    return {
        "value": round(per_pass * passes / elapsed / 1e9, 4),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{passes} full pass(es) over all {batch.num_seqs} sequences of the same "
                  f"workload, per-request torch-backend decode (bf16) on {cores} host "
                  f"threads, {elapsed:.1f} s",
    }


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--pages-per-split", type=int, default=0)
    parser.add_argument("--cpu-seconds", type=float, default=10.0)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="after the bench, run a 1 GiB device copy (counter calibration)")
    args = parser.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU runs are not part of this build", file=sys.stderr)
        return 2

    import torch

    from tokserve_amd import workloads
    from tokserve_amd.kernels import ops

    device = torch.device("cuda:0")
    batch = workloads.decode_llama3_8b(device, seed=args.seed)
    out = torch.empty_like(batch.query)
    nbytes = ops.decode_workspace_bytes(batch.num_seqs, 32, 8, 128, 16, batch.max_seq_len,
                                        args.pages_per_split)
    workspace = torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=device)
    # Host-side plan from the lengths the scheduler holds: longest sequences first.
    order = ops.longest_first(batch.contexts, device)

    def step() -> None:
        ops.paged_attention_decode(
            batch.query, batch.key_cache, batch.value_cache, batch.block_tables,
            batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len, out=out,
            workspace=workspace, pages_per_split=args.pages_per_split, seq_order=order,
        )

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(device)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(args.steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps

    total_bytes = algorithmic_bytes(batch)
    achieved = total_bytes / (ms * 1e-3) / 1e9
    traffic = measured_traffic()
    result = {
        "metric": METRIC,
        "value": round(achieved, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "decode_llama3_8b: paged-attention decode, 256 seqs, context "
                        "log-uniform [128, 8192], Hq 32 / Hkv 8, Dh 128, block 16, bf16",
            "num_seqs": batch.num_seqs,
            "context_tokens": sum(batch.contexts),
            "algorithmic_bytes_per_step": total_bytes,
            "pages_per_split": args.pages_per_split or "auto",
            "schedule": "longest-first sequence order (host plan)",
        },
        "pct_of_peak_hbm": round(100.0 * achieved / PEAK_HBM_GBPS, 2),
        "decode_tokens_per_s_one_layer": round(batch.num_seqs / (ms * 1e-3), 1),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBPS, 4),
            "traffic": traffic,
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(batch, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    if args.copy_calibration:
        copy_calibration(device)
    return 0


def copy_calibration(device, gib: int = 1, repeats: int = 5) -> None:
    """A plain device copy of known size, for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE:
    each launch reads and writes exactly `gib` GiB."""

    import torch

    src = torch.empty(gib << 30, dtype=torch.uint8, device=device).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(repeats):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_per_launch": gib << 30, "launches": repeats}),
          flush=True)


if __name__ == "__main__":
    sys.exit(main())
