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
    """Every visible K/V byte once (with its row scale when the pools have per-row
    scales), Q in and O out, block ids and lengths."""

    kv = batch.kv_bytes_read()
    qo = 2 * batch.query.numel() * batch.query.element_size()
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


BF16_ATOL = 2e-2  # bf16 outputs within 2e-2 absolute of the reference's path


def _abs_err(actual, expected) -> float:
    return float((actual.float().cpu() - expected.float()).abs().max()) if expected.numel() else 0.0


def _attention_parity(pairs: list[tuple], what: str) -> dict:
    """pairs of (GPU output, torch-backend oracle output, fp32-arithmetic oracle output):
    the largest absolute error against either of the reference's arithmetics, against
    the bf16 bound."""

    vs_torch = max(_abs_err(gpu, ref) for gpu, ref, _ in pairs)
    vs_fp32 = max(_abs_err(gpu, ref) for gpu, _, ref in pairs)
    worst = max(vs_torch, vs_fp32)
    return {"checked": what, "max_abs_err": round(worst, 6),
            "max_abs_err_vs_torch_backend": round(vs_torch, 6),
            "max_abs_err_vs_fp32_arithmetic": round(vs_fp32, 6), "atol": BF16_ATOL,
            "ok": bool(worst <= BF16_ATOL)}


def cpu_baseline(batch, out, target_seconds: float) -> tuple[dict, dict]:
    """Time the oracle's per-request decode (gather + repeat_kv + causal_attention, bf16)
    on the host over the sequences of the same workload, in batch order, repeating whole
    passes until target_seconds of CPU work (at least one full pass).

    The first pass's outputs, and one more pass in the reference kernel's arithmetic
    (fp32 scores, softmax and accumulator, one rounding on the store), check `out`, the
    GPU's output for the same batch: (baseline, parity)."""

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
    outputs = []
    while passes == 0 or elapsed < target_seconds:
        start = time.perf_counter()
        outputs = [paged.decode_batch(q, kc, vc, table, lens, 0)
                   for q, kc, vc, table, lens in requests]
        elapsed += time.perf_counter() - start
        passes += 1
    fp32 = [paged.decode_batch(q, kc, vc, table, lens, 0, torch.float32)
            for q, kc, vc, table, lens in requests]
    parity = _attention_parity([(out, torch.cat(outputs), torch.cat(fp32))],
                               f"all {batch.num_seqs} sequences x 32 heads x 128 of the timed "
                               "launch's output, against the oracle")
    baseline = {
        "value": round(per_pass * passes / elapsed / 1e9, 4),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{passes} full pass(es) over all {batch.num_seqs} sequences of the same "
                  f"workload, per-request torch-backend decode (bf16) on {cores} host "
                  f"threads, {elapsed:.1f} s",
    }
    return baseline, parity


def _cpu_threads() -> int:
    import torch

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    return cores


def _cpu_median(fn, target_seconds: float) -> tuple[float, int]:
    """Median seconds of fn() on the host after one untimed call: at least 3 runs, more
    until target_seconds have passed."""

    fn()
    times: list[float] = []
    start = time.perf_counter()
    while len(times) < 3 or time.perf_counter() - start < target_seconds:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


FP32_TOL = dict(rtol=1e-5, atol=1e-6)  # fp32 outputs within 1e-5 relative


def _close(actual, expected, rtol: float, atol: float) -> dict:
    """Largest absolute error and whether every element is within atol + rtol * |expected|."""

    actual, expected = actual.float().cpu(), expected.float()
    err = (actual - expected).abs()
    return {"max_abs_err": round(float(err.max()), 9),
            "ok": bool((err <= atol + rtol * expected.abs()).all())}


def cpu_small_fp32_step(target_seconds: float, gpu: dict | None = None) -> tuple[dict, dict]:
    """The fp32 decode step of measure_small_fp32_step through the oracle (the reference's
    torch backend, request by request): RMSNorm, RoPE of each new Q/K at its position, the
    slot write, then the paged decode of every sequence.

    gpu: the GPU's first step (normed rows, attention output, both pools): the oracle's
    step must give the same pools bit for bit and outputs within 1e-5 relative."""

    import torch

    from oracle import paged, torch_path
    from tokserve_amd import workloads

    cores = _cpu_threads()
    batch = workloads.decode_fp32_small("cpu", seed=0)
    g = torch.Generator().manual_seed(1)
    hidden = torch.randn(8, 512, generator=g)
    weight = 1.0 + 0.02 * torch.randn(512, generator=g)
    new_k = torch.randn(8, 2, 64, generator=g)
    new_v = torch.randn(8, 2, 64, generator=g)
    key_cache, value_cache = batch.key_cache.clone(), batch.value_cache.clone()

    def step():
        normed = torch_path.rms_norm(hidden, weight, 1e-5)
        rotated = []
        for b, ctx in enumerate(batch.contexts):
            q, k = torch_path.apply_rope(batch.query[b][None, :, None, :],
                                         new_k[b][None, :, None, :], torch.tensor([ctx - 1]),
                                         theta=10_000.0)
            block, offset = int(batch.block_tables[b, (ctx - 1) // 16]), (ctx - 1) % 16
            key_cache[0, block, :, offset, :] = k[0, :, 0, :]
            value_cache[0, block, :, offset, :] = new_v[b]
            rotated.append(q[0, :, 0, :])
        out = paged.decode_batch(torch.stack(rotated), key_cache, value_cache,
                                 batch.block_tables, batch.seq_lens, 0)
        return normed, out

    seconds, runs = _cpu_median(step, target_seconds)
    baseline = {"value": round(seconds * 1e6, 1), "unit": "us per step", "cores": cores,
                "kind": "port",
                "sample": f"the whole step, median of {runs} runs on {cores} host threads"}
    if gpu is None:
        return baseline, None
    normed, out = step()
    norm = _close(gpu["normed"], normed, **FP32_TOL)
    attention = _close(gpu["out"], out, **FP32_TOL)
    pools = bool(torch.equal(gpu["key_cache"].cpu(), key_cache)
                 and torch.equal(gpu["value_cache"].cpu(), value_cache))
    parity = {"checked": "the step's RMSNorm rows, attention output and both pools after "
                         "the RoPE + append, against the oracle",
              "max_abs_err": max(norm["max_abs_err"], attention["max_abs_err"]),
              "rtol": FP32_TOL["rtol"], "atol": FP32_TOL["atol"],
              "pools_bit_exact": pools, "ok": norm["ok"] and attention["ok"] and pools}
    return baseline, parity


def cpu_norm_rope(target_seconds: float, gpu: dict | None = None) -> tuple[dict, dict]:
    """The packed RMSNorm and RoPE of measure_norm_rope through the oracle (the reference's
    torch ops, bf16 in, fp32 weight): GB/s of the same algorithmic bytes.

    gpu: the GPU's outputs for the same stream (normed rows, rotated Q and K): RoPE must
    match the oracle bit for bit, and RMSNorm (fp32 out) lie within the bf16 bound (the
    oracle rounds the normalised row to bf16 before the fp32 weight)."""

    import torch

    from oracle import torch_path
    from tokserve_amd import workloads

    cores = _cpu_threads()
    data = workloads.norm_rope_packed("cpu", seed=0)
    n = data.hidden.shape[0]
    query = data.query.permute(1, 0, 2).unsqueeze(0)  # (1, Hq, N, Dh)
    key = data.key.permute(1, 0, 2).unsqueeze(0)
    norm_s, norm_runs = _cpu_median(
        lambda: torch_path.rms_norm(data.hidden, data.weight, data.epsilon), target_seconds / 2)
    rope_s, rope_runs = _cpu_median(
        lambda: torch_path.apply_rope(query, key, data.positions, theta=data.theta),
        target_seconds / 2)
    norm_bytes = n * 4096 * (2 + 4) + 4096 * 4
    rope_bytes = n * (40 * 128 * 2 * 2 + 8)
    baseline = {"rmsnorm_gbps": round(norm_bytes / norm_s / 1e9, 2),
                "rope_gbps": round(rope_bytes / rope_s / 1e9, 2), "unit": "GB/s",
                "cores": cores, "kind": "port",
                "sample": f"the whole {n}-token stream, medians of {norm_runs} / {rope_runs} "
                          f"runs on {cores} host threads"}
    if gpu is None:
        return baseline, None
    norm = _close(gpu["normed"], torch_path.rms_norm(data.hidden, data.weight, data.epsilon),
                  rtol=0.0, atol=BF16_ATOL)
    rq, rk = torch_path.apply_rope(query, key, data.positions, theta=data.theta)
    rope = bool(torch.equal(gpu["query"].cpu(), rq) and torch.equal(gpu["key"].cpu(), rk))
    parity = {"checked": f"all {n} RMSNorm rows and all rotated Q/K rows, against the oracle",
              "max_abs_err": norm["max_abs_err"], "atol": BF16_ATOL,
              "rope_bit_exact": rope, "ok": norm["ok"] and rope}
    return baseline, parity


def cpu_mixed(pre, dec, rows, pools_before, out_p, out_d,
              target_seconds: float) -> tuple[dict, dict]:
    """The whole mixed step through the oracle (the reference's torch backend, bf16,
    request by request): the append of the step's new rows into the pools as they were
    before the GPU's step (the C oracle's scatter, not timed), then all 16 chunks'
    prefill and all 240 decodes, timed until target_seconds (at least 2 runs).

    The GPU's pools after its append must equal the oracle's bit for bit, and its
    prefill and decode outputs (out_p, out_d) must lie within the bf16 bound of the
    oracle's, in both of the reference's arithmetics: (baseline, parity)."""

    import torch

    from oracle import kvslots, paged

    cores = _cpu_threads()
    k_ref, v_ref = pools_before
    kvslots.kv_append(rows.key.cpu(), rows.value.cpu(), k_ref, v_ref, rows.slots.cpu(), 0)
    pools_equal = bool(torch.equal(pre.key_cache.cpu(), k_ref)
                       and torch.equal(pre.value_cache.cpu(), v_ref))
    qp, btp, lp, cup = (pre.query.cpu(), pre.block_tables.cpu(), pre.seq_lens.cpu(),
                        pre.cu_seqlens_q.cpu())
    qd, btd, ld = dec.query.cpu(), dec.block_tables.cpu(), dec.seq_lens.cpu()

    def step(compute=None):
        return (paged.prefill_batch(qp, k_ref, v_ref, btp, lp, cup, 0, compute),
                paged.decode_batch(qd, k_ref, v_ref, btd, ld, 0, compute))

    times: list[float] = []
    first = None
    while len(times) < 2 or sum(times) < target_seconds:
        t0 = time.perf_counter()
        outputs = step()
        times.append(time.perf_counter() - t0)
        first = first or outputs
    fp32 = step(torch.float32)
    parity = _attention_parity([(out_p, first[0], fp32[0]), (out_d, first[1], fp32[1])],
                               "all 16 chunks (8,192 query rows) and all 240 decodes of the "
                               "step's output, against the oracle")
    parity["append_pools_bit_exact"] = pools_equal
    parity["ok"] = parity["ok"] and pools_equal
    times.sort()
    baseline = {"value": round(times[len(times) // 2] * 1e3, 1), "unit": "ms per step",
                "cores": cores, "kind": "port",
                "sample": f"the whole step's attention (16 prefill chunks + 240 decodes, "
                          f"request by request), median of {len(times)} runs on {cores} host "
                          "threads; the append is not timed"}
    return baseline, parity


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    # 400 launches (~0.12 s of back-to-back work) bring the GPU's clocks out of idle.
    parser.add_argument("--warmup", type=int, default=400)
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--pages-per-split", type=int, default=0)
    parser.add_argument("--cpu-seconds", type=float, default=10.0)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-secondary", action="store_true",
                        help="skip the mixed-step and packed norm/RoPE measurements")
    parser.add_argument("--secondary", default="",
                        help="comma-separated subset of the secondary measurements to run "
                             "(default: all)")
    parser.add_argument("--no-e2e", action="store_true",
                        help="skip the end-to-end TinyLlama serving run")
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

    # Parity before timing (the reference's benchmark establishes parity before it times
    # anything): the CPU baseline leg runs the oracle over the same batch, and its
    # outputs check this launch's output; a mismatch ends the run without a figure.
    step()
    torch.cuda.synchronize()
    baseline = parity = None
    if not args.no_cpu_baseline:
        baseline, parity = cpu_baseline(batch, out.clone(), args.cpu_seconds)
        if not parity["ok"]:
            print(json.dumps({"parity_failed": "decode_llama3_8b", "parity": parity}),
                  file=sys.stderr, flush=True)
            return 1

    # At least `--warmup` launches and at least 150 ms of back-to-back work: clocks
    # leave their idle state only after ~50 ms of sustained load.
    _settle(step, args.warmup)
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
    # The same launch timed alone (HIP events around each launch, no inter-launch
    # gap), then with the last-level cache flushed before each launch.
    ms_alone = _time_ms_cold(step, args.steps, torch.zeros(1, device=device))
    flush = _llc_flush_buffer(device)
    ms_cold = _time_ms_cold(step, args.steps, flush)
    del flush
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
        "per_launch": {
            "note": "each launch bracketed by its own HIP events (back-to-back steps also "
                    "hold the gap between consecutive launches)",
            "ms": round(ms_alone, 5),
            "gbps": round(total_bytes / (ms_alone * 1e-3) / 1e9, 2),
            "llc_flushed_ms": round(ms_cold, 5),
            "llc_flushed_gbps": round(total_bytes / (ms_cold * 1e-3) / 1e9, 2),
        },
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
    def cpu_or(seconds: float) -> float | None:
        return None if args.no_cpu_baseline else seconds

    if not args.no_secondary:
        secondaries = {
            "mixed_step": lambda: measure_mixed(device, 20, 5, cpu_seconds=cpu_or(3.0)),
            "mixed_step_fp8_kv": lambda: measure_mixed(device, 20, 5,
                                                       kv_dtype=torch.float8_e4m3fn),
            "prefill_long": lambda: measure_prefill_long(device),
            "norm_rope": lambda: measure_norm_rope(device, 20, 5, cpu_seconds=cpu_or(4.0)),
            "small_fp32_step": lambda: measure_small_fp32_step(device, 50, 10,
                                                               cpu_seconds=cpu_or(2.0)),
            "decode_fp8_kv": lambda: measure_decode_fp8(device, args.seed, 50, 10),
            "decode_fp8_kv_rows": lambda: measure_decode_fp8(device, args.seed, 50, 10,
                                                             rows=True),
            "decode_small_batches": lambda: measure_decode_small_batches(device, args.seed, 50,
                                                                         10),
            "decode_serving_shape": lambda: measure_decode_serving_shape(device, args.seed, 50,
                                                                         10),
        }
        chosen = [n for n in args.secondary.split(",") if n] or list(secondaries)
        unknown = set(chosen) - set(secondaries)
        if unknown:
            print(f"unknown secondary measurement(s): {sorted(unknown)}", file=sys.stderr)
            return 2
        result["secondary"] = {name: secondaries[name]() for name in chosen}
    if not args.no_e2e:
        e2e = measure_e2e(device, args.seed,
                          None if args.no_cpu_baseline else args.cpu_seconds)
        result["decode_tokens_per_s_e2e"] = e2e["tokens_per_s"]
        result.setdefault("secondary", {})["e2e_tinyllama"] = e2e
        if not args.no_secondary:
            result["secondary"]["e2e_tinyllama_fp8_kv"] = measure_e2e(
                device, args.seed, None, kv_dtype=torch.float8_e4m3fn)
            result["secondary"]["e2e_tinyllama_fp8_kv_rows"] = measure_e2e(
                device, args.seed, None, kv_dtype=torch.float8_e4m3fn, scale_granularity="row")
            result["secondary"]["e2e_tinyllama_fp32"] = measure_e2e(
                device, args.seed, None, dtype=torch.float32)
    if baseline is not None:
        result["cpu_baseline"] = baseline
    result["parity"] = parity
    checks = [parity] + [entry["parity"] for entry in result.get("secondary", {}).values()
                         if isinstance(entry, dict) and entry.get("parity")]
    result["parity_all_ok"] = None if parity is None else all(c["ok"] for c in checks)
    print(json.dumps(result), flush=True)
    if args.copy_calibration:
        copy_calibration(device)
    return 0 if result["parity_all_ok"] in (None, True) else 1


def _settle(fn, warmup: int, seconds: float = 0.15) -> None:
    """Untimed warm-up: at least `warmup` calls and at least `seconds` of back-to-back
    work, so the GPU's clocks have left their idle state (from idle, a 250 us kernel runs
    ~25 % slower in its first 5 ms of launches than after ~50 ms of sustained work)."""

    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start = time.perf_counter()
    while time.perf_counter() - start < seconds:
        for _ in range(4):
            fn()
        torch.cuda.synchronize()


def _time_ms(fn, steps: int, warmup: int) -> float:
    """Mean time of fn() over `steps` launches, HIP events on the current stream."""

    import torch

    _settle(fn, warmup)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def _time_ms_cold(fn, steps: int, flush) -> float:
    """Mean time of fn() with the last-level cache flushed before each launch: every
    launch is bracketed by its own HIP events, the flush (a read of a buffer twice the
    256 MB Infinity Cache, so no dirty lines are left to write back) stays outside them."""

    import torch

    stream = torch.cuda.current_stream()
    events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(steps)]
    for start, end in events:
        flush.sum()
        start.record(stream)
        fn()
        end.record(stream)
    torch.cuda.synchronize()
    return sum(start.elapsed_time(end) for start, end in events) / steps


def _llc_flush_buffer(device):
    import torch

    return torch.zeros(512 << 20, dtype=torch.uint8, device=device)


def measure_mixed(device, steps: int, warmup: int, kv_dtype=None,
                  cpu_seconds: float | None = None) -> dict:
    """Mixed chunked-prefill + decode step (Llama-3-8B layer shape, bf16): 16 chunks of
    512 tokens on prior contexts U[0, 2048] and 240 decodes on contexts U[256, 4096].
    kv_dtype torch.float8_e4m3fn: the same step over fp8 pools (scale 1). cpu_seconds:
    before timing, the first step's pools and outputs are checked by the CPU baseline
    leg (cpu_mixed), which runs that long."""

    import torch

    from tokserve_amd import workloads
    from tokserve_amd.kernels import ops

    pre, dec = workloads.mixed_llama3_8b(device, seed=0, kv_dtype=kv_dtype)
    scales = {"k_scale": pre.k_scale, "v_scale": pre.v_scale}
    out_p = torch.empty_like(pre.query)
    out_d = torch.empty_like(dec.query)
    order = ops.longest_first(dec.contexts, device)
    pre_order = ops.longest_first(pre.contexts, device)
    # The step's new K/V rows (every prefill token and every decode token, 8,432 rows),
    # scattered through slot_mapping into their sequences' paged blocks before attention.
    rows = workloads.step_new_rows([pre, dec])

    def append() -> None:
        ops.kv_append(rows.key, rows.value, pre.key_cache, pre.value_cache, rows.slots, 0,
                      **scales)

    def prefill() -> None:
        ops.paged_attention_prefill(
            pre.query, pre.key_cache, pre.value_cache, pre.block_tables, pre.seq_lens,
            pre.cu_seqlens_q, layer_index=0, max_query_len=pre.max_query_len,
            max_seq_len=pre.max_seq_len, out=out_p, seq_order=pre_order, **scales)

    def decode() -> None:
        ops.paged_attention_decode(
            dec.query, dec.key_cache, dec.value_cache, dec.block_tables, dec.seq_lens,
            layer_index=0, max_seq_len=dec.max_seq_len, out=out_d, seq_order=order, **scales)

    def step() -> None:
        append()
        prefill()
        decode()

    checked = None
    if cpu_seconds is not None:
        before = (pre.key_cache.cpu(), pre.value_cache.cpu())
        step()
        torch.cuda.synchronize()
        checked = cpu_mixed(pre, dec, rows, before, out_p.clone(), out_d.clone(), cpu_seconds)
        del before
    ms_app = _time_ms(append, steps, warmup)
    ms_pre = _time_ms(prefill, steps, warmup)
    ms_dec = _time_ms(decode, steps, warmup)
    ms_step = _time_ms(step, steps, warmup)
    hq, dh = 32, 128
    flops = 0
    for ctx, ql in zip(pre.contexts, pre.query_lens):
        prior = ctx - ql
        visible = ql * prior + ql * (ql + 1) // 2  # sum over queries of (prior + i + 1)
        flops += 4 * hq * dh * visible
    dec_bytes = (sum(dec.contexts) * 8 * dh * 2 * dec.key_cache.element_size()
                 + 2 * dec.query.numel() * 2)
    n_rows = rows.slots.shape[0]
    app_bytes = n_rows * (2 * 8 * 128 * 2 + 2 * 8 * 128 * pre.key_cache.element_size() + 8)
    result = {
        "workload": "mixed_llama3_8b: 16 x 512-token prefill chunks (prior U[0,2048]) + 240 "
                    "decodes (ctx U[256,4096]), Hq 32 / Hkv 8, Dh 128, block 16, bf16"
                    + ("" if kv_dtype is None else "; fp8 e4m3 K/V pools")
                    + "; step = KV append of the 8,432 new rows + prefill + decode attention",
        "ms_per_step": round(ms_step, 5),
        "append_ms": round(ms_app, 5),
        "append_gbps": round(app_bytes / (ms_app * 1e-3) / 1e9, 1),
        "prefill_ms": round(ms_pre, 5),
        "prefill_tflops": round(flops / (ms_pre * 1e-3) / 1e12, 2),
        "prefill_mfma_frac_of_2500_tflops": round(flops / (ms_pre * 1e-3) / 2.5e15, 4),
        "decode_ms": round(ms_dec, 5),
        "decode_gbps": round(dec_bytes / (ms_dec * 1e-3) / 1e9, 1),
    }
    if checked is not None:
        result["cpu_baseline"], result["parity"] = checked
    return result


def _clock_power() -> dict | None:
    """The GPU's current shader clock (MHz, the starred level of pp_dpm_sclk) and socket
    power and power cap (W, hwmon power1_input / power1_cap), read from sysfs at the
    moment of the call; None where the files are absent."""

    import glob
    import re

    for dev in sorted(glob.glob("/sys/class/drm/card*/device")):
        try:
            levels = Path(dev, "pp_dpm_sclk").read_text()
        except OSError:
            continue
        current = re.search(r"(\d+)\s*[Mm]hz\s*\*", levels)
        result = {"gfx_clock_mhz": int(current.group(1)) if current else None}
        for name, key in (("power1_input", "socket_power_w"), ("power1_cap", "power_cap_w")):
            for path in glob.glob(f"{dev}/hwmon/hwmon*/{name}"):
                try:
                    result[key] = round(int(Path(path).read_text()) / 1e6, 1)
                except (OSError, ValueError):
                    pass
        return result
    return None


def measure_prefill_long(device, seconds: float = 1.0) -> dict:
    """Long causal prefill (2 sequences x 8,192 tokens from position 0, Hq 32 / Hkv 8,
    Dh 128, block 16, bf16) over `seconds` of back-to-back launches, with the GPU's
    clocks and socket power sampled half way through: the MFMA rate the kernel reaches
    once the clocks have settled under its sustained load, and the clock that rate is
    reached at."""

    import threading

    import torch

    from tokserve_amd import workloads
    from tokserve_amd.kernels import ops

    contexts, qlens = [8192, 8192], [8192, 8192]
    pb = workloads.paged_batch(contexts, qlens, num_q_heads=32, num_kv_heads=8, head_dim=128,
                               block_size=16, dtype=torch.bfloat16, device=device, seed=1,
                               pool_on_device_rng=True)
    out = torch.empty_like(pb.query)

    def prefill() -> None:
        ops.paged_attention_prefill(
            pb.query, pb.key_cache, pb.value_cache, pb.block_tables, pb.seq_lens,
            pb.cu_seqlens_q, layer_index=0, max_query_len=8192, max_seq_len=8192, out=out)

    _settle(prefill, 5)
    sample: dict = {}
    probe = threading.Timer(seconds / 2, lambda: sample.update(_clock_power() or {}))
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    launches = 0
    begin = time.perf_counter()
    probe.start()
    start.record()
    while time.perf_counter() - begin < seconds:
        for _ in range(10):
            prefill()
        launches += 10
        torch.cuda.synchronize()
    end.record()
    torch.cuda.synchronize()
    probe.join()
    ms = start.elapsed_time(end) / launches
    flops = sum(4 * 32 * 128 * (ql * (c - ql) + ql * (ql + 1) // 2) for c, ql in zip(contexts, qlens))
    tflops = flops / (ms * 1e-3) / 1e12
    result = {
        "workload": "2 x 8,192-token causal prefill from position 0, Hq 32 / Hkv 8, Dh 128, "
                    "block 16, bf16",
        "launches": launches,
        "ms": round(ms, 5),
        "tflops": round(tflops, 1),
        "mfma_frac_of_2500_tflops": round(tflops / 2500.0, 4),
    }
    if sample.get("gfx_clock_mhz"):
        # The 2.5 PFLOP/s dense bf16 peak assumes the 2,400 MHz maximum clock.
        result["mfma_frac_of_peak_at_sampled_clock"] = round(
            tflops / (2500.0 * sample["gfx_clock_mhz"] / 2400.0), 4)
    result.update(sample)
    return result


def measure_decode_fp8(device, seed: int, steps: int, warmup: int, rows: bool = False) -> dict:
    """The headline decode workload with fp8 e4m3 K/V pools (bf16 queries and output):
    half the K/V bytes per decode token. rows: one fp32 scale per pool row, whose
    4 bytes per key row count in the algorithmic bytes."""

    import torch

    from tokserve_amd import workloads
    from tokserve_amd.kernels import ops

    if rows:
        batch = workloads.decode_llama3_8b_fp8_rows(device, seed=seed)
    else:
        batch = workloads.decode_llama3_8b_fp8(device, seed=seed)
    out = torch.empty_like(batch.query)
    order = ops.longest_first(batch.contexts, device)

    def step() -> None:
        ops.paged_attention_decode(
            batch.query, batch.key_cache, batch.value_cache, batch.block_tables,
            batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len, out=out,
            seq_order=order, **batch.scale_kwargs)

    ms = _time_ms(step, steps, warmup)
    nbytes = algorithmic_bytes(batch)
    scales = ("one fp32 scale per pool row (rows scaled by 2^U[-6, 0] first)" if rows
              else "one scale per pool")
    return {
        "workload": "decode_llama3_8b_fp8: the headline decode batch (256 seqs, ctx "
                    "log-uniform [128, 8192], Hq 32 / Hkv 8, Dh 128, block 16) with e4m3 K/V "
                    f"pools, {scales}, bf16 queries",
        "ms_per_step": round(ms, 5),
        "algorithmic_bytes": nbytes,
        "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
        "decode_tokens_per_s_one_layer": round(batch.num_seqs / (ms * 1e-3), 1),
    }


def measure_decode_serving_shape(device, seed: int, steps: int, warmup: int) -> dict:
    """Decode attention at the end-to-end serving shape: 128 sequences of the TinyLlama
    workload (prompts U[64, 1024] + 64 generated tokens), Hq 32 / Hkv 4, Dh 64, block 16,
    bf16 (auto key splits, longest-first order)."""

    import torch

    from tokserve_amd import workloads
    from tokserve_amd.kernels import ops

    contexts = [len(spec.prompt) + 64 for spec in workloads.tinyllama_requests(seed=seed)]
    batch = workloads.paged_batch(contexts, [1] * len(contexts), num_q_heads=32,
                                  num_kv_heads=4, head_dim=64, block_size=16,
                                  dtype=torch.bfloat16, device=device, seed=seed + 5,
                                  pool_on_device_rng=True)
    out = torch.empty_like(batch.query)
    order = ops.longest_first(batch.contexts, device)

    def step() -> None:
        ops.paged_attention_decode(
            batch.query, batch.key_cache, batch.value_cache, batch.block_tables,
            batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len, out=out,
            seq_order=order)

    ms_eager = _time_ms(step, steps, warmup)
    ms = _graph_ms(step, warmup)
    nbytes = algorithmic_bytes(batch)

    # The engine's decode layer: RoPE of the new query and key, the append of the new
    # K/V rows at position len - 1, and the attention, as one fused call and as the
    # RoPE + append launch followed by the decode.
    n, hq, hkv, dh = len(contexts), 32, 4, 64
    gen = torch.Generator(device=device).manual_seed(seed + 7)
    qkv = torch.randn(n, (hq + 2 * hkv) * dh, generator=gen, device=device).to(torch.bfloat16)
    query = qkv[:, : hq * dh].view(n, hq, dh)
    key = qkv[:, hq * dh : (hq + hkv) * dh].view(n, hkv, dh)
    value = qkv[:, (hq + hkv) * dh :].view(n, hkv, dh)
    pos = batch.seq_lens.to(torch.int64) - 1
    tables = batch.block_tables.to(torch.int64)
    slots = tables[torch.arange(n, device=device), pos // 16] * 16 + pos % 16
    table = ops.RotaryTable(dh, theta=10_000.0, max_position=2048, dtype=torch.bfloat16,
                            device=device)
    rotated = torch.empty_like(query)

    def fused() -> None:
        ops.rope_append_paged_decode(
            query, key, value, pos, table, batch.key_cache, batch.value_cache, slots,
            batch.block_tables, batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len,
            out=out, seq_order=order)

    def two_launches() -> None:
        ops.rope_kv_append(query, key, value, pos, table, batch.key_cache, batch.value_cache,
                           slots, 0, query_out=rotated)
        ops.paged_attention_decode(
            rotated, batch.key_cache, batch.value_cache, batch.block_tables, batch.seq_lens,
            layer_index=0, max_seq_len=batch.max_seq_len, out=out, seq_order=order)

    ms_fused = _graph_ms(fused, warmup)
    ms_two = _graph_ms(two_launches, warmup)
    return {
        "workload": "decode at the e2e serving shape: 128 seqs, ctx = prompt U[64,1024] + 64, "
                    "Hq 32 / Hkv 4, Dh 64, block 16, bf16",
        "note": "ms_per_step from a HIP graph of 20 launches (as the engine replays decode); "
                "eager launches are bound by the host's per-call cost at this size",
        "ms_per_step": round(ms, 5),
        "ms_per_step_eager": round(ms_eager, 5),
        "algorithmic_bytes": nbytes,
        "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
        "rope_append_decode": {
            "note": "a decode layer's RoPE + KV append + attention, HIP graph of 20 launches",
            "fused_ms": round(ms_fused, 5),
            "rope_kv_append_then_decode_ms": round(ms_two, 5),
        },
    }


def _graph_ms(fn, warmup: int, launches: int = 20, replays: int = 10) -> float:
    """Mean time of fn() captured `launches` times in one HIP graph, over `replays`
    replays (no host work between launches)."""

    import torch

    fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(launches):
            fn()
    return _time_ms(graph.replay, replays, max(1, warmup // launches)) / launches


def measure_decode_small_batches(device, seed: int, steps: int, warmup: int) -> dict:
    """The headline decode shape at 16, 32 and 64 sequences (auto key splits)."""

    import torch

    from tokserve_amd import workloads
    from tokserve_amd.kernels import ops

    rows = {}
    for num_seqs in (16, 32, 64):
        batch = workloads.decode_llama3_8b(device, seed=seed, num_seqs=num_seqs)
        out = torch.empty_like(batch.query)
        order = ops.longest_first(batch.contexts, device)

        def step() -> None:
            ops.paged_attention_decode(
                batch.query, batch.key_cache, batch.value_cache, batch.block_tables,
                batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len, out=out,
                seq_order=order)

        ms = _time_ms(step, steps, warmup)
        nbytes = algorithmic_bytes(batch)
        rows[str(num_seqs)] = {"ms_per_step": round(ms, 5),
                               "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1)}
        del batch, out
    return {
        "workload": "decode_llama3_8b at 16 / 32 / 64 seqs (ctx log-uniform [128, 8192], "
                    "Hq 32 / Hkv 8, Dh 128, block 16, bf16; auto key splits)",
        "by_num_seqs": rows,
    }


def measure_small_fp32_step(device, steps: int, warmup: int,
                            cpu_seconds: float | None = None) -> dict:
    """The CPU-runnable fp32 decode step (8 sequences, contexts U[16, 512] + 1, 8/2 heads,
    Dh 64, block 16, 512-block pool): RMSNorm (hidden 512, eps 1e-5), then RoPE (theta 1e4)
    of the new Q/K at each sequence's last position, the KV append through slot_mapping and
    split-K decode attention in one call (as the model layer runs them; also timed as the
    RoPE + append launch followed by the decode). Launch-bound: reported in microseconds,
    eager and as a HIP graph. cpu_seconds: before timing, the first step's outputs and
    pools are checked by the CPU baseline leg (cpu_small_fp32_step), which runs that long."""

    import torch

    from tokserve_amd import workloads
    from tokserve_amd.kernels import ops

    batch = workloads.decode_fp32_small(device, seed=0)
    g = torch.Generator().manual_seed(1)
    hidden = torch.randn(8, 512, generator=g).to(device)
    weight = (1.0 + 0.02 * torch.randn(512, generator=g)).to(device)
    normed = torch.empty_like(hidden)
    new_k = torch.randn(8, 2, 64, generator=g).to(device)
    new_v = torch.randn(8, 2, 64, generator=g).to(device)
    positions = torch.tensor([c - 1 for c in batch.contexts], dtype=torch.int64, device=device)
    tables = batch.block_tables.cpu()
    slots = torch.tensor([int(tables[b, (c - 1) // 16]) * 16 + (c - 1) % 16
                          for b, c in enumerate(batch.contexts)], dtype=torch.int64, device=device)
    table = ops.RotaryTable(64, theta=10_000.0, max_position=1024, dtype=torch.float32, device=device)
    out = torch.empty_like(batch.query)
    q_rot = torch.empty_like(batch.query)

    def step() -> None:
        ops.rms_norm(hidden, weight, 1e-5, out=normed)
        ops.rope_append_paged_decode(
            batch.query, new_k, new_v, positions, table, batch.key_cache, batch.value_cache,
            slots, batch.block_tables, batch.seq_lens, layer_index=0,
            max_seq_len=batch.max_seq_len, out=out)

    def step_two_launches() -> None:
        ops.rms_norm(hidden, weight, 1e-5, out=normed)
        ops.rope_kv_append(batch.query, new_k, new_v, positions, table, batch.key_cache,
                           batch.value_cache, slots, 0, query_out=q_rot)
        ops.paged_attention_decode(
            q_rot, batch.key_cache, batch.value_cache, batch.block_tables,
            batch.seq_lens, layer_index=0, max_seq_len=batch.max_seq_len, out=out)

    def captured(fn):
        fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn()
        return graph

    checked = None
    if cpu_seconds is not None:
        step()
        torch.cuda.synchronize()
        checked = cpu_small_fp32_step(cpu_seconds, {
            "normed": normed.clone(), "out": out.clone(), "key_cache": batch.key_cache.clone(),
            "value_cache": batch.value_cache.clone()})
    eager_us = _time_ms(step, steps, warmup) * 1e3
    graph = captured(step)
    graph_us = _time_ms(graph.replay, steps, warmup) * 1e3
    flush = _llc_flush_buffer(device)
    graph_us_cold = _time_ms_cold(graph.replay, steps, flush) * 1e3
    del flush
    graph_two = captured(step_two_launches)
    graph_two_us = _time_ms(graph_two.replay, steps, warmup) * 1e3
    kv_bytes = sum(batch.contexts) * 2 * 64 * 2 * 4
    result = {
        "workload": "decode_fp32_small: 8 seqs, ctx U[16,512]+1, Hq 8 / Hkv 2, Dh 64, block 16, "
                    "fp32; RMSNorm 512 + RoPE with KV append + decode attention",
        "step_us_eager": round(eager_us, 2),
        "step_us_graph": round(graph_us, 2),
        "step_us_graph_llc_flushed": round(graph_us_cold, 2),
        "step_us_graph_rope_append_then_decode": round(graph_two_us, 2),
        "kv_bytes": kv_bytes,
    }
    if checked is not None:
        result["cpu_baseline"], result["parity"] = checked
    return result


def measure_norm_rope(device, steps: int, warmup: int, cpu_seconds: float | None = None) -> dict:
    """RMSNorm (hidden 4096, fp32 weight -> fp32 out, the Triton wrapper's contract) and
    RoPE (32 + 8 heads x 128, theta 5e5, in place) on a packed ragged bf16 stream.

    warm: the same buffers launch after launch (the ~212 / ~170 MB streams partly stay in
    the 256 MB last-level cache). cold: launches rotate over 4 buffer sets (~850 / ~680 MB,
    more than the cache), timed back to back, so every launch reads and writes HBM; also
    the old per-launch flush measurement (a 512 MB read before each launch, each launch
    bracketed by its own HIP events). Ceiling: torch's own elementwise kernels moving the
    same bytes in the same directions (a bf16 -> fp32 conversion of the rows; copies of
    Q and K), timed the same two ways. cpu_seconds: before timing, one launch of each
    (RoPE out of place) is checked by the CPU baseline leg (cpu_norm_rope), which runs
    that long."""

    import torch

    from tokserve_amd import workloads
    from tokserve_amd.kernels import ops

    data = workloads.norm_rope_packed(device, seed=0)
    n = data.hidden.shape[0]
    sets = 4
    hidden = [data.hidden] + [data.hidden.clone() for _ in range(sets - 1)]
    outs = [torch.empty(data.hidden.shape, dtype=torch.float32, device=device)
            for _ in range(sets)]
    queries = [data.query] + [data.query.clone() for _ in range(sets - 1)]
    keys = [data.key] + [data.key.clone() for _ in range(sets - 1)]
    table = ops.RotaryTable(128, theta=data.theta, max_position=4096 + 257,
                            dtype=torch.bfloat16, device=device)

    def norm(i: int):
        return lambda: ops.rms_norm(hidden[i], data.weight, data.epsilon, out=outs[i])

    def rope(i: int):
        q4 = queries[i].permute(1, 0, 2).unsqueeze(0)
        k4 = keys[i].permute(1, 0, 2).unsqueeze(0)
        return lambda: ops.rope(q4, k4, data.positions, table, query_out=q4, key_out=k4)

    def convert(i: int):
        return lambda: outs[i].copy_(hidden[i])

    def copy(i: int):
        j = (i + 1) % sets
        return lambda: (queries[i].copy_(queries[j]), keys[i].copy_(keys[j]))

    def rotating(make):
        fns = [make(i) for i in range(sets)]
        return lambda: [fn() for fn in fns]

    checked = None
    if cpu_seconds is not None:
        q4 = data.query.permute(1, 0, 2).unsqueeze(0)
        k4 = data.key.permute(1, 0, 2).unsqueeze(0)
        normed = ops.rms_norm(data.hidden, data.weight, data.epsilon)
        rq, rk = ops.rope(q4, k4, data.positions, table)
        torch.cuda.synchronize()
        checked = cpu_norm_rope(cpu_seconds, {"normed": normed, "query": rq, "key": rk})
        del normed, rq, rk
    norm_bytes = n * 4096 * (2 + 4) + 4096 * 4
    rope_bytes = n * (40 * 128 * 2 * 2 + 8)
    result = {
        "workload": f"norm_rope_packed: 64 seqs, {n} tokens (lengths U[1,256]), hidden 4096, "
                    "Q 32 x 128 / K 8 x 128, bf16",
    }
    flush = _llc_flush_buffer(device)
    for name, make, nbytes in (("rmsnorm", norm, norm_bytes), ("rope", rope, rope_bytes),
                               ("torch_convert_same_bytes_as_rmsnorm", convert, norm_bytes),
                               ("torch_copy_same_bytes_as_rope", copy, rope_bytes)):
        warm = _time_ms(make(0), steps, warmup)
        cold = _time_ms(rotating(make), steps, warmup) / sets
        entry = {"warm_ms": round(warm, 5), "warm_gbps": round(nbytes / (warm * 1e-3) / 1e9, 1),
                 "cold_ms": round(cold, 5), "cold_gbps": round(nbytes / (cold * 1e-3) / 1e9, 1)}
        if not name.startswith("torch"):
            flushed = _time_ms_cold(make(0), steps, flush)
            entry["per_launch_flushed_ms"] = round(flushed, 5)
            entry["per_launch_flushed_gbps"] = round(nbytes / (flushed * 1e-3) / 1e9, 1)
        result[name] = entry
    del flush
    for name, ref in (("rmsnorm", "torch_convert_same_bytes_as_rmsnorm"),
                      ("rope", "torch_copy_same_bytes_as_rope")):
        result[name]["cold_frac_of_same_bytes_torch"] = round(
            result[ref]["cold_ms"] / result[name]["cold_ms"], 3)
    if checked is not None:
        result["cpu_baseline"], result["parity"] = checked
    return result


def _e2e_engine(model, specs, device, block_size: int = 16, kv_dtype=None, overlap=True,
                num_blocks: int | None = None, scale_granularity: str = "pool"):
    from tokserve_amd import workloads
    from tokserve_amd.batching.engine import ContinuousBatchEngine
    from tokserve_amd.engine.paged.manager import PagedKVCacheManager
    from tokserve_amd.scheduler.scheduler import RequestScheduler

    config = model.config
    manager = PagedKVCacheManager(
        num_layers=config.num_hidden_layers,
        num_blocks=num_blocks or workloads.pool_blocks(specs, block_size),
        num_key_value_heads=config.num_key_value_heads, block_size=block_size,
        head_dim=config.head_dim, device=device, dtype=model.embed_tokens.weight.dtype,
        kv_dtype=kv_dtype, **({} if kv_dtype is None else {"scale_granularity": scale_granularity}))
    scheduler = RequestScheduler(max_running_requests=128, cache_manager=manager)
    engine = ContinuousBatchEngine(model, scheduler, manager, overlap_decode=overlap)
    _submit(engine, specs, device)
    return engine


def _submit(engine, specs, device, prefix: str = "") -> None:
    import torch

    from tokserve_amd.generation.types import GenerationConfig
    from tokserve_amd.scheduler.request import ScheduledRequest

    for spec in specs:
        prompt = torch.tensor([spec.prompt], dtype=torch.int64, device=device)
        engine.scheduler.submit(ScheduledRequest(
            prefix + spec.request_id, prompt,
            GenerationConfig(max_new_tokens=spec.max_new_tokens)))


def measure_e2e(device, seed: int, cpu_seconds: float | None, kv_dtype=None,
                dtype=None, scale_granularity: str = "pool") -> dict:
    """TinyLlama-1.1B (random init, bf16) serving 128 requests, prompts U[64, 1024],
    128 greedy tokens each, block size 16, max 128 running: the whole run through the
    continuous-batching engine, timed on the host wall clock (each step ends with its
    tokens on the host). tokens/s = generated tokens / wall time. kv_dtype
    torch.float8_e4m3fn runs the same workload over fp8 K/V pools (scale 1, or with
    scale_granularity="row" one scale per pool row, set by each append); dtype
    torch.float32 runs it with the model in fp32 (the configuration whose greedy tokens
    must equal the reference's)."""

    import torch

    from tokserve_amd import workloads
    from tokserve_amd.engine.config import tinyllama_1_1b
    from tokserve_amd.engine.model import LlamaModel

    config = tinyllama_1_1b(max_position_embeddings=2048)
    dtype = torch.bfloat16 if dtype is None else dtype
    torch.manual_seed(seed)
    if dtype == torch.float32:
        # Drawn on the host, as the fp32 greedy-token fixture's weights were.
        model = LlamaModel(config).to(device)
    else:
        with torch.device(device):
            model = LlamaModel(config)
    model = model.to(dtype).eval()
    specs = workloads.tinyllama_requests(seed=seed)
    # The server's warm-up: each engine first serves another request set of the same
    # shape (prompts U[64, 1024] of other token ids, 128 tokens each) to completion, so
    # the library GEMM kernels are loaded and the decode HIP graphs of every (batch,
    # block-table width) the timed set meets are captured, as a server does once at
    # start-up. Then the timed set is submitted to the same engine: fresh requests,
    # every token computed, the pool's blocks all free again.
    warm = workloads.tinyllama_requests(seed=seed + 1)
    blocks = max(workloads.pool_blocks(warm, 16), workloads.pool_blocks(specs, 16))

    def serve(overlap: bool):
        engine = _e2e_engine(model, warm, device, kv_dtype=kv_dtype, overlap=overlap,
                             num_blocks=blocks, scale_granularity=scale_granularity)
        engine.run_until_idle()
        torch.cuda.synchronize()
        first, done = len(engine.history), len(engine.results)
        _submit(engine, specs, device, prefix="timed-")
        step_s = []
        start = time.perf_counter()
        while engine.scheduler.waiting_count or engine.scheduler.running_count:
            t0 = time.perf_counter()
            engine.step()
            step_s.append(time.perf_counter() - t0)
        wall = time.perf_counter() - start
        return engine.history[first:], engine.results[done:], engine, step_s, wall

    # Decode iteration i+1 queued before iteration i's tokens are read back (the
    # engine's overlap_decode), then the same run one iteration at a time.
    history, results, engine, step_s, wall = serve(True)
    *_, wall_sequential = serve(False)
    generated = sum(r.num_generated_tokens for r in results)
    decode_steps = step_s[1:]
    # Device time of one replay of the largest captured decode graph (the engine has
    # finished; a replay rewrites the last step's K/V with the same values).
    graphs = engine.executor.graphs
    replay_ms = None
    if graphs is not None and graphs._graphs:
        captured = graphs._graphs[max(graphs._graphs)]
        replay_ms = _time_ms(captured.graph.replay, 20, 3)
    pools = "" if kv_dtype is None else (
        "; fp8 e4m3 K/V pools" + (", one scale per pool row" if scale_granularity == "row" else ""))
    dtype_name = {torch.bfloat16: "bf16", torch.float32: "fp32"}.get(dtype, str(dtype))
    result = {
        "workload": "e2e_tinyllama: TinyLlama-1.1B shape (22 layers, hidden 2048, 32/4 heads, "
                    "Dh 64, MLP 5632, vocab 32000), random init, " + dtype_name + "; 128 requests, prompts "
                    "U[64,1024], 128 greedy tokens, block 16, max_running 128" + pools
                    + "; decode iteration i+1 queued before iteration i is read back; "
                    "timed on an engine warmed by another 128-request set of the same shape "
                    "(decode graphs captured once, as at server start-up)",
        "requests": len(specs),
        "prompt_tokens": sum(len(s.prompt) for s in specs),
        "generated_tokens": generated,
        "iterations": len(step_s),
        "wall_s": round(wall, 4),
        "tokens_per_s": round(generated / wall, 1),
        "tokens_per_s_one_iteration_at_a_time": round(generated / wall_sequential, 1),
        "prefill_step_s": round(step_s[0], 4),
        "decode_step_ms_mean": round(1e3 * sum(decode_steps) / max(len(decode_steps), 1), 3),
        "decode_step_ms_median": round(1e3 * sorted(decode_steps)[len(decode_steps) // 2], 3)
        if decode_steps else None,
        "decode_graph_replay_ms": None if replay_ms is None else round(replay_ms, 4),
        "decode_tokens_per_s": round(
            sum(len(r.decode_ids) for r in history[1:]) / max(sum(decode_steps), 1e-9), 1),
    }
    if dtype == torch.float32 and seed == 0:
        result["parity"] = fixture_token_parity(engine, history, "timed-")
    if cpu_seconds is not None:
        result["cpu_baseline"] = e2e_cpu_baseline(model, specs, cpu_seconds)
    return result


FP32_TOKENS = ROOT / "tests" / "golden" / "e2e_tinyllama_fp32_tokens.pt"


def fixture_token_parity(engine, history, prefix: str) -> dict | None:
    """The fp32 run's greedy tokens and iteration records against the committed fixture
    of the reference's torch backend on the same workload (made on the host by
    tests/golden/make_e2e_fp32_tokens.py): tokens match up to each request's first
    differing token (after it, the two continuations attend to different tokens)."""

    import torch

    if not FP32_TOKENS.is_file():
        return None
    fixture = torch.load(FP32_TOKENS, weights_only=True)
    matched = total = identical = 0
    first = None
    for i, rid in enumerate(fixture["request_ids"]):
        expected = fixture["tokens"][i].tolist()
        got = engine.scheduler.get_request(prefix + rid).result.generated_token_ids[0].tolist()
        total += len(expected)
        same = next((j for j, (a, b) in enumerate(zip(got, expected)) if a != b),
                    min(len(got), len(expected)))
        matched += same
        if got == expected:
            identical += 1
        elif first is None:
            first = {"request": rid, "token": same,
                     "fixture_top2_margin": float(fixture["margins"][i][same])
                     if same < len(expected) else None}

    def strip(ids):
        return [x[len(prefix):] for x in ids]

    records = [{"admitted": strip(r.admitted_ids), "prefill": strip(r.prefill_ids),
                "decode": strip(r.decode_ids), "completed": strip(r.completed_ids),
                "active": strip(r.active_ids)} for r in history]
    same_records = records == fixture["records"]
    return {"checked": f"{total} greedy tokens of {len(fixture['request_ids'])} requests and "
                       f"{len(fixture['records'])} iteration records against the fixture",
            "tokens_matched": matched, "tokens": total, "requests_identical": identical,
            "first_divergence": first, "records_identical": same_records,
            "ok": matched == total and same_records}


def e2e_cpu_baseline(model, specs, target_seconds: float) -> dict:
    """The oracle's per-request engine (the reference's torch backend, bf16) on the host:
    the first 4 requests of the same workload, engine steps until target_seconds (at
    least the prefill step and one decode step); tokens/s over the steps run."""

    import torch

    from oracle import engine as oracle_engine

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    state = {k: v.detach().cpu() for k, v in model.state_dict().items()}
    config = {k: getattr(model.config, k) for k in (
        "vocab_size", "hidden_size", "intermediate_size", "num_hidden_layers",
        "num_attention_heads", "num_key_value_heads", "max_position_embeddings",
        "rms_norm_eps", "rope_theta")}
    sample = specs[:4]
    engine = oracle_engine.Engine(state, config, num_blocks=10_000, block_size=16, max_running=128)
    for spec in sample:
        engine.submit(oracle_engine.Request(spec.request_id, list(spec.prompt),
                                            spec.max_new_tokens))
    elapsed = 0.0
    steps = 0
    while (engine.waiting or engine.running) and (steps < 2 or elapsed < target_seconds):
        start = time.perf_counter()
        engine.step()
        elapsed += time.perf_counter() - start
        steps += 1
    tokens = sum(len(r.generated) for r in
                 list(engine.running.values()) + list(engine.finished.values()))
    return {
        "value": round(tokens / elapsed, 3),
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{steps} engine steps (prefill + {steps - 1} decode) of the first "
                  f"{len(sample)} requests ({sum(len(s.prompt) for s in sample)} prompt tokens), "
                  f"per-request torch-backend forward in bf16 on {cores} host threads, "
                  f"{tokens} tokens in {elapsed:.1f} s",
    }


def copy_calibration(device, gib: int = 1, repeats: int = 5) -> None:
    """Kernels of known HBM bytes, for scaling rocprofv3 read/write counters: a plain
    device copy (`gib` GiB read and written per launch), then this library's
    tks_vector_add over two `gib`/2 GiB fp32 inputs (`gib` GiB read, `gib`/2 written)."""

    import torch

    from tokserve_amd.kernels import ops

    src = torch.empty(gib << 30, dtype=torch.uint8, device=device).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(repeats):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    half = (gib << 30) // 8  # fp32 elements of gib / 2 GiB
    x = torch.ones(half, dtype=torch.float32, device=device)
    y = torch.ones_like(x)
    out = torch.empty_like(x)
    for _ in range(repeats):
        ops.vector_add(x, y, out=out)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_per_launch": gib << 30,
                      "vector_add_read_bytes_per_launch": 2 * half * 4,
                      "vector_add_write_bytes_per_launch": half * 4, "launches": repeats}),
          flush=True)


if __name__ == "__main__":
    sys.exit(main())
