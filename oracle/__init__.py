"""CPU oracle for tokserve's continuous-batching hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what tokserve's own reference path computes
for the hot path, so that the HIP kernels in `tokserve_amd` can be checked
against it. It is the checker, never the thing measured or shipped: only
`tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py`
may import it, and nothing in `tokserve_amd` imports it.

Modules
  torch_path  the reference's torch-backend float math, op for op, with the
              same rounding points (torch CPU ops in the input dtype):
              RMSNorm, RoPE tables and rotation, repeat_kv + causal_attention,
              online-softmax tiles, greedy argmax.
  paged       paged-KV semantics on CPU pools: slots, block-table gathers,
              per-request paged attention (the torch backend's read_layer +
              causal_attention), batched decode/prefill loops.
  kvslots     ctypes binding of kvslots.c, a plain-C restatement of the
              integer/byte work (slot mapping, KV append scatter, block-table
              gather), bit-exact by construction.
  fp64        float64 NumPy closed forms (textbook attention, RoPE, RMSNorm)
              used to pin the torch-path restatement independently.
  model       the torch-backend Llama forward from a state dict, with a
              contiguous per-sequence K/V cache (greedy-token identity).
  engine      the reference's continuous-batching loop (FIFO admission under
              slot and block reservations, per-request prefill then decode,
              lowest-id block allocation) driving `model`.

Each function cites the reference file:line it follows (paths relative to the
reference repository root). Pinning: tests/test_oracle_pins.py checks every
function against the golden vectors, known answers and closed forms the
reference's own tests hold (see the docstring of each test).
"""
