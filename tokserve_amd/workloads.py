"""Seeded synthetic workloads at the hot path's benchmark shapes.

Shapes (all block_size 16 unless noted):
  decode_fp32_small   8 sequences, context U[16, 512], Hq 8 / Hkv 2, Dh 64, fp32,
                      a 512-block pool with disjoint random block tables.
  norm_rope_packed    64 sequences, lengths U[1, 256] packed by cu_seqlens,
                      positions from offsets U[0, 4096]; hidden 4096, Q 32 x 128,
                      K 8 x 128, theta 500000, bf16.
  decode_llama3_8b    256 sequences, context log-uniform in [128, 8192],
                      Hq 32 / Hkv 8, Dh 128, bf16, pool sized to the total block
                      count, tables from one random permutation.
  mixed_llama3_8b     16 prefill chunks of 512 tokens on prior contexts U[0, 2048]
                      plus 240 decodes on contexts U[256, 4096], Hq 32 / Hkv 8,
                      Dh 128, bf16; step_new_rows gives the 8,432 K/V rows the
                      step appends before attention.
Random numbers come from a seeded CPU torch.Generator (small shapes) or a
seeded device generator (pool contents of the large shapes), so a workload is
a pure function of its seed.
"""

from __future__ import annotations

from dataclasses import dataclass
from math import exp, log

import torch


@dataclass
class PagedBatch:
    """A paged KV pool plus the ragged batch metadata of one attention step."""

    query: torch.Tensor           # (N, Hq, Dh): N = B for decode, packed tokens for prefill
    key_cache: torch.Tensor       # (1, NB, Hkv, BS, Dh)
    value_cache: torch.Tensor
    block_tables: torch.Tensor    # (B, max_blocks) int32
    seq_lens: torch.Tensor        # (B,) int32: keys visible to the sequence's last query
    cu_seqlens_q: torch.Tensor    # (B+1,) int32
    contexts: list[int]           # host copy of seq_lens
    query_lens: list[int]         # host copy of per-sequence query counts
    k_scale: float = 1.0          # pool decode factors (fp8 pools)
    v_scale: float = 1.0
    k_scales: torch.Tensor | None = None  # per-row decode factors (1, NB, Hkv, BS) float32
    v_scales: torch.Tensor | None = None

    @property
    def scale_kwargs(self) -> dict:
        """The pools' decode factors as the operators' keyword arguments."""

        if self.k_scales is not None:
            return {"k_scales": self.k_scales, "v_scales": self.v_scales}
        return {"k_scale": self.k_scale, "v_scale": self.v_scale}

    @property
    def num_seqs(self) -> int:
        return len(self.contexts)

    @property
    def max_seq_len(self) -> int:
        return max(self.contexts) if self.contexts else 0

    @property
    def max_query_len(self) -> int:
        return max(self.query_lens) if self.query_lens else 0

    def kv_bytes_read(self) -> int:
        """Algorithmic K+V bytes one decode pass reads: every visible key once."""

        _, _, hkv, _, dh = self.key_cache.shape
        per_row = dh * self.key_cache.element_size()
        if self.k_scales is not None:
            per_row += self.k_scales.element_size()  # each row's scale is read with it
        return sum(self.contexts) * hkv * 2 * per_row


def _tables(
    block_counts: list[int], num_blocks: int, generator: torch.Generator
) -> torch.Tensor:
    """Disjoint random block tables: one permutation of the pool split by counts."""

    total = sum(block_counts)
    if total > num_blocks:
        raise ValueError("pool too small for the requested contexts")
    perm = torch.randperm(num_blocks, generator=generator)[:total].to(torch.int32)
    width = max(block_counts) if block_counts else 1
    tables = torch.zeros((len(block_counts), max(width, 1)), dtype=torch.int32)
    start = 0
    for b, count in enumerate(block_counts):
        tables[b, :count] = perm[start : start + count]
        start += count
    return tables


def paged_batch(
    contexts: list[int],
    query_lens: list[int],
    *,
    num_q_heads: int,
    num_kv_heads: int,
    head_dim: int,
    block_size: int,
    dtype: torch.dtype,
    device: torch.device | str,
    seed: int,
    num_blocks: int | None = None,
    pool_on_device_rng: bool = False,
    kv_dtype: torch.dtype | None = None,
    k_scale: float = 1.0,
    v_scale: float = 1.0,
    scale_granularity: str = "pool",
) -> PagedBatch:
    """Build a batch where sequence b has contexts[b] keys, the last query_lens[b] of them queried.

    kv_dtype=torch.float8_e4m3fn stores the (same) pools as fp8:
    e4m3(clamp(x / scale, -448, 448)) with the given per-pool scales, or, with
    scale_granularity="row", each pool row (token, KV head) scaled by a seeded
    factor 2^U[-6, 0] first (values stay O(1)) and stored with a scale of its own,
    s = max|row| / 448.
    """

    device = torch.device(device)
    generator = torch.Generator().manual_seed(seed)
    counts = [(c + block_size - 1) // block_size for c in contexts]
    pool = num_blocks if num_blocks is not None else max(sum(counts), 1)
    tables = _tables(counts, pool, generator)
    shape = (1, pool, num_kv_heads, block_size, head_dim)
    if pool_on_device_rng:
        device_gen = torch.Generator(device=device).manual_seed(seed + 1)
        key_cache = torch.randn(shape, generator=device_gen, device=device, dtype=torch.float32)
        key_cache = key_cache.to(dtype)
        value_cache = torch.randn(shape, generator=device_gen, device=device, dtype=torch.float32)
        value_cache = value_cache.to(dtype)
    else:
        key_cache = torch.randn(shape, generator=generator).to(dtype).to(device)
        value_cache = torch.randn(shape, generator=generator).to(dtype).to(device)
    k_scales = v_scales = None
    if scale_granularity not in ("pool", "row"):
        raise ValueError('scale_granularity must be "pool" or "row"')
    if kv_dtype is not None and kv_dtype != dtype:
        if kv_dtype != torch.float8_e4m3fn:
            raise ValueError("kv_dtype must be the batch dtype or torch.float8_e4m3fn")
        if scale_granularity == "row":
            if k_scale != 1.0 or v_scale != 1.0:
                raise ValueError("per-row scales take no pool scales")
            row_gen = torch.Generator().manual_seed(seed + 2)
            pools = []
            for pool in (key_cache, value_cache):
                factor = 2.0 ** (-6.0 * torch.rand(shape[:4], generator=row_gen))
                rows = pool.float() * factor.to(pool.device).unsqueeze(-1)
                amax = rows.abs().amax(dim=-1)
                s = amax / 448.0
                s = torch.where((s > 0) & torch.isfinite(s), s, torch.ones_like(s))
                codes = (rows / s.unsqueeze(-1)).clamp(-448.0, 448.0).to(kv_dtype)
                pools.append((codes, s.contiguous()))
            (key_cache, k_scales), (value_cache, v_scales) = pools
        else:
            key_cache = (key_cache.float() / k_scale).clamp(-448.0, 448.0).to(kv_dtype)
            value_cache = (value_cache.float() / v_scale).clamp(-448.0, 448.0).to(kv_dtype)
    else:
        if scale_granularity == "row":
            raise ValueError("per-row scales need fp8 pools")
        k_scale = v_scale = 1.0
    n_tokens = sum(query_lens)
    query = torch.randn((n_tokens, num_q_heads, head_dim), generator=generator).to(dtype)
    cu = torch.zeros(len(query_lens) + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(query_lens, dtype=torch.int32), 0)
    return PagedBatch(
        query=query.to(device),
        key_cache=key_cache,
        value_cache=value_cache,
        block_tables=tables.to(device),
        seq_lens=torch.tensor(contexts, dtype=torch.int32).to(device),
        cu_seqlens_q=cu.to(device),
        contexts=list(contexts),
        query_lens=list(query_lens),
        k_scale=float(k_scale),
        v_scale=float(v_scale),
        k_scales=k_scales,
        v_scales=v_scales,
    )


def log_uniform_contexts(n: int, low: int, high: int, generator: torch.Generator) -> list[int]:
    """round(exp(U(ln low, ln high))) per sequence."""

    u = torch.rand(n, generator=generator, dtype=torch.float64)
    return [int(round(exp(log(low) + float(x) * (log(high) - log(low))))) for x in u]


def uniform_ints(n: int, low: int, high: int, generator: torch.Generator) -> list[int]:
    """n integers uniform in [low, high]."""

    return torch.randint(low, high + 1, (n,), generator=generator).tolist()


def decode_llama3_8b(
    device: torch.device | str, *, seed: int = 0, num_seqs: int = 256
) -> PagedBatch:
    """Paged decode at the Llama-3-8B layer shape (32/8 heads, Dh 128, bf16)."""

    gen = torch.Generator().manual_seed(seed)
    contexts = log_uniform_contexts(num_seqs, 128, 8192, gen)
    return paged_batch(
        contexts, [1] * num_seqs, num_q_heads=32, num_kv_heads=8, head_dim=128,
        block_size=16, dtype=torch.bfloat16, device=device, seed=seed + 7,
        pool_on_device_rng=torch.device(device).type == "cuda",
    )


def decode_llama3_8b_fp8(
    device: torch.device | str, *, seed: int = 0, num_seqs: int = 256
) -> PagedBatch:
    """The Llama-3-8B decode workload with fp8 e4m3 K/V pools (scale 1: N(0, 1) values)."""

    gen = torch.Generator().manual_seed(seed)
    contexts = log_uniform_contexts(num_seqs, 128, 8192, gen)
    return paged_batch(
        contexts, [1] * num_seqs, num_q_heads=32, num_kv_heads=8, head_dim=128,
        block_size=16, dtype=torch.bfloat16, device=device, seed=seed + 7,
        pool_on_device_rng=torch.device(device).type == "cuda", kv_dtype=torch.float8_e4m3fn,
    )


def decode_llama3_8b_fp8_rows(
    device: torch.device | str, *, seed: int = 0, num_seqs: int = 256
) -> PagedBatch:
    """The Llama-3-8B decode workload with fp8 e4m3 K/V pools and one scale per pool row
    (each row first scaled by 2^U[-6, 0], so the scales span two decades)."""

    gen = torch.Generator().manual_seed(seed)
    contexts = log_uniform_contexts(num_seqs, 128, 8192, gen)
    return paged_batch(
        contexts, [1] * num_seqs, num_q_heads=32, num_kv_heads=8, head_dim=128,
        block_size=16, dtype=torch.bfloat16, device=device, seed=seed + 7,
        pool_on_device_rng=torch.device(device).type == "cuda", kv_dtype=torch.float8_e4m3fn,
        scale_granularity="row",
    )


def decode_fp32_small(device: torch.device | str, *, seed: int = 0) -> PagedBatch:
    """8 sequences, context U[16, 512] (+1 appended token), 8/2 heads, Dh 64, fp32, 512 blocks."""

    gen = torch.Generator().manual_seed(seed)
    contexts = [c + 1 for c in uniform_ints(8, 16, 512, gen)]
    return paged_batch(
        contexts, [1] * 8, num_q_heads=8, num_kv_heads=2, head_dim=64, block_size=16,
        dtype=torch.float32, device=device, seed=seed + 7, num_blocks=512,
    )


def mixed_llama3_8b(
    device: torch.device | str, *, seed: int = 0, chunks: int = 16, decodes: int = 240,
    kv_dtype: torch.dtype | None = None,
) -> tuple[PagedBatch, PagedBatch]:
    """(prefill part, decode part) of the mixed chunked-prefill + decode step.

    Both parts share one KV pool. Prefill chunk c has 512 query tokens on a prior
    context P_c ~ U[0, 2048] (so it sees P_c + 512 keys); decode d sees
    ctx_d ~ U[256, 4096] keys. kv_dtype torch.float8_e4m3fn: fp8 pools, scale 1.
    """

    gen = torch.Generator().manual_seed(seed)
    priors = uniform_ints(chunks, 0, 2048, gen)
    decode_ctx = uniform_ints(decodes, 256, 4096, gen)
    contexts = [p + 512 for p in priors] + decode_ctx
    qlens = [512] * chunks + [1] * decodes
    full = paged_batch(
        contexts, qlens, num_q_heads=32, num_kv_heads=8, head_dim=128, block_size=16,
        dtype=torch.bfloat16, device=device, seed=seed + 7,
        pool_on_device_rng=torch.device(device).type == "cuda", kv_dtype=kv_dtype,
    )
    n_pre = chunks * 512
    cu_pre = full.cu_seqlens_q[: chunks + 1]
    prefill = PagedBatch(
        query=full.query[:n_pre], key_cache=full.key_cache, value_cache=full.value_cache,
        block_tables=full.block_tables[:chunks], seq_lens=full.seq_lens[:chunks],
        cu_seqlens_q=cu_pre, contexts=contexts[:chunks], query_lens=qlens[:chunks],
    )
    cu_dec = torch.arange(decodes + 1, dtype=torch.int32, device=full.query.device)
    decode = PagedBatch(
        query=full.query[n_pre:], key_cache=full.key_cache, value_cache=full.value_cache,
        block_tables=full.block_tables[chunks:], seq_lens=full.seq_lens[chunks:],
        cu_seqlens_q=cu_dec, contexts=contexts[chunks:], query_lens=qlens[chunks:],
    )
    return prefill, decode


@dataclass
class NewRows:
    """The K/V rows one step appends: row i goes to pool slot slots[i]."""

    key: torch.Tensor         # (N, Hkv, Dh)
    value: torch.Tensor       # (N, Hkv, Dh)
    slots: torch.Tensor       # (N,) int64: block_id * block_size + offset


def step_new_rows(parts: list[PagedBatch], *, seed: int = 3) -> NewRows:
    """The new K/V rows of a step over `parts` (e.g. the prefill and decode halves of
    mixed_llama3_8b): every query token of every sequence, in packed order, at its
    position (the last query_lens[b] of the contexts[b] positions), slot from the
    sequence's block table. Values N(0, 1) from a device generator seeded `seed`,
    rounded to the pool's model dtype (the query dtype)."""

    first = parts[0]
    device = first.query.device
    _, _, hkv, bs, dh = first.key_cache.shape
    slots: list[int] = []
    for part in parts:
        tables = part.block_tables.cpu()
        for b, (ctx, ql) in enumerate(zip(part.contexts, part.query_lens)):
            row = tables[b].tolist()
            slots.extend(row[p // bs] * bs + p % bs for p in range(ctx - ql, ctx))
    n = len(slots)
    gen = torch.Generator(device=device).manual_seed(seed)
    key = torch.randn((n, hkv, dh), generator=gen, device=device).to(first.query.dtype)
    value = torch.randn((n, hkv, dh), generator=gen, device=device).to(first.query.dtype)
    return NewRows(key, value, torch.tensor(slots, dtype=torch.int64, device=device))


@dataclass
class PackedTokens:
    """Packed ragged token stream for RMSNorm + RoPE."""

    hidden: torch.Tensor      # (N, D)
    weight: torch.Tensor      # (D,)
    query: torch.Tensor       # (N, Hq, Dh)
    key: torch.Tensor         # (N, Hkv, Dh)
    positions: torch.Tensor   # (N,) int64
    cu_seqlens: torch.Tensor  # (B+1,) int32
    theta: float
    epsilon: float


def norm_rope_packed(
    device: torch.device | str,
    *,
    seed: int = 0,
    num_seqs: int = 64,
    dtype: torch.dtype = torch.bfloat16,
    weight_dtype: torch.dtype = torch.float32,
) -> PackedTokens:
    """64 sequences, lengths U[1, 256], start positions U[0, 4096]; D 4096, 32/8 x 128."""

    gen = torch.Generator().manual_seed(seed)
    lengths = uniform_ints(num_seqs, 1, 256, gen)
    starts = uniform_ints(num_seqs, 0, 4096, gen)
    positions = torch.cat(
        [torch.arange(s, s + n, dtype=torch.int64) for s, n in zip(starts, lengths)]
    )
    n = int(positions.shape[0])
    cu = torch.zeros(num_seqs + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(torch.tensor(lengths, dtype=torch.int32), 0)
    hidden = torch.randn((n, 4096), generator=gen).to(dtype)
    weight = (1.0 + 0.02 * torch.randn(4096, generator=gen)).to(weight_dtype)
    query = torch.randn((n, 32, 128), generator=gen).to(dtype)
    key = torch.randn((n, 8, 128), generator=gen).to(dtype)
    dev = torch.device(device)
    return PackedTokens(
        hidden.to(dev), weight.to(dev), query.to(dev), key.to(dev), positions.to(dev),
        cu.to(dev), 500000.0, 1e-5,
    )


@dataclass(frozen=True)
class RequestSpec:
    request_id: str
    prompt: tuple[int, ...]
    max_new_tokens: int


def tinyllama_requests(
    *, seed: int = 0, num_requests: int = 128, min_prompt: int = 64, max_prompt: int = 1024,
    max_new_tokens: int = 128, vocab_size: int = 32_000,
) -> list[RequestSpec]:
    """End-to-end serving workload: prompt lengths U[min_prompt, max_prompt] of random
    token ids, max_new_tokens greedy tokens each (TinyLlama-1.1B shape, block size 16)."""

    generator = torch.Generator().manual_seed(seed)
    lengths = uniform_ints(num_requests, min_prompt, max_prompt, generator)
    specs = []
    for index, length in enumerate(lengths):
        ids = torch.randint(0, vocab_size, (length,), generator=generator).tolist()
        specs.append(RequestSpec(f"req{index:04d}", tuple(ids), max_new_tokens))
    return specs


def pool_blocks(specs: list[RequestSpec], block_size: int) -> int:
    """Blocks that hold every request's prompt + generated tokens at once."""

    return sum((len(s.prompt) + s.max_new_tokens + block_size - 1) // block_size for s in specs)
