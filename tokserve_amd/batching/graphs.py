"""HIP-graph replay of decode-only iterations.

A decode iteration of a serving batch is ~12 kernel launches per layer plus
host work per launch: at batch 128 on a 22-layer model the host, not the GPU,
sets the step time. A decode-only iteration with B sequences whose block
tables fit W blocks always launches the same kernels with the same grids, so
it is captured once per (B, W) into a HIP graph and replayed: per step, the
new metadata (tokens, positions, slots, lengths, block tables, order) is
copied into the graph's static buffers with one host -> device copy, the graph
replays, and the greedy tokens come back with one device -> host copy.

Static metadata layout for (B, W): token_ids, positions, slot_mapping,
logits_rows (B int64 each), decode_seq_lens (B int32), decode_block_tables
(B x W int32, unused entries 0), decode_seq_order (B int32), each section
16-byte aligned in one device byte buffer. The decode kernels are launched
with max_seq_len = W * block_size, the bound every sequence of the graph
stays within. W is rounded up to a multiple of `width_quantum` blocks so that
growing sequences reuse a graph for many steps.

The first iteration of a new shape runs eagerly (which also allocates the
decode workspace, the RoPE table and the fused weights outside the capture),
then the same metadata is captured; the capture records and does not execute.

Two pinned staging buffers alternate, each reused only once the copy out of
it has completed (an event per buffer), so the host can fill the next
iteration's metadata while the previous one's copy and replay are still
queued. An iteration's token ids may come from a device tensor instead of
the host (the previous iteration's greedy tokens, copied device to device
after the metadata): the host then need not have read them back yet.
"""

from __future__ import annotations

import numpy as np
import torch

from tokserve_amd.batching.metadata import PackedBatch, SequenceWork
from tokserve_amd.kernels import ops

__all__ = ["DecodeGraphs"]


class _Captured:
    def __init__(self, graph, static: torch.Tensor, logits: torch.Tensor, tokens: torch.Tensor,
                 offsets: dict[str, tuple[int, int]]) -> None:
        self.graph, self.static, self.logits, self.tokens, self.offsets = (
            graph, static, logits, tokens, offsets)


class DecodeGraphs:
    """Captured decode iterations keyed by (batch size, block-table width)."""

    def __init__(self, model, storage, *, width_quantum: int = 64, max_graphs: int = 64) -> None:
        self.model = model
        self.storage = storage
        self.block_size = storage.block_size
        self.device = storage.device
        self.width_quantum = width_quantum
        self.max_graphs = max_graphs
        self._graphs: dict[tuple[int, int], _Captured] = {}
        self._staging: list[torch.Tensor | None] = [None, None]
        self._staged: list[torch.cuda.Event | None] = [None, None]
        self._turn = 0

    def supported(self) -> bool:
        return self.device.type == "cuda"

    def width_for(self, works: list[SequenceWork]) -> int:
        blocks = max((w.start + 1 + self.block_size - 1) // self.block_size for w in works)
        q = self.width_quantum
        return (blocks + q - 1) // q * q

    def _layout(self, b: int, w: int) -> tuple[dict[str, tuple[int, int, torch.dtype, tuple]], int]:
        sections = [("token_ids", 8 * b, torch.int64, (b,)), ("positions", 8 * b, torch.int64, (b,)),
                    ("slot_mapping", 8 * b, torch.int64, (b,)),
                    ("logits_rows", 8 * b, torch.int64, (b,)),
                    ("decode_seq_lens", 4 * b, torch.int32, (b,)),
                    ("decode_block_tables", 4 * b * w, torch.int32, (b, w)),
                    ("decode_seq_order", 4 * b, torch.int32, (b,))]
        layout = {}
        total = 0
        for name, nbytes, dtype, shape in sections:
            layout[name] = (total, nbytes, dtype, shape)
            total += (nbytes + 15) // 16 * 16
        return layout, total

    def _host_bytes(self, works: list[SequenceWork], w: int) -> np.ndarray:
        b = len(works)
        bs = self.block_size
        layout, total = self._layout(b, w)
        out = np.zeros(total, dtype=np.uint8)
        starts = np.fromiter((wk.start for wk in works), dtype=np.int64, count=b)
        # Every sequence's block ids in one flat array, scattered into the (B, W) table.
        widths = np.fromiter((len(wk.block_ids) for wk in works), dtype=np.int64, count=b)
        flat = np.concatenate([np.asarray(wk.block_ids) for wk in works])
        rows = np.repeat(np.arange(b), widths)
        cols = np.arange(flat.size) - np.repeat(np.cumsum(widths) - widths, widths)
        tables = np.zeros((b, w), dtype=np.int32)
        tables[rows, cols] = flat
        lens = (starts + 1).astype(np.int32)
        values = {
            "token_ids": np.fromiter((wk.tokens[0] for wk in works), dtype=np.int64, count=b),
            "positions": starts,
            "slot_mapping": tables[np.arange(b), starts // bs].astype(np.int64) * bs + starts % bs,
            "logits_rows": np.arange(b, dtype=np.int64),
            "decode_seq_lens": lens,
            "decode_block_tables": tables,
            "decode_seq_order": np.argsort(-lens, kind="stable").astype(np.int32),
        }
        for name, (begin, nbytes, _, _) in layout.items():
            out[begin : begin + nbytes] = np.ascontiguousarray(values[name]).view(np.uint8).reshape(-1)
        return out

    def _batch(self, static: torch.Tensor, b: int, w: int) -> PackedBatch:
        layout, _ = self._layout(b, w)
        views = {name: static[begin : begin + nbytes].view(dtype).view(shape)
                 for name, (begin, nbytes, dtype, shape) in layout.items()}
        empty32 = torch.empty(0, dtype=torch.int32, device=self.device)
        return PackedBatch(
            num_prefill_tokens=0, prefill_cu_seqlens_q=empty32, prefill_seq_lens=empty32,
            prefill_block_tables=empty32.view(0, 1), prefill_seq_order=empty32,
            prefill_max_query_len=0,
            prefill_max_seq_len=0, decode_max_seq_len=w * self.block_size, **views)

    def _upload(self, host: np.ndarray, static: torch.Tensor, b: int,
                token_source: torch.Tensor | None) -> None:
        turn = self._turn
        self._turn ^= 1
        n = host.nbytes
        if self._staged[turn] is not None:
            self._staged[turn].synchronize()  # the copy out of this buffer has run
        staging = self._staging[turn]
        if staging is None or staging.numel() < n:
            staging = torch.empty(max(n, 1 << 16), dtype=torch.uint8, pin_memory=True)
            self._staging[turn] = staging
        staging[:n].numpy()[:] = host
        static[:n].copy_(staging[:n], non_blocking=True)
        if self._staged[turn] is None:
            self._staged[turn] = torch.cuda.Event()
        self._staged[turn].record()
        if token_source is not None:
            # token_ids is the first section of the layout
            static[: 8 * b].view(torch.int64).copy_(token_source, non_blocking=True)

    def run(self, works: list[SequenceWork], *,
            token_source: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """Logits (B, V) and greedy tokens (B,) of one decode-only iteration.
        token_source: (B,) int64 device tensor of the token ids, in place of the works'
        tokens (read on the stream, after everything queued before this call)."""

        b = len(works)
        w = self.width_for(works)
        key = (b, w)
        host = self._host_bytes(works, w)
        captured = self._graphs.get(key)
        if captured is not None:
            self._upload(host, captured.static, b, token_source)
            captured.graph.replay()
            return captured.logits, captured.tokens
        _, total = self._layout(b, w)
        static = torch.zeros(total, dtype=torch.uint8, device=self.device)
        self._upload(host, static, b, token_source)
        batch = self._batch(static, b, w)
        logits = self.model.forward_packed(batch, self.storage)  # eager: this step's result
        tokens = ops.greedy_argmax(logits).view(-1)
        if len(self._graphs) < self.max_graphs:
            torch.cuda.synchronize(self.device)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                g_logits = self.model.forward_packed(batch, self.storage)
                g_tokens = ops.greedy_argmax(g_logits).view(-1)
            self._graphs[key] = _Captured(graph, static, g_logits, g_tokens, {})
        return logits, tokens
