"""Packed ragged-batch metadata of one continuous-batching iteration.

One iteration of the engine runs every prefill chunk and every decode token
of the running sequences as a single packed token stream of N rows:
prefill chunks first (sequence order of the plan), then one row per decode
sequence. The metadata is the layout the kernels take (the batch-metadata
names of the hot path):

  token_ids      (N,) int64   tokens appended this iteration
  positions      (N,) int64   absolute position of each row
  slot_mapping   (N,) int64   pool slot block_ids[p // BS] * BS + p % BS of each row
  prefill_*      cu_seqlens_q (Bp+1,) int32, seq_lens (Bp,) int32 (keys after
                 the append), block_tables (Bp, W) int32, seq_order (Bp,) int32
                 (most keys first, the order chunks reach the GPU)
  decode_*       seq_lens (Bd,) int32, block_tables (Bd, W) int32, seq_order
                 (Bd,) int32 (longest first, the order sequences reach the GPU)
  logits_rows    (B,) int64   row of each sequence's last token

Everything is built on the host with NumPy in one byte buffer and moved to the
device with a single asynchronous copy from a reused pinned staging buffer.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import numpy as np
import torch

__all__ = ["SequenceWork", "PackedBatch", "PackedBatchBuilder"]


@dataclass(frozen=True)
class SequenceWork:
    """One sequence's share of an iteration: `tokens` appended at positions
    start .. start + len(tokens) - 1, through the sequence's block table."""

    tokens: Sequence[int] | np.ndarray
    start: int
    block_ids: Sequence[int]


@dataclass
class PackedBatch:
    token_ids: torch.Tensor
    positions: torch.Tensor
    slot_mapping: torch.Tensor
    logits_rows: torch.Tensor
    num_prefill_tokens: int
    prefill_cu_seqlens_q: torch.Tensor
    prefill_seq_lens: torch.Tensor
    prefill_block_tables: torch.Tensor
    prefill_max_query_len: int
    prefill_max_seq_len: int
    prefill_seq_order: torch.Tensor
    decode_seq_lens: torch.Tensor
    decode_block_tables: torch.Tensor
    decode_seq_order: torch.Tensor
    decode_max_seq_len: int

    @property
    def num_tokens(self) -> int:
        return int(self.token_ids.shape[0])

    @property
    def num_sequences(self) -> int:
        return int(self.logits_rows.shape[0])


class PackedBatchBuilder:
    """Builds PackedBatch objects for one device and block size.

    The pinned staging buffer is reused across iterations; a new build may only
    start after the previous iteration's copy has completed, which the engine
    guarantees by reading the iteration's tokens back before the next build.
    """

    def __init__(self, device: torch.device, block_size: int) -> None:
        self.device = torch.device(device)
        self.block_size = block_size
        self._staging: torch.Tensor | None = None

    def build(self, prefill: list[SequenceWork], decode: list[SequenceWork]) -> PackedBatch:
        if not prefill and not decode:
            raise ValueError("an iteration needs at least one sequence")
        for work in decode:
            if len(work.tokens) != 1:
                raise ValueError("a decode sequence appends exactly one token")
        bs = self.block_size
        works = prefill + decode
        lengths = np.array([len(w.tokens) for w in works], dtype=np.int64)
        if (lengths < 1).any():
            raise ValueError("every sequence must append at least one token")
        starts = np.array([w.start for w in works], dtype=np.int64)
        n = int(lengths.sum())
        token_ids = np.concatenate([np.asarray(w.tokens, dtype=np.int64) for w in works])
        offsets = np.concatenate(([0], np.cumsum(lengths)))
        row_seq = np.repeat(np.arange(len(works)), lengths)
        positions = starts[row_seq] + (np.arange(n) - offsets[row_seq])
        ends = starts + lengths  # keys of each sequence after the append
        width = max(1, int(max((len(w.block_ids) for w in works), default=1)))
        tables = np.zeros((len(works), width), dtype=np.int32)
        for i, w in enumerate(works):
            needed = (int(ends[i]) + bs - 1) // bs
            if len(w.block_ids) < needed:
                raise ValueError("block table does not cover the appended positions")
            tables[i, : len(w.block_ids)] = w.block_ids
        slot_mapping = tables[row_seq, positions // bs].astype(np.int64) * bs + positions % bs
        n_pre = len(prefill)
        num_prefill_tokens = int(offsets[n_pre])
        logits_rows = offsets[1:] - 1
        cu = offsets[: n_pre + 1].astype(np.int32)
        dec_lens = ends[n_pre:].astype(np.int32)
        order = np.argsort(-dec_lens, kind="stable").astype(np.int32)
        pre_order = np.argsort(-ends[:n_pre], kind="stable").astype(np.int32)

        sections = [
            ("token_ids", token_ids), ("positions", positions.astype(np.int64)),
            ("slot_mapping", slot_mapping), ("logits_rows", logits_rows.astype(np.int64)),
            ("prefill_cu_seqlens_q", cu), ("prefill_seq_lens", ends[:n_pre].astype(np.int32)),
            ("prefill_block_tables", tables[:n_pre]), ("prefill_seq_order", pre_order),
            ("decode_seq_lens", dec_lens),
            ("decode_block_tables", tables[n_pre:]), ("decode_seq_order", order),
        ]
        layout = []
        total = 0
        for name, array in sections:
            array = np.ascontiguousarray(array)
            layout.append((name, total, array))
            total += (array.nbytes + 15) // 16 * 16
        staging = self._staging_buffer(total)
        host = staging.numpy()
        for _, begin, array in layout:
            host[begin : begin + array.nbytes] = array.view(np.uint8).reshape(-1)
        device_bytes = staging[:total].to(self.device, non_blocking=True)
        fields = {}
        for name, begin, array in layout:
            dtype = torch.int64 if array.dtype == np.int64 else torch.int32
            view = device_bytes[begin : begin + array.nbytes].view(dtype)
            fields[name] = view.view(array.shape)
        return PackedBatch(
            num_prefill_tokens=num_prefill_tokens,
            prefill_max_query_len=int(lengths[:n_pre].max()) if n_pre else 0,
            prefill_max_seq_len=int(ends[:n_pre].max()) if n_pre else 0,
            decode_max_seq_len=int(dec_lens.max()) if len(decode) else 0,
            **fields,
        )

    def _staging_buffer(self, nbytes: int) -> torch.Tensor:
        if self._staging is None or self._staging.numel() < nbytes:
            size = max(nbytes, 2 * (0 if self._staging is None else self._staging.numel()), 1 << 22)
            pin = self.device.type == "cuda"
            self._staging = torch.empty(size, dtype=torch.uint8, pin_memory=pin)
        return self._staging
