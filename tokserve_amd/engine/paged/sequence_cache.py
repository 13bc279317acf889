"""One sequence's blocks and logical K/V state (tokserve/engine/paged/sequence_cache.py).

A sequence holds a block table and its valid length; an append in progress is
one `_Append` record (where it starts, how many positions, which blocks it
took from the pool, which layers have written, its pool slots), so the three
ways an append ends are one line each: finish (every layer wrote, through
write_layer), commit (a packed forward wrote every layer with one KV-append
launch per layer over the whole batch's slots), abort (the blocks it took go
back to the pool, for a batch that failed before its forward). The protocol
and its checks are the reference's (sequence_cache.py:56-84,195-224):
begin_append reserves blocks for T new positions, write_layer writes one layer's
(Hkv, T, Dh) K/V, finish_append validates the positions once all layers wrote.
Each write_layer is one KV-append kernel launch; read_layer is one gather launch.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from tokserve_amd.engine.paged.allocator import PhysicalBlockAllocator
from tokserve_amd.engine.paged.block_table import SequenceBlockTable
from tokserve_amd.engine.paged.storage import PagedKVStorage

__all__ = ["SequencePagedKVCache"]

_NO_BLOCKS = np.empty(0, dtype=np.int64)


@dataclass
class _Append:
    start: int               # first new position
    count: int               # positions being appended
    kept_blocks: int         # table length before the append took new blocks
    written: int = 0         # bit l set: layer l has written the new positions
    slots: torch.Tensor | None = None


class SequencePagedKVCache:
    """One sequence's K/V values in a shared physical block pool."""

    def __init__(
        self,
        *,
        allocator: PhysicalBlockAllocator,
        storage: PagedKVStorage,
        max_sequence_length: int,
    ) -> None:
        if allocator.num_blocks != storage.num_blocks:
            raise ValueError("allocator and storage block counts must match")
        if max_sequence_length < 1:
            raise ValueError("max_sequence_length must be positive")
        self.allocator = allocator
        self.storage = storage
        self.max_sequence_length = max_sequence_length
        self.block_table = SequenceBlockTable(storage.block_size)
        self._valid = 0
        self._append: _Append | None = None
        self._every_layer = (1 << storage.num_layers) - 1
        self._live = True

    # ------------------------------------------------------------ state

    @property
    def current_length(self) -> int:
        """Fully written, valid token positions."""

        return self._active()._valid

    @property
    def pending_length(self) -> int:
        """Positions reserved by the append in progress (0 if none)."""

        append = self._active()._append
        return 0 if append is None else append.count

    @property
    def is_live(self) -> bool:
        """False once release() has run."""

        return self._live

    @property
    def num_blocks(self) -> int:
        return self._active().block_table.num_blocks

    @property
    def block_ids(self) -> tuple[int, ...]:
        return self._active().block_table.block_ids

    # ----------------------------------------------------------- append

    def begin_append(self, sequence_length: int) -> None:
        """Reserve physical slots for `sequence_length` new positions."""

        self.check_append(sequence_length)
        short = self.blocks_short(sequence_length)
        self.open_append(sequence_length,
                         self.allocator.take_lowest(short) if short > 0 else _NO_BLOCKS)

    def check_append(self, sequence_length: int) -> None:
        """Raise what begin_append would raise before taking any block."""

        self._active()
        if self._append is not None:
            raise RuntimeError("an append is already in progress")
        if sequence_length < 1:
            raise ValueError("sequence_length must be positive")
        if self._valid + sequence_length > self.max_sequence_length:
            raise ValueError("sequence exceeds max_sequence_length")

    def blocks_short(self, sequence_length: int) -> int:
        """Blocks an append of `sequence_length` positions takes from the pool."""

        table = self.block_table
        return max(0, -(-(self._valid + sequence_length) // table.block_size) - table.num_blocks)

    def open_append(self, sequence_length: int, fresh_blocks: np.ndarray) -> None:
        """Begin a checked append whose blocks_short() new blocks the caller took from
        this pool's allocator (a batch takes all of its sequences' blocks at once)."""

        kept = self.block_table.num_blocks
        if fresh_blocks.size:
            self.block_table.extend_fresh(fresh_blocks)
        self._append = _Append(start=self._valid, count=sequence_length, kept_blocks=kept)

    def reserve(self, sequence_length: int) -> np.ndarray:
        """begin_append for the batched executor; returns the live block ids
        (a read-only view) that now cover the new positions."""

        self.begin_append(sequence_length)
        return self.block_table.view()

    def pending_slots(self) -> torch.Tensor:
        """Pool slots (int64, on the storage device) of the pending positions."""

        append = self._pending("begin_append must be called before write_layer")
        if append.slots is None:
            slots = self.block_table.slots(append.start, append.count)
            append.slots = torch.from_numpy(slots).to(self.storage.device)
        return append.slots

    def write_layer(self, layer_index: int, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Write the pending positions' K/V, each shaped (Hkv, T, Dh), for one layer."""

        append = self._pending("begin_append must be called before write_layer")
        if not 0 <= layer_index < self.storage.num_layers:
            raise IndexError("layer_index is out of range")
        if append.written >> layer_index & 1:
            raise ValueError("layer has already written this append")
        storage = self.storage
        expected = (storage.num_key_value_heads, append.count, storage.head_dim)
        if keys.shape != expected or values.shape != expected:
            raise ValueError("keys and values must have shape (Hkv, T, Dh)")
        if keys.device != storage.device or values.device != storage.device:
            raise ValueError("keys and values must match the storage device")
        if keys.dtype != storage.dtype or values.dtype != storage.dtype:
            raise ValueError("keys and values must match the storage dtype")
        # (T, Hkv, Dh) views: the kernel takes token and head strides.
        storage.write_slots(layer_index, self.pending_slots(), keys.transpose(0, 1),
                            values.transpose(0, 1))
        append.written |= 1 << layer_index

    def finish_append(self) -> None:
        """Make the pending positions valid once every layer has written them."""

        append = self._pending("no append is in progress")
        if append.written != self._every_layer:
            raise RuntimeError("every layer must write before finishing an append")
        self._close(keep=True)

    def commit(self) -> None:
        """finish_append after a packed forward's KV-append launches wrote every layer."""

        self._pending("no append is in progress")
        self._close(keep=True)

    def abort_append(self) -> None:
        """Drop the append in progress and return the blocks it took to the pool."""

        append = self._pending("no append is in progress")
        taken = self.block_table.truncate(append.kept_blocks)
        if taken:
            self.allocator.release_many(taken)
        self._close(keep=False)

    def _close(self, *, keep: bool) -> None:
        if keep and self._append is not None:
            self._valid += self._append.count
        self._append = None

    # ------------------------------------------------------------- read

    def read_layer(
        self, layer_index: int, *, include_pending: bool = False
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """One layer's K/V in logical order, each shaped (1, Hkv, S, Dh)."""

        self._active()
        if not 0 <= layer_index < self.storage.num_layers:
            raise IndexError("layer_index is out of range")
        length = self._valid
        append = self._append
        if include_pending and append is not None:
            if not append.written >> layer_index & 1:
                raise RuntimeError("pending K/V for this layer have not been written")
            length += append.count
        keys, values = self.storage.gather(layer_index, self.block_table.block_ids, length)
        return keys.transpose(0, 1).unsqueeze(0), values.transpose(0, 1).unsqueeze(0)

    # ---------------------------------------------------------- release

    def release(self) -> None:
        """Return every owned block and invalidate this cache."""

        self._active()
        self.allocator.release_many(self.block_table.clear())
        self._valid = 0
        self._append = None
        self._live = False

    def _active(self) -> SequencePagedKVCache:
        if not self._live:
            raise RuntimeError("sequence cache has been released")
        return self

    def _pending(self, message: str) -> _Append:
        self._active()
        if self._append is None:
            raise RuntimeError(message)
        return self._append
