"""One sequence's blocks and logical K/V state (tokserve/engine/paged/sequence_cache.py).

An append is bracketed: begin_append reserves blocks for T new positions
(lowest free ids first), every layer then writes its (Hkv, T, Dh) K/V with
write_layer, and finish_append makes the positions valid once all layers have
written (sequence_cache.py:56-84,195-208). The T pool slots of an append are
computed once, at begin_append, and each write_layer is one KV-append kernel
launch over them; read_layer is one gather kernel launch.
"""

from __future__ import annotations

import torch

from tokserve_amd.engine.paged.allocator import PhysicalBlockAllocator
from tokserve_amd.engine.paged.block_table import SequenceBlockTable
from tokserve_amd.engine.paged.storage import PagedKVStorage

__all__ = ["SequencePagedKVCache"]


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
        self._length = 0
        self._pending = 0
        self._pending_slots: torch.Tensor | None = None
        self._written: set[int] = set()
        self._all_layers = frozenset(range(storage.num_layers))
        self._released = False

    @property
    def current_length(self) -> int:
        """Fully written, valid token positions."""

        self._require_active()
        return self._length

    @property
    def pending_length(self) -> int:
        """Positions reserved by the append in progress (0 if none)."""

        self._require_active()
        return self._pending

    @property
    def num_blocks(self) -> int:
        self._require_active()
        return self.block_table.num_blocks

    @property
    def block_ids(self) -> tuple[int, ...]:
        self._require_active()
        return self.block_table.block_ids

    def begin_append(self, sequence_length: int) -> None:
        """Reserve physical slots for `sequence_length` new positions."""

        self._require_active()
        if self._pending != 0:
            raise RuntimeError("an append is already in progress")
        if sequence_length < 1:
            raise ValueError("sequence_length must be positive")
        new_length = self._length + sequence_length
        if new_length > self.max_sequence_length:
            raise ValueError("sequence exceeds max_sequence_length")
        size = self.storage.block_size
        missing = (new_length + size - 1) // size - self.block_table.num_blocks
        if missing > 0:
            for block_id in self.allocator.allocate_many(missing):
                self.block_table.append_block(block_id)
        self._pending = sequence_length
        self._pending_slots = None
        self._written.clear()

    def pending_slots(self) -> torch.Tensor:
        """Pool slots (int64, on the storage device) of the pending positions."""

        self._require_active()
        if self._pending == 0:
            raise RuntimeError("begin_append must be called before write_layer")
        if self._pending_slots is None:
            slots = self.block_table.slots(self._length, self._pending)
            self._pending_slots = torch.tensor(slots, dtype=torch.int64).to(self.storage.device)
        return self._pending_slots

    def write_layer(self, layer_index: int, keys: torch.Tensor, values: torch.Tensor) -> None:
        """Write the pending positions' K/V, each shaped (Hkv, T, Dh), for one layer."""

        self._require_active()
        if self._pending == 0:
            raise RuntimeError("begin_append must be called before write_layer")
        if layer_index < 0 or layer_index >= self.storage.num_layers:
            raise IndexError("layer_index is out of range")
        if layer_index in self._written:
            raise ValueError("layer has already written this append")
        expected = (self.storage.num_key_value_heads, self._pending, self.storage.head_dim)
        if keys.shape != expected or values.shape != expected:
            raise ValueError("keys and values must have shape (Hkv, T, Dh)")
        if keys.device != self.storage.device or values.device != self.storage.device:
            raise ValueError("keys and values must match the storage device")
        if keys.dtype != self.storage.dtype or values.dtype != self.storage.dtype:
            raise ValueError("keys and values must match the storage dtype")
        # (T, Hkv, Dh) views: the kernel takes token and head strides.
        self.storage.write_slots(
            layer_index, self.pending_slots(), keys.transpose(0, 1), values.transpose(0, 1)
        )
        self._written.add(layer_index)

    def mark_layers_written(self) -> None:
        """Record that every layer's K/V of the pending positions was written by packed
        KV-append launches (one per layer over a whole batch's slots)."""

        self._require_active()
        if self._pending == 0:
            raise RuntimeError("begin_append must be called before write_layer")
        self._written = self._all_layers

    def reserve(self, sequence_length: int) -> list[int]:
        """begin_append for the batched executor: returns the live block-id list
        (read-only for the caller) after reserving the new positions."""

        self.begin_append(sequence_length)
        return self.block_table._ids

    def commit(self) -> None:
        """finish_append after packed KV-append launches wrote every layer."""

        if self._released:
            raise RuntimeError("sequence cache has been released")
        if self._pending == 0:
            raise RuntimeError("no append is in progress")
        self._length += self._pending
        self._pending = 0
        self._pending_slots = None
        self._written = set()

    def read_layer(
        self, layer_index: int, *, include_pending: bool = False
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """One layer's K/V in logical order, each shaped (1, Hkv, S, Dh)."""

        self._require_active()
        if layer_index < 0 or layer_index >= self.storage.num_layers:
            raise IndexError("layer_index is out of range")
        length = self._length
        if include_pending and self._pending != 0:
            if layer_index not in self._written:
                raise RuntimeError("pending K/V for this layer have not been written")
            length += self._pending
        keys, values = self.storage.gather(layer_index, self.block_table.block_ids, length)
        return keys.transpose(0, 1).unsqueeze(0), values.transpose(0, 1).unsqueeze(0)

    def finish_append(self) -> None:
        """Make the pending positions valid once every layer has written them."""

        self._require_active()
        if self._pending == 0:
            raise RuntimeError("no append is in progress")
        if len(self._written) != self.storage.num_layers:
            raise RuntimeError("every layer must write before finishing an append")
        self._length += self._pending
        self._pending = 0
        self._pending_slots = None
        self._written.clear()

    def release(self) -> None:
        """Return every owned block and invalidate this cache."""

        self._require_active()
        self.allocator.release_many(self.block_table.clear())
        self._length = 0
        self._pending = 0
        self._pending_slots = None
        self._written.clear()
        self._released = True

    def _require_active(self) -> None:
        if self._released:
            raise RuntimeError("sequence cache has been released")
