"""Logical -> physical block mapping of one sequence (tokserve/engine/paged/block_table.py).

Token position p lives in physical block ids[p // block_size] at offset
p % block_size, i.e. in pool slot ids[p // block_size] * block_size +
p % block_size (block_table.py:53-67), the slot the KV-append kernel takes.
The ids sit in a growable int64 array whose live prefix (`view()`) the batched
executor copies straight into its block-table rows, and whose slots for a run
of positions come out of one vectorised expression.
"""

from __future__ import annotations

from collections.abc import Iterable
from dataclasses import dataclass

import numpy as np

__all__ = ["PhysicalTokenLocation", "SequenceBlockTable"]


@dataclass(frozen=True)
class PhysicalTokenLocation:
    """Physical block id and in-block offset of one token position."""

    block_id: int
    offset: int


class SequenceBlockTable:
    """Physical block ids of one sequence in logical order."""

    def __init__(self, block_size: int) -> None:
        if block_size < 1:
            raise ValueError("block_size must be positive")
        self.block_size = block_size
        self._store = np.empty(8, dtype=np.int64)
        self._used = 0

    def view(self) -> np.ndarray:
        """The live ids (a view: valid until the table next grows or clears)."""

        return self._store[: self._used]

    @property
    def block_ids(self) -> tuple[int, ...]:
        return tuple(self.view().tolist())

    @property
    def num_blocks(self) -> int:
        return self._used

    @property
    def capacity(self) -> int:
        return self._used * self.block_size

    def append_block(self, physical_block_id: int) -> None:
        self.extend((physical_block_id,))

    def extend(self, physical_block_ids: Iterable[int] | np.ndarray) -> None:
        """Map the next logical blocks to these physical ids (checked before any is added)."""

        new = np.asarray(physical_block_ids, dtype=np.int64).reshape(-1)
        if (new < 0).any():
            raise ValueError("physical_block_id must be nonnegative")
        held = set(self.view().tolist())
        held_new = set(new.tolist())
        if len(held_new) != new.size or not held.isdisjoint(held_new):
            raise ValueError("physical block is already in this block table")
        self.extend_fresh(new)

    def extend_fresh(self, new: np.ndarray) -> None:
        """extend() for ids straight from the pool's allocator, which never hands out an id
        that some table holds: no membership checks."""

        needed = self._used + new.size
        if needed > self._store.size:
            grown = np.empty(max(needed, 2 * self._store.size), dtype=np.int64)
            grown[: self._used] = self.view()
            self._store = grown
        self._store[self._used : needed] = new
        self._used = needed

    def truncate(self, num_blocks: int) -> tuple[int, ...]:
        """Drop the mappings past the first num_blocks and return their ids."""

        dropped = tuple(self._store[num_blocks : self._used].tolist())
        self._used = min(self._used, max(num_blocks, 0))
        return dropped

    def resolve(self, position: int) -> PhysicalTokenLocation:
        if position < 0:
            raise ValueError("position must be nonnegative")
        block, offset = divmod(position, self.block_size)
        if block >= self._used:
            raise IndexError("position exceeds block table capacity")
        return PhysicalTokenLocation(block_id=int(self._store[block]), offset=offset)

    def slots(self, start: int, count: int) -> np.ndarray:
        """Pool slots (int64) of positions start .. start+count-1, all of them mapped."""

        if start < 0 or count < 0:
            raise ValueError("position must be nonnegative")
        if start + count > self.capacity:
            raise IndexError("position exceeds block table capacity")
        positions = np.arange(start, start + count, dtype=np.int64)
        return self._store[positions // self.block_size] * self.block_size + (
            positions % self.block_size)

    def clear(self) -> tuple[int, ...]:
        return self.truncate(0)
