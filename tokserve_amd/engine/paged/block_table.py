"""Logical -> physical block mapping of one sequence (tokserve/engine/paged/block_table.py).

Token position p lives in physical block block_ids[p // block_size] at offset
p % block_size, i.e. in pool slot block_ids[p // block_size] * block_size +
p % block_size (block_table.py:53-67): the slot the KV-append kernel takes.
"""

from __future__ import annotations

from dataclasses import dataclass

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
        self._ids: list[int] = []

    @property
    def block_ids(self) -> tuple[int, ...]:
        return tuple(self._ids)

    @property
    def num_blocks(self) -> int:
        return len(self._ids)

    @property
    def capacity(self) -> int:
        return len(self._ids) * self.block_size

    def append_block(self, physical_block_id: int) -> None:
        if physical_block_id < 0:
            raise ValueError("physical_block_id must be nonnegative")
        if physical_block_id in self._ids:
            raise ValueError("physical block is already in this block table")
        self._ids.append(physical_block_id)

    def resolve(self, position: int) -> PhysicalTokenLocation:
        if position < 0:
            raise ValueError("position must be nonnegative")
        logical_block, offset = divmod(position, self.block_size)
        if logical_block >= len(self._ids):
            raise IndexError("position exceeds block table capacity")
        return PhysicalTokenLocation(block_id=self._ids[logical_block], offset=offset)

    def slots(self, start: int, count: int) -> list[int]:
        """Pool slots of positions start .. start+count-1 (all must be mapped)."""

        if start < 0 or count < 0:
            raise ValueError("position must be nonnegative")
        if start + count > self.capacity:
            raise IndexError("position exceeds block table capacity")
        size = self.block_size
        ids = self._ids
        return [ids[p // size] * size + p % size for p in range(start, start + count)]

    def clear(self) -> tuple[int, ...]:
        released = tuple(self._ids)
        self._ids.clear()
        return released
