"""Physical KV block ownership over a free map (tokserve/engine/paged/allocator.py).

The pool's block ids 0 .. NB-1 are one boolean free map (NumPy) plus a floor
below which no id is free. A request for k blocks scans the map upward from the
floor, in windows that double until k free ids are found, and takes the k
lowest: the lowest-id-first order of the reference's min-heap
(allocator.py:19-21,53), on which every block id the engine tests pin depends,
at the cost of one vectorised scan per request instead of k heap operations.
Releasing sets the bits back and lowers the floor. Every check runs before the
map changes, so a failed call leaves the allocator as it was.
"""

from __future__ import annotations

from collections.abc import Iterable

import numpy as np

__all__ = ["BlockExhaustedError", "PhysicalBlockAllocator"]

_FIRST_WINDOW = 64


class BlockExhaustedError(RuntimeError):
    """The pool has fewer free blocks than an allocation needs."""


class PhysicalBlockAllocator:
    """Owner of block ids 0 .. num_blocks-1 of one paged KV pool."""

    def __init__(self, num_blocks: int) -> None:
        if num_blocks < 1:
            raise ValueError("num_blocks must be positive")
        self._free = np.ones(num_blocks, dtype=np.bool_)
        self._available = num_blocks
        self._floor = 0

    @property
    def num_blocks(self) -> int:
        return int(self._free.size)

    @property
    def free_count(self) -> int:
        return self._available

    @property
    def allocated_count(self) -> int:
        return int(self._free.size) - self._available

    @property
    def allocated_blocks(self) -> frozenset[int]:
        return frozenset(np.flatnonzero(~self._free).tolist())

    def allocate(self) -> int:
        """The lowest free block id."""

        if self._available == 0:
            raise BlockExhaustedError("no free physical KV blocks remain")
        return int(self._take(1)[0])

    def allocate_many(self, count: int) -> tuple[int, ...]:
        """The `count` lowest free ids, all or none."""

        return tuple(self.take_lowest(count).tolist())

    def take_lowest(self, count: int) -> np.ndarray:
        """allocate_many as an int64 array (the sequence caches' bulk path)."""

        if count < 1:
            raise ValueError("count must be positive")
        if count > self._available:
            raise BlockExhaustedError("not enough free physical KV blocks remain")
        return self._take(count)

    def release(self, block_id: int) -> None:
        self.release_many((block_id,))

    def release_many(self, block_ids: Iterable[int]) -> None:
        """Return blocks to the pool; nothing is released unless all of them can be."""

        ids = np.array([int(b) for b in block_ids], dtype=np.int64)
        if ids.size == 0:
            return
        if np.unique(ids).size != ids.size:
            raise ValueError("block_ids must not contain duplicates")
        outside = (ids < 0) | (ids >= self._free.size)
        unowned = ~outside & self._free[np.where(outside, 0, ids)]
        rejected = outside | unowned
        if rejected.any():
            first = int(np.argmax(rejected))
            if outside[first]:
                raise ValueError("physical block ID is out of range")
            raise ValueError("physical block is not currently allocated")
        self._free[ids] = True
        self._available += int(ids.size)
        self._floor = min(self._floor, int(ids.min()))

    def _take(self, count: int) -> np.ndarray:
        size = self._free.size
        start, window = self._floor, max(_FIRST_WINDOW, count)
        found = np.flatnonzero(self._free[start : start + window]) + start
        while found.size < count:
            start, window = start + window, 2 * window
            more = np.flatnonzero(self._free[start : start + window]) + start
            found = np.concatenate((found, more))
            if start >= size:
                break
        taken = found[:count]
        self._free[taken] = False
        self._available -= count
        self._floor = int(taken[-1]) + 1
        return taken
