"""Physical KV block ownership (tokserve/engine/paged/allocator.py).

The free list is a binary min-heap, so allocation always hands out the lowest
free block id: block ids, and with them every block table the scheduler
builds, are a deterministic function of the request history, which is what
the reference's tests pin (allocator.py:19-21,53).
"""

from __future__ import annotations

import heapq
from collections.abc import Iterable

__all__ = ["BlockExhaustedError", "PhysicalBlockAllocator"]


class BlockExhaustedError(RuntimeError):
    """The pool has fewer free blocks than an allocation needs."""


class PhysicalBlockAllocator:
    """Owner of block ids 0 .. num_blocks-1 of one paged KV pool."""

    def __init__(self, num_blocks: int) -> None:
        if num_blocks < 1:
            raise ValueError("num_blocks must be positive")
        self._num_blocks = num_blocks
        self._heap: list[int] = list(range(num_blocks))  # sorted, hence a valid heap
        self._owned: set[int] = set()

    @property
    def num_blocks(self) -> int:
        return self._num_blocks

    @property
    def free_count(self) -> int:
        return len(self._heap)

    @property
    def allocated_count(self) -> int:
        return len(self._owned)

    @property
    def allocated_blocks(self) -> frozenset[int]:
        return frozenset(self._owned)

    def allocate(self) -> int:
        """Take the lowest free block id."""

        if not self._heap:
            raise BlockExhaustedError("no free physical KV blocks remain")
        block_id = heapq.heappop(self._heap)
        self._owned.add(block_id)
        return block_id

    def allocate_many(self, count: int) -> tuple[int, ...]:
        """Take the `count` lowest free ids, or none of them."""

        if count < 1:
            raise ValueError("count must be positive")
        if count > len(self._heap):
            raise BlockExhaustedError("not enough free physical KV blocks remain")
        return tuple(self.allocate() for _ in range(count))

    def release(self, block_id: int) -> None:
        self._check_owned(block_id)
        self._owned.discard(block_id)
        heapq.heappush(self._heap, block_id)

    def release_many(self, block_ids: Iterable[int]) -> None:
        """Return several blocks; nothing is released unless all of them can be."""

        ids = tuple(block_ids)
        if len(set(ids)) != len(ids):
            raise ValueError("block_ids must not contain duplicates")
        for block_id in ids:
            self._check_owned(block_id)
        for block_id in ids:
            self.release(block_id)

    def _check_owned(self, block_id: int) -> None:
        if not 0 <= block_id < self._num_blocks:
            raise ValueError("physical block ID is out of range")
        if block_id not in self._owned:
            raise ValueError("physical block is not currently allocated")
