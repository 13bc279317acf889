"""Sequences sharing one paged pool (tokserve/engine/paged/manager.py).

Besides the reference's registry (create / get / release a sequence by id),
the manager hands the batched executor a `StepReservation`: every sequence an
iteration opens and every append it begins go through it, and if anything
fails before the iteration commits (an exhausted pool halfway through a
batch, a failed launch) the reservation undoes them all, newest first:
pending appends are aborted, returning the blocks they took, and sequences
opened by the iteration are released. The pool and every sequence are then as
they were before the iteration.
"""

from __future__ import annotations

import numpy as np
import torch

from tokserve_amd.engine.paged.allocator import PhysicalBlockAllocator
from tokserve_amd.engine.paged.sequence_cache import SequencePagedKVCache
from tokserve_amd.engine.paged.storage import PagedKVStorage

__all__ = ["PagedKVCacheManager", "StepReservation"]

_NONE = np.empty(0, dtype=np.int64)


class PagedKVCacheManager:
    """Sequence caches over one allocator and one K/V storage pool."""

    def __init__(
        self,
        *,
        num_layers: int,
        num_blocks: int,
        num_key_value_heads: int,
        block_size: int,
        head_dim: int,
        device: torch.device,
        dtype: torch.dtype,
        kv_dtype: torch.dtype | None = None,
        k_scale: float = 1.0,
        v_scale: float = 1.0,
        scale_granularity: str = "pool",
    ) -> None:
        self.allocator = PhysicalBlockAllocator(num_blocks)
        self.storage = PagedKVStorage(
            num_layers=num_layers, num_blocks=num_blocks, num_key_value_heads=num_key_value_heads,
            block_size=block_size, head_dim=head_dim, device=device, dtype=dtype,
            kv_dtype=kv_dtype, k_scale=k_scale, v_scale=v_scale,
            scale_granularity=scale_granularity,
        )
        self._registry: dict[str, SequencePagedKVCache] = {}

    @property
    def active_sequence_ids(self) -> tuple[str, ...]:
        """Active sequence ids in creation order."""

        return tuple(self._registry)

    def create_sequence(self, sequence_id: str, *, max_sequence_length: int) -> SequencePagedKVCache:
        if not sequence_id:
            raise ValueError("sequence_id must be nonempty")
        if sequence_id in self._registry:
            raise ValueError("sequence_id is already active")
        cache = SequencePagedKVCache(allocator=self.allocator, storage=self.storage,
                                     max_sequence_length=max_sequence_length)
        self._registry[sequence_id] = cache
        return cache

    def get_sequence(self, sequence_id: str) -> SequencePagedKVCache:
        cache = self._registry.get(sequence_id)
        if cache is None:
            raise KeyError("unknown sequence_id")
        return cache

    def release_sequence(self, sequence_id: str) -> None:
        self.get_sequence(sequence_id).release()
        del self._registry[sequence_id]

    def reservation(self) -> StepReservation:
        """An all-or-nothing reservation scope for one batched iteration."""

        return StepReservation(self)


class StepReservation:
    """The sequences and appends one iteration has opened, undone together on failure.

    Use as a context manager: leaving it with an exception rolls back whatever
    was not committed; `commit()` makes every begun append valid.
    """

    def __init__(self, manager: PagedKVCacheManager) -> None:
        self.manager = manager
        self._opened: list[str] = []
        self._appending: list[SequencePagedKVCache] = []

    def open(self, sequence_id: str, *, max_sequence_length: int) -> SequencePagedKVCache:
        cache = self.manager.create_sequence(sequence_id, max_sequence_length=max_sequence_length)
        self._opened.append(sequence_id)
        return cache

    def extend(self, cache: SequencePagedKVCache, count: int) -> np.ndarray:
        """Begin an append of `count` positions; the block ids that cover them."""

        blocks = cache.reserve(count)
        self._appending.append(cache)
        return blocks

    def extend_all(self, appends: list[tuple[SequencePagedKVCache, int]]) -> list[np.ndarray]:
        """Begin an append on every (cache, positions) pair, in order. Every check runs
        first; then the blocks of all of them come from the pool in one lowest-first
        allocation, dealt out in order, so each cache gets exactly the ids it would get
        appending one after another. Returns each cache's live block ids."""

        for cache, count in appends:
            cache.check_append(count)
        shorts = [cache.blocks_short(count) for cache, count in appends]
        total = sum(shorts)
        fresh = self.manager.allocator.take_lowest(total) if total else None
        tables = []
        offset = 0
        for (cache, count), short in zip(appends, shorts):
            cache.open_append(count, fresh[offset : offset + short] if short else _NONE)
            offset += short
            self._appending.append(cache)
            tables.append(cache.block_table.view())
        return tables

    def commit(self) -> None:
        for cache in self._appending:
            cache.commit()
        self._appending.clear()
        self._opened.clear()

    def rollback(self) -> None:
        for cache in reversed(self._appending):
            if cache.is_live:  # a sequence released meanwhile gave its blocks back itself
                cache.abort_append()
        self._appending.clear()
        for sequence_id in reversed(self._opened):
            self.manager.release_sequence(sequence_id)
        self._opened.clear()

    def __enter__(self) -> StepReservation:
        return self

    def __exit__(self, kind, error, trace) -> None:
        if kind is not None:
            self.rollback()
