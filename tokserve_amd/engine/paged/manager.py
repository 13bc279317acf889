"""Sequences sharing one paged pool (tokserve/engine/paged/manager.py)."""

from __future__ import annotations

import torch

from tokserve_amd.engine.paged.allocator import PhysicalBlockAllocator
from tokserve_amd.engine.paged.sequence_cache import SequencePagedKVCache
from tokserve_amd.engine.paged.storage import PagedKVStorage

__all__ = ["PagedKVCacheManager"]


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
    ) -> None:
        self.allocator = PhysicalBlockAllocator(num_blocks)
        self.storage = PagedKVStorage(
            num_layers=num_layers,
            num_blocks=num_blocks,
            num_key_value_heads=num_key_value_heads,
            block_size=block_size,
            head_dim=head_dim,
            device=device,
            dtype=dtype,
            kv_dtype=kv_dtype,
            k_scale=k_scale,
            v_scale=v_scale,
        )
        self._sequences: dict[str, SequencePagedKVCache] = {}

    @property
    def active_sequence_ids(self) -> tuple[str, ...]:
        """Active sequence ids in creation order."""

        return tuple(self._sequences)

    def create_sequence(self, sequence_id: str, *, max_sequence_length: int) -> SequencePagedKVCache:
        if not sequence_id:
            raise ValueError("sequence_id must be nonempty")
        if sequence_id in self._sequences:
            raise ValueError("sequence_id is already active")
        cache = SequencePagedKVCache(
            allocator=self.allocator, storage=self.storage, max_sequence_length=max_sequence_length
        )
        self._sequences[sequence_id] = cache
        return cache

    def get_sequence(self, sequence_id: str) -> SequencePagedKVCache:
        try:
            return self._sequences[sequence_id]
        except KeyError as error:
            raise KeyError("unknown sequence_id") from error

    def release_sequence(self, sequence_id: str) -> None:
        cache = self.get_sequence(sequence_id)
        cache.release()
        del self._sequences[sequence_id]
