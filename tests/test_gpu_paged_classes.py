"""SequencePagedKVCache and PagedKVCacheManager over a GPU pool: the data behaviour of the
reference's tests/unit/engine/paged/test_sequence_cache.py:51-254 and test_manager.py:40-230
(layer l's keys = token value + 100 l, values = keys + 1000), with the writes and reads
going through the HIP append and gather kernels. Values are small integers, exact in fp32.
"""

import pytest
import torch
from torch.testing import assert_close

from tokserve_amd.engine.paged.allocator import BlockExhaustedError, PhysicalBlockAllocator
from tokserve_amd.engine.paged.manager import PagedKVCacheManager
from tokserve_amd.engine.paged.sequence_cache import SequencePagedKVCache
from tokserve_amd.engine.paged.storage import PagedKVStorage

pytestmark = pytest.mark.gpu


def _cache(device, num_blocks=5, block_size=4, max_sequence_length=20):
    allocator = PhysicalBlockAllocator(num_blocks=num_blocks)
    storage = PagedKVStorage(num_layers=2, num_blocks=num_blocks, num_key_value_heads=2,
                             block_size=block_size, head_dim=3, device=device,
                             dtype=torch.float32)
    cache = SequencePagedKVCache(allocator=allocator, storage=storage,
                                 max_sequence_length=max_sequence_length)
    return cache, allocator


def _append(cache, values, device):
    cache.begin_append(len(values))
    for layer in range(cache.storage.num_layers):
        keys = torch.tensor(values, device=device).view(1, -1, 1).expand(2, -1, 3) + 100.0 * layer
        cache.write_layer(layer, keys, keys + 1000.0)
    cache.finish_append()


def test_blocks_are_allocated_as_tokens_arrive(device) -> None:
    cache, allocator = _cache(device)
    assert (cache.current_length, cache.num_blocks, cache.block_ids) == (0, 0, ())
    keys, values = cache.read_layer(0)
    assert keys.shape == values.shape == (1, 2, 0, 3)
    _append(cache, [1.0], device)
    assert (cache.current_length, cache.block_ids, allocator.free_count) == (1, (0,), 4)
    for v in (2.0, 3.0, 4.0):
        _append(cache, [v], device)
    assert (cache.current_length, cache.num_blocks, allocator.free_count) == (4, 1, 4)
    _append(cache, [5.0], device)
    assert (cache.current_length, cache.block_ids, allocator.free_count) == (5, (0, 1), 3)
    other, other_allocator = _cache(device)
    _append(other, [float(p) for p in range(10)], device)
    assert (other.num_blocks, other.block_ids, other_allocator.free_count) == (3, (0, 1, 2), 2)


def test_read_reconstructs_logical_order_per_layer(device) -> None:
    cache, _ = _cache(device)
    _append(cache, [1.0, 2.0, 3.0, 4.0], device)
    _append(cache, [5.0, 6.0], device)
    keys, values = cache.read_layer(0)
    assert keys.shape == values.shape == (1, 2, 6, 3)
    for position, number in enumerate((1.0, 2.0, 3.0, 4.0, 5.0, 6.0)):
        assert_close(keys[0, :, position].cpu(), torch.full((2, 3), number))
        assert_close(values[0, :, position].cpu(), torch.full((2, 3), number + 1000.0))
    second, _ = cache.read_layer(1)
    assert_close(second, keys + 100.0)


def test_pending_positions_are_hidden_until_layer_writes(device) -> None:
    cache, _ = _cache(device)
    cache.begin_append(2)
    assert cache.read_layer(0)[0].shape[2] == 0
    with pytest.raises(RuntimeError, match="pending K/V for this layer have not been written"):
        cache.read_layer(0, include_pending=True)
    keys = torch.ones(2, 2, 3, device=device)
    values = torch.full((2, 2, 3), 2.0, device=device)
    cache.write_layer(0, keys, values)
    visible_keys, visible_values = cache.read_layer(0, include_pending=True)
    assert visible_keys.shape == (1, 2, 2, 3)
    assert_close(visible_keys[0], keys)
    assert_close(visible_values[0], values)
    assert cache.read_layer(1)[0].shape[2] == 0
    with pytest.raises(RuntimeError, match="every layer must write"):
        cache.finish_append()
    assert cache.current_length == 0


def test_exhaustion_release_and_length_limits(device) -> None:
    cache, allocator = _cache(device, num_blocks=1, block_size=2, max_sequence_length=8)
    _append(cache, [1.0, 2.0], device)
    with pytest.raises(BlockExhaustedError, match="not enough free physical KV blocks remain"):
        cache.begin_append(1)
    assert (cache.current_length, cache.num_blocks, allocator.free_count) == (2, 1, 0)
    cache, allocator = _cache(device)
    _append(cache, [1.0, 2.0, 3.0, 4.0, 5.0], device)
    assert allocator.free_count == 3
    cache.release()
    assert (allocator.free_count, allocator.allocated_count) == (5, 0)
    with pytest.raises(RuntimeError, match="sequence cache has been released"):
        cache.read_layer(0)
    with pytest.raises(RuntimeError, match="sequence cache has been released"):
        cache.release()
    cache, allocator = _cache(device, max_sequence_length=4)
    with pytest.raises(ValueError, match="sequence exceeds max_sequence_length"):
        cache.begin_append(5)
    assert (allocator.free_count, cache.current_length) == (5, 0)


def _manager(device, num_blocks=8, block_size=2):
    return PagedKVCacheManager(num_layers=2, num_blocks=num_blocks, num_key_value_heads=2,
                               block_size=block_size, head_dim=3, device=device,
                               dtype=torch.float32)


def _owned(manager):
    return [b for s in manager.active_sequence_ids for b in manager.get_sequence(s).block_ids]


def test_sequences_never_share_blocks_and_release_keeps_the_others(device) -> None:
    manager = _manager(device)
    a, b, c = (manager.create_sequence(s, max_sequence_length=8) for s in "ABC")
    assert a.allocator is b.allocator and a.storage is b.storage
    assert a.block_table is not b.block_table
    _append(a, [1.0, 2.0, 3.0], device)
    _append(b, [4.0, 5.0], device)
    _append(c, [6.0, 7.0], device)
    owned = _owned(manager)
    assert len(owned) == len(set(owned)) and manager.allocator.allocated_count == len(owned)
    b_before = [t.clone() for t in b.read_layer(0)]
    c_before = [t.clone() for t in c.read_layer(1)]
    a_blocks = set(a.block_ids)
    manager.release_sequence("A")
    assert "A" not in manager.active_sequence_ids and a_blocks.isdisjoint(_owned(manager))
    for before, after in zip(b_before + c_before, list(b.read_layer(0)) + list(c.read_layer(1))):
        assert torch.equal(before, after)
    d = manager.create_sequence("D", max_sequence_length=8)
    _append(d, [8.0, 9.0, 10.0], device)  # reuses A's released blocks
    assert set(d.block_ids) & a_blocks
    for before, after in zip(b_before + c_before, list(b.read_layer(0)) + list(c.read_layer(1))):
        assert torch.equal(before, after)


def test_reused_block_does_not_expose_stale_positions(device) -> None:
    manager = _manager(device, num_blocks=2, block_size=4)
    a = manager.create_sequence("A", max_sequence_length=4)
    _append(a, [1.0, 2.0, 3.0, 4.0], device)
    released = a.block_ids[0]
    manager.release_sequence("A")
    with pytest.raises(RuntimeError, match="sequence cache has been released"):
        a.read_layer(0)
    b = manager.create_sequence("B", max_sequence_length=4)
    assert b.current_length == 0 and b.read_layer(0)[0].shape[2] == 0
    _append(b, [9.0], device)
    assert b.block_ids == (released,)
    keys, values = b.read_layer(0)
    assert_close(keys.cpu(), torch.full((1, 2, 1, 3), 9.0))
    assert_close(values.cpu(), torch.full((1, 2, 1, 3), 1009.0))
    manager.release_sequence("B")
    assert manager.allocator.free_count == 2 and manager.allocator.allocated_count == 0
