"""Host logic of the paged-KV mirror: allocator, block table, storage and
sequence-cache bookkeeping, manager (tokserve/engine/paged/*.py).

Expected block ids come from the reference's contract: the lowest free id is
allocated first (allocator.py:19-21,53), so every id below is a known answer
(tests/unit/engine/paged/test_allocator.py, test_block_table.py,
test_sequence_cache.py, test_manager.py). Writes and reads need a HIP device
and are covered by tests/test_gpu_dropin.py.
"""

import pytest
import torch

from tokserve_amd.engine.paged.allocator import BlockExhaustedError, PhysicalBlockAllocator
from tokserve_amd.engine.paged.block_table import PhysicalTokenLocation, SequenceBlockTable
from tokserve_amd.engine.paged.manager import PagedKVCacheManager
from tokserve_amd.engine.paged.sequence_cache import SequencePagedKVCache
from tokserve_amd.engine.paged.storage import PagedKVStorage


def _storage(num_blocks=4, block_size=2, layers=2, device="cpu"):
    return PagedKVStorage(num_layers=layers, num_blocks=num_blocks, num_key_value_heads=2,
                          block_size=block_size, head_dim=4, device=torch.device(device),
                          dtype=torch.float32)


# ---------------------------------------------------------------- allocator

def test_allocator_hands_out_lowest_ids_and_reuses_released_ones() -> None:
    allocator = PhysicalBlockAllocator(5)
    assert (allocator.free_count, allocator.allocated_count) == (5, 0)
    assert [allocator.allocate() for _ in range(3)] == [0, 1, 2]
    allocator.release(1)
    allocator.release(0)
    assert allocator.allocate_many(3) == (0, 1, 3)
    assert allocator.allocated_blocks == frozenset({0, 1, 2, 3})
    assert allocator.free_count == 1


def test_allocator_exhaustion_and_atomic_failures() -> None:
    allocator = PhysicalBlockAllocator(3)
    allocator.allocate_many(2)
    with pytest.raises(BlockExhaustedError, match="not enough free physical KV blocks remain"):
        allocator.allocate_many(2)
    assert allocator.free_count == 1
    allocator.allocate()
    with pytest.raises(BlockExhaustedError, match="no free physical KV blocks remain"):
        allocator.allocate()
    allocator.release(2)
    with pytest.raises(ValueError, match="physical block is not currently allocated"):
        allocator.release_many([0, 2])  # 2 is free: nothing may be released
    assert allocator.allocated_blocks == frozenset({0, 1})
    with pytest.raises(ValueError, match="block_ids must not contain duplicates"):
        allocator.release_many([1, 1])


@pytest.mark.parametrize("block_id", [-1, 3])
def test_allocator_rejects_foreign_ids(block_id) -> None:
    with pytest.raises(ValueError, match="physical block ID is out of range"):
        PhysicalBlockAllocator(3).release(block_id)


@pytest.mark.parametrize("count", [0, -1])
def test_allocator_argument_checks(count) -> None:
    with pytest.raises(ValueError, match="num_blocks must be positive"):
        PhysicalBlockAllocator(count)
    with pytest.raises(ValueError, match="count must be positive"):
        PhysicalBlockAllocator(2).allocate_many(count)


# -------------------------------------------------------------- block table

def test_block_table_resolves_positions_and_slots() -> None:
    table = SequenceBlockTable(4)
    for block_id in (7, 2, 5):
        table.append_block(block_id)
    assert table.block_ids == (7, 2, 5) and table.capacity == 12
    assert table.resolve(0) == PhysicalTokenLocation(7, 0)
    assert table.resolve(3) == PhysicalTokenLocation(7, 3)
    assert table.resolve(4) == PhysicalTokenLocation(2, 0)
    assert table.resolve(11) == PhysicalTokenLocation(5, 3)
    # slot = block * BS + offset, the closed form of block_table.py:53-67.
    assert table.slots(2, 5).tolist() == [30, 31, 8, 9, 10]
    with pytest.raises(IndexError, match="exceeds block table capacity"):
        table.resolve(12)
    with pytest.raises(IndexError, match="exceeds block table capacity"):
        table.slots(10, 3)
    with pytest.raises(ValueError, match="position must be nonnegative"):
        table.resolve(-1)
    with pytest.raises(ValueError, match="already in this block table"):
        table.append_block(2)
    with pytest.raises(ValueError, match="physical_block_id must be nonnegative"):
        table.append_block(-3)
    assert table.clear() == (7, 2, 5) and table.num_blocks == 0
    with pytest.raises(ValueError, match="block_size must be positive"):
        SequenceBlockTable(0)


# ------------------------------------------------------------------ storage

def test_storage_shape_and_argument_checks() -> None:
    storage = _storage()
    assert storage.storage_shape == (2, 4, 2, 2, 4)
    assert storage.key_storage.shape == storage.value_storage.shape == (2, 4, 2, 2, 4)
    for name in ("num_layers", "num_blocks", "num_key_value_heads", "block_size", "head_dim"):
        kwargs = dict(num_layers=1, num_blocks=1, num_key_value_heads=1, block_size=1, head_dim=1)
        kwargs[name] = 0
        with pytest.raises(ValueError, match=f"{name} must be positive"):
            PagedKVStorage(**kwargs, device=torch.device("cpu"), dtype=torch.float32)


@pytest.mark.parametrize(("where", "message"), [
    (dict(layer_index=2, block_id=0, offset=0), "layer_index is out of range"),
    (dict(layer_index=0, block_id=4, offset=0), "block_id is out of range"),
    (dict(layer_index=0, block_id=0, offset=2), "offset is out of range"),
    (dict(layer_index=-1, block_id=0, offset=0), "layer_index is out of range"),
])
def test_storage_rejects_invalid_locations(where, message) -> None:
    storage = _storage()
    keys = torch.zeros(2, 4)
    with pytest.raises(IndexError, match=message):
        storage.read_token(**where)
    with pytest.raises(IndexError, match=message):
        storage.write_token(**where, keys=keys, values=keys)


def test_storage_rejects_bad_token_tensors() -> None:
    storage = _storage()
    with pytest.raises(ValueError, match=r"shape \(Hkv, Dh\)"):
        storage.write_token(layer_index=0, block_id=0, offset=0, keys=torch.zeros(3, 4),
                            values=torch.zeros(3, 4))
    with pytest.raises(ValueError, match="match the storage dtype"):
        storage.write_token(layer_index=0, block_id=0, offset=0,
                            keys=torch.zeros(2, 4, dtype=torch.float16),
                            values=torch.zeros(2, 4, dtype=torch.float16))


def test_storage_writes_need_a_hip_device() -> None:
    """No CPU fallback: the KV-append kernel is the only write path."""

    storage = _storage()
    with pytest.raises(ValueError, match="HIP device"):
        storage.write_token(layer_index=0, block_id=0, offset=0, keys=torch.zeros(2, 4),
                            values=torch.zeros(2, 4))


# ----------------------------------------------------------- sequence cache

def _sequence(num_blocks=4, block_size=2, max_len=8):
    storage = _storage(num_blocks, block_size)
    allocator = PhysicalBlockAllocator(num_blocks)
    return SequencePagedKVCache(allocator=allocator, storage=storage,
                                max_sequence_length=max_len), allocator


def test_sequence_allocates_exactly_the_blocks_it_needs() -> None:
    cache, allocator = _sequence(num_blocks=6, block_size=2, max_len=12)
    assert (cache.current_length, cache.num_blocks) == (0, 0)
    cache.begin_append(1)
    assert cache.block_ids == (0,)
    cache._append.written = 0b11  # both layers written (the write itself needs a HIP device)
    cache.finish_append()
    cache.begin_append(1)  # same block
    assert cache.block_ids == (0,)
    cache._append.written = 0b11
    cache.finish_append()
    cache.begin_append(1)  # crosses a block boundary
    assert cache.block_ids == (0, 1)
    cache._append.written = 0b11
    cache.finish_append()
    cache.begin_append(5)  # positions 3..7: blocks 1, 2, 3
    assert cache.block_ids == (0, 1, 2, 3) and cache.pending_length == 5
    assert cache.block_table.slots(3, 5).tolist() == [3, 4, 5, 6, 7]
    assert allocator.free_count == 2


def test_sequence_append_protocol_errors() -> None:
    cache, allocator = _sequence(num_blocks=2, block_size=2, max_len=6)
    with pytest.raises(RuntimeError, match="no append is in progress"):
        cache.finish_append()
    with pytest.raises(RuntimeError, match="begin_append must be called before write_layer"):
        cache.write_layer(0, torch.zeros(2, 1, 4), torch.zeros(2, 1, 4))
    with pytest.raises(ValueError, match="sequence exceeds max_sequence_length"):
        cache.begin_append(7)
    assert allocator.free_count == 2
    with pytest.raises(BlockExhaustedError, match="not enough free physical KV blocks remain"):
        cache.begin_append(5)
    assert (allocator.free_count, cache.num_blocks) == (2, 0)
    cache.begin_append(3)
    with pytest.raises(RuntimeError, match="an append is already in progress"):
        cache.begin_append(1)
    with pytest.raises(RuntimeError, match="every layer must write"):
        cache.finish_append()
    with pytest.raises(RuntimeError, match="pending K/V for this layer have not been written"):
        cache.read_layer(0, include_pending=True)
    with pytest.raises(ValueError, match=r"shape \(Hkv, T, Dh\)"):
        cache.write_layer(0, torch.zeros(2, 2, 4), torch.zeros(2, 2, 4))
    with pytest.raises(IndexError, match="layer_index is out of range"):
        cache.write_layer(2, torch.zeros(2, 3, 4), torch.zeros(2, 3, 4))
    cache.release()
    assert allocator.free_count == 2
    with pytest.raises(RuntimeError, match="sequence cache has been released"):
        cache.begin_append(1)
    with pytest.raises(RuntimeError, match="sequence cache has been released"):
        _ = cache.current_length


def test_sequence_cache_argument_checks() -> None:
    storage = _storage(num_blocks=4)
    with pytest.raises(ValueError, match="block counts must match"):
        SequencePagedKVCache(allocator=PhysicalBlockAllocator(3), storage=storage,
                             max_sequence_length=4)
    with pytest.raises(ValueError, match="max_sequence_length must be positive"):
        SequencePagedKVCache(allocator=PhysicalBlockAllocator(4), storage=storage,
                             max_sequence_length=0)


# ------------------------------------------------------------------ manager

def test_manager_sequences_share_the_pool() -> None:
    manager = PagedKVCacheManager(num_layers=1, num_blocks=6, num_key_value_heads=2, block_size=2,
                                  head_dim=4, device=torch.device("cpu"), dtype=torch.float32)
    a = manager.create_sequence("a", max_sequence_length=8)
    b = manager.create_sequence("b", max_sequence_length=8)
    a.begin_append(3)
    b.begin_append(2)
    assert (a.block_ids, b.block_ids) == ((0, 1), (2,))
    assert manager.active_sequence_ids == ("a", "b")
    with pytest.raises(ValueError, match="sequence_id is already active"):
        manager.create_sequence("a", max_sequence_length=8)
    with pytest.raises(ValueError, match="sequence_id must be nonempty"):
        manager.create_sequence("", max_sequence_length=8)
    manager.release_sequence("a")
    assert manager.active_sequence_ids == ("b",)
    c = manager.create_sequence("c", max_sequence_length=8)
    c.begin_append(5)
    assert c.block_ids == (0, 1, 3)  # released ids first, lowest first
    with pytest.raises(KeyError, match="unknown sequence_id"):
        manager.get_sequence("a")
    with pytest.raises(KeyError, match="unknown sequence_id"):
        manager.release_sequence("a")
    assert manager.allocator.allocated_count == 4
