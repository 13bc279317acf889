"""tks_paged_attention_decode_noalloc (split partials in the library's static device
buffer) called through the C ABI against tks_paged_attention_decode (partials in a
caller workspace): the same kernels, so the outputs must be bit-identical.

Two calls in a row share the static buffer; the second has a smaller batch, so
any partial the first call left behind would show up as a difference.
"""

import ctypes

import pytest
import torch

from oracle import paged
from tokserve_amd import workloads
from tokserve_amd.kernels import _lib

pytestmark = pytest.mark.gpu


def _args(batch, out, pages_per_split):
    _, nb, hkv, bs, dh = batch.key_cache.shape
    return (
        batch.query.data_ptr(), batch.query.stride(0), batch.query.stride(1),
        batch.key_cache.data_ptr(), batch.value_cache.data_ptr(), 1, nb, hkv, bs, dh, 0,
        batch.block_tables.data_ptr(), batch.block_tables.shape[1], batch.seq_lens.data_ptr(),
        None, batch.num_seqs, batch.query.shape[1], batch.max_seq_len,
        1.0 / dh ** 0.5, pages_per_split, out.data_ptr(), out.stride(0), out.stride(1),
    )


def _with_workspace(library, batch, pages_per_split):
    _, _, hkv, bs, dh = batch.key_cache.shape
    nbytes = library.tks_paged_attention_decode_workspace_bytes(
        batch.num_seqs, batch.query.shape[1], hkv, dh, bs, batch.max_seq_len, pages_per_split)
    assert nbytes > 0
    workspace = torch.empty(nbytes, dtype=torch.uint8, device=batch.query.device)
    out = torch.empty_like(batch.query)
    status = library.tks_paged_attention_decode(
        *_args(batch, out, pages_per_split), workspace.data_ptr(), nbytes,
        _lib.dtype_code(batch.query.dtype), _lib.stream_of(batch.query))
    assert status == _lib.TKS_OK
    return out


def _no_alloc(library, batch, pages_per_split):
    out = torch.empty_like(batch.query)
    status = library.tks_paged_attention_decode_noalloc(
        *_args(batch, out, pages_per_split), _lib.dtype_code(batch.query.dtype),
        _lib.stream_of(batch.query))
    assert status == _lib.TKS_OK, library.tks_status_string(status)
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_no_alloc_decode_matches_workspace_decode(device, dtype) -> None:
    library = _lib.load()
    large = workloads.paged_batch([2049, 700, 160, 5, 1300, 33], [1] * 6, num_q_heads=32,
                                  num_kv_heads=8, head_dim=128, block_size=16, dtype=dtype,
                                  device=device, seed=61)
    small = workloads.paged_batch([300, 17], [1] * 2, num_q_heads=32, num_kv_heads=8,
                                  head_dim=128, block_size=16, dtype=dtype, device=device,
                                  seed=62)
    for batch in (large, small):
        for pages_per_split in (2, 0):
            expected = _with_workspace(library, batch, pages_per_split)
            actual = _no_alloc(library, batch, pages_per_split)
            torch.cuda.synchronize()
            assert torch.equal(actual, expected)
    # The shared kernels themselves against the oracle (tolerances of the decode tests).
    oracle = paged.decode_batch(small.query.cpu(), small.key_cache.cpu(),
                                small.value_cache.cpu(), small.block_tables.cpu(),
                                small.seq_lens.cpu(), 0,
                                None if dtype == torch.float32 else torch.float32)
    tol = dict(rtol=1e-5, atol=1e-6) if dtype == torch.float32 else dict(rtol=0, atol=2e-2)
    torch.testing.assert_close(actual.cpu(), oracle, **tol)


def test_no_alloc_decode_rejects_batches_beyond_the_static_buffer(device) -> None:
    library = _lib.load()
    limit = library.tks_paged_attention_decode_noalloc_max_workspace_bytes()
    assert limit == 32 << 20
    # 4096 sequences x 32 heads split into 64 one-page splits: GiBs of partials.
    needed = library.tks_paged_attention_decode_workspace_bytes(4096, 32, 8, 128, 16, 1024, 1)
    assert needed > limit
    status = library.tks_paged_attention_decode_noalloc(
        None, 0, 0, None, None, 1, 65536, 8, 16, 128, 0, None, 64, None, None, 4096, 32, 1024,
        0.1, 1, None, 0, 0, 2, None)
    assert status == _lib.TKS_ERR_WORKSPACE
    assert ctypes.c_int32(status).value == -4


def test_no_alloc_decode_allocates_nothing_and_replays_in_a_graph(device) -> None:
    """What the entry point is for: a multi-split batch (pages_per_split 2, so the split
    partials go to the static buffer) leaves torch's allocated device memory unchanged
    when called eagerly, and the call captured in a HIP graph gives the workspace entry's
    output on every replay, with eager work and synchronisations between the replays."""

    library = _lib.load()
    batch = workloads.paged_batch([2049, 700, 160, 5], [1] * 4, num_q_heads=32,
                                  num_kv_heads=8, head_dim=128, block_size=16,
                                  dtype=torch.bfloat16, device=device, seed=63)
    other = workloads.paged_batch([900, 31], [1] * 2, num_q_heads=32, num_kv_heads=8,
                                  head_dim=128, block_size=16, dtype=torch.bfloat16,
                                  device=device, seed=64)
    expected = _with_workspace(library, batch, 2)
    expected_other = _with_workspace(library, other, 2)
    out = torch.empty_like(batch.query)
    code = _lib.dtype_code(batch.query.dtype)
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated(device)
    status = library.tks_paged_attention_decode_noalloc(*_args(batch, out, 2), code,
                                                        _lib.stream_of(batch.query))
    torch.cuda.synchronize()
    assert status == _lib.TKS_OK
    assert torch.cuda.memory_allocated(device) == before
    assert torch.equal(out, expected)

    captured = torch.zeros_like(batch.query)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        status = library.tks_paged_attention_decode_noalloc(
            *_args(batch, captured, 2), code, _lib.stream_of(batch.query))
    assert status == _lib.TKS_OK
    for _ in range(3):
        captured.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, expected)
        # An eager call on another batch between replays reuses the static buffer.
        assert torch.equal(_no_alloc(library, other, 2), expected_other)
        torch.cuda.synchronize()
