"""ctypes binding of oracle/kvslots.c and oracle/e4m3.c (TEST INFRASTRUCTURE ONLY).

Bit-exact CPU restatement of slot mapping, KV append and block-table gather
(tokserve/engine/paged/block_table.py:53-67, storage.py:64-116,
sequence_cache.py:86-193), and of the OCP fp8 e4m3 encoding of fp8 pools.
Operates on contiguous CPU tensors.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import torch

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle_kv.so"
_lib: ctypes.CDLL | None = None

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64


def build() -> Path:
    """Compile kvslots.c with gcc (idempotent)."""

    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def _load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.is_file():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        lib.oracle_slot.restype = _i64
        lib.oracle_slot.argtypes = [_p, _i64, _i32, _i64]
        lib.oracle_slot_mapping.restype = _i32
        lib.oracle_slot_mapping.argtypes = [_p, _i32, _p, _p, _i32, _i32, _p]
        lib.oracle_kv_append.restype = _i32
        lib.oracle_kv_append.argtypes = [
            _p, _i64, _i64, _p, _i64, _i64, _i64, _p, _p, _i64, _i32, _i32, _i32, _i32, _p, _i32,
        ]
        lib.oracle_paged_gather.restype = _i32
        lib.oracle_paged_gather.argtypes = [
            _p, _p, _i64, _i32, _i32, _i32, _i32, _p, _i32, _p, _p, _i32, _p, _p, _i64, _i64, _i32,
        ]
        lib.oracle_e4m3_encode_array.restype = None
        lib.oracle_e4m3_encode_array.argtypes = [_p, _i64, ctypes.c_float, _p]
        lib.oracle_e4m3_decode_array.restype = None
        lib.oracle_e4m3_decode_array.argtypes = [_p, _i64, _p]
        lib.oracle_e4m3_encode_rows.restype = None
        lib.oracle_e4m3_encode_rows.argtypes = [_p, _i64, _i64, _p, _p]
        _lib = lib
    return _lib


def _cpu(t: torch.Tensor) -> None:
    if t.device.type != "cpu":
        raise ValueError("oracle tensors must be on the CPU")


def slot(block_ids: list[int], block_size: int, position: int) -> int:
    """Slot of one logical position (-1 past the table)."""

    table = torch.tensor(block_ids, dtype=torch.int32)
    return int(_load().oracle_slot(table.data_ptr(), len(block_ids), block_size, position))


def slot_mapping(
    block_tables: torch.Tensor, start: torch.Tensor, new_lens: torch.Tensor, block_size: int
) -> torch.Tensor:
    """Slots of positions start[b] .. start[b]+new_lens[b]-1 for each sequence, packed."""

    tables = block_tables.to(torch.int32).contiguous()
    start = start.to(torch.int64).contiguous()
    new_lens = new_lens.to(torch.int64).contiguous()
    out = torch.empty(int(new_lens.sum()), dtype=torch.int64)
    status = _load().oracle_slot_mapping(
        tables.data_ptr(), tables.shape[1], start.data_ptr(), new_lens.data_ptr(),
        tables.shape[0], block_size, out.data_ptr(),
    )
    if status != 0:
        raise IndexError("position exceeds block table capacity")
    return out


def kv_append(
    key: torch.Tensor,
    value: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    slots: torch.Tensor,
    layer: int,
) -> None:
    """In-place scatter of (N, Hkv, Dh) rows into CPU pools."""

    for t in (key, value, key_cache, value_cache, slots):
        _cpu(t)
    key = key.contiguous()
    value = value.contiguous()
    slots = slots.to(torch.int64).contiguous()
    _, num_blocks, num_kv_heads, block_size, head_dim = key_cache.shape
    status = _load().oracle_kv_append(
        key.data_ptr(), key.stride(0), key.stride(1), value.data_ptr(), value.stride(0),
        value.stride(1), key.shape[0], key_cache.data_ptr(), value_cache.data_ptr(),
        num_blocks, num_kv_heads, block_size, head_dim, layer, slots.data_ptr(),
        key.element_size(),
    )
    if status != 0:
        raise IndexError("slot is out of range")


def paged_gather(
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    layer: int,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(S_total, Hkv, Dh) logical-order K/V of every sequence, packed by cu_seqlens."""

    _, num_blocks, num_kv_heads, block_size, head_dim = key_cache.shape
    tables = block_tables.to(torch.int32).contiguous()
    lens = seq_lens.to(torch.int32).contiguous()
    cu = torch.zeros(lens.shape[0] + 1, dtype=torch.int32)
    cu[1:] = torch.cumsum(lens, 0)
    total = int(cu[-1])
    key_out = torch.empty((total, num_kv_heads, head_dim), dtype=key_cache.dtype)
    value_out = torch.empty_like(key_out)
    status = _load().oracle_paged_gather(
        key_cache.data_ptr(), value_cache.data_ptr(), num_blocks, num_kv_heads, block_size,
        head_dim, layer, tables.data_ptr(), tables.shape[1], lens.data_ptr(), cu.data_ptr(),
        lens.shape[0], key_out.data_ptr(), value_out.data_ptr(), key_out.stride(0),
        key_out.stride(1), key_cache.element_size(),
    )
    if status != 0:
        raise IndexError("position exceeds block table capacity")
    return key_out, value_out


def e4m3_encode(x: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """uint8 codes of e4m3(clamp(x / scale, -448, 448)) (x as float32), from e4m3.c."""

    _cpu(x)
    values = x.to(torch.float32).contiguous()
    out = torch.empty(values.shape, dtype=torch.uint8)
    _load().oracle_e4m3_encode_array(values.data_ptr(), values.numel(), scale, out.data_ptr())
    return out


def e4m3_decode(codes: torch.Tensor) -> torch.Tensor:
    """float32 values of uint8 e4m3 codes, from e4m3.c."""

    _cpu(codes)
    codes = codes.to(torch.uint8).contiguous()
    out = torch.empty(codes.shape, dtype=torch.float32)
    _load().oracle_e4m3_decode_array(codes.data_ptr(), codes.numel(), out.data_ptr())
    return out


def e4m3_encode_rows(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(uint8 codes, float32 scales) of x (..., n) with one scale per row, from e4m3.c:
    s = max|row| / 448 (1 when that is 0, NaN or infinite), codes of x / s."""

    _cpu(x)
    values = x.to(torch.float32).contiguous()
    n = values.shape[-1]
    rows = values.numel() // n if n else 0
    out = torch.empty(values.shape, dtype=torch.uint8)
    scales = torch.empty(values.shape[:-1], dtype=torch.float32)
    _load().oracle_e4m3_encode_rows(values.data_ptr(), rows, n, out.data_ptr(),
                                    scales.data_ptr())
    return out, scales
