"""Paged K/V pools (tokserve/engine/paged/storage.py).

Two pools, K and V, shaped [L, NB, Hkv, BS, Dh] (the reference layout,
storage.py:40-56), allocated uninitialised like the reference's torch.empty.
Writes go through the KV-append kernel (tks_kv_append), reads through the
block-table gather kernel (tks_paged_gather); the kernels run on HIP devices
only, and a storage on another device rejects them.

A pool variant the reference lacks: `kv_dtype=torch.float8_e4m3fn` stores
K and V as OCP fp8 e4m3 with one fp32 scale per pool (stored =
e4m3(clamp(x / scale, -448, 448)), decoded = float(stored) * scale), half the
bytes of bf16 pools. The API is unchanged: writes take rows in `dtype`, reads
and attention see the decoded values. With `scale_granularity="row"` every pool
row (one token of one KV head) gets a scale of its own, s = max|row| / 448
(1 for an all-zero or non-finite maximum), kept beside the pools as float32
[L, NB, Hkv, BS] arrays that the append kernels write and the attention and
gather kernels read (4 bytes per Dh code bytes: 1/32 more at Dh 128).
"""

from __future__ import annotations

import torch

from tokserve_amd.kernels import ops

__all__ = ["PagedKVStorage"]


class PagedKVStorage:
    """Per-layer K/V values in shared physical blocks."""

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
        for name, size in (
            ("num_layers", num_layers),
            ("num_blocks", num_blocks),
            ("num_key_value_heads", num_key_value_heads),
            ("block_size", block_size),
            ("head_dim", head_dim),
        ):
            if size < 1:
                raise ValueError(f"{name} must be positive")
        self.num_layers = num_layers
        self.num_blocks = num_blocks
        self.num_key_value_heads = num_key_value_heads
        self.block_size = block_size
        self.head_dim = head_dim
        self.device = torch.device(device)
        self.dtype = dtype
        self.kv_dtype = dtype if kv_dtype is None else kv_dtype
        if self.kv_dtype not in (dtype, ops.FP8_POOL_DTYPE):
            raise ValueError("kv_dtype must be the model dtype or torch.float8_e4m3fn")
        self.k_scale = float(k_scale)
        self.v_scale = float(v_scale)
        if self.kv_dtype == ops.FP8_POOL_DTYPE:
            if not (0.0 < self.k_scale < float("inf") and 0.0 < self.v_scale < float("inf")):
                raise ValueError("k_scale and v_scale must be positive finite floats")
        elif self.k_scale != 1.0 or self.v_scale != 1.0:
            raise ValueError("k_scale and v_scale apply to fp8 pools only")
        if scale_granularity not in ("pool", "row"):
            raise ValueError('scale_granularity must be "pool" or "row"')
        if scale_granularity == "row" and (self.kv_dtype != ops.FP8_POOL_DTYPE
                                           or self.k_scale != 1.0 or self.v_scale != 1.0):
            raise ValueError("per-row scales need fp8 pools and no pool scales")
        self.scale_granularity = scale_granularity
        shape = (num_layers, num_blocks, num_key_value_heads, block_size, head_dim)
        self._key_storage = torch.empty(shape, device=self.device, dtype=self.kv_dtype)
        self._value_storage = torch.empty(shape, device=self.device, dtype=self.kv_dtype)
        self._key_scales: torch.Tensor | None = None
        self._value_scales: torch.Tensor | None = None
        if scale_granularity == "row":
            self._key_scales = torch.ones(shape[:4], device=self.device, dtype=torch.float32)
            self._value_scales = torch.ones(shape[:4], device=self.device, dtype=torch.float32)

    @property
    def storage_shape(self) -> tuple[int, ...]:
        return tuple(self._key_storage.shape)

    @property
    def key_storage(self) -> torch.Tensor:
        """The physical K pool, for kernels."""

        return self._key_storage

    @property
    def value_storage(self) -> torch.Tensor:
        """The physical V pool, for kernels."""

        return self._value_storage

    @property
    def key_scales(self) -> torch.Tensor | None:
        """Per-row K scales, float32 [L, NB, Hkv, BS] (None with per-pool scales)."""

        return self._key_scales

    @property
    def value_scales(self) -> torch.Tensor | None:
        """Per-row V scales, float32 [L, NB, Hkv, BS] (None with per-pool scales)."""

        return self._value_scales

    @property
    def scales(self) -> dict[str, float | torch.Tensor]:
        """Decode factors as the kernels' keyword arguments: the pool scales, or the
        per-row scale arrays."""

        if self._key_scales is not None:
            return {"k_scales": self._key_scales, "v_scales": self._value_scales}
        return {"k_scale": self.k_scale, "v_scale": self.v_scale}

    # ------------------------------------------------------------- single slot

    def write_token(
        self,
        *,
        layer_index: int,
        block_id: int,
        offset: int,
        keys: torch.Tensor,
        values: torch.Tensor,
    ) -> None:
        """Write one token's K/V, each shaped (Hkv, Dh)."""

        self._check_location(layer_index, block_id, offset)
        expected = (self.num_key_value_heads, self.head_dim)
        if keys.shape != expected or values.shape != expected:
            raise ValueError("keys and values must have shape (Hkv, Dh)")
        if keys.device != self.device or values.device != self.device:
            raise ValueError("keys and values must match the storage device")
        if keys.dtype != self.dtype or values.dtype != self.dtype:
            raise ValueError("keys and values must match the storage dtype")
        slot = torch.tensor([block_id * self.block_size + offset], dtype=torch.int64)
        self.write_slots(layer_index, slot.to(self.device), keys.unsqueeze(0), values.unsqueeze(0))

    def read_token(
        self,
        *,
        layer_index: int,
        block_id: int,
        offset: int,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Copies of one physical slot's K/V, each shaped (Hkv, Dh)."""

        self._check_location(layer_index, block_id, offset)
        # The slot is position `offset` of a one-block table holding block_id.
        keys, values = self.gather(layer_index, (block_id,), offset + 1)
        return keys[offset].clone(), values[offset].clone()

    # ----------------------------------------------------------------- batched

    def write_slots(
        self,
        layer_index: int,
        slot_mapping: torch.Tensor,
        keys: torch.Tensor,
        values: torch.Tensor,
    ) -> None:
        """KV append: row i of keys/values (N, Hkv, Dh) goes to pool slot slot_mapping[i]."""

        if layer_index < 0 or layer_index >= self.num_layers:
            raise IndexError("layer_index is out of range")
        ops.kv_append(keys, values, self._key_storage, self._value_storage, slot_mapping,
                      layer_index, **self.scales)

    def gather(
        self, layer_index: int, block_ids: tuple[int, ...] | list[int], length: int
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """K/V of logical positions 0 .. length-1 of a block table, each (length, Hkv, Dh)."""

        if layer_index < 0 or layer_index >= self.num_layers:
            raise IndexError("layer_index is out of range")
        shape = (length, self.num_key_value_heads, self.head_dim)
        keys = torch.empty(shape, device=self.device, dtype=self.dtype)
        values = torch.empty(shape, device=self.device, dtype=self.dtype)
        if length == 0:
            return keys, values
        needed = (length + self.block_size - 1) // self.block_size
        if len(block_ids) < needed:
            raise ValueError("block table does not cover the requested length")
        meta = torch.tensor([*block_ids[:needed], length, 0], dtype=torch.int32).to(self.device)
        ops.paged_gather(
            self._key_storage, self._value_storage, meta[:needed].view(1, needed),
            meta[needed : needed + 1], meta[needed + 1 :], layer_index, length, keys, values,
            **self.scales,
        )
        return keys, values

    def _check_location(self, layer_index: int, block_id: int, offset: int) -> None:
        for name, index, bound in (("layer_index", layer_index, self.num_layers),
                                   ("block_id", block_id, self.num_blocks),
                                   ("offset", offset, self.block_size)):
            if not 0 <= index < bound:
                raise IndexError(f"{name} is out of range")
