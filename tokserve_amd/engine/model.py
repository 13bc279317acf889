"""Llama decoder model (tokserve/engine/model.py).

Module names, shapes and creation order match the reference's LlamaModel
(embed_tokens; per layer input_norm, self_attention.{q,k,v,o}_proj,
post_attention_norm, mlp.{gate,up,down}_proj; final_norm; lm_head), so state
dicts are interchangeable and torch.manual_seed(s); LlamaModel(config) draws
the same random weights in both. Pre-norm blocks: h += attn(norm(h));
h += mlp(norm(h)); logits = lm_head(norm(h)) (model.py:45-82,117-206).

`backend` ("torch" or "triton", the reference's switch, model.py:85-97) is
checked and kept; both run the same HIP kernels.

`forward` is the reference's one-sequence interface (token_ids (1, T), an
optional SequencePagedKVCache). `forward_packed` is the batched executor's: a
whole continuous-batching iteration (prefill chunks and decode tokens of many
sequences) as one packed (N,) token stream, returning logits only for each
sequence's last token. Both run on HIP tensors only.
"""

from __future__ import annotations

from typing import TYPE_CHECKING

import torch
from torch import nn

from tokserve_amd.engine.attention import GroupedQueryAttention, reject_contiguous_cache
from tokserve_amd.engine.config import LlamaConfig
from tokserve_amd.engine.kernel_backend import KernelBackend, check_backend
from tokserve_amd.engine.layers import RMSNorm, SwiGLU
from tokserve_amd.kernels import ops

if TYPE_CHECKING:
    from tokserve_amd.batching.metadata import PackedBatch
    from tokserve_amd.engine.paged.sequence_cache import SequencePagedKVCache
    from tokserve_amd.engine.paged.storage import PagedKVStorage

__all__ = ["LlamaDecoderBlock", "LlamaModel"]


class LlamaDecoderBlock(nn.Module):
    """One pre-norm Llama decoder block."""

    def __init__(self, config: LlamaConfig, *, backend: KernelBackend = "torch") -> None:
        super().__init__()
        self.backend = check_backend(backend)
        self.hidden_size = config.hidden_size
        self.input_norm = RMSNorm(config.hidden_size, epsilon=config.rms_norm_eps)
        self.self_attention = GroupedQueryAttention(config, backend=backend)
        self.post_attention_norm = RMSNorm(config.hidden_size, epsilon=config.rms_norm_eps)
        self.mlp = SwiGLU(config.hidden_size, config.intermediate_size)

    def forward(
        self,
        inputs: torch.Tensor,
        positions: torch.Tensor,
        *,
        cache: None = None,
        paged_cache: SequencePagedKVCache | None = None,
        layer_index: int | None = None,
    ) -> torch.Tensor:
        """One block on (B, T, D) inputs; `cache` must be None (the reference's contiguous
        cache is not provided, see reject_contiguous_cache)."""

        if inputs.ndim != 3:
            raise ValueError("inputs must have shape (B, T, D)")
        reject_contiguous_cache(cache, paged_cache)
        if inputs.shape[-1] != self.hidden_size:
            raise ValueError("inputs must use the configured hidden_size")
        attended = self.self_attention(self.input_norm(inputs), positions,
                                       paged_cache=paged_cache, layer_index=layer_index)
        residual = inputs + attended
        return residual + self.mlp(self.post_attention_norm(residual))


class LlamaModel(nn.Module):
    """Forward-only Llama inference model."""

    def __init__(self, config: LlamaConfig, *, backend: KernelBackend = "torch") -> None:
        super().__init__()
        self.backend = check_backend(backend)
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList(LlamaDecoderBlock(config, backend=backend)
                                    for _ in range(config.num_hidden_layers))
        self.final_norm = RMSNorm(config.hidden_size, epsilon=config.rms_norm_eps)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        self._rotary: ops.RotaryTable | None = None

    def rotary_table(self) -> ops.RotaryTable:
        """cos/sin rows for positions [0, max_position_embeddings) in the model dtype."""

        weight = self.embed_tokens.weight
        table = self._rotary
        if table is None or table.dtype != weight.dtype or table.device != weight.device:
            table = ops.RotaryTable(
                self.config.head_dim, theta=self.config.rope_theta,
                max_position=self.config.max_position_embeddings, dtype=weight.dtype,
                device=weight.device,
            )
            self._rotary = table
        return table

    # ------------------------------------------------------------ one sequence

    @torch.inference_mode()
    def forward(
        self, token_ids: torch.Tensor, *, cache: None = None,
        paged_cache: SequencePagedKVCache | None = None,
    ) -> torch.Tensor:
        """token_ids (1, T) -> logits (1, T, V); with a paged cache the T tokens are
        appended after its current_length positions (model.py:119-206). `cache` must be
        None (the reference's contiguous cache is not provided)."""

        if token_ids.ndim != 2:
            raise ValueError("token_ids must have shape (B, T)")
        reject_contiguous_cache(cache, paged_cache)
        if token_ids.dtype not in (torch.int32, torch.int64):
            raise TypeError("token_ids must contain integers")
        batch, length = token_ids.shape
        if batch < 1:
            raise ValueError("batch size must be positive")
        if length < 1:
            raise ValueError("sequence length must be positive")
        if token_ids.device != self.embed_tokens.weight.device:
            raise ValueError("token_ids and model parameters must use the same device")
        cache_length = 0
        if paged_cache is not None:
            self._validate_paged_cache(paged_cache, batch)
            cache_length = paged_cache.current_length
        total = cache_length + length
        if total > self.config.max_position_embeddings:
            raise ValueError("sequence length exceeds max_position_embeddings")
        if paged_cache is not None and total > paged_cache.max_sequence_length:
            raise ValueError("sequence exceeds paged cache max_sequence_length")
        hidden = self.embed_tokens(token_ids)
        positions = torch.arange(cache_length, total, dtype=torch.int64, device=token_ids.device)
        if paged_cache is not None:
            paged_cache.begin_append(length)
        for index, block in enumerate(self.layers):
            hidden = block(hidden, positions, paged_cache=paged_cache,
                           layer_index=index if paged_cache is not None else None)
        if paged_cache is not None:
            paged_cache.finish_append()
        return self.lm_head(self.final_norm(hidden))

    def _validate_paged_cache(self, paged_cache: SequencePagedKVCache, batch: int) -> None:
        if batch != 1:
            raise ValueError("paged model execution currently supports batch size 1")
        self.validate_storage(paged_cache.storage)
        if paged_cache.max_sequence_length > self.config.max_position_embeddings:
            raise ValueError("paged cache maximum cannot exceed max_position_embeddings")

    def validate_storage(self, storage: PagedKVStorage) -> None:
        """A paged pool this model can use (tokserve/engine/paged/inference.py:21-43)."""

        parameter = self.embed_tokens.weight
        if storage.num_layers != self.config.num_hidden_layers:
            raise ValueError("paged pool layer count must match the model")
        if storage.num_key_value_heads != self.config.num_key_value_heads:
            raise ValueError("paged pool KV head count must match the model")
        if storage.head_dim != self.config.head_dim:
            raise ValueError("paged pool head_dim must match the model")
        if storage.device != parameter.device:
            raise ValueError("paged pool device must match the model device")
        if storage.dtype != parameter.dtype:
            raise ValueError("paged pool dtype must match the model dtype")

    # ----------------------------------------------------------- packed batch

    @torch.inference_mode()
    def forward_packed(self, batch: PackedBatch, storage: PagedKVStorage) -> torch.Tensor:
        """Logits (B, V) of the last token of each sequence of a packed iteration.

        Each residual add is fused into the following RMSNorm launch; the final
        norm and lm_head run on the B last-token rows only.
        """

        rotary = self.rotary_table()
        hidden = self.embed_tokens(batch.token_ids)
        residual: torch.Tensor | None = None
        for index, block in enumerate(self.layers):
            if residual is None:
                normed, residual = self._first_norm(block, hidden)
            else:
                normed, residual = block.input_norm(hidden, residual)
            hidden = block.self_attention.forward_packed(normed, batch, storage, index, rotary)
            normed, residual = block.post_attention_norm(hidden, residual)
            hidden = block.mlp(normed)
        rows = batch.logits_rows
        last_hidden = hidden.index_select(0, rows)
        last_residual = residual.index_select(0, rows) if residual is not None else None
        if last_residual is None:
            normed = self.final_norm(last_hidden)
        else:
            normed, _ = self.final_norm(last_hidden, last_residual)
        return self.lm_head(normed)

    @staticmethod
    def _first_norm(block: LlamaDecoderBlock, hidden: torch.Tensor):
        return block.input_norm(hidden), hidden
