"""Llama forward of the reference's torch backend, restated on the CPU (test infrastructure).

Op order and dtypes follow tokserve/engine/model.py:45-206 with the torch
backend of tokserve/engine/attention.py:175-368 and layers.py:29-91:
  h = embed(ids)
  per layer: x = rms_norm(h); q, k, v = x Wq^T, x Wk^T, x Wv^T; RoPE(q, k) at
             positions cache_len ..; K/V appended to the layer's cache; causal GQA
             over cache_len + T keys with offset cache_len; r = h + o_proj(attn);
             h = r + down(silu(gate(rms_norm(r))) * up(rms_norm(r)))
  logits = lm_head(rms_norm(h))
Weights come from a state dict with the reference's parameter names. The paged
pool is replaced by a per-layer contiguous K/V cache in logical order, which is
what the reference's read_layer rebuilds (sequence_cache.py:133-193).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch
from torch.nn import functional

from oracle.paged import (dequantize_e4m3, dequantize_e4m3_rows, quantize_e4m3,
                          quantize_e4m3_rows)
from oracle.torch_path import apply_rope, gqa_attention, rms_norm


@dataclass
class SequenceKV:
    """Per-layer (1, Hkv, S, Dh) K/V of one sequence, in logical order."""

    keys: list[torch.Tensor] = field(default_factory=list)
    values: list[torch.Tensor] = field(default_factory=list)

    @property
    def length(self) -> int:
        return 0 if not self.keys else self.keys[0].shape[2]


def forward(state: dict[str, torch.Tensor], config: dict, token_ids: torch.Tensor,
            cache: SequenceKV | None = None,
            kv_quant: tuple[float, float] | str | None = None) -> torch.Tensor:
    """token_ids (1, T) -> logits (1, T, V); appends the T tokens' K/V to `cache`.

    kv_quant = (k_scale, v_scale) models fp8 e4m3 pools: every K/V row attention
    sees has been through quantize_e4m3 / dequantize_e4m3 with those scales;
    kv_quant = "row" models fp8 pools with one scale per (token, KV head) row
    (quantize_e4m3_rows / dequantize_e4m3_rows).
    """

    hq, hkv = config["num_attention_heads"], config["num_key_value_heads"]
    hidden_size = config["hidden_size"]
    dh = hidden_size // hq
    eps, theta = config["rms_norm_eps"], config["rope_theta"]
    length = token_ids.shape[1]
    start = 0 if cache is None else cache.length
    positions = torch.arange(start, start + length, dtype=torch.int64)
    hidden = functional.embedding(token_ids, state["embed_tokens.weight"])
    for layer in range(config["num_hidden_layers"]):
        p = f"layers.{layer}."
        x = rms_norm(hidden, state[p + "input_norm.weight"], eps)
        q = functional.linear(x, state[p + "self_attention.q_proj.weight"])
        k = functional.linear(x, state[p + "self_attention.k_proj.weight"])
        v = functional.linear(x, state[p + "self_attention.v_proj.weight"])
        q = q.reshape(1, length, hq, dh).transpose(1, 2)
        k = k.reshape(1, length, hkv, dh).transpose(1, 2)
        v = v.reshape(1, length, hkv, dh).transpose(1, 2)
        q, k = apply_rope(q, k, positions, theta=theta)
        if kv_quant == "row":
            k = dequantize_e4m3_rows(*quantize_e4m3_rows(k), k.dtype)
            v = dequantize_e4m3_rows(*quantize_e4m3_rows(v), v.dtype)
        elif kv_quant is not None:
            k = dequantize_e4m3(quantize_e4m3(k, kv_quant[0]), kv_quant[0], k.dtype)
            v = dequantize_e4m3(quantize_e4m3(v, kv_quant[1]), kv_quant[1], v.dtype)
        if cache is not None:
            if len(cache.keys) <= layer:
                cache.keys.append(k)
                cache.values.append(v)
            else:
                cache.keys[layer] = torch.cat((cache.keys[layer], k), dim=2)
                cache.values[layer] = torch.cat((cache.values[layer], v), dim=2)
            k, v = cache.keys[layer], cache.values[layer]
        attended = gqa_attention(q, k, v, query_position_offset=start)
        merged = attended.transpose(1, 2).contiguous().reshape(1, length, hidden_size)
        residual = hidden + functional.linear(merged, state[p + "self_attention.o_proj.weight"])
        x = rms_norm(residual, state[p + "post_attention_norm.weight"], eps)
        gate = functional.silu(functional.linear(x, state[p + "mlp.gate_proj.weight"]))
        up = functional.linear(x, state[p + "mlp.up_proj.weight"])
        hidden = residual + functional.linear(gate * up, state[p + "mlp.down_proj.weight"])
    normed = rms_norm(hidden, state["final_norm.weight"], eps)
    return functional.linear(normed, state["lm_head.weight"])
