"""Pins the CPU oracle before it is trusted as the checker of the HIP kernels.

Every oracle function is checked against something that does not share its
code: the known answers of the reference's own tests (cited per test), float64
closed forms written independently (oracle/fp64.py), or a second independent
implementation (the C restatement vs torch indexing). Each check is chosen so a
plausible mistake -- a dropped term, a wrong sign or index, a swapped operand,
an off-by-one in the causal mask or in a block offset -- fails it; a few tests
plant such a mistake in a copy of the oracle and assert the pin catches it.
"""

from math import prod

import numpy as np
import pytest
import torch
from torch.testing import assert_close

from oracle import fp64, kvslots, paged, torch_path


# --------------------------------------------------------------------------
# Attention


@pytest.mark.parametrize(("hq", "hkv"), [(2, 2), (4, 2), (8, 2), (32, 8)])
@pytest.mark.parametrize("offset_extra", [0, 3])
def test_causal_gqa_matches_fp64_closed_form(hq: int, hkv: int, offset_extra: int) -> None:
    """tests/unit/engine/test_attention_contract.py:62-130 (GQA ratios) vs float64 brute force."""

    g = torch.Generator().manual_seed(100 + hq)
    tq, dh = 5, 8
    tk = tq + offset_extra
    q = torch.randn(2, hq, tq, dh, generator=g)
    k = torch.randn(2, hkv, tk, dh, generator=g)
    v = torch.randn(2, hkv, tk, dh, generator=g)
    actual = torch_path.gqa_attention(q, k, v, query_position_offset=offset_extra)
    expected = fp64.attention(q.numpy(), k.numpy(), v.numpy(), query_position_offset=offset_extra)
    np.testing.assert_allclose(actual.numpy(), expected, rtol=1e-5, atol=1e-6)


def test_head_distinct_values_pin_gqa_mapping() -> None:
    """Known answer of tests/unit/engine/test_attention_contract.py:133-158."""

    query = torch.zeros(1, 4, 1, 2)
    key = torch.zeros(1, 2, 1, 2)
    value = torch.tensor([[[[10.0, 11.0]], [[20.0, 21.0]]]])
    output = torch_path.gqa_attention(query, key, value, query_position_offset=0)
    assert_close(output[0, 0], value[0, 0])
    assert_close(output[0, 1], value[0, 0])
    assert_close(output[0, 2], value[0, 1])
    assert_close(output[0, 3], value[0, 1])


def test_decode_query_uses_absolute_position() -> None:
    """tests/unit/engine/test_attention_contract.py:161-188: offset 4 sees all 5 keys."""

    g = torch.Generator().manual_seed(101)
    q, k, v = (torch.randn(1, 4, 1, 8, generator=g), torch.randn(1, 4, 5, 8, generator=g),
               torch.randn(1, 4, 5, 8, generator=g))
    _, weights = torch_path.causal_attention(q, k, v, query_position_offset=4)
    assert weights.shape == (1, 4, 1, 5)
    assert torch.all(weights > 0)


def test_continuation_masks_future_keys() -> None:
    """tests/unit/engine/test_attention_contract.py:191-220 mask pattern."""

    g = torch.Generator().manual_seed(102)
    q = torch.randn(1, 4, 3, 4, generator=g)
    k = torch.randn(1, 4, 7, 4, generator=g)
    v = torch.randn(1, 4, 7, 4, generator=g)
    _, w = torch_path.causal_attention(q, k, v, query_position_offset=4)
    assert torch.all(w[:, :, 0, 5:] == 0)
    assert torch.all(w[:, :, 1, 6:] == 0)
    assert torch.all(w[:, :, 2, :7] > 0)


def test_future_key_changes_cannot_affect_earlier_queries() -> None:
    """tests/unit/engine/test_attention_contract.py:256-282 (atol 0)."""

    g = torch.Generator().manual_seed(104)
    q, k, v = (torch.randn(1, 2, 5, 4, generator=g) for _ in range(3))
    base, _ = torch_path.causal_attention(q, k, v)
    k2, v2 = k.clone(), v.clone()
    k2[:, :, 4, :] = 10_000.0
    v2[:, :, 4, :] = -10_000.0
    changed, _ = torch_path.causal_attention(q, k2, v2)
    assert_close(changed[:, :, :4, :], base[:, :, :4, :], rtol=0, atol=0)


def test_planted_mask_off_by_one_is_caught() -> None:
    """A causal mask of k < pos (instead of k <= pos) must fail the fp64 pin."""

    g = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn(1, 2, 4, 4, generator=g) for _ in range(3))
    scores = torch.matmul(q, k.transpose(-1, -2)) / 2.0
    wrong = scores.masked_fill(~(torch.arange(4)[None, :] < torch.arange(4)[:, None] + 0)
                               [None, None], float("-inf"))
    wrong_out = torch.matmul(torch.softmax(wrong, dim=-1).nan_to_num(0.0), v)
    expected = fp64.attention(q.numpy(), k.numpy(), v.numpy(), query_position_offset=0)
    assert not np.allclose(wrong_out.numpy(), expected, rtol=1e-5, atol=1e-6)


# --------------------------------------------------------------------------
# Online softmax / tiles


def _ordinary(scores: torch.Tensor, values: torch.Tensor) -> torch.Tensor:
    return torch.matmul(torch.softmax(scores, dim=-1), values)


def test_online_softmax_tiles_match_ordinary_softmax() -> None:
    """Closed-form tiles of tests/unit/engine/test_online_softmax.py:44-100."""

    scores = torch.tensor([[[[1.0, -2.0, 3.0, 0.5, 4.0]]]])
    values = torch.tensor([[[[1.0, 10.0], [2.0, 20.0], [3.0, 30.0], [4.0, 40.0], [5.0, 50.0]]]])
    m = torch.full((1, 1, 1, 1), float("-inf"))
    s = torch.zeros(1, 1, 1, 1)
    acc = torch.zeros(1, 1, 1, 2)
    for a, b in ((0, 2), (2, 4), (4, 5)):
        m, s, acc = torch_path.online_softmax_update(m, s, acc, scores[..., a:b], values[..., a:b, :])
    assert_close(acc / s, _ordinary(scores, values), rtol=1e-6, atol=1e-6)
    assert float(m) == 4.0


def test_online_softmax_rescales_old_accumulator() -> None:
    """A later tile with a larger maximum must rescale the earlier partials."""

    m = torch.full((1, 1, 1, 1), float("-inf"))
    s = torch.zeros(1, 1, 1, 1)
    acc = torch.zeros(1, 1, 1, 1)
    m, s, acc = torch_path.online_softmax_update(m, s, acc, torch.tensor([[[[0.0]]]]),
                                                torch.tensor([[[[1.0]]]]))
    m, s, acc = torch_path.online_softmax_update(m, s, acc, torch.tensor([[[[10.0]]]]),
                                                torch.tensor([[[[2.0]]]]))
    expected = (np.exp(-10.0) * 1.0 + 2.0) / (np.exp(-10.0) + 1.0)
    assert abs(float(acc / s) - expected) < 1e-6


@pytest.mark.parametrize(("bq", "bk"), [(1, 1), (3, 5), (16, 16), (64, 7)])
def test_tiled_attention_is_tile_size_independent(bq: int, bk: int) -> None:
    """tests/unit/engine/test_tiled_attention.py:185-213 vs the ordinary path."""

    g = torch.Generator().manual_seed(9)
    q = torch.randn(1, 4, 13, 8, generator=g)
    k = torch.randn(1, 2, 20, 8, generator=g)
    v = torch.randn(1, 2, 20, 8, generator=g)
    tiled = torch_path.tiled_attention(q, k, v, query_position_offset=7, query_block_size=bq,
                                       key_block_size=bk)
    plain = torch_path.gqa_attention(q, k, v, query_position_offset=7)
    assert_close(tiled, plain, rtol=1e-5, atol=1e-6)


# --------------------------------------------------------------------------
# RMSNorm


@pytest.mark.parametrize("shape", [(4, 7), (2, 3, 8), (1, 13)])
@pytest.mark.parametrize("epsilon", [1e-6, 1e-3])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
def test_rmsnorm_explicit_formula(shape: tuple[int, ...], epsilon: float, dtype: torch.dtype) -> None:
    """Inputs and weights of tests/unit/engine/test_rmsnorm_contract.py:11-38; fp64 closed form."""

    hidden = shape[-1]
    x = (torch.arange(prod(shape), dtype=torch.float32).reshape(shape) / 7.0 - 1.0).to(dtype)
    w = torch.linspace(0.5, 1.5, hidden, dtype=torch.float32)
    out = torch_path.rms_norm(x, w, epsilon)
    assert out.dtype == torch.float32  # fp32 weight promotes
    expected = fp64.rms_norm(x.to(torch.float64).numpy(), w.numpy(), epsilon)
    # The only rounding beyond fp32 is the cast of the normalised value to dtype.
    tol = {torch.float32: 1e-6, torch.float16: 1e-3, torch.bfloat16: 8e-3}[dtype]
    np.testing.assert_allclose(out.numpy(), expected, rtol=tol, atol=tol)


def test_rmsnorm_rounds_before_weight_multiply() -> None:
    """bf16: the normalised value is rounded to bf16 before the fp32 weight product
    (tokserve/engine/layers.py:42): a weight of 1 + 2^-12 must survive in the output."""

    x = torch.tensor([[1.0, 1.0, 1.0, 1.0]], dtype=torch.bfloat16)
    w = torch.full((4,), 1.0 + 2.0**-12, dtype=torch.float32)
    out = torch_path.rms_norm(x, w, 1e-30)
    assert torch.all(out == torch.tensor(1.0 + 2.0**-12, dtype=torch.float32))


# --------------------------------------------------------------------------
# RoPE


def test_rope_matches_numpy_reference_values() -> None:
    """tests/unit/engine/test_rope.py:16-45: arange inputs, positions 0..3, rtol 1e-5."""

    q = np.arange(32, dtype=np.float64).reshape(1, 2, 4, 4)
    k = np.arange(16, dtype=np.float64).reshape(1, 1, 4, 4)
    pos = np.arange(4, dtype=np.int64)
    tq, tk = torch_path.apply_rope(torch.tensor(q, dtype=torch.float32),
                                   torch.tensor(k, dtype=torch.float32),
                                   torch.tensor(pos), theta=10_000.0)
    eq, ek = fp64.rope(q, k, pos, theta=10_000.0)
    np.testing.assert_allclose(tq.numpy(), eq, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(tk.numpy(), ek, rtol=1e-5, atol=1e-6)


def test_rope_position_zero_identity_and_norm_preservation() -> None:
    """tests/unit/engine/test_rope.py:48-101."""

    q = torch.tensor([[[[1.0, 2.0, 3.0, 4.0]]]])
    k = torch.tensor([[[[4.0, 3.0, 2.0, 1.0]]]])
    rq, rk = torch_path.apply_rope(q, k, torch.tensor([0]), theta=10_000.0)
    assert_close(rq, q)
    assert_close(rk, k)
    g = torch.Generator().manual_seed(17)
    q = torch.randn(1, 2, 3, 4, generator=g)
    k = torch.randn(1, 1, 3, 4, generator=g)
    rq, rk = torch_path.apply_rope(q, k, torch.arange(3), theta=10_000.0)
    assert_close(torch.linalg.vector_norm(rq, dim=-1), torch.linalg.vector_norm(q, dim=-1))
    assert_close(torch.linalg.vector_norm(rk, dim=-1), torch.linalg.vector_norm(k, dim=-1))


def test_rope_large_positions_theta_500k_fp32_close_to_fp64() -> None:
    """Positions up to 4351 with theta 5e5 (the packed norm+rope shape): fp32 angles,
    one rounding each, stay within fp32 angle error of the float64 formula."""

    g = torch.Generator().manual_seed(3)
    pos = torch.tensor([0, 1, 17, 1000, 4095, 4351])
    q = torch.randn(1, 2, pos.numel(), 128, generator=g)
    k = torch.randn(1, 1, pos.numel(), 128, generator=g)
    tq, tk = torch_path.apply_rope(q, k, pos, theta=500000.0)
    eq, ek = fp64.rope(q.double().numpy(), k.double().numpy(), pos.numpy(), theta=500000.0)
    # angle = pos * inv_freq rounded to fp32: |err| <= 4351 * 2^-24 ~ 2.6e-4 rad.
    np.testing.assert_allclose(tq.numpy(), eq, atol=2e-3)
    np.testing.assert_allclose(tk.numpy(), ek, atol=2e-3)


def test_planted_rotate_half_sign_error_is_caught() -> None:
    q = np.arange(32, dtype=np.float64).reshape(1, 2, 4, 4)
    pos = np.arange(4, dtype=np.int64)
    qt = torch.tensor(q, dtype=torch.float32)
    cos, sin = torch_path.rotary_cos_sin(torch.tensor(pos), 4, theta=10_000.0, dtype=torch.float32)
    half = 2
    wrong_rot = torch.cat((qt[..., half:], -qt[..., :half]), dim=-1)  # sign swapped
    wrong = qt * cos + wrong_rot * sin
    eq, _ = fp64.rope(q, q, pos, theta=10_000.0)
    assert not np.allclose(wrong.numpy(), eq, rtol=1e-5, atol=1e-6)


# --------------------------------------------------------------------------
# Paged KV: slots, append, gather


def test_slot_closed_form_matches_block_table_resolve() -> None:
    """slot = block_ids[p // BS] * BS + p % BS (tokserve/engine/paged/block_table.py:53-67)."""

    ids = [7, 3, 11, 0]
    for bs in (1, 2, 4, 16):
        for p in range(len(ids) * bs):
            assert kvslots.slot(ids, bs, p) == ids[p // bs] * bs + p % bs
        assert kvslots.slot(ids, bs, len(ids) * bs) == -1  # past the table


def test_c_append_then_gather_round_trip_and_sentinels() -> None:
    """Distinct values per layer (tests/integration/test_paged_kv_cache_parity.py:54-76):
    K = v + 100 * layer, V = K + 1000; unwritten slots keep their sentinel."""

    layers, nb, hkv, bs, dh = 2, 8, 2, 4, 3
    kc = torch.full((layers, nb, hkv, bs, dh), 50_000.0)
    vc = torch.full((layers, nb, hkv, bs, dh), -50_000.0)
    tables = torch.tensor([[5, 2, 7], [1, 6, 0]], dtype=torch.int32)
    lens = torch.tensor([9, 6])
    slots = kvslots.slot_mapping(tables, torch.zeros(2, dtype=torch.int64), lens, bs)
    tokens = int(lens.sum())
    base = torch.arange(tokens, dtype=torch.float32) + 1.0
    for layer in range(layers):
        keys = (base + 100.0 * layer).view(-1, 1, 1).expand(tokens, hkv, dh).contiguous()
        kvslots.kv_append(keys, keys + 1000.0, kc, vc, slots, layer)
    for layer in range(layers):
        k_out, v_out = kvslots.paged_gather(kc, vc, tables, lens, layer)
        assert torch.equal(k_out[:, 0, 0], base + 100.0 * layer)
        assert torch.equal(v_out, k_out + 1000.0)
    # 15 tokens written per layer into 4-token blocks: exactly 32 - 15 = 17 slots per
    # layer still hold the sentinel (blocks 3 and 4 untouched, 1 slot in block 7, 2 in 0).
    untouched = (kc[:, :, 0, :, 0] == 50_000.0).sum().item()
    assert untouched == layers * (nb * bs - tokens)


def test_c_gather_matches_torch_index_gather() -> None:
    """Two independent gathers (C loop vs torch advanced indexing) agree bit for bit."""

    g = torch.Generator().manual_seed(4)
    kc = torch.randn(3, 20, 2, 16, 8, generator=g).to(torch.bfloat16)
    vc = torch.randn(3, 20, 2, 16, 8, generator=g).to(torch.bfloat16)
    tables = torch.randperm(20, generator=g)[:12].view(3, 4).to(torch.int32)
    lens = torch.tensor([64, 1, 37])
    k_c, v_c = kvslots.paged_gather(kc, vc, tables, lens, 2)
    start = 0
    for b in range(3):
        k_t, v_t = paged.read_layer(kc, vc, tables[b], 2, int(lens[b]))
        n = int(lens[b])
        assert torch.equal(k_c[start:start + n], k_t[0].permute(1, 0, 2))
        assert torch.equal(v_c[start:start + n], v_t[0].permute(1, 0, 2))
        start += n


def test_paged_attention_noncontiguous_pages_match_contiguous() -> None:
    """Sentinel pool, pages (3, 1, 2), key_length 5
    (tests/gpu/test_paged_tiled_attention.py:30-79), on the CPU oracle."""

    g = torch.Generator().manual_seed(700)
    kc = torch.full((1, 4, 2, 2, 8), 50_000.0)
    vc = torch.full((1, 4, 2, 2, 8), -50_000.0)
    block_ids = (3, 1, 2)
    q = torch.randn(1, 4, 1, 8, generator=g)
    lk = torch.randn(1, 2, 5, 8, generator=g)
    lv = torch.randn(1, 2, 5, 8, generator=g)
    for p in range(5):
        kc[0, block_ids[p // 2], :, p % 2, :] = lk[0, :, p, :]
        vc[0, block_ids[p // 2], :, p % 2, :] = lv[0, :, p, :]
    actual = paged.paged_attention(q, kc, vc, block_ids, layer=0, key_length=5,
                                   query_position_offset=4)
    expected = fp64.attention(q.numpy(), lk.numpy(), lv.numpy(), query_position_offset=4)
    np.testing.assert_allclose(actual.numpy(), expected, rtol=1e-5, atol=1e-6)


def test_batched_decode_and_prefill_oracles_match_fp64() -> None:
    g = torch.Generator().manual_seed(11)
    hq, hkv, dh, bs = 4, 2, 8, 4
    contexts, qlens = [5, 9, 1], [2, 9, 1]
    nb = 10
    kc = torch.randn(1, nb, hkv, bs, dh, generator=g)
    vc = torch.randn(1, nb, hkv, bs, dh, generator=g)
    tables = torch.tensor([[4, 0, 0], [9, 2, 7], [3, 0, 0]], dtype=torch.int32)
    cu = torch.tensor([0, 2, 11, 12], dtype=torch.int32)
    q = torch.randn(12, hq, dh, generator=g)
    out = paged.prefill_batch(q, kc, vc, tables, torch.tensor(contexts), cu, 0)
    for b, (ctx, ql) in enumerate(zip(contexts, qlens)):
        k, v = paged.read_layer(kc, vc, tables[b], 0, ctx)
        qb = q[cu[b]:cu[b + 1]].permute(1, 0, 2).unsqueeze(0)
        exp = fp64.attention(qb.numpy(), k.numpy(), v.numpy(), query_position_offset=ctx - ql)
        np.testing.assert_allclose(out[cu[b]:cu[b + 1]].permute(1, 0, 2).numpy(), exp[0],
                                   rtol=1e-5, atol=1e-6)
    dec = paged.decode_batch(q[:3], kc, vc, tables, torch.tensor(contexts), 0)
    for b, ctx in enumerate(contexts):
        k, v = paged.read_layer(kc, vc, tables[b], 0, ctx)
        exp = fp64.attention(q[b][None, :, None, :].numpy(), k.numpy(), v.numpy(),
                             query_position_offset=ctx - 1)
        np.testing.assert_allclose(dec[b].numpy(), exp[0, :, 0, :], rtol=1e-5, atol=1e-6)


def test_kernel_arithmetic_oracle_is_fp64_rounded_once() -> None:
    """compute_dtype=float32 (the reference GPU kernel's arithmetic) on bf16 inputs equals the
    fp64 attention of the same bf16 values rounded once to bf16 (one bf16 ulp at most), while
    the torch-backend arithmetic rounds after every op and lands measurably further away."""

    g = torch.Generator().manual_seed(12)
    hq, hkv, dh, bs, ctx, ql = 8, 2, 64, 16, 200, 40
    kc = torch.randn(1, 16, hkv, bs, dh, generator=g).bfloat16()
    vc = torch.randn(1, 16, hkv, bs, dh, generator=g).bfloat16()
    table = torch.randperm(16, generator=g)[:13].to(torch.int32)[None]
    q = torch.randn(ql, hq, dh, generator=g).bfloat16()
    lens, cu = torch.tensor([ctx]), torch.tensor([0, ql], dtype=torch.int32)
    fast = paged.prefill_batch(q, kc, vc, table, lens, cu, 0, torch.float32)
    slow = paged.prefill_batch(q, kc, vc, table, lens, cu, 0)
    k, v = paged.read_layer(kc, vc, table[0], 0, ctx)
    exact = fp64.attention(q.permute(1, 0, 2)[None].double().numpy(), k.double().numpy(),
                           v.double().numpy(), query_position_offset=ctx - ql)
    exact = torch.from_numpy(exact[0]).permute(1, 0, 2)
    ulp = torch.finfo(torch.bfloat16).eps * exact.abs().clamp_min(2.0 ** -8)
    assert ((fast.double() - exact).abs() <= ulp).all()
    assert (slow.double() - exact).abs().max() > (fast.double() - exact).abs().max()


# --------------------------------------------------------------------------
# Greedy


def test_greedy_first_index_on_ties_and_nan() -> None:
    logits = torch.tensor([[1.0, 3.0, 3.0, 2.0], [0.0, float("nan"), 5.0, float("nan")],
                           [-float("inf")] * 4])
    assert torch_path.select_greedy(logits).flatten().tolist() == [1, 1, 0]


# --------------------------------------------------------------------------
# fp8 (e4m3) pools: the torch restatement (oracle/paged.py) against the C
# encoder written from the OCP format definition (oracle/e4m3.c) and against
# hand-worked codes.


def _e4m3_values() -> torch.Tensor:
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    return codes.view(torch.float8_e4m3fn).float()


def test_e4m3_decode_known_codes_and_table() -> None:
    """All 256 codes decode alike in C and torch; hand-worked codes pin the format."""

    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    c = kvslots.e4m3_decode(codes)
    t = _e4m3_values()
    assert torch.equal(torch.isnan(c), torch.isnan(t))
    assert torch.equal(c[~torch.isnan(c)], t[~torch.isnan(t)])
    known = {0x00: 0.0, 0x01: 2.0 ** -9, 0x07: 7 * 2.0 ** -9, 0x08: 2.0 ** -6, 0x38: 1.0,
             0x39: 1.125, 0x3F: 1.875, 0x40: 2.0, 0x7E: 448.0, 0xB8: -1.0, 0xFE: -448.0}
    for code, value in known.items():
        assert float(c[code]) == value, hex(code)
    assert torch.isnan(c[0x7F]) and torch.isnan(c[0xFF])
    assert int(torch.isnan(c).sum()) == 2


def test_e4m3_encode_ties_saturation_and_nan_known_answers() -> None:
    x = torch.tensor([1.0625, 1.1875, 2.0 ** -10, 3 * 2.0 ** -10, 464.0, 1e30, float("inf"),
                      -float("inf"), -0.0, 0.0, 440.0, 432.0, float("nan"), 2.0 ** -6 - 2.0 ** -10])
    # 1.0625 is the midpoint of 1.0 (m 0) and 1.125 (m 1): even -> 0x38; 1.1875 -> 1.25 (m 2);
    # 2^-10 -> 0 (even), 3*2^-10 -> 2^-8 (m 2); beyond 448 saturates to 448 (0x7E);
    # 440 lies above 432, the midpoint of 416 (m 5) and 448 (m 6) -> 448; 432 itself ties
    # -> even m 6 = 448; 2^-6 - 2^-10 = 7.5 * 2^-9 ties -> 8 * 2^-9 = 2^-6 (0x08).
    expected = [0x38, 0x3A, 0x00, 0x02, 0x7E, 0x7E, 0x7E, 0xFE, 0x80, 0x00, 0x7E, 0x7E, None,
                0x08]
    for got in (kvslots.e4m3_encode(x), paged.quantize_e4m3(x, 1.0).view(torch.uint8)):
        for i, want in enumerate(expected):
            if want is None:
                assert int(got[i]) & 0x7F == 0x7F
            else:
                assert int(got[i]) == want, (float(x[i]), hex(int(got[i])))


@pytest.mark.parametrize("scale", [1.0, 0.37, 3.3, 2.0 ** -4])
def test_e4m3_quantize_matches_c_encoder(scale: float) -> None:
    """Random magnitudes over 2^-14 .. 2^11, every midpoint between neighbouring codes and
    the floats either side of it: torch's conversion equals the C encoder."""

    g = torch.Generator().manual_seed(7)
    x = torch.cat([torch.randn(50_000, generator=g) * 2.0 ** e for e in range(-14, 12, 2)])
    pos = _e4m3_values()
    pos = pos[~torch.isnan(pos) & (pos >= 0)].unique().sort().values
    mids = ((pos[:-1].double() + pos[1:].double()) / 2).float() * scale
    up = torch.nextafter(mids, torch.full_like(mids, float("inf")))
    down = torch.nextafter(mids, torch.zeros_like(mids))
    x = torch.cat([x, mids, -mids, up, down])
    assert torch.equal(kvslots.e4m3_encode(x, scale), paged.quantize_e4m3(x, scale).view(torch.uint8))


def test_e4m3_planted_truncation_is_caught() -> None:
    """A quantizer that truncates (largest code <= |x|) instead of rounding to nearest
    even disagrees with the C encoder; the torch restatement agrees with it."""

    x = torch.linspace(0.01, 400.0, 10_001)
    values = _e4m3_values()
    values = values[~torch.isnan(values) & (values >= 0)].unique().sort().values
    truncated = values[torch.searchsorted(values, x, right=True) - 1]
    rounded = kvslots.e4m3_decode(kvslots.e4m3_encode(x))
    assert not torch.equal(truncated, rounded)
    assert torch.equal(kvslots.e4m3_encode(x), paged.quantize_e4m3(x, 1.0).view(torch.uint8))


# fp8 pools with one scale per pool row: the torch restatement against the C
# quantizer, closed forms of the scale rule, and a planted mistake.


def _row_cases() -> torch.Tensor:
    g = torch.Generator().manual_seed(17)
    magnitude = 2.0 ** torch.randint(-30, 30, (400, 1), generator=g).float()
    x = torch.randn(400, 64, generator=g) * magnitude
    x[0] = 0.0
    x[1, 5] = float("nan")
    x[2, 9] = float("inf")
    x[3, 2] = -float("inf")
    x[4] = -x[4].abs()
    x[5] = torch.randn(64, generator=g) * 1e-41     # subnormal row
    x[6] = 3e38                                     # amax / 448 finite, x / s = 448
    x[7] = 448.0
    x[8, 0] = -0.0
    return x


def test_e4m3_row_quantizer_matches_c() -> None:
    x = _row_cases()
    codes, scales = kvslots.e4m3_encode_rows(x)
    t_codes, t_scales = paged.quantize_e4m3_rows(x)
    assert torch.equal(scales, t_scales)
    assert torch.equal(codes, t_codes.view(torch.uint8))


def test_e4m3_row_scale_closed_forms() -> None:
    """s = max|row| / 448 for finite nonzero rows, so every such row's largest magnitude
    is code 448 (0x7E / 0xFE) and every element decodes within half an e4m3 step of x
    (2^-4 relative, 2^-10 s absolute below the normal range); zero, NaN and infinite
    maxima give s = 1."""

    x = _row_cases()
    codes, scales = kvslots.e4m3_encode_rows(x)
    amax = x.abs().amax(dim=1)
    regular = torch.isfinite(amax) & (amax > 0)
    assert torch.equal(scales[regular], (amax / 448.0)[regular])
    assert torch.equal(scales[~regular], torch.ones(int((~regular).sum())))
    assert int((~regular).sum()) == 4  # rows 0, 1, 2, 3
    top = x.abs().argmax(dim=1)
    top_codes = codes[torch.arange(x.shape[0]), top]
    assert torch.all(top_codes[regular] & 0x7F == 0x7E)
    decoded = paged.dequantize_e4m3_rows(codes.view(torch.float8_e4m3fn), scales, torch.float32)
    finite = regular.unsqueeze(1).expand_as(x)
    bound = torch.maximum(x.abs() * 2.0 ** -4, scales.unsqueeze(1) * 2.0 ** -10)
    assert torch.all((decoded - x).abs()[finite] <= bound[finite])
    assert torch.isnan(decoded[1, 5]) and int(codes[2, 9]) == 0x7E and int(codes[3, 2]) == 0xFE


def test_e4m3_row_quantizer_planted_mistakes_are_caught() -> None:
    """A scale from the signed maximum (max x instead of max |x|), or one that keeps 0 for
    an all-zero row, disagrees with the C quantizer."""

    x = _row_cases()
    codes, scales = kvslots.e4m3_encode_rows(x)
    signed = x.amax(dim=1) / 448.0
    signed = torch.where((signed > 0) & torch.isfinite(signed), signed, torch.ones_like(signed))
    assert not torch.equal(signed, scales)
    assert not torch.equal(torch.clamp(x / signed.unsqueeze(1), -448, 448)
                           .to(torch.float8_e4m3fn).view(torch.uint8), codes)
    zero_kept = torch.where(torch.isfinite(x.abs().amax(dim=1)), x.abs().amax(dim=1) / 448.0,
                            torch.ones(x.shape[0]))
    assert not torch.equal(zero_kept, scales)
