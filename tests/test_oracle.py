"""Pins of the CPU oracle (CPU only).

Each oracle function is checked against something that does not share its
formula: the reference's own known answers (test_forward.py,
tests/test_pisa_attention.py, tests/test_generic_pisa.py), a library routine
(torch SDPA, numpy.linalg.norm, torch reshape/permute tilings), brute force
on tiny inputs, or a mathematical invariant chosen so that a plausible
mistake (dropped term, wrong index, transposed operand) fails.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oatt
from oracle import layout as olayout
from oracle import pisa as opisa
from oracle.numerics import round_bf16, softmax_lse

D = 128


def _rng_bf16(shape, seed, scale=1.0):
    return round_bf16(np.random.default_rng(seed).standard_normal(shape) * scale)


# ----------------------------------------------------------------------------- numerics
def test_round_bf16_matches_torch():
    x = np.random.default_rng(0).standard_normal(10000).astype(np.float32) * 10.0
    x[:4] = [65504.0, 3.3895313892515355e38, -1e-40, 1.00390625]
    ours = round_bf16(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(ours, theirs)


def test_softmax_lse_matches_torch():
    s = np.random.default_rng(1).standard_normal((5, 7)) * 4
    s[0, :3] = -np.inf
    p, lse = softmax_lse(s)
    np.testing.assert_allclose(p, torch.softmax(torch.from_numpy(s), -1).numpy(), rtol=1e-12)
    np.testing.assert_allclose(lse, torch.logsumexp(torch.from_numpy(s), -1).numpy(), rtol=1e-12)


# ----------------------------------------------------------------------------- layout
def test_ordered_to_raster_known_prefix():
    # packed prefix of the 96x96 Anima grid (test_forward.py:211-219)
    assert olayout.ordered_to_raster(np.arange(16)).tolist() == list(range(8)) + list(range(96, 104))


@pytest.mark.parametrize("grid", [(1, 96, 96), (1, 16, 16), (4, 16, 16), (2, 32, 64), (3, 8, 24)])
def test_tile_order_is_the_torch_tiling(grid):
    frames, height, width = grid
    tokens = frames * height * width
    raster = torch.arange(tokens).reshape(frames, height // 8, 8, width // 8, 8)
    packed = raster.permute(0, 1, 3, 2, 4).reshape(-1)  # generic_pisa.py:17-20 per frame
    np.testing.assert_array_equal(olayout.tile_order(*grid), packed.numpy())
    assert sorted(olayout.tile_order(*grid).tolist()) == list(range(tokens))


def test_pack_unpack_round_trip():
    order = olayout.tile_order(2, 16, 32)
    x = np.random.default_rng(2).standard_normal((3, 1024, 4))
    np.testing.assert_array_equal(olayout.unpack(olayout.pack(x, order), order), x)
    assert not np.array_equal(olayout.pack(x, order), x)
    assert olayout.ordered_to_raster(np.arange(9216)).tolist() == olayout.tile_order(1, 96, 96).tolist()


def test_h3_pack_profiles():
    q, k, v = (np.arange(12, dtype=np.float32) + i for i in range(3))
    assert olayout.pack_minimax_h3_qkv(q, k, v, 9170)[3] == "kv"
    assert olayout.pack_minimax_h3_qkv(q, k, v, 12000)[3] == "qkv"


# ----------------------------------------------------------------------------- attention
@pytest.mark.parametrize("q_tokens,kv_tokens,head_dim", [(17, 31, 64), (65, 137, 128), (129, 33, 64)])
def test_dense_attention_is_sdpa(q_tokens, kv_tokens, head_dim):
    rng = np.random.default_rng(q_tokens)
    q = rng.standard_normal((2, q_tokens, head_dim))
    k = rng.standard_normal((2, kv_tokens, head_dim))
    v = rng.standard_normal((2, kv_tokens, head_dim))
    for scale in (None, 0.05):
        expected = F.scaled_dot_product_attention(*(torch.from_numpy(x) for x in (q, k, v)), scale=scale).numpy()
        np.testing.assert_allclose(oatt.dense_attention(q, k, v, scale), expected, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("tokens", [64, 65, 127, 192])
@pytest.mark.parametrize("causal", [False, True])
def test_fixed_block_equals_masked_dense_softmax(tokens, causal):
    rng = np.random.default_rng(tokens + causal)
    q, k, v = (rng.standard_normal((2, tokens, 32)) for _ in range(3))
    mask = oatt.block_diagonal_mask(tokens, 64, causal)
    scores = np.where(mask, q @ np.swapaxes(k, -1, -2) / math.sqrt(32), -np.inf)
    p, _ = softmax_lse(scores)
    np.testing.assert_allclose(oatt.fixed_block_attention(q, k, v, causal=causal), p @ v, rtol=1e-5, atol=1e-6)
    # the torch SDPA restatement with a block mask (reference.py:244-272 semantics)
    expected = F.scaled_dot_product_attention(*(torch.from_numpy(x) for x in (q, k, v)),
                                              attn_mask=torch.from_numpy(mask)).numpy()
    np.testing.assert_allclose(oatt.fixed_block_attention(q, k, v, causal=causal), expected, rtol=1e-5, atol=1e-6)


def test_fixed_block_mask_pins():
    """Masked block loop (reference.py:186-195) against identities that do not restate it."""
    rng = np.random.default_rng(11)
    tokens = 150
    q, k, v = (rng.standard_normal((3, tokens, 32)) for _ in range(3))
    plain = oatt.fixed_block_attention(q, k, v)
    # all-true bool mask and zero additive mask change nothing
    np.testing.assert_array_equal(oatt.fixed_block_attention(q, k, v, mask=np.ones((tokens, tokens), bool)), plain)
    np.testing.assert_array_equal(oatt.fixed_block_attention(q, k, v, mask=np.zeros((tokens, tokens))), plain)
    # a lower-triangular bool mask is causal attention
    tril = np.tril(np.ones((tokens, tokens), bool))
    np.testing.assert_allclose(oatt.fixed_block_attention(q, k, v, mask=tril),
                               oatt.fixed_block_attention(q, k, v, causal=True), rtol=0, atol=0)
    # softmax is shift invariant per row: a per-row constant additive mask changes nothing
    shift = np.broadcast_to(rng.standard_normal((tokens, 1)) * 5, (tokens, tokens))
    np.testing.assert_allclose(oatt.fixed_block_attention(q, k, v, mask=shift), plain, rtol=1e-9, atol=1e-12)
    # -inf additive entries are the same as false bool entries
    keep = rng.random((3, tokens, tokens)) < 0.6
    np.fill_diagonal(keep[0], True)
    keep[1:] |= np.eye(tokens, dtype=bool)
    additive = np.where(keep, 0.0, -np.inf)
    np.testing.assert_array_equal(oatt.fixed_block_attention(q, k, v, mask=additive),
                                  oatt.fixed_block_attention(q, k, v, mask=keep))
    # one kept key per row returns that key's value row exactly
    one = np.zeros((tokens, tokens), bool)
    target = np.array([(i // 64) * 64 + (i * 7) % min(64, tokens - (i // 64) * 64) for i in range(tokens)])
    one[np.arange(tokens), target] = True
    np.testing.assert_array_equal(oatt.fixed_block_attention(q, k, v, mask=one), v[:, target, :].astype(np.float32))
    # a row with nothing kept is NaN (torch.softmax of an all -inf row), other rows unaffected
    hole = np.ones((tokens, tokens), bool)
    hole[5, :] = False
    out = oatt.fixed_block_attention(q, k, v, mask=hole)
    assert np.isnan(out[:, 5]).all()
    np.testing.assert_array_equal(np.delete(out, 5, axis=1), np.delete(plain, 5, axis=1))
    # torch restatement: SDPA with (block mask AND user mask)
    user = rng.random((tokens, tokens)) < 0.7
    user |= np.eye(tokens, dtype=bool)
    combined = oatt.block_diagonal_mask(tokens, 64) & user
    expected = F.scaled_dot_product_attention(*(torch.from_numpy(x) for x in (q, k, v)),
                                              attn_mask=torch.from_numpy(combined)).numpy()
    np.testing.assert_allclose(oatt.fixed_block_attention(q, k, v, mask=user), expected, rtol=1e-5, atol=1e-6)


# ----------------------------------------------------------------------------- statistics
def test_hyd_stats_textbook():
    q, k, v = (_rng_bf16((2, 200, D), s) for s in (3, 4, 5))
    st = opisa.block_stats(q, k, v, "hyd")
    lengths = [64, 64, 64, 8]
    for b, length in enumerate(lengths):
        sl = slice(64 * b, 64 * b + length)
        np.testing.assert_allclose(st["k_centroids"][:, b], k[:, sl].astype(np.float64).mean(axis=1), rtol=1e-6,
                                   atol=1e-7)
        centred = k[:, sl].astype(np.float64) - k[:, sl].astype(np.float64).mean(axis=1, keepdims=True)
        h_b = np.einsum("bti,btj->bij", centred, v[:, sl].astype(np.float64))
        np.testing.assert_allclose(st["h_blocks"][:, b], h_b, rtol=1e-5, atol=1e-4)
        np.testing.assert_allclose(st["h_norm"][:, b], np.linalg.norm(h_b, axis=(-2, -1)), rtol=1e-5)
    np.testing.assert_allclose(st["h_sum"], st["h_blocks"].sum(axis=1), rtol=1e-5, atol=1e-3)
    # q_bar / v_bar are the bf16 roundings of the means
    np.testing.assert_array_equal(st["q_centroids"], round_bf16(st["q_centroids_f32"]))


def test_constant_keys_per_block_give_zero_covariance():
    keys = np.repeat(_rng_bf16((1, 3, D), 7), 64, axis=1)
    st = opisa.block_stats(_rng_bf16((1, 192, D), 8), keys, _rng_bf16((1, 192, D), 9), "hyd")
    assert np.count_nonzero(st["h_sum"]) == 0
    assert np.count_nonzero(st["h_norm"]) == 0


def test_means_mode_keeps_bfloat16_extrema_finite():
    big = np.full((1, 65, D), float(torch.finfo(torch.bfloat16).max), dtype=np.float32)
    st = opisa.block_stats(big, big, big, "means")
    for key in ("q_centroids", "k_centroids", "v_means"):
        assert np.isfinite(st[key]).all() and (st[key] > 0).all()


def test_generic_stats_round_centred_keys_to_dtype():
    q, k, v = (_rng_bf16((1, 128, D), s, 3.0) for s in (10, 11, 12))
    hyd = opisa.block_stats(q, k, v, "hyd")
    gen = opisa.block_stats(q, k, v, "generic")
    assert not np.array_equal(hyd["h_sum"], gen["h_sum"])  # the rounding point matters
    np.testing.assert_allclose(gen["h_sum"], hyd["h_sum"], rtol=5e-2, atol=0.5)


# ----------------------------------------------------------------------------- selection
def test_topk_matches_brute_force_with_ties_nan_and_sink():
    rng = np.random.default_rng(13)
    scores = rng.integers(-3, 4, size=(4, 9, 37)).astype(np.float32)  # many exact ties
    scores[0, 0, 5] = np.nan
    scores[1, 2, 7] = -0.0
    for k in (1, 5, 37):
        got = opisa.topk_ascending(scores, k)
        for b in range(4):
            for i in range(9):
                row = scores[b, i]
                key = [(np.inf if np.isnan(x) else (0.0 if x == 0 else float(x)), -j) for j, x in enumerate(row)]
                brute = sorted(sorted(range(37), key=lambda j: key[j], reverse=True)[:k])
                assert got[b, i].tolist() == brute
    r = opisa.route_scores(rng.standard_normal((1, 10, D)), rng.standard_normal((1, 10, D)), 0.1, sink_block=-1)
    assert (opisa.topk_ascending(r, 1) == 9).all()


def test_route_scores_hyd_bias_and_rounding():
    rng = np.random.default_rng(14)
    qc, kc = rng.standard_normal((1, 6, D)), rng.standard_normal((1, 6, D))
    hn = rng.random((1, 6)) + 0.1
    r = opisa.route_scores(qc, kc, 0.125, hn)
    expected = (round_bf16(qc).astype(np.float64) @ round_bf16(kc).astype(np.float64).transpose(0, 2, 1)) * 0.125
    expected += np.log(hn + 1e-5)[:, None, :]
    np.testing.assert_allclose(r, expected, rtol=1e-5, atol=1e-5)


# ----------------------------------------------------------------------------- PISA forward known answers
def test_hyd_all_blocks_is_dense():
    q, k, v = (_rng_bf16((2, 130, D), s) for s in (15, 16, 17))
    np.testing.assert_allclose(opisa.hyd_forward(q, k, v, 3), oatt.dense_attention(q, k, v, out_dtype="bf16"))


def test_hyd_constant_values_are_returned_exactly():
    q, k = _rng_bf16((1, 128, D), 18), _rng_bf16((1, 128, D), 19)
    v = np.full((1, 128, D), 2000.0, dtype=np.float32)
    np.testing.assert_array_equal(opisa.hyd_forward(q, k, v, 1), v)


@pytest.mark.parametrize("forward", [opisa.hyd_forward, opisa.generic_forward, opisa.reference_forward])
def test_constant_keys_per_block_make_the_tail_exact(forward):
    # tests/test_pisa_attention.py:99-109: with K constant in every block the centroid tail is exact
    # and the covariance vanishes, so any budget equals dense attention.
    q = _rng_bf16((2, 192, D), 20)
    k = np.repeat(_rng_bf16((2, 3, D), 21), 64, axis=1)
    v = _rng_bf16((2, 192, D), 22)
    dense = oatt.dense_attention(q, k, v)
    for exact in (0, 1):
        np.testing.assert_allclose(forward(q, k, v, exact), dense, atol=2e-2, rtol=2e-2)


def test_merge_form_equals_concat_softmax_form():
    q, k, v = (_rng_bf16((2, 200, D), s) for s in (23, 24, 25))
    for exact, sink in ((1, None), (2, 0), (1, -1)):
        merged = opisa.hyd_forward(q, k, v, exact, sink_block=sink)
        concat = opisa.hyd_forward_concat(q, k, v, exact, sink_block=sink)
        np.testing.assert_allclose(merged, concat, atol=1e-2, rtol=1e-2)


def test_reference_first_order_matches_closed_form():
    # tests/test_pisa_attention.py:124-146 (exact_blocks=0, two blocks)
    rng = np.random.default_rng(1234)
    q = rng.standard_normal((2, 128, D)).astype(np.float16).astype(np.float32)
    k = rng.standard_normal((2, 128, D)).astype(np.float16).astype(np.float32)
    v = (0.5 * k + np.roll(k, 1, axis=-1)).astype(np.float16).astype(np.float32)
    out = opisa.reference_forward(q, k, v, 0, dtype="f16")
    s = D ** -0.5
    kb, vb = k.reshape(2, 2, 64, D).astype(np.float64), v.reshape(2, 2, 64, D).astype(np.float64)
    k_means, v_sums = kb.mean(axis=2), vb.sum(axis=2)
    h_sum = sum(np.einsum("bti,btj->bij", kb[:, b] - k_means[:, b, None], vb[:, b]) for b in range(2))
    alpha = np.exp(np.einsum("btd,bnd->btn", q, k_means) * s)
    denominator = alpha.sum(axis=-1) * 64
    zeroth = np.einsum("btn,bnd->btd", alpha, v_sums)
    correction = np.einsum("btd,bde->bte", q, h_sum) * (s / 128) * denominator[..., None]
    expected = (zeroth + correction) / denominator[..., None]
    np.testing.assert_allclose(out, expected, atol=2e-3, rtol=2e-3)
    assert np.abs(correction).mean() > 0.01


def test_reference_budget_one_is_dense_and_resolution_rules():
    q, k, v = (_rng_bf16((2, 128, D), s) for s in (26, 27, 28))
    np.testing.assert_allclose(opisa.reference_forward(q, k, v, 2), oatt.dense_attention(q, k, v, out_dtype="bf16"),
                               atol=1e-2, rtol=1e-2)
    assert opisa.resolve_exact_blocks(144, exact_budget=0.15625) == 23
    assert opisa.resolve_exact_blocks(512, exact_budget=0.15625) == 80
    assert opisa.resolve_exact_blocks(2) == 1
    assert opisa.resolve_exact_blocks(10, exact_blocks=0, sink_block=0) == 1
    with pytest.raises(ValueError):
        opisa.resolve_exact_blocks(10, exact_budget=0.5, sparsity=0.5)


def test_a_dropped_correction_is_detected():
    # planted mistake on the CPU: the first-order term is not negligible on correlated data
    q, k, v = (_rng_bf16((1, 256, D), s) for s in (29, 30, 31))
    v = round_bf16(0.5 * k + np.roll(k, 3, axis=-1))
    with_term = opisa.generic_forward(q, k, v, 1, first_order=True)
    without = opisa.generic_forward(q, k, v, 1, first_order=False)
    assert np.abs(with_term - without).max() > 5e-2


# ----------------------------------------------------------------------------- fp32 torch CPU baseline
@pytest.mark.parametrize("forward", ["hyd", "generic", "generic_hyd"])
def test_torch_cpu_baseline_matches_the_oracle(forward):
    """oracle.torch_cpu (the fp32 torch port timed as bench.py's cpu_baseline) against the float64
    numpy oracle: same outputs within the bf16 tolerance on a short last block."""
    from oracle import torch_cpu

    rng = np.random.default_rng(11)
    q, k, v = (round_bf16(rng.standard_normal((2, 1000, D)) * 0.7) for _ in range(3))
    tq, tk, tv = (torch.from_numpy(x) for x in (q, k, v))
    if forward == "hyd":
        got = torch_cpu.hyd_forward(tq, tk, tv, 4).numpy()
        expected = opisa.hyd_forward(q, k, v, 4)
    else:
        stats = "hyd" if forward == "generic_hyd" else "generic"
        got = torch_cpu.generic_forward(tq, tk, tv, 4, stats=stats).numpy()
        expected = opisa.generic_forward(q, k, v, 4, stats=stats)
    np.testing.assert_allclose(got, expected, atol=5e-2, rtol=5e-2)
    assert np.mean(np.abs(got - expected)) < 2e-3
