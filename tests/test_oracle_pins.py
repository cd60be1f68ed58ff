"""Pins of the oracle's routing and statistics rounding points (CPU only).

Each test builds inputs whose expected selection or statistic is fixed by
construction or by exact rational arithmetic (fractions.Fraction with an
explicit fp32 rounding at each step), not by the oracle's own formula, and is
chosen so that the plausible misreadings of the reference fail:

* the HYD bias + ln(||H_b|| + 1e-5) (native/rdna35_pisa_ck/rdna35_pisa_ck/__init__.py:258-264)
  missing or with the wrong sign;
* the routing product transposed or not the q_bar . k_bar of the reference;
* the bf16 rounding of both centroids before the fp32 product (__init__.py:255-259)
  moved or dropped, and the generic path rounding where it does not
  (generic_pisa.py:172-173);
* the Triton statistics' dtype rounding of the centred keys
  (pisa_kernel.py:80-81) against fp32 centring (pisa_kernels.cu:222-226);
* the pre-scaled running mean of block_stats_kernel (pisa_kernels.cu:148-158)
  against sum-then-scale and against separately rounded products;
* the fixed-block Triton path's rounding of the normalised probabilities to
  the input dtype (triton_kernel.py:92-96) against rounding before normalising
  and against no rounding.
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import layout as olayout
from oracle import pisa as opisa
from oracle.numerics import round_bf16

D = 128
N = 8
T = N * 64


def _f32(x) -> np.float32:
    return np.float32(float(x))


def _blocks(rows_of_block):
    """[1, T, D] tensor whose block b has the 64 rows rows_of_block(b) ([64, D])."""
    return np.concatenate([rows_of_block(b) for b in range(N)], axis=0)[None].astype(np.float32)


def _bf16(x) -> float:
    return float(round_bf16(np.float32(x))[0])


def _constant_rows(vec):
    return np.repeat(np.asarray(vec, dtype=np.float32)[None], 64, axis=0)


def _unit(dim, value=1.0):
    e = np.zeros(D, dtype=np.float32)
    e[dim] = value
    return e


# ----------------------------------------------------------------------------- HYD bias
def test_orthogonal_centroids_select_the_largest_covariance_norms():
    """q_bar . k_bar = 0 everywhere: the HYD score is ln(||H_b|| + 1e-5) alone, so the
    selection is the k blocks with the largest textbook ||H_b||_F."""
    amp = np.array([1, 8, 2, 7, 3, 6, 4, 5], dtype=np.float32) / 8.0
    sign = np.where(np.arange(64) % 2 == 0, 1.0, -1.0).astype(np.float32)

    def k_rows(b):  # +-amp_b on dim 64: k_bar = 0, centred keys = the rows
        rows = np.zeros((64, D), dtype=np.float32)
        rows[:, 64] = sign * amp[b]
        return rows

    def v_rows(b):  # +-1 on dim 1 with the same sign: H_b = 64 amp_b e_64 (x) e_1
        rows = np.zeros((64, D), dtype=np.float32)
        rows[:, 1] = sign
        return rows

    q = _blocks(lambda b: _constant_rows(_unit(0)))
    k = _blocks(k_rows)
    v = _blocks(v_rows)
    textbook = np.array([np.linalg.norm(np.outer(k_rows(b)[:, 64], v_rows(b)[:, 1])) for b in range(N)])
    expected = np.sort(np.argsort(-textbook, kind="stable")[:3])
    assert expected.tolist() == [1, 3, 5]
    _, scores, idx = opisa.hyd_forward(q, k, v, 3, return_selection=True)
    assert (idx == expected[None, None]).all(), idx[0, 0]
    # a dropped bias would tie every block (selection [0, 1, 2]); a negated one picks [0, 2, 4]
    st = opisa.block_stats(q, k, v, "hyd")
    np.testing.assert_allclose(st["h_norm"][0], textbook, rtol=1e-6)


def test_equal_covariance_norms_select_the_largest_centroid_products():
    """Constant keys per block give H_b = 0 for every block (equal bias ln 1e-5): the
    selection of query block i is the top q_bar_i . k_bar_j, here w[i][j] = (3i + 5j) % 8 + 1
    on one-hot key centroids; the transpose w[j][i] selects differently."""
    w = (3 * np.arange(N)[:, None] + 5 * np.arange(N)[None, :]) % 8 + 1
    q = _blocks(lambda i: _constant_rows(np.concatenate([w[i].astype(np.float32), np.zeros(D - N, np.float32)])))
    k = _blocks(lambda j: _constant_rows(_unit(j)))
    v = np.random.default_rng(0).standard_normal((1, T, D)).astype(np.float32)
    v = round_bf16(v)
    expected = np.sort(np.argsort(-w, axis=1, kind="stable")[:, :3], axis=1)
    transposed = np.sort(np.argsort(-w.T, axis=1, kind="stable")[:, :3], axis=1)
    assert not np.array_equal(expected, transposed)
    _, _, idx = opisa.hyd_forward(q, k, v, 3, return_selection=True)
    np.testing.assert_array_equal(idx[0], expected)
    _, _, idx_g = opisa.generic_forward(q, k, v, 3, return_selection=True)
    np.testing.assert_array_equal(idx_g[0], expected)


# ----------------------------------------------------------------------------- rounding point
def test_hyd_routing_rounds_both_centroids_to_bf16_before_the_product():
    """Block 0's key mean 1 + (29/64) 2^-7 rounds to 1.0 in bf16; block 1's mean [1, x] is
    bf16 exact with 0 < x < (29/64) 2^-7.  Against q_bar = e0 + e1 the fp32 product prefers
    block 0, the bf16 product block 1: HYD (rounded) selects 1, generic (fp32) selects 0."""
    hi = 1.0 + 2.0 ** -7
    x = _bf16(0.00235)
    assert 0 < x < (29 / 64) * 2.0 ** -7

    def k_rows(b):
        rows = np.zeros((64, D), dtype=np.float32)
        if b == 0:
            rows[:, 0] = np.where(np.arange(64) < 29, hi, 1.0)
        elif b == 1:
            rows[:, 0] = 1.0
            rows[:, 1] = x
        else:
            rows[:, 0] = -1.0
        return rows

    q = _blocks(lambda b: _constant_rows(_unit(0) + _unit(1)))
    k = _blocks(k_rows)
    v = np.zeros((1, T, D), dtype=np.float32)  # H_b = 0: equal bias for every block
    mean0 = Fraction(29, 64) * Fraction(hi) + Fraction(35, 64)
    assert _bf16(float(mean0)) == 1.0 and float(mean0) - 1.0 > x
    _, _, idx = opisa.hyd_forward(q, k, v, 1, return_selection=True)
    assert (idx[0, :, 0] == 1).all()
    _, _, idx_g = opisa.generic_forward(q, k, v, 1, return_selection=True)
    assert (idx_g[0, :, 0] == 0).all()
    # generic routing on HYD statistics rounds q_bar (bf16 mean) but keeps k_bar fp32
    _, _, idx_gh = opisa.generic_forward(q, k, v, 1, return_selection=True, stats="hyd")
    assert (idx_gh[0, :, 0] == 0).all()


def test_generic_on_hyd_statistics_rounds_the_query_centroid():
    """The HYD statistics return q_bar in the input dtype and generic routing multiplies it,
    as fp32, with the fp32 k_bar (generic_pisa.py:120-126,172-173).  q_bar = [1 + d, 1] with
    d = (29/64) 2^-7 (bf16: [1, 1]); k_bar_0 = [1, 0], k_bar_1 = [1/2, 1/2 + 2^-10] (a mean of
    bf16 rows, kept fp32).  Rounded q_bar prefers block 1 (1.00098 > 1), fp32 q_bar block 0
    (1.00354 > 1.00275)."""
    hi = 1.0 + 2.0 ** -7

    def q_rows(b):
        rows = np.zeros((64, D), dtype=np.float32)
        rows[:, 0] = np.where(np.arange(64) < 29, hi, 1.0)
        rows[:, 1] = 1.0
        return rows

    def k_rows(b):
        rows = np.zeros((64, D), dtype=np.float32)
        if b == 0:
            rows[:, 0] = 1.0
        elif b == 1:
            rows[:, 0] = 0.5
            rows[:, 1] = np.where(np.arange(64) < 16, 0.5 + 2.0 ** -8, 0.5)
        else:
            rows[:, 0] = -1.0
        return rows

    q = _blocks(q_rows)
    k = _blocks(k_rows)
    v = np.zeros((1, T, D), dtype=np.float32)
    q0 = Fraction(29, 64) * Fraction(hi) + Fraction(35, 64)
    k11 = Fraction(1, 2) + Fraction(1, 1024)
    assert _bf16(float(q0)) == 1.0
    assert Fraction(1, 2) + k11 > 1                      # rounded q_bar: block 1 wins
    assert Fraction(1, 2) * q0 + k11 < q0                # fp32 q_bar: block 0 wins
    _, _, idx_gh = opisa.generic_forward(q, k, v, 1, return_selection=True, stats="hyd")
    assert (idx_gh[0, :, 0] == 1).all()
    _, _, idx_g = opisa.generic_forward(q, k, v, 1, return_selection=True, stats="generic")
    assert (idx_g[0, :, 0] == 0).all()


def test_zero_covariance_norm_adds_exactly_ln_1e5():
    qc = round_bf16(np.random.default_rng(3).standard_normal((1, N, D)))
    kc = round_bf16(np.random.default_rng(4).standard_normal((1, N, D)))
    s = 1.0 / np.sqrt(D)
    with_bias = opisa.route_scores(qc, kc, s, h_norm=np.zeros((1, N), np.float32))
    without = opisa.route_scores(qc, kc, s)
    bias = np.float32(np.log(np.float64(np.float32(1e-5))))
    # fp32 add of the fp32 bias: equal to the exact sum rounded once
    expected = (without.astype(np.float64) + np.float64(bias)).astype(np.float32)
    np.testing.assert_array_equal(with_bias, expected)
    assert abs(float(bias) - np.log(1e-5)) < 1e-6


# ----------------------------------------------------------------------------- statistics
def test_generic_statistics_round_the_centred_keys_hyd_keeps_them_fp32():
    """One 3-token block, dim 0 of k = [1, 1 + 2^-7, 1 + 2^-7], v = e0 on the first row:
    H_sum[0][0] is the first centred key, dtype-rounded (Triton, pisa_kernel.py:80-81) or
    fp32 (HYD, pisa_kernels.cu:222-226); the keys themselves are bf16 already, so rounding
    K before centring would give the fp32 value."""
    k = np.zeros((1, 3, D), dtype=np.float32)
    k[0, :, 0] = [1.0, 1.0 + 2.0 ** -7, 1.0 + 2.0 ** -7]
    v = np.zeros((1, 3, D), dtype=np.float32)
    v[0, 0, 0] = 1.0
    q = np.zeros((1, 3, D), dtype=np.float32)
    total = _f32(Fraction(1) + 2 * Fraction(1.0 + 2.0 ** -7))  # exact in fp32
    mean_generic = _f32(Fraction(float(total)) / 3)                     # sum / len
    mean_hyd = _f32(Fraction(float(total)) * Fraction(float(_f32(Fraction(1, 3)))))  # sum * fp32(1/len)
    centred_generic = _bf16(_f32(Fraction(1) - Fraction(float(mean_generic))))
    centred_hyd = float(_f32(Fraction(1) - Fraction(float(mean_hyd))))
    assert centred_generic != float(_f32(Fraction(1) - Fraction(float(mean_generic))))
    gen = opisa.block_stats(q, k, v, "generic")
    hyd = opisa.block_stats(q, k, v, "hyd")
    assert float(gen["h_sum"][0, 0, 0]) == centred_generic
    assert float(hyd["h_sum"][0, 0, 0]) == centred_hyd
    assert float(gen["k_centroids"][0, 0, 0]) == float(mean_generic)
    assert float(hyd["k_centroids"][0, 0, 0]) == float(mean_hyd)


@pytest.mark.parametrize("values", [(1.0, 11.0, 5.0), (1.0, 1.0, 7.0)])
def test_means_mode_prescales_each_row_with_one_fma(values):
    """block_stats_kernel accumulates mean += x * (1/len) row by row (pisa_kernels.cu:148-158),
    one fp32 fma per row.  (1, 11, 5): differs from sum-then-scale; (1, 1, 7): differs from
    rounding each product before the add."""
    inv = Fraction(float(_f32(Fraction(1, 3))))
    fma = _f32(0)
    separate = _f32(0)
    for x in values:
        fma = _f32(Fraction(x) * inv + Fraction(float(fma)))
        separate = _f32(Fraction(float(separate)) + Fraction(float(_f32(Fraction(x) * inv))))
    sum_then_scale = _f32(Fraction(float(_f32(sum(values)))) * inv)
    assert fma != separate or fma != sum_then_scale
    x = np.zeros((1, 3, D), dtype=np.float32)
    x[0, :, 5] = values
    st = opisa.block_stats(x, x, x, "means")
    assert float(st["k_centroids"][0, 0, 5]) == float(fma)
    assert float(st["q_centroids_f32"][0, 0, 5]) == float(fma)


# ----------------------------------------------------------------------------- H3 pack
@pytest.mark.parametrize("tokens,profile", [(11999, "kv"), (12000, "qkv"), (4608, "kv"), (16500, "qkv")])
def test_h3_pack_copies_bit_exactly(tokens, profile):
    """minimax_h3_gfx1151_attention.py:60-74: below 12000 tokens K and V are stacked into one
    buffer (q passed through), from 12000 Q, K and V; every packed view equals its input."""
    rng = np.random.default_rng(tokens)
    q, k, v = (rng.standard_normal((2, 3, 4)).astype(np.float32) for _ in range(3))
    pq, pk, pv, got = olayout.pack_minimax_h3_qkv(q, k, v, tokens)
    assert got == profile
    for a, b in ((pq, q), (pk, k), (pv, v)):
        np.testing.assert_array_equal(a, b)
    if profile == "kv":
        assert pq is q and pk.base is pv.base and pk.base is not None
    else:
        assert pq.base is pk.base and pk.base is pv.base and pq.base is not None
    tq, tk, tv = (torch.from_numpy(x) for x in (q, k, v))
    ref = torch.stack((tq, tk, tv)) if profile == "qkv" else torch.stack((tk, tv))
    np.testing.assert_array_equal(pk, ref[-2].numpy())
    np.testing.assert_array_equal(pv, ref[-1].numpy())


def test_fixed_block_16bit_probabilities_round_after_normalising():
    """Scores [0, ln 2] in one block give the probabilities [1/3, 2/3]; the Triton kernel rounds
    the normalised probabilities to the input dtype before P @ V (triton_kernel.py:92-96).  With
    V = [1, 0] the first output is exactly bf16(1/3) = 0.333984375 (fp16(1/3) = 0.333251953125);
    rounding the unnormalised exponentials [1, 2] instead, or not rounding, gives 1/3."""
    from oracle import attention as oatt

    q = np.array([[1.0], [0.0]], dtype=np.float32)
    k = np.array([[0.0], [np.log(2.0)]], dtype=np.float32)
    v = np.array([[1.0], [0.0]], dtype=np.float32)
    bf = oatt.fixed_block_attention(q, k, v, scale=1.0, prob_dtype="bf16")
    hf = oatt.fixed_block_attention(q, k, v, scale=1.0, prob_dtype="f16")
    unrounded = oatt.fixed_block_attention(q, k, v, scale=1.0)
    k_f32_ln2 = float(np.float32(np.log(2.0)))  # the fp32 ln 2 the oracle multiplies
    third = 1.0 / (1.0 + np.exp(k_f32_ln2))     # softmax weight of key 0
    assert abs(third - 1.0 / 3.0) < 1e-7
    assert float(bf[0, 0]) == 0.333984375
    assert float(hf[0, 0]) == 0.333251953125
    assert abs(float(unrounded[0, 0]) - third) < 1e-7
