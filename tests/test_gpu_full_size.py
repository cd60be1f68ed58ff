"""GPU checks at the full BASELINE configurations.

The oracle cannot run a whole config in seconds, so each config is checked
by (a) size-independent properties at full size - bit-exact selection
against the CPU top-k of the kernel's own scores, constant values returned
exactly, per-block-constant keys reducing PISA to dense attention, strided
and packed layouts giving identical bits - and (b) oracle comparisons on a
subset of heads or query rows of the full-size problem.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import assert_close, np32, packed_to_merged, spatial_to_packed
from oracle import attention as oatt
from oracle import layout as olayout
from oracle import pisa as opisa

pytestmark = pytest.mark.gpu
D = 128


@pytest.fixture(scope="module")
def native():
    import mi355x_pisa

    return mi355x_pisa


@pytest.fixture(scope="module")
def anima():
    from mi355x_pisa.synthetic import anima_qkv

    return anima_qkv(batch=2, heads=16, seed=0, device="cuda")


def test_c4_selection_bit_exact_and_oracle_heads(native, anima):
    q, k, v = anima
    out, scores, idx = native.forward_with_routing(q, k, v, 23, D ** -0.5, token_grid=(1, 96, 96))
    assert torch.isfinite(out).all()
    np.testing.assert_array_equal(idx.cpu().numpy(), opisa.topk_ascending(np32(scores), 23))
    # the spatial entry point gives the same bits
    spatial = native.forward_spatial_bhtd(q, k, v, exact_blocks=23)
    assert torch.equal(spatial.view(2, 9216, 16, D).permute(0, 2, 1, 3), out)
    # flat heads 0, 9, 18 and 31: with 4 consecutive heads per XCD in the attention kernel's schedule
    # (4608 query blocks over 8 XCDs), these run on XCDs 0, 2, 4 and 7
    heads = [(0, 0), (0, 9), (1, 2), (1, 15)]
    for b, h in heads:
        print(f"C4 oracle head (b={b}, h={h})", flush=True)
        packed = [spatial_to_packed(t[b:b + 1, h:h + 1], 1, 96, 96) for t in (q, k, v)]
        expected, exp_scores, _ = opisa.hyd_forward(*packed, 23, return_selection=True)
        assert_close(np32(scores[b * 16 + h]), exp_scores[0], 1e-4, 1e-4, "C4 routing scores")
        merged = packed_to_merged(expected, 1, 1, 1, 96, 96)
        assert_close(np32(out[b, h]), merged[0], 5e-2, 5e-2, f"C4 head {(b, h)}")


def _selection_agreement(kernel_idx: np.ndarray, oracle_scores: np.ndarray, k: int, tol: float):
    """Rows where the kernel's selection equals the oracle's, and whether every other row is a near-tie:
    the oracle's k-th and (k+1)-th largest scores within `tol` (the routing-score tolerance), so that
    a last-bit difference of the fp32 sums can swap the blocks at the boundary."""
    expected = opisa.topk_ascending(oracle_scores, k)
    equal = np.all(kernel_idx == expected, axis=-1)
    ordered = -np.sort(-oracle_scores, axis=-1)
    gap = ordered[..., k - 1] - ordered[..., k]
    near_tie = gap <= tol * np.maximum(1.0, np.abs(ordered[..., k - 1]))
    return equal, near_tie


def test_c4_selection_agrees_with_the_oracle_on_every_head(native, anima):
    """The kernel's selection against the oracle's own (oracle statistics -> oracle scores -> top-k)
    for all 32 heads of C4: every row that differs must be a near-tie of the oracle's scores."""
    q, k, v = anima
    _, _, idx = native.forward_with_routing(q, k, v, 23, D ** -0.5, token_grid=(1, 96, 96))
    packed = [spatial_to_packed(t, 1, 96, 96) for t in (q, k, v)]
    st = opisa.block_stats(*packed, "hyd", "bf16")
    scores = opisa.route_scores(st["q_centroids_f32"], st["k_centroids"], np.float32(D ** -0.5), st["h_norm"])
    equal, near_tie = _selection_agreement(idx.cpu().numpy(), scores, 23, 1e-4)
    print(f"C4 selection: {equal.sum()} / {equal.size} query blocks equal the oracle's "
          f"({100.0 * equal.mean():.3f} %); differing rows that are near-ties: {near_tie[~equal].sum()}")
    assert np.all(equal | near_tie)
    assert equal.mean() >= 0.99


def test_c4_routing_row_tiling_does_not_change_bits(native, anima):
    """C4 (32 heads) routes in workgroups of 8 query blocks, the same heads twice (64 heads, enough
    workgroups to fill every CU twice) in workgroups of 16: each score is the same MFMA sum either way,
    so scores and selections must be bit-identical.  The outputs agree to rounding only: the statistics
    grid also depends on the head count (64 heads: 8 chunks of 18 blocks per head instead of 16 of 9),
    and H_sum sums its chunk partials in a different grouping."""
    q, k, v = anima
    out, scores, idx = native.forward_with_routing(q, k, v, 23, D ** -0.5, token_grid=(1, 96, 96))
    q2, k2, v2 = (torch.cat([t, t]) for t in (q, k, v))
    out2, scores2, idx2 = native.forward_with_routing(q2, k2, v2, 23, D ** -0.5, token_grid=(1, 96, 96))
    for half in (slice(0, 32), slice(32, 64)):
        assert torch.equal(scores2[half], scores)
        assert torch.equal(idx2[half], idx)
    for part in (out2[:2], out2[2:]):
        torch.testing.assert_close(part.float(), out.float(), atol=1e-2, rtol=1e-2)


def test_c4_constant_values_are_exact(native, anima):
    q, k, _ = anima
    v = torch.full_like(q, 0.3125)  # exactly representable; any convex combination returns it
    out = native.forward_spatial_bhtd(q, k, v, exact_blocks=23)
    assert torch.equal(out, torch.full_like(out, 0.3125))


def test_c4_blockwise_constant_keys_reduce_to_dense(native, anima):
    q, k, v = anima
    order = torch.from_numpy(olayout.tile_order(1, 96, 96)).cuda()
    blocks = k[:, :, order].reshape(2, 16, 144, 64, D)[:, :, :, :1].expand(2, 16, 144, 64, D)
    k_const = torch.empty_like(k).contiguous()
    k_const[:, :, order] = blocks.reshape(2, 16, 9216, D)
    storage = k_const.permute(0, 2, 1, 3).contiguous()
    k_view = storage.permute(0, 2, 1, 3)
    sparse = native.forward_spatial_bhtd(q, k_view, v, exact_blocks=23)
    dense = native.forward_spatial_bhtd(q, k_view, v, exact_blocks=144)
    torch.testing.assert_close(sparse.float(), dense.float(), atol=5e-2, rtol=5e-2)


def test_c2_dense_self_and_cross(native):
    from mi355x_pisa.synthetic import normal_qkv

    q, k, v = normal_qkv((2, 16, 9216, D), seed=2, scale=0.5, device="cuda")
    out = native.dense_attention(q, k, v, D ** -0.5)
    assert torch.isfinite(out).all()
    rows = slice(0, 256)
    for b, h in ((0, 0), (1, 9)):
        expected = oatt.dense_attention(np32(q[b, h, rows]), np32(k[b, h]), np32(v[b, h]))
        assert_close(np32(out[b, h, rows]), expected, 5e-2, 5e-2, f"C2 head {(b, h)}")
    # query blocks 80.. of head 3 lie in the last-round range of their XCD's
    # blocks (run as two one-tile halves): the same tolerance holds there
    split_rows = slice(80 * 64, 84 * 64)
    expected = oatt.dense_attention(np32(q[0, 3, split_rows]), np32(k[0, 3]), np32(v[0, 3]))
    assert_close(np32(out[0, 3, split_rows]), expected, 5e-2, 5e-2, "C2 split blocks")
    ones = torch.full_like(v, -1.5)
    assert torch.equal(native.dense_attention(q, k, ones, D ** -0.5), ones)
    kc, vc = (t[:, :, :512].contiguous() for t in (k, v))
    cross = native.dense_attention(q, kc, vc, D ** -0.5)
    for b, h in ((0, 3), (1, 15)):
        expected = oatt.dense_attention(np32(q[b, h, rows]), np32(kc[b, h]), np32(vc[b, h]))
        assert_close(np32(cross[b, h, rows]), expected, 5e-2, 5e-2, "C2 cross")


@pytest.mark.parametrize("tokens", [9170, 16500])
def test_c3_h3_strided_equals_packed(native, tokens):
    gen = torch.Generator().manual_seed(tokens)
    qkv = torch.randn((1, tokens, 3, 56, D), generator=gen).to(torch.bfloat16).cuda()
    q, k, v = (qkv[:, :, i].permute(0, 2, 1, 3) for i in range(3))
    v = v.clone()  # the reference benchmark clones V (nodes.py:334-337)
    strided = native.dense_attention(q, k, v, D ** -0.5, merged_output=True)
    packed = native.dense_attention(q.contiguous(), k.contiguous(), v.contiguous(), D ** -0.5, merged_output=True)
    assert torch.equal(strided, packed)
    rows = slice(tokens - 200, tokens)
    # head 6's last blocks are the last work items of XCD 0 on the persistent
    # grid (8 x 128 wave slots): whole extra blocks at T=9170 (1008 blocks per
    # XCD = 7 x 128 + 112), one-tile halves at T=16500 (1806 = 14 x 128 + 14)
    for head in (17, 6):
        expected = oatt.dense_attention(np32(q[0, head, rows]), np32(k[0, head]), np32(v[0, head]))
        got = np32(strided).reshape(tokens, 56, D)[rows, head]
        assert_close(got, expected, 5e-2, 5e-2, f"C3 head {head}")


def test_c1_fixed_block_fp32(native):
    from mi355x_pisa.synthetic import normal_qkv

    q, k, v = normal_qkv((1, 8, 4096, 64), seed=1, dtype=torch.float32, device="cuda")
    out = native.fixed_block_attention(q, k, v, 1 / 8.0)
    expected = oatt.fixed_block_attention(np32(q), np32(k), np32(v), scale=1 / 8.0)
    assert_close(np32(out), expected, 1e-5, 1e-5, "C1")


def test_c5_video_selection_and_one_head(native):
    from mi355x_pisa.synthetic import video_qkv

    grid = (16, 32, 64)
    q, k, v = video_qkv(batch=1, heads=40, grid=grid, seed=5, device="cuda")
    exact = math.ceil(0.15625 * 512)
    out, scores, idx = native.forward_with_routing(q, k, v, exact, D ** -0.5, hyd=False, token_grid=grid)
    assert torch.isfinite(out).all()
    np.testing.assert_array_equal(idx.cpu().numpy(), opisa.topk_ascending(np32(scores), exact))
    merged = native.generic_forward(q, k, v, exact, D ** -0.5, True, token_grid=grid)
    assert torch.equal(merged.permute(0, 2, 1, 3), out)
    packed = [spatial_to_packed(t[:, 21:22], *grid) for t in (q, k, v)]
    expected = packed_to_merged(opisa.generic_forward(*packed, exact, dtype="bf16"), 1, 1, *grid)
    assert_close(np32(out[0, 21]), expected[0], 5e-2, 5e-2, "C5 head 21")
    # the kernel's selection against the oracle's for all 40 heads (T = 32768 > 9216: the
    # Triton-semantics statistics, fp32 means, generic_pisa.py:128-138)
    assert native.generic_stats_mode(32768, D, torch.bfloat16) == "generic"
    all_packed = [spatial_to_packed(t, *grid) for t in (q, k, v)]
    st = opisa.block_stats(*all_packed, "generic", "bf16", covariance=False)
    oracle_scores = opisa.route_scores(st["q_centroids"], st["k_centroids"], np.float32(D ** -0.5), None, None, False)
    equal, near_tie = _selection_agreement(idx.cpu().numpy(), oracle_scores, exact, 1e-4)
    print(f"C5 selection: {equal.sum()} / {equal.size} query blocks equal the oracle's "
          f"({100.0 * equal.mean():.3f} %); differing rows that are near-ties: {near_tie[~equal].sum()}")
    assert np.all(equal | near_tie)
    assert equal.mean() >= 0.99


def test_max_size_video_pisa_matches_oracle(native):
    """T = 65536, the largest sequence the native path takes (1024 blocks): routing over 1024 candidates per row
    (16 per lane in the selection), 16 centroid chunks in the attention tail; one head against the oracle."""
    from mi355x_pisa.synthetic import video_qkv

    grid = (16, 64, 64)
    q, k, v = video_qkv(batch=1, heads=2, grid=grid, seed=11, device="cuda")
    exact = 16
    out, scores, idx = native.forward_with_routing(q, k, v, exact, D ** -0.5, hyd=False, token_grid=grid)
    assert scores.shape == (2, 1024, 1024) and idx.shape == (2, 1024, exact)
    assert torch.isfinite(out).all()
    np.testing.assert_array_equal(idx.cpu().numpy(), opisa.topk_ascending(np32(scores), exact))
    packed = [spatial_to_packed(t[:, 1:2], *grid) for t in (q, k, v)]
    expected = packed_to_merged(opisa.generic_forward(*packed, exact, dtype="bf16"), 1, 1, *grid)
    assert_close(np32(out[0, 1]), expected[0], 5e-2, 5e-2, "T=65536 head 1")


@pytest.mark.parametrize("grid", [(2, 64, 64), (1, 64, 128), (8, 32, 32)])
def test_wan_ltx_t8192_generic_routes_on_hyd_statistics(native, grid):
    """Generic PISA at T = 8192, D = 128, bf16 (the Wan/LTX regime of the reference's README.md:110-112): the
    reference routes on the native HYD statistics there (generic_pisa.py:120-126).  Selection
    against the oracle's for every head, output against the oracle on two heads."""
    from mi355x_pisa.synthetic import video_qkv

    assert native.generic_stats_mode(8192, D, torch.bfloat16) == "hyd"
    heads = 4
    q, k, v = video_qkv(batch=1, heads=heads, grid=grid, seed=sum(grid), device="cuda")
    exact = math.ceil(0.15625 * 128)
    out, scores, idx = native.forward_with_routing(q, k, v, exact, D ** -0.5, token_grid=grid, mode="generic_hyd")
    merged = native.generic_forward(q, k, v, exact, D ** -0.5, True, token_grid=grid)
    assert torch.equal(merged.permute(0, 2, 1, 3), out)
    np.testing.assert_array_equal(idx.cpu().numpy(), opisa.topk_ascending(np32(scores), exact))
    packed = [spatial_to_packed(t, *grid) for t in (q, k, v)]
    st = opisa.block_stats(*packed, "hyd", "bf16", covariance=False)
    oracle_scores = opisa.route_scores(st["q_centroids"], st["k_centroids"], np.float32(D ** -0.5), None, None, False)
    assert_close(np32(scores), oracle_scores, 1e-4, 1e-4, "T=8192 routing scores")
    equal, near_tie = _selection_agreement(idx.cpu().numpy(), oracle_scores, exact, 1e-4)
    assert np.all(equal | near_tie) and equal.mean() >= 0.99
    for head in (0, 3):
        one = [p[head:head + 1] for p in packed]
        expected = packed_to_merged(opisa.generic_forward(*one, exact, dtype="bf16", stats="hyd"), 1, 1, *grid)
        assert_close(np32(out[0, head]), expected[0], 5e-2, 5e-2, f"T=8192 head {head}")
