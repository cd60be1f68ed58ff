"""GPU parity of the native HIP ops (mi355x_pisa) against the CPU oracle.

Mirrors native/rdna35_pisa_ck/tests/test_forward.py (seeds, shapes and known
answers) and adds bit-exact selection checks and layout/epilogue checks.
Tolerances: bf16 outputs atol=rtol=5e-2 (the reference's gate), statistics
at fp32 accuracy.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import assert_close, np32, packed_to_merged, spatial_to_packed
from oracle import attention as oatt
from oracle import layout as olayout
from oracle import pisa as opisa

pytestmark = pytest.mark.gpu

BLOCK = 64
D = 128


@pytest.fixture(scope="module")
def native():
    import mi355x_pisa

    return mi355x_pisa


def _inputs(tokens, dtype=torch.bfloat16, seed=0, bh=1, scale=1.0):
    gen = torch.Generator().manual_seed(seed)
    return tuple((scale * torch.randn((bh, tokens, D), generator=gen)).to(dtype).cuda() for _ in range(3))


# ----------------------------------------------------------------------------- statistics
@pytest.mark.parametrize("tokens,seed", [(128, 61), (200, 3), (65, 7)])
def test_hyd_stats_match_oracle(native, tokens, seed):
    q, k, v = _inputs(tokens, seed=seed, bh=2)
    qc, kc, vm, hs, hn = native._C.block_stats_hyd(q, k, v)
    st = opisa.block_stats(np32(q), np32(k), np32(v), "hyd", "bf16")
    assert_close(np32(kc), st["k_centroids"], 1e-6, 1e-5, "k_centroids")
    assert_close(np32(qc), st["q_centroids"], 1e-2, 1e-2, "q_centroids")
    assert_close(np32(vm), st["v_means"], 1e-2, 1e-2, "v_means")
    scale_h = np.abs(st["h_sum"]).max()
    assert_close(np32(hs), st["h_sum"], 1e-4 * scale_h, 1e-4, "h_sum")
    assert_close(np32(hn), st["h_norm"], 1e-3, 1e-4, "h_norm")


def test_hyd_stats_native_equals_wrapper(native):
    q, k, v = _inputs(128, seed=61)
    qc, kc, vm, hs = native.block_stats_hyd(q, k, v)
    raw = native._C.block_stats_hyd(q, k, v)
    assert len(raw) == 5
    for a, b in zip(raw[:4], (qc, kc, vm, hs)):
        assert torch.equal(a, b)
    # h_norm equals the Frobenius norm of the per-block covariance (test_forward.py:191-201)
    h_blocks = torch.stack([
        (k[:, s:s + BLOCK].float() - kc[:, i, None]).transpose(1, 2).cpu() @ v[:, s:s + BLOCK].float().cpu()
        for i, s in enumerate(range(0, 128, BLOCK))
    ], dim=1)
    torch.testing.assert_close(raw[4].cpu(), torch.linalg.matrix_norm(h_blocks, dim=(-2, -1)), atol=1e-2, rtol=1e-3)


def test_block_stats_average_bfloat16_extrema_without_overflow(native):
    maximum = torch.finfo(torch.bfloat16).max
    q = torch.full((1, 65, D), maximum, device="cuda", dtype=torch.bfloat16)
    for tensor in native._C.block_stats(q, q, q):
        assert torch.isfinite(tensor).all()
        assert (tensor > 0).all()


def test_constant_keys_per_block_have_zero_covariance(native):
    gen = torch.Generator().manual_seed(5)
    keys = torch.randn((1, 3, 1, D), generator=gen).expand(1, 3, BLOCK, D).reshape(1, 3 * BLOCK, D)
    k = keys.to(torch.bfloat16).cuda()
    q, _, v = _inputs(3 * BLOCK, seed=6)
    _, _, _, hs, hn = native._C.block_stats_hyd(q, k, v)
    assert torch.count_nonzero(hs) == 0
    assert torch.count_nonzero(hn) == 0


def test_generic_stats_match_oracle(native):
    q, k, v = _inputs(256, dtype=torch.float16, seed=11, bh=2)
    qc, kc, vm, hs, hn = native._block_stats(q, k, v, 2, torch.float32)
    st = opisa.block_stats(np32(q), np32(k), np32(v), "generic", "f16")
    assert_close(np32(qc), st["q_centroids"], 1e-6, 1e-5, "q_centroids")
    assert_close(np32(kc), st["k_centroids"], 1e-6, 1e-5, "k_centroids")
    assert_close(np32(vm), st["v_means"], 1e-6, 1e-5, "v_means")
    scale_h = np.abs(st["h_sum"]).max()
    assert_close(np32(hs), st["h_sum"], 1e-4 * scale_h, 1e-4, "h_sum")


# ----------------------------------------------------------------------------- routing
def test_route_topk_is_bit_exact_on_its_scores(native):
    gen = torch.Generator().manual_seed(1234)
    bh, n = 3, 144
    qc = torch.randn((bh, n, D), generator=gen)
    kc = torch.randn((bh, n, D), generator=gen)
    kc[:, 10] = kc[:, 20]  # duplicated key centroids: exact ties
    kc[:, 77] = kc[:, 20]
    hn = torch.rand((bh, n), generator=gen) + 0.5
    hn[:, 10] = hn[:, 20]
    hn[:, 77] = hn[:, 20]
    for sink in (None, 0, -1):
        scores, idx = native.route_topk(qc.cuda(), kc.cuda(), hn.cuda(), 23, 1 / math.sqrt(D), sink)
        cpu_idx = opisa.topk_ascending(np32(scores), 23)
        np.testing.assert_array_equal(idx.cpu().numpy(), cpu_idx)
        expected = opisa.route_scores(qc.numpy(), kc.numpy(), 1 / math.sqrt(D), hn.numpy(), sink, True)
        assert_close(np32(scores), expected, 1e-5, 1e-5, "route scores")
        if sink is not None:
            assert (idx.cpu().numpy() == (sink % n)).any(axis=-1).all()


@pytest.mark.parametrize("n,head_dim,k,round_bf16", [(37, 64, 5, True), (64, 128, 64, False), (65, 32, 1, True),
                                                     (300, 100, 40, True), (700, 256, 350, False),
                                                     (1024, 128, 144, True)])
def test_route_topk_sizes_bit_exact(native, n, head_dim, k, round_bf16):
    gen = torch.Generator().manual_seed(n + head_dim)
    bh = 2
    qc = torch.randn((bh, n, head_dim), generator=gen)
    kc = torch.randn((bh, n, head_dim), generator=gen)
    kc[:, n // 2] = kc[:, n // 3]  # exact ties
    hn = torch.rand((bh, n), generator=gen) + 0.1 if round_bf16 else None
    scores, idx = native.route_topk(qc.cuda(), kc.cuda(), None if hn is None else hn.cuda(), k,
                                    1 / math.sqrt(head_dim), -1, round_bf16=round_bf16)
    np.testing.assert_array_equal(idx.cpu().numpy(), opisa.topk_ascending(np32(scores), k))
    expected = opisa.route_scores(qc.numpy(), kc.numpy(), 1 / math.sqrt(head_dim),
                                  None if hn is None else hn.numpy(), -1, round_bf16)
    assert_close(np32(scores), expected, 1e-5, 1e-5, "route scores")


def test_route_topk_nonfinite_scores_and_empty_selection(native):
    gen = torch.Generator().manual_seed(7)
    bh, n = 1, 90
    qc = torch.randn((bh, n, D), generator=gen)
    kc = torch.randn((bh, n, D), generator=gen)
    kc[0, 3] = float("nan")     # NaN scores rank above +inf
    kc[0, 8] = float("inf")
    kc[0, 9] = -float("inf")
    scores, idx = native.route_topk(qc.cuda(), kc.cuda(), None, 12, 0.1, None, round_bf16=False)
    np.testing.assert_array_equal(idx.cpu().numpy(), opisa.topk_ascending(np32(scores), 12))
    assert (idx.cpu().numpy() == 3).any(axis=-1).all()  # the NaN column is in every row's selection
    _, none = native.route_topk(qc.cuda(), kc.cuda(), None, 0, 0.1, None, round_bf16=False)
    assert none.shape == (bh, n, 0)


def test_route_topk_ties_go_to_lowest_index(native):
    bh, n = 1, 200
    qc = torch.zeros((bh, n, D))
    kc = torch.zeros((bh, n, D))
    scores, idx = native.route_topk(qc.cuda(), kc.cuda(), None, 7, 0.1, None, round_bf16=False)
    assert torch.count_nonzero(scores) == 0
    np.testing.assert_array_equal(idx.cpu().numpy(), np.broadcast_to(np.arange(7), (1, n, 7)))


# ----------------------------------------------------------------------------- PISA forward
@pytest.mark.parametrize("tokens,seed,exact", [(128, 19, 1), (200, 5, 2), (1024, 9, 4)])
def test_partial_matches_oracle(native, tokens, seed, exact):
    q, k, v = _inputs(tokens, seed=seed)
    actual = native.forward(q, k, v, exact_blocks=exact)
    expected = opisa.hyd_forward(np32(q), np32(k), np32(v), exact)
    assert_close(np32(actual), expected, 5e-2, 5e-2, "forward")
    # the reference's own restatement (test_forward.py:34-104)
    concat = opisa.hyd_forward_concat(np32(q), np32(k), np32(v), exact)
    assert_close(np32(actual), concat, 5e-2, 5e-2, "forward vs concat")


def test_partial_tail_matches_oracle_with_sink(native):
    q, k, v = _inputs(65, seed=23)
    for sink in (0, -1):
        actual = native.forward(q, k, v, exact_blocks=1, sink_block=sink)
        expected = opisa.hyd_forward(np32(q), np32(k), np32(v), 1, sink_block=sink)
        assert_close(np32(actual), expected, 5e-2, 5e-2, f"sink={sink}")


def test_first_order_correction_centers_before_gemm(native):
    gen = torch.Generator().manual_seed(37)
    tokens = 256
    q = (torch.randn((1, tokens, D), generator=gen) * 16.0).to(torch.bfloat16)
    offsets = torch.randn((1, tokens // BLOCK, 1, D), generator=gen) * 64.0
    noise = torch.randn((1, tokens // BLOCK, BLOCK, D), generator=gen) * 0.125
    k = (offsets + noise).flatten(1, 2).to(torch.bfloat16)
    v = torch.randn((1, tokens, D), generator=gen).to(torch.bfloat16)
    actual = native.forward(q.cuda(), k.cuda(), v.cuda(), exact_blocks=0)
    expected = opisa.hyd_forward(np32(q), np32(k), np32(v), 0)
    assert_close(np32(actual), expected, 6e-2, 5e-2, "exact_blocks=0")


def test_exact_matches_dense(native):
    q, k, v = _inputs(128, seed=17)
    actual = native.forward(q, k, v, exact_blocks=2, scale=0.125)
    expected = oatt.dense_attention(np32(q), np32(k), np32(v), 0.125)
    assert_close(np32(actual), expected, 2e-2, 2e-2, "dense")


def test_large_finite_values_and_constant_v_are_exact(native):
    q = torch.zeros((1, 128, D), device="cuda", dtype=torch.bfloat16)
    k = torch.zeros_like(q)
    v = torch.full_like(q, 2000.0)
    out = native.forward(q, k, v, exact_blocks=1)
    assert torch.isfinite(out).all()
    assert torch.equal(out, v)


def test_invalid_scale_and_shape(native):
    q, k, v = _inputs(128, seed=29)
    for scale in (0.0, -1.0, math.inf, math.nan, 1e100):
        with pytest.raises(ValueError, match="scale"):
            native.forward(q, k, v, exact_blocks=1, scale=scale)
    with pytest.raises(ValueError, match=r"matching \[BH,T,D\]"):
        native.forward(q[0], k[0], v[0], exact_blocks=1)
    with pytest.raises(ValueError, match=r"matching \[BH,T,D\]"):
        native.forward(q, k[:, :-1].contiguous(), v, exact_blocks=1)
    with pytest.raises(ValueError, match="D=128"):
        native.forward(q[..., :64].contiguous(), k[..., :64].contiguous(), v[..., :64].contiguous(), exact_blocks=1)
    with pytest.raises(ValueError, match="contiguous"):
        native.forward(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), exact_blocks=1)
    fp16 = q.to(torch.float16)
    with pytest.raises(ValueError, match="bfloat16"):
        native.forward(fp16, fp16, fp16, exact_blocks=1)


def test_selection_is_bit_exact_against_cpu_topk(native):
    gen = torch.Generator().manual_seed(71)
    q4, k4, v4 = (torch.randn((1, 2, 640, D), generator=gen).to(torch.bfloat16).cuda() for _ in range(3))
    out, scores, idx = native.forward_with_routing(q4, k4, v4, 3, 1 / math.sqrt(D))
    np.testing.assert_array_equal(idx.cpu().numpy(), opisa.topk_ascending(np32(scores), 3))
    qf, kf, vf = (np32(t).reshape(2, 640, D) for t in (q4, k4, v4))
    expected, exp_scores, exp_idx = opisa.hyd_forward(qf, kf, vf, 3, return_selection=True)
    assert_close(np32(scores), exp_scores, 1e-4, 1e-4, "route scores vs oracle")
    assert_close(np32(out).reshape(2, 640, D), expected, 5e-2, 5e-2, "forward_with_routing")


def test_outer_torch_compile_fullgraph(native):
    q, k, v = _inputs(64, seed=31)

    def target(q, k, v):
        return native.forward(q, k, v, exact_blocks=0)

    expected = target(q, k, v)
    actual = torch.compile(target, backend="inductor", fullgraph=True)(q, k, v)
    torch.testing.assert_close(actual, expected, atol=1e-3, rtol=1e-3)


def test_current_stream_is_used(native):
    q, k, v = _inputs(256, seed=41)
    expected = native.forward(q, k, v, exact_blocks=1)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        out = native.forward(q, k, v, exact_blocks=1)
    torch.cuda.current_stream().wait_stream(stream)
    assert torch.equal(out, expected)


# ----------------------------------------------------------------------------- spatial (Anima)
def _spatial_inputs(seed, heads=2):
    gen = torch.Generator().manual_seed(seed)
    bthd = [torch.randn((1, 9216, heads, D), generator=gen).to(torch.bfloat16).cuda() for _ in range(3)]
    return tuple(t.permute(0, 2, 1, 3) for t in bthd)


def test_spatial_sparse_matches_oracle(native):
    from mi355x_pisa.synthetic import anima_qkv

    q, k, v = anima_qkv(batch=1, heads=2, seed=3, device="cuda")
    out = native.forward_spatial_bhtd(q, k, v, exact_blocks=23)
    assert out.shape == (1, 9216, 2 * D)
    packed = [spatial_to_packed(t, 1, 96, 96) for t in (q, k, v)]
    expected = packed_to_merged(opisa.hyd_forward(*packed, 23), 1, 2, 1, 96, 96)
    assert_close(np32(out), expected, 5e-2, 5e-2, "spatial 23/144")


def test_spatial_exact_matches_dense(native):
    q, k, v = _spatial_inputs(43)
    actual = native.forward_spatial_bhtd(q, k, v, exact_blocks=144)
    expected = F.scaled_dot_product_attention(q.float().cpu(), k.float().cpu(), v.float().cpu())
    expected = expected.permute(0, 2, 1, 3).reshape(1, 9216, 2 * D)
    torch.testing.assert_close(actual.float().cpu(), expected, atol=2e-2, rtol=2e-2)
    with pytest.raises(ValueError, match="views of contiguous"):
        native.forward_spatial_bhtd(q.contiguous(), k.contiguous(), v.contiguous(), exact_blocks=1)
    for exact in (0, 22, 24, 143):
        with pytest.raises(ValueError, match="supports exact_blocks=23"):
            native.forward_spatial_bhtd(q, k, v, exact_blocks=exact)


def test_spatial_sparse_is_finite_on_side_stream(native):
    stream = torch.cuda.Stream()
    for seed in (41, 47):
        q, k, v = _spatial_inputs(seed)
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            out = native.forward_spatial_bhtd(q, k, v, exact_blocks=23)
        torch.cuda.current_stream().wait_stream(stream)
        assert out.shape == (1, 9216, 2 * D)
        assert torch.isfinite(out).all()


def test_spatial_pack_and_unpack_round_trip(native):
    batch, heads, tokens = 1, 2, 9216
    raster = torch.arange(tokens, dtype=torch.float32).to(torch.bfloat16)
    base = raster.view(1, tokens, 1, 1).expand(batch, tokens, heads, D).contiguous().cuda()
    bhtd = base.permute(0, 2, 1, 3)
    pq, pk, pv = native._C.pack_spatial_qkv(bhtd, bhtd, bhtd)
    assert pq[0, :16, 0].float().tolist() == list(range(8)) + list(range(96, 104))
    assert torch.equal(pq, pk) and torch.equal(pq, pv)
    restored = native._C.unpack_spatial_output(pq, batch, heads)
    assert torch.equal(restored, base.flatten(2))
    order = olayout.ordered_to_raster(np.arange(tokens))
    np.testing.assert_array_equal(np32(pq)[0, :, 0], np32(raster)[order])


def test_spatial_fused_epilogue_matches_merge(native):
    batch, heads, tokens = 1, 2, 9216
    gen = torch.Generator().manual_seed(53)
    exact = torch.randn((2, tokens, D), generator=gen).to(torch.bfloat16)
    approx = torch.randn((2, tokens, D), generator=gen).to(torch.bfloat16)
    corr = torch.randn((2, tokens, D), generator=gen)
    le = torch.randn((2, tokens), generator=gen)
    la = torch.randn((2, tokens), generator=gen)
    total = torch.logaddexp(le, la)
    merged = (exact.float() * torch.exp(le - total)[..., None]
              + (approx.float() + corr) * torch.exp(la - total)[..., None]).to(torch.bfloat16)
    order = olayout.ordered_to_raster(np.arange(tokens))
    expected = packed_to_merged(np32(merged), batch, heads, 1, 96, 96)
    actual = native._C.fuse_spatial_epilogue(exact.cuda(), le.cuda(), approx.cuda(), la.cuda(), corr.cuda(),
                                             batch, heads)
    assert_close(np32(actual), expected, 0.03125, 0.0, "fused epilogue")
    del order


# ----------------------------------------------------------------------------- generic / video
@pytest.mark.parametrize("grid,dtype,first_order", [
    ((1, 32, 32), torch.bfloat16, True),
    ((2, 16, 32), torch.float16, False),
    ((0, 0, 0), torch.bfloat16, True),
])
def test_generic_forward_matches_oracle(native, grid, dtype, first_order):
    tokens = 1024
    gen = torch.Generator().manual_seed(97)
    q4, k4, v4 = (torch.randn((1, 2, tokens, D), generator=gen).to(dtype).cuda() for _ in range(3))
    exact = 3
    out = native.generic_forward(q4, k4, v4, exact, 1 / math.sqrt(D), first_order,
                                 token_grid=grid if grid[0] else None)
    if grid[0]:
        packed = [spatial_to_packed(t, *grid) for t in (q4, k4, v4)]
    else:
        packed = [np32(t).reshape(2, tokens, D) for t in (q4, k4, v4)]
    name = "bf16" if dtype == torch.bfloat16 else "f16"
    # the statistics the reference's generic path takes for this shape (HYD for bf16 at T <= 9216)
    stats = native.generic_stats_mode(tokens, D, dtype)
    assert stats == ("hyd" if dtype == torch.bfloat16 else "generic")
    ref = opisa.generic_forward(*packed, exact, first_order=first_order, dtype=name, stats=stats)
    if grid[0]:
        expected = packed_to_merged(ref, 1, 2, *grid)
    else:
        expected = ref.reshape(1, 2, tokens, D).transpose(0, 2, 1, 3).reshape(1, tokens, 2 * D)
    assert_close(np32(out).reshape(1, tokens, 2 * D), expected, 5e-2, 5e-2, "generic")


# ----------------------------------------------------------------------------- dense attention
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("q_tokens,kv_tokens,head_dim", [(17, 31, 64), (64, 64, 128), (65, 137, 128), (129, 33, 64)])
def test_dense_matches_oracle(native, dtype, q_tokens, kv_tokens, head_dim):
    gen = torch.Generator().manual_seed(q_tokens + kv_tokens + head_dim)
    q = torch.randn((2, 1, q_tokens, head_dim), generator=gen).to(dtype).cuda()
    k = torch.randn((2, 1, kv_tokens, head_dim), generator=gen).to(dtype).cuda()
    v = torch.randn((2, 1, kv_tokens, head_dim), generator=gen).to(dtype).cuda()
    out = native.dense_attention(q, k, v, 1 / math.sqrt(head_dim))
    expected = oatt.dense_attention(np32(q), np32(k), np32(v))
    tol = 2e-2 if dtype == torch.float16 else 5e-2
    assert_close(np32(out), expected, tol, tol, "dense")


def test_dense_custom_scale(native):
    gen = torch.Generator().manual_seed(3)
    q = torch.randn((1, 1, 37, 128), generator=gen).to(torch.float16).cuda()
    k = torch.randn((1, 1, 71, 128), generator=gen).to(torch.float16).cuda()
    v = torch.randn((1, 1, 71, 128), generator=gen).to(torch.float16).cuda()
    out = native.dense_attention(q, k, v, 0.05)
    assert_close(np32(out), oatt.dense_attention(np32(q), np32(k), np32(v), 0.05), 2e-2, 2e-2, "scale 0.05")


def test_h3_strided_views_equal_packed_copies(native):
    tokens, heads = 700, 4
    gen = torch.Generator().manual_seed(tokens)
    qkv = torch.randn((1, tokens, 3, heads, D), generator=gen).to(torch.bfloat16).cuda()
    q, k, v = (qkv[:, :, i].permute(0, 2, 1, 3) for i in range(3))
    strided = native.dense_attention(q, k, v, 1 / math.sqrt(D), merged_output=True)
    packed = native.dense_attention(q.contiguous(), k.contiguous(), v.contiguous(), 1 / math.sqrt(D),
                                    merged_output=True)
    assert torch.equal(strided, packed)
    expected = oatt.dense_attention(np32(q), np32(k), np32(v)).transpose(0, 2, 1, 3).reshape(1, tokens, heads * D)
    assert_close(np32(strided), expected, 5e-2, 5e-2, "h3")


# ----------------------------------------------------------------------------- fixed block-diagonal
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [32, 64, 128])
@pytest.mark.parametrize("tokens", [64, 65, 200])
@pytest.mark.parametrize("causal", [False, True])
def test_fixed_block_matches_oracle(native, dtype, head_dim, tokens, causal):
    """fp16/bf16 run the matrix-core kernel with the Triton kernel's rounding of the normalised
    probabilities to the input dtype (triton_kernel.py:92-96); fp32 the fp32 kernel."""
    gen = torch.Generator().manual_seed(tokens + head_dim)
    q, k, v = (torch.randn((1, 2, tokens, head_dim), generator=gen).to(dtype).cuda() for _ in range(3))
    out = native.fixed_block_attention(q, k, v, 1 / math.sqrt(head_dim), causal)
    name = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}[dtype]
    prob = None if dtype == torch.float32 else name
    expected = oatt.fixed_block_attention(np32(q), np32(k), np32(v), causal=causal, out_dtype=name, prob_dtype=prob)
    tol = {torch.float32: 1e-5, torch.float16: 2e-3, torch.bfloat16: 1e-2}[dtype]
    assert_close(np32(out), expected, tol, tol, "fixed block")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fixed_block_replays_in_a_hip_graph(native, dtype):
    """The fixed-block entry point launches only its kernel, on the caller's stream, so callers
    (and bench.py's C1 kernel timing) can capture it in a HIP graph: every replay, with other
    eager work and synchronisations between replays, equals the eager result bit for bit."""
    gen = torch.Generator().manual_seed(5)
    q, k, v = (torch.randn((1, 8, 4096, 64), generator=gen).to(dtype).cuda() for _ in range(3))
    eager = native.fixed_block_attention(q, k, v, 0.125)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        native.fixed_block_attention(q, k, v, 0.125)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = native.fixed_block_attention(q, k, v, 0.125)
    for replay in range(4):
        other = native.fixed_block_attention(k, q, v, 0.25 + replay)  # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), f"replay {replay}"
        assert not torch.equal(other, eager)


def _graph_calls(native):
    from mi355x_pisa.synthetic import anima_qkv

    spatial = anima_qkv(batch=1, heads=2, seed=11, device="cuda")
    gen = torch.Generator().manual_seed(12)
    video = [torch.randn((1, 3, 4096, D), generator=gen).to(torch.bfloat16).cuda() for _ in range(3)]
    cross_q = torch.randn((1, 3, 1000, D), generator=gen).to(torch.bfloat16).cuda()
    return {
        "spatial": (lambda a, b, c: native.forward_spatial_bhtd(a, b, c, exact_blocks=23), spatial),
        "generic": (lambda a, b, c: native.generic_forward(a, b, c, 10, D ** -0.5, True, token_grid=(4, 32, 32),
                                                           stats="generic"), video),
        "dense": (lambda a, b, c: native.dense_attention(a, b, c, D ** -0.5), (cross_q, video[1], video[2])),
    }


@pytest.mark.parametrize("call", ["spatial", "generic", "dense"])
def test_forwards_replay_in_a_hip_graph(native, call):
    """The PISA and dense entry points launch kernels on the caller's stream and nothing else
    (no host synchronisation, no memset, workspace from the caller's allocator), so a caller can
    capture a whole call in a HIP graph: every replay, with other eager work of the same entry
    point and synchronisations between replays, equals the eager result bit for bit."""
    fn, (q, k, v) = _graph_calls(native)[call]
    eager = fn(q, k, v)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn(q, k, v)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = fn(q, k, v)
    for replay in range(4):
        other = fn(q, v, k)  # eager work of the same shapes between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), f"{call} replay {replay}"
        assert not torch.equal(other, eager)


def test_outputs_are_bit_reproducible_run_to_run(native):
    """No float atomics anywhere (H_sum is summed in a fixed chunk order, the routing select is a total
    order with ties to the lowest index): the Anima call at full size, the generic call and dense attention
    give the same bits on every run, with other work and a side stream between the runs."""
    from mi355x_pisa.synthetic import anima_qkv

    q, k, v = anima_qkv(batch=2, heads=16, seed=17, device="cuda")
    gen = torch.Generator().manual_seed(18)
    video = [torch.randn((1, 4, 8192, D), generator=gen).to(torch.bfloat16).cuda() for _ in range(3)]
    calls = [
        lambda: native.forward_spatial_bhtd(q, k, v, exact_blocks=23),
        lambda: native.generic_forward(*video, 21, D ** -0.5, True, token_grid=(2, 64, 64)),
        lambda: native.dense_attention(video[0], q[:1, :4], v[:1, :4], D ** -0.5),  # Tq 8192 over Tk 9216
    ]
    first = [fn() for fn in calls]
    side = torch.cuda.Stream()
    for run in range(3):
        native.dense_attention(q, k, v, D ** -0.5)  # other work between the runs
        if run == 1:
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                again = [fn() for fn in calls]
            torch.cuda.current_stream().wait_stream(side)
        else:
            again = [fn() for fn in calls]
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(first, again)):
            assert torch.equal(a, b), f"call {i} run {run}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fixed_block_16bit_paths_on_large_and_unaligned_inputs(native, dtype):
    """Many blocks through the matrix-core kernel (B=2 H=16 T=4096 D=128, a ComfyUI-sized call),
    and rows whose stride is not a multiple of 8 elements, which take the fp32 kernel instead."""
    gen = torch.Generator().manual_seed(41)
    name = {torch.float16: "f16", torch.bfloat16: "bf16"}[dtype]
    tol = {torch.float16: 2e-3, torch.bfloat16: 1e-2}[dtype]
    q, k, v = (torch.randn((2, 16, 4096, 128), generator=gen).to(dtype).cuda() for _ in range(3))
    out = native.fixed_block_attention(q, k, v, 128 ** -0.5, True)
    for b, h in ((0, 0), (1, 15)):
        expected = oatt.fixed_block_attention(np32(q[b, h]), np32(k[b, h]), np32(v[b, h]), causal=True,
                                              out_dtype=name, prob_dtype=name)
        assert_close(np32(out[b, h]), expected, tol, tol, f"fixed block head {(b, h)}")
    wide = [torch.randn((1, 2, 130, 68), generator=gen).to(dtype).cuda() for _ in range(3)]
    qs, ks, vs = (t[..., :64] for t in wide)  # token stride 68: not 16-byte aligned rows
    out = native.fixed_block_attention(qs, ks, vs, 0.125, False)
    expected = oatt.fixed_block_attention(np32(qs), np32(ks), np32(vs), scale=0.125, out_dtype=name)
    assert_close(np32(out), expected, tol, tol, "fixed block unaligned")
