"""Seeded random sweep of the sparse PISA forward over small shapes, against the numpy oracle.

Each case draws a routing regime (HYD, generic on the generic statistics, generic routing on the HYD
statistics), a dtype, a head dim, a token count or a frames x height x width grid, an exact block count
(0, 1, N-1 and values between), a sink block (HYD) and the first-order term (generic), and checks through
``mi355x_pisa.forward_with_routing``:

* the routing scores against ``oracle.pisa.route_scores`` on the oracle's statistics (1e-4 + 1e-4 relative);
* the selection against the stable top-k of the kernel's own scores (bit-exact; ties to the lowest index);
* the output against the oracle's forward (``oracle.pisa._sparse_parts`` / ``_correction`` / ``_merge``, the
  restatement of __init__.py:233-316 and generic_pisa.py:141-232) on the kernel's selection, so a near-tie
  between two blocks cannot move a row (bf16 atol = rtol = 5e-2, fp16 2e-2).

The exact attention and fixed block-diagonal kernels get sweeps of their own (below).  The cases are listed in
the test ids; every run draws the same ones.  MI355X_SWEEP_SCALE (an integer, default 1) multiplies the number of
cases and MI355X_SWEEP_SEED (default 0) offsets the seeds, for longer runs over other cases.
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

from helpers import assert_close, np32
from oracle import attention as oatt
from oracle import layout as olayout
from oracle import numerics as onum
from oracle import pisa as opisa

pytestmark = pytest.mark.gpu
TOL = {torch.bfloat16: 5e-2, torch.float16: 2e-2}
SCALE = int(os.environ.get("MI355X_SWEEP_SCALE", "1"))
SEED = int(os.environ.get("MI355X_SWEEP_SEED", "0"))


def _cases(count=120 * SCALE, seed=2026 + SEED):
    rng = np.random.default_rng(seed)
    grids = [(1, 16, 24), (2, 16, 16), (1, 32, 32), (3, 8, 24), (1, 8, 8)]
    cases = []
    sinks = 0
    for i in range(count):
        mode = ["hyd", "generic", "generic_hyd"][i % 3]
        dtype = [torch.bfloat16, torch.float16][(i // 3) % 2]
        head_dim = 128 if mode != "generic" else int(rng.choice([64, 96, 128, 160]))
        grid = None
        if i % 4 == 0:
            grid = grids[(i // 4) % len(grids)]
            tokens = grid[0] * grid[1] * grid[2]
        else:
            tokens = int(rng.integers(65, 1500))
        blocks = (tokens + 63) // 64
        exact = min([0, 1, blocks - 1, int(rng.integers(0, blocks))][int(rng.integers(0, 4))], blocks - 1)
        sink = None
        if mode == "hyd" and exact > 0 and rng.random() < 0.5:
            sink = [0, -1][sinks % 2]  # both sink positions (__init__.py:260-263)
            sinks += 1
        first_order = True if mode == "hyd" else bool(i % 2)
        heads = int(rng.integers(1, 4))
        cases.append((mode, dtype, head_dim, tokens, grid, exact, sink, first_order, heads, int(rng.integers(1 << 30))))
    return cases


def _case_id(c):
    mode, dtype, d, t, grid, exact, sink, fo, heads, _ = c
    where = "x".join(map(str, grid)) if grid else f"T{t}"
    return f"{mode}-{'bf16' if dtype == torch.bfloat16 else 'f16'}-D{d}-{where}-e{exact}-s{sink}-fo{int(fo)}-h{heads}"


@pytest.fixture(scope="module")
def native():
    import mi355x_pisa

    return mi355x_pisa


@pytest.mark.parametrize("case", _cases(), ids=_case_id)
def test_random_case_matches_oracle(native, case):
    mode, dtype, head_dim, tokens, grid, exact, sink, first_order, heads, seed = case
    print(f"[sweep] {_case_id(case)}", flush=True)
    gen = torch.Generator().manual_seed(seed)
    # raster [1, T, H, D] storage read as [1, H, T, D] views, as the ComfyUI callers pass them
    q4, k4, v4 = (torch.randn((1, tokens, heads, head_dim), generator=gen).to(dtype).cuda().permute(0, 2, 1, 3)
                  for _ in range(3))
    s = float(np.float32(1.0 / math.sqrt(head_dim)))
    out, scores, idx = native.forward_with_routing(q4, k4, v4, exact, s, sink_block=sink, mode=mode,
                                                   first_order=first_order, token_grid=grid)
    name = "bf16" if dtype == torch.bfloat16 else "f16"
    order = olayout.tile_order(*grid) if grid else np.arange(tokens)
    qp, kp, vp = (olayout.pack(np32(t).reshape(heads, tokens, head_dim), order) for t in (q4, k4, v4))
    st = opisa.block_stats(qp, kp, vp, "generic" if mode == "generic" else "hyd", name)
    idx = idx.cpu().numpy().astype(np.int64)
    if exact > 0:
        if mode == "hyd":
            ref_scores = opisa.route_scores(st["q_centroids_f32"], st["k_centroids"], s, st["h_norm"], sink, True)
        else:
            ref_scores = opisa.route_scores(st["q_centroids"], st["k_centroids"], s, None, None, False)
        got = scores.cpu().numpy()
        assert_close(got, ref_scores, 1e-4, 1e-4, "routing scores")
        assert np.array_equal(idx, opisa.topk_ascending(got, exact)), "selection is not the top-k of its scores"
    k_tail = onum.round_dtype(st["k_centroids"], "bf16" if (mode == "hyd" and name == "bf16") else name)
    o_e, l_e, o_a, l_a = opisa._sparse_parts(qp, kp, vp, idx, k_tail, st["v_means"], st["lengths"], s)
    o_a = onum.round_dtype(o_a, name).astype(np.float64)
    corr = opisa._correction(qp, st["h_sum"], s, tokens, name) if first_order else None
    if exact == 0 and mode == "hyd":
        ref = onum.round_dtype(o_a + corr, name)
    else:
        ref = opisa._merge(onum.round_dtype(o_e, name).astype(np.float64), l_e, o_a, l_a, corr, name)
    raster = np.empty_like(ref)
    raster[:, order] = ref
    assert_close(np32(out[0]), raster, TOL[dtype], TOL[dtype], _case_id(case))


def _dense_cases(count=60 * SCALE, seed=77 + SEED):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        dtype = [torch.bfloat16, torch.float16][i % 2]
        head_dim = int(rng.choice([8, 40, 64, 80, 96, 128, 160, 200, 256]))
        q_tokens = int(rng.choice([1, 63, 64, int(rng.integers(2, 700))]))
        kv_tokens = int(rng.choice([1, 64, 65, int(rng.integers(2, 700))]))
        layout = ["bhtd", "bthd"][int(rng.integers(0, 2))]
        cases.append((dtype, head_dim, q_tokens, kv_tokens, int(rng.integers(1, 3)), int(rng.integers(1, 5)),
                      layout, bool(rng.random() < 0.3), int(rng.integers(1 << 30))))
    return cases


def _dense_id(c):
    dtype, d, tq, tk, b, h, layout, merged, _ = c
    return f"{'bf16' if dtype == torch.bfloat16 else 'f16'}-D{d}-Tq{tq}-Tk{tk}-B{b}H{h}-{layout}{'-merged' if merged else ''}"


@pytest.mark.parametrize("case", _dense_cases(), ids=_dense_id)
def test_random_dense_case_matches_oracle(native, case):
    """Exact attention (triton_kernel.py:113-197 semantics) on seeded random shapes: ragged and single-token query
    and key counts, head dims 8-256, contiguous [B,H,T,D] or raster [B,T,H,D] storage, merged [B,T,H*D] output."""
    dtype, head_dim, q_tokens, kv_tokens, batch, heads, layout, merged, seed = case
    print(f"[sweep dense] {_dense_id(case)}", flush=True)
    gen = torch.Generator().manual_seed(seed)

    def make(tokens):
        if layout == "bhtd":
            return torch.randn((batch, heads, tokens, head_dim), generator=gen).to(dtype).cuda()
        return torch.randn((batch, tokens, heads, head_dim), generator=gen).to(dtype).cuda().permute(0, 2, 1, 3)

    q, k, v = make(q_tokens), make(kv_tokens), make(kv_tokens)
    s = head_dim ** -0.5
    out = native.dense_attention(q, k, v, s, merged_output=merged)
    ref = oatt.dense_attention(np32(q), np32(k), np32(v), s)
    got = np32(out.view(batch, q_tokens, heads, head_dim).permute(0, 2, 1, 3)) if merged else np32(out)
    assert_close(got, ref, TOL[dtype], TOL[dtype], _dense_id(case))


FIXED_TOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 5e-2}  # masked: fp32 probabilities
FIXED_TOL_TRITON = {torch.float16: 2e-3, torch.bfloat16: 1e-2}                # unmasked 16-bit: probabilities in dtype


def _fixed_cases(count=60 * SCALE, seed=91 + SEED):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        dtype = [torch.float32, torch.bfloat16, torch.float16][i % 3]
        mask = ["none", "none", "bool", "f32", "f16", "bf16"][int(rng.integers(0, 6))]
        broadcast = ["full", "batch", "head", "shared"][int(rng.integers(0, 4))]
        cases.append((dtype, int(rng.choice([32, 64, 128])), int(rng.choice([1, 64, 65, int(rng.integers(2, 600))])),
                      int(rng.integers(1, 3)), int(rng.integers(1, 4)), bool(rng.random() < 0.5), mask, broadcast,
                      int(rng.integers(1 << 30))))
    return cases


def _fixed_id(c):
    dtype, d, t, b, h, causal, mask, bc, _ = c
    name = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[dtype]
    return f"{name}-D{d}-T{t}-B{b}H{h}-c{int(causal)}-{mask}{'-' + bc if mask != 'none' else ''}"


@pytest.mark.parametrize("case", _fixed_cases(), ids=_fixed_id)
def test_random_fixed_block_case_matches_oracle(native, case):
    """Fixed 64-token block-diagonal attention (reference.py:159-200; triton_kernel.py:53-100 for unmasked 16-bit
    calls, whose probabilities are rounded to the dtype) on seeded random shapes: ragged last blocks, T = 1, causal,
    bool and additive masks broadcast over batch, heads or both through zero strides."""
    dtype, head_dim, tokens, batch, heads, causal, mask_kind, broadcast, seed = case
    print(f"[sweep fixed] {_fixed_id(case)}", flush=True)
    gen = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn((batch, heads, tokens, head_dim), generator=gen).to(dtype).cuda() for _ in range(3))
    s = head_dim ** -0.5
    view = None
    if mask_kind != "none":
        shape = {"full": (batch, heads), "batch": (batch, 1), "head": (1, heads), "shared": (1, 1)}[broadcast]
        raw = torch.rand((*shape, tokens, tokens), generator=gen)
        keep_own = torch.eye(tokens, dtype=torch.bool)  # every row keeps its own key
        if mask_kind == "bool":
            m = (raw < 0.7) | keep_own
        else:
            m = torch.where(raw < 0.2, torch.tensor(float("-inf")), raw * 3.0 - 1.5)
            m = torch.where(keep_own, raw * 0.1, m).to({"f32": torch.float32, "f16": torch.float16,
                                                       "bf16": torch.bfloat16}[mask_kind])
        view = m.cuda().expand(batch, heads, tokens, tokens)
    out = native.fixed_block_attention(q, k, v, s, causal, view)
    if view is None:
        prob = None if dtype == torch.float32 else ("bf16" if dtype == torch.bfloat16 else "f16")
        expected = oatt.fixed_block_attention(np32(q), np32(k), np32(v), 64, s, causal, prob_dtype=prob)
        tol = FIXED_TOL[dtype] if dtype == torch.float32 else FIXED_TOL_TRITON[dtype]
    else:
        host = view.cpu().numpy() if mask_kind == "bool" else np32(view)
        expected = oatt.fixed_block_attention(np32(q), np32(k), np32(v), 64, s, causal, mask=host)
        tol = FIXED_TOL[dtype]
    assert_close(np32(out), expected, tol, tol, _fixed_id(case))
