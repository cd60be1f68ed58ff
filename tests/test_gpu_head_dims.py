"""Head dims other than 128 on the MI355X: generic PISA without the
first-order term (what the ComfyUI override asks for off 128 bf16,
generic_pisa.py:332-333), with it (a direct generic_pisa_attention call, whose
Triton statistics form H_sum at any width, pisa_kernel.py:90-130), and dense
attention, against the numpy oracle.  The kernels run at a padded width (64/96/128/160/192/256)
with zero dims in the packed tables; these tests cover every padded width,
both dtypes, raster and video token grids and short last blocks."""
from __future__ import annotations

import math

import pytest
import torch

from helpers import assert_close, np32, packed_to_merged, spatial_to_packed
from oracle import attention as oatt
from oracle import pisa as opisa

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 2e-2, torch.bfloat16: 5e-2}


@pytest.fixture(scope="module")
def native():
    import mi355x_pisa

    return mi355x_pisa


@pytest.mark.parametrize("head_dim,dtype,tokens,exact", [
    (40, torch.float16, 1000, 4),     # SD1.5 widths (tests/test_generic_pisa.py:93-99)
    (80, torch.float16, 1024, 4),
    (160, torch.float16, 777, 3),
    (64, torch.bfloat16, 1024, 5),    # SDXL / LTX
    (64, torch.float16, 640, 10),
    (96, torch.bfloat16, 900, 2),
    (192, torch.bfloat16, 512, 2),
    (256, torch.float16, 512, 3),
    (128, torch.float16, 1024, 4),    # fp16 at 128: no first-order term either
])
def test_generic_forward_head_dims_match_oracle(native, head_dim, dtype, tokens, exact):
    gen = torch.Generator().manual_seed(head_dim * 1000 + tokens)
    bh = 3
    q4, k4, v4 = (torch.randn((1, bh, tokens, head_dim), generator=gen).to(dtype).cuda() for _ in range(3))
    s = 1 / math.sqrt(head_dim)
    print(f"generic D={head_dim} {dtype} T={tokens} exact={exact}", flush=True)
    out = native.generic_forward(q4, k4, v4, exact, s, False)
    name = "bf16" if dtype == torch.bfloat16 else "f16"
    ref = opisa.generic_forward(*(np32(t).reshape(bh, tokens, head_dim) for t in (q4, k4, v4)), exact, s,
                                first_order=False, dtype=name)
    expected = ref.reshape(1, bh, tokens, head_dim).transpose(0, 2, 1, 3)
    assert out.shape == (1, tokens, bh, head_dim)
    assert_close(np32(out), expected, TOL[dtype], TOL[dtype], f"generic D={head_dim}")


@pytest.mark.parametrize("head_dim,grid,first_order", [(80, (2, 16, 32), False), (64, (1, 32, 32), False),
                                                       (160, (1, 24, 32), False), (80, (2, 16, 32), True),
                                                       (192, (1, 16, 32), True)])
def test_generic_forward_head_dims_on_token_grids(native, head_dim, grid, first_order):
    tokens = math.prod(grid)
    gen = torch.Generator().manual_seed(head_dim + tokens)
    q4, k4, v4 = (torch.randn((1, 2, tokens, head_dim), generator=gen).to(torch.float16).cuda() for _ in range(3))
    if first_order:  # values correlated with keys: a first-order term well above the tolerance
        v4 = 2 * k4 + 0.1 * v4
    exact = 3
    out = native.generic_forward(q4, k4, v4, exact, 1 / math.sqrt(head_dim), first_order, token_grid=grid)
    packed = [spatial_to_packed(t, *grid) for t in (q4, k4, v4)]
    ref = opisa.generic_forward(*packed, exact, first_order=first_order, dtype="f16")
    expected = packed_to_merged(ref, 1, 2, *grid)
    assert_close(np32(out).reshape(1, tokens, 2 * head_dim), expected, 2e-2, 2e-2, f"grid D={head_dim}")


@pytest.mark.parametrize("head_dim,dtype,tokens,exact", [
    (8, torch.bfloat16, 300, 1),      # padded 64, one 8-dim piece per slice
    (40, torch.float16, 1000, 2),     # padded 64
    (64, torch.bfloat16, 1024, 2),
    (96, torch.bfloat16, 900, 3),
    (120, torch.bfloat16, 640, 2),    # padded 128, head dim below it
    (128, torch.float16, 1024, 2),    # the statistics kernel's own H_sum (fp16, generic statistics)
    (160, torch.float16, 777, 2),     # above 128: the epilogue streams the H_sum fragments
    (192, torch.bfloat16, 512, 1),
    (256, torch.float16, 512, 2),     # query fragments in LDS
])
def test_generic_first_order_at_every_width_matches_oracle(native, head_dim, dtype, tokens, exact):
    """v = 2k + noise makes H_sum large (about 2T times the keys' covariance), so the first-order term is
    several times the output tolerance: checked both in the output and as the difference it makes."""
    gen = torch.Generator().manual_seed(head_dim * 31 + tokens)
    bh = 2
    q4, k4, n4 = (torch.randn((1, bh, tokens, head_dim), generator=gen) for _ in range(3))
    v4 = 2 * k4 + 0.1 * n4
    q4, k4, v4 = (t.to(dtype).cuda() for t in (q4, k4, v4))
    s = 1 / math.sqrt(head_dim)
    print(f"generic first-order D={head_dim} {dtype} T={tokens} exact={exact}", flush=True)
    out = native.generic_forward(q4, k4, v4, exact, s, True, stats="generic")
    out0 = native.generic_forward(q4, k4, v4, exact, s, False, stats="generic")
    name = "bf16" if dtype == torch.bfloat16 else "f16"
    packed = [np32(t).reshape(bh, tokens, head_dim) for t in (q4, k4, v4)]
    ref = opisa.generic_forward(*packed, exact, s, first_order=True, dtype=name)
    ref0 = opisa.generic_forward(*packed, exact, s, first_order=False, dtype=name)
    to_out = lambda r: r.reshape(1, bh, tokens, head_dim).transpose(0, 2, 1, 3)
    tol = TOL[dtype]
    assert_close(np32(out), to_out(ref), tol, tol, f"first-order D={head_dim}")
    term = to_out(ref) - to_out(ref0)
    assert abs(term).max() > 4 * tol, "the first-order term is too small to be checked"
    assert_close(np32(out) - np32(out0), term, 2 * tol, 2 * tol, f"first-order term D={head_dim}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("q_tokens,kv_tokens,head_dim", [
    (100, 130, 40), (64, 257, 80), (77, 64, 160), (130, 190, 192), (65, 99, 256), (33, 700, 96), (129, 64, 8),
])
def test_dense_head_dims_match_oracle(native, dtype, q_tokens, kv_tokens, head_dim):
    gen = torch.Generator().manual_seed(q_tokens * 7 + kv_tokens + head_dim)
    q = torch.randn((2, 2, q_tokens, head_dim), generator=gen).to(dtype).cuda()
    k = torch.randn((2, 2, kv_tokens, head_dim), generator=gen).to(dtype).cuda()
    v = torch.randn((2, 2, kv_tokens, head_dim), generator=gen).to(dtype).cuda()
    print(f"dense D={head_dim} {dtype} Tq={q_tokens} Tk={kv_tokens}", flush=True)
    out = native.dense_attention(q, k, v, 1 / math.sqrt(head_dim))
    expected = oatt.dense_attention(np32(q), np32(k), np32(v))
    assert_close(np32(out), expected, TOL[dtype], TOL[dtype], f"dense D={head_dim}")


def test_dense_head_dim_strided_merged_output(native):
    """SD1.5-style [B,T,H*D] storage read as BHTD views, merged output (the ComfyUI layout)."""
    batch, tokens, heads, head_dim = 1, 300, 8, 40
    gen = torch.Generator().manual_seed(40)
    x = torch.randn((3, batch, tokens, heads * head_dim), generator=gen).to(torch.float16).cuda()
    q, k, v = (t.view(batch, tokens, heads, head_dim).transpose(1, 2) for t in x)
    out = native.dense_attention(q, k, v, 1 / math.sqrt(head_dim), merged_output=True)
    expected = oatt.dense_attention(np32(q), np32(k), np32(v)).transpose(0, 2, 1, 3).reshape(batch, tokens, -1)
    assert_close(np32(out), expected, 2e-2, 2e-2, "dense merged D=40")


def _nan_padded(shape, head_dim, gen, dtype):
    """[..., head_dim] views of [..., head_dim + 8] storage whose last 8 columns hold NaN."""
    buf = torch.full((*shape, head_dim + 8), float("nan"), dtype=dtype)
    buf[..., :head_dim] = torch.randn((*shape, head_dim), generator=gen).to(dtype)
    return buf.cuda()[..., :head_dim]


@pytest.mark.parametrize("head_dim", [104, 112, 120])
def test_padded_128_head_dims_stay_inside_rows(native, head_dim):
    """Head dims 104..120 run at the padded width 128.  The query dims past the real head dim are
    read as zero (NaN stored after each row would reach every score otherwise) and the stores stop
    at the real dims (the storage after each output row keeps its sentinel)."""
    gen = torch.Generator().manual_seed(head_dim)
    dtype = torch.bfloat16
    q, k, v = (_nan_padded((2, 2, 200), head_dim, gen, dtype) for _ in range(3))
    s = 1 / math.sqrt(head_dim)
    out_buf = torch.full((2, 2, 200, head_dim + 8), 3.0, dtype=dtype, device="cuda")
    print(f"dense D={head_dim} padded views", flush=True)
    native._launch_dense(q, k, v, out_buf[..., :head_dim], s)
    torch.cuda.synchronize()
    expected = oatt.dense_attention(np32(q), np32(k), np32(v))
    assert_close(np32(out_buf[..., :head_dim]), expected, TOL[dtype], TOL[dtype], f"dense D={head_dim}")
    assert bool((out_buf[..., head_dim:] == 3.0).all()), "stores past the real head dim"

    print(f"generic D={head_dim} padded views", flush=True)
    out = native.generic_forward(q, k, v, 2, s, False)
    ref = opisa.generic_forward(*(np32(t).reshape(4, 200, head_dim) for t in (q, k, v)), 2, s,
                                first_order=False, dtype="bf16")
    assert_close(np32(out), ref.reshape(2, 2, 200, head_dim).transpose(0, 2, 1, 3), TOL[dtype], TOL[dtype],
                 f"generic D={head_dim}")
