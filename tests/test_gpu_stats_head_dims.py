"""GPU parity of the HYD block statistics at head dims other than 128.

The reference's ``_C.block_stats_hyd`` takes fp16/bf16 [BH,T,D] at any
0<D<=256 and returns q_bar, k_bar, v_bar, H_sum and ||H_b||_F at every width
(native/rdna35_pisa_ck/csrc/pisa_kernels.cu:167-244,597-635;
rdna35_pisa_ck/__init__.py:216-230).  Here every width off 128 runs on the
means + covariance kernels (16-byte row pieces at multiples of 8, element
loads at odd widths); each output is compared with
``oracle.pisa.block_stats(..., "hyd")`` (fp32 sums times fp32(1/len), q_bar and
v_bar rounded to the dtype, keys centred in fp32, float64 products).
Tolerances: k_bar at fp32 accuracy, q_bar / v_bar within one dtype rounding
step, H_sum 1e-4 of its largest element, h_norm 1e-4 relative.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_close, dtype_name, np32
from oracle import pisa as opisa

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def native():
    import mi355x_pisa

    return mi355x_pisa


def _inputs(bh, tokens, head_dim, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    return tuple(torch.randn((bh, tokens, head_dim), generator=gen).to(dtype).cuda() for _ in range(3))


def _check_hyd(outputs, q, k, v, dtype):
    qc, kc, vm, hs, hn = outputs
    st = opisa.block_stats(np32(q), np32(k), np32(v), "hyd", dtype_name(dtype))
    step = 1e-2 if dtype == torch.bfloat16 else 2e-3
    assert qc.dtype == dtype and vm.dtype == dtype and kc.dtype == torch.float32
    assert_close(np32(kc), st["k_centroids"], 1e-6, 1e-5, "k_centroids")
    assert_close(np32(qc), st["q_centroids"], step, step, "q_centroids")
    assert_close(np32(vm), st["v_means"], step, step, "v_means")
    scale_h = float(np.abs(st["h_sum"]).max())
    assert_close(np32(hs), st["h_sum"], 1e-4 * scale_h, 1e-4, "h_sum")
    assert_close(np32(hn), st["h_norm"], 1e-4 * float(st["h_norm"].max()), 1e-4, "h_norm")


@pytest.mark.parametrize("tokens", [65, 576, 9216])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("head_dim", [32, 64, 80, 200, 256, 1, 37, 100, 255])
def test_hyd_stats_every_head_dim_match_oracle(native, head_dim, dtype, tokens):
    print(f"[hyd stats] D={head_dim} {dtype} T={tokens}", flush=True)
    bh = 2 if tokens < 9216 else 1
    q, k, v = _inputs(bh, tokens, head_dim, dtype, seed=head_dim * 7 + tokens)
    raw = native._C.block_stats_hyd(q, k, v)
    assert len(raw) == 5 and raw[4].shape == (bh, (tokens + 63) // 64)
    _check_hyd(raw, q, k, v, dtype)
    # the public wrapper returns the first four outputs, bit-equal
    for a, b in zip(native.block_stats_hyd(q, k, v), raw[:4]):
        assert torch.equal(a, b)


def test_hyd_stats_other_widths_through_the_reference_name(native):
    """rdna35_pisa_ck (the reference's module name) gives the same statistics at D=64 and refuses T>9216."""
    import rdna35_pisa_ck

    q, k, v = _inputs(2, 300, 64, torch.float16, seed=3)
    ours = native._C.block_stats_hyd(q, k, v)
    theirs = rdna35_pisa_ck._C.block_stats_hyd(q, k, v)
    for a, b in zip(ours, theirs):
        assert torch.equal(a, b)
    long = torch.zeros((1, 9280, 64), dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="T<=9216"):
        rdna35_pisa_ck._C.block_stats_hyd(long, long, long)
    with pytest.raises(ValueError, match="0<T<=9216"):
        rdna35_pisa_ck.block_stats_hyd(long, long, long)
    # mi355x_pisa itself takes the longer sequence
    assert native.block_stats_hyd(long, long, long)[0].shape == (1, 145, 64)


def test_constant_keys_per_block_have_zero_covariance_at_head_dim_96(native):
    gen = torch.Generator().manual_seed(8)
    keys = torch.randn((1, 3, 1, 96), generator=gen).expand(1, 3, 64, 96).reshape(1, 192, 96)
    k = keys.to(torch.bfloat16).cuda()
    q, _, v = _inputs(1, 192, 96, torch.bfloat16, seed=9)
    _, _, _, hs, hn = native._C.block_stats_hyd(q, k, v)
    assert torch.count_nonzero(hs) == 0
    assert torch.count_nonzero(hn) == 0


@pytest.mark.parametrize("dtype_name_, tokens", [("bfloat16", 8192), ("float16", 8192), ("bfloat16", 16384)])
def test_reference_stats_choice_on_device_matches_generic_stats_mode(native, dtype_name_, tokens):
    """The reference's _block_stats rule (generic_pisa.py:119-128), run on device tensors against the
    reference-named module, picks the regime of mi355x_pisa.generic_stats_mode."""
    import rdna35_pisa_ck
    from test_abi import _reference_stats_choice

    dtype = getattr(torch, dtype_name_)
    x = torch.zeros((1, tokens, 128), dtype=dtype, device="cuda")
    assert _reference_stats_choice(rdna35_pisa_ck, x, x, x) == native.generic_stats_mode(tokens, 128, dtype)


def test_reference_name_traces_under_torch_compile(native):
    """torch.compile(fullgraph=True) through rdna35_pisa_ck (the reference compiles its ops the same way,
    test_forward.py:203-209): HYD statistics at head dim 64 and the HYD forward give the eager bits."""
    import rdna35_pisa_ck

    q, k, v = _inputs(2, 300, 64, torch.bfloat16, seed=5)

    def stats(q, k, v):
        return rdna35_pisa_ck.block_stats_hyd(q, k, v)

    for a, b in zip(torch.compile(stats, backend="inductor", fullgraph=True)(q, k, v), stats(q, k, v)):
        assert torch.equal(a, b)
    q2, k2, v2 = _inputs(2, 256, 128, torch.bfloat16, seed=6)

    def forward(q, k, v):
        return rdna35_pisa_ck.forward(q, k, v, exact_blocks=1)

    assert torch.equal(torch.compile(forward, backend="inductor", fullgraph=True)(q2, k2, v2), forward(q2, k2, v2))


@pytest.mark.parametrize("head_dim", [128, 64, 37])
def test_fp16_keys_near_the_range_limit_centre_without_overflow(native, head_dim):
    """Keys of -60000 with one +60000 row per block centre to about 1.18e5, past fp16's 65504: the reference
    centres in fp32 (pisa_kernels.cu:225-227) and its H_b stays finite, and so must the fp16 statistics here
    (head dim 128: stats_kernel; others: stats_cov_kernel)."""
    print(f"[hyd stats fp16 near max] D={head_dim}", flush=True)
    gen = torch.Generator().manual_seed(head_dim)
    k = torch.full((2, 300, head_dim), -60000.0)
    k[:, ::64] = 60000.0
    q, v = (torch.randn((2, 300, head_dim), generator=gen) for _ in range(2))
    q, k, v = (t.to(torch.float16).cuda() for t in (q, k, v))
    qc, kc, vm, hs, hn = native._C.block_stats_hyd(q, k, v)
    assert torch.isfinite(hs).all() and torch.isfinite(hn).all()
    _check_hyd((qc, kc, vm, hs, hn), q, k, v, torch.float16)
