"""Masked fixed block-diagonal attention on the MI355X kernel (the calls the
reference sends to its eager loop, reference.py:186-195) against the numpy
oracle: bool and additive masks, every broadcast shape of _mask_block
(reference.py:114-156), causal + mask, fully masked rows (NaN)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from helpers import assert_close, np32
from oracle import attention as oatt

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 5e-2}


@pytest.fixture(scope="module")
def native():
    import mi355x_pisa

    return mi355x_pisa


def _mask(kind, shape, gen):
    raw = torch.rand(shape, generator=gen)
    if kind == "bool":
        m = raw < 0.7
        return m | torch.eye(shape[-1], dtype=torch.bool).expand(shape)  # every row keeps its own key
    additive = torch.where(raw < 0.2, torch.tensor(float("-inf")), raw * 3.0 - 1.5)
    additive = torch.where(torch.eye(shape[-1], dtype=torch.bool).expand(shape), raw * 0.1, additive)
    return additive.to({"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16, "f64": torch.float64}[kind])


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("kind", ["bool", "f32", "f16", "bf16"])
@pytest.mark.parametrize("causal", [False, True])
def test_native_masked_matches_oracle(native, dtype, kind, causal):
    batch, heads, tokens, head_dim = 2, 3, 150, 64
    gen = torch.Generator().manual_seed(len(kind) * 10 + causal)
    q, k, v = (torch.randn((batch, heads, tokens, head_dim), generator=gen).to(dtype).cuda() for _ in range(3))
    mask = _mask(kind, (batch, 1, tokens, tokens), gen)          # per batch, broadcast over heads
    view = mask.cuda().expand(batch, heads, tokens, tokens)
    s = 1 / math.sqrt(head_dim)
    out = native.fixed_block_attention(q, k, v, s, causal, view)
    host_mask = view.cpu().numpy() if kind == "bool" else np32(view)  # bool stays a keep-mask
    expected = oatt.fixed_block_attention(np32(q), np32(k), np32(v), 64, s, causal, mask=host_mask)
    assert_close(np32(out), expected, TOL[dtype], TOL[dtype], f"masked {kind} causal={causal}")


@pytest.mark.parametrize("layout,shape,heads,mask_shape", [
    ("bhtd", (2, 3, 130, 32), None, (130, 130)),
    ("bhtd", (2, 3, 130, 32), None, (2, 130, 130)),
    ("bhtd", (2, 3, 130, 32), None, (6, 130, 130)),
    ("bhtd", (2, 3, 130, 32), None, (1, 3, 130, 130)),
    ("bthd", (2, 200, 4 * 128), 4, (2, 4, 200, 200)),   # [B,T,H*D] (the ComfyUI layout)
    ("bthd", (1, 96, 4 * 32), 4, (1, 96, 96)),
    ("bh_t_d", (5, 64, 32), None, (5, 64, 64)),
    ("auto", (1, 2, 70, 64), None, (70, 70)),
])
@pytest.mark.parametrize("kind", ["bool", "f64"])
def test_dispatch_masked_runs_hip_and_matches_eager(layout, shape, heads, mask_shape, kind):
    from rdna35_block_attention import fixed_block_attention
    from rdna35_block_attention.reference import fixed_block_attention_ref

    gen = torch.Generator().manual_seed(sum(shape))
    q, k, v = (torch.randn(shape, generator=gen).to(torch.float16).cuda() for _ in range(3))
    mask = _mask(kind, mask_shape, gen).cuda()
    out, info = fixed_block_attention(q, k, v, layout=layout, heads=heads, mask=mask, return_diagnostics=True)
    assert info["backend"] == "hip", info
    # eager restatement on fp32 copies (torch's block loop, the reference's own path)
    ref = fixed_block_attention_ref(q.float(), k.float(), v.float(), layout=layout, heads=heads, mask=mask)
    assert_close(np32(out), np32(ref), 2e-2, 2e-2, f"dispatch {layout} {mask_shape} {kind}")


def test_fully_masked_row_is_nan_like_torch(native):
    tokens = 100
    q = torch.randn((1, 2, tokens, 32), dtype=torch.float16, device="cuda")
    mask = torch.ones((tokens, tokens), dtype=torch.bool)
    mask[7, :] = False            # query 7 keeps nothing
    mask[70, 64:] = False         # query 70 keeps nothing inside its block (keys 0..63 are outside the block)
    view = mask.cuda().expand(1, 2, tokens, tokens)
    out = np32(native.fixed_block_attention(q, q, q, 0.2, False, view))
    assert np.isnan(out[:, :, [7, 70]]).all()
    rest = np.delete(out, [7, 70], axis=2)
    assert np.isfinite(rest).all()
    eager = torch.softmax(torch.full((4,), float("-inf")), dim=0)
    assert torch.isnan(eager).all()  # the torch behaviour mirrored
