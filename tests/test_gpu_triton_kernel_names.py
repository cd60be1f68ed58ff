"""The reference's rdna35_block_attention/triton_kernel.py entry points (triton_kernel.py:166-244) on the HIP
kernels, against the numpy oracle."""
from __future__ import annotations

import math

import pytest
import torch

from helpers import assert_close, np32
from oracle import attention as oatt

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("head_dim,dtype,causal", [(64, torch.bfloat16, False), (128, torch.float16, True),
                                                   (32, torch.float16, False)])
def test_fixed_block_attention_triton_bh_matches_oracle(head_dim, dtype, causal):
    from rdna35_block_attention.triton_kernel import fixed_block_attention_triton_bh

    gen = torch.Generator().manual_seed(head_dim + int(causal))
    q, k, v = (torch.randn((3, 200, head_dim), generator=gen).to(dtype).cuda() for _ in range(3))
    out = fixed_block_attention_triton_bh(q, k, v, causal=causal)
    name = "bf16" if dtype == torch.bfloat16 else "f16"
    ref = oatt.fixed_block_attention(np32(q), np32(k), np32(v), causal=causal, out_dtype=name, prob_dtype=name)
    assert out.shape == q.shape and out.dtype == dtype
    tol = 2e-2 if dtype == torch.float16 else 5e-2
    assert_close(np32(out), ref, tol, tol, f"fixed block D={head_dim}")


def test_full_attention_triton_bh_matches_oracle():
    from rdna35_block_attention.triton_kernel import full_attention_triton_bh

    gen = torch.Generator().manual_seed(5)
    q = torch.randn((2, 300, 128), generator=gen).to(torch.bfloat16).cuda()
    k, v = (torch.randn((2, 200, 128), generator=gen).to(torch.bfloat16).cuda() for _ in range(2))
    s = 1 / math.sqrt(128)
    out = full_attention_triton_bh(q, k, v, scale=s, block_m=32, block_n=32, num_warps=4, waves_per_eu=1)
    ref = oatt.dense_attention(np32(q), np32(k), np32(v), s, out_dtype="bf16")
    assert out.shape == q.shape and out.dtype == q.dtype
    assert_close(np32(out), ref, 5e-2, 5e-2, "full attention")
