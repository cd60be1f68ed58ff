"""pisa_prepare_triton (the reference's rdna35_block_attention/pisa_kernel.py:90-131) on the HIP statistics
kernels: key means, value sums and H_sum of the Triton statistics (centred keys rounded to the input dtype)
at head dim 128 and at other widths, against the numpy oracle."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import assert_close, np32
from oracle import pisa as opisa

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("head_dim,dtype,tokens", [
    (128, torch.bfloat16, 1000),   # the statistics kernel's generic mode
    (64, torch.bfloat16, 1000),    # means + covariance kernels, ragged last block
    (40, torch.float16, 640),      # padded to 64
    (200, torch.float16, 576),     # padded to 256
    (96, torch.bfloat16, 64),      # a single block
    (100, torch.bfloat16, 300),    # odd widths: element loads, padded to 128 (the reference pads to 128 too)
    (37, torch.float16, 130),
])
def test_pisa_prepare_matches_oracle(head_dim, dtype, tokens):
    from rdna35_block_attention.pisa_kernel import pisa_prepare_triton

    gen = torch.Generator().manual_seed(head_dim * 7 + tokens)
    bh = 3
    k, v = (torch.randn((bh, tokens, head_dim), generator=gen).to(dtype).cuda() for _ in range(2))
    print(f"prepare D={head_dim} {dtype} T={tokens}", flush=True)
    k_means, v_sums, h_sum, lengths = pisa_prepare_triton(k, v, block_size=64)
    blocks = (tokens + 63) // 64
    assert lengths == [min(64, tokens - 64 * b) for b in range(blocks)]
    assert k_means.shape == v_sums.shape == (bh, blocks, head_dim) and h_sum.shape == (bh, head_dim, head_dim)
    assert k_means.dtype == v_sums.dtype == h_sum.dtype == torch.float32
    name = "bf16" if dtype == torch.bfloat16 else "f16"
    kn, vn = np32(k), np32(v)
    ref = opisa.block_stats(kn, kn, vn, "generic", name)
    assert_close(np32(k_means), ref["k_centroids"], 1e-6, 1e-5, "k means")
    pad = blocks * 64 - tokens
    vb = np.pad(vn, ((0, 0), (0, pad), (0, 0))).reshape(bh, blocks, 64, head_dim).astype(np.float64)
    assert_close(np32(v_sums), vb.sum(axis=2), 1e-5, 2e-6, "v sums")
    scale = float(np.abs(ref["h_sum"]).max())
    assert_close(np32(h_sum), ref["h_sum"], 1e-5 * scale, 1e-5, "H_sum")
