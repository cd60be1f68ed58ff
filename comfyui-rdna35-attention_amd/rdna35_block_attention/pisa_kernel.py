"""PISA preparation statistics (the reference's rdna35_block_attention/pisa_kernel.py).

pisa_prepare_triton keeps its name, arguments, checks and outputs
(pisa_kernel.py:90-131): per 64-token block the fp32 key means and value sums,
H_sum = sum over blocks of dtype(K_b - k_bar_b)^T V_b in fp32 (the centred keys
rounded to the input dtype, pisa_kernel.py:80-81), and the block lengths.  It
runs on the library's HIP statistics kernels for gfx950 (the statistics kernel
at head dim 128, the means and covariance kernels at other widths); H_sum is
summed in a fixed order, without the reference's float atomics.  Any head
dim up to 256 is taken, as the reference pads any width (the kernels read
16-byte pieces at multiples of 8 and single elements otherwise).  The value
sums are the fp32 sums of each block's rows (pisa_kernel.py:74,78).
"""
from __future__ import annotations

import math

import torch

from . import diagnostics


def pisa_prepare_triton(k: torch.Tensor, v: torch.Tensor, *, block_size: int = 64):
    """(k_means [BH,N,D] fp32, v_sums [BH,N,D] fp32, h_sum [BH,D,D] fp32, lengths) of [BH,T,D] k/v."""
    if k.ndim != 3 or k.shape != v.shape:
        raise ValueError("PISA Triton preparation expects matching [BH,T,D] k/v.")
    if block_size != 64:
        raise ValueError("PISA Triton preparation requires block_size=64.")
    if k.dtype not in (torch.float16, torch.bfloat16) or v.dtype != k.dtype:
        raise ValueError("PISA Triton preparation requires matching fp16/bf16 k/v.")
    if not k.is_cuda or not v.is_cuda:
        raise ValueError("PISA Triton preparation requires CUDA/HIP tensors.")
    if not k.is_contiguous() or not v.is_contiguous():
        raise ValueError("PISA Triton preparation requires contiguous k/v.")
    batch_heads, tokens, head_dim = k.shape
    if head_dim > 256:
        raise ValueError(f"PISA Triton preparation requires D<=256, got D={head_dim}.")
    native = diagnostics.load_native()
    # the query means are not part of this output: k stands in for q
    _, k_means, v_sums, h_sum, _ = native._block_stats(k, k, v, native._lib.STATS_GENERIC, torch.float32,
                                                       value_sums=True)
    total_blocks = math.ceil(tokens / block_size)
    lengths = [min(block_size, tokens - block * block_size) for block in range(total_blocks)]
    return k_means, v_sums, h_sum, lengths
