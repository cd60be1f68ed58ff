"""The reference's rdna35_block_attention/triton_kernel.py entry points on the HIP kernels.

fixed_block_attention_triton_bh and full_attention_triton_bh keep their names,
keyword arguments, checks and outputs (triton_kernel.py:166-244); the work runs
on the library's gfx950 kernels: fixed_block_mfma_kernel (the Triton kernel's
semantics: fp32 scores and softmax, probabilities rounded to the input dtype
before P.V) and the dense attention kernel.  The tile arguments of
full_attention_triton_bh (block_m, block_n, num_warps, waves_per_eu) are
accepted and not used: the HIP kernel has its own tiling.
"""
from __future__ import annotations

import math

import torch

from . import diagnostics


def full_attention_triton_bh(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, scale: float, block_m: int,
                             block_n: int, num_warps: int, waves_per_eu: int) -> torch.Tensor:
    """softmax(scale q k^T) v of [BH,Q,D] q and [BH,K,D] k/v, [BH,Q,D] output in q's dtype."""
    del block_m, block_n, num_warps, waves_per_eu
    native = diagnostics.load_native()
    return native.dense_attention(q.unsqueeze(1), k.unsqueeze(1), v.unsqueeze(1), float(scale))[:, 0]


def fixed_block_attention_triton_bh(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, block_size: int = 64,
                                    scale: float | None = None, causal: bool = False) -> torch.Tensor:
    """Fixed 64-token block-diagonal attention of [BH,T,D] fp16/bf16 q/k/v."""
    if q.ndim != 3:
        raise ValueError(f"Triton path expects [BH,T,D], got rank {q.ndim}.")
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError("Triton path requires identical q/k/v shapes.")
    if block_size != 64:
        raise ValueError("Triton path only supports block_size=64.")
    if q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError(f"Triton path supports fp16/bf16 only, got {q.dtype}.")
    if not q.is_cuda:
        raise ValueError("Triton path requires a CUDA/HIP device tensor.")
    head_dim = q.shape[-1]
    if head_dim not in (32, 64, 128):
        raise ValueError(f"Triton path supports head_dim 32/64/128 only, got {head_dim}.")
    scale_value = float(scale) if scale is not None else 1.0 / math.sqrt(head_dim)
    native = diagnostics.load_native()
    q_c, k_c, v_c = (x.contiguous() for x in (q, k, v))
    return native.fixed_block_attention(q_c.unsqueeze(1), k_c.unsqueeze(1), v_c.unsqueeze(1), scale_value,
                                        bool(causal), None)[:, 0]
