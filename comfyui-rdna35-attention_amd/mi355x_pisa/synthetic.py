"""Seeded synthetic workloads for the benchmark and the parity tests.

The PISA configurations are quoted on smooth image/video activations: a
low-frequency Gaussian random field (isotropic, correlation length about 8
tokens) per (batch, head, channel) plus 0.3 * N(0, 1) noise.  The field is
white noise filtered in Fourier space with a Gaussian kernel and normalised
to unit variance.  Everything is generated on the CPU with torch.Generator so
that a seed fixes the tensor bit for bit on every machine.
"""
from __future__ import annotations

import math

import torch


def gaussian_field(shape_grid: tuple[int, ...], channels: int, *, sigma: float = 8.0, noise: float = 0.3,
                   seed: int = 0, leading: tuple[int, ...] = ()) -> torch.Tensor:
    """Field of shape [*leading, prod(shape_grid), channels] (float32, raster token order)."""
    gen = torch.Generator().manual_seed(seed)
    n_tokens = math.prod(shape_grid)
    batch = math.prod(leading) if leading else 1
    white = torch.randn((batch, channels, *shape_grid), generator=gen, dtype=torch.float32)
    spec = torch.fft.fftn(white, dim=tuple(range(2, 2 + len(shape_grid))))
    kernel = torch.ones(shape_grid, dtype=torch.float32)
    for axis, size in enumerate(shape_grid):
        freq = torch.fft.fftfreq(size)
        gain = torch.exp(-0.5 * (2.0 * math.pi * freq * sigma) ** 2)
        view = [1] * len(shape_grid)
        view[axis] = size
        kernel = kernel * gain.view(view)
    field = torch.fft.ifftn(spec * kernel, dim=tuple(range(2, 2 + len(shape_grid)))).real
    field = field.reshape(batch, channels, n_tokens)
    field = (field - field.mean(dim=-1, keepdim=True)) / field.std(dim=-1, keepdim=True).clamp_min(1e-6)
    field = field + noise * torch.randn(field.shape, generator=gen, dtype=torch.float32)
    return field.transpose(1, 2).contiguous().reshape(*leading, n_tokens, channels)


def anima_qkv(batch: int = 2, heads: int = 16, side: int = 96, head_dim: int = 128, seed: int = 0,
              dtype: torch.dtype = torch.bfloat16, device: str | torch.device = "cpu"):
    """q, k, v as BHTD views of contiguous [B, side*side, H, D] raster storage (the Anima layout)."""
    tensors = []
    for offset in range(3):
        field = gaussian_field((side, side), heads * head_dim, seed=seed * 3 + offset + 1, leading=(batch,))
        bthd = field.reshape(batch, side * side, heads, head_dim).to(dtype).contiguous().to(device)
        tensors.append(bthd.permute(0, 2, 1, 3))
    return tuple(tensors)


def video_qkv(batch: int = 1, heads: int = 40, grid: tuple[int, int, int] = (16, 32, 64), head_dim: int = 128,
              seed: int = 0, dtype: torch.dtype = torch.bfloat16, device: str | torch.device = "cpu"):
    """q, k, v as BHTD views of contiguous [B, F*H*W, heads, D] raster storage."""
    tensors = []
    tokens = math.prod(grid)
    for offset in range(3):
        field = gaussian_field(grid, heads * head_dim, seed=seed * 3 + offset + 1, leading=(batch,))
        bthd = field.reshape(batch, tokens, heads, head_dim).to(dtype).contiguous().to(device)
        tensors.append(bthd.permute(0, 2, 1, 3))
    return tuple(tensors)


def normal_qkv(shape: tuple[int, ...], *, seed: int = 0, scale: float = 1.0, dtype: torch.dtype = torch.bfloat16,
               device: str | torch.device = "cpu"):
    """Three independent N(0, scale^2) tensors of the given shape."""
    gen = torch.Generator().manual_seed(seed)
    return tuple((scale * torch.randn(shape, generator=gen)).to(dtype).to(device) for _ in range(3))
