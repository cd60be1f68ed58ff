"""Helpers shared by the tests (oracle adapters, tensor conversions)."""
from __future__ import annotations

import numpy as np
import torch

from oracle import layout as olayout


def np32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def dtype_name(dtype: torch.dtype) -> str:
    return {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[dtype]


def spatial_to_packed(x_bhtd: torch.Tensor, frames: int, height: int, width: int) -> np.ndarray:
    """[B,H,T,D] raster tensor -> oracle [B*H, T, D] block-major float32 array."""
    b, h, t, d = x_bhtd.shape
    order = olayout.tile_order(frames, height, width)
    return olayout.pack(np32(x_bhtd).reshape(b * h, t, d), order)


def packed_to_merged(out: np.ndarray, batch: int, heads: int, frames: int, height: int, width: int) -> np.ndarray:
    """oracle [B*H, T, D] block-major output -> [B, T, H*D] raster."""
    bh, t, d = out.shape
    order = olayout.tile_order(frames, height, width)
    raster = olayout.unpack(out, order).reshape(batch, heads, t, d)
    return raster.transpose(0, 2, 1, 3).reshape(batch, t, heads * d)


def assert_close(actual, expected, atol, rtol, msg=""):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, (a.shape, e.shape)
    same = (a == e) | (np.isnan(a) & np.isnan(e))  # equal infinities and NaN positions
    with np.errstate(invalid="ignore"):
        bad = ~(same | (np.abs(a - e) <= atol + rtol * np.abs(e)))
    if bad.any():
        idx = np.argwhere(bad)[:5]
        worst = np.max(np.abs(a - e)[bad])
        raise AssertionError(f"{msg} {bad.sum()} / {a.size} elements differ (max abs {worst:.4g}); first {idx.tolist()}")
