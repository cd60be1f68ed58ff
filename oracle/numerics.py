"""Floating-point helpers of the oracle (test infrastructure only)."""
from __future__ import annotations

import numpy as np


def round_bf16(x) -> np.ndarray:
    """Round to bfloat16 (round to nearest even) and return float32 values."""
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    bits = a.view(np.uint32).astype(np.uint64)
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) << 16
    out = rounded.astype(np.uint32).view(np.float32).copy()
    nan = np.isnan(a)
    if nan.any():
        out[nan] = np.nan
    return out


def round_f16(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_dtype(x, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "f16":
        return round_f16(x)
    if dtype == "f32":
        return np.asarray(x, dtype=np.float32)
    raise ValueError(dtype)


def f32(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32)


def softmax_lse(scores: np.ndarray, axis: int = -1) -> tuple[np.ndarray, np.ndarray]:
    """Numerically stable softmax and natural-log LSE (float64); fully -inf rows give 0 and -inf."""
    s = np.asarray(scores, dtype=np.float64)
    m = np.max(s, axis=axis, keepdims=True)
    m_safe = np.where(np.isfinite(m), m, 0.0)
    e = np.exp(s - m_safe)
    z = np.sum(e, axis=axis, keepdims=True)
    with np.errstate(divide="ignore", invalid="ignore"):
        p = np.where(z > 0, e / z, 0.0)
        lse = np.where(z > 0, np.log(z) + m_safe, -np.inf)
    return p, np.squeeze(lse, axis=axis)
