"""Exact and fixed block-diagonal attention oracles (test infrastructure only)."""
from __future__ import annotations

import math

import numpy as np

from .numerics import round_dtype, softmax_lse


def dense_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float | None = None,
                    out_dtype: str = "f32", return_lse: bool = False):
    """softmax(s q k^T) v over the last two axes, float64 math.

    Semantics of full_attention_sdpa_bhtd (reference.py:275-293) and of the
    online-softmax kernel (triton_kernel.py:113-160): non-causal, no mask,
    q_tokens and kv_tokens independent.
    """
    q64 = np.asarray(q, dtype=np.float64)
    k64 = np.asarray(k, dtype=np.float64)
    v64 = np.asarray(v, dtype=np.float64)
    s = 1.0 / math.sqrt(q64.shape[-1]) if scale is None else float(scale)
    scores = np.matmul(q64, np.swapaxes(k64, -1, -2)) * s
    p, lse = softmax_lse(scores)
    out = round_dtype(np.matmul(p, v64), out_dtype)
    return (out, lse) if return_lse else out


def fixed_block_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, block_size: int = 64,
                          scale: float | None = None, causal: bool = False, out_dtype: str = "f32",
                          mask: np.ndarray | None = None, prob_dtype: str | None = None) -> np.ndarray:
    """Block loop of fixed_block_attention_ref (reference.py:159-200) on [..., T, D] arrays.

    Each block of block_size tokens attends only to itself (the last block
    may be shorter); causal masks keys after the query inside the block.
    `mask` ([..., T, T], broadcastable to q's leading axes) is applied after
    the causal fill (reference.py:190-195): bool keeps a score where True
    (-inf elsewhere), any other dtype is added to the scaled score.  A row
    with every score -inf gives NaN, the value torch.softmax returns.
    Scores, softmax and P@V in float64; output rounded to out_dtype.
    prob_dtype rounds the normalised probabilities before P@V: the Triton
    kernel's `probs.to(v.dtype)` (triton_kernel.py:92-96), used for fp16/bf16.
    """
    q64 = np.asarray(q, dtype=np.float64)
    k64 = np.asarray(k, dtype=np.float64)
    v64 = np.asarray(v, dtype=np.float64)
    tokens, head_dim = q64.shape[-2:]
    s = 1.0 / math.sqrt(head_dim) if scale is None else float(scale)
    out = np.empty(q64.shape, dtype=np.float64)
    for start in range(0, tokens, block_size):
        end = min(start + block_size, tokens)
        scores = np.matmul(q64[..., start:end, :], np.swapaxes(k64[..., start:end, :], -1, -2)) * s
        if causal:
            n = end - start
            scores = np.where(np.triu(np.ones((n, n), dtype=bool), 1), -np.inf, scores)
        if mask is not None:
            part = np.asarray(mask)[..., start:end, start:end]
            if part.dtype == np.bool_:
                scores = np.where(part, scores, -np.inf)
            else:
                scores = scores + part.astype(np.float64)
        p, _ = softmax_lse(scores)
        dead = np.all(np.isneginf(scores), axis=-1, keepdims=True)
        p = np.where(dead, np.nan, p)
        if prob_dtype is not None:
            p = round_dtype(p, prob_dtype).astype(np.float64)
        out[..., start:end, :] = np.matmul(p, v64[..., start:end, :])
    return round_dtype(out, out_dtype)


def block_diagonal_mask(tokens: int, block_size: int = 64, causal: bool = False) -> np.ndarray:
    """Boolean [T, T] mask of block_diagonal_sdpa_mask (reference.py:227-241)."""
    pos = np.arange(tokens)
    ids = pos // block_size
    mask = ids[:, None] == ids[None, :]
    if causal:
        mask &= pos[None, :] <= pos[:, None]
    return mask
