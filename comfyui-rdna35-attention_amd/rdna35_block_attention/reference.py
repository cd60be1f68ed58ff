"""Layout normalisation and the eager ("reference" backend) implementations.

Public names and behaviour follow the reference's reference.py:
normalize_qkv_to_bh_t_d (:38-111), per-block mask slicing (:114-156),
fixed_block_attention_ref (:159-200), fixed_block_attention_bthd (:203-224),
block_diagonal_sdpa_mask (:227-241), fixed_block_attention_sdpa (:244-272)
and full_attention_sdpa_bhtd (:275-293).  These eager versions serve the
calls the HIP kernels do not take (masks, CPU tensors, unsupported shapes)
and the explicit ``mode="reference"``; eligible ROCm calls never use them.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable

import torch

_LAYOUT_ALIASES = {
    "auto": "auto",
    "bhtd": "bhtd",
    "b,h,t,d": "bhtd",
    "bh_t_d": "bh_t_d",
    "bhtd_flat": "bh_t_d",
    "bhtdflat": "bh_t_d",
    "bthd": "bthd",
    "b,t,h*d": "bthd",
    "b_t_hd": "bthd",
}


@dataclass(frozen=True)
class LayoutInfo:
    layout: str
    batch: int | None
    heads: int | None
    tokens: int
    head_dim: int
    restore: Callable[[torch.Tensor], torch.Tensor]


def _canonical_layout(layout: str) -> str:
    key = layout.lower().replace("-", "_").replace(" ", "")
    if key not in _LAYOUT_ALIASES:
        raise ValueError(f"Unsupported layout '{layout}'.")
    return _LAYOUT_ALIASES[key]


# Rank and shape wording of each canonical layout (the accepted layouts and their errors
# are the reference's interface, reference.py:38-111).
_LAYOUT_RANK = {"bhtd": 4, "bh_t_d": 3, "bthd": 3}
_LAYOUT_SHAPE = {"bhtd": "[B,H,T,D]", "bh_t_d": "[BH,T,D]", "bthd": "[B,T,H*D]"}


def _bhtd_view(x: torch.Tensor, layout: str, heads: int | None) -> torch.Tensor:
    """x in `layout` as a [B, H, T, D] tensor (a view where the strides allow; flat [BH,T,D] is B = 1)."""
    if layout == "bhtd":
        return x
    if layout == "bh_t_d":
        return x.unsqueeze(0)
    b, t, channels = x.shape
    return x.reshape(b, t, heads, channels // heads).permute(0, 2, 1, 3)


def normalize_qkv_to_bh_t_d(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, layout: str = "auto",
                            heads: int | None = None):
    """Flatten q/k/v to contiguous [B*H, T, D]; returns (q, k, v, LayoutInfo with restore()).

    Every layout is first seen as [B, H, T, D] (_bhtd_view); restore() maps a [B*H, T, D] result back to
    the caller's layout and shape.  LayoutInfo reports B and H where the layout defines them.
    """
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError(
            f"Fixed block self-attention requires q/k/v to have identical shapes, got {q.shape}, {k.shape}, {v.shape}.")
    chosen = _canonical_layout(layout)
    if chosen == "auto":
        chosen = {4: "bhtd", 3: "bh_t_d"}.get(q.ndim, "")
        if not chosen:
            raise ValueError(f"Cannot infer layout for rank-{q.ndim} tensor.")
    if q.ndim != _LAYOUT_RANK[chosen]:
        raise ValueError(f"layout='{chosen}' expects {_LAYOUT_SHAPE[chosen]}, got rank {q.ndim}.")
    if chosen == "bthd":
        if heads is None or heads <= 0:
            raise ValueError("layout='bthd' requires a positive heads argument.")
        if q.shape[-1] % heads:
            raise ValueError(f"channels={q.shape[-1]} is not divisible by heads={heads}.")
    views = [_bhtd_view(x, chosen, heads) for x in (q, k, v)]
    b, h, t, d = views[0].shape
    flat = [x.reshape(b * h, t, d).contiguous() for x in views]
    caller_shape = q.shape

    def restore(out: torch.Tensor) -> torch.Tensor:
        out4 = out.reshape(b, h, t, d)
        if chosen == "bthd":
            out4 = out4.permute(0, 2, 1, 3)
        return out4.contiguous().reshape(caller_shape)

    known = chosen != "bh_t_d"
    return (*flat, LayoutInfo(chosen, b if known else None, h if known else None, t, d, restore))


def mask_view_bhtt(mask: torch.Tensor, *, batch_heads: int, info: LayoutInfo,
                   device: torch.device) -> torch.Tensor:
    """The whole mask as a [B', H', T, T] broadcast view with B' * H' = BH, row bh = b' * H' + h'.

    The one statement of the mask shape rules (the accepted shapes and errors
    of reference.py:114-156): the HIP fixed-block kernel reads this view (zero
    strides for broadcast dims) and the eager path reads its diagonal blocks
    (_diagonal_blocks, _mask_block).  Masks that are neither bool nor fp32/fp16/bf16 become
    fp32, the dtype they are added in.
    """
    m = mask.to(device=device)
    if m.dtype != torch.bool and m.dtype not in (torch.float32, torch.float16, torch.bfloat16):
        m = m.to(torch.float32)
    tokens = info.tokens
    square = (tokens, tokens)
    if m.ndim == 2:
        if tuple(m.shape[-2:]) != square:
            raise ValueError(f"2D mask must have shape [T,T], got {tuple(m.shape)}.")
        return m.view(1, 1, tokens, tokens).expand(batch_heads, 1, tokens, tokens)
    if m.ndim == 3:
        if tuple(m.shape[-2:]) != square:
            raise ValueError(f"3D mask must end with [T,T], got {tuple(m.shape)}.")
        lead = m.shape[0]
        if info.batch is not None and lead == info.batch:
            return m.unsqueeze(1).expand(info.batch, info.heads, tokens, tokens)
        if lead == 1:
            return m.unsqueeze(1).expand(batch_heads, 1, tokens, tokens)
        if lead == batch_heads:
            return m.unsqueeze(1)
        raise ValueError(f"3D mask batch dimension {lead} is not compatible with BH={batch_heads}.")
    if m.ndim == 4:
        if info.batch is None or info.heads is None:
            raise ValueError("4D mask requires a layout with known B and H.")
        if tuple(m.shape[-2:]) != square:
            raise ValueError(f"4D mask must end with [T,T], got {tuple(m.shape)}.")
        if m.shape[0] not in (1, info.batch):
            raise ValueError(f"4D mask batch dimension {m.shape[0]} is not compatible with B={info.batch}.")
        if m.shape[1] not in (1, info.heads):
            raise ValueError(f"4D mask head dimension {m.shape[1]} is not compatible with H={info.heads}.")
        return m.expand(info.batch, info.heads, tokens, tokens)
    raise ValueError(f"Unsupported mask rank {m.ndim}.")


def _mask_block(mask: torch.Tensor | None, start: int, end: int, *, batch_heads: int, info: LayoutInfo,
                device: torch.device) -> torch.Tensor | None:
    """The [BH, n, n] diagonal block of mask_view_bhtt's view for tokens [start, end)."""
    if mask is None:
        return None
    n = end - start
    view = mask_view_bhtt(mask, batch_heads=batch_heads, info=info, device=device)
    return view[:, :, start:end, start:end].reshape(batch_heads, n, n)


def _diagonal_blocks(view: torch.Tensor, start: int, count: int, size: int) -> torch.Tensor:
    """[B', H', count, size, size]: the diagonal blocks of a [B', H', T, T] view starting at token `start`.

    One strided view (block j begins size * (query stride + key stride) elements after block j-1);
    nothing is copied, broadcast dims keep their zero strides.
    """
    sub = view[:, :, start:, start:]
    sb, sh, sq, sk = sub.stride()
    return sub.as_strided((sub.shape[0], sub.shape[1], count, size, size), (sb, sh, size * (sq + sk), sq, sk),
                          sub.storage_offset())


_SCORE_BUDGET = 1 << 24  # fp32 scores materialised at once by the eager path (64 MiB)


def fixed_block_attention_ref(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_size: int = 64,
                              scale: float | None = None, causal: bool = False, layout: str = "auto", *,
                              heads: int | None = None, mask: torch.Tensor | None = None) -> torch.Tensor:
    """Eager fixed block-diagonal attention: every block of `block_size` tokens attends to itself.

    fp32 scores, softmax and products, output in the input dtype (reference.py:159-200); the short last
    block has T mod block_size tokens.  Equal-size blocks run as one batched product over
    [BH, blocks, size, D] (in groups that keep the scores within _SCORE_BUDGET), with the causal mask and
    the diagonal blocks of the caller's mask (mask_view_bhtt) applied to the scores.
    """
    qf, kf, vf, info = normalize_qkv_to_bh_t_d(q, k, v, layout=layout, heads=heads)
    if block_size <= 0:
        raise ValueError("block_size must be positive.")
    bh, tokens, head_dim = qf.shape
    s = float(scale) if scale is not None else 1.0 / math.sqrt(head_dim)
    view = None if mask is None else mask_view_bhtt(mask, batch_heads=bh, info=info, device=q.device)
    out = torch.empty_like(qf)
    full, tail = divmod(tokens, block_size)
    runs = [(0, full, block_size)] if full else []
    if tail:
        runs.append((full * block_size, 1, tail))
    for first, count, size in runs:
        group = max(1, _SCORE_BUDGET // (bh * size * size))
        upper = torch.ones((size, size), dtype=torch.bool, device=q.device).triu(1) if causal else None
        for j0 in range(0, count, group):
            n = min(group, count - j0)
            lo = first + j0 * size
            hi = lo + n * size
            qb, kb, vb = (x[:, lo:hi].float().reshape(bh, n, size, head_dim) for x in (qf, kf, vf))
            scores = torch.matmul(qb, kb.transpose(-2, -1)) * s
            if upper is not None:
                scores = scores.masked_fill(upper, -torch.inf)
            if view is not None:
                blocks = _diagonal_blocks(view, lo, n, size).reshape(bh, n, size, size)
                if blocks.dtype == torch.bool:
                    scores = scores.masked_fill(~blocks, -torch.inf)
                else:
                    scores = scores + blocks.to(scores.dtype)
            out[:, lo:hi] = torch.matmul(torch.softmax(scores, dim=-1), vb).reshape(bh, n * size, head_dim).to(qf.dtype)
    return info.restore(out)


def fixed_block_attention_bthd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, heads: int, block_size: int = 64,
                               scale: float | None = None, causal: bool = False, *,
                               mask: torch.Tensor | None = None) -> torch.Tensor:
    return fixed_block_attention_ref(q, k, v, block_size=block_size, scale=scale, causal=causal, layout="bthd",
                                     heads=heads, mask=mask)


def block_diagonal_sdpa_mask(tokens: int, *, block_size: int = 64, causal: bool = False,
                             device: torch.device | None = None) -> torch.Tensor:
    if block_size <= 0:
        raise ValueError("block_size must be positive.")
    pos = torch.arange(tokens, device=device)
    mask = (pos[:, None] // block_size) == (pos[None, :] // block_size)
    if causal:
        mask = mask & (pos[None, :] <= pos[:, None])
    return mask


def fixed_block_attention_sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, block_size: int = 64,
                               scale: float | None = None, causal: bool = False, layout: str = "auto", *,
                               heads: int | None = None) -> torch.Tensor:
    qf, kf, vf, info = normalize_qkv_to_bh_t_d(q, k, v, layout=layout, heads=heads)
    mask = block_diagonal_sdpa_mask(info.tokens, block_size=block_size, causal=causal, device=qf.device)
    extra = {} if scale is None else {"scale": float(scale)}
    out = torch.nn.functional.scaled_dot_product_attention(qf[:, None], kf[:, None], vf[:, None], attn_mask=mask,
                                                           dropout_p=0.0, is_causal=False, **extra)[:, 0]
    return info.restore(out.to(qf.dtype))


def full_attention_sdpa_bhtd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, scale: float | None = None,
                             causal: bool = False) -> torch.Tensor:
    extra = {} if scale is None else {"scale": float(scale)}
    return torch.nn.functional.scaled_dot_product_attention(q, k, v, dropout_p=0.0, is_causal=causal, **extra)
