"""fixed_block_attention: the block-diagonal entry point (reference dispatch.py:82-186).

Modes: ``auto`` (HIP kernel when the call is eligible, eager reference with a
reason string otherwise), ``reference`` (always eager) and ``hip`` (same as
auto, but the reason says the kernel was requested).  ``triton`` is accepted
as an alias of ``hip`` so existing callers keep working.

Eligible calls (ROCm device, fp32/fp16/bf16, head_dim 32/64/128,
block_size 64, no autograd) always run the gfx950 kernel, attention masks
included (the reference sends masked calls to its eager loop; the kernel
applies the same 2-D/3-D/4-D masks, reference.py:114-156,186-195); a missing
or failing HIP library raises instead of silently falling back.
"""
from __future__ import annotations

from typing import Any

import torch

from . import diagnostics
from .reference import fixed_block_attention_ref, mask_view_bhtt, normalize_qkv_to_bh_t_d

SUPPORTED_HEAD_DIMS = {32, 64, 128}
SUPPORTED_DTYPES = {torch.float16, torch.bfloat16, torch.float32}
_MODES = {"auto", "reference", "hip", "triton"}


def _fallback(q, k, v, *, block_size, scale, causal, layout, heads, mask, reason, return_diagnostics):
    out = fixed_block_attention_ref(q, k, v, block_size=block_size, scale=scale, causal=causal, layout=layout,
                                    heads=heads, mask=mask)
    info = {"backend": "reference", "fallback_reason": reason, "optimized": False}
    return (out, info) if return_diagnostics else out


def _hip_reject_reason(q_flat: torch.Tensor, k_flat: torch.Tensor, v_flat: torch.Tensor, *, block_size: int,
                       mask: torch.Tensor | None) -> str | None:
    """First reason the HIP kernel cannot take the call, in the reference's order (dispatch.py:50-79)."""
    if mask is not None and not isinstance(mask, torch.Tensor):
        return "mask_is_not_a_tensor"
    if any(t.requires_grad for t in (q_flat, k_flat, v_flat)) or (mask is not None and mask.requires_grad):
        return "requires_grad_uses_reference"
    if block_size != 64:
        return f"unsupported_block_size_{block_size}"
    if q_flat.shape != k_flat.shape or q_flat.shape != v_flat.shape:
        return "qkv_shape_mismatch"
    if q_flat.dtype not in SUPPORTED_DTYPES or k_flat.dtype != q_flat.dtype or v_flat.dtype != q_flat.dtype:
        return f"unsupported_dtype_{q_flat.dtype}"
    if q_flat.shape[-1] not in SUPPORTED_HEAD_DIMS:
        return f"unsupported_head_dim_{q_flat.shape[-1]}"
    if q_flat.device != k_flat.device or q_flat.device != v_flat.device:
        return "qkv_device_mismatch"
    if q_flat.device.type != "cuda":
        return f"not_cuda_or_hip_device_{q_flat.device.type}"
    if not diagnostics.is_rocm_pytorch():
        return "torch_version_hip_not_detected"
    return None


def fixed_block_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, block_size: int = 64,
                          scale: float | None = None, causal: bool = False, layout: str = "auto",
                          heads: int | None = None, mode: str = "auto", allow_approximate: bool = False,
                          return_diagnostics: bool = False, mask: torch.Tensor | None = None) -> Any:
    """Exact fixed block-diagonal attention; returns out (and the diagnostics dict when asked)."""
    del allow_approximate  # the operation is exact for block-diagonal semantics
    if mode not in _MODES:
        raise ValueError("mode must be one of: auto, reference, hip (alias: triton).")
    common = dict(block_size=block_size, scale=scale, causal=causal, layout=layout, heads=heads, mask=mask,
                  return_diagnostics=return_diagnostics)
    if mode == "reference":
        return _fallback(q, k, v, reason="mode_reference", **common)
    try:
        q_flat, k_flat, v_flat, info = normalize_qkv_to_bh_t_d(q, k, v, layout=layout, heads=heads)
    except Exception as exc:
        return _fallback(q, k, v, reason=f"layout_normalization_failed_{type(exc).__name__}: {exc}", **common)
    reason = _hip_reject_reason(q_flat, k_flat, v_flat, block_size=block_size, mask=mask)
    if reason is not None:
        return _fallback(q, k, v, reason=reason if mode == "auto" else f"requested_hip_but_{reason}", **common)

    mask4 = None
    if mask is not None:  # shape errors raise ValueError exactly as the eager loop would
        mask4 = mask_view_bhtt(mask, batch_heads=q_flat.shape[0], info=info, device=q_flat.device)
    native = diagnostics.load_native()
    head_dim = info.head_dim
    s = float(scale) if scale is not None else head_dim ** -0.5
    out_flat = native.fixed_block_attention(q_flat.unsqueeze(1), k_flat.unsqueeze(1), v_flat.unsqueeze(1), s,
                                            causal, mask4)[:, 0]
    out = info.restore(out_flat)
    details = {"backend": "hip", "fallback_reason": None, "optimized": True, "layout": info.layout,
               "tokens": info.tokens, "head_dim": head_dim, "mask": None if mask4 is None else str(mask4.dtype)}
    return (out, details) if return_diagnostics else out
