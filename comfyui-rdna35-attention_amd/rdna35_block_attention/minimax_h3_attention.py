"""MiniMax-H3 interleaved-QKV exact attention.

The H3 model hands attention strided views into one fused projection
[B, T, 3, H, D] (token stride 3*H*D).  The reference
(minimax_h3_gfx1151_attention.py:60-215) repacks K/V (T < 12000) or Q/K/V
(T >= 12000) with one torch.stack and then chains the existing SDPA backend,
because that backend is slow on strided inputs.  The gfx950 dense kernel
reads strided rows directly, so the override here runs it on the views as
they are - no pack copy - and returns the merged [B, T, H*D] output the
original function would have returned.  pack_minimax_h3_qkv is kept with the
reference's profiles for callers that want the packed layout.
"""
from __future__ import annotations

import logging
from typing import Any, Callable

import torch

from . import diagnostics

LOG_PREFIX = "MI355X MiniMax-H3 Attention"
MINIMAX_H3_HEADS = 56
MINIMAX_H3_HEAD_DIM = 128
MINIMAX_H3_MIN_PACK_TOKENS = 4608
MINIMAX_H3_PACK_ALL_TOKENS = 12000
MINIMAX_H3_MAX_PACK_TOKENS = 16500
# The reference stops at 16500 tokens because its packed copies must pay for
# themselves; reading the strided views in place has no copy, so the override
# here takes longer H3 sequences too (MI355X: 2.3x / 1.7x faster than strided
# SDPA at T = 9170 / 16500).
MINIMAX_H3_MAX_TOKENS = 65536


def _fallback_call(previous_override: Callable | None, original_func: Callable, *args, **kwargs):
    if previous_override is not None:
        return previous_override(original_func, *args, **kwargs)
    return original_func(*args, **kwargs)


def _gfx950_device_index() -> tuple[int | None, str | None]:
    if not torch.cuda.is_available() or torch.version.hip is None:
        return None, "PyTorch ROCm device is unavailable"
    try:
        index = torch.cuda.current_device()
        props = torch.cuda.get_device_properties(index)
    except (RuntimeError, AssertionError) as exc:
        return None, f"could not query the current ROCm device ({type(exc).__name__}: {exc})"
    target = str(getattr(props, "gcnArchName", "")).split(":", 1)[0]
    if target != diagnostics.TARGET:
        return None, f"{diagnostics.TARGET} is required, got {target or 'unknown'}"
    return index, None


def _locate_minimax_h3(model: Any) -> Any | None:
    if hasattr(model, "get_model_object"):
        try:
            found = model.get_model_object("diffusion_model")
        except (AttributeError, KeyError):
            found = None
        if found is not None:
            return found
    return getattr(getattr(model, "model", None), "diffusion_model", None)


def _is_native_minimax_h3(model: Any) -> bool:
    found = _locate_minimax_h3(model)
    return (found is not None and type(found).__module__ == "comfy.ldm.minimax.model"
            and type(found).__name__ == "MiniMaxH3Model" and hasattr(found, "blocks")
            and hasattr(found, "hidden_size"))


def minimax_h3_pack_profile(tokens: int) -> str:
    return "qkv" if tokens >= MINIMAX_H3_PACK_ALL_TOKENS else "kv"


def pack_minimax_h3_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    """Contiguous copies in one allocation: K/V below 12000 tokens, Q/K/V from 12000."""
    profile = minimax_h3_pack_profile(q.shape[2])
    if profile == "qkv":
        packed = torch.stack((q, k, v))
        return packed[0], packed[1], packed[2], profile
    packed = torch.stack((k, v))
    return q, packed[0], packed[1], profile


def _reject_reason(q, k, v, heads, mask, skip_reshape, skip_output_reshape, device_index, kwargs) -> str | None:
    if mask is not None:
        return "attention_mask_is_not_supported"
    if not skip_reshape or skip_output_reshape:
        return "minimax_h3_merged_output_contract_is_required"
    if kwargs.get("enable_gqa", False):
        return "gqa_is_not_supported"
    if kwargs.get("is_causal", False) or kwargs.get("causal", False):
        return "causal_attention_is_not_supported"
    if kwargs.get("attn_bias") is not None:
        return "attention_bias_is_not_supported"
    if not all(isinstance(t, torch.Tensor) for t in (q, k, v)):
        return "qkv_are_not_tensors"
    if q.ndim != 4 or q.shape != k.shape or q.shape != v.shape:
        return "matching_bhtd_qkv_are_required"
    if q.shape[0] != 1 or q.shape[1] != MINIMAX_H3_HEADS or heads != MINIMAX_H3_HEADS or q.shape[3] != MINIMAX_H3_HEAD_DIM:
        return "minimax_h3_b1_h56_d128_is_required"
    if q.shape[2] < MINIMAX_H3_MIN_PACK_TOKENS:
        return f"tokens_below_{MINIMAX_H3_MIN_PACK_TOKENS}"
    if q.shape[2] > MINIMAX_H3_MAX_TOKENS:
        return f"tokens_above_{MINIMAX_H3_MAX_TOKENS}"
    if q.dtype != torch.bfloat16 or k.dtype != q.dtype or v.dtype != q.dtype:
        return "matching_bfloat16_qkv_are_required"
    if q.device != k.device or q.device != v.device or q.device.type != "cuda":
        return "matching_rocm_qkv_device_is_required"
    index = q.device.index if q.device.index is not None else torch.cuda.current_device()
    if index != device_index:
        return "qkv_are_not_on_the_validated_gfx950_device"
    if any(t.requires_grad for t in (q, k, v)):
        return "forward_only_requires_grad_not_supported"
    if any(t.stride(3) != 1 for t in (q, k, v)):
        return "contiguous_head_dimension_is_required"
    if any(t.stride(2) % 8 or t.stride(1) % 8 or t.stride(0) % 8 or t.data_ptr() % 16 for t in (q, k, v)):
        return "sixteen_byte_aligned_rows_are_required"
    return None


def make_minimax_h3_attention_override(*, device_index: int, verbose_fallbacks: bool,
                                       previous_override: Callable | None) -> Callable:
    def attention_override(original_func, q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False,
                           skip_output_reshape=False, **kwargs):
        reason = _reject_reason(q, k, v, heads, mask, skip_reshape, skip_output_reshape, device_index, kwargs)
        if reason is not None:
            if verbose_fallbacks:
                logging.info("%s: existing backend used: %s", LOG_PREFIX, reason)
            return _fallback_call(previous_override, original_func, q, k, v, heads, mask=mask,
                                  attn_precision=attn_precision, skip_reshape=skip_reshape,
                                  skip_output_reshape=skip_output_reshape, **kwargs)
        native = diagnostics.load_native()
        scale = kwargs.get("scale")
        s = float(scale) if scale is not None else q.shape[-1] ** -0.5
        if verbose_fallbacks:
            logging.info("%s: strided exact attention at T=%d", LOG_PREFIX, q.shape[2])
        return native.dense_attention(q, k, v, s, merged_output=True)

    return attention_override


def patch_minimax_h3_attention(model, *, enabled: bool, verbose_fallbacks: bool):
    """Install the H3 override on a clone of `model`; returns (model, info string)."""
    if not enabled:
        return model, "disabled; model returned unchanged"
    if not hasattr(model, "clone") or not hasattr(model, "model_options"):
        return model, "MODEL does not expose ComfyUI ModelPatcher clone/model_options; model returned unchanged"
    if not _is_native_minimax_h3(model):
        return model, "native ComfyUI MiniMaxH3Model was not found; model returned unchanged"
    device_index, device_error = _gfx950_device_index()
    if device_index is None:
        return model, f"{device_error}; model returned unchanged"
    previous = model.model_options.get("transformer_options", {}).get("optimized_attention_override")
    if previous is not None and getattr(previous, "container_function", None) is not None:
        return model, "container-aware optimized_attention_override is already installed; model returned unchanged"
    patched = model.clone()
    options = patched.model_options.setdefault("transformer_options", {})
    options["optimized_attention_override"] = make_minimax_h3_attention_override(
        device_index=device_index, verbose_fallbacks=verbose_fallbacks, previous_override=previous)
    info = ("model-local MiniMax-H3 gfx950 exact attention override installed for BF16 B=1,H=56,D=128 with "
            f"{MINIMAX_H3_MIN_PACK_TOKENS}<=T<={MINIMAX_H3_MAX_TOKENS}; strided Q/K/V views are read in place")
    if previous is not None:
        info += "; existing optimized_attention_override is chained for fallback"
    return patched, info


# names of the reference API (minimax_h3_gfx1151_attention.py:124,179)
make_minimax_h3_gfx1151_attention_override = make_minimax_h3_attention_override
patch_minimax_h3_gfx1151_attention = patch_minimax_h3_attention
