"""Model-local optimized_attention_override for fixed block-diagonal attention.

Behaviour of the reference's comfy_patch.py (:14-203): the override acts only
on calls marked ``rdna35_attention_semantics="fixed_block_diagonal"`` (or, in
``experimental_force_block_local`` mode, on calls that declare or prove
self-attention), runs fixed_block_attention, and otherwise chains the
previously installed override or ComfyUI's original function.  It is
installed on a clone of the ModelPatcher, never globally.
"""
from __future__ import annotations

import logging
from typing import Any, Callable

import torch

from .diagnostics import NativeUnavailableError
from .dispatch import fixed_block_attention
from .gates import chain as _fallback_call

LOG_PREFIX = "MI355X FixedBlockAttention"


def _options(kwargs: dict[str, Any]) -> dict:
    return kwargs.get("transformer_options") or {}


def _has_fixed_block_marker(kwargs: dict[str, Any]) -> bool:
    marker = "fixed_block_diagonal"
    return kwargs.get("rdna35_attention_semantics") == marker or \
        _options(kwargs).get("rdna35_attention_semantics") == marker


def _declares_self_attention(q, k, v, kwargs: dict[str, Any]) -> bool:
    if kwargs.get("rdna35_is_self_attention") is True or _options(kwargs).get("rdna35_is_self_attention") is True:
        return True
    try:
        return q.data_ptr() == k.data_ptr() == v.data_ptr()
    except Exception:
        return False


def _format_call_reason(info: dict[str, Any]) -> str:
    reason = info.get("fallback_reason")
    return f"{info.get('backend')}: {reason}" if reason else str(info.get("backend"))


def make_attention_override(*, mode: str, semantic_mode: str, block_size: int, causal: bool, verbose_fallbacks: bool,
                            previous_override: Callable | None) -> Callable:
    def attention_override(original_func, q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False,
                           skip_output_reshape=False, **kwargs):
        def passthrough(note: str):
            if verbose_fallbacks:
                logging.info("%s: original attention used; %s", LOG_PREFIX, note)
            return _fallback_call(previous_override, original_func, q, k, v, heads, mask=mask,
                                  attn_precision=attn_precision, skip_reshape=skip_reshape,
                                  skip_output_reshape=skip_output_reshape, **kwargs)

        marked = _has_fixed_block_marker(kwargs)
        if not marked:
            if semantic_mode != "experimental_force_block_local":
                return passthrough("call is not proven fixed block-diagonal self-attention.")
            if not _declares_self_attention(q, k, v, kwargs):
                return passthrough("experimental mode could not prove self-attention.")
        try:
            if skip_reshape:
                out, info = fixed_block_attention(q, k, v, block_size=block_size, causal=causal, layout="bhtd",
                                                  mode=mode, return_diagnostics=True, mask=mask)
                if not skip_output_reshape:
                    b, h, t, d = out.shape
                    out = out.transpose(1, 2).contiguous().reshape(b, t, h * d)
            else:
                out, info = fixed_block_attention(q, k, v, block_size=block_size, causal=causal, layout="bthd",
                                                  heads=heads, mode=mode, return_diagnostics=True, mask=mask)
                if skip_output_reshape:
                    b, t, channels = out.shape
                    out = out.reshape(b, t, heads, channels // heads).permute(0, 2, 1, 3).contiguous()
        except Exception as exc:
            if isinstance(exc, (torch.OutOfMemoryError, NativeUnavailableError)):
                raise
            logging.warning("%s: fixed block attention failed; original attention used: %s: %s", LOG_PREFIX,
                            type(exc).__name__, exc)
            return _fallback_call(previous_override, original_func, q, k, v, heads, mask=mask,
                                  attn_precision=attn_precision, skip_reshape=skip_reshape,
                                  skip_output_reshape=skip_output_reshape, **kwargs)
        if verbose_fallbacks and info.get("fallback_reason"):
            logging.info("%s: %s", LOG_PREFIX, _format_call_reason(info))
        return out

    return attention_override


def patch_model_attention(model, *, enabled: bool, mode: str, semantic_mode: str, block_size: int, causal: bool,
                          verbose_fallbacks: bool):
    """Clone `model` and install the override on the clone; returns (model, info string)."""
    if not enabled:
        return model, "disabled; model returned unchanged"
    if block_size != 64:
        return model, f"unsupported block_size={block_size}; only 64 is implemented, model returned unchanged"
    if semantic_mode not in {"exact_only", "experimental_force_block_local"}:
        return model, f"unsupported semantic_mode={semantic_mode}; model returned unchanged"
    if not hasattr(model, "clone") or not hasattr(model, "model_options"):
        return model, "MODEL does not expose ComfyUI ModelPatcher clone/model_options; model returned unchanged"
    patched = model.clone()
    options = patched.model_options.setdefault("transformer_options", {})
    previous = options.get("optimized_attention_override")
    options["optimized_attention_override"] = make_attention_override(
        mode=mode, semantic_mode=semantic_mode, block_size=block_size, causal=causal,
        verbose_fallbacks=verbose_fallbacks, previous_override=previous)
    if semantic_mode == "exact_only":
        info = ("model-local optimized_attention_override installed in exact_only mode; normal ComfyUI attention "
                "calls are left unchanged unless they explicitly declare "
                "rdna35_attention_semantics='fixed_block_diagonal'")
    else:
        info = ("model-local optimized_attention_override installed in experimental_force_block_local mode; only "
                "calls explicitly marked as fixed block-diagonal or self-attention are eligible; unproven calls fall "
                "back to the original attention backend")
    if previous is not None:
        info += "; existing optimized_attention_override is chained for fallback"
    return patched, info
