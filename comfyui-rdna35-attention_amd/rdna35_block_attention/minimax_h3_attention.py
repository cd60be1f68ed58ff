"""MiniMax-H3 interleaved-QKV exact attention.

The H3 model hands attention strided views into one fused projection
[B, T, 3, H, D] (token stride 3*H*D).  The reference
(minimax_h3_gfx1151_attention.py:60-215) repacks K/V (T < 12000) or Q/K/V
(T >= 12000) with one torch.stack and then chains the existing SDPA backend,
because that backend is slow on strided inputs.  The gfx950 dense kernel
reads strided rows directly, so the override here runs it on the views as
they are - no pack copy - and returns the merged [B, T, H*D] output the
original function would have returned.  The names, signatures, profiles and
reason strings are the reference's; eligibility is the rule table
gates.H3_OVERRIDE_RULES.  pack_minimax_h3_qkv keeps the reference's packed
layout for callers that want it.
"""
from __future__ import annotations

import logging
from typing import Any, Callable

import torch

from . import diagnostics, gates

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
_H3_MODEL = ("comfy.ldm.minimax.model", "MiniMaxH3Model")

# looked up at call time, so tests and hosts can substitute the device gate
_gfx950_device_index = diagnostics.gfx950_device_index


def _diffusion_model(model: Any) -> Any | None:
    """The patcher's diffusion model object, through get_model_object or model.diffusion_model."""
    getter = getattr(model, "get_model_object", None)
    if getter is not None:
        try:
            found = getter("diffusion_model")
        except (AttributeError, KeyError):
            found = None
        if found is not None:
            return found
    return getattr(getattr(model, "model", None), "diffusion_model", None)


def _is_native_minimax_h3(model: Any) -> bool:
    found = _diffusion_model(model)
    if found is None:
        return False
    kind = type(found)
    return (kind.__module__, kind.__name__) == _H3_MODEL and hasattr(found, "blocks") and hasattr(found, "hidden_size")


def minimax_h3_pack_profile(tokens: int) -> str:
    return "qkv" if tokens >= MINIMAX_H3_PACK_ALL_TOKENS else "kv"


def pack_minimax_h3_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    """Contiguous copies sharing one allocation: K/V below 12000 tokens (q passed through), Q/K/V from 12000."""
    profile = minimax_h3_pack_profile(q.shape[2])
    members = (q, k, v) if profile == "qkv" else (k, v)
    packed = torch.stack(members).unbind(0)
    if profile == "qkv":
        return (*packed, profile)
    return (q, *packed, profile)


def _reject_reason(q, k, v, heads, mask, skip_reshape, skip_output_reshape, device_index, kwargs) -> str | None:
    call = gates.Call(q, k, v, heads, mask, None, skip_reshape, skip_output_reshape, kwargs,
                      {"heads": MINIMAX_H3_HEADS, "head_dim": MINIMAX_H3_HEAD_DIM,
                       "min_tokens": MINIMAX_H3_MIN_PACK_TOKENS, "max_tokens": MINIMAX_H3_MAX_TOKENS,
                       "device_index": device_index})
    return gates.first_failure(gates.H3_OVERRIDE_RULES, call)


def make_minimax_h3_attention_override(*, device_index: int, verbose_fallbacks: bool,
                                       previous_override: Callable | None) -> Callable:
    def attention_override(original_func, q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False,
                           skip_output_reshape=False, **kwargs):
        reason = _reject_reason(q, k, v, heads, mask, skip_reshape, skip_output_reshape, device_index, kwargs)
        if reason is not None:
            if verbose_fallbacks:
                logging.info("%s: existing backend used: %s", LOG_PREFIX, reason)
            return gates.chain(previous_override, original_func, q, k, v, heads, mask=mask,
                               attn_precision=attn_precision, skip_reshape=skip_reshape,
                               skip_output_reshape=skip_output_reshape, **kwargs)
        scale = kwargs.get("scale")
        if verbose_fallbacks:
            logging.info("%s: strided exact attention at T=%d", LOG_PREFIX, q.shape[2])
        return diagnostics.load_native().dense_attention(
            q, k, v, q.shape[-1] ** -0.5 if scale is None else float(scale), merged_output=True)

    return attention_override


def patch_minimax_h3_attention(model, *, enabled: bool, verbose_fallbacks: bool):
    """Install the H3 override on a clone of `model`; returns (model, info string)."""
    if not enabled:
        return model, "disabled; model returned unchanged"
    if not (hasattr(model, "clone") and hasattr(model, "model_options")):
        return model, "MODEL does not expose ComfyUI ModelPatcher clone/model_options; model returned unchanged"
    if not _is_native_minimax_h3(model):
        return model, "native ComfyUI MiniMaxH3Model was not found; model returned unchanged"
    device_index, device_error = _gfx950_device_index()
    if device_index is None:
        return model, f"{device_error}; model returned unchanged"
    previous = model.model_options.get("transformer_options", {}).get("optimized_attention_override")
    if getattr(previous, "container_function", None) is not None:
        return model, "container-aware optimized_attention_override is already installed; model returned unchanged"
    patched = model.clone()
    patched.model_options.setdefault("transformer_options", {})["optimized_attention_override"] = \
        make_minimax_h3_attention_override(device_index=device_index, verbose_fallbacks=verbose_fallbacks,
                                           previous_override=previous)
    info = ("model-local MiniMax-H3 gfx950 exact attention override installed for BF16 B=1,H=56,D=128 with "
            f"{MINIMAX_H3_MIN_PACK_TOKENS}<=T<={MINIMAX_H3_MAX_TOKENS}; strided Q/K/V views are read in place")
    if previous is not None:
        info += "; existing optimized_attention_override is chained for fallback"
    return patched, info


# names of the reference API (minimax_h3_gfx1151_attention.py:124,179)
make_minimax_h3_gfx1151_attention_override = make_minimax_h3_attention_override
patch_minimax_h3_gfx1151_attention = patch_minimax_h3_attention
