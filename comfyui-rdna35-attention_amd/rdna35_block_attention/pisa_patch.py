"""PISA installer for ComfyUI models: Anima direct patch, Anima override, generic override.

Interface of the reference's pisa_patch.py (:28-284): the same function names,
signatures, token policies, reason strings and info strings.
patch_model_pisa_attention works on a clone of the ModelPatcher and picks one
of three installations:

* a validated Anima model (28 blocks of H=16, D=128 self-attention) gets the
  direct ``attn_op`` object patch on layers start..end, with exact blocks
  ceil(budget * 144), which the native op must list in
  capabilities()["spatial_sparse_exact_blocks"];
* an Anima-like patcher without object patches gets the Anima
  ``optimized_attention_override`` (make_pisa_attention_override);
* any other model gets the generic T >= 8192 override.

The override's eligibility is the rule table gates.ANIMA_OVERRIDE_RULES; an
ineligible call goes to the previously installed override (or ComfyUI's own
function), an eligible call's native failure propagates.
"""
from __future__ import annotations

import logging
import math
from typing import Callable

from . import diagnostics, gates
from .anima_pisa_integration import (
    ANIMA_PISA_FIRST_LAYER,
    ANIMA_PISA_LAST_LAYER,
    install_anima_pisa_attention,
    validate_anima_pisa_model,
)
from .generic_pisa import make_generic_pisa_override
from .pisa_runtime import PISA_RUNTIME_ATTACHMENT, PISARuntimeState

LOG_PREFIX = "MI355X PISA"
TOKEN_POLICIES = {
    "anima_1536_spatial": frozenset((9216,)),
    "auto_9216": frozenset((9216,)),
}
SPATIAL_BLOCK_EDGE = 8
ANIMA_TOKEN_SHAPE = (1, 96, 96)
ANIMA_BLOCKS = 144

# looked up at call time, so tests and hosts can substitute the device gate
_gfx950_device_index = diagnostics.gfx950_device_index

_UNCHANGED = "; model returned unchanged"


def _exact_blocks(tokens: int, exact_budget: float) -> int:
    total = math.ceil(tokens / 64)
    return min(total, math.ceil(exact_budget * total))


def _pisa_reject_reason(q, k, v, heads, mask, attn_precision, skip_reshape, skip_output_reshape,
                        allowed_tokens: frozenset, expected_token_shape: tuple, device_index: int,
                        kwargs: dict) -> str | None:
    """First reason the Anima override cannot take the call (rules of pisa_patch.py:61-116)."""
    call = gates.Call(q, k, v, heads, mask, attn_precision, skip_reshape, skip_output_reshape, kwargs,
                      {"allowed_tokens": allowed_tokens, "token_shape": tuple(expected_token_shape),
                       "device_index": device_index})
    return gates.first_failure(gates.ANIMA_OVERRIDE_RULES, call)


def make_pisa_attention_override(*, exact_budget: float, allowed_tokens: frozenset, expected_token_shape: tuple,
                                 device_index: int, native_forward: Callable, verbose_fallbacks: bool,
                                 previous_override: Callable | None) -> Callable:
    def attention_override(original_func, q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False,
                           skip_output_reshape=False, **kwargs):
        reason = _pisa_reject_reason(q, k, v, heads, mask, attn_precision, skip_reshape, skip_output_reshape,
                                     allowed_tokens, expected_token_shape, device_index, kwargs)
        if reason is None:
            return native_forward(q, k, v, _exact_blocks(q.shape[-2], exact_budget), scale=kwargs.get("scale"))
        if verbose_fallbacks:
            logging.info("%s: original attention used: %s", LOG_PREFIX, reason)
        return gates.chain(previous_override, original_func, q, k, v, heads, mask=mask,
                           attn_precision=attn_precision, skip_reshape=skip_reshape,
                           skip_output_reshape=skip_output_reshape, **kwargs)

    return attention_override


def _arguments_problem(model, exact_budget, token_policy, start_layer, end_layer) -> str | None:
    checks = (
        (0.0 <= exact_budget <= 1.0, f"invalid exact_budget={exact_budget}"),
        (token_policy in TOKEN_POLICIES, f"unsupported token_policy={token_policy}"),
        (0 <= start_layer <= end_layer < 28, f"invalid Anima layer range {start_layer}:{end_layer}"),
        (hasattr(model, "clone") and hasattr(model, "model_options"),
         "MODEL does not expose ComfyUI ModelPatcher clone/model_options"),
    )
    return next((message for ok, message in checks if not ok), None)


def _is_validated_anima(model) -> bool:
    if not (hasattr(model, "get_model_object") and hasattr(model, "add_object_patch")):
        return False
    try:
        validate_anima_pisa_model(model)
    except (AttributeError, TypeError, ValueError):
        return False
    return True


def _set_override(patched, make: Callable) -> bool:
    """Install make(previous) as the clone's override; True when one was already there (it is chained)."""
    options = patched.model_options.setdefault("transformer_options", {})
    previous = options.get("optimized_attention_override")
    options["optimized_attention_override"] = make(previous)
    return previous is not None


def _chained(info: str, chained: bool) -> str:
    return info + ("; existing optimized_attention_override is chained for fallback" if chained else "")


def _install_generic(model, exact_budget: float, device_index: int, verbose_fallbacks: bool):
    patched = model.clone()
    state = PISARuntimeState(armed=True)
    if hasattr(patched, "set_attachments"):
        patched.set_attachments(PISA_RUNTIME_ATTACHMENT, state)
    chained = _set_override(patched, lambda previous: make_generic_pisa_override(
        exact_budget=exact_budget, device_index=device_index, previous_override=previous, runtime_state=state,
        validate_output=verbose_fallbacks))
    return patched, _chained("model-local generic gfx950 PISA installed for explicit self-attention with T>=8192",
                             chained)


def _native_for_anima(exact_budget: float):
    """(native module, exact blocks, None) or (None, None, reason) for the Anima spatial op."""
    try:
        native = diagnostics.load_native()
        info, capabilities = native.build_info(), native.capabilities()
        native.prepare()
    except (ImportError, OSError, RuntimeError, AttributeError) as exc:
        return None, None, f"mi355x-pisa is unavailable ({type(exc).__name__}: {exc})"
    if info.get("architecture") != diagnostics.TARGET:
        return None, None, f"mi355x-pisa is built for {info.get('architecture')}"
    exact_blocks = math.ceil(exact_budget * ANIMA_BLOCKS)
    validated = capabilities.get("spatial_sparse_exact_blocks")
    if not isinstance(validated, (tuple, list)) or exact_blocks not in validated:
        return None, None, (f"exact_budget={exact_budget:.6g} selects {exact_blocks} blocks, but this build validates "
                            f"sparse blocks {validated}")
    return native, exact_blocks, None


def patch_model_pisa_attention(model, *, enabled: bool, exact_budget: float, token_policy: str,
                               verbose_fallbacks: bool, start_layer: int = ANIMA_PISA_FIRST_LAYER,
                               end_layer: int = ANIMA_PISA_LAST_LAYER):
    """Install PISA on a clone of `model`; returns (model, info string)."""
    if not enabled:
        return model, "disabled; model returned unchanged"
    problem = _arguments_problem(model, exact_budget, token_policy, start_layer, end_layer)
    if problem is not None:
        return model, problem + _UNCHANGED
    device_index, device_error = _gfx950_device_index()
    if device_index is None:
        return model, device_error + _UNCHANGED
    if not _is_validated_anima(model):
        return _install_generic(model, exact_budget, device_index, verbose_fallbacks)

    native, exact_blocks, problem = _native_for_anima(exact_budget)
    if problem is not None:
        return model, problem + _UNCHANGED
    patched = model.clone()
    if hasattr(patched, "get_model_object") and hasattr(patched, "add_object_patch"):
        state = PISARuntimeState(armed=True, expected_layers=tuple(range(start_layer, end_layer + 1)))
        patched.set_attachments(PISA_RUNTIME_ATTACHMENT, state)
        try:
            count = install_anima_pisa_attention(
                patched, native_forward=native.forward_spatial_bhtd, exact_blocks=exact_blocks,
                device_index=device_index, first_layer=start_layer, last_layer=end_layer,
                runtime_state=state if verbose_fallbacks else None)
        except (AttributeError, TypeError, ValueError) as exc:
            return model, f"validated Anima direct PISA integration is unavailable ({exc})" + _UNCHANGED
        return patched, (
            f"model-local gfx950 direct PISA installed on Anima self-attention blocks {start_layer}:{end_layer} "
            f"at T=9216; exact_blocks={exact_blocks}; patched_blocks={count}; "
            f"runtime_accounting={'enabled' if verbose_fallbacks else 'disabled'}")

    chained = _set_override(patched, lambda previous: make_pisa_attention_override(
        exact_budget=exact_budget, allowed_tokens=TOKEN_POLICIES[token_policy],
        expected_token_shape=ANIMA_TOKEN_SHAPE, device_index=device_index,
        native_forward=native.forward_spatial_bhtd, verbose_fallbacks=verbose_fallbacks,
        previous_override=previous))
    tokens = ",".join(map(str, sorted(TOKEN_POLICIES[token_policy])))
    return patched, _chained(f"model-local gfx950 PISA override installed for Anima spatial self-attention at "
                             f"T={tokens}; exact_budget={exact_budget:.6g}; layers={start_layer}:{end_layer}", chained)
