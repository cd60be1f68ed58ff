"""Eligibility rules of the model-local attention overrides, stated as data.

The Anima override, the Anima ``attn_op`` patch and the MiniMax-H3 override
each decide whether a call may take the HIP path, and otherwise report why
not with the reason strings the reference uses (pisa_patch.py:61-116,
anima_pisa_integration.py:39-56, minimax_h3_gfx1151_attention.py:77-121;
they appear in runtime reports and fallback logs, so they are kept verbatim).
Here every override is an ordered tuple of ``Rule(reason, passes)``: the
first rule whose ``passes(call)`` is false names the reason, and a call that
passes them all is eligible.  ``Call`` holds the arguments of one attention
call plus the override's configuration and derives the facts the rules test.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any, Callable, Iterable, Union

import torch

Reason = Union[str, Callable[["Call"], str]]


@dataclass(frozen=True)
class Rule:
    reason: Reason
    passes: Callable[["Call"], bool]


@dataclass
class Call:
    """One attention call as an override sees it."""

    q: Any
    k: Any
    v: Any
    heads: int | None = None
    mask: Any = None
    attn_precision: Any = None
    skip_reshape: bool = False
    skip_output_reshape: bool = False
    kwargs: dict = field(default_factory=dict)
    config: dict = field(default_factory=dict)

    @property
    def qkv(self) -> tuple:
        return self.q, self.k, self.v

    def tensors(self) -> bool:
        return all(isinstance(t, torch.Tensor) for t in self.qkv)

    def matching(self, ndim: int) -> bool:
        return self.q.ndim == ndim and self.q.shape == self.k.shape == self.v.shape

    def dtype_is(self, dtype: torch.dtype) -> bool:
        return self.q.dtype == dtype and self.k.dtype == dtype and self.v.dtype == dtype

    def one_device(self) -> bool:
        return self.q.device == self.k.device == self.v.device

    def none(self, test: Callable[[torch.Tensor], bool]) -> bool:
        return not any(test(t) for t in self.qkv)

    def flag(self, name: str, default: Any = None) -> Any:
        return self.kwargs.get(name, default)


def first_failure(rules: Iterable[Rule], call: Call) -> str | None:
    """Reason of the first rule the call fails, or None when it passes every rule."""
    for rule in rules:
        if not rule.passes(call):
            return rule.reason(call) if callable(rule.reason) else rule.reason
    return None


def _bthd_view_strides(q: torch.Tensor) -> tuple:
    """Strides of a [B,H,T,D] view of contiguous [B,T,H,D] storage (the Anima layout)."""
    _, heads, tokens, head_dim = q.shape
    return tokens * heads * head_dim, head_dim, heads * head_dim, 1


def _square_tiles(tokens: int, edge: int = 8) -> bool:
    side = math.isqrt(tokens)
    return side * side == tokens and side % edge == 0


# ----------------------------------------------------------------------------- Anima override
# config: allowed_tokens (frozenset), token_shape (tuple), device_index (int)
ANIMA_OVERRIDE_RULES = (
    Rule("call_is_not_explicitly_self_attention", lambda c: c.flag("is_self_attention") is True),
    Rule("attention_mask_is_not_supported", lambda c: c.mask is None),
    Rule("pre_reshaped_qkv_is_required", lambda c: bool(c.skip_reshape)),
    Rule("merged_attention_output_is_required", lambda c: not c.skip_output_reshape),
    Rule("qkv_are_not_tensors", Call.tensors),
    Rule("matching_bhtd_qkv_are_required", lambda c: c.matching(4)),
    Rule("unsupported_batch_heads_or_head_dim",
         lambda c: c.q.shape[0] > 0 and c.q.shape[1] == c.heads and c.q.shape[-1] == 128),
    Rule(lambda c: f"tokens_{c.q.shape[-2]}_are_not_enabled", lambda c: c.q.shape[-2] in c.config["allowed_tokens"]),
    Rule(lambda c: f"token_shape_{c.flag('attention_token_shape')}_is_not_{c.config['token_shape']}",
         lambda c: isinstance(c.flag("attention_token_shape"), (tuple, list))
         and tuple(c.flag("attention_token_shape")) == c.config["token_shape"]),
    Rule("square_spatial_tokens_divisible_by_8_are_required", lambda c: _square_tiles(c.q.shape[-2])),
    Rule("initial_or_unmarked_transformer_block", lambda c: c.flag("is_initial_transformer_block") is False),
    Rule("matching_bfloat16_qkv_are_required", lambda c: c.dtype_is(torch.bfloat16)),
    Rule("qkv_must_share_one_device", Call.one_device),
    Rule("rocm_cuda_device_is_required", lambda c: c.q.device.type == "cuda"),
    Rule(lambda c: f"rocm_device_{c.q.device.index}_is_not_validated_device_{c.config['device_index']}",
         lambda c: c.q.device.index == c.config["device_index"]),
    Rule("bhtd_views_over_contiguous_bthd_storage_are_required",
         lambda c: c.none(lambda t: t.stride() != _bthd_view_strides(c.q))),
    Rule("forward_only_qkv_are_required", lambda c: c.none(lambda t: t.requires_grad)),
    Rule("float32_attention_precision_is_not_supported", lambda c: c.attn_precision != torch.float32),
    Rule("gqa_is_not_supported", lambda c: not c.flag("enable_gqa", False)),
)

# ----------------------------------------------------------------------------- Anima attn_op patch
# config: tokens, heads, head_dim, device_index; q/k/v are [B, T, H, D]
ANIMA_ATTN_OP_RULES = (
    Rule("qkv_are_not_tensors", Call.tensors),
    Rule("matching_bshd_qkv_are_required", lambda c: c.matching(4)),
    Rule(lambda c: f"shape_{tuple(c.q.shape[1:])}_is_not_t9216_h16_d128",
         lambda c: tuple(c.q.shape[1:]) == (c.config["tokens"], c.config["heads"], c.config["head_dim"])),
    Rule("matching_bfloat16_qkv_are_required", lambda c: c.dtype_is(torch.bfloat16)),
    Rule("qkv_must_share_one_device", Call.one_device),
    Rule("validated_gfx950_device_is_required",
         lambda c: c.q.device.type == "cuda" and c.q.device.index == c.config["device_index"]),
    Rule("contiguous_bshd_qkv_are_required", lambda c: c.none(lambda t: not t.is_contiguous())),
    Rule("forward_only_qkv_are_required", lambda c: c.none(lambda t: t.requires_grad)),
)


# ----------------------------------------------------------------------------- MiniMax-H3 override
def _resolved_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def _aligned_rows(t: torch.Tensor) -> bool:
    return all(s % 8 == 0 for s in t.stride()[:3]) and t.data_ptr() % 16 == 0


# config: heads, head_dim, min_tokens, max_tokens, device_index
H3_OVERRIDE_RULES = (
    Rule("attention_mask_is_not_supported", lambda c: c.mask is None),
    Rule("minimax_h3_merged_output_contract_is_required", lambda c: bool(c.skip_reshape) and not c.skip_output_reshape),
    Rule("gqa_is_not_supported", lambda c: not c.flag("enable_gqa", False)),
    Rule("causal_attention_is_not_supported", lambda c: not (c.flag("is_causal", False) or c.flag("causal", False))),
    Rule("attention_bias_is_not_supported", lambda c: c.flag("attn_bias") is None),
    Rule("qkv_are_not_tensors", Call.tensors),
    Rule("matching_bhtd_qkv_are_required", lambda c: c.matching(4)),
    Rule("minimax_h3_b1_h56_d128_is_required",
         lambda c: c.q.shape[0] == 1 and c.q.shape[1] == c.config["heads"] == c.heads
         and c.q.shape[3] == c.config["head_dim"]),
    Rule(lambda c: f"tokens_below_{c.config['min_tokens']}", lambda c: c.q.shape[2] >= c.config["min_tokens"]),
    Rule(lambda c: f"tokens_above_{c.config['max_tokens']}", lambda c: c.q.shape[2] <= c.config["max_tokens"]),
    Rule("matching_bfloat16_qkv_are_required", lambda c: c.dtype_is(torch.bfloat16)),
    Rule("matching_rocm_qkv_device_is_required", lambda c: c.one_device() and c.q.device.type == "cuda"),
    Rule("qkv_are_not_on_the_validated_gfx950_device",
         lambda c: _resolved_index(c.q.device) == c.config["device_index"]),
    Rule("forward_only_requires_grad_not_supported", lambda c: c.none(lambda t: t.requires_grad)),
    Rule("contiguous_head_dimension_is_required", lambda c: c.none(lambda t: t.stride(3) != 1)),
    Rule("sixteen_byte_aligned_rows_are_required", lambda c: c.none(lambda t: not _aligned_rows(t))),
)


def chain(previous_override: Callable | None, original_func: Callable, *args, **kwargs):
    """Hand a call the override does not take to the override installed before it, else to ComfyUI's own
    attention function (comfy_patch.py:14-17)."""
    if previous_override is not None:
        return previous_override(original_func, *args, **kwargs)
    return original_func(*args, **kwargs)
