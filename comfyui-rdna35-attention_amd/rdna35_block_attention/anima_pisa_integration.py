"""Direct ``attn_op`` object patch of the Anima (Cosmos-Predict2) self-attention layers.

The production call site (interface of the reference's
anima_pisa_integration.py:21-127): ``diffusion_model.blocks.{i}.self_attn.attn_op``
for i in [first, last] receives contiguous [B, 9216, 16, 128] bf16 q/k/v.  The
patched op hands BHTD *views* of them (no copy) to the native spatial PISA op
and returns its merged [B, 9216, 2048] output.  Calls outside that profile
(rule table gates.ANIMA_ATTN_OP_RULES) go to the original op; a failure of an
eligible call is raised, never hidden by a fallback.
"""
from __future__ import annotations

from typing import Any, Callable

import torch

from . import gates

ANIMA_BLOCK_COUNT = 28
ANIMA_PISA_TOKENS = 9216
ANIMA_PISA_HEADS = 16
ANIMA_PISA_HEAD_DIM = 128
ANIMA_PISA_FIRST_LAYER = 20
ANIMA_PISA_LAST_LAYER = 27


def _attention_of(block, index: int):
    attn = getattr(block, "self_attn", None)
    if attn is None:
        raise ValueError(f"Anima block {index} has no self_attn")
    return attn


def validate_anima_pisa_model(model_patcher) -> None:
    """Raise ValueError unless the diffusion model is 28 blocks of H=16, D=128 self-attention."""
    blocks = getattr(model_patcher.get_model_object("diffusion_model"), "blocks", None)
    if blocks is None or len(blocks) != ANIMA_BLOCK_COUNT:
        raise ValueError(f"validated Anima model requires {ANIMA_BLOCK_COUNT} blocks")
    profile = (ANIMA_PISA_HEADS, ANIMA_PISA_HEAD_DIM)
    for index, block in enumerate(blocks):
        attn = _attention_of(block, index)
        if (getattr(attn, "n_heads", None), getattr(attn, "head_dim", None)) != profile:
            raise ValueError(f"Anima block {index} is not the validated H=16 D=128 attention profile")


def _eligible_reason(q, k, v, device_index: int) -> str | None:
    call = gates.Call(q, k, v, config={"tokens": ANIMA_PISA_TOKENS, "heads": ANIMA_PISA_HEADS,
                                       "head_dim": ANIMA_PISA_HEAD_DIM, "device_index": device_index})
    return gates.first_failure(gates.ANIMA_ATTN_OP_RULES, call)


def make_anima_pisa_attn_op(original_op: Callable, *, native_forward: Callable, exact_blocks: int, device_index: int,
                            layer_index: int, runtime_state: Any | None = None) -> Callable:
    """The replacement attn_op of one layer (reference call signature of Anima's attn_op)."""
    def account(q, **facts) -> None:
        if runtime_state is None:
            return
        shape = None
        if isinstance(q, torch.Tensor) and q.ndim == 4:
            b, t, h, d = q.shape
            shape = (b, h, t, d)
        runtime_state.record(is_self_attention=True, shape=shape, **facts)

    def anima_pisa_attn_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, transformer_options: dict | None = None,
                           is_self_attention: bool = False, is_initial_transformer_block: bool | None = None):
        reason = _eligible_reason(q, k, v, device_index)
        if reason is not None:
            account(q, fallback_reason=reason)
            return original_op(q, k, v, transformer_options=transformer_options)
        views = [t.transpose(1, 2) for t in (q, k, v)]  # [B,T,H,D] storage read as [B,H,T,D]
        try:
            merged = native_forward(*views, exact_blocks=exact_blocks)
        except Exception as exc:
            account(q, error=exc)
            raise RuntimeError("MI355X PISA failed for the eligible Anima T=9216 BF16 profile") from exc
        account(q, layer=layer_index)
        return merged

    return anima_pisa_attn_op


def install_anima_pisa_attention(model_patcher, *, native_forward: Callable, exact_blocks: int, device_index: int,
                                 first_layer: int, last_layer: int, runtime_state: Any | None = None) -> int:
    """Object-patch the attn_op of layers first..last; returns the number of patched layers."""
    validate_anima_pisa_model(model_patcher)
    if not 0 <= first_layer <= last_layer < ANIMA_BLOCK_COUNT:
        raise ValueError(f"expected 0 <= first_layer <= last_layer < {ANIMA_BLOCK_COUNT}")
    blocks = model_patcher.get_model_object("diffusion_model").blocks
    layers = range(first_layer, last_layer + 1)
    for index in layers:
        op = make_anima_pisa_attn_op(blocks[index].self_attn.attn_op, native_forward=native_forward,
                                     exact_blocks=exact_blocks, device_index=device_index, layer_index=index,
                                     runtime_state=runtime_state)
        model_patcher.add_object_patch(f"diffusion_model.blocks.{index}.self_attn.attn_op", op)
    return len(layers)
