"""The reference's module name for the MiniMax-H3 override (minimax_h3_gfx1151_attention.py).

Its public names resolve to this package's gfx950 implementation in
minimax_h3_attention: callers that import the reference's module and
functions (make_minimax_h3_gfx1151_attention_override,
patch_minimax_h3_gfx1151_attention, pack_minimax_h3_qkv,
minimax_h3_pack_profile) get the same objects under either name.
"""
from __future__ import annotations

from .minimax_h3_attention import (  # noqa: F401
    LOG_PREFIX,
    MINIMAX_H3_HEAD_DIM,
    MINIMAX_H3_HEADS,
    MINIMAX_H3_MAX_PACK_TOKENS,
    MINIMAX_H3_MIN_PACK_TOKENS,
    MINIMAX_H3_PACK_ALL_TOKENS,
    make_minimax_h3_attention_override,
    minimax_h3_pack_profile,
    pack_minimax_h3_qkv,
    patch_minimax_h3_attention,
)

make_minimax_h3_gfx1151_attention_override = make_minimax_h3_attention_override
patch_minimax_h3_gfx1151_attention = patch_minimax_h3_attention
