"""Token orders of the PISA blocks (test infrastructure only).

ordered_to_raster restates pisa_kernels.cu:55-64 (96x96 Anima grid, 8x8
tiles); tile_order generalises it to the per-frame tiling of
_pack_video_blocks (generic_pisa.py:37-52), of which the 2-D square layout
(generic_pisa.py:17-34) is the frames=1 case.
"""
from __future__ import annotations

import numpy as np

TILE = 8
SPATIAL_SIDE = 96


def ordered_to_raster(ordered: np.ndarray | int, side: int = SPATIAL_SIDE) -> np.ndarray:
    """Block-major position -> raster token on a side x side grid (pisa_kernels.cu:55-64)."""
    o = np.asarray(ordered, dtype=np.int64)
    block = o // (TILE * TILE)
    intra = o % (TILE * TILE)
    tiles_per_row = side // TILE
    tile_row = block // tiles_per_row
    tile_col = block % tiles_per_row
    return (tile_row * TILE + intra // TILE) * side + tile_col * TILE + intra % TILE


def tile_order(frames: int, height: int, width: int) -> np.ndarray:
    """raster index of every block-major position for a frames x height x width grid."""
    if height % TILE or width % TILE:
        raise ValueError("height and width must be multiples of 8")
    frame_tokens = height * width
    o = np.arange(frames * frame_tokens, dtype=np.int64)
    f = o // frame_tokens
    w = o % frame_tokens
    tile = w // (TILE * TILE)
    intra = w % (TILE * TILE)
    tiles_per_row = width // TILE
    tr = tile // tiles_per_row
    tc = tile % tiles_per_row
    return f * frame_tokens + (tr * TILE + intra // TILE) * width + tc * TILE + intra % TILE


def pack(x: np.ndarray, order: np.ndarray) -> np.ndarray:
    """x [..., T, D] in raster order -> block-major order along the token axis."""
    return np.take(x, order, axis=-2)


def unpack(x: np.ndarray, order: np.ndarray) -> np.ndarray:
    out = np.empty_like(x)
    out[..., order, :] = x
    return out


def pack_minimax_h3_qkv(q, k, v, tokens: int):
    """Profiles of minimax_h3_gfx1151_attention.py:60-74: KV packed below 12000 tokens, QKV from 12000."""
    if tokens >= 12000:
        packed = np.stack((q, k, v))
        return packed[0], packed[1], packed[2], "qkv"
    packed = np.stack((k, v))
    return q, packed[0], packed[1], "kv"
