"""The reference's native module name, with the reference's contract, on the gfx950 kernels.

Callers of the reference import its native PISA package by name
(``import rdna35_pisa_ck``: rdna35_block_attention/pisa_attention.py:216,
generic_pisa.py:121, pisa_patch.py:226) and choose their path from what it
reports and accepts.  This module gives them the ``mi355x_pisa`` kernels
behind the reference's limits, so such code takes the same decisions it takes
on the reference:

* ``MAX_BLOCKS`` = 144 and ``MAX_TOKENS`` = 9216 (native/rdna35_pisa_ck/
  rdna35_pisa_ck/__init__.py:27-29); ``forward``, ``block_stats_hyd`` and
  ``_C.block_stats*`` refuse longer sequences with the reference's errors
  (``__init__.py:93-94,219-220``, ``pisa_kernels.cu:572,606``);
* ``capabilities()`` lists ``hyd_stats_dtypes`` = (bfloat16,),
  ``hyd_stats_head_dims`` = (128,) and ``max_blocks`` = 144
  (``__init__.py:455-474``).

The reference's generic ``_block_stats`` (generic_pisa.py:119-128) reads
exactly these to pick HYD or Triton statistics.  ``mi355x_pisa`` itself keeps
its wider limits (T up to 65536).  ``build_info()["architecture"]`` reports
gfx950: callers that insist on gfx1151 see a clear mismatch instead of a
silent substitution.
"""
from __future__ import annotations

import torch

import mi355x_pisa as _impl
from mi355x_pisa import (  # noqa: F401  (re-exported surface)
    BLOCK_SIZE,
    HEAD_DIM,
    SPATIAL_SPARSE_EXACT_BLOCKS,
    SPATIAL_TOKENS,
    __version__,
    build_info,
    clear_compile_cache,
    forward_spatial_bhtd,
    prepare,
)

MAX_BLOCKS = 144
MAX_TOKENS = BLOCK_SIZE * MAX_BLOCKS


def _tokens(tensor) -> int | None:
    """Token count of a [BH,T,D] tensor, or None when the shape checks of the implementation should answer."""
    if isinstance(tensor, torch.Tensor) and tensor.ndim == 3:
        return int(tensor.shape[1])
    return None


def capabilities() -> dict[str, object]:
    caps = dict(_impl.capabilities())
    caps["max_blocks"] = MAX_BLOCKS
    caps["hyd_stats_head_dims"] = (HEAD_DIM,)
    caps["hyd_stats_dtypes"] = (torch.bfloat16,)
    return caps


def forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, exact_blocks: int, scale: float | None = None,
            sink_block: int | None = None) -> torch.Tensor:
    """mi355x_pisa.forward at the reference's T <= 9216 (__init__.py:381-403)."""
    tokens = _tokens(q)
    if tokens is not None and tokens > MAX_TOKENS:
        raise ValueError(f"PISA CK requires BH>0, 0<T<={MAX_TOKENS}, and D={HEAD_DIM}.")
    return _impl.forward(q, k, v, exact_blocks, scale=scale, sink_block=sink_block)


def block_stats_hyd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    """mi355x_pisa.block_stats_hyd at the reference's T <= 9216 (__init__.py:216-230)."""
    tokens = _tokens(q)
    if tokens is not None and tokens > MAX_TOKENS:
        raise ValueError(f"PISA CK HYD requires BH>0, 0<T<={MAX_TOKENS}, and 0<D<=256.")
    return _impl.block_stats_hyd(q, k, v)


class _NativeNamespace:
    """``_C`` of the reference (bindings.cpp:34-83): mi355x_pisa._C with the T <= 9216 checks of
    pisa_kernels.cu:572,606 (raised as RuntimeError, as TORCH_CHECK does)."""

    def __getattr__(self, name):
        return getattr(_impl._C, name)

    @staticmethod
    def block_stats(q, k, v):
        tokens = _tokens(q)
        if tokens is not None and tokens > MAX_TOKENS:
            raise RuntimeError(f"PISA CK supports T<={MAX_TOKENS}.")
        return _impl._C.block_stats(q, k, v)

    @staticmethod
    def block_stats_hyd(q, k, v):
        tokens = _tokens(q)
        if tokens is not None and tokens > MAX_TOKENS:
            raise RuntimeError(f"PISA CK HYD supports T<={MAX_TOKENS}.")
        return _impl._C.block_stats_hyd(q, k, v)


_C = _NativeNamespace()

__all__ = [
    "BLOCK_SIZE",
    "HEAD_DIM",
    "MAX_BLOCKS",
    "SPATIAL_SPARSE_EXACT_BLOCKS",
    "SPATIAL_TOKENS",
    "block_stats_hyd",
    "build_info",
    "capabilities",
    "clear_compile_cache",
    "forward",
    "forward_spatial_bhtd",
    "prepare",
]
