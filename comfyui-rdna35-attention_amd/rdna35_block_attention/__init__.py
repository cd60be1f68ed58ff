"""Drop-in host package of the MI355X attention path.

Same public names as the reference package ``rdna35_block_attention``
(rdna35_block_attention/__init__.py:1-24) - fixed_block_attention,
full_attention_*, pisa_attention, the layout/reference helpers and the
ComfyUI override factories in the submodules - backed by the gfx950 HIP
kernels of ``mi355x_pisa``.
"""
from .diagnostics import (detect_runtime, explain_dispatch, get_device_name, has_triton, is_rocm_pytorch,
                          native_status)
from .dispatch import fixed_block_attention
from .full_attention import full_attention_hip, full_attention_triton
from .pisa_attention import pisa_attention
from .reference import fixed_block_attention_bthd, fixed_block_attention_ref

__all__ = [
    "detect_runtime",
    "explain_dispatch",
    "fixed_block_attention",
    "fixed_block_attention_bthd",
    "fixed_block_attention_ref",
    "full_attention_hip",
    "full_attention_triton",
    "get_device_name",
    "has_triton",
    "is_rocm_pytorch",
    "native_status",
    "pisa_attention",
]
