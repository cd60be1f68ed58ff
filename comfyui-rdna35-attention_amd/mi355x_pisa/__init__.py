"""MI355X (gfx950) native PISA attention ops.

Drop-in counterpart of the reference's ``rdna35_pisa_ck`` package
(native/rdna35_pisa_ck/rdna35_pisa_ck/__init__.py): same entry points
(``forward``, ``forward_spatial_bhtd``, ``block_stats_hyd``, ``prepare``,
``build_info``, ``capabilities``, ``clear_compile_cache``), same argument
meaning, validation messages and error types, registered as
``torch.library`` custom ops with fake implementations so they trace under
``torch.compile(fullgraph=True)``.  The work itself runs in hand-written HIP
kernels (libpisa_hip.so, C ABI in include/pisa_hip.h):

    stats (1 launch) -> H_sum reduction (1) -> routing + top-k (1)
    -> fused exact + tail + first-order + merge + raster store (1)

instead of the reference's pack / CK stats / bmm / topk / FlexAttention x2 /
bmm / epilogue sequence.  No Triton, FlexAttention or CK is involved, and
there is no fallback implementation: if the library is missing, importing
this package raises.
"""
from __future__ import annotations

import math
import struct

from typing import Optional

import torch

from . import _lib
from ._lib import LIB, check, dtype_code, grid, on_device, ptr, stream_of, view3, view4

__version__ = "1.0.0"

BLOCK_SIZE = 64
HEAD_DIM = 128
GENERIC_HEAD_DIMS = tuple(range(8, 257, 8))  # generic PISA (first-order term included) and dense attention
MAX_BLOCKS = 1024
MAX_TOKENS = BLOCK_SIZE * MAX_BLOCKS
SPATIAL_SIDE = 96
SPATIAL_TOKENS = SPATIAL_SIDE * SPATIAL_SIDE
SPATIAL_SPARSE_EXACT_BLOCKS = 23
ARCHITECTURE = "gfx950"
_SUPPORTED_DTYPES = {torch.bfloat16}


def _float32(value: float) -> float:
    """Round to float32; positive finite only (__init__.py:80-87)."""
    try:
        converted = struct.unpack("f", struct.pack("f", float(value)))[0]
    except (OverflowError, struct.error, TypeError, ValueError) as exc:
        raise ValueError("scale must be representable as a positive finite float32 value.") from exc
    if not math.isfinite(converted) or converted <= 0.0:
        raise ValueError("scale must be representable as a positive finite float32 value.")
    return converted


_HIP = torch.version.hip is not None  # a ROCm build of PyTorch (its "cuda" devices are HIP devices)


def _is_rocm_device(tensor: torch.Tensor) -> bool:
    return tensor.device.type == "cuda" and _HIP


def _validate_qkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """__init__.py:90-104, with this library's token limit."""
    if not all(isinstance(tensor, torch.Tensor) for tensor in (q, k, v)):
        raise TypeError("q, k, and v must be torch tensors.")
    if q.ndim != 3 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("PISA HIP expects matching [BH,T,D] q/k/v tensors.")
    if q.shape[0] <= 0 or q.shape[1] <= 0 or q.shape[1] > MAX_TOKENS or q.shape[2] != HEAD_DIM:
        raise ValueError(f"PISA HIP requires BH>0, 0<T<={MAX_TOKENS}, and D={HEAD_DIM}.")
    if q.device != k.device or q.device != v.device or not _is_rocm_device(q):
        raise ValueError("PISA HIP requires q/k/v on one PyTorch ROCm device.")
    if q.dtype not in _SUPPORTED_DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("PISA HIP requires matching bfloat16 q/k/v.")
    if not q.is_contiguous() or not k.is_contiguous() or not v.is_contiguous():
        raise ValueError("PISA HIP requires contiguous q/k/v.")
    if q.requires_grad or k.requires_grad or v.requires_grad:
        raise ValueError("PISA HIP is forward-only.")


def _validate_spatial_bhtd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """__init__.py:107-123."""
    if not all(isinstance(tensor, torch.Tensor) for tensor in (q, k, v)):
        raise TypeError("q, k, and v must be torch tensors.")
    if q.ndim != 4 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("PISA spatial HIP expects matching [B,H,T,D] q/k/v tensors.")
    batch, heads, tokens, head_dim = q.shape
    if batch <= 0 or heads <= 0 or tokens != SPATIAL_TOKENS or head_dim != HEAD_DIM:
        raise ValueError(f"PISA spatial HIP requires B>0, H>0, T={SPATIAL_TOKENS}, and D={HEAD_DIM}.")
    if q.device != k.device or q.device != v.device or not _is_rocm_device(q):
        raise ValueError("PISA spatial HIP requires q/k/v on one PyTorch ROCm device.")
    if q.dtype not in _SUPPORTED_DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("PISA spatial HIP requires matching bfloat16 q/k/v.")
    expected_stride = (tokens * heads * head_dim, head_dim, heads * head_dim, 1)
    if q.stride() != expected_stride or k.stride() != expected_stride or v.stride() != expected_stride:
        raise ValueError("PISA spatial HIP requires BHTD views of contiguous [B,T,H,D] storage.")
    if any(tensor.requires_grad for tensor in (q, k, v)):
        raise ValueError("PISA spatial HIP is forward-only.")


def _check_inputs(what: str, q, k, v, *, dtypes, same_tokens: bool) -> None:
    """Shape, dtype and device agreement of [B,H,T,D] q/k/v before any pointer reaches the C ABI.

    k and v must match each other; q must share their batch, heads and head
    dim, and their token count unless `same_tokens` is False (cross attention).
    Every attribute is read once: this runs on every eager call, whose host time
    bounds small calls (C1's kernel runs 9 us).
    """
    if not (isinstance(q, torch.Tensor) and isinstance(k, torch.Tensor) and isinstance(v, torch.Tensor)):
        raise TypeError(f"{what}: q, k, and v must be torch tensors.")
    qs, ks, vs = q.shape, k.shape, v.shape
    if len(qs) != 4 or len(ks) != 4 or len(vs) != 4:
        raise ValueError(f"{what}: expects [B,H,T,D] q/k/v, got {len(qs)}-D/{len(ks)}-D/{len(vs)}-D")
    if ks != vs:
        raise ValueError(f"{what}: k {tuple(ks)} and v {tuple(vs)} must match")
    if qs[0] != ks[0] or qs[1] != ks[1] or qs[3] != ks[3]:
        raise ValueError(f"{what}: q {tuple(qs)} and k/v {tuple(ks)} must share batch, heads and head dim")
    if same_tokens and qs[2] != ks[2]:
        raise ValueError(f"{what}: q and k/v must have the same token count, got {qs[2]} and {ks[2]}")
    if min(qs) <= 0 or min(ks) <= 0:
        raise ValueError(f"{what}: every dimension must be positive")
    device = q.device
    if device != k.device or device != v.device or device.type != "cuda" or not _HIP:
        raise ValueError(f"{what}: q/k/v must be on one PyTorch ROCm device.")
    dtype = q.dtype
    if dtype not in dtypes or k.dtype != dtype or v.dtype != dtype:
        names = "/".join(str(d).replace("torch.", "") for d in dtypes)
        raise ValueError(f"{what}: q/k/v must share one dtype of {names}, got {dtype}/{k.dtype}/{v.dtype}")
    if q.stride(3) != 1 or k.stride(3) != 1 or v.stride(3) != 1:
        raise ValueError(f"{what}: head_dim must have unit stride")


def _check_exact_and_sink(exact_blocks, blocks: int, sink_block) -> None:
    if isinstance(exact_blocks, bool) or not isinstance(exact_blocks, int):
        raise TypeError("exact_blocks must be an integer.")
    if exact_blocks < 0 or exact_blocks > blocks:
        raise ValueError(f"exact_blocks must be in [0,{blocks}].")
    if sink_block not in (None, -1, 0):
        raise ValueError("sink_block must be None, -1, or 0.")
    if sink_block is not None and exact_blocks == 0:
        raise ValueError("sink_block requires at least one exact block.")


# --------------------------------------------------------------------------- launchers
def _launch_pisa(q4, k4, v4, out4, token_grid, exact_blocks, scale, sink_block, stats_mode, route_mode,
                 first_order, debug_indices=None, debug_scores=None):
    batch, heads, tokens, head_dim = q4.shape
    with on_device(q4.device):
        ws_bytes = LIB.pisa_hip_forward_workspace_bytes(batch, heads, tokens, head_dim, exact_blocks)
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q4.device)
        check(
            LIB.pisa_hip_forward(
                dtype_code(q4.dtype), batch, heads, tokens, head_dim,
                view4(q4), view4(k4), view4(v4), view4(out4), token_grid,
                exact_blocks, scale, sink_block, stats_mode, route_mode, int(first_order),
                ptr(debug_indices), ptr(debug_scores), workspace.data_ptr(), ws_bytes, stream_of(q4.device),
            ),
            "pisa_hip_forward",
        )


def _launch_dense(q4, k4, v4, out4, scale):
    batch, heads, q_tokens, head_dim = q4.shape
    kv_tokens = k4.shape[2]
    with on_device(q4.device):
        ws_bytes = LIB.attn_hip_dense_workspace_bytes(batch, heads, kv_tokens, head_dim)
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q4.device)
        check(
            LIB.attn_hip_dense_forward(
                dtype_code(q4.dtype), batch, heads, q_tokens, kv_tokens, head_dim,
                view4(q4), view4(k4), view4(v4), view4(out4), scale,
                workspace.data_ptr(), ws_bytes, stream_of(q4.device),
            ),
            "attn_hip_dense_forward",
        )


_MASK_KINDS = {torch.bool: _lib.MASK_BOOL, torch.float32: _lib.MASK_ADD_F32, torch.float16: _lib.MASK_ADD_F16,
               torch.bfloat16: _lib.MASK_ADD_BF16}


_NO_MASK = _lib.PisaMask(None, _lib.MASK_NONE, 1, 0, 0, 0, 0)  # passed by value: one shared instance


def _mask_struct(mask: torch.Tensor | None) -> _lib.PisaMask:
    """pisa_mask of a [B', H', T, T] view (0 strides broadcast; B' * H' = the kernel's B*H)."""
    if mask is None:
        return _NO_MASK
    if mask.ndim != 4 or mask.dtype not in _MASK_KINDS:
        raise ValueError("the fixed-block mask view must be 4-D bool/float32/float16/bfloat16")
    sb, sh, sq, sk = mask.stride()
    return _lib.PisaMask(mask.data_ptr(), _MASK_KINDS[mask.dtype], mask.shape[1], sb, sh, sq, sk)


def _launch_fixed_block(q4, k4, v4, out4, scale, causal, mask=None):
    batch, heads, tokens, head_dim = q4.shape
    with on_device(q4.device):
        check(
            LIB.attn_hip_fixed_block_forward_masked(
                dtype_code(q4.dtype), batch, heads, tokens, head_dim, BLOCK_SIZE,
                view4(q4), view4(k4), view4(v4), view4(out4), scale, int(bool(causal)), _mask_struct(mask),
                stream_of(q4.device),
            ),
            "attn_hip_fixed_block_forward_masked",
        )


def _as4(tensor: torch.Tensor) -> torch.Tensor:
    """[BH,T,D] -> [BH,1,T,D] view."""
    return tensor.unsqueeze(1)


def _forward_impl(q, k, v, exact_blocks, scale, sink_block, token_grid=None, out4=None):
    """Sparse or dense PISA over [B,H,T,D] views q/k/v (__init__.py:233-316).

    exact_blocks == N is exact dense attention (the reference calls SDPA,
    __init__.py:251-252); otherwise HYD statistics, HYD routing, exact tiles,
    centroid tail and first-order correction, merged in one kernel.
    """
    batch, heads, tokens, _ = q.shape
    blocks = (tokens + BLOCK_SIZE - 1) // BLOCK_SIZE
    if exact_blocks < 0 or exact_blocks > blocks:
        raise ValueError(f"exact_blocks must be in [0,{blocks}].")
    if sink_block not in (-2, -1, 0):
        raise ValueError("sink_block must be None, -1, or 0.")
    if sink_block != -2 and exact_blocks == 0:
        raise ValueError("sink_block requires at least one exact block.")
    if out4 is None:
        out4 = torch.empty_like(q, memory_format=torch.contiguous_format)
    if exact_blocks == blocks:
        _launch_dense(q, k, v, out4, scale)
    else:
        _launch_pisa(q, k, v, out4, token_grid or grid(), exact_blocks, scale, sink_block,
                     _lib.STATS_HYD, _lib.ROUTE_HYD, True)
    return out4


# --------------------------------------------------------------------------- custom ops
# Every op is a torch.library custom op with a fake implementation, so it
# traces under torch.compile(fullgraph=True) (the reference registers its ops
# the same way, __init__.py:197-213,319-378).  Eager calls on real tensors run
# the kernel function directly: the custom op's first eager call imports
# torch._dynamo (0.5-1 s of host time, during which the GPU idles), and an
# eager caller gains nothing from the dispatcher.
def _eager(*tensors) -> bool:
    """True outside a compiler trace when every tensor is a plain torch.Tensor (not fake/functional)."""
    if torch.compiler.is_compiling():
        return False
    return all(type(t) is torch.Tensor for t in tensors if t is not None)


def _forward_kernel(q, k, v, exact_blocks: int, scale: float, sink_block: int) -> torch.Tensor:
    out = torch.empty_like(q)
    _forward_impl(_as4(q), _as4(k), _as4(v), exact_blocks, scale, sink_block, out4=_as4(out))
    return out


@torch.library.custom_op("mi355x_pisa::forward", mutates_args=(), device_types="cuda")
def _forward_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, exact_blocks: int, scale: float,
                sink_block: int) -> torch.Tensor:
    return _forward_kernel(q, k, v, exact_blocks, scale, sink_block)


@_forward_op.register_fake
def _forward_op_fake(q, k, v, exact_blocks, scale, sink_block):
    del k, v, exact_blocks, scale, sink_block
    return torch.empty_like(q)


def _forward_spatial_kernel(q, k, v, exact_blocks: int, scale: float, sink_block: int) -> torch.Tensor:
    batch, heads, tokens, head_dim = q.shape
    out = q.new_empty((batch, tokens, heads * head_dim))
    out4 = out.view(batch, tokens, heads, head_dim).permute(0, 2, 1, 3)
    # Dense attention is order independent, so the exact profile needs no tiling.
    token_grid = grid(1, SPATIAL_SIDE, SPATIAL_SIDE)
    _forward_impl(q, k, v, exact_blocks, scale, sink_block, token_grid=token_grid, out4=out4)
    return out


@torch.library.custom_op("mi355x_pisa::forward_spatial_bhtd", mutates_args=(), device_types="cuda")
def _forward_spatial_bhtd_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, exact_blocks: int, scale: float,
                             sink_block: int) -> torch.Tensor:
    return _forward_spatial_kernel(q, k, v, exact_blocks, scale, sink_block)


@_forward_spatial_bhtd_op.register_fake
def _forward_spatial_bhtd_op_fake(q, k, v, exact_blocks, scale, sink_block):
    del k, v, exact_blocks, scale, sink_block
    return q.new_empty((q.shape[0], q.shape[2], q.shape[1] * q.shape[3]))


@torch.library.custom_op("mi355x_pisa::block_stats_hyd", mutates_args=(), device_types="cuda")
def _block_stats_hyd_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> tuple[
        torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    return _block_stats(q, k, v, _lib.STATS_HYD, q.dtype)


@_block_stats_hyd_op.register_fake
def _block_stats_hyd_op_fake(q, k, v):
    del k, v
    blocks = (q.shape[1] + BLOCK_SIZE - 1) // BLOCK_SIZE
    shape = (q.shape[0], blocks, q.shape[2])
    return (
        q.new_empty(shape),
        q.new_empty(shape, dtype=torch.float32),
        q.new_empty(shape),
        q.new_empty((q.shape[0], q.shape[2], q.shape[2]), dtype=torch.float32),
        q.new_empty((q.shape[0], blocks), dtype=torch.float32),
    )


def _generic_forward_kernel(q, k, v, exact_blocks: int, scale: float, first_order: bool, sink_block: int,
                            frames: int, height: int, width: int, stats_mode: int) -> torch.Tensor:
    batch, heads, tokens, head_dim = q.shape
    out = q.new_empty((batch, tokens, heads, head_dim))
    out4 = out.permute(0, 2, 1, 3)
    blocks = (tokens + BLOCK_SIZE - 1) // BLOCK_SIZE
    if exact_blocks == blocks:
        _launch_dense(q, k, v, out4, scale)
    else:
        _launch_pisa(q, k, v, out4, grid(frames, height, width), exact_blocks, scale, sink_block,
                     stats_mode, _lib.ROUTE_CENTROID, first_order)
    return out


@torch.library.custom_op("mi355x_pisa::generic_forward", mutates_args=(), device_types="cuda")
def _generic_forward_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, exact_blocks: int, scale: float,
                        first_order: bool, sink_block: int, frames: int, height: int, width: int,
                        stats_mode: int) -> torch.Tensor:
    return _generic_forward_kernel(q, k, v, exact_blocks, scale, first_order, sink_block, frames, height, width,
                                   stats_mode)


@_generic_forward_op.register_fake
def _generic_forward_op_fake(q, k, v, exact_blocks, scale, first_order, sink_block, frames, height, width,
                             stats_mode):
    del k, v, exact_blocks, scale, first_order, sink_block, frames, height, width, stats_mode
    return q.new_empty((q.shape[0], q.shape[2], q.shape[1], q.shape[3]))


def _dense_attention_kernel(q, k, v, scale: float, merged_output: bool) -> torch.Tensor:
    batch, heads, q_tokens, head_dim = q.shape
    if merged_output:
        out = q.new_empty((batch, q_tokens, heads * head_dim))
        out4 = out.view(batch, q_tokens, heads, head_dim).permute(0, 2, 1, 3)
    else:
        out = q.new_empty((batch, heads, q_tokens, head_dim))
        out4 = out
    _launch_dense(q, k, v, out4, scale)
    return out


@torch.library.custom_op("mi355x_pisa::dense_attention", mutates_args=(), device_types="cuda")
def _dense_attention_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
                        merged_output: bool) -> torch.Tensor:
    return _dense_attention_kernel(q, k, v, scale, merged_output)


@_dense_attention_op.register_fake
def _dense_attention_op_fake(q, k, v, scale, merged_output):
    del k, v, scale
    batch, heads, q_tokens, head_dim = q.shape
    if merged_output:
        return q.new_empty((batch, q_tokens, heads * head_dim))
    return q.new_empty((batch, heads, q_tokens, head_dim))


def _fixed_block_kernel(q, k, v, scale: float, causal: bool, mask) -> torch.Tensor:
    out = q.new_empty(q.shape)
    _launch_fixed_block(q, k, v, out, scale, causal, mask)
    return out


@torch.library.custom_op("mi355x_pisa::fixed_block_attention", mutates_args=(), device_types="cuda")
def _fixed_block_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, causal: bool,
                    mask: Optional[torch.Tensor]) -> torch.Tensor:
    return _fixed_block_kernel(q, k, v, scale, causal, mask)


@_fixed_block_op.register_fake
def _fixed_block_op_fake(q, k, v, scale, causal, mask):
    del k, v, scale, causal, mask
    return q.new_empty(q.shape)


# --------------------------------------------------------------------------- statistics
def _block_stats(q, k, v, mode, out_dtype, value_sums: bool = False):
    """q/k/v: [BH,T,D] (or [B,H,T,D] views).  Returns the 5 HYD outputs (3 for MEANS); h_norm is formed at every
    head dim for HYD statistics and is None for GENERIC statistics off head dim 128 (the Triton statistics form
    no norms).  value_sums (fp32 outputs): the third output holds the per-block value sums instead of the means."""
    q4 = q if q.ndim == 4 else _as4(q)
    k4 = k if k.ndim == 4 else _as4(k)
    v4 = v if v.ndim == 4 else _as4(v)
    batch, heads, tokens, head_dim = q4.shape
    bh = batch * heads
    blocks = (tokens + BLOCK_SIZE - 1) // BLOCK_SIZE
    shape = (bh, blocks, head_dim)
    q_centroids = q.new_empty(shape, dtype=out_dtype)
    k_centroids = q.new_empty(shape, dtype=torch.float32)
    v_means = q.new_empty(shape, dtype=out_dtype)
    cov = mode != _lib.STATS_MEANS
    h_sum = q.new_empty((bh, head_dim, head_dim), dtype=torch.float32) if cov else None
    with_norm = cov and (mode == _lib.STATS_HYD or head_dim == HEAD_DIM)
    h_norm = q.new_empty((bh, blocks), dtype=torch.float32) if with_norm else None
    with on_device(q.device):
        ws_bytes = LIB.pisa_hip_block_stats_workspace_bytes(batch, heads, tokens, head_dim) if cov else 0
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
        check(
            LIB.pisa_hip_block_stats(
                dtype_code(q.dtype), dtype_code(out_dtype), batch, heads, tokens, head_dim,
                view4(q4), view4(k4), view4(v4), grid(), mode | (_lib.STATS_FLAG_VALUE_SUMS if value_sums else 0),
                q_centroids.data_ptr(), k_centroids.data_ptr(), v_means.data_ptr(), ptr(h_sum), ptr(h_norm),
                workspace.data_ptr(), ws_bytes, stream_of(q.device),
            ),
            "pisa_hip_block_stats",
        )
    if not cov:
        return q_centroids, k_centroids, v_means
    return q_centroids, k_centroids, v_means, h_sum, h_norm


HYD_STATS_HEAD_DIMS = tuple(range(1, 257))  # block_stats_hyd: any 0<D<=256, as the reference's


def block_stats_hyd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor):
    """(q_bar, k_bar fp32, v_bar, H_sum fp32) of [BH,T,D] q/k/v (__init__.py:216-230).

    Any head dim 0<D<=256, fp16 or bf16.
    """
    if q.ndim != 3 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("PISA HIP HYD expects matching [BH,T,D] q/k/v tensors.")
    if q.shape[0] <= 0 or q.shape[1] <= 0 or q.shape[1] > MAX_TOKENS or q.shape[2] not in HYD_STATS_HEAD_DIMS:
        raise ValueError(f"PISA HIP HYD requires BH>0, 0<T<={MAX_TOKENS}, and 0<D<=256.")
    if q.device != k.device or q.device != v.device or not _is_rocm_device(q):
        raise ValueError("PISA HIP HYD requires q/k/v on one PyTorch ROCm device.")
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("PISA HIP HYD requires matching fp16/bf16 q/k/v.")
    if not q.is_contiguous() or not k.is_contiguous() or not v.is_contiguous():
        raise ValueError("PISA HIP HYD requires contiguous q/k/v.")
    if q.requires_grad or k.requires_grad or v.requires_grad:
        raise ValueError("PISA HIP HYD is forward-only.")
    if _eager(q, k, v):
        return _block_stats(q, k, v, _lib.STATS_HYD, q.dtype)[:4]
    return _block_stats_hyd_op(q, k, v)[:4]


# --------------------------------------------------------------------------- public API
def forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, exact_blocks: int, scale: float | None = None,
            sink_block: int | None = None) -> torch.Tensor:
    """PISA HYD attention of contiguous [BH,T,128] bf16 q/k/v (__init__.py:381-403)."""
    _validate_qkv(q, k, v)
    blocks = (q.shape[1] + BLOCK_SIZE - 1) // BLOCK_SIZE
    _check_exact_and_sink(exact_blocks, blocks, sink_block)
    scale_value = _float32(1.0 / math.sqrt(HEAD_DIM) if scale is None else scale)
    fn = _forward_kernel if _eager(q, k, v) else _forward_op
    return fn(q, k, v, exact_blocks, scale_value, -2 if sink_block is None else sink_block)


def forward_spatial_bhtd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, exact_blocks: int,
                         scale: float | None = None, sink_block: int | None = None) -> torch.Tensor:
    """Anima spatial PISA: [B,H,9216,128] BHTD views of [B,9216,H,128] storage -> [B,9216,H*128].

    Blocks are the 8x8 tiles of the 96x96 token grid (__init__.py:406-433); the
    kernels read the raster layout through the tile map and write the raster
    output directly, so no pack or unpack pass runs.
    """
    _validate_spatial_bhtd(q, k, v)
    blocks = SPATIAL_TOKENS // BLOCK_SIZE
    if isinstance(exact_blocks, bool) or not isinstance(exact_blocks, int):
        raise TypeError("exact_blocks must be an integer.")
    if exact_blocks < 0 or exact_blocks > blocks:
        raise ValueError(f"exact_blocks must be in [0,{blocks}].")
    if exact_blocks not in (SPATIAL_SPARSE_EXACT_BLOCKS, blocks):
        raise ValueError(
            f"spatial PISA supports exact_blocks={SPATIAL_SPARSE_EXACT_BLOCKS}; "
            f"use exact_blocks={blocks} only for dense SDPA validation."
        )
    _check_exact_and_sink(exact_blocks, blocks, sink_block)
    scale_value = _float32(1.0 / math.sqrt(HEAD_DIM) if scale is None else scale)
    fn = _forward_spatial_kernel if _eager(q, k, v) else _forward_spatial_bhtd_op
    return fn(q, k, v, exact_blocks, scale_value, -2 if sink_block is None else sink_block)


# The generic path routes on the HYD statistics of the native module when that
# module takes the shape (generic_pisa.py:106-126): head dim 128, bfloat16 (the
# dtypes its capabilities list, __init__.py:472-473) and at most 9216 tokens
# (its block_stats_hyd limit, __init__.py:30,219-220); otherwise on the
# statistics of the Triton kernel (pisa_kernel.py:49-84).
GENERIC_HYD_STATS_MAX_TOKENS = 9216


def generic_stats_mode(tokens: int, head_dim: int, dtype: torch.dtype) -> str:
    """'hyd' or 'generic': the statistics the reference's generic path uses for this shape."""
    if head_dim == HEAD_DIM and dtype == torch.bfloat16 and 0 < tokens <= GENERIC_HYD_STATS_MAX_TOKENS:
        return "hyd"
    return "generic"


_GENERIC_STATS = {"hyd": _lib.STATS_HYD, "generic": _lib.STATS_GENERIC}


def generic_forward(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, exact_blocks: int, scale: float,
                    first_order: bool, token_grid: tuple[int, int, int] | None = None,
                    sink_block: int | None = None, stats: str | None = None) -> torch.Tensor:
    """Generic PISA over [B,H,T,D] views (generic_pisa.py:141-232 semantics).

    Centroid routing without the HYD bias, optional first-order correction.
    `stats` picks the block statistics: "hyd" (dtype-rounded q_bar routed
    against fp32 k_bar, keys centred in fp32), "generic" (fp32 means,
    dtype-rounded centred keys) or None for the reference's own choice
    (generic_stats_mode).  token_grid=(frames, height, width) selects per-frame
    8x8 tile blocks; the output is [B,T,H,D] contiguous.
    """
    _check_inputs("generic PISA", q, k, v, dtypes=(torch.bfloat16, torch.float16), same_tokens=True)
    frames, height, width = token_grid if token_grid is not None else (0, 0, 0)
    blocks = (q.shape[2] + BLOCK_SIZE - 1) // BLOCK_SIZE
    _check_exact_and_sink(exact_blocks, blocks, sink_block)
    mode = generic_stats_mode(q.shape[2], q.shape[3], q.dtype) if stats is None else stats
    if mode not in _GENERIC_STATS:
        raise ValueError("stats must be None, 'hyd' or 'generic'")
    if mode == "hyd" and q.shape[3] != HEAD_DIM:
        raise ValueError(f"HYD statistics require head_dim={HEAD_DIM}")
    fn = _generic_forward_kernel if _eager(q, k, v) else _generic_forward_op
    return fn(q, k, v, int(exact_blocks), _float32(scale), bool(first_order),
              -2 if sink_block is None else int(sink_block), int(frames), int(height), int(width), _GENERIC_STATS[mode])


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
                    merged_output: bool = False) -> torch.Tensor:
    """Exact attention of [B,H,Tq,D] q over [B,H,Tk,D] k/v (any strides, unit D stride).

    Returns [B,H,Tq,D] contiguous, or [B,Tq,H*D] when merged_output is set.
    """
    _check_inputs("dense attention", q, k, v, dtypes=(torch.bfloat16, torch.float16), same_tokens=False)
    fn = _dense_attention_kernel if _eager(q, k, v) else _dense_attention_op
    return fn(q, k, v, float(scale), bool(merged_output))


def fixed_block_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
                          causal: bool = False, mask: torch.Tensor | None = None) -> torch.Tensor:
    """64-token block-diagonal attention of [B,H,T,D] q/k/v -> [B,H,T,D] contiguous.

    mask: optional [B', H', T, T] view on q's device with B' * H' = B * H
    (broadcast dims as 0 strides): bool keeps a score where True, a float mask
    is added to the scaled scores (reference.py:186-195).
    """
    _check_inputs("fixed-block attention", q, k, v, dtypes=(torch.bfloat16, torch.float16, torch.float32),
                  same_tokens=True)
    if mask is not None:
        batch, heads, tokens, _ = q.shape
        if not isinstance(mask, torch.Tensor) or mask.ndim != 4 or mask.device != q.device:
            raise ValueError("fixed-block mask must be a 4-D tensor on q's device")
        if tuple(mask.shape[2:]) != (tokens, tokens) or mask.shape[0] * mask.shape[1] != batch * heads:
            raise ValueError(f"fixed-block mask must be [B',H',{tokens},{tokens}] with B'*H' = {batch * heads}, "
                             f"got {tuple(mask.shape)}")
    fn = _fixed_block_kernel if _eager(q, k, v, mask) else _fixed_block_op
    return fn(q, k, v, float(scale), bool(causal), mask)


def route_topk(q_centroids: torch.Tensor, k_centroids: torch.Tensor, h_norm: torch.Tensor | None,
               exact_blocks: int, scale: float, sink_block: int | None = None,
               round_bf16: bool = True) -> tuple[torch.Tensor, torch.Tensor]:
    """Routing scores [BH,N,N] and ascending top-k indices [BH,N,k] (int32).

    q/k centroids are fp32 [BH,N,D]; h_norm (fp32 [BH,N]) adds ln(h_norm+1e-5).
    """
    if not isinstance(q_centroids, torch.Tensor) or not isinstance(k_centroids, torch.Tensor):
        raise TypeError("centroids must be torch tensors")
    if q_centroids.ndim != 3 or k_centroids.shape != q_centroids.shape:
        raise ValueError("route_topk expects matching [BH,N,D] q/k centroids")
    bh, blocks, head_dim = q_centroids.shape
    if h_norm is not None and tuple(h_norm.shape) != (bh, blocks):
        raise ValueError(f"h_norm must be [BH,N] = [{bh},{blocks}]")
    for tensor in (q_centroids, k_centroids, h_norm):
        if tensor is not None and (tensor.device != q_centroids.device or not _is_rocm_device(tensor)):
            raise ValueError("route_topk requires every tensor on one PyTorch ROCm device")
    if isinstance(exact_blocks, bool) or not isinstance(exact_blocks, int) or not 0 <= exact_blocks <= blocks:
        raise ValueError(f"exact_blocks must be an integer in [0,{blocks}]")
    qc = q_centroids.float().contiguous()
    kc = k_centroids.float().contiguous()
    hn = None if h_norm is None else h_norm.float().contiguous()
    indices = torch.empty((bh, blocks, max(exact_blocks, 1)), dtype=torch.int32, device=qc.device)
    scores = torch.empty((bh, blocks, blocks), dtype=torch.float32, device=qc.device)
    with on_device(qc.device):
        check(
            LIB.pisa_hip_route_topk(bh, blocks, head_dim, qc.data_ptr(), kc.data_ptr(), ptr(hn), int(round_bf16),
                                    float(scale), -2 if sink_block is None else int(sink_block), int(exact_blocks),
                                    indices.data_ptr(), scores.data_ptr(), stream_of(qc.device)),
            "pisa_hip_route_topk",
        )
    return scores, indices[..., :exact_blocks]


_ROUTING_MODES = {
    "hyd": (_lib.STATS_HYD, _lib.ROUTE_HYD),                # __init__.py:233-316
    "generic": (_lib.STATS_GENERIC, _lib.ROUTE_CENTROID),   # generic_pisa.py:128-138 statistics
    "generic_hyd": (_lib.STATS_HYD, _lib.ROUTE_CENTROID),   # generic_pisa.py:120-126 statistics
}


def forward_with_routing(q4: torch.Tensor, k4: torch.Tensor, v4: torch.Tensor, exact_blocks: int, scale: float,
                         sink_block: int | None = None, hyd: bool = True, first_order: bool = True,
                         token_grid: tuple[int, int, int] | None = None, mode: str | None = None):
    """Sparse PISA forward that also returns the routing scores and selection.

    Diagnostic entry point for parity checks: (out [B,H,T,D] contiguous,
    scores fp32 [BH,N,N], indices int32 [BH,N,k]).  `mode` is "hyd", "generic"
    or "generic_hyd" (generic routing on HYD statistics); None takes `hyd`.
    """
    _check_inputs("PISA", q4, k4, v4, dtypes=(torch.bfloat16, torch.float16), same_tokens=True)
    mode = ("hyd" if hyd else "generic") if mode is None else mode
    if mode not in _ROUTING_MODES:
        raise ValueError(f"mode must be one of {sorted(_ROUTING_MODES)}")
    batch, heads, tokens, head_dim = q4.shape
    blocks = (tokens + BLOCK_SIZE - 1) // BLOCK_SIZE
    out = q4.new_empty(q4.shape)
    scores = torch.empty((batch * heads, blocks, blocks), dtype=torch.float32, device=q4.device)
    indices = torch.empty((batch * heads, blocks, max(exact_blocks, 1)), dtype=torch.int32, device=q4.device)
    frames, height, width = token_grid if token_grid is not None else (0, 0, 0)
    _launch_pisa(q4, k4, v4, out, grid(frames, height, width), exact_blocks, _float32(scale),
                 -2 if sink_block is None else sink_block, *_ROUTING_MODES[mode],
                 first_order, debug_indices=indices, debug_scores=scores)
    return out, scores, indices[..., :exact_blocks]


class PisaPlan:
    """One sparse PISA problem bound to its workspace, run as two stages.

    ``prepare()`` enqueues the statistics, H_sum reduction and routing
    kernels, ``attend()`` the fused exact/tail/correction/merge kernel that
    reads the prepared workspace; ``forward()`` runs both and equals
    ``forward_spatial_bhtd`` / ``generic_forward`` on the same arguments.
    q4/k4/v4/out4 are [B,H,T,D] views; they must stay alive and unchanged
    between prepare() and attend().
    """

    def __init__(self, q4, k4, v4, out4, exact_blocks: int, scale: float | None = None,
                 sink_block: int | None = None, hyd: bool = True, first_order: bool = True,
                 token_grid: tuple[int, int, int] | None = None):
        batch, heads, tokens, head_dim = q4.shape
        self.tensors = (q4, k4, v4, out4)
        self.shape = (batch, heads, tokens, head_dim)
        self.exact_blocks = int(exact_blocks)
        self.scale = _float32(1.0 / math.sqrt(head_dim) if scale is None else scale)
        self.sink_block = -2 if sink_block is None else int(sink_block)
        self.modes = (_lib.STATS_HYD, _lib.ROUTE_HYD) if hyd else (_lib.STATS_GENERIC, _lib.ROUTE_CENTROID)
        self.first_order = int(bool(first_order))
        self.grid = grid(*(token_grid or (0, 0, 0)))
        self.device = q4.device
        self.workspace_bytes = LIB.pisa_hip_forward_workspace_bytes(batch, heads, tokens, head_dim, self.exact_blocks)
        self.workspace = torch.empty(self.workspace_bytes, dtype=torch.uint8, device=self.device)

    def _args(self):
        q4, k4, v4, out4 = self.tensors
        return (dtype_code(q4.dtype), *self.shape, view4(q4), view4(k4), view4(v4), view4(out4), self.grid,
                self.exact_blocks, self.scale, self.sink_block, *self.modes, self.first_order,
                self.workspace.data_ptr(), self.workspace_bytes, stream_of(self.device))

    def prepare(self) -> None:
        with on_device(self.device):
            check(LIB.pisa_hip_prepare(*self._args()), "pisa_hip_prepare")

    def attend(self) -> torch.Tensor:
        with on_device(self.device):
            check(LIB.pisa_hip_attend(*self._args()), "pisa_hip_attend")
        return self.tensors[3]

    def forward(self) -> torch.Tensor:
        self.prepare()
        return self.attend()


def prepare(device_index: int | None = None) -> None:
    """Nothing is compiled at run time; only checks that a ROCm device is present."""
    if not torch.cuda.is_available() or torch.version.hip is None:
        raise RuntimeError("mi355x-pisa requires a PyTorch ROCm device.")
    index = torch.cuda.current_device() if device_index is None else int(device_index)
    torch.cuda.get_device_properties(index)


def build_info() -> dict[str, object]:
    info: dict[str, object] = {}
    for item in _lib.build_info_string().split(";"):
        key, _, value = item.partition("=")
        info[key] = int(value) if value.isdigit() else value
    info["package_version"] = __version__
    info["torch_runtime_version"] = torch.__version__
    info["hip_runtime_version"] = torch.version.hip
    return info


def capabilities() -> dict[str, object]:
    return {
        "architecture": ARCHITECTURE,
        "block_size": BLOCK_SIZE,
        "head_dim": HEAD_DIM,
        "max_blocks": MAX_BLOCKS,
        "dtypes": (torch.bfloat16,),
        "causal": False,
        "backward": False,
        "first_order_tail": True,
        "first_order_routing_bias": True,
        "flex_attention": False,
        "outer_torch_compile": True,
        "outer_torch_compile_requires_prepare": False,
        "spatial_bhtd": True,
        "spatial_tokens": SPATIAL_TOKENS,
        "spatial_sparse_exact_blocks": (SPATIAL_SPARSE_EXACT_BLOCKS,),
        # where the generic path routes on HYD statistics (generic_stats_mode; the reference's
        # _block_stats reads these two keys, generic_pisa.py:123-124) ...
        "hyd_stats_head_dims": (HEAD_DIM,),
        "hyd_stats_dtypes": (torch.bfloat16,),
        # ... and what block_stats_hyd itself accepts
        "block_stats_hyd_head_dims": HYD_STATS_HEAD_DIMS,
        "block_stats_hyd_dtypes": (torch.bfloat16, torch.float16),
        "block_stats_hyd_max_tokens": MAX_TOKENS,
        "generic_head_dims": GENERIC_HEAD_DIMS,
        "generic_dtypes": (torch.bfloat16, torch.float16),
        "dense_head_dims": GENERIC_HEAD_DIMS,
        "fixed_block_head_dims": (32, 64, 128),
        "fixed_block_dtypes": (torch.bfloat16, torch.float16, torch.float32),
    }


def clear_compile_cache() -> None:
    """No run-time compilation happens; kept for API compatibility."""


def _spatial_side(tokens: int) -> int:
    side = math.isqrt(tokens)
    if side * side != tokens or side % 8:
        raise RuntimeError(f"spatial layouts need a square token grid with a side divisible by 8, got T={tokens}")
    return side


def _check_native(name: str, tensor, shape: tuple, dtypes: tuple, device=None) -> None:
    """The reference's per-tensor TORCH_CHECKs of its native entry points (pisa_kernels.cu:719-745):
    device tensor, exact shape, contiguous, dtype, forward-only.  Raised as RuntimeError."""
    if not isinstance(tensor, torch.Tensor) or not _is_rocm_device(tensor):
        raise RuntimeError(f"{name} must be a ROCm device tensor.")
    if device is not None and tensor.device != device:
        raise RuntimeError(f"{name} must be on {device}.")
    if tuple(tensor.shape) != tuple(shape):
        raise RuntimeError(f"{name} must have shape {list(shape)}, got {list(tensor.shape)}.")
    if not tensor.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous.")
    if tensor.dtype not in dtypes:
        raise RuntimeError(f"{name} must be {' or '.join(str(d).replace('torch.', '') for d in dtypes)}.")
    if tensor.requires_grad:
        raise RuntimeError(f"{name} is forward-only.")


class _NativeNamespace:
    """The reference's pybind module surface (bindings.cpp:34-83) on HIP kernels.

    Inputs are checked before any pointer reaches the C ABI, and tensors are
    passed as they are (no temporary copies whose storage could be recycled
    before the kernel runs)."""

    @staticmethod
    def build_info() -> dict[str, object]:
        return build_info()

    @staticmethod
    def _stats_inputs(q, k, v, head_dims, max_tokens=MAX_TOKENS):
        if not all(isinstance(t, torch.Tensor) for t in (q, k, v)) or q.ndim != 3:
            raise RuntimeError("block statistics expect matching [BH,T,D] q/k/v.")
        for name, tensor in (("q", q), ("k", k), ("v", v)):
            _check_native(name, tensor, tuple(q.shape), (torch.bfloat16, torch.float16), q.device)
        if k.dtype != q.dtype or v.dtype != q.dtype:
            raise RuntimeError("q, k, and v must have the same dtype.")
        if q.shape[0] <= 0 or q.shape[1] <= 0 or q.shape[2] not in head_dims:
            dims = f"D={HEAD_DIM}" if tuple(head_dims) == (HEAD_DIM,) else "0<D<=256"
            raise RuntimeError(f"block statistics require BH>0, T>0, and {dims}.")
        if q.shape[1] > max_tokens:
            raise RuntimeError(f"block statistics support T<={max_tokens}.")

    @staticmethod
    def block_stats(q, k, v):
        """Plain means at D=128 (pisa_kernels.cu:563-595)."""
        _NativeNamespace._stats_inputs(q, k, v, (HEAD_DIM,))
        return _block_stats(q, k, v, _lib.STATS_MEANS, q.dtype)

    @staticmethod
    def block_stats_hyd(q, k, v):
        """HYD statistics, all five outputs, at any head dim 0<D<=256 (pisa_kernels.cu:597-635)."""
        _NativeNamespace._stats_inputs(q, k, v, HYD_STATS_HEAD_DIMS)
        return _block_stats(q, k, v, _lib.STATS_HYD, q.dtype)

    @staticmethod
    def pack_spatial_qkv(q, k, v):
        if not all(isinstance(t, torch.Tensor) for t in (q, k, v)) or q.ndim != 4:
            raise RuntimeError("spatial QKV pack expects matching [B,H,T,D] q/k/v.")
        for name, tensor in (("k", k), ("v", v)):
            if tuple(tensor.shape) != tuple(q.shape) or tensor.device != q.device or tensor.dtype != q.dtype:
                raise RuntimeError(f"{name} must match q in shape, dtype and device.")
        if not _is_rocm_device(q) or q.dtype not in (torch.bfloat16, torch.float16):
            raise RuntimeError("spatial QKV pack requires bf16/fp16 ROCm device tensors.")
        if any(t.requires_grad for t in (q, k, v)):
            raise RuntimeError("spatial QKV pack is forward-only.")
        batch, heads, tokens, head_dim = q.shape
        side = _spatial_side(tokens)
        packed = [torch.empty((batch * heads, tokens, head_dim), dtype=q.dtype, device=q.device) for _ in range(3)]
        with on_device(q.device):
            check(
                LIB.pisa_hip_pack_spatial_qkv(
                    dtype_code(q.dtype), batch, heads, tokens, head_dim, view4(q), view4(k), view4(v),
                    grid(1, side, side), packed[0].data_ptr(), packed[1].data_ptr(), packed[2].data_ptr(),
                    stream_of(q.device),
                ),
                "pisa_hip_pack_spatial_qkv",
            )
        return tuple(packed)

    @staticmethod
    def unpack_spatial_output(output, batch, heads):
        if not isinstance(output, torch.Tensor) or output.ndim != 3:
            raise RuntimeError("spatial output unpack expects a [B*H,T,D] tensor.")
        batch, heads = int(batch), int(heads)
        if batch <= 0 or heads <= 0:
            raise RuntimeError("spatial output unpack requires positive batch and heads.")
        bh, tokens, head_dim = output.shape
        _check_native("output", output, (batch * heads, tokens, head_dim), (torch.bfloat16, torch.float16))
        side = _spatial_side(tokens)
        out = output.new_empty((batch, tokens, heads * head_dim))
        with on_device(output.device):
            check(
                LIB.pisa_hip_unpack_spatial_output(
                    dtype_code(output.dtype), batch, heads, tokens, head_dim, output.data_ptr(),
                    grid(1, side, side), out.data_ptr(), stream_of(output.device),
                ),
                "pisa_hip_unpack_spatial_output",
            )
        return out

    @staticmethod
    def fuse_spatial_epilogue(exact_output, exact_lse, approximate_output, approximate_lse, correction, batch, heads):
        if not isinstance(exact_output, torch.Tensor) or exact_output.ndim != 3:
            raise RuntimeError("exact_output must have shape [B*H,T,D].")
        batch, heads = int(batch), int(heads)
        if batch <= 0 or heads <= 0:
            raise RuntimeError("fused epilogue requires positive batch and heads.")
        _, tokens, head_dim = exact_output.shape
        rows = (batch * heads, tokens, head_dim)
        device = exact_output.device
        _check_native("exact_output", exact_output, rows, (torch.bfloat16, torch.float16), device)
        _check_native("approximate_output", approximate_output, rows, (exact_output.dtype,), device)
        _check_native("exact_lse", exact_lse, rows[:2], (torch.float32,), device)
        _check_native("approximate_lse", approximate_lse, rows[:2], (torch.float32,), device)
        _check_native("correction", correction, rows, (torch.float32,), device)
        side = _spatial_side(tokens)
        out = exact_output.new_empty((batch, tokens, heads * head_dim))
        with on_device(device):
            check(
                LIB.pisa_hip_fuse_spatial_epilogue(
                    dtype_code(exact_output.dtype), batch, heads, tokens, head_dim,
                    exact_output.data_ptr(), exact_lse.data_ptr(), approximate_output.data_ptr(),
                    approximate_lse.data_ptr(), correction.data_ptr(), grid(1, side, side), out.data_ptr(),
                    stream_of(device),
                ),
                "pisa_hip_fuse_spatial_epilogue",
            )
        return out


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
    "dense_attention",
    "fixed_block_attention",
    "forward",
    "forward_spatial_bhtd",
    "forward_with_routing",
    "PisaPlan",
    "generic_forward",
    "generic_stats_mode",
    "prepare",
    "route_topk",
]
