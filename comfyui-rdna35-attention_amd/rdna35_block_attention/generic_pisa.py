"""Generic PISA for long image/video self-attention (T >= 8192) on gfx950.

Contract of the reference's generic_pisa.py (:141-391):
generic_pisa_attention computes PISA on flat [BH,T,D] tensors with
``exact = min(N, max(1, ceil(budget N)))`` exact blocks (dense attention when
that is all of them), centroid routing without the HYD bias and an optional
first-order correction; make_generic_pisa_override is the model-local
ComfyUI override with its fallback reasons, runtime accounting and
first-call finiteness validation.

Difference in mechanism: the reference packs 8x8 spatial / per-frame video
tiles with torch permute copies, runs Triton statistics, FlexAttention and a
compiled dense tail, and unpacks.  Here the kernels read the raster layout
through the tile map and write the merged [B,T,H*D] output directly, so
neither the pack nor the unpack copy exists.  The torch tile permutations
stay available for callers and tests.
"""
from __future__ import annotations

import math
from typing import Callable

import torch
import torch.nn.functional as F

from . import diagnostics

BLOCK_SIZE = 64
MIN_TOKENS = 8192
SPATIAL_BLOCK_EDGE = 8
# Head dims the HIP kernels take (multiples of 8 up to 256; dims are padded to
# 64/96/128/160/192/256 inside).  The ComfyUI override asks for the
# first-order term at 128 bf16 only, as the reference's does
# (generic_pisa.py:332); a direct call gets it at any of these widths.
SUPPORTED_HEAD_DIMS = tuple(range(8, 257, 8))


# ----------------------------------------------------------------------------- tile permutations
def _pack_spatial_blocks_2d(tensor: torch.Tensor, height: int, width: int) -> torch.Tensor:
    """[..., H*W, D] raster -> 8x8 tile-major order (tiles row-major, tokens row-major inside a tile)."""
    lead, d = tensor.shape[:-2], tensor.shape[-1]
    e = SPATIAL_BLOCK_EDGE
    tiles = tensor.reshape(*lead, height // e, e, width // e, e, d).transpose(-4, -3)
    return tiles.reshape(*lead, height * width, d).contiguous()


def _unpack_spatial_blocks_2d(tensor: torch.Tensor, height: int, width: int) -> torch.Tensor:
    lead, d = tensor.shape[:-2], tensor.shape[-1]
    e = SPATIAL_BLOCK_EDGE
    raster = tensor.reshape(*lead, height // e, width // e, e, e, d).transpose(-4, -3)
    return raster.reshape(*lead, height * width, d).contiguous()


def _pack_spatial_blocks(tensor: torch.Tensor, side: int) -> torch.Tensor:
    return _pack_spatial_blocks_2d(tensor, side, side)


def _unpack_spatial_blocks(tensor: torch.Tensor, side: int) -> torch.Tensor:
    return _unpack_spatial_blocks_2d(tensor, side, side)


def _check_video(tensor: torch.Tensor, grid_sizes) -> tuple[int, int, int]:
    frames, height, width = grid_sizes
    if tensor.shape[2] != frames * height * width:
        raise ValueError("video token shape does not match grid_sizes")
    return frames, height, width


def _pack_video_blocks(tensor: torch.Tensor, grid_sizes) -> torch.Tensor:
    """[B,H,F*h*w,D] -> per-frame 8x8 tile order (frames stay contiguous)."""
    frames, height, width = _check_video(tensor, grid_sizes)
    b, h, _, d = tensor.shape
    framed = tensor.reshape(b, h, frames, height * width, d)
    return _pack_spatial_blocks_2d(framed, height, width).reshape(b, h, frames * height * width, d)


def _unpack_video_blocks(tensor: torch.Tensor, grid_sizes) -> torch.Tensor:
    frames, height, width = _check_video(tensor, grid_sizes)
    b, h, _, d = tensor.shape
    framed = tensor.reshape(b, h, frames, height * width, d)
    return _unpack_spatial_blocks_2d(framed, height, width).reshape(b, h, frames * height * width, d)


# ----------------------------------------------------------------------------- statistics / attention
def _block_stats(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, return_backend: bool = False):
    """(q_bar, k_bar fp32, v_bar, H_sum fp32, lengths) of [BH,T,D] q/k/v on the HIP statistics kernel.

    The statistics the reference picks for the shape (generic_pisa.py:106-138):
    the native HYD statistics at head dim 128, bfloat16, T <= 9216 (q_bar and
    v_bar in the input dtype, keys centred in fp32; backend "hip_hyd"), else
    the Triton semantics (fp32 means, centred keys rounded to the input dtype;
    backend "hip_triton_stats").
    """
    native = diagnostics.load_native()
    tokens = q.shape[1]
    blocks = math.ceil(tokens / BLOCK_SIZE)
    lengths = torch.full((blocks,), BLOCK_SIZE, device=q.device, dtype=torch.float32)
    lengths[-1] = tokens - (blocks - 1) * BLOCK_SIZE
    if native.generic_stats_mode(tokens, q.shape[-1], q.dtype) == "hyd":
        q_c, k_c, v_m, h_sum, _ = native._block_stats(q, k, v, native._lib.STATS_HYD, q.dtype)
        backend = "hip_hyd"
    else:
        q_c, k_c, v_m, h_sum, _ = native._block_stats(q, k, v, native._lib.STATS_GENERIC, torch.float32)
        backend = "hip_triton_stats"
    result = (q_c, k_c, v_m, h_sum, lengths)
    return (*result, backend) if return_backend else result


def _nonfinite(named) -> list[str]:
    return [name for name, tensor in named if not torch.isfinite(tensor).all().item()]


def _partials_nonfinite(q_b, k_b, v_b, idx, k_c, v_m, lengths, scale: float) -> list[str]:
    """Non-finite partials of one head (debug only): the exact softmax over each query block's selected key
    blocks and the centroid tail over the others, their outputs and natural-log LSEs, in fp32
    (generic_pisa.py:188-209 computes the same four tensors with FlexAttention).

    q_b/k_b/v_b: [N, 64, D] block-major (zero rows past T), idx: [N, k] selected blocks, k_c/v_m: [N, D]
    centroids, lengths: [N] tokens per block.
    """
    blocks, _, head_dim = q_b.shape
    valid = torch.arange(BLOCK_SIZE, device=q_b.device)[None, :] < lengths[:, None]      # [N, 64]
    qf = q_b.float()
    k_sel = k_b.float()[idx.long()].reshape(blocks, -1, head_dim)                          # [N, k*64, D]
    v_sel = v_b.float()[idx.long()].reshape(blocks, -1, head_dim)
    scores = torch.matmul(qf, k_sel.transpose(1, 2).contiguous()) * scale                 # [N, 64, k*64]
    scores = scores.masked_fill(~valid[idx.long()].reshape(blocks, 1, -1), -torch.inf)
    exact_lse = torch.logsumexp(scores, dim=-1)
    exact_out = torch.matmul(torch.softmax(scores, dim=-1), v_sel)
    selected = torch.zeros((blocks, blocks), dtype=torch.bool, device=q_b.device)
    selected.scatter_(1, idx.long(), True)
    tail = torch.matmul(qf, k_c.float().t().contiguous()) * scale + lengths.float().log()[None, None, :]
    tail = tail.masked_fill(selected[:, None, :], -torch.inf)
    approx_lse = torch.logsumexp(tail, dim=-1)
    approx_out = torch.matmul(torch.softmax(tail, dim=-1), v_m.float())
    rows = valid[:, :, None]
    named = (("exact_output", exact_out.masked_fill(~rows, 0.0)), ("exact_lse", exact_lse.masked_fill(~valid, 0.0)),
             ("approximate_output", approx_out.masked_fill(~rows, 0.0)),
             ("approximate_lse", approx_lse.masked_fill(~valid, 0.0)))
    return _nonfinite(named)


def _debug_stages(q, k, v, exact_blocks: int, scale: float, grid_sizes) -> None:
    """debug_finite stage checks (generic_pisa.py:174-183,210-219).

    The block statistics and routing scores are recomputed here on the same
    inputs (block-major order of the token grid) and checked; then, since the
    fused kernel never materialises the exact and approximate partial outputs
    and LSEs, those four are recomputed head by head from the kernel's own
    selection (_partials_nonfinite) and checked.  The fused output is checked
    after the call.
    """
    native = diagnostics.load_native()
    q4, k4, v4 = (t.unsqueeze(1) for t in (q, k, v))
    if grid_sizes is not None:
        q4, k4, v4 = (_pack_video_blocks(t, grid_sizes) for t in (q4, k4, v4))
    mode = native.generic_stats_mode(q.shape[1], q.shape[2], q.dtype)
    if mode == "hyd":
        q_c, k_c, v_m, _, _ = native._block_stats(q4, k4, v4, native._lib.STATS_HYD, q.dtype)
    else:
        q_c, k_c, v_m, _, _ = native._block_stats(q4, k4, v4, native._lib.STATS_GENERIC, torch.float32)
    scores, idx = native.route_topk(q_c.float(), k_c, None, exact_blocks, scale, round_bf16=False)
    failed = _nonfinite((("q_centroids", q_c), ("k_centroids", k_c), ("v_means", v_m), ("route_scores", scores)))
    if failed:
        raise ValueError(f"generic PISA non-finite stages: {','.join(failed)}")
    bh, tokens, head_dim = q.shape
    blocks = math.ceil(tokens / BLOCK_SIZE)
    lengths = torch.full((blocks,), BLOCK_SIZE, device=q.device, dtype=torch.float32)
    lengths[-1] = tokens - (blocks - 1) * BLOCK_SIZE
    pad = blocks * BLOCK_SIZE - tokens
    failed = set()
    for h in range(bh):
        q_b, k_b, v_b = (torch.nn.functional.pad(t[h, 0], (0, 0, 0, pad)).reshape(blocks, BLOCK_SIZE, head_dim)
                         for t in (q4, k4, v4))
        failed.update(_partials_nonfinite(q_b, k_b, v_b, idx[h], k_c[h].to(q.dtype), v_m[h], lengths, scale))
    if failed:
        order = ("exact_output", "exact_lse", "approximate_output", "approximate_lse")
        raise ValueError(f"generic PISA non-finite stages: {','.join(n for n in order if n in failed)}")


def generic_pisa_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, exact_budget: float,
                           scale: float | None = None, return_backend: bool = False, use_first_order: bool = True,
                           debug_finite: bool = False, grid_sizes: tuple[int, int, int] | None = None):
    """PISA of [BH,T,D] fp16/bf16 tensors (T >= 8192).

    grid_sizes=(frames, height, width) declares a raster token grid; blocks are
    then its per-frame 8x8 tiles (the layout the reference obtains by packing).
    Statistics follow the reference's choice for the shape (_block_stats); the
    first-order term is applied at every head dim, as the reference's Triton
    statistics form H_sum at any width up to 256 (pisa_kernel.py:90-130).
    """
    if q.ndim != 3 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("generic PISA requires matching [BH,T,D] q/k/v")
    if q.shape[1] < MIN_TOKENS:
        raise ValueError(f"generic PISA requires at least {MIN_TOKENS} tokens")
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("generic PISA requires matching fp16/bf16 q/k/v")
    if not q.is_cuda or q.device != k.device or q.device != v.device:
        raise ValueError("generic PISA requires q/k/v on one CUDA/HIP device")
    if q.shape[-1] not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"generic PISA HIP kernels support head_dim {SUPPORTED_HEAD_DIMS}, got {q.shape[-1]}")
    bh, tokens, head_dim = q.shape
    blocks = math.ceil(tokens / BLOCK_SIZE)
    exact_blocks = min(blocks, max(1, math.ceil(exact_budget * blocks)))
    s = float(scale) if scale is not None else 1.0 / math.sqrt(head_dim)
    native = diagnostics.load_native()
    if debug_finite and exact_blocks < blocks:
        _debug_stages(q, k, v, exact_blocks, s, grid_sizes)
    out = native.generic_forward(q.unsqueeze(1), k.unsqueeze(1), v.unsqueeze(1), exact_blocks, s, use_first_order,
                                 token_grid=grid_sizes)
    out = out.reshape(bh, tokens, head_dim)
    backend = _backend_name(tokens, head_dim, q.dtype, exact_blocks == blocks, use_first_order)
    if debug_finite:
        failed = _nonfinite((("output", out),))
        if failed:
            raise ValueError(f"generic PISA non-finite stages: {','.join(failed)}")
    return (out, backend) if return_backend else out


def _backend_name(tokens: int, head_dim: int, dtype, dense: bool, first_order: bool) -> str:
    """hip_generic[_0th] on the Triton-semantics statistics, hip_generic_hyd[_0th] on the HYD ones
    (the reference reports ck_hyd / triton_hyd and *_0th the same way, generic_pisa.py:231)."""
    if dense:
        return "dense_hip"
    native = diagnostics.load_native()
    name = "hip_generic_hyd" if native.generic_stats_mode(tokens, head_dim, dtype) == "hyd" else "hip_generic"
    return name if first_order else name + "_0th"


def make_generic_pisa_override(*, exact_budget: float, device_index: int, previous_override: Callable | None,
                               runtime_state, validate_output: bool = False) -> Callable:
    def fallback(original_func, *args, **kwargs):
        if previous_override is not None:
            return previous_override(original_func, *args, **kwargs)
        return original_func(*args, **kwargs)

    def attention_override(original_func, q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False,
                           skip_output_reshape=False, **kwargs):
        options = kwargs.get("transformer_options") or {}
        block = options.get("block")
        block_index = options.get("block_index", 0)
        context = f"{block[0]}:{block[1]}:{block_index}" if isinstance(block, (tuple, list)) and len(block) == 2 else None
        passthrough = dict(mask=mask, attn_precision=attn_precision, skip_reshape=skip_reshape,
                           skip_output_reshape=skip_output_reshape, **kwargs)

        reason = None
        if kwargs.get("is_self_attention") is not True:
            reason = "not_explicit_self_attention"
        elif kwargs.get("is_kv_cached_attention", False):
            reason = "kv_cached_attention_is_not_supported"
        elif mask is not None:
            reason = "attention_mask_is_not_supported"
        elif kwargs.get("enable_gqa", False):
            reason = "gqa_is_not_supported"
        elif not all(isinstance(t, torch.Tensor) for t in (q, k, v)):
            reason = "qkv_are_not_tensors"
        elif q.device.type != "cuda" or q.device.index != device_index:
            reason = "validated_gfx950_device_is_required"
        elif k.device != q.device or v.device != q.device:
            reason = "qkv_must_share_one_device"
        elif q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype or v.dtype != q.dtype:
            reason = "matching_fp16_or_bf16_qkv_are_required"

        if reason is None:
            if skip_reshape:
                if q.ndim != 4 or q.shape != k.shape or q.shape != v.shape:
                    reason = "matching_bhtd_qkv_are_required"
                elif q.shape[1] != heads:
                    reason = "head_count_mismatch"
                else:
                    batch, _, tokens, head_dim = q.shape
                    q4, k4, v4 = q, k, v
            else:
                if q.ndim != 3 or q.shape != k.shape or q.shape != v.shape or q.shape[-1] % heads:
                    reason = "matching_btc_qkv_divisible_by_heads_are_required"
                else:
                    batch, tokens, channels = q.shape
                    head_dim = channels // heads
                    q4, k4, v4 = (t.unflatten(2, (heads, head_dim)).transpose(1, 2) for t in (q, k, v))
            if reason is None and tokens < MIN_TOKENS:
                reason = f"tokens_{tokens}_below_{MIN_TOKENS}"

        if reason is not None:
            shape = tuple(q.shape) if isinstance(q, torch.Tensor) and q.ndim >= 2 else None
            runtime_state.record(is_self_attention=kwargs.get("is_self_attention"), shape=shape,
                                 fallback_reason=reason, context=context)
            return fallback(original_func, q, k, v, heads, **passthrough)

        grid = options.get("attention_token_grid", options.get("grid_sizes"))
        video = (isinstance(grid, (tuple, list)) and len(grid) == 3
                 and all(isinstance(x, int) and x > 0 for x in grid) and math.prod(grid) == tokens
                 and grid[1] % SPATIAL_BLOCK_EDGE == 0 and grid[2] % SPATIAL_BLOCK_EDGE == 0)
        side = math.isqrt(tokens)
        square = side * side == tokens and side % SPATIAL_BLOCK_EDGE == 0
        run_shape = (batch, heads, tokens, head_dim)
        if square and isinstance(block, (tuple, list)) and block[0] == "input":
            reason = "spatial_input_stage_uses_dense_attention"
            runtime_state.record(is_self_attention=True, shape=run_shape, fallback_reason=reason, context=context)
            return fallback(original_func, q, k, v, heads, **passthrough)
        token_grid = tuple(grid) if video else ((1, side, side) if square else None)

        first_order = head_dim == 128 and q.dtype == torch.bfloat16
        budget = exact_budget if first_order else max(0.25, exact_budget)
        try:
            output, backend = _generic_pisa_bhtd(q4, k4, v4, budget, kwargs.get("scale"), first_order, token_grid)
            profile = (backend, batch, heads, tokens, head_dim, str(q.dtype))
            if not runtime_state.is_profile_validated(profile):
                if not torch.isfinite(output).all().item():
                    raise ValueError("generic PISA produced non-finite output")
                runtime_state.mark_profile_validated(profile)
        except (RuntimeError, ValueError, NotImplementedError) as exc:
            if isinstance(exc, (torch.OutOfMemoryError, diagnostics.NativeUnavailableError)):
                raise
            runtime_state.record(is_self_attention=True, shape=run_shape,
                                 fallback_reason=f"pisa_backend_error_{type(exc).__name__}", context=context,
                                 error=exc if validate_output else None)
            return fallback(original_func, q, k, v, heads, **passthrough)

        quality = None
        if validate_output and runtime_state.quality_sample is None:
            reference = F.scaled_dot_product_attention(q4.float(), k4.float(), v4.float(),
                                                       scale=kwargs.get("scale")).transpose(1, 2)
            got = output.float()
            cosine = F.cosine_similarity(got.flatten(), reference.flatten(), dim=0).item()
            mae = (got - reference).abs().mean().item()
            quality = (f"cos={cosine:.6f},mae={mae:.6g},pisa_max={got.abs().max().item():.6g},"
                       f"sdpa_max={reference.abs().max().item():.6g}")
        runtime_state.record(layer=-1, is_self_attention=True, shape=run_shape, backend=backend, context=context,
                             quality=quality)
        if skip_output_reshape:
            return output.transpose(1, 2)
        return output.reshape(batch, tokens, heads * head_dim)

    return attention_override


def _generic_pisa_bhtd(q4, k4, v4, exact_budget, scale, first_order, token_grid):
    """generic_pisa_attention on [B,H,T,D] views; output [B,T,H,D] contiguous (merged layout)."""
    batch, heads, tokens, head_dim = q4.shape
    if head_dim not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"generic PISA HIP kernels support head_dim {SUPPORTED_HEAD_DIMS}, got {head_dim}")
    blocks = math.ceil(tokens / BLOCK_SIZE)
    exact_blocks = min(blocks, max(1, math.ceil(exact_budget * blocks)))
    s = float(scale) if scale is not None else 1.0 / math.sqrt(head_dim)
    native = diagnostics.load_native()
    out = native.generic_forward(q4, k4, v4, exact_blocks, s, first_order, token_grid=token_grid)
    return out, _backend_name(tokens, head_dim, q4.dtype, exact_blocks == blocks, first_order)
