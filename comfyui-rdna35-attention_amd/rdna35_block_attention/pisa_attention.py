"""pisa_attention: training-free PISA forward for contiguous non-causal [BH,T,128] tensors.

Public contract of the reference's pisa_attention.py (:15-373): one of
exact_budget / sparsity / exact_blocks picks the exact key blocks per query
block (default budget 0.25, ceil, a sink forces at least one), the rest of the
keys are approximated by their block centroids (zeroth order) plus a global
first-order covariance term.  Backends:

* ``hip`` / ``auto`` - the gfx950 kernels.  bf16 uses the HYD statistics and
  routing of the native CK backend (backend name ``hip_hyd``); fp16 uses
  centroid routing (``hip_centroid``), the semantics of the reference's
  staged Triton path.
* ``ck`` and ``triton`` - accepted for compatibility and mapped to
  ``hip_hyd`` and ``hip_centroid``.
* ``reference`` - the eager torch implementation below (fp32 statistics,
  exact softmax over the selected blocks, shared numerator/denominator with
  the centroid tail), used for ineligible inputs with the reason reported.
"""
from __future__ import annotations

import math
from typing import Any

import torch

from . import diagnostics

BLOCK_SIZE = 64
HEAD_DIM = 128
SUPPORTED_DTYPES = {torch.float16, torch.bfloat16}
_BACKENDS = {"auto", "hip", "ck", "triton", "reference"}


def _validate_qkv(q, k, v, block_size: int) -> None:
    if not all(isinstance(x, torch.Tensor) for x in (q, k, v)):
        raise TypeError("q, k, and v must be torch tensors.")
    if q.ndim != 3:
        raise ValueError(f"PISA expects contiguous [BH,T,D] tensors, got rank {q.ndim}.")
    if q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f"PISA self-attention requires identical q/k/v shapes, got {q.shape}, {k.shape}, {v.shape}.")
    if q.shape[-1] != HEAD_DIM:
        raise ValueError(f"PISA currently requires D={HEAD_DIM}, got D={q.shape[-1]}.")
    if q.shape[1] == 0:
        raise ValueError("PISA requires at least one token.")
    if q.dtype not in SUPPORTED_DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"PISA requires matching fp16/bf16 q/k/v, got {q.dtype}, {k.dtype}, {v.dtype}.")
    if q.device != k.device or q.device != v.device:
        raise ValueError(f"PISA requires q/k/v on one device, got {q.device}, {k.device}, {v.device}.")
    if not q.is_contiguous() or not k.is_contiguous() or not v.is_contiguous():
        raise ValueError("PISA expects contiguous q/k/v tensors.")
    if any(x.requires_grad for x in (q, k, v)):
        raise ValueError("PISA is a training-free forward prototype and does not accept tensors requiring gradients.")
    if block_size != BLOCK_SIZE:
        raise ValueError(f"PISA currently supports block_size={BLOCK_SIZE} only, got {block_size}.")


def _resolve_exact_blocks(total_blocks: int, *, exact_budget, sparsity, exact_blocks, sink_block) -> tuple[int, float]:
    """Exact blocks per query block and the resulting budget (pisa_attention.py:38-70)."""
    if sum(x is not None for x in (exact_budget, sparsity, exact_blocks)) > 1:
        raise ValueError("Set only one of exact_budget, sparsity, or exact_blocks.")
    if exact_blocks is not None:
        if isinstance(exact_blocks, bool) or not isinstance(exact_blocks, int):
            raise TypeError("exact_blocks must be an integer.")
        if not 0 <= exact_blocks <= total_blocks:
            raise ValueError(f"exact_blocks must be in [0,{total_blocks}], got {exact_blocks}.")
        count = exact_blocks
    else:
        budget = exact_budget
        if sparsity is not None:
            if not 0.0 <= float(sparsity) <= 1.0:
                raise ValueError(f"sparsity must be in [0,1], got {sparsity}.")
            budget = 1.0 - float(sparsity)
        elif budget is None:
            budget = 0.25
        if not 0.0 <= float(budget) <= 1.0:
            raise ValueError(f"exact_budget must be in [0,1], got {budget}.")
        count = min(total_blocks, int(math.ceil(float(budget) * total_blocks)))
    if sink_block is not None:
        if sink_block not in (0, -1):
            raise ValueError("sink_block must be 0, -1, or None.")
        count = max(1, count)
    return count, count / total_blocks


# ----------------------------------------------------------------------------- eager reference backend
def _blocks(x: torch.Tensor, block_size: int) -> torch.Tensor:
    bh, tokens, d = x.shape
    n = math.ceil(tokens / block_size)
    pad = n * block_size - tokens
    if pad:
        x = torch.nn.functional.pad(x, (0, 0, 0, pad))
    return x.reshape(bh, n, block_size, d)


def _reference_block_stats(k: torch.Tensor, v: torch.Tensor, block_size: int):
    """fp32 key means, value sums, H_sum = sum_b (K_b - kbar_b)^T V_b, and block lengths."""
    tokens = k.shape[1]
    n = math.ceil(tokens / block_size)
    lengths = [min(block_size, tokens - b * block_size) for b in range(n)]
    length_t = torch.tensor(lengths, dtype=torch.float32, device=k.device)
    kb = _blocks(k.float(), block_size)
    vb = _blocks(v.float(), block_size)
    k_means = kb.sum(dim=2) / length_t[None, :, None]
    v_sums = vb.sum(dim=2)
    valid = (torch.arange(block_size, device=k.device)[None, :] < length_t[:, None])[None, :, :, None]
    centred = torch.where(valid, kb - k_means[:, :, None, :], torch.zeros((), device=k.device))
    h_sum = torch.einsum("bnti,bntj->bij", centred, vb)
    return k_means, v_sums, h_sum, lengths


def _topk_lowest_index(scores: torch.Tensor, k: int) -> torch.Tensor:
    """Indices of the k largest scores, ties to the lowest index."""
    return torch.sort(scores, dim=-1, descending=True, stable=True).indices[..., :k]


def _select_blocks(q, k_means, *, exact_count: int, block_size: int, scale: float, sink_block):
    bh, tokens, _ = q.shape
    n = k_means.shape[1]
    if exact_count == n:
        return torch.ones((bh, n, n), dtype=torch.bool, device=q.device)
    if exact_count == 0:
        return torch.zeros((bh, n, n), dtype=torch.bool, device=q.device)
    lengths = torch.tensor([min(block_size, tokens - b * block_size) for b in range(n)], dtype=torch.float32,
                           device=q.device)
    q_means = _blocks(q.float(), block_size).sum(dim=2) / lengths[None, :, None]
    scores = torch.einsum("bid,bjd->bij", q_means, k_means) * scale
    if sink_block is not None:
        scores[..., sink_block] = torch.inf
    selected = torch.zeros_like(scores, dtype=torch.bool)
    selected.scatter_(-1, _topk_lowest_index(scores, exact_count), True)
    return selected


def _piecewise_forward(q, k, v, k_means, v_sums, h_sum, lengths, selected, *, block_size: int, scale: float):
    """Shared-normaliser softmax over [selected tokens ; centroids of the other blocks] plus first order.

    Same result as the online per-block loop of pisa_attention.py:130-185:
    out = (sum_exact e^s v + sum_tail e^{s_j} sum(v_j) + C sum_tail len_j e^{s_j})
          / (sum_exact e^s + sum_tail len_j e^{s_j}),  C = s/T * q . H_sum.
    """
    bh, tokens, d = q.shape
    n = len(lengths)
    length_t = torch.tensor(lengths, dtype=torch.float32, device=q.device)
    qf, kf, vf = q.float(), k.float(), v.float()
    out = torch.empty_like(q)
    for qb in range(n):
        start, end = qb * block_size, min(tokens, (qb + 1) * block_size)
        q_blk = qf[:, start:end]
        exact = torch.matmul(q_blk, kf.transpose(1, 2)) * scale
        token_sel = selected[:, qb].repeat_interleave(block_size, dim=1)[:, :tokens]
        exact = exact.masked_fill(~token_sel[:, None, :], -torch.inf)
        tail = torch.matmul(q_blk, k_means.transpose(1, 2)) * scale
        tail = tail.masked_fill(selected[:, qb][:, None, :], -torch.inf)
        m = torch.maximum(exact.amax(dim=-1), tail.amax(dim=-1))
        m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))[..., None]
        w_exact = torch.exp(exact - m)
        w_tail = torch.exp(tail - m)
        tail_den = (w_tail * length_t).sum(dim=-1, keepdim=True)
        numerator = torch.matmul(w_exact, vf) + torch.matmul(w_tail, v_sums)
        numerator = numerator + torch.matmul(q_blk, h_sum) * (scale / tokens) * tail_den
        denominator = w_exact.sum(dim=-1, keepdim=True) + tail_den
        out[:, start:end] = (numerator / denominator).to(q.dtype)
    return out


# ----------------------------------------------------------------------------- HIP backends
def _hip_reject_reason(q: torch.Tensor, hyd: bool) -> str | None:
    if q.device.type != "cuda":
        return f"hip_requires_cuda_hip_device_not_{q.device.type}"
    if not getattr(torch.version, "hip", None):
        return "torch_version_hip_not_detected"
    target = diagnostics.device_gfx_target(q.device)
    if target != diagnostics.TARGET:
        return f"hip_targets_{diagnostics.TARGET}_not_{target or 'unknown'}"
    if hyd and q.dtype != torch.bfloat16:
        return f"hip_hyd_dtype_{q.dtype}_is_not_supported"
    native = diagnostics.load_native()
    if q.shape[1] > native.MAX_TOKENS:
        return f"hip_tokens_{q.shape[1]}_exceed_{native.MAX_TOKENS}"
    return None


def _run_hip(q, k, v, exact_count: int, scale: float, sink_block, hyd: bool) -> torch.Tensor:
    native = diagnostics.load_native()
    if hyd:
        return native.forward(q, k, v, exact_count, scale=scale, sink_block=sink_block)
    # the staged Triton backend's statistics (pisa_attention.py:314-320): fp32
    # means, centred keys rounded to the input dtype
    out = native.generic_forward(q.unsqueeze(1), k.unsqueeze(1), v.unsqueeze(1), exact_count, scale, True,
                                 sink_block=sink_block, stats="generic")
    return out.reshape(q.shape)


def pisa_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, exact_budget: float | None = None,
                   sparsity: float | None = None, exact_blocks: int | None = None, block_size: int = BLOCK_SIZE,
                   scale: float | None = None, sink_block: int | None = None, backend: str = "auto",
                   strict_backend: bool = False, return_diagnostics: bool = False):
    """PISA attention of [BH,T,128] fp16/bf16 q/k/v (see the module docstring for backends)."""
    _validate_qkv(q, k, v, block_size)
    if backend not in _BACKENDS:
        raise ValueError("backend must be one of: auto, hip, ck, triton, reference.")
    if not isinstance(strict_backend, bool):
        raise TypeError("strict_backend must be bool.")
    total_blocks = math.ceil(q.shape[1] / block_size)
    exact_count, budget = _resolve_exact_blocks(total_blocks, exact_budget=exact_budget, sparsity=sparsity,
                                                exact_blocks=exact_blocks, sink_block=sink_block)
    s = float(scale) if scale is not None else 1.0 / math.sqrt(q.shape[-1])
    if not math.isfinite(s) or s <= 0.0:
        raise ValueError(f"scale must be finite and positive, got {s}.")

    used = "reference"
    fallback_reason = None
    output = None
    if backend != "reference":
        hyd = backend == "ck" or (backend in ("auto", "hip") and q.dtype == torch.bfloat16)
        reason = _hip_reject_reason(q, hyd)
        if reason is None:
            output = _run_hip(q, k, v, exact_count, s, sink_block, hyd)
            used = "hip_hyd" if hyd else "hip_centroid"
        else:
            fallback_reason = reason
            if strict_backend:
                label = {"ck": "CK", "triton": "Triton"}.get(backend, "HIP")
                raise RuntimeError(f"PISA {label} backend unavailable: {reason}")
    if output is None:
        k_means, v_sums, h_sum, lengths = _reference_block_stats(k, v, block_size)
        selected = _select_blocks(q, k_means, exact_count=exact_count, block_size=block_size, scale=s,
                                  sink_block=sink_block)
        output = _piecewise_forward(q, k, v, k_means, v_sums, h_sum, lengths, selected, block_size=block_size,
                                    scale=s)
    info: dict[str, Any] = {
        "backend": used,
        "requested_backend": backend,
        "optimized": used != "reference",
        "fallback_reason": fallback_reason,
        "shape": tuple(q.shape),
        "dtype": str(q.dtype),
        "block_size": block_size,
        "total_blocks": total_blocks,
        "exact_blocks_per_query": exact_count,
        "approximate_blocks_per_query": total_blocks - exact_count,
        "exact_budget": budget,
        "sparsity": 1.0 - budget,
        "scale": s,
        "selection": "query_centroid_key_centroid_topk" + ("_hyd_norm_bias" if used == "hip_hyd" else ""),
        "tail_approximation": "block_centered_zeroth_plus_global_first_order",
        "exact_online_softmax": True,
        "shared_numerator_denominator_normalization": True,
        "materialized_token_qk": False,
        "routing_score_elements": q.shape[0] * total_blocks * total_blocks,
        "gfx_target": diagnostics.device_gfx_target(q.device) if q.device.type == "cuda" else None,
    }
    return (output, info) if return_diagnostics else output


def pisa_attention_reference(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, **kwargs):
    kwargs["backend"] = "reference"
    return pisa_attention(q, k, v, **kwargs)
