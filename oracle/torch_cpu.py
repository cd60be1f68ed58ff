"""fp32 torch restatement of the PISA forward for the CPU baseline (test infrastructure only).

The same algorithm as oracle.pisa (HYD: native/rdna35_pisa_ck/rdna35_pisa_ck/__init__.py:233-316;
generic: generic_pisa.py:141-232), written the way the reference's own
PyTorch path would run on a CPU: float32 tensors, batched matmuls per query
block, torch's thread pool.  bench.py times it as the `cpu_baseline` leg;
tests/test_oracle.py pins it against the float64 numpy oracle (same
selection, outputs within the bf16 tolerance).  Inputs are [BH, T, D]
float32 tensors in block-major token order holding bf16 values, on any
device (tests/test_gpu_full_size_all_heads.py runs the sparse forward on the
GPU as the fp32 reference of the full-size configurations).
"""
from __future__ import annotations

import math

import torch

BLOCK = 64


def _bf16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.bfloat16).float()


def _blocks(x: torch.Tensor) -> torch.Tensor:
    bh, t, d = x.shape
    n = (t + BLOCK - 1) // BLOCK
    if n * BLOCK != t:
        x = torch.nn.functional.pad(x, (0, 0, 0, n * BLOCK - t))
    return x.reshape(bh, n, BLOCK, d)


def _lengths(tokens: int, device=None) -> torch.Tensor:
    n = (tokens + BLOCK - 1) // BLOCK
    lengths = torch.full((n,), float(BLOCK), device=device)
    lengths[-1] = tokens - (n - 1) * BLOCK
    return lengths


def _topk_ascending(scores: torch.Tensor, k: int) -> torch.Tensor:
    """k largest per row, ties to the lowest index (stable descending sort), ascending indices."""
    return torch.sort(scores, dim=-1, descending=True, stable=True).indices[..., :k].sort(dim=-1).values


def _stats(q, k, v, mode: str):
    """Block means and H_sum / ||H_b|| in fp32 (pisa_kernels.cu:192-243; pisa_kernel.py:71-81)."""
    tokens = q.shape[1]
    lengths = _lengths(tokens, q.device)
    qb, kb, vb = _blocks(q), _blocks(k), _blocks(v)
    sums = [x.sum(dim=2) for x in (qb, kb, vb)]
    if mode == "hyd":
        inv = (1.0 / lengths)[None, :, None]
        q_mean, k_mean, v_mean = (s * inv for s in sums)
    else:
        q_mean, k_mean, v_mean = (s / lengths[None, :, None] for s in sums)
    valid = (torch.arange(BLOCK, device=q.device)[None, :] < lengths[:, None])[None, :, :, None]
    centred = torch.where(valid, kb - k_mean[:, :, None, :], torch.zeros((), device=q.device))
    if mode == "generic":
        centred = _bf16(centred)
    h_blocks = torch.matmul(centred.transpose(-1, -2).contiguous(), vb)  # [BH, N, D, D]
    h_norm = h_blocks.flatten(2).norm(dim=-1)
    return q_mean, k_mean, v_mean, h_blocks.sum(dim=1), h_norm, lengths


def _sparse_forward(q, k, v, idx, k_tail, v_tail, lengths, h_sum, scale):
    """Exact softmax over the selected blocks and the centroid tail, merged by LSE, plus
    the first-order term weighted by the tail's share (__init__.py:270-316)."""
    bh, tokens, d = q.shape
    n = lengths.numel()
    exact = idx.shape[-1]
    qb, kb, vb = _blocks(q), _blocks(k), _blocks(v)
    key_valid = torch.arange(BLOCK, device=q.device)[None, :] < lengths[:, None]  # [N, 64]
    log_len = lengths.log()
    out = torch.empty((bh, n, BLOCK, d), device=q.device)
    h_dtype = _bf16(h_sum)
    for b in range(bh):
        selected = torch.zeros((n, n), dtype=torch.bool, device=q.device)
        selected.scatter_(1, idx[b], True)
        tail = torch.matmul(qb[b], k_tail[b].T.contiguous()) * scale + log_len  # [N, 64, N]
        tail = tail.masked_fill(selected[:, None, :], -math.inf)
        l_a = torch.logsumexp(tail, dim=-1)
        o_a = _bf16(torch.matmul(torch.softmax(tail, dim=-1), v_tail[b]))
        if exact:
            keys = kb[b][idx[b]].reshape(n, exact * BLOCK, d)
            vals = vb[b][idx[b]].reshape(n, exact * BLOCK, d)
            ok = key_valid[idx[b]].reshape(n, 1, exact * BLOCK)
            scores = torch.matmul(qb[b], keys.transpose(1, 2).contiguous()) * scale
            scores = scores.masked_fill(~ok, -math.inf)
            l_e = torch.logsumexp(scores, dim=-1)
            o_e = _bf16(torch.matmul(torch.softmax(scores, dim=-1), vals))
            total = torch.logaddexp(l_e, l_a)
            w_e, w_a = torch.exp(l_e - total)[..., None], torch.exp(l_a - total)[..., None]
        else:
            o_e, w_e, w_a = torch.zeros_like(o_a), 0.0, 1.0
        corr = torch.matmul(qb[b], h_dtype[b]) * (scale / tokens)
        out[b] = o_e * w_e + (o_a + corr) * w_a
    return _bf16(out.reshape(bh, n * BLOCK, d)[:, :tokens])


def hyd_forward(q, k, v, exact_blocks: int, scale: float | None = None) -> torch.Tensor:
    """HYD statistics, bf16-rounded centroid routing + ln(||H_b|| + 1e-5), sparse forward."""
    s = float(torch.tensor(1.0 / math.sqrt(q.shape[-1]) if scale is None else scale, dtype=torch.float32))
    q_mean, k_mean, v_mean, h_sum, h_norm, lengths = _stats(q, k, v, "hyd")
    scores = torch.matmul(_bf16(q_mean), _bf16(k_mean).transpose(1, 2).contiguous()) * s \
        + torch.log(h_norm + 1e-5)[:, None, :]
    idx = _topk_ascending(scores, exact_blocks)
    return _sparse_forward(q, k, v, idx, _bf16(k_mean), _bf16(v_mean), lengths, h_sum, s)


def generic_forward(q, k, v, exact_blocks: int, scale: float | None = None, stats: str = "generic") -> torch.Tensor:
    """Centroid routing without the HYD bias on the chosen statistics, sparse forward."""
    s = 1.0 / math.sqrt(q.shape[-1]) if scale is None else float(scale)
    q_mean, k_mean, v_mean, h_sum, _, lengths = _stats(q, k, v, stats)
    q_route = _bf16(q_mean) if stats == "hyd" else q_mean
    scores = torch.matmul(q_route, k_mean.transpose(1, 2).contiguous()) * s
    idx = _topk_ascending(scores, exact_blocks)
    v_tail = _bf16(v_mean) if stats == "hyd" else v_mean
    return _sparse_forward(q, k, v, idx, _bf16(k_mean), v_tail, lengths, h_sum, s)
