"""PISA block-sparse attention oracle (test infrastructure only).

Arrays are float32 numpy arrays holding values already representable in the
input dtype ("bf16" / "f16"), shaped [BH, T, D] in block-major token order
(block b = tokens [64b, 64b+64)); spatial and video layouts are handled by
packing with oracle.layout first.  Math is float64 unless a rounding point
of the reference is being reproduced.

Reference semantics restated here:
  HYD statistics        pisa_kernels.cu:167-244 (block_stats_hyd_kernel)
  plain means           pisa_kernels.cu:130-164 (block_stats_kernel)
  generic statistics    generic_pisa.py:106-138, pisa_kernel.py:49-84
  HYD forward           native/rdna35_pisa_ck/rdna35_pisa_ck/__init__.py:233-316
  generic forward       generic_pisa.py:141-232
  reference backend     pisa_attention.py:73-185 (pisa_attention(backend="reference"))
  concat-softmax form   native/rdna35_pisa_ck/tests/test_forward.py:34-104
"""
from __future__ import annotations

import math

import numpy as np

from .attention import dense_attention
from .numerics import f32, round_bf16, round_dtype, softmax_lse

BLOCK = 64


def block_lengths(tokens: int) -> np.ndarray:
    """Token count of every block; the last may be short (__init__.py:179-183)."""
    blocks = (tokens + BLOCK - 1) // BLOCK
    lengths = np.full(blocks, BLOCK, dtype=np.int64)
    lengths[-1] = tokens - (blocks - 1) * BLOCK
    return lengths


def _block_view(x: np.ndarray, tokens: int) -> np.ndarray:
    """[BH, T, D] -> zero padded [BH, N, 64, D] float64."""
    bh, t, d = x.shape
    blocks = (tokens + BLOCK - 1) // BLOCK
    padded = np.zeros((bh, blocks * BLOCK, d), dtype=np.float64)
    padded[:, :t] = x
    return padded.reshape(bh, blocks, BLOCK, d)


def block_stats(q: np.ndarray, k: np.ndarray, v: np.ndarray, mode: str = "hyd", dtype: str = "bf16",
                covariance: bool = True) -> dict:
    """Per-block statistics.

    mode "means"  : every element pre-scaled by 1/len while summing in row order
                    (one fp32 fma per row); q_bar and v_bar rounded to dtype,
                    k_bar fp32 (pisa_kernels.cu:148-163).
    mode "hyd"    : fp32 sums then * fp32(1/len); q_bar, v_bar rounded to dtype,
                    k_bar fp32; H_b = sum (k - k_bar)^T v with fp32 centring;
                    h_norm = ||H_b||_F; H_sum = sum_b H_b (pisa_kernels.cu:192-243).
    mode "generic": fp32 sums / len for all three (fp32 outputs); H_b from the
                    centred keys rounded to dtype (pisa_kernel.py:71-81,
                    generic_pisa.py:130-134).
    covariance=False stops after the means (no H_b, h_norm or H_sum).
    """
    bh, tokens, d = q.shape
    lengths = block_lengths(tokens)
    inv = f32(1.0 / lengths.astype(np.float32))  # fp32 1/len, as the kernel
    qb, kb, vb = (_block_view(x, tokens) for x in (q, k, v))
    out: dict = {"lengths": lengths}
    if mode == "means":
        # row by row, acc = fma(x, 1/len, acc): the kernel's `mean += x * inverse_length`
        # (pisa_kernels.cu:148-158) as hipcc contracts it; x * inv is exact in float64
        # (8 + 24 significant bits), so rounding the float64 sum is one fp32 fma
        def prescaled_mean(xb):
            acc = np.zeros(xb.shape[:2] + xb.shape[3:], dtype=np.float32)
            for r in range(BLOCK):
                acc = f32(acc.astype(np.float64) + xb[:, :, r] * inv[None, :, None].astype(np.float64))
            return acc
        means = [prescaled_mean(xb) for xb in (qb, kb, vb)]
        out["q_centroids"] = round_dtype(means[0], dtype)
        out["q_centroids_f32"] = means[0]
        out["k_centroids"] = means[1]
        out["v_means"] = round_dtype(means[2], dtype)
        return out
    sums = [f32(np.sum(xb, axis=2)) for xb in (qb, kb, vb)]
    if mode == "hyd":
        means = [f32(s.astype(np.float64) * inv[None, :, None]) for s in sums]
        out["q_centroids"] = round_dtype(means[0], dtype)
        out["v_means"] = round_dtype(means[2], dtype)
    elif mode == "generic":
        means = [f32(s.astype(np.float64) / lengths[None, :, None]) for s in sums]
        out["q_centroids"] = means[0]
        out["v_means"] = means[2]
    else:
        raise ValueError(mode)
    out["q_centroids_f32"] = means[0]
    k_mean = means[1]
    out["k_centroids"] = k_mean
    if not covariance:  # means only (routing without the HYD bias needs nothing else)
        return out
    valid = (np.arange(BLOCK)[None, :] < lengths[:, None])[None, :, :, None]
    centred = f32(np.where(valid, kb - k_mean[:, :, None, :].astype(np.float64), 0.0))
    if mode == "generic":
        centred = round_dtype(centred, dtype)
    h_blocks = np.matmul(np.swapaxes(centred.astype(np.float64), -1, -2), vb)  # sum_t centred[t,i] v[t,j]
    out["h_blocks"] = h_blocks
    out["h_norm"] = f32(np.sqrt(np.sum(h_blocks * h_blocks, axis=(-2, -1))))
    out["h_sum"] = f32(np.sum(h_blocks, axis=1))
    return out


def route_scores(q_centroids: np.ndarray, k_centroids: np.ndarray, scale: float, h_norm: np.ndarray | None = None,
                 sink_block: int | None = None, round_to_bf16: bool = True) -> np.ndarray:
    """r = s * (qbar . kbar) (+ ln(h_norm + 1e-5)), sink column = +inf.

    HYD (__init__.py:255-263): both centroids rounded to bf16, fp32 product.
    Generic (generic_pisa.py:303-304): fp32 centroids, no bias.
    """
    qc = round_bf16(q_centroids) if round_to_bf16 else f32(q_centroids)
    kc = round_bf16(k_centroids) if round_to_bf16 else f32(k_centroids)
    dots = f32(np.einsum("bid,bjd->bij", qc.astype(np.float64), kc.astype(np.float64)))
    r = f32(dots * np.float32(scale))
    if h_norm is not None:
        r = f32(r + np.log(f32(f32(h_norm) + np.float32(1e-5)))[:, None, :])
    if sink_block is not None:
        r[..., sink_block] = np.inf
    return r


def order_key(x: np.ndarray) -> np.ndarray:
    """Total order on float32 used for selection: NaN largest, -0 == +0."""
    a = np.ascontiguousarray(f32(x))
    bits = a.view(np.uint32).copy()
    bits[bits == 0x80000000] = 0
    key = np.where(bits & 0x80000000, ~bits, bits | 0x80000000).astype(np.uint32)
    key[np.isnan(a)] = 0xFFFFFFFF
    return key


def topk_ascending(scores: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest scores per row, ties to the lowest index, returned ascending."""
    n = scores.shape[-1]
    key = order_key(scores).astype(np.uint64)
    idx = np.arange(n, dtype=np.uint64)
    composite = (key << np.uint64(20)) | (np.uint64((1 << 20) - 1) - idx)
    order = np.argsort(composite, axis=-1)[..., ::-1]  # composite keys are unique
    top = order[..., :k]
    return np.sort(top, axis=-1).astype(np.int64)


def selection_mask(indices: np.ndarray, blocks: int) -> np.ndarray:
    bh, n, _ = indices.shape
    selected = np.zeros((bh, n, blocks), dtype=bool)
    np.put_along_axis(selected, indices, True, axis=-1)
    return selected


def _sparse_parts(q, k, v, indices, k_tail, v_tail, lengths, scale, chunk=16):
    """Exact (O_e, L_e) and tail (O_a, L_a) softmaxes for every query block, float64.

    exact: softmax over the tokens of the selected key blocks indices[b, i, :]
           (keys past the end of a short last block excluded).
    tail : scores s q.k_tail_j + ln(len_j) over the unselected blocks j,
           values v_tail.
    """
    bh, tokens, d = q.shape
    blocks = len(lengths)
    exact = indices.shape[-1]
    selected = selection_mask(indices, blocks)
    qb = _block_view(q, tokens)
    kb = _block_view(k, tokens)
    vb = _block_view(v, tokens)
    key_valid = np.arange(BLOCK)[None, :] < lengths[:, None]  # [N, 64]
    log_len = np.log(lengths.astype(np.float64))
    o_e = np.zeros((bh, blocks, BLOCK, d))
    l_e = np.full((bh, blocks, BLOCK), -np.inf)
    o_a = np.zeros_like(o_e)
    l_a = np.full_like(l_e, -np.inf)
    for b in range(bh):
        tail_scores = np.matmul(qb[b], k_tail[b].astype(np.float64).T) * scale + log_len
        tail_scores = np.where(selected[b][:, None, :], -np.inf, tail_scores)
        p, lse = softmax_lse(tail_scores)
        o_a[b] = np.matmul(p, v_tail[b].astype(np.float64))
        l_a[b] = lse
        if exact == 0:
            continue
        for start in range(0, blocks, chunk):
            stop = min(blocks, start + chunk)
            idx = indices[b, start:stop]  # [c, k]
            keys = kb[b][idx].reshape(stop - start, exact * BLOCK, d)
            vals = vb[b][idx].reshape(stop - start, exact * BLOCK, d)
            ok = key_valid[idx].reshape(stop - start, 1, exact * BLOCK)
            scores = np.matmul(qb[b, start:stop], np.swapaxes(keys, -1, -2)) * scale
            p, lse = softmax_lse(np.where(ok, scores, -np.inf))
            o_e[b, start:stop] = np.matmul(p, vals)
            l_e[b, start:stop] = lse
    flat = lambda x: x.reshape(bh, blocks * BLOCK, *x.shape[3:])[:, :tokens]  # noqa: E731
    return flat(o_e), flat(l_e), flat(o_a), flat(l_a)


def _merge(o_e, l_e, o_a, l_a, correction, out_dtype):
    """L = logaddexp(L_e, L_a); out = O_e w_e + O_a w_a + C w_a (__init__.py:310-316)."""
    total = np.logaddexp(l_e, l_a)
    with np.errstate(invalid="ignore"):
        w_e = np.where(np.isfinite(l_e), np.exp(l_e - total), 0.0)[..., None]
        w_a = np.where(np.isfinite(l_a), np.exp(l_a - total), 0.0)[..., None]
    out = o_e * w_e + o_a * w_a
    if correction is not None:
        out = out + correction * w_a
    return round_dtype(out, out_dtype)


def _correction(q, h, scale, tokens, dtype):
    """C = fp32(q . dtype(H)) * fp32(s / T)   (__init__.py:281-282)."""
    hq = round_dtype(h, dtype).astype(np.float64)
    c = f32(np.einsum("btd,bde->bte", np.asarray(q, dtype=np.float64), hq))
    return c.astype(np.float64) * float(np.float32(np.float32(scale) / np.float32(tokens)))


def hyd_forward(q, k, v, exact_blocks: int, scale: float | None = None, sink_block: int | None = None,
                dtype: str = "bf16", return_selection: bool = False):
    """rdna35_pisa_ck._forward_impl (__init__.py:233-316) on [BH, T, D] block-major inputs."""
    bh, tokens, d = q.shape
    blocks = (tokens + BLOCK - 1) // BLOCK
    s = float(np.float32(1.0 / math.sqrt(d) if scale is None else scale))
    if exact_blocks == blocks:
        out = dense_attention(q, k, v, s, out_dtype=dtype)
        return (out, None, None) if return_selection else out
    st = block_stats(q, k, v, "hyd", dtype)
    lengths = st["lengths"]
    k_tail = round_bf16(st["k_centroids"]) if dtype == "bf16" else round_dtype(st["k_centroids"], dtype)
    scores = None
    if exact_blocks > 0:
        scores = route_scores(st["q_centroids_f32"], st["k_centroids"], s, st["h_norm"], sink_block, True)
        indices = topk_ascending(scores, exact_blocks)
    else:
        indices = np.zeros((bh, blocks, 0), dtype=np.int64)
    o_e, l_e, o_a, l_a = _sparse_parts(q, k, v, indices, k_tail, st["v_means"], lengths, s)
    o_a = round_dtype(o_a, dtype).astype(np.float64)
    corr = _correction(q, st["h_sum"], s, tokens, dtype)
    if exact_blocks == 0:
        out = round_dtype(o_a + corr, dtype)
    else:
        o_e = round_dtype(o_e, dtype).astype(np.float64)
        out = _merge(o_e, l_e, o_a, l_a, corr, dtype)
    return (out, scores, indices) if return_selection else out


def hyd_forward_concat(q, k, v, exact_blocks: int, scale: float | None = None, sink_block: int | None = None):
    """Single softmax over [exact tokens ; tail centroids], restating _pisa_reference
    (native/rdna35_pisa_ck/tests/test_forward.py:34-104): q_bar and k_bar rounded to
    bf16, v_bar = bf16(sum v) / len, tail mass weights the fp32 correction."""
    bh, tokens, d = q.shape
    blocks = (tokens + BLOCK - 1) // BLOCK
    s = 1.0 / math.sqrt(d) if scale is None else float(scale)
    lengths = block_lengths(tokens)
    qb, kb, vb = (_block_view(x, tokens) for x in (q, k, v))
    q_c = round_bf16(qb.sum(axis=2) / lengths[None, :, None]).astype(np.float64)
    k_c_f = kb.sum(axis=2) / lengths[None, :, None]
    k_c = round_bf16(k_c_f).astype(np.float64)
    v_means = round_bf16(vb.sum(axis=2)).astype(np.float64) / lengths[None, :, None]
    valid = (np.arange(BLOCK)[None, :] < lengths[:, None])[None, :, :, None]
    centred = round_bf16(np.where(valid, kb - k_c_f[:, :, None, :], 0.0)).astype(np.float64)
    h_blocks = np.einsum("bnti,bntj->bnij", centred, vb)
    h_sum = h_blocks.sum(axis=1)
    h_norms = np.sqrt(np.sum(h_blocks ** 2, axis=(-2, -1)))
    selected = np.zeros((bh, blocks, blocks), dtype=bool)
    if exact_blocks:
        r = np.einsum("bid,bjd->bij", q_c, k_c) * s + np.log(h_norms + 1e-5)[:, None, :]
        if sink_block is not None:
            r[..., sink_block] = np.inf
        selected = selection_mask(topk_ascending(f32(r), exact_blocks), blocks)
    q64 = np.asarray(q, dtype=np.float64)
    correction = np.einsum("btd,bde->bte", q64, h_sum) * (s / tokens)
    keys = np.asarray(k, dtype=np.float64)
    values = np.concatenate((np.asarray(v, dtype=np.float64), v_means), axis=1)
    out = np.empty_like(q64)
    for qblock in range(blocks):
        start, end = qblock * BLOCK, min(qblock * BLOCK + BLOCK, tokens)
        q_blk = q64[:, start:end]
        exact = np.einsum("btd,bsd->bts", q_blk, keys) * s
        token_mask = np.repeat(selected[:, qblock], BLOCK, axis=1)[:, :tokens]
        exact = np.where(token_mask[:, None, :], exact, -np.inf)
        approx = np.einsum("btd,bjd->btj", q_blk, k_c) * s + np.log(lengths)[None, None, :]
        approx = np.where(selected[:, qblock][:, None, :], -np.inf, approx)
        p, _ = softmax_lse(np.concatenate((exact, approx), axis=-1))
        mass = p[..., tokens:].sum(axis=-1, keepdims=True)
        out[:, start:end] = np.einsum("bts,bsd->btd", p, values) + correction[:, start:end] * mass
    return out


def generic_forward(q, k, v, exact_blocks: int, scale: float | None = None, first_order: bool = True,
                    dtype: str = "bf16", return_selection: bool = False, stats: str = "generic"):
    """generic_pisa_attention (generic_pisa.py:141-232).

    stats "generic": the Triton statistics path (generic_pisa.py:128-138,
    pisa_kernel.py:71-81): fp32 centroids, dtype-rounded centred keys.
    stats "hyd": the native block_stats_hyd path (generic_pisa.py:120-126),
    taken by the reference for head dim 128, bfloat16 and T <= 9216: q_bar and
    v_bar rounded to dtype, fp32 k_bar, keys centred in fp32.  Routing is
    q_bar.float() . k_bar_fp32 * s in both (generic_pisa.py:172-173), with no
    HYD bias; the tail uses dtype(k_bar) (generic_pisa.py:203-209)."""
    bh, tokens, d = q.shape
    blocks = (tokens + BLOCK - 1) // BLOCK
    s = 1.0 / math.sqrt(d) if scale is None else float(scale)
    if exact_blocks == blocks:
        out = dense_attention(q, k, v, s, out_dtype=dtype)
        return (out, None, None) if return_selection else out
    if stats not in ("generic", "hyd"):
        raise ValueError(stats)
    st = block_stats(q, k, v, stats, dtype)
    lengths = st["lengths"]
    scores = route_scores(st["q_centroids"], st["k_centroids"], s, None, None, False)
    indices = topk_ascending(scores, exact_blocks)
    k_tail = round_dtype(st["k_centroids"], dtype)
    o_e, l_e, o_a, l_a = _sparse_parts(q, k, v, indices, k_tail, st["v_means"], lengths, s)
    o_e = round_dtype(o_e, dtype).astype(np.float64)
    o_a = round_dtype(o_a, dtype).astype(np.float64)
    corr = _correction(q, st["h_sum"], s, tokens, dtype) if first_order else None
    out = _merge(o_e, l_e, o_a, l_a, corr, dtype)
    return (out, scores, indices) if return_selection else out


def resolve_exact_blocks(total_blocks: int, exact_budget=None, sparsity=None, exact_blocks=None, sink_block=None):
    """_resolve_exact_blocks (pisa_attention.py:38-70)."""
    controls = sum(x is not None for x in (exact_budget, sparsity, exact_blocks))
    if controls > 1:
        raise ValueError("Set only one of exact_budget, sparsity, or exact_blocks.")
    if exact_blocks is not None:
        count = int(exact_blocks)
    else:
        budget = 0.25 if exact_budget is None and sparsity is None else exact_budget
        if sparsity is not None:
            budget = 1.0 - float(sparsity)
        count = min(total_blocks, int(math.ceil(float(budget) * total_blocks)))
    if sink_block is not None:
        count = max(1, count)
    return count


def reference_forward(q, k, v, exact_blocks: int, scale: float | None = None, sink_block: int | None = None,
                      dtype: str = "bf16", centred_keys: str = "f32", return_selection: bool = False):
    """pisa_attention(backend="reference") (pisa_attention.py:73-185): fp32 block means,
    centroid routing without bias, exact online softmax over selected blocks, tail
    e^{s q.kbar_j} * sum(v_j) / (e^{s q.kbar_j} * len_j), first-order term
    (q . H_sum * s/T) weighted by the tail denominator.

    centred_keys "f32" is the reference backend's H_sum (_reference_block_stats,
    pisa_attention.py:73-91); "dtype" is the backend="triton" statistics
    (pisa_prepare_triton, pisa_kernel.py:80-81: centred keys rounded to the
    input dtype), which feed the same selection and piecewise forward
    (pisa_attention.py:314-345)."""
    bh, tokens, d = q.shape
    blocks = (tokens + BLOCK - 1) // BLOCK
    s = 1.0 / math.sqrt(d) if scale is None else float(scale)
    lengths = block_lengths(tokens)
    qb, kb, vb = (_block_view(x, tokens) for x in (q, k, v))
    k_means = f32(kb.sum(axis=2) / lengths[None, :, None])
    v_sums = f32(vb.sum(axis=2))
    valid = (np.arange(BLOCK)[None, :] < lengths[:, None])[None, :, :, None]
    centred = np.where(valid, kb - k_means[:, :, None, :].astype(np.float64), 0.0)
    if centred_keys == "dtype":
        centred = round_dtype(f32(centred), dtype).astype(np.float64)
    elif centred_keys != "f32":
        raise ValueError(centred_keys)
    h_sum = np.einsum("bnti,bntj->bij", centred, vb)
    r = None
    if exact_blocks == blocks:
        selected = np.ones((bh, blocks, blocks), dtype=bool)
    elif exact_blocks == 0:
        selected = np.zeros((bh, blocks, blocks), dtype=bool)
    else:
        q_means = f32(qb.sum(axis=2) / lengths[None, :, None])
        r = f32(np.einsum("bid,bjd->bij", q_means.astype(np.float64), k_means.astype(np.float64)) * s)
        if sink_block is not None:
            r[..., sink_block] = np.inf
        selected = selection_mask(topk_ascending(r, exact_blocks), blocks)
    q64 = np.asarray(q, dtype=np.float64)
    keys = np.asarray(k, dtype=np.float64)
    out = np.empty_like(q64)
    for qblock in range(blocks):
        start, end = qblock * BLOCK, min(qblock * BLOCK + BLOCK, tokens)
        q_blk = q64[:, start:end]
        exact = np.einsum("btd,bsd->bts", q_blk, keys) * s
        token_mask = np.repeat(selected[:, qblock], BLOCK, axis=1)[:, :tokens]
        exact = np.where(token_mask[:, None, :], exact, -np.inf)
        tail = np.einsum("btd,bjd->btj", q_blk, k_means.astype(np.float64)) * s
        tail = np.where(selected[:, qblock][:, None, :], -np.inf, tail)
        m = np.maximum(exact.max(axis=-1), tail.max(axis=-1))[..., None]
        w_exact = np.exp(exact - m)
        w_tail = np.exp(tail - m)
        numerator = np.einsum("bts,bsd->btd", w_exact, np.asarray(v, dtype=np.float64))
        numerator += np.einsum("btj,bjd->btd", w_tail, v_sums.astype(np.float64))
        tail_den = (w_tail * lengths[None, None, :]).sum(axis=-1)
        denominator = w_exact.sum(axis=-1) + tail_den
        correction = np.einsum("btd,bde->bte", q_blk, h_sum) * (s / tokens)
        numerator += correction * tail_den[..., None]
        out[:, start:end] = numerator / denominator[..., None]
    if return_selection:
        return round_dtype(out, dtype), r, selected
    return round_dtype(out, dtype)
