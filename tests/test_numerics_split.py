"""The three-part bf16 split of fixed_block_f32x3_kernel (csrc/fixed_block.hip), restated in numpy on the CPU.

The kernel splits every fp32 operand x by truncation into hi = x with its low 16 bits cleared, mid likewise of
x - hi, lo = x - hi - mid, stores each part as the high half of its fp32 bits (a bf16), and forms a product a.b
from the six terms mm, hl, lh, hm, mh, hh.  Checked here: the split is exact (hi + mid + lo == x, each part a
bf16 value) for |x| >= 2^-110 and loses at most 2^-133 below, and six-term dot products of the C1 shape's
length stay within fp32 accuracy of the float64 ones, while dropping any of the kept terms would not.
"""
from __future__ import annotations

import numpy as np

MASK = np.uint32(0xFFFF0000)


def split(x: np.ndarray):
    x = np.asarray(x, dtype=np.float32)
    hi = (x.view(np.uint32) & MASK).view(np.float32)
    r = (x - hi).astype(np.float32)
    mid = (r.view(np.uint32) & MASK).view(np.float32)
    lo = (r - mid).astype(np.float32)
    return hi, mid, lo


def is_bf16(x: np.ndarray) -> bool:
    return bool(np.all((np.asarray(x, dtype=np.float32).view(np.uint32) & np.uint32(0xFFFF)) == 0))


def six_term_dot(a: np.ndarray, b: np.ndarray, terms=("mm", "hl", "lh", "hm", "mh", "hh")) -> np.ndarray:
    pa, pb = dict(zip("hml", split(a))), dict(zip("hml", split(b)))
    acc = np.zeros(a.shape[:-1], dtype=np.float64)
    for t in terms:  # each bf16 x bf16 product is exact in fp32; the sum is fp32 (float64 bounds it)
        acc = (acc + (pa[t[0]].astype(np.float64) * pb[t[1]]).sum(axis=-1)).astype(np.float32).astype(np.float64)
    return acc


def test_split_is_exact_and_each_part_is_bf16():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(100000), rng.standard_normal(1000) * 1e-30, rng.standard_normal(1000) * 1e30,
                        [0.0, -0.0, 1.0, -1.0, np.float32(np.pi), 3.4e38, -3.4e38]]).astype(np.float32)
    x = x[(np.abs(x) >= 2.0 ** -110) | (x == 0)]
    hi, mid, lo = split(x)
    assert is_bf16(hi) and is_bf16(mid) and is_bf16(lo)
    assert np.all(hi.astype(np.float64) + mid.astype(np.float64) + lo.astype(np.float64) == x.astype(np.float64))


def test_split_below_the_normal_range_loses_at_most_2_pow_minus_133():
    """Below |x| = 2^-110 the low part is an fp32 denormal; keeping its high 16 bits loses at most 2^-133."""
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(10000) * 1e-36).astype(np.float32)
    hi, mid, lo = split(x)
    lo_bf16 = (lo.view(np.uint32) & MASK).view(np.float32)
    assert not is_bf16(lo)  # the case exists
    err = np.abs(hi.astype(np.float64) + mid + lo_bf16 - x.astype(np.float64))
    assert err.max() <= 2.0 ** -133


def test_six_terms_are_fp32_accurate_and_five_are_not():
    rng = np.random.default_rng(1)
    a = rng.standard_normal((4096, 64)).astype(np.float32)
    b = rng.standard_normal((4096, 64)).astype(np.float32)
    exact = (a.astype(np.float64) * b).sum(axis=-1)
    scale = np.abs(a.astype(np.float64) * b).sum(axis=-1)  # the sum's condition: errors relative to sum |a_i b_i|
    six = np.max(np.abs(six_term_dot(a, b) - exact) / scale)
    fp32 = np.max(np.abs(np.einsum("nd,nd->n", a, b, dtype=np.float32) - exact) / scale)
    assert six < 4 * 2.0 ** -24, six
    assert six < 4 * fp32 + 2.0 ** -24, (six, fp32)
    for dropped in ("mm", "hl", "hm"):
        kept = tuple(t for t in ("mm", "hl", "lh", "hm", "mh", "hh") if t != dropped)
        err = np.max(np.abs(six_term_dot(a, b, kept) - exact) / scale)
        assert err > 16 * six, (dropped, err, six)
