"""Host logic of the fixed-block and full-attention entry points (CPU).

Mirrors tests/test_reference.py, tests/test_dispatch_fallbacks.py and the CPU
part of tests/test_triton_forward.py of the reference, and checks the eager
reference backend against the oracle.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from rdna35_block_attention import comfy_patch
from rdna35_block_attention.dispatch import fixed_block_attention
from rdna35_block_attention.full_attention import full_attention_hip, validate_full_attention_triton_bh
from rdna35_block_attention.reference import (
    fixed_block_attention_bthd,
    fixed_block_attention_ref,
    fixed_block_attention_sdpa,
    normalize_qkv_to_bh_t_d,
)


def _torch_block_loop(q, k, v, block_size, causal):
    out = torch.empty_like(q)
    scale = 1.0 / math.sqrt(q.shape[-1])
    for start in range(0, q.shape[-2], block_size):
        end = min(start + block_size, q.shape[-2])
        s = q[..., start:end, :] @ k[..., start:end, :].transpose(-2, -1) * scale
        if causal:
            s = s.masked_fill(torch.ones(end - start, end - start, dtype=torch.bool).triu(1), -torch.inf)
        out[..., start:end, :] = torch.softmax(s, -1) @ v[..., start:end, :]
    return out


@pytest.mark.parametrize("batch,heads", [(1, 1), (2, 4)])
@pytest.mark.parametrize("tokens", [64, 128, 192])
@pytest.mark.parametrize("head_dim", [32, 64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_reference_matches_block_loop_and_oracle(batch, heads, tokens, head_dim, causal):
    torch.manual_seed(batch * 100000 + heads * 1000 + tokens + head_dim)
    q, k, v = (torch.randn(batch, heads, tokens, head_dim) for _ in range(3))
    actual = fixed_block_attention_ref(q, k, v, block_size=64, causal=causal, layout="bhtd")
    torch.testing.assert_close(actual, _torch_block_loop(q, k, v, 64, causal), atol=1e-5, rtol=1e-5)
    expected = oatt.fixed_block_attention(q.numpy(), k.numpy(), v.numpy(), causal=causal)
    np.testing.assert_allclose(actual.numpy(), expected, atol=1e-5, rtol=1e-5)


def test_layouts():
    q, k, v = (torch.randn(8, 65, 32) for _ in range(3))
    flat = fixed_block_attention_ref(q, k, v, layout="bh_t_d")
    four = fixed_block_attention_ref(q.reshape(2, 4, 65, 32), k.reshape(2, 4, 65, 32), v.reshape(2, 4, 65, 32),
                                     layout="bhtd").reshape(8, 65, 32)
    torch.testing.assert_close(flat, four, atol=1e-5, rtol=1e-5)
    b, h, t, d = 2, 4, 127, 32
    q, k, v = (torch.randn(b, t, h * d) for _ in range(3))
    actual = fixed_block_attention_bthd(q, k, v, heads=h)
    to4 = lambda x: x.reshape(b, t, h, d).permute(0, 2, 1, 3).contiguous()  # noqa: E731
    expected = fixed_block_attention_ref(to4(q), to4(k), to4(v), layout="bhtd").permute(0, 2, 1, 3).reshape(b, t, h * d)
    torch.testing.assert_close(actual, expected, atol=1e-5, rtol=1e-5)
    with pytest.raises(ValueError, match="Unsupported layout"):
        normalize_qkv_to_bh_t_d(q, k, v, layout="tbhd")
    with pytest.raises(ValueError, match="heads"):
        normalize_qkv_to_bh_t_d(q, k, v, layout="bthd")


@pytest.mark.parametrize("tokens", [64, 127, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_sdpa_block_mask_matches_reference(tokens, causal):
    q, k, v = (torch.randn(2, 3, tokens, 32) for _ in range(3))
    torch.testing.assert_close(fixed_block_attention_sdpa(q, k, v, causal=causal, layout="bhtd"),
                               fixed_block_attention_ref(q, k, v, causal=causal, layout="bhtd"), atol=1e-5, rtol=1e-5)


def test_masks_are_applied_per_block():
    q, k, v = (torch.randn(1, 2, 100, 16) for _ in range(3))
    mask = torch.ones(100, 100, dtype=torch.bool).tril()
    masked = fixed_block_attention_ref(q, k, v, layout="bhtd", mask=mask)
    causal = fixed_block_attention_ref(q, k, v, layout="bhtd", causal=True)
    torch.testing.assert_close(masked, causal)
    additive = torch.zeros(1, 1, 100, 100).masked_fill(~mask, -torch.inf)
    torch.testing.assert_close(fixed_block_attention_ref(q, k, v, layout="bhtd", mask=additive), causal)


class DummyModel:
    def __init__(self):
        self.model_options = {"transformer_options": {}}

    def clone(self):
        cloned = DummyModel()
        cloned.model_options = {"transformer_options": dict(self.model_options["transformer_options"])}
        return cloned


@pytest.mark.parametrize("kwargs,reason", [
    (dict(), "not_cuda"),
    (dict(block_size=32), "unsupported_block_size_32"),
    (dict(mask=torch.zeros(64, 64)), "not_cuda"),     # masks run on the kernel; CPU tensors do not
])
def test_dispatch_fallback_reasons(kwargs, reason):
    q = torch.randn(1, 1, 64, 32, dtype=torch.float16)
    out, info = fixed_block_attention(q, q, q, layout="bhtd", return_diagnostics=True, **kwargs)
    assert out.shape == q.shape
    assert info["backend"] == "reference"
    assert reason in info["fallback_reason"]


def test_dispatch_other_reasons():
    assert "unsupported_head_dim_160" in fixed_block_attention(*(torch.randn(1, 1, 64, 160, dtype=torch.float16),) * 3,
                                                               layout="bhtd", return_diagnostics=True)[1]["fallback_reason"]
    q = torch.randn(1, 1, 64, 32, dtype=torch.float16, requires_grad=True)
    assert "requires_grad" in fixed_block_attention(q, q, q, layout="bhtd", return_diagnostics=True)[1]["fallback_reason"]
    q = torch.randn(1, 1, 64, 32, dtype=torch.float64)
    assert "unsupported_dtype" in fixed_block_attention(q, q, q, layout="bhtd", return_diagnostics=True)[1]["fallback_reason"]
    q = torch.randn(1, 1, 64, 32)
    _, info = fixed_block_attention(q, q, q, layout="bhtd", mode="hip", return_diagnostics=True)
    assert info["fallback_reason"].startswith("requested_hip_but_not_cuda")
    _, info = fixed_block_attention(q, q, q, layout="bhtd", mode="reference", return_diagnostics=True)
    assert info["fallback_reason"] == "mode_reference"
    with pytest.raises(ValueError, match="mode"):
        fixed_block_attention(q, q, q, mode="flash")
    with pytest.raises(ValueError, match="Unsupported layout"):  # the eager fallback re-raises, as the reference does
        fixed_block_attention(q, q, q, layout="bad", return_diagnostics=True)


def test_model_patch_is_model_local_and_exact_only_is_safe():
    model = DummyModel()
    patched, info = comfy_patch.patch_model_attention(model, enabled=True, mode="auto", semantic_mode="exact_only",
                                                      block_size=64, causal=False, verbose_fallbacks=False)
    assert patched is not model
    assert "optimized_attention_override" not in model.model_options["transformer_options"]
    override = patched.model_options["transformer_options"]["optimized_attention_override"]
    assert "exact_only" in info
    q = torch.randn(1, 64, 32)
    assert override(lambda *a, **kw: "original", q, q, q, 1) == "original"


def test_override_runs_marked_calls_and_chains_previous():
    previous_calls = []

    def previous(original_func, *args, **kwargs):
        previous_calls.append(args)
        return "previous"

    model = DummyModel()
    model.model_options["transformer_options"]["optimized_attention_override"] = previous
    patched, info = comfy_patch.patch_model_attention(model, enabled=True, mode="auto",
                                                      semantic_mode="experimental_force_block_local", block_size=64,
                                                      causal=False, verbose_fallbacks=True)
    assert "chained" in info
    override = patched.model_options["transformer_options"]["optimized_attention_override"]
    q, k = torch.randn(1, 64, 64), torch.randn(1, 64, 64)
    assert override(None, q, k, k, 2) == "previous"  # not proven self-attention
    out = override(None, q, k, k, 2, rdna35_attention_semantics="fixed_block_diagonal")
    expected = fixed_block_attention_bthd(q, k, k, heads=2)
    torch.testing.assert_close(out, expected)
    out4 = override(None, q, q, q, 2, skip_output_reshape=True)  # same storage: proven self-attention
    assert out4.shape == (1, 2, 64, 32)
    for bad in (dict(enabled=False), dict(block_size=32), dict(semantic_mode="nope")):
        args = dict(enabled=True, mode="auto", semantic_mode="exact_only", block_size=64, causal=False,
                    verbose_fallbacks=False)
        args.update(bad)
        assert comfy_patch.patch_model_attention(model, **args)[0] is model


def test_full_attention_validation_reasons():
    q = torch.randn(2, 5, 128, dtype=torch.float16)
    k = torch.randn(2, 7, 128, dtype=torch.float16)
    info = validate_full_attention_triton_bh(q, k, torch.randn_like(k))
    assert not info["supported"]
    assert info["reason"] == "not_cuda_or_hip_device_cpu"
    assert (info["q_tokens"], info["kv_tokens"]) == (5, 7)
    assert validate_full_attention_triton_bh(q, k, torch.randn(2, 8, 128, dtype=torch.float16))["reason"] == \
        "key_value_length_mismatch"
    assert validate_full_attention_triton_bh(q.float(), k.float(), k.float())["reason"].startswith("unsupported_dtype")
    assert validate_full_attention_triton_bh(q[..., :96], k[..., :96], k[..., :96])["reason"] == "unsupported_head_dim_96"
    with pytest.raises(ValueError, match="unavailable: not_cuda"):
        full_attention_hip(q, k, torch.randn_like(k))


@pytest.mark.parametrize("layout,shape,mask_shape", [
    ("bhtd", (2, 3, 130, 32), (130, 130)),
    ("bhtd", (2, 3, 130, 32), (2, 130, 130)),        # per batch, repeated over heads
    ("bhtd", (2, 3, 130, 32), (1, 130, 130)),
    ("bhtd", (2, 3, 130, 32), (6, 130, 130)),        # per (batch, head)
    ("bhtd", (2, 3, 130, 32), (2, 3, 130, 130)),
    ("bhtd", (2, 3, 130, 32), (1, 3, 130, 130)),
    ("bhtd", (2, 3, 130, 32), (2, 1, 130, 130)),
    ("bh_t_d", (6, 130, 32), (6, 130, 130)),
    ("bh_t_d", (6, 130, 32), (1, 130, 130)),
])
@pytest.mark.parametrize("dtype", [torch.bool, torch.float32, torch.float64])
def test_kernel_mask_view_matches_eager_slices(layout, shape, mask_shape, dtype):
    """The [B',H',T,T] view the kernel reads equals the eager loop's per-block slices (reference.py:114-156)."""
    from rdna35_block_attention.reference import _mask_block, mask_view_bhtt, normalize_qkv_to_bh_t_d

    q = torch.randn(shape)
    q_flat, _, _, info = normalize_qkv_to_bh_t_d(q, q, q, layout=layout)
    bh = q_flat.shape[0]
    gen = torch.Generator().manual_seed(sum(mask_shape))
    raw = torch.rand(mask_shape, generator=gen)
    mask = raw < 0.5 if dtype == torch.bool else raw.to(dtype)
    view = mask_view_bhtt(mask, batch_heads=bh, info=info, device=q.device)
    assert view.ndim == 4 and view.shape[0] * view.shape[1] == bh
    assert view.dtype == (torch.bool if dtype == torch.bool else torch.float32)
    flat = view.reshape(bh, info.tokens, info.tokens)
    for start in range(0, info.tokens, 64):
        end = min(start + 64, info.tokens)
        eager = _mask_block(mask, start, end, batch_heads=bh, info=info, device=q.device)
        torch.testing.assert_close(flat[:, start:end, start:end], eager.to(flat.dtype))


def test_kernel_mask_view_errors_match_eager():
    from rdna35_block_attention.reference import _mask_block, mask_view_bhtt, normalize_qkv_to_bh_t_d

    q = torch.randn(2, 3, 130, 32)
    _, _, _, info = normalize_qkv_to_bh_t_d(q, q, q, layout="bhtd")
    bad = [torch.zeros(130, 129), torch.zeros(4, 130, 130), torch.zeros(3, 3, 130, 130), torch.zeros(2, 2, 130, 130),
           torch.zeros(2, 3, 130, 130, 1)]
    for mask in bad:
        with pytest.raises(ValueError) as eager:
            _mask_block(mask, 0, 64, batch_heads=6, info=info, device=q.device)
        with pytest.raises(ValueError) as kernel:
            mask_view_bhtt(mask, batch_heads=6, info=info, device=q.device)
        assert str(kernel.value) == str(eager.value)
    q3 = torch.randn(6, 130, 32)
    _, _, _, info3 = normalize_qkv_to_bh_t_d(q3, q3, q3, layout="bh_t_d")
    with pytest.raises(ValueError, match="4D mask requires"):
        mask_view_bhtt(torch.zeros(1, 1, 130, 130), batch_heads=6, info=info3, device=q.device)
