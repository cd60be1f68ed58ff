"""GPU tests of the drop-in host API: every eligible call must run the HIP kernels
(diagnostics report backend hip*) and match the oracle / eager reference."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import assert_close, np32, packed_to_merged, spatial_to_packed
from oracle import attention as oatt
from oracle import pisa as opisa

pytestmark = pytest.mark.gpu
D = 128


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("tokens,head_dim", [(64, 32), (128, 64), (256, 128), (200, 64)])
def test_fixed_block_dispatch_uses_hip(dtype, tokens, head_dim):
    from rdna35_block_attention import fixed_block_attention, fixed_block_attention_ref

    torch.manual_seed(tokens + head_dim)
    q, k, v = (torch.randn(1, 2, tokens, head_dim, device="cuda", dtype=dtype) for _ in range(3))
    out, info = fixed_block_attention(q, k, v, block_size=64, layout="bhtd", mode="auto", return_diagnostics=True)
    assert info["backend"] == "hip", info
    ref = fixed_block_attention_ref(q.cpu(), k.cpu(), v.cpu(), block_size=64, layout="bhtd")
    tol = {torch.float16: 5e-2, torch.bfloat16: 1e-1, torch.float32: 1e-5}[dtype]
    torch.testing.assert_close(out.float().cpu(), ref.float(), atol=tol, rtol=tol)


def test_fixed_block_bthd_and_override_on_gpu():
    from rdna35_block_attention import comfy_patch
    from rdna35_block_attention.reference import fixed_block_attention_bthd

    class Model:
        model_options = {"transformer_options": {}}

        def clone(self):
            m = Model()
            m.model_options = {"transformer_options": {}}
            return m

    patched, _ = comfy_patch.patch_model_attention(Model(), enabled=True, mode="auto", semantic_mode="exact_only",
                                                   block_size=64, causal=True, verbose_fallbacks=False)
    override = patched.model_options["transformer_options"]["optimized_attention_override"]
    torch.manual_seed(5)
    q, k, v = (torch.randn(2, 130, 4 * 64, device="cuda", dtype=torch.bfloat16) for _ in range(3))
    out = override(None, q, k, v, 4, rdna35_attention_semantics="fixed_block_diagonal")
    ref = fixed_block_attention_bthd(q.cpu().float(), k.cpu().float(), v.cpu().float(), heads=4, causal=True)
    torch.testing.assert_close(out.float().cpu(), ref, atol=5e-2, rtol=5e-2)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("q_tokens,kv_tokens,head_dim", [(17, 31, 64), (64, 64, 128), (65, 137, 128), (129, 33, 64)])
def test_full_attention_matches_sdpa(dtype, q_tokens, kv_tokens, head_dim):
    from rdna35_block_attention import full_attention_triton

    torch.manual_seed(q_tokens + kv_tokens + head_dim)
    q = torch.randn(2, q_tokens, head_dim, device="cuda", dtype=dtype)
    k = torch.randn(2, kv_tokens, head_dim, device="cuda", dtype=dtype)
    v = torch.randn_like(k)
    out, info = full_attention_triton(q, k, v, return_diagnostics=True)
    assert info["supported"] and info["backend"] == "hip" and info["gfx950_optimized"]
    ref = F.scaled_dot_product_attention(q.float().cpu(), k.float().cpu(), v.float().cpu())
    tol = 2e-2 if dtype == torch.float16 else 5e-2
    torch.testing.assert_close(out.float().cpu(), ref, atol=tol, rtol=tol)


def test_full_attention_custom_scale_and_cross_shape():
    from rdna35_block_attention import full_attention_hip

    q = torch.randn(1, 37, 128, device="cuda", dtype=torch.float16)
    k = torch.randn(1, 71, 128, device="cuda", dtype=torch.float16)
    v = torch.randn_like(k)
    ref = F.scaled_dot_product_attention(q.float().cpu(), k.float().cpu(), v.float().cpu(), scale=0.05)
    torch.testing.assert_close(full_attention_hip(q, k, v, scale=0.05).float().cpu(), ref, atol=2e-2, rtol=2e-2)
    gen = torch.Generator().manual_seed(2)
    q = (0.5 * torch.randn(4, 1024, 128, generator=gen)).to(torch.bfloat16).cuda()
    kv = [(0.5 * torch.randn(4, 512, 128, generator=gen)).to(torch.bfloat16).cuda() for _ in range(2)]
    out = full_attention_hip(q, *kv)
    expected = oatt.dense_attention(np32(q), np32(kv[0]), np32(kv[1]))
    assert_close(np32(out), expected, 5e-2, 5e-2, "cross attention Tk=512")


@pytest.mark.parametrize("tokens,exact,sink", [(128, 1, None), (192, 2, 0), (640, 3, -1)])
def test_pisa_attention_auto_bf16_is_hip_hyd(tokens, exact, sink):
    from rdna35_block_attention import pisa_attention

    gen = torch.Generator().manual_seed(tokens)
    q, k, v = (torch.randn(2, tokens, D, generator=gen).to(torch.bfloat16).cuda() for _ in range(3))
    out, info = pisa_attention(q, k, v, exact_blocks=exact, sink_block=sink, return_diagnostics=True)
    assert info["backend"] == "hip_hyd", info
    expected = opisa.hyd_forward(np32(q), np32(k), np32(v), exact, sink_block=sink)
    assert_close(np32(out), expected, 5e-2, 5e-2, "pisa auto bf16")
    ck, info = pisa_attention(q, k, v, exact_blocks=exact, sink_block=sink, backend="ck", strict_backend=True,
                              return_diagnostics=True)
    assert info["backend"] == "hip_hyd" and torch.equal(ck, out)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_pisa_attention_triton_is_hip_centroid(dtype):
    from rdna35_block_attention import pisa_attention

    gen = torch.Generator().manual_seed(19)
    q, k, v = (torch.randn(1, 320, D, generator=gen).to(dtype).cuda() for _ in range(3))
    out, info = pisa_attention(q, k, v, exact_budget=0.5, backend="triton", strict_backend=True,
                               return_diagnostics=True)
    assert info["backend"] == "hip_centroid"
    name = "bf16" if dtype == torch.bfloat16 else "f16"
    # the reference's staged Triton backend (pisa_attention.py:310-345): Triton statistics
    # (dtype-rounded centred keys), fp32-mean selection, piecewise shared-normaliser forward
    expected, ref_scores, ref_selected = opisa.reference_forward(np32(q), np32(k), np32(v), 3, dtype=name,
                                                                 centred_keys="dtype", return_selection=True)
    assert_close(np32(out), expected, 5e-2, 5e-2, "pisa triton backend")
    import mi355x_pisa

    _, scores, idx = mi355x_pisa.forward_with_routing(q.unsqueeze(1), k.unsqueeze(1), v.unsqueeze(1), 3, D ** -0.5,
                                                      mode="generic")
    assert_close(np32(scores), ref_scores, 1e-4, 1e-4, "triton backend routing scores")
    kernel_selected = opisa.selection_mask(idx.cpu().numpy().astype(np.int64), ref_selected.shape[-1])
    np.testing.assert_array_equal(kernel_selected, ref_selected)
    if dtype == torch.float16:
        _, auto = pisa_attention(q, k, v, exact_budget=0.5, return_diagnostics=True)
        assert auto["backend"] == "hip_centroid"
        with pytest.raises(RuntimeError, match="CK backend unavailable"):
            pisa_attention(q, k, v, backend="ck", strict_backend=True)


def test_pisa_attention_reference_backend_on_gpu_matches_oracle():
    from rdna35_block_attention import pisa_attention

    gen = torch.Generator().manual_seed(23)
    q, k, v = (torch.randn(2, 200, D, generator=gen).to(torch.bfloat16).cuda() for _ in range(3))
    out = pisa_attention(q, k, v, exact_blocks=2, backend="reference")
    expected = opisa.reference_forward(np32(q), np32(k), np32(v), 2)
    assert_close(np32(out), expected, 2e-2, 2e-2, "reference backend")


def test_anima_attn_op_end_to_end():
    import mi355x_pisa
    from mi355x_pisa.synthetic import anima_qkv
    from rdna35_block_attention.anima_pisa_integration import make_anima_pisa_attn_op
    from rdna35_block_attention.pisa_runtime import PISARuntimeState

    q4, k4, v4 = anima_qkv(batch=1, heads=16, seed=11, device="cuda")
    q, k, v = (t.permute(0, 2, 1, 3) for t in (q4, k4, v4))  # contiguous [B,T,H,D]
    assert q.is_contiguous()
    state = PISARuntimeState(armed=True)
    op = make_anima_pisa_attn_op(lambda *a, **kw: "original", native_forward=mi355x_pisa.forward_spatial_bhtd,
                                 exact_blocks=23, device_index=torch.cuda.current_device(), layer_index=20,
                                 runtime_state=state)
    out = op(q, k, v)
    assert out.shape == (1, 9216, 16 * D) and state.per_layer_hits[20] == 1
    heads = (0, 7)
    sub = [t[:, list(heads)] for t in (q4, k4, v4)]
    packed = [spatial_to_packed(t, 1, 96, 96) for t in sub]
    expected = packed_to_merged(opisa.hyd_forward(*packed, 23), 1, 2, 1, 96, 96)
    got = np32(out).reshape(1, 9216, 16, D)[:, :, list(heads)].reshape(1, 9216, 2 * D)
    assert_close(got, expected, 5e-2, 5e-2, "anima layers")


def test_generic_override_on_video_grid():
    from mi355x_pisa.synthetic import video_qkv
    from rdna35_block_attention.generic_pisa import make_generic_pisa_override
    from rdna35_block_attention.pisa_runtime import PISARuntimeState

    grid = (2, 64, 64)
    heads = 2
    q4, k4, v4 = video_qkv(batch=1, heads=heads, grid=grid, seed=4, device="cuda")
    merged = [t.permute(0, 2, 1, 3).reshape(1, 8192, heads * D) for t in (q4, k4, v4)]
    state = PISARuntimeState(armed=True)
    override = make_generic_pisa_override(exact_budget=0.15625, device_index=torch.cuda.current_device(),
                                          previous_override=None, runtime_state=state)
    out = override(lambda *a, **kw: "original", *merged, heads, is_self_attention=True,
                   transformer_options={"grid_sizes": grid})
    # T = 8192, D = 128, bf16: routed on the HYD statistics, as the reference (generic_pisa.py:120-126)
    assert state.backend_counts["hip_generic_hyd"] == 1, state.report()
    packed = [spatial_to_packed(t, *grid) for t in (q4, k4, v4)]
    expected = packed_to_merged(opisa.generic_forward(*packed, 20, dtype="bf16", stats="hyd"), 1, heads, *grid)
    assert_close(np32(out), expected, 5e-2, 5e-2, "generic video override")


@pytest.mark.parametrize("head_dim,dtype", [(40, torch.float16), (80, torch.float16), (160, torch.float16),
                                             (64, torch.bfloat16)])
def test_generic_override_sd_head_dims(head_dim, dtype):
    """SD1.5 / SDXL-style flattened self-attention (tests/test_generic_pisa.py:93-125 profiles) on the HIP path:
    no first-order term and a budget of at least 0.25 off 128 bf16 (generic_pisa.py:332-333)."""
    from rdna35_block_attention.generic_pisa import make_generic_pisa_override
    from rdna35_block_attention.pisa_runtime import PISARuntimeState

    heads, tokens = 2, 8192
    gen = torch.Generator().manual_seed(head_dim)
    merged = [torch.randn((1, tokens, heads * head_dim), generator=gen).to(dtype).cuda() for _ in range(3)]
    state = PISARuntimeState(armed=True)
    override = make_generic_pisa_override(exact_budget=0.15625, device_index=torch.cuda.current_device(),
                                          previous_override=None, runtime_state=state)
    out = override(lambda *a, **kw: "original", *merged, heads, is_self_attention=True, transformer_options={})
    assert state.backend_counts["hip_generic_0th"] == 1, state.report()
    assert out.shape == (1, tokens, heads * head_dim)
    bhtd = [np32(t).reshape(1, tokens, heads, head_dim).transpose(0, 2, 1, 3).reshape(heads, tokens, head_dim)
            for t in merged]
    exact = math.ceil(0.25 * (tokens // 64))  # budget raised to 0.25
    name = "bf16" if dtype == torch.bfloat16 else "f16"
    ref = opisa.generic_forward(*bhtd, exact, first_order=False, dtype=name)
    expected = ref.reshape(1, heads, tokens, head_dim).transpose(0, 2, 1, 3).reshape(1, tokens, heads * head_dim)
    tol = 2e-2 if dtype == torch.float16 else 5e-2
    assert_close(np32(out), expected, tol, tol, f"generic override D={head_dim}")


@pytest.mark.parametrize("tokens", [4608, 17000])  # 17000: past the reference's pack bound (16500)
def test_h3_override_reads_strided_views(tokens):
    from rdna35_block_attention.minimax_h3_attention import make_minimax_h3_attention_override

    heads = 56
    gen = torch.Generator().manual_seed(tokens)
    qkv = torch.randn((1, tokens, 3, heads, D), generator=gen).to(torch.bfloat16).cuda()
    q, k, v = (qkv[:, :, i].permute(0, 2, 1, 3) for i in range(3))
    override = make_minimax_h3_attention_override(device_index=torch.cuda.current_device(), verbose_fallbacks=False,
                                                  previous_override=None)
    out = override(None, q, k, v, heads, skip_reshape=True)
    assert out.shape == (1, tokens, heads * D)
    import mi355x_pisa

    packed = mi355x_pisa.dense_attention(q.contiguous(), k.contiguous(), v.contiguous(), D ** -0.5,
                                         merged_output=True)
    assert torch.equal(out, packed)
    sel = [0, 55]
    rows = slice(0, 1024)  # query rows checked against the oracle (all keys)
    expected = oatt.dense_attention(np32(q[:, sel, rows]), np32(k[:, sel]), np32(v[:, sel]))
    got = np32(out).reshape(1, tokens, heads, D)[:, rows][:, :, sel].transpose(0, 2, 1, 3)
    assert_close(got, expected, 5e-2, 5e-2, "h3 heads")


@pytest.mark.parametrize("head_dim,grid", [(128, None), (64, (2, 64, 64))])
def test_generic_debug_finite_checks_every_stage(head_dim, grid):
    """debug_finite (generic_pisa.py:172-219): finite inputs pass every stage check and give the same bits as
    the plain call; an infinite key fails the statistics stage."""
    from rdna35_block_attention.generic_pisa import generic_pisa_attention

    torch.manual_seed(head_dim)
    tokens = 8192
    q, k, v = (torch.randn(2, tokens, head_dim, device="cuda", dtype=torch.bfloat16) for _ in range(3))
    print(f"debug_finite D={head_dim} grid={grid}", flush=True)
    plain = generic_pisa_attention(q, k, v, exact_budget=0.15, grid_sizes=grid)
    checked = generic_pisa_attention(q, k, v, exact_budget=0.15, grid_sizes=grid, debug_finite=True)
    assert torch.equal(plain, checked)
    k_bad = k.clone()
    k_bad[1, 100, 3] = float("inf")
    with pytest.raises(ValueError, match="non-finite stages: .*k_centroids"):
        generic_pisa_attention(q, k_bad, v, exact_budget=0.15, grid_sizes=grid, debug_finite=True)
