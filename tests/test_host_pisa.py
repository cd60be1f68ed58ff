"""Host logic of the PISA entry points and ComfyUI patches (CPU, fakes only).

Mirrors tests/test_pisa_attention.py, test_pisa_patch.py,
test_anima_pisa_integration.py, test_pisa_runtime.py,
test_pisa_runtime_report.py, test_generic_pisa.py and
test_minimax_h3_gfx1151_attention.py of the reference.  Native calls are
replaced by mocks; a FakeCudaTensor reports device cuda:N on the CPU.
"""
from __future__ import annotations

import math
from types import SimpleNamespace
from unittest import mock

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import pisa as opisa
from rdna35_block_attention import anima_pisa_integration as anima
from rdna35_block_attention import diagnostics, generic_pisa, minimax_h3_attention as h3, pisa_patch
from rdna35_block_attention.pisa_attention import _reference_block_stats, pisa_attention
from rdna35_block_attention.pisa_runtime import PISARuntimeState

D = 128


class FakeCudaTensor(torch.Tensor):
    device_index = 0

    @staticmethod
    def __new__(cls, tensor):
        return torch.Tensor._make_subclass(cls, tensor, tensor.requires_grad)

    @property
    def device(self):
        return torch.device("cuda", self.device_index)

    @property
    def is_cuda(self):
        return True


class OtherFakeCudaTensor(FakeCudaTensor):
    device_index = 1


def _inputs(tokens=128, dtype=torch.float16):
    gen = torch.Generator().manual_seed(1234)
    return tuple(torch.randn((2, tokens, D), generator=gen).to(dtype).contiguous() for _ in range(3))


def _dense(q, k, v):
    return F.scaled_dot_product_attention(q.float()[:, None], k.float()[:, None], v.float()[:, None])[:, 0]


# ----------------------------------------------------------------------------- pisa_attention (reference backend)
def test_exact_budget_one_matches_dense():
    q, k, v = _inputs()
    out, info = pisa_attention(q, k, v, exact_budget=1.0, backend="reference", return_diagnostics=True)
    torch.testing.assert_close(out.float(), _dense(q, k, v), atol=2e-3, rtol=2e-3)
    assert info["exact_blocks_per_query"] == 2 and info["approximate_blocks_per_query"] == 0
    assert info["exact_online_softmax"]


def test_centered_tail_uses_numerator_and_denominator():
    q, _, v = _inputs()
    gen = torch.Generator().manual_seed(4321)
    k = torch.randn((2, 2, D), generator=gen).to(torch.float16).repeat_interleave(64, dim=1).contiguous()
    out, info = pisa_attention(q, k, v, exact_blocks=0, backend="reference", return_diagnostics=True)
    torch.testing.assert_close(out.float(), _dense(q, k, v), atol=2e-3, rtol=2e-3)
    assert info["tail_approximation"] == "block_centered_zeroth_plus_global_first_order"
    assert info["shared_numerator_denominator_normalization"]


def test_approximation_tracks_dense_on_clustered_keys():
    q, _, v = _inputs(192)
    gen = torch.Generator().manual_seed(99)
    centers = torch.randn((2, 3, D), generator=gen)
    noise = torch.randn((2, 192, D), generator=gen) * 0.01
    k = (centers.repeat_interleave(64, dim=1) + noise).to(torch.bfloat16).contiguous()
    q, v = q.to(torch.bfloat16), v.to(torch.bfloat16)
    out = pisa_attention(q, k, v, sparsity=2 / 3, backend="reference")
    assert torch.isfinite(out).all()
    assert (out.float() - _dense(q, k, v)).abs().mean().item() < 0.02


@pytest.mark.parametrize("tokens,exact,sink", [(128, 1, None), (200, 2, 0), (65, 1, -1), (256, 0, None)])
def test_reference_backend_matches_oracle(tokens, exact, sink):
    q, k, v = (x.to(torch.bfloat16) for x in _inputs(tokens))
    out = pisa_attention(q, k, v, exact_blocks=exact, sink_block=sink, backend="reference")
    expected = opisa.reference_forward(*(x.float().numpy() for x in (q, k, v)), exact, sink_block=sink)
    np.testing.assert_allclose(out.float().numpy(), expected, atol=2e-2, rtol=2e-2)


def test_reference_block_stats_against_oracle():
    q, k, v = _inputs(200)
    k_means, v_sums, h_sum, lengths = _reference_block_stats(k, v, 64)
    assert lengths == [64, 64, 64, 8]
    st = opisa.block_stats(*(x.float().numpy() for x in (q, k, v)), "generic", "f32")
    np.testing.assert_allclose(k_means.numpy(), st["k_centroids"], rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(h_sum.numpy(), st["h_sum"], rtol=1e-4, atol=1e-3)


def test_shape_dtype_and_training_validation():
    q, k, v = _inputs()
    with pytest.raises(ValueError, match="D=128"):
        pisa_attention(q[..., :64].contiguous(), k[..., :64].contiguous(), v[..., :64].contiguous())
    with pytest.raises(ValueError, match="identical"):
        pisa_attention(q, k[:, :-1].contiguous(), v)
    with pytest.raises(ValueError, match="fp16/bf16"):
        pisa_attention(q.float(), k.float(), v.float())
    with pytest.raises(ValueError, match="requiring gradients"):
        pisa_attention(q.clone().requires_grad_(), k, v)
    with pytest.raises(ValueError, match="block_size=64"):
        pisa_attention(q, k, v, block_size=32)


def test_budget_validation_and_fallback_reporting():
    q, k, v = _inputs()
    with pytest.raises(ValueError, match="only one"):
        pisa_attention(q, k, v, exact_budget=0.5, sparsity=0.5)
    with pytest.raises(ValueError, match="backend"):
        pisa_attention(q, k, v, backend="unknown")
    for backend in ("triton", "ck", "hip", "auto"):
        out, info = pisa_attention(q, k, v, exact_budget=0.5, backend=backend, return_diagnostics=True)
        assert info["backend"] == "reference"
        assert "requires_cuda_hip" in info["fallback_reason"]
        assert torch.isfinite(out).all()
    with pytest.raises(RuntimeError, match="Triton backend unavailable"):
        pisa_attention(q, k, v, backend="triton", strict_backend=True)
    with pytest.raises(RuntimeError, match="CK backend unavailable"):
        pisa_attention(q, k, v, backend="ck", strict_backend=True)


# ----------------------------------------------------------------------------- Anima override (pisa_patch)
TOKENS = 64


def _tensor(shape=(1, 2, TOKENS, D), *, value=0.0, dtype=torch.bfloat16, requires_grad=False, cls=FakeCudaTensor):
    b, h, t, d = shape
    storage = torch.full((b, t, h, d), value, dtype=dtype, requires_grad=requires_grad)
    return cls(storage.permute(0, 2, 1, 3))


class DummyModel:
    def __init__(self, transformer_options=None):
        self.model_options = {"transformer_options": dict(transformer_options or {})}

    def clone(self):
        return DummyModel(self.model_options["transformer_options"])


def _make_override(previous=None, native=None):
    return pisa_patch.make_pisa_attention_override(
        exact_budget=0.25, allowed_tokens=frozenset((TOKENS,)), expected_token_shape=(1, 8, 8), device_index=0,
        native_forward=native or mock.Mock(name="native_forward"), verbose_fallbacks=False,
        previous_override=previous)


def _native_module():
    native = mock.Mock()
    native.build_info.return_value = {"api": 1, "architecture": "gfx950"}
    native.capabilities.return_value = {"spatial_sparse_exact_blocks": (23,)}
    return native


def test_patch_is_installed_only_on_cloned_model():
    previous = mock.Mock(name="previous_override")
    model = DummyModel({"optimized_attention_override": previous})
    with mock.patch.object(pisa_patch, "_gfx950_device_index", return_value=(0, None)), \
            mock.patch.object(diagnostics, "load_native", return_value=_native_module()):
        patched, _ = pisa_patch.patch_model_pisa_attention(model, enabled=True, exact_budget=0.15625,
                                                           token_policy="auto_9216", verbose_fallbacks=False)
    assert patched is not model
    assert model.model_options["transformer_options"]["optimized_attention_override"] is previous
    assert patched.model_options["transformer_options"]["optimized_attention_override"] is not previous


def test_generic_patch_for_non_anima_models_and_rejections():
    model = DummyModel()
    with mock.patch.object(pisa_patch, "_gfx950_device_index", return_value=(0, None)):
        patched, info = pisa_patch.patch_model_pisa_attention(model, enabled=True, exact_budget=0.25,
                                                              token_policy="auto_9216", verbose_fallbacks=False)
    assert patched is not model and "generic gfx950 PISA" in info
    for kwargs in (dict(enabled=False), dict(exact_budget=1.5), dict(token_policy="x"), dict(start_layer=30)):
        args = dict(enabled=True, exact_budget=0.25, token_policy="auto_9216", verbose_fallbacks=False)
        args.update(kwargs)
        assert pisa_patch.patch_model_pisa_attention(model, **args)[0] is model
    with mock.patch.object(pisa_patch, "_gfx950_device_index", return_value=(None, "gfx950 is required, got gfx90a")):
        kept, info = pisa_patch.patch_model_pisa_attention(model, enabled=True, exact_budget=0.25,
                                                           token_policy="auto_9216", verbose_fallbacks=False)
    assert kept is model and "gfx950 is required" in info


def test_explicit_self_attention_marker_is_required():
    q, k, v = _tensor(value=1.0), _tensor(value=2.0), _tensor(value=3.0)
    previous = mock.Mock(return_value="previous")
    native = mock.Mock(return_value=torch.zeros((1, TOKENS, 2 * D), dtype=q.dtype))
    override = _make_override(previous, native)
    assert override(mock.Mock(), q, k, v, 2, skip_reshape=True) == "previous"
    assert override(mock.Mock(), q, k, v, 2, skip_reshape=True, is_self_attention=False) == "previous"
    override(mock.Mock(), q, k, v, 2, skip_reshape=True, is_self_attention=True, is_initial_transformer_block=False,
             attention_token_shape=(1, 8, 8))
    assert previous.call_count == 2
    native.assert_called_once()


def test_unsupported_calls_chain_previous_or_original():
    q = torch.zeros((1, 2, 64, D), dtype=torch.bfloat16)
    previous, original = mock.Mock(return_value="previous"), mock.Mock(return_value="original")
    assert _make_override(previous)(original, q, q, q, 2, skip_reshape=True, is_self_attention=False) == "previous"
    original.assert_not_called()
    assert _make_override()(original, q, q, q, 2, skip_reshape=True, is_self_attention=False) == "original"


def test_ineligible_calls_never_enter_native_pisa():
    q, k, v = _tensor(value=1.0), _tensor(value=2.0), _tensor(value=3.0)
    triple = lambda **kw: (_tensor(**kw),) * 3  # noqa: E731
    cases = (
        ((q, k, v), {"mask": object(), "skip_reshape": True}),
        ((q, k, v), {"skip_reshape": False}),
        ((q, k, v), {"skip_reshape": True, "skip_output_reshape": True}),
        ((q, _tensor(shape=(1, 2, TOKENS - 1, D)), v), {"skip_reshape": True}),
        ((q, k, v), {"heads": 1, "skip_reshape": True}),
        (triple(shape=(1, 2, TOKENS, 64)), {"skip_reshape": True}),
        (triple(dtype=torch.float16), {"skip_reshape": True}),
        ((q, _tensor(dtype=torch.float16), v), {"skip_reshape": True}),
        ((q, _tensor(cls=OtherFakeCudaTensor), v), {"skip_reshape": True}),
        ((_tensor(requires_grad=True), k, v), {"skip_reshape": True}),
        (triple(shape=(1, 2, 128, D)), {"skip_reshape": True}),
        ((q, k, v), {"attn_precision": torch.float32, "skip_reshape": True}),
        ((q, k, v), {"enable_gqa": True, "skip_reshape": True}),
        (tuple(t.contiguous() for t in (q, k, v)), {"skip_reshape": True, "attention_token_shape": (1, 8, 8)}),
    )
    for tensors, kwargs in cases:
        heads = kwargs.pop("heads", 2)
        kwargs.setdefault("attention_token_shape", (1, 8, 8))
        previous, native = mock.Mock(return_value="previous"), mock.Mock()
        result = _make_override(previous, native)(mock.Mock(), *tensors, heads, is_self_attention=True,
                                                  is_initial_transformer_block=False, **kwargs)
        assert result == "previous", kwargs
        native.assert_not_called()
    cpu = torch.zeros((1, 2, TOKENS, D), dtype=torch.bfloat16)
    previous, native = mock.Mock(return_value="previous"), mock.Mock()
    assert _make_override(previous, native)(mock.Mock(), cpu, cpu, cpu, 2, skip_reshape=True, is_self_attention=True,
                                            is_initial_transformer_block=False) == "previous"
    native.assert_not_called()


def test_eligible_call_forwards_bhtd_views_and_merged_output():
    batch, heads = 2, 2
    q, k, v = (_tensor((batch, heads, TOKENS, D), value=x) for x in (1.0, 2.0, 3.0))
    merged = torch.arange(batch * TOKENS * heads * D, dtype=q.dtype).reshape(batch, TOKENS, heads * D)
    native = mock.Mock(return_value=merged)
    out = _make_override(native=native)(mock.Mock(), q, k, v, heads, skip_reshape=True, is_self_attention=True,
                                        is_initial_transformer_block=False, attention_token_shape=(1, 8, 8))
    args = native.call_args.args
    assert args[0] is q and args[1] is k and args[2] is v
    assert args[3] == 1  # ceil(0.25 * 1 block)
    assert out is merged


def test_native_exception_propagates_without_fallback():
    q = _tensor(value=1.0)
    previous, original = mock.Mock(return_value="previous"), mock.Mock(return_value="original")
    override = _make_override(previous, mock.Mock(side_effect=RuntimeError("native failure")))
    with pytest.raises(RuntimeError, match="native failure"):
        override(original, q, q, q, 2, skip_reshape=True, is_self_attention=True, is_initial_transformer_block=False,
                 attention_token_shape=(1, 8, 8))
    previous.assert_not_called()
    original.assert_not_called()


def test_initial_block_chains_to_previous():
    q = _tensor(value=1.0)
    previous, native = mock.Mock(return_value="previous"), mock.Mock()
    result = _make_override(previous, native)(mock.Mock(), q, q, q, 2, skip_reshape=True, is_self_attention=True,
                                              is_initial_transformer_block=True, attention_token_shape=(1, 8, 8))
    assert result == "previous"
    native.assert_not_called()


# ----------------------------------------------------------------------------- Anima direct attn_op
def _qkv(tokens=anima.ANIMA_PISA_TOKENS, dtype=torch.bfloat16):
    t = FakeCudaTensor(torch.zeros((1, tokens, anima.ANIMA_PISA_HEADS, anima.ANIMA_PISA_HEAD_DIM), dtype=dtype))
    return t, t, t


class DummyPatcher:
    def __init__(self):
        attn = lambda: SimpleNamespace(n_heads=16, head_dim=128, attn_op=mock.Mock())  # noqa: E731
        self.model = SimpleNamespace(blocks=[SimpleNamespace(self_attn=attn()) for _ in range(28)])
        self.object_patches = {}
        self.attachments = {}

    def get_model_object(self, name):
        return self.model

    def add_object_patch(self, name, value):
        self.object_patches[name] = value

    def clone(self):
        return self

    model_options = {"transformer_options": {}}

    def set_attachments(self, key, value):
        self.attachments[key] = value


def test_direct_op_hits_native_without_markers():
    q, k, v = _qkv()
    out_shape = (1, anima.ANIMA_PISA_TOKENS, anima.ANIMA_PISA_HEADS * anima.ANIMA_PISA_HEAD_DIM)
    native = mock.Mock(return_value=torch.zeros(out_shape, dtype=torch.bfloat16))
    original = mock.Mock()
    state = PISARuntimeState(armed=True)
    op = anima.make_anima_pisa_attn_op(original, native_forward=native, exact_blocks=23, device_index=0,
                                       layer_index=4, runtime_state=state)
    assert op(q, k, v).shape == out_shape
    original.assert_not_called()
    assert native.call_args.kwargs["exact_blocks"] == 23
    assert native.call_args.args[0].shape == (1, 16, 9216, 128)
    assert native.call_args.args[0].stride() == (9216 * 16 * 128, 128, 16 * 128, 1)  # a view, no copy
    assert state.per_layer_hits == {4: 1}
    assert state.shape_counts[(1, 16, 9216, 128)] == 1


def test_other_profile_chains_original_op():
    q, k, v = _qkv(tokens=64)
    original = mock.Mock(return_value="fallback")
    state = PISARuntimeState(armed=True)
    op = anima.make_anima_pisa_attn_op(original, native_forward=mock.Mock(), exact_blocks=23, device_index=0,
                                       layer_index=4, runtime_state=state)
    assert op(q, k, v) == "fallback"
    original.assert_called_once_with(q, k, v, transformer_options=None)
    assert state.fallback_reasons["shape_(64, 16, 128)_is_not_t9216_h16_d128"] == 1


def test_eligible_native_failure_is_loud():
    state = PISARuntimeState(armed=True)
    op = anima.make_anima_pisa_attn_op(mock.Mock(), native_forward=mock.Mock(side_effect=ValueError("boom")),
                                       exact_blocks=23, device_index=0, layer_index=4, runtime_state=state)
    with pytest.raises(RuntimeError, match="eligible Anima"):
        op(*_qkv())
    assert state.failed


def test_installs_requested_layer_range_and_full_patch():
    patcher = DummyPatcher()
    assert anima.install_anima_pisa_attention(patcher, native_forward=mock.Mock(), exact_blocks=23, device_index=0,
                                              first_layer=8, last_layer=19) == 12
    assert "diffusion_model.blocks.7.self_attn.attn_op" not in patcher.object_patches
    assert "diffusion_model.blocks.8.self_attn.attn_op" in patcher.object_patches
    assert "diffusion_model.blocks.20.self_attn.attn_op" not in patcher.object_patches
    fresh = DummyPatcher()
    with mock.patch.object(pisa_patch, "_gfx950_device_index", return_value=(0, None)), \
            mock.patch.object(diagnostics, "load_native", return_value=_native_module()):
        patched, info = pisa_patch.patch_model_pisa_attention(fresh, enabled=True, exact_budget=0.15625,
                                                               token_policy="anima_1536_spatial",
                                                               verbose_fallbacks=True)
    assert "exact_blocks=23" in info and len(patched.object_patches) == 8
    with mock.patch.object(pisa_patch, "_gfx950_device_index", return_value=(0, None)), \
            mock.patch.object(diagnostics, "load_native", return_value=_native_module()):
        kept, info = pisa_patch.patch_model_pisa_attention(DummyPatcher(), enabled=True, exact_budget=0.25,
                                                           token_policy="auto_9216", verbose_fallbacks=False)
    assert "selects 36 blocks" in info


# ----------------------------------------------------------------------------- runtime accounting
def test_runtime_state_verify_report_reset():
    state = PISARuntimeState(armed=True, expected_layers=(20, 21))
    assert PISARuntimeState.expected_calls(3, layers=(20, 21)) == 6
    for layer in (20, 21):
        state.record(layer=layer, is_self_attention=True, shape=(1, 16, 9216, 128), backend="hip", context="x")
    state.record(is_self_attention=False, fallback_reason="cross")
    assert state.verify(1)
    report = state.report()
    assert "verified=1" in report and "hits=2/2" in report and "cross:1" in report and "hip:2" in report
    state.record(layer=20, is_self_attention=True)
    assert not state.verify(1)
    assert state.first_error == "PISA hits=3, expected=2"
    state.reset(armed=False)
    assert not state.armed and sum(state.per_layer_hits.values()) == 0 and state.first_error is None
    with pytest.raises(ValueError):
        PISARuntimeState.expected_calls(-1)
    state.record(error=RuntimeError("x"))
    assert not state.verify(0)
    state.mark_profile_validated(("a",))
    assert state.is_profile_validated(("a",))


# ----------------------------------------------------------------------------- generic override
def _cuda_tensor(shape, dtype=torch.float16, cls=FakeCudaTensor):
    return cls(torch.zeros(shape, dtype=dtype))


def test_spatial_and_video_round_trips_match_oracle_order():
    from oracle import layout as olayout

    tensor = torch.arange(2 * 3 * 256 * 4).reshape(2, 3, 256, 4)
    packed = generic_pisa._pack_spatial_blocks(tensor, 16)
    assert not torch.equal(packed, tensor)
    torch.testing.assert_close(generic_pisa._unpack_spatial_blocks(packed, 16), tensor)
    for grid in ((4, 16, 16), (2, 32, 64)):
        tokens = math.prod(grid)
        x = torch.arange(2 * 3 * tokens * 4).reshape(2, 3, tokens, 4)
        p = generic_pisa._pack_video_blocks(x, grid)
        torch.testing.assert_close(generic_pisa._unpack_video_blocks(p, grid), x)
        np.testing.assert_array_equal(p[0, 0, :, 0].numpy() // 4, olayout.tile_order(*grid))


def test_generic_profiles_route_through_hip_generic():
    profiles = (("sd15", 8, 40), ("sd15", 8, 80), ("sd15", 8, 160), ("sdxl", 10, 64), ("wan", 12, 128),
                ("ltx", 16, 64))
    for _, heads, head_dim in profiles:
        q = _cuda_tensor((1, generic_pisa.MIN_TOKENS, heads * head_dim))
        state = PISARuntimeState(armed=True)
        override = generic_pisa.make_generic_pisa_override(exact_budget=0.25, device_index=0, previous_override=None,
                                                           runtime_state=state)
        out = torch.zeros((1, generic_pisa.MIN_TOKENS, heads, head_dim), dtype=q.dtype)
        with mock.patch.object(generic_pisa, "_generic_pisa_bhtd", return_value=(out, "hip_generic")) as run:
            result = override(mock.Mock(), q, q, q, heads, is_self_attention=True,
                              transformer_options={"block": ("output", 4), "block_index": 1})
        assert result.shape == q.shape
        assert run.call_args.args[3] == 0.25  # budget
        assert run.call_args.args[5] == (head_dim == 128 and q.dtype == torch.bfloat16)  # first order
        assert state.backend_counts["hip_generic"] == 1 and state.per_layer_hits[-1] == 1
        assert state.hit_context_counts["output:4:1"] == 1


def test_wan_grid_is_passed_to_the_kernel():
    heads, head_dim = 2, 8
    for grid in ((2, 64, 64), (4, 32, 64)):
        tokens = math.prod(grid)
        q = FakeCudaTensor(torch.randn(1, tokens, heads * head_dim).to(torch.float16))
        state = PISARuntimeState(armed=True)
        override = generic_pisa.make_generic_pisa_override(exact_budget=0.25, device_index=0, previous_override=None,
                                                           runtime_state=state)

        def identity(q4, k4, v4, budget, scale, first_order, token_grid):
            assert token_grid == grid
            return q4.transpose(1, 2).contiguous(), "hip_generic"

        with mock.patch.object(generic_pisa, "_generic_pisa_bhtd", side_effect=identity):
            out = override(mock.Mock(), q, q, q, heads, is_self_attention=True, transformer_options={"grid_sizes": grid})
        assert torch.equal(out.as_subclass(torch.Tensor), q.as_subclass(torch.Tensor))


def test_square_input_stage_stays_dense_and_fallback_reasons():
    heads, head_dim = 10, 64
    q = _cuda_tensor((1, 9216, heads * head_dim))
    previous = mock.Mock(return_value="dense")
    state = PISARuntimeState(armed=True)
    override = generic_pisa.make_generic_pisa_override(exact_budget=0.25, device_index=0, previous_override=previous,
                                                       runtime_state=state)
    assert override(mock.Mock(), q, q, q, heads, is_self_attention=True,
                    transformer_options={"block": ("input", 4), "block_index": 0}) == "dense"
    assert state.fallback_reasons["spatial_input_stage_uses_dense_attention"] == 1

    heads, head_dim = 4, 16
    mt = generic_pisa.MIN_TOKENS
    eligible = _cuda_tensor((1, mt, heads * head_dim))
    short = _cuda_tensor((1, mt - 64, heads * head_dim))
    cached = _cuda_tensor((1, mt + 64, heads * head_dim))
    other = _cuda_tensor(eligible.shape, cls=OtherFakeCudaTensor)
    bf16 = _cuda_tensor(eligible.shape, dtype=torch.bfloat16)
    previous = mock.Mock(return_value="fallback")
    state = PISARuntimeState(armed=True)
    override = generic_pisa.make_generic_pisa_override(exact_budget=0.25, device_index=0, previous_override=previous,
                                                       runtime_state=state)
    cases = (
        (eligible, eligible, eligible, {"is_self_attention": False}, "not_explicit_self_attention"),
        (eligible, eligible, eligible, {"is_self_attention": True, "mask": torch.ones(1)}, "attention_mask_is_not_supported"),
        (eligible, eligible, eligible, {"is_self_attention": True, "enable_gqa": True}, "gqa_is_not_supported"),
        (eligible, eligible, eligible, {"is_self_attention": True, "is_kv_cached_attention": True},
         "kv_cached_attention_is_not_supported"),
        (eligible, other, other, {"is_self_attention": True}, "qkv_must_share_one_device"),
        (eligible, bf16, bf16, {"is_self_attention": True}, "matching_fp16_or_bf16_qkv_are_required"),
        (short, short, short, {"is_self_attention": True}, f"tokens_{mt - 64}_below_{mt}"),
        (eligible, cached, cached, {"is_self_attention": True}, "matching_btc_qkv_divisible_by_heads_are_required"),
    )
    for q_, k_, v_, kwargs, reason in cases:
        assert override(mock.Mock(), q_, k_, v_, heads, **kwargs) == "fallback"
        assert state.fallback_reasons[reason] == 1, reason


def test_backend_errors_fall_back_but_oom_and_missing_library_are_loud():
    heads, head_dim = 4, 16
    q = _cuda_tensor((1, generic_pisa.MIN_TOKENS, heads * head_dim))
    previous = mock.Mock(return_value="fallback")
    state = PISARuntimeState(armed=True)
    override = generic_pisa.make_generic_pisa_override(exact_budget=0.25, device_index=0, previous_override=previous,
                                                       runtime_state=state)
    with mock.patch.object(generic_pisa, "_generic_pisa_bhtd", side_effect=ValueError("head_dim 16")):
        assert override(mock.Mock(), q, q, q, heads, is_self_attention=True) == "fallback"
    assert state.fallback_reasons["pisa_backend_error_ValueError"] == 1
    for exc in (torch.OutOfMemoryError("oom"), diagnostics.NativeUnavailableError("missing")):
        with mock.patch.object(generic_pisa, "_generic_pisa_bhtd", side_effect=exc):
            with pytest.raises(type(exc)):
                override(mock.Mock(), q, q, q, heads, is_self_attention=True)
    bad = torch.full((1, generic_pisa.MIN_TOKENS, heads, head_dim), torch.nan, dtype=q.dtype)
    with mock.patch.object(generic_pisa, "_generic_pisa_bhtd", return_value=(bad, "hip_generic_0th")):
        assert override(mock.Mock(), q, q, q, heads, is_self_attention=True) == "fallback"
    assert state.fallback_reasons["pisa_backend_error_ValueError"] == 2
    assert sum(state.per_layer_hits.values()) == 0


# ----------------------------------------------------------------------------- MiniMax-H3
class H3Model:
    def __init__(self, diffusion_model=None):
        self.diffusion_model = diffusion_model
        self.model_options = {"transformer_options": {}}

    def get_model_object(self, name):
        if name != "diffusion_model" or self.diffusion_model is None:
            raise KeyError(name)
        return self.diffusion_model

    def clone(self):
        cloned = H3Model(self.diffusion_model)
        cloned.model_options = {"transformer_options": dict(self.model_options["transformer_options"])}
        return cloned


def _h3_model():
    cls = type("MiniMaxH3Model", (), {})
    cls.__module__ = "comfy.ldm.minimax.model"
    inner = cls()
    inner.blocks, inner.hidden_size = [], 5376
    return H3Model(inner)


def test_h3_pack_profiles_keep_values_in_one_allocation():
    short = torch.arange(9170 * 3, dtype=torch.float32).reshape(1, 9170, 3, 1, 1)
    q, k, v = (short[:, :, i].permute(0, 2, 1, 3) for i in range(3))
    pq, pk, pv, profile = h3.pack_minimax_h3_qkv(q, k, v)
    assert profile == "kv" and pq is q and pk.is_contiguous() and torch.equal(pk, k) and torch.equal(pv, v)
    assert pk._base is pv._base
    long = torch.arange(12000 * 3, dtype=torch.float32).reshape(1, 12000, 3, 1, 1)
    q, k, v = (long[:, :, i].permute(0, 2, 1, 3) for i in range(3))
    pq, pk, pv, profile = h3.pack_minimax_h3_qkv(q, k, v)
    assert profile == "qkv" and torch.equal(pq, q) and pq._base is pk._base is pv._base


def test_h3_reject_reasons():
    q = torch.randn(1, 56, 8, 128, dtype=torch.bfloat16)
    assert h3._reject_reason(q, q, q, 56, None, True, False, 0, {}) == "tokens_below_4608"
    longer = torch.empty(1, 56, 16501, 128, dtype=torch.bfloat16, device="meta")  # past the reference's pack bound
    assert h3._reject_reason(longer, longer, longer, 56, None, True, False, 0, {}) == \
        "matching_rocm_qkv_device_is_required"
    big = torch.empty(1, 56, 65537, 128, dtype=torch.bfloat16, device="meta")
    assert h3._reject_reason(big, big, big, 56, None, True, False, 0, {}) == "tokens_above_65536"
    ok = torch.empty(1, 56, 9170, 128, dtype=torch.bfloat16, device="meta")
    assert h3._reject_reason(ok, ok, ok, 56, None, True, False, 0, {"is_causal": True}) == \
        "causal_attention_is_not_supported"
    assert h3._reject_reason(ok, ok, ok, 56, object(), True, False, 0, {}) == "attention_mask_is_not_supported"
    assert h3._reject_reason(ok, ok, ok, 56, None, False, False, 0, {}) == "minimax_h3_merged_output_contract_is_required"
    assert h3._reject_reason(ok, ok, ok, 56, None, True, False, 0, {}) == "matching_rocm_qkv_device_is_required"


def test_h3_override_chains_unsupported_calls_and_patch_rules():
    q = torch.randn(1, 2, 3, 4)
    calls = []

    def previous(original_func, pq, pk, pv, heads, **kwargs):
        calls.append(kwargs)
        return "previous"

    override = h3.make_minimax_h3_attention_override(device_index=0, verbose_fallbacks=False,
                                                     previous_override=previous)
    assert override(None, q, q, q, 2, skip_reshape=True, transformer_options={"x": 1}) == "previous"
    assert calls[0]["transformer_options"] == {"x": 1} and calls[0]["skip_reshape"] is True
    model = _h3_model()
    with mock.patch.object(h3, "_gfx950_device_index", return_value=(0, None)):
        patched, info = h3.patch_minimax_h3_attention(model, enabled=True, verbose_fallbacks=False)
    assert patched is not model and "strided" in info
    assert "optimized_attention_override" not in model.model_options["transformer_options"]
    aware = mock.Mock()
    aware.container_function = object()
    model.model_options["transformer_options"]["optimized_attention_override"] = aware
    with mock.patch.object(h3, "_gfx950_device_index", return_value=(0, None)):
        kept, info = h3.patch_minimax_h3_attention(model, enabled=True, verbose_fallbacks=False)
    assert kept is model and "container-aware" in info
    assert h3.patch_minimax_h3_attention(H3Model(), enabled=True, verbose_fallbacks=False)[0] is not None


def test_pisa_prepare_validation_matches_the_reference_messages():
    """pisa_prepare_triton's checks in the reference's order and words (pisa_kernel.py:96-111)."""
    from rdna35_block_attention.pisa_kernel import pisa_prepare_triton

    k = torch.zeros((2, 64, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match=r"matching \[BH,T,D\] k/v"):
        pisa_prepare_triton(k[0], k[0])
    with pytest.raises(ValueError, match="block_size=64"):
        pisa_prepare_triton(k, k, block_size=32)
    with pytest.raises(ValueError, match="fp16/bf16"):
        pisa_prepare_triton(k.float(), k.float())
    with pytest.raises(ValueError, match="CUDA/HIP tensors"):
        pisa_prepare_triton(k, k)


def test_fixed_block_triton_name_validation_matches_the_reference_messages():
    """fixed_block_attention_triton_bh's checks in the reference's order and words (triton_kernel.py:209-223)."""
    from rdna35_block_attention.triton_kernel import fixed_block_attention_triton_bh

    q = torch.zeros((2, 64, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="expects \\[BH,T,D\\], got rank 2"):
        fixed_block_attention_triton_bh(q[0], q[0], q[0])
    with pytest.raises(ValueError, match="identical q/k/v shapes"):
        fixed_block_attention_triton_bh(q, q[:, :32], q)
    with pytest.raises(ValueError, match="block_size=64"):
        fixed_block_attention_triton_bh(q, q, q, block_size=32)
    with pytest.raises(ValueError, match="fp16/bf16 only"):
        fixed_block_attention_triton_bh(q.float(), q.float(), q.float())
    with pytest.raises(ValueError, match="CUDA/HIP device tensor"):
        fixed_block_attention_triton_bh(q, q, q)


def test_reference_module_and_probe_names_resolve():
    """Callers importing the reference's module names get this package's objects."""
    import rdna35_block_attention as rba
    from rdna35_block_attention import minimax_h3_attention as h3
    from rdna35_block_attention import minimax_h3_gfx1151_attention as h3_ref_name

    assert h3_ref_name.make_minimax_h3_gfx1151_attention_override is h3.make_minimax_h3_attention_override
    assert h3_ref_name.patch_minimax_h3_gfx1151_attention is h3.patch_minimax_h3_attention
    assert h3_ref_name.pack_minimax_h3_qkv is h3.pack_minimax_h3_qkv
    available, detail = rba.has_triton(import_module=False)
    assert isinstance(available, bool) and isinstance(detail, str)
    assert "has_triton" in rba.__all__


def test_debug_partials_name_the_nonfinite_stage():
    """debug_finite's partial-stage check (generic_pisa.py:210-219): a NaN in a selected key block's values
    reaches only the exact partial, a NaN centroid value only the approximate one; rows past T are ignored."""
    gen = torch.Generator().manual_seed(4)
    blocks, d = 4, 16
    q_b, k_b, v_b = (torch.randn((blocks, 64, d), generator=gen) for _ in range(3))
    lengths = torch.tensor([64.0, 64.0, 64.0, 10.0])
    for t in (q_b, k_b, v_b):
        t[3, 10:] = 0.0                                  # zero rows past T, as the caller pads
    idx = torch.tensor([[0], [1], [1], [3]], dtype=torch.int32)
    k_c, v_m = k_b.sum(1) / lengths[:, None], v_b.sum(1) / lengths[:, None]
    check = generic_pisa._partials_nonfinite
    assert check(q_b, k_b, v_b, idx, k_c, v_m, lengths, 0.25) == []
    q_pad = q_b.clone()
    q_pad[3, 20:] = float("nan")                         # rows past T never count
    assert check(q_pad, k_b, v_b, idx, k_c, v_m, lengths, 0.25) == []
    v_bad = v_b.clone()
    v_bad[1, 5, 2] = float("nan")                        # block 1 is selected by query blocks 1 and 2
    assert check(q_b, k_b, v_bad, idx, k_c, v_m, lengths, 0.25) == ["exact_output"]
    v_m_bad = v_m.clone()
    v_m_bad[2, 0] = float("nan")                         # centroid 2 is unselected for every query block
    assert check(q_b, k_b, v_b, idx, k_c, v_m_bad, lengths, 0.25) == ["approximate_output"]
    k_bad = k_b.clone()
    k_bad[0, 0, 0] = float("inf")
    q_pos = q_b.abs() + 0.1                              # +inf score -> NaN softmax row, inf LSE
    failed = check(q_pos, k_bad, v_b, idx, k_c, v_m, lengths, 0.25)
    assert "exact_lse" in failed and "exact_output" in failed
