"""ComfyUI node classes of the MI355X attention path.

The node ids, input sockets, widgets, outputs and category strings are those
of the reference's nodes.py (nodes.py:30-609), so saved workflows
(workflows/*.json) load unchanged; the nodes call this build's host package
(``rdna35_block_attention``) and through it the gfx950 HIP library.

* patch nodes - RDNA35PatchModelAttention (fixed block-diagonal override),
  RDNA35PatchAnimaPISAAttention (Anima attn_op PISA, layers 20-27 by
  default, budget 0.15625 = 23 of 144 blocks) and
  RDNA35PatchMiniMaxH3GFX1151Attention (strided exact attention) clone the
  MODEL and install on the clone (nodes.py:45-141);
* RDNA35PISARuntimeReport checks, after a sampler ran, that the PISA patch
  executed on every expected layer the same number of times
  (nodes.py:550-582);
* the benchmark nodes time this build's kernels against PyTorch with HIP
  events (median of 20 after 5 warm-ups, nodes.py:149-169) and report
  errors against the torch references;
* RDNA35BlockAttentionDiagnostics prints the runtime / library state.

The reference's gfx1151 device gate is the gfx950 gate here: the MiniMax-H3
benchmark refuses to run on anything but an MI355X.
"""
from __future__ import annotations

import pathlib
import statistics
import sys
import time
from typing import Any

import torch

# ComfyUI imports this folder as a package; the host package and the native
# op module are top-level modules in it (the tests import them the same way).
_HERE = pathlib.Path(__file__).resolve().parent
if str(_HERE) not in sys.path:
    sys.path.insert(0, str(_HERE))

from rdna35_block_attention import diagnostics  # noqa: E402
from rdna35_block_attention.anima_pisa_integration import ANIMA_PISA_FIRST_LAYER, ANIMA_PISA_LAST_LAYER  # noqa: E402
from rdna35_block_attention.comfy_patch import patch_model_attention  # noqa: E402
from rdna35_block_attention.diagnostics import detect_runtime, explain_dispatch  # noqa: E402
from rdna35_block_attention.dispatch import fixed_block_attention  # noqa: E402
from rdna35_block_attention.full_attention import full_attention_triton  # noqa: E402
from rdna35_block_attention.generic_pisa import generic_pisa_attention  # noqa: E402
from rdna35_block_attention.minimax_h3_attention import minimax_h3_pack_profile, patch_minimax_h3_attention  # noqa: E402
from rdna35_block_attention.pisa_attention import pisa_attention  # noqa: E402
from rdna35_block_attention.pisa_patch import patch_model_pisa_attention  # noqa: E402
from rdna35_block_attention.pisa_runtime import PISA_RUNTIME_ATTACHMENT  # noqa: E402
from rdna35_block_attention.reference import (  # noqa: E402
    fixed_block_attention_ref,
    fixed_block_attention_sdpa,
    full_attention_sdpa_bhtd,
)

ANIMA_PISA_BUDGET = 0.15625  # 23 of 144 blocks (nodes.py:110)


# ---------------------------------------------------------------- timing
def _sync(device: torch.device) -> None:
    if device.type == "cuda":
        torch.cuda.synchronize(device)


def _median_ms(fn, device: torch.device, iterations: int = 20, warmup: int = 5) -> float:
    """Median wall time of fn() in ms: HIP events on the current stream on a GPU, perf_counter on the CPU."""
    for _ in range(warmup):
        fn()
    _sync(device)
    if device.type == "cuda":
        events = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                  for _ in range(iterations)]
        for start, end in events:
            start.record()
            fn()
            end.record()
        torch.cuda.synchronize(device)
        return float(statistics.median(start.elapsed_time(end) for start, end in events))
    samples = []
    for _ in range(iterations):
        t0 = time.perf_counter()
        fn()
        samples.append((time.perf_counter() - t0) * 1e3)
    return float(statistics.median(samples))


def _alternating_medians_ms(first_fn, second_fn, device: torch.device, iterations: int,
                            warmup: int) -> tuple[float, float]:
    """Medians of two functions timed in alternation (same clocks and cache state for both)."""
    for _ in range(warmup):
        first_fn()
        second_fn()
    _sync(device)
    pairs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(iterations)]
    for e in pairs:
        e[0].record()
        first_fn()
        e[1].record()
        e[2].record()
        second_fn()
        e[3].record()
    torch.cuda.synchronize(device)
    return (float(statistics.median(e[0].elapsed_time(e[1]) for e in pairs)),
            float(statistics.median(e[2].elapsed_time(e[3]) for e in pairs)))


def _dtype(name: str) -> torch.dtype:
    return torch.float16 if name == "float16" else torch.bfloat16


def _require_mi355x(device: torch.device) -> None:
    if not torch.cuda.is_available() or torch.version.hip is None:
        raise RuntimeError("PyTorch ROCm GPU is required")
    target = diagnostics.device_gfx_target(device)
    if target != diagnostics.TARGET:
        raise RuntimeError(f"{diagnostics.TARGET} (MI355X) is required, got {target or 'unknown'}")


def _max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return (a.float() - b.float()).abs().max().item()


def _cosine(a: torch.Tensor, b: torch.Tensor) -> float:
    return torch.nn.functional.cosine_similarity(a.float().flatten(), b.float().flatten(), dim=0).item()


# ---------------------------------------------------------------- nodes
class RDNA35BlockAttentionDiagnostics:
    @classmethod
    def INPUT_TYPES(cls):
        return {"required": {}}

    RETURN_TYPES = ("STRING",)
    RETURN_NAMES = ("diagnostics",)
    FUNCTION = "run"
    CATEGORY = "RDNA35/Fixed Block Attention"
    OUTPUT_NODE = True

    def run(self):
        return (explain_dispatch(),)


class RDNA35PatchModelAttention:
    @classmethod
    def INPUT_TYPES(cls):
        return {
            "required": {
                "model": ("MODEL",),
                "enabled": ("BOOLEAN", {"default": True}),
                "mode": (["auto", "reference", "triton"], {"default": "auto"}),
                "semantic_mode": (["exact_only", "experimental_force_block_local"], {"default": "exact_only"}),
                "block_size": ("INT", {"default": 64, "min": 64, "max": 64, "step": 64}),
                "causal": ("BOOLEAN", {"default": False}),
                "verbose_fallbacks": ("BOOLEAN", {"default": False}),
            }
        }

    RETURN_TYPES = ("MODEL", "STRING")
    RETURN_NAMES = ("model", "info")
    FUNCTION = "patch"
    CATEGORY = "RDNA35/Fixed Block Attention"
    EXPERIMENTAL = True

    def patch(self, model, enabled, mode, semantic_mode, block_size, causal, verbose_fallbacks):
        # "triton" is the reference's name for its optimised kernel; here it selects the HIP kernel.
        return patch_model_attention(model, enabled=enabled, mode=mode, semantic_mode=semantic_mode,
                                     block_size=block_size, causal=causal, verbose_fallbacks=verbose_fallbacks)


class RDNA35PatchAnimaPISAAttention:
    @classmethod
    def INPUT_TYPES(cls):
        return {
            "required": {
                "model": ("MODEL",),
                "enabled": ("BOOLEAN", {"default": True}),
                "verbose_fallbacks": ("BOOLEAN", {"default": False}),
            },
            "optional": {
                "first_pisa_layer": ("INT", {"default": ANIMA_PISA_FIRST_LAYER, "min": 0, "max": 27}),
                "last_pisa_layer": ("INT", {"default": ANIMA_PISA_LAST_LAYER, "min": 0, "max": 27}),
            },
        }

    RETURN_TYPES = ("MODEL", "STRING")
    RETURN_NAMES = ("model", "info")
    FUNCTION = "patch"
    CATEGORY = "RDNA35/Attention Research"
    EXPERIMENTAL = True

    def patch(self, model, enabled, verbose_fallbacks, first_pisa_layer=ANIMA_PISA_FIRST_LAYER,
              last_pisa_layer=ANIMA_PISA_LAST_LAYER):
        return patch_model_pisa_attention(model, enabled=enabled, exact_budget=ANIMA_PISA_BUDGET,
                                          token_policy="anima_1536_spatial", start_layer=first_pisa_layer,
                                          end_layer=last_pisa_layer, verbose_fallbacks=verbose_fallbacks)


class RDNA35PatchMiniMaxH3GFX1151Attention:
    """Node id kept from the reference (workflows name it); installs the gfx950 strided exact attention."""

    @classmethod
    def INPUT_TYPES(cls):
        return {
            "required": {
                "model": ("MODEL",),
                "enabled": ("BOOLEAN", {"default": True}),
                "verbose_fallbacks": ("BOOLEAN", {"default": False}),
            }
        }

    RETURN_TYPES = ("MODEL", "STRING")
    RETURN_NAMES = ("model", "info")
    FUNCTION = "patch"
    CATEGORY = "RDNA35/Attention Research"
    EXPERIMENTAL = True

    def patch(self, model, enabled, verbose_fallbacks):
        return patch_minimax_h3_attention(model, enabled=enabled, verbose_fallbacks=verbose_fallbacks)


class RDNA35FixedBlockAttentionBenchmark:
    @classmethod
    def INPUT_TYPES(cls):
        return {
            "required": {
                "batch": ("INT", {"default": 1, "min": 1, "max": 8}),
                "heads": ("INT", {"default": 4, "min": 1, "max": 32}),
                "tokens": ("INT", {"default": 128, "min": 1, "max": 8192, "step": 64}),
                "head_dim": ("INT", {"default": 64, "min": 32, "max": 128, "step": 32}),
                "dtype": (["float16", "bfloat16"], {"default": "float16"}),
                "mode": (["auto", "triton", "reference"], {"default": "auto"}),
                "causal": ("BOOLEAN", {"default": False}),
            }
        }

    RETURN_TYPES = ("STRING",)
    RETURN_NAMES = ("benchmark",)
    FUNCTION = "run"
    CATEGORY = "RDNA35/Fixed Block Attention"
    OUTPUT_NODE = True

    def run(self, batch, heads, tokens, head_dim, dtype, mode, causal):
        runtime = detect_runtime()
        device = torch.device("cuda") if runtime["torch_cuda_is_available"] else torch.device("cpu")
        dt = _dtype(dtype)
        q = torch.randn(batch, heads, tokens, head_dim, device=device, dtype=dt)
        k = torch.randn_like(q)
        v = torch.randn_like(q)
        opts = dict(block_size=64, causal=causal, layout="bhtd")
        ref = fixed_block_attention_ref(q, k, v, **opts)
        sdpa_block = fixed_block_attention_sdpa(q, k, v, **opts)
        sdpa_full = full_attention_sdpa_bhtd(q, k, v, causal=causal)
        out, info = fixed_block_attention(q, k, v, mode=mode, return_diagnostics=True, **opts)
        ref_ms = _median_ms(lambda: fixed_block_attention_ref(q, k, v, **opts), device)
        block_ms = _median_ms(lambda: fixed_block_attention_sdpa(q, k, v, **opts), device)
        full_ms = _median_ms(lambda: full_attention_sdpa_bhtd(q, k, v, causal=causal), device)
        lines = [
            "RDNA35 Fixed Block Attention Benchmark (MI355X HIP)",
            f"device: {runtime['device']} ({runtime['gfx_target']})",
            f"torch: {runtime['torch_version']} hip={runtime['torch_version_hip']}",
            f"HIP library: {runtime['native_available']} ({runtime['native_info']})",
            f"shape: B={batch} H={heads} T={tokens} D={head_dim} dtype={dt} causal={causal}",
            f"reference median: {ref_ms:.3f} ms",
            f"PyTorch SDPA block-mask median: {block_ms:.3f} ms",
            f"PyTorch SDPA full-attention median: {full_ms:.3f} ms",
            f"dispatch backend: {info.get('backend')}",
            f"fallback reason: {info.get('fallback_reason')}",
            f"max abs error vs reference: {_max_abs(out, ref):.6g}",
            f"SDPA block-mask max abs error vs reference: {_max_abs(sdpa_block, ref):.6g}",
            f"full SDPA semantic delta vs fixed-block reference: {_max_abs(sdpa_full, ref):.6g}",
        ]
        if info.get("optimized"):
            hip_ms = _median_ms(lambda: fixed_block_attention(q, k, v, mode="hip", **opts), device)
            lines += [
                f"HIP kernel median: {hip_ms:.3f} ms",
                f"measured speedup vs reference: {ref_ms / hip_ms:.3f}x",
                f"measured speedup vs PyTorch SDPA block-mask: {block_ms / hip_ms:.3f}x",
                f"latency ratio vs PyTorch full SDPA (different semantics): {hip_ms / full_ms:.3f}x",
            ]
        else:
            lines.append("measured speedup: unavailable because optimized path did not run")
        return ("\n".join(lines),)


class RDNA35FullAttentionBenchmark:
    @classmethod
    def INPUT_TYPES(cls):
        return {
            "required": {
                "batch": ("INT", {"default": 1, "min": 1, "max": 4}),
                "heads": ("INT", {"default": 16, "min": 1, "max": 40}),
                "query_tokens": ("INT", {"default": 4096, "min": 64, "max": 9216, "step": 64}),
                "key_tokens": ("INT", {"default": 4096, "min": 64, "max": 9216, "step": 64}),
                "head_dim": ([64, 128], {"default": 128}),
                "dtype": (["float16", "bfloat16"], {"default": "bfloat16"}),
            }
        }

    RETURN_TYPES = ("STRING",)
    RETURN_NAMES = ("benchmark",)
    FUNCTION = "run"
    CATEGORY = "RDNA35/Attention Research"
    OUTPUT_NODE = True
    EXPERIMENTAL = True

    def run(self, batch, heads, query_tokens, key_tokens, head_dim, dtype):
        device = torch.device("cuda")
        dt = _dtype(dtype)
        q = torch.randn(batch, heads, query_tokens, head_dim, device=device, dtype=dt)
        k = torch.randn(batch, heads, key_tokens, head_dim, device=device, dtype=dt)
        v = torch.randn_like(k)
        q_bh, k_bh, v_bh = (t.flatten(0, 1).contiguous() for t in (q, k, v))
        # float32 reference: torch's bf16 attention math path is not used as the yardstick
        reference = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float())
        output, info = full_attention_triton(q_bh, k_bh, v_bh, return_diagnostics=True)
        output = output.unflatten(0, (batch, heads))
        sdpa_ms = _median_ms(lambda: torch.nn.functional.scaled_dot_product_attention(q, k, v), device)
        hip_ms = _median_ms(lambda: full_attention_triton(q_bh, k_bh, v_bh), device)
        flops = 4.0 * batch * heads * query_tokens * key_tokens * head_dim
        return ("\n".join([
            "RDNA35 Exact Full Attention Benchmark (MI355X HIP)",
            f"shape: B={batch} H={heads} Q={query_tokens} K={key_tokens} D={head_dim} dtype={dt}",
            f"PyTorch SDPA median: {sdpa_ms:.3f} ms",
            f"gfx950 HIP median: {hip_ms:.3f} ms ({flops / hip_ms / 1e9:.1f} TFLOP/s)",
            f"HIP/SDPA ratio: {hip_ms / sdpa_ms:.3f}x",
            f"max abs error: {_max_abs(output, reference):.6g}",
            f"kernel config: {info.get('config')}",
        ]),)


class RDNA35MiniMaxH3GFX1151AttentionBenchmark:
    @classmethod
    def INPUT_TYPES(cls):
        return {"required": {"tokens": ("INT", {"default": 9170, "min": 4608, "max": 16500, "step": 1})}}

    RETURN_TYPES = ("STRING",)
    RETURN_NAMES = ("benchmark",)
    FUNCTION = "run"
    CATEGORY = "RDNA35/Attention Research"
    OUTPUT_NODE = True
    EXPERIMENTAL = True

    def run(self, tokens):
        device = torch.device("cuda")
        _require_mi355x(device)
        native = diagnostics.load_native()
        qkv = torch.randn(1, tokens, 3, 56, 128, device=device, dtype=torch.bfloat16)
        q = qkv[:, :, 0].permute(0, 2, 1, 3)
        k = qkv[:, :, 1].permute(0, 2, 1, 3)
        v = qkv[:, :, 2].clone().permute(0, 2, 1, 3)
        s = 128 ** -0.5

        def existing_attention():
            return torch.nn.functional.scaled_dot_product_attention(q, k, v).transpose(1, 2).contiguous()

        def strided_hip_attention():
            return native.dense_attention(q, k, v, s)

        existing = existing_attention()
        hip_out = strided_hip_attention().transpose(1, 2)
        if not torch.isfinite(hip_out).all():
            raise RuntimeError("strided HIP attention produced non-finite output")
        if not torch.allclose(hip_out.float(), existing.float(), atol=5e-2, rtol=5e-2):
            raise RuntimeError("strided HIP attention failed the BF16 correctness check")
        existing_ms, hip_ms = _alternating_medians_ms(existing_attention, strided_hip_attention, device,
                                                      iterations=5, warmup=2)
        return ("\n".join([
            "RDNA35 MiniMax-H3 Attention Benchmark (MI355X HIP, strided views read in place)",
            f"torch: {torch.__version__} hip={torch.version.hip}",
            f"shape: B=1 H=56 T={tokens} D=128 dtype={torch.bfloat16}",
            "timing: 2 warmups, 5 alternating GPU-event samples (quick diagnostic)",
            f"reference packing profile at this T: {minimax_h3_pack_profile(tokens).upper()} (not needed here)",
            f"existing strided SDPA median: {existing_ms:.3f} ms",
            f"strided HIP median: {hip_ms:.3f} ms",
            f"measured speedup: {existing_ms / hip_ms:.3f}x",
            f"time reduction: {existing_ms - hip_ms:.3f} ms ({(1.0 - hip_ms / existing_ms) * 100.0:.1f}%)",
            f"max abs error: {_max_abs(hip_out, existing):.6g}",
            f"cosine similarity: {_cosine(hip_out, existing):.9f}",
        ]),)


class RDNA35PISAAttentionBenchmark:
    @classmethod
    def INPUT_TYPES(cls):
        return {
            "required": {
                "batch_heads": ("INT", {"default": 1, "min": 1, "max": 40}),
                "tokens": ("INT", {"default": 9216, "min": 128, "max": 9216, "step": 64}),
                "exact_budget": ("FLOAT", {"default": 0.15625, "min": 0.015625, "max": 1.0, "step": 0.015625}),
                "dtype": (["bfloat16"], {"default": "bfloat16"}),
                "backend": (["ck", "auto", "triton", "reference"], {"default": "ck"}),
            }
        }

    RETURN_TYPES = ("STRING",)
    RETURN_NAMES = ("benchmark",)
    FUNCTION = "run"
    CATEGORY = "RDNA35/Attention Research"
    OUTPUT_NODE = True
    EXPERIMENTAL = True

    def run(self, batch_heads, tokens, exact_budget, dtype, backend):
        device = torch.device("cuda")
        dt = _dtype(dtype)
        q = torch.randn(batch_heads, tokens, 128, device=device, dtype=dt)
        k = torch.randn_like(q)
        v = torch.randn_like(q)
        reference = torch.nn.functional.scaled_dot_product_attention(
            q.float().unsqueeze(0), k.float().unsqueeze(0), v.float().unsqueeze(0)).squeeze(0)
        strict = backend in {"ck", "triton"}
        _sync(device)
        t0 = time.perf_counter()
        output, info = pisa_attention(q, k, v, exact_budget=exact_budget, backend=backend, strict_backend=strict,
                                      return_diagnostics=True)
        _sync(device)
        cold_ms = (time.perf_counter() - t0) * 1e3
        pisa_ms = _median_ms(lambda: pisa_attention(q, k, v, exact_budget=exact_budget, backend=backend,
                                                    strict_backend=strict), device)
        sdpa_ms = _median_ms(lambda: torch.nn.functional.scaled_dot_product_attention(
            q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0)), device)
        optimized = bool(info.get("optimized"))
        return ("\n".join([
            "RDNA35 PISA Attention Benchmark (MI355X HIP)",
            f"shape: BH={batch_heads} T={tokens} D=128 dtype={dt}",
            f"backend: {info.get('backend')}",
            f"exact blocks: {info.get('exact_blocks_per_query')}/{info.get('total_blocks')}",
            f"PISA cold call: {cold_ms:.3f} ms",
            f"PISA steady-state median: {pisa_ms:.3f} ms",
            f"dense SDPA steady-state median: {sdpa_ms:.3f} ms",
            f"PISA/dense latency ratio: {pisa_ms / sdpa_ms:.3f}x",
            f"cosine vs dense attention: {_cosine(reference, output):.9f}",
            f"mean abs error: {(output.float() - reference).abs().mean().item():.6g}",
            f"fallback: {info.get('fallback_reason')}",
            ("gfx950 HIP block statistics + routing + fused exact/tail/first-order attention kernel."
             if optimized else "The HIP path did not run; see backend and fallback above."),
        ]),)


class RDNA35GenericPISABenchmark:
    @classmethod
    def INPUT_TYPES(cls):
        return {
            "required": {
                "batch": ("INT", {"default": 1, "min": 1, "max": 8}),
                "heads": ("INT", {"default": 10, "min": 1, "max": 40}),
                "tokens": ("INT", {"default": 8192, "min": 8192, "max": 32768, "step": 64}),
                "head_dim": ("INT", {"default": 64, "min": 32, "max": 256, "step": 8}),
                "exact_budget": ("FLOAT", {"default": 0.25, "min": 0.015625, "max": 1.0, "step": 0.015625}),
                "dtype": (["float16", "bfloat16"], {"default": "float16"}),
            }
        }

    RETURN_TYPES = ("STRING",)
    RETURN_NAMES = ("benchmark",)
    FUNCTION = "run"
    CATEGORY = "RDNA35/Attention Research"
    OUTPUT_NODE = True
    EXPERIMENTAL = True

    def run(self, batch, heads, tokens, head_dim, exact_budget, dtype):
        device = torch.device("cuda")
        dt = _dtype(dtype)
        q = torch.randn(batch, heads, tokens, head_dim, device=device, dtype=dt)
        k = torch.randn_like(q)
        v = torch.randn_like(q)
        q_flat, k_flat, v_flat = (t.flatten(0, 1).contiguous() for t in (q, k, v))
        # generic_pisa.py:332-333: the first-order term only for D=128 bf16, otherwise budget >= 0.25
        first_order = head_dim == 128 and dt == torch.bfloat16
        budget = exact_budget if first_order else max(0.25, exact_budget)
        output, backend = generic_pisa_attention(q_flat, k_flat, v_flat, exact_budget=budget,
                                                 use_first_order=first_order, return_backend=True)
        reference = torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float())
        pisa_ms = _median_ms(lambda: generic_pisa_attention(q_flat, k_flat, v_flat, exact_budget=budget,
                                                            use_first_order=first_order),
                             device, iterations=10, warmup=3)
        try:  # ComfyUI's own PyTorch attention when this runs inside ComfyUI
            from comfy.ldm.modules.attention import attention_pytorch

            def baseline():
                return attention_pytorch(q, k, v, heads, skip_reshape=True, skip_output_reshape=True)

            baseline_name = "ComfyUI PyTorch SDPA"
        except ImportError:
            def baseline():
                return torch.nn.functional.scaled_dot_product_attention(q, k, v)

            baseline_name = "PyTorch SDPA"
        base_ms = _median_ms(baseline, device, iterations=10, warmup=3)
        return ("\n".join([
            "RDNA35 Generic PISA Benchmark (MI355X HIP)",
            f"shape: B={batch} H={heads} T={tokens} D={head_dim} dtype={dt}",
            f"statistics backend: {backend}",
            f"exact budget: {budget:.6g} first-order: {first_order}",
            f"PISA median: {pisa_ms:.3f} ms",
            f"{baseline_name} median: {base_ms:.3f} ms; PISA/SDPA={pisa_ms / base_ms:.3f}x",
            f"cosine vs dense attention: {_cosine(reference.flatten(0, 1), output):.9f}",
            f"mean abs error: {(output.float() - reference.flatten(0, 1)).abs().mean().item():.6g}",
        ]),)


class RDNA35PISARuntimeReport:
    @classmethod
    def INPUT_TYPES(cls):
        return {"required": {"model": ("MODEL",), "latent": ("LATENT",)}}

    RETURN_TYPES = ("LATENT", "STRING")
    RETURN_NAMES = ("latent", "report")
    FUNCTION = "run"
    CATEGORY = "RDNA35/Attention Research"
    OUTPUT_NODE = True
    EXPERIMENTAL = True

    def run(self, model, latent):
        state = model.get_attachment(PISA_RUNTIME_ATTACHMENT) if hasattr(model, "get_attachment") else None
        if state is None:
            raise RuntimeError("RDNA35 PISA runtime state is not attached to this MODEL")
        if sum(state.per_layer_hits.values()) == 0:
            raise RuntimeError(f"INVALID BENCHMARK: PISA backend was not executed: {state.report()}")
        if set(state.per_layer_hits) == {-1}:  # the generic override records layer -1
            if state.failed:
                raise RuntimeError(f"Generic PISA runtime failed: {state.report()}")
            return {"ui": {"text": [state.report()]}, "result": (latent, state.report())}
        counts = set(state.per_layer_hits.values())
        expected = set(state.expected_layers or range(ANIMA_PISA_FIRST_LAYER, ANIMA_PISA_LAST_LAYER + 1))
        if set(state.per_layer_hits) != expected or len(counts) != 1:
            raise RuntimeError(f"Incomplete PISA layer accounting: {state.report()}")
        state.verify(counts.pop())
        if not state.verified:
            raise RuntimeError(f"PISA runtime verification failed: {state.report()}")
        report = state.report()
        return {"ui": {"text": [report]}, "result": (latent, report)}


NODE_CLASS_MAPPINGS: dict[str, Any] = {
    "RDNA35BlockAttentionDiagnostics": RDNA35BlockAttentionDiagnostics,
    "RDNA35PatchModelAttention": RDNA35PatchModelAttention,
    "RDNA35PatchAnimaPISAAttention": RDNA35PatchAnimaPISAAttention,
    "RDNA35PatchMiniMaxH3GFX1151Attention": RDNA35PatchMiniMaxH3GFX1151Attention,
    "RDNA35FixedBlockAttentionBenchmark": RDNA35FixedBlockAttentionBenchmark,
    "RDNA35FullAttentionBenchmark": RDNA35FullAttentionBenchmark,
    "RDNA35MiniMaxH3GFX1151AttentionBenchmark": RDNA35MiniMaxH3GFX1151AttentionBenchmark,
    "RDNA35PISAAttentionBenchmark": RDNA35PISAAttentionBenchmark,
    "RDNA35GenericPISABenchmark": RDNA35GenericPISABenchmark,
    "RDNA35PISARuntimeReport": RDNA35PISARuntimeReport,
}

NODE_DISPLAY_NAME_MAPPINGS = {
    "RDNA35BlockAttentionDiagnostics": "RDNA35 Block Attention Diagnostics (MI355X)",
    "RDNA35PatchModelAttention": "RDNA35 Patch Model Attention (MI355X)",
    "RDNA35PatchAnimaPISAAttention": "RDNA35 Patch PISA Attention (MI355X)",
    "RDNA35PatchMiniMaxH3GFX1151Attention": "RDNA35 Patch MiniMax-H3 Attention (MI355X)",
    "RDNA35FixedBlockAttentionBenchmark": "RDNA35 Fixed Block Attention Benchmark (MI355X)",
    "RDNA35FullAttentionBenchmark": "RDNA35 Exact Full Attention Benchmark (MI355X)",
    "RDNA35MiniMaxH3GFX1151AttentionBenchmark": "RDNA35 MiniMax-H3 Attention Benchmark (MI355X)",
    "RDNA35PISAAttentionBenchmark": "RDNA35 PISA Attention Benchmark (MI355X)",
    "RDNA35GenericPISABenchmark": "RDNA35 Generic PISA Benchmark (MI355X)",
    "RDNA35PISARuntimeReport": "RDNA35 PISA Runtime Report (MI355X)",
}
