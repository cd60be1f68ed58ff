"""ComfyUI node classes on the MI355X: the benchmark nodes run the HIP path and
report errors within the bf16/fp16 tolerance; the PISA patch node installs
the gfx950 override on a clone.  Small shapes (each node call is < 1 s)."""
from __future__ import annotations

import re

import pytest

from test_nodes import FakeModelPatcher, load_custom_node_package

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def nodes():
    return load_custom_node_package()


def _number(text: str, label: str) -> float:
    m = re.search(re.escape(label) + r"\s*([-+0-9.eE]+|inf|nan)", text)
    assert m, (label, text)
    return float(m.group(1))


def test_pisa_benchmark_node_runs_hip_hyd(nodes):
    (text,) = nodes.NODE_CLASS_MAPPINGS["RDNA35PISAAttentionBenchmark"]().run(2, 1024, 0.25, "bfloat16", "ck")
    print(text)
    assert "backend: hip_hyd" in text
    assert "exact blocks: 4/16" in text
    # white-noise inputs at a 25 % budget: the tail approximation is coarse
    # (kernel parity against the oracle is tested in test_gpu_native.py)
    assert 0.5 < _number(text, "cosine vs dense attention:") <= 1.0


def test_full_attention_benchmark_node(nodes):
    (text,) = nodes.NODE_CLASS_MAPPINGS["RDNA35FullAttentionBenchmark"]().run(1, 2, 256, 512, 128, "bfloat16")
    print(text)
    assert _number(text, "max abs error:") < 5e-2


def test_fixed_block_benchmark_node_uses_hip(nodes):
    (text,) = nodes.NODE_CLASS_MAPPINGS["RDNA35FixedBlockAttentionBenchmark"]().run(
        1, 2, 256, 64, "float16", "auto", True)
    print(text)
    assert "dispatch backend: hip" in text
    assert _number(text, "max abs error vs reference:") < 2e-2
    assert "HIP kernel median" in text


def test_minimax_h3_benchmark_node(nodes):
    (text,) = nodes.NODE_CLASS_MAPPINGS["RDNA35MiniMaxH3GFX1151AttentionBenchmark"]().run(4608)
    print(text)
    assert _number(text, "max abs error:") < 5e-2
    assert _number(text, "cosine similarity:") > 0.999


def test_generic_pisa_benchmark_node(nodes):
    (text,) = nodes.NODE_CLASS_MAPPINGS["RDNA35GenericPISABenchmark"]().run(1, 2, 8192, 128, 0.25, "bfloat16")
    print(text)
    assert "statistics backend: hip_generic" in text
    assert 0.5 < _number(text, "cosine vs dense attention:") <= 1.0


def test_pisa_patch_node_installs_generic_override_on_clone(nodes):
    model = FakeModelPatcher()
    out, info = nodes.NODE_CLASS_MAPPINGS["RDNA35PatchAnimaPISAAttention"]().patch(model, True, False)
    print(info)
    assert out is not model
    assert "gfx950" in info
    assert callable(out.model_options["transformer_options"]["optimized_attention_override"])
    assert "optimized_attention_override" not in model.model_options["transformer_options"]
