"""ComfyUI node classes (nodes.py): ids, sockets, patch behaviour and the runtime report, on the CPU.

Mirrors the reference's node contract (nodes.py:30-609); ComfyUI itself is
not installed, so MODEL is a small stand-in with the ModelPatcher methods
the patch functions use (clone, model_options, attachments).
"""
from __future__ import annotations

import copy
import importlib.util
import sys

import pytest
import torch

from conftest import PACKAGE_DIR
from rdna35_block_attention.pisa_runtime import PISA_RUNTIME_ATTACHMENT, PISARuntimeState

EXPECTED_IDS = {
    "RDNA35BlockAttentionDiagnostics", "RDNA35PatchModelAttention", "RDNA35PatchAnimaPISAAttention",
    "RDNA35PatchMiniMaxH3GFX1151Attention", "RDNA35FixedBlockAttentionBenchmark", "RDNA35FullAttentionBenchmark",
    "RDNA35MiniMaxH3GFX1151AttentionBenchmark", "RDNA35PISAAttentionBenchmark", "RDNA35GenericPISABenchmark",
    "RDNA35PISARuntimeReport",
}


def load_custom_node_package():
    """Import the package folder the way ComfyUI does (a module named after the folder, from __init__.py)."""
    name = "comfyui_rdna35_attention_amd_under_test"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, PACKAGE_DIR / "__init__.py",
                                                  submodule_search_locations=[str(PACKAGE_DIR)])
    module = importlib.util.module_from_spec(spec)
    sys.modules[name] = module
    spec.loader.exec_module(module)
    return module


class FakeModelPatcher:
    def __init__(self):
        self.model_options = {"transformer_options": {}}
        self.attachments = {}

    def clone(self):
        other = FakeModelPatcher()
        other.model_options = copy.deepcopy(self.model_options)
        other.attachments = dict(self.attachments)
        return other

    def set_attachments(self, key, value):
        self.attachments[key] = value

    def get_attachment(self, key):
        return self.attachments.get(key)


@pytest.fixture(scope="module")
def nodes():
    return load_custom_node_package()


def test_node_ids_and_display_names_match_the_reference(nodes):
    assert set(nodes.NODE_CLASS_MAPPINGS) == EXPECTED_IDS
    assert set(nodes.NODE_DISPLAY_NAME_MAPPINGS) == EXPECTED_IDS


@pytest.mark.parametrize("node_id", sorted(EXPECTED_IDS))
def test_node_contract(nodes, node_id):
    cls = nodes.NODE_CLASS_MAPPINGS[node_id]
    spec = cls.INPUT_TYPES()
    assert "required" in spec
    assert isinstance(cls.RETURN_TYPES, tuple) and len(cls.RETURN_TYPES) == len(cls.RETURN_NAMES)
    assert callable(getattr(cls(), cls.FUNCTION))
    assert cls.CATEGORY.startswith("RDNA35/")


def test_patch_node_sockets_match_reference(nodes):
    req = nodes.NODE_CLASS_MAPPINGS["RDNA35PatchModelAttention"].INPUT_TYPES()["required"]
    assert list(req) == ["model", "enabled", "mode", "semantic_mode", "block_size", "causal", "verbose_fallbacks"]
    assert req["mode"][0] == ["auto", "reference", "triton"]
    anima = nodes.NODE_CLASS_MAPPINGS["RDNA35PatchAnimaPISAAttention"].INPUT_TYPES()
    assert anima["optional"]["first_pisa_layer"][1]["default"] == 20
    assert anima["optional"]["last_pisa_layer"][1]["default"] == 27
    assert nodes.NODE_CLASS_MAPPINGS["RDNA35PISARuntimeReport"].RETURN_TYPES == ("LATENT", "STRING")


def test_disabled_patches_return_the_model_unchanged(nodes):
    model = FakeModelPatcher()
    m = nodes.NODE_CLASS_MAPPINGS
    out, info = m["RDNA35PatchModelAttention"]().patch(model, False, "auto", "exact_only", 64, False, False)
    assert out is model and "disabled" in info
    out, info = m["RDNA35PatchAnimaPISAAttention"]().patch(model, False, False)
    assert out is model and "disabled" in info
    out, info = m["RDNA35PatchMiniMaxH3GFX1151Attention"]().patch(model, False, False)
    assert out is model


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-MI355X path")
def test_pisa_patch_without_mi355x_leaves_model_alone(nodes):
    model = FakeModelPatcher()
    out, info = nodes.NODE_CLASS_MAPPINGS["RDNA35PatchAnimaPISAAttention"]().patch(model, True, False)
    assert out is model
    assert "unchanged" in info
    assert "optimized_attention_override" not in model.model_options["transformer_options"]


def test_fixed_block_patch_installs_on_a_clone(nodes):
    model = FakeModelPatcher()
    out, info = nodes.NODE_CLASS_MAPPINGS["RDNA35PatchModelAttention"]().patch(
        model, True, "auto", "exact_only", 64, False, False)
    assert out is not model
    assert "optimized_attention_override" not in model.model_options["transformer_options"]
    assert callable(out.model_options["transformer_options"]["optimized_attention_override"])
    assert isinstance(info, str) and info


def _report(nodes, model):
    return nodes.NODE_CLASS_MAPPINGS["RDNA35PISARuntimeReport"]().run(model, {"samples": None})


def test_runtime_report_requires_attached_executed_state(nodes):
    model = FakeModelPatcher()
    with pytest.raises(RuntimeError, match="not attached"):
        _report(nodes, model)
    model.set_attachments(PISA_RUNTIME_ATTACHMENT, PISARuntimeState(armed=True))
    with pytest.raises(RuntimeError, match="INVALID BENCHMARK"):
        _report(nodes, model)


def test_runtime_report_verifies_every_layer_ran_equally(nodes):
    model = FakeModelPatcher()
    state = PISARuntimeState(armed=True, expected_layers=tuple(range(20, 28)))
    model.set_attachments(PISA_RUNTIME_ATTACHMENT, state)
    for _ in range(3):
        for layer in range(20, 28):
            state.record(layer=layer, is_self_attention=True, backend="hip_hyd")
    result = _report(nodes, model)
    latent, report = result["result"]
    assert latent == {"samples": None}
    assert state.verified and "verified=1" in report and "hits=24/24" in report
    # one layer short -> incomplete accounting
    broken = PISARuntimeState(armed=True, expected_layers=tuple(range(20, 28)))
    for layer in range(20, 27):
        broken.record(layer=layer, is_self_attention=True, backend="hip_hyd")
    model.set_attachments(PISA_RUNTIME_ATTACHMENT, broken)
    with pytest.raises(RuntimeError, match="Incomplete PISA layer accounting"):
        _report(nodes, model)


def test_runtime_report_generic_layer(nodes):
    model = FakeModelPatcher()
    state = PISARuntimeState(armed=True)
    model.set_attachments(PISA_RUNTIME_ATTACHMENT, state)
    state.record(layer=-1, is_self_attention=True, backend="hip_generic")
    assert "hits=1" in _report(nodes, model)["result"][1]
    state.record(layer=-1, error="boom")
    with pytest.raises(RuntimeError, match="Generic PISA runtime failed"):
        _report(nodes, model)


def test_diagnostics_node_reports_runtime(nodes):
    (text,) = nodes.NODE_CLASS_MAPPINGS["RDNA35BlockAttentionDiagnostics"]().run()
    assert "gfx" in text and "HIP library" in text


def test_fixed_block_benchmark_runs_reference_on_cpu(nodes):
    if torch.cuda.is_available():
        pytest.skip("CPU behaviour")
    (text,) = nodes.NODE_CLASS_MAPPINGS["RDNA35FixedBlockAttentionBenchmark"]().run(
        1, 2, 128, 32, "float16", "auto", False)
    assert "dispatch backend: reference" in text
    assert "max abs error vs reference: 0" in text


WIDGET_TYPES = ("BOOLEAN", "INT", "FLOAT", "STRING")


def _widget_ok(spec, value) -> bool:
    kind = spec[0]
    opts = spec[1] if len(spec) > 1 else {}
    if isinstance(kind, list):
        return value in kind
    if kind == "BOOLEAN":
        return isinstance(value, bool)
    if kind == "INT":
        return isinstance(value, int) and opts.get("min", value) <= value <= opts.get("max", value)
    if kind == "FLOAT":
        return isinstance(value, (int, float)) and opts.get("min", value) <= value <= opts.get("max", value)
    return isinstance(value, str)


def test_reference_workflows_load_on_these_nodes(nodes):
    """The attention nodes of the reference's saved workflows (tests/golden/reference_workflow_nodes.json, written
    from /root/reference/workflows by tests/golden/make_workflow_nodes.py) bind to these node classes: same node
    id, the saved widget values valid for the widgets in declaration order, the same socket names, and the patch
    accepts the values."""
    import json
    import pathlib

    fixture = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_workflow_nodes.json").read_text())
    assert sum(len(rows) for rows in fixture.values()) == 3
    for workflow, rows in fixture.items():
        for row in rows:
            cls = nodes.NODE_CLASS_MAPPINGS[row["type"]]
            spec = cls.INPUT_TYPES()
            ordered = list(spec["required"].items()) + list(spec.get("optional", {}).items())
            widgets = [(name, s) for name, s in ordered if isinstance(s[0], list) or s[0] in WIDGET_TYPES]
            sockets = [name for name, s in ordered if not (isinstance(s[0], list) or s[0] in WIDGET_TYPES)]
            values = row["widgets_values"]
            assert len(values) <= len(widgets), (workflow, row["type"])
            for (name, s), value in zip(widgets, values):
                assert _widget_ok(s, value), (workflow, row["type"], name, value)
            assert row["inputs"] == sockets, (workflow, row["type"])
            assert list(cls.RETURN_NAMES) == row["outputs"], (workflow, row["type"])
            model = FakeModelPatcher()
            kwargs = {name: value for (name, _), value in zip(widgets, values)}
            out, info = getattr(cls(), cls.FUNCTION)(model, **kwargs)
            assert isinstance(info, str) and out is not None
