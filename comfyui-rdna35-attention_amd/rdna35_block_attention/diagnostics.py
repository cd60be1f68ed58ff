"""The gfx950 device gate and the HIP library loader.

Everything that decides whether a call may take the HIP path asks two
questions, answered here: is this a gfx950 device of a ROCm PyTorch build,
and does the gfx950 library (mi355x_pisa) load.  The package's public
``detect_runtime`` / ``explain_dispatch`` (names of the reference's
rdna35_block_attention/__init__.py:1-7) report exactly those facts.
"""
from __future__ import annotations

import re
from typing import Any

import torch

TARGET = "gfx950"


class NativeUnavailableError(RuntimeError):
    """The gfx950 HIP library is needed for an eligible call but cannot be loaded."""


def _gfx(text: Any) -> str | None:
    found = re.search(r"gfx[0-9a-z]+", str(text or ""))
    return found.group(0) if found else None


def is_rocm_pytorch() -> bool:
    return torch.version.hip is not None


def _have_device() -> bool:
    try:
        return torch.cuda.is_available()
    except Exception:
        return False


def device_gfx_target(device) -> str | None:
    """gfx target of a device from its properties (None without a visible ROCm device)."""
    if not _have_device():
        return None
    try:
        return _gfx(torch.cuda.get_device_properties(device).gcnArchName)
    except Exception:
        return None


def gfx950_device_index() -> tuple[int | None, str | None]:
    """(index of the current device, None) when it is a gfx950 under ROCm PyTorch, else (None, reason)."""
    if not _have_device() or not is_rocm_pytorch():
        return None, "PyTorch ROCm device is unavailable"
    try:
        index = torch.cuda.current_device()
        target = device_gfx_target(index)
    except (RuntimeError, AssertionError) as exc:
        return None, f"could not query the current ROCm device ({type(exc).__name__}: {exc})"
    if target != TARGET:
        return None, f"{TARGET} is required, got {target or 'unknown'}"
    return index, None


def load_native():
    """The HIP op module; raises NativeUnavailableError (never falls back) when it cannot load."""
    try:
        import mi355x_pisa
    except Exception as exc:
        raise NativeUnavailableError(f"the gfx950 HIP library (mi355x_pisa) is required on ROCm devices but failed "
                                     f"to load: {type(exc).__name__}: {exc}") from exc
    return mi355x_pisa


def has_triton(import_module: bool = True) -> tuple[bool, str]:
    """(available, version or reason) of a Triton install - the reference's probe of the same name
    (diagnostics.py:79); nothing in this package runs Triton, the report is for callers that ask."""
    import importlib.metadata
    import importlib.util

    if importlib.util.find_spec("triton") is None:
        return False, "triton module not found"
    if not import_module:
        for dist in ("triton", "triton-windows"):
            try:
                return True, importlib.metadata.version(dist)
            except importlib.metadata.PackageNotFoundError:
                continue
        return True, "installed"
    try:
        import triton
    except Exception as exc:
        return False, f"{type(exc).__name__}: {exc}"
    return True, str(getattr(triton, "__version__", "installed"))


def native_status() -> tuple[bool, str]:
    """(loaded, implementation or the load error) of the gfx950 HIP library."""
    try:
        return True, str(load_native().build_info().get("implementation"))
    except Exception as exc:
        return False, f"{type(exc).__name__}: {exc}"


def get_device_name(index: int = 0) -> str:
    if not _have_device():
        return "cuda/hip device unavailable"
    try:
        return torch.cuda.get_device_name(index)
    except Exception as exc:
        return f"device name unavailable: {type(exc).__name__}: {exc}"


def detect_runtime() -> dict[str, Any]:
    """The facts the gate and the loader use, as one dict."""
    available = _have_device()
    target = device_gfx_target(0) if available else None
    loaded, detail = native_status()
    return {
        "torch_imported": True,
        "torch_error": None,
        "torch_version": torch.__version__,
        "torch_version_hip": torch.version.hip,
        "torch_cuda_is_available": available,
        "device": get_device_name(),
        "gfx_target": target,
        "is_rocm_pytorch": is_rocm_pytorch(),
        "is_mi355x": target == TARGET,
        "native_available": loaded,
        "native_info": detail,
    }


def explain_dispatch(info: dict[str, Any] | None = None) -> str:
    """Text report of detect_runtime(), plus the diagnostics dict of a dispatch when given."""
    runtime = detect_runtime()
    labels = (("torch", "torch_version"), ("torch.version.hip", "torch_version_hip"),
              ("torch.cuda.is_available", "torch_cuda_is_available"), ("device", "device"),
              ("gfx target", "gfx_target"), (f"MI355X ({TARGET}) target", "is_mi355x"))
    lines = ["MI355X attention dispatch diagnostics"]
    lines += [f"{label}: {runtime[key]}" for label, key in labels]
    lines.append(f"HIP library: {runtime['native_available']} ({runtime['native_info']})")
    if info:
        lines.append("last dispatch:")
        lines += [f"  {key}: {info[key]}" for key in sorted(info)]
    return "\n".join(lines)
