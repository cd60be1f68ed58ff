"""Runtime detection used by the dispatch layers (reason strings, device gate).

The reference probes Triton and RDNA3.5 targets (diagnostics.py:22-157); this
build needs to know whether torch is a ROCm build, which gfx target the
device is, and whether the gfx950 HIP library loads.
"""
from __future__ import annotations

import importlib
import os
import re
from typing import Any

TARGET = "gfx950"


def _torch():
    try:
        return importlib.import_module("torch"), None
    except Exception as exc:  # pragma: no cover - host without torch
        return None, f"{type(exc).__name__}: {exc}"


def is_rocm_pytorch() -> bool:
    torch, _ = _torch()
    return bool(torch is not None and getattr(getattr(torch, "version", None), "hip", None))


def _cuda_available(torch) -> bool:
    try:
        return bool(torch.cuda.is_available())
    except Exception:
        return False


def get_device_name(index: int = 0) -> str:
    torch, error = _torch()
    if torch is None:
        return f"torch unavailable: {error}"
    if not _cuda_available(torch):
        return "cuda/hip device unavailable"
    try:
        return str(torch.cuda.get_device_name(index))
    except Exception as exc:
        return f"device name unavailable: {type(exc).__name__}: {exc}"


def _gfx(value: Any) -> str | None:
    match = re.search(r"gfx[0-9a-zA-Z]+", str(value)) if value is not None else None
    return match.group(0) if match else None


def best_effort_gfx_target(index: int = 0) -> str | None:
    """gfx target from the usual build variables, else from the device properties."""
    for name in ("PYTORCH_ROCM_ARCH", "GPU_ARCHS", "AMDGPU_TARGETS", "ROCM_ARCH"):
        target = _gfx(os.environ.get(name))
        if target:
            return target
    torch, _ = _torch()
    if torch is None or not _cuda_available(torch):
        return None
    try:
        props = torch.cuda.get_device_properties(index)
    except Exception:
        return None
    for attr in ("gcnArchName", "gfx_version", "name"):
        target = _gfx(getattr(props, attr, None))
        if target:
            return target
    return None


def device_gfx_target(device) -> str | None:
    """gfx target of a concrete device, from its properties only."""
    torch, _ = _torch()
    if torch is None or not _cuda_available(torch):
        return None
    try:
        return _gfx(getattr(torch.cuda.get_device_properties(device), "gcnArchName", None))
    except Exception:
        return None


def native_status() -> tuple[bool, str]:
    """(loaded, detail) of the gfx950 HIP library."""
    try:
        import mi355x_pisa

        return True, str(mi355x_pisa.build_info().get("implementation"))
    except Exception as exc:
        return False, f"{type(exc).__name__}: {exc}"


class NativeUnavailableError(RuntimeError):
    """The gfx950 HIP library is needed for an eligible call but cannot be loaded."""


def load_native():
    """Import the HIP ops; raise NativeUnavailableError (never fall back) when they are missing."""
    try:
        import mi355x_pisa
    except Exception as exc:
        raise NativeUnavailableError(f"the gfx950 HIP library (mi355x_pisa) is required on ROCm devices but failed to load: "
                           f"{type(exc).__name__}: {exc}") from exc
    return mi355x_pisa


def detect_runtime() -> dict[str, Any]:
    torch, torch_error = _torch()
    info: dict[str, Any] = {
        "torch_imported": torch is not None,
        "torch_error": torch_error,
        "torch_version": getattr(torch, "__version__", None) if torch is not None else None,
        "torch_version_hip": getattr(getattr(torch, "version", None), "hip", None) if torch is not None else None,
        "torch_cuda_is_available": _cuda_available(torch) if torch is not None else False,
        "device": get_device_name(),
        "gfx_target": best_effort_gfx_target(),
        "is_rocm_pytorch": is_rocm_pytorch(),
    }
    info["is_mi355x"] = info["gfx_target"] == TARGET
    loaded, detail = native_status()
    info["native_available"] = loaded
    info["native_info"] = detail
    return info


def explain_dispatch(info: dict[str, Any] | None = None) -> str:
    runtime = detect_runtime()
    lines = [
        "MI355X attention dispatch diagnostics",
        f"torch: {runtime['torch_version']} imported={runtime['torch_imported']}",
        f"torch.version.hip: {runtime['torch_version_hip']}",
        f"torch.cuda.is_available: {runtime['torch_cuda_is_available']}",
        f"device: {runtime['device']}",
        f"gfx target: {runtime['gfx_target']}",
        f"MI355X (gfx950) target: {runtime['is_mi355x']}",
        f"HIP library: {runtime['native_available']} ({runtime['native_info']})",
    ]
    if info:
        lines.append("last dispatch:")
        lines.extend(f"  {key}: {info[key]}" for key in sorted(info))
    return "\n".join(lines)
