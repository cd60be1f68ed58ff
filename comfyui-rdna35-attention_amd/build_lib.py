"""Build libpisa_hip.so (gfx950) from csrc/ with hipcc.

Each translation unit is compiled in parallel to an object file under
``_build/`` and linked into ``mi355x_pisa/libpisa_hip.so`` (in-tree, so the
library travels with the source tree).  Run ``python build_lib.py`` or call
``build()``; both always recompile.
"""
from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

PACKAGE_DIR = pathlib.Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
BUILD_DIR = PACKAGE_DIR / "_build"
LIB_PATH = PACKAGE_DIR / "mi355x_pisa" / "libpisa_hip.so"
ARCH = "gfx950"

SOURCES = ("api.hip", "stats.hip", "route.hip", "attention.hip", "attention_dense.hip", "fixed_block.hip", "layout.hip")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # code object v5 loads under every ROCm 6.x/7.x runtime, including the one
    # bundled with PyTorch wheels
    "-mcode-object-version=5",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-function",
    # Keep hipcc from forming packed fp32 instructions (v_pk_*_f32).
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # MFMA accumulators in architectural VGPRs: the softmax reads and rescales
    # them with VALU ops, and the AGPR form costs a v_accvgpr copy per value
    # (and spills in the attention kernels).
    "-mllvm",
    "-amdgpu-mfma-vgpr-form=1",
    f"-I{REPO_ROOT / 'include'}",
]


# Per-source additions: the dense attention kernels (attention_dense.hip) are
# scheduled by LLVM's max-memory-clause strategy, which measured 1.6 % faster
# on them than the default and slower on the sparse kernels.
EXTRA_FLAGS = {"attention_dense.hip": ["-mllvm", "-amdgpu-sched-strategy=max-memory-clause"]}


def flags_for(name: str) -> list[str]:
    """Compiler flags of one source file of csrc/."""
    return [*COMMON_FLAGS, *EXTRA_FLAGS.get(name, [])]


def _hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and pathlib.Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; a ROCm toolchain is required to build libpisa_hip.so")


def _run(cmd: list[str]) -> None:
    result = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    stderr = "\n".join(line for line in result.stderr.splitlines() if noise not in line)
    if result.returncode != 0:
        raise RuntimeError(f"command failed ({result.returncode}): {' '.join(cmd)}\n{stderr}")
    if stderr.strip():
        print(stderr, file=sys.stderr)


def build(jobs: int | None = None) -> pathlib.Path:
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    objects = [BUILD_DIR / (name.rsplit(".", 1)[0] + ".o") for name in SOURCES]
    commands = [[hipcc, *flags_for(name), "-c", str(CSRC / name), "-o", str(obj)] for name, obj in zip(SOURCES, objects)]
    workers = jobs or min(len(commands), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        for future in [pool.submit(_run, cmd) for cmd in commands]:
            future.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-mcode-object-version=5", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)])
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build())
