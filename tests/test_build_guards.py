"""Guards on toolchain behaviour the attention kernels rely on (CPU; needs hipcc).

The persistent attention kernel copies the next block's query rows and first
chunk to LDS with inline ``global_load_lds_dwordx4`` (M0 holds the LDS base),
hidden from the compiler's memory counters, and orders those copies with
explicit ``s_waitcnt`` immediates (csrc/common.hpp kWaitVm0 / kWaitLgkm0).
Both rest on facts of the current toolchain that a compiler or assembler
change could break without any test of the outputs noticing at once:

* the immediates must assemble to exactly the waits they are named for;
* nothing but those copies may write or read M0 in the compiled kernels (the
  compiler reserves M0; if it started to use it, a copy's LDS base could be
  overwritten between the ``s_mov_b32 m0`` and the load);
* every copy must be issued right after its ``s_mov_b32 m0``.

A fourth guard: no kernel may spill vector registers to scratch.  The
attention kernels run at up to 512 registers per lane; when one spilled, the
register allocator rebuilt a spilled query fragment inside the chunk loop
with one of its four dwords taken from the previous iteration's scores (the
head-dim 256 kernel, whose query fragments now live in LDS instead).

These tests compile the sources to gfx950 assembly with the library's own
flags (about a minute) and fail with the offending lines if any of this stops
holding.
"""
from __future__ import annotations

import pathlib
import re
import shutil
import subprocess
import sys

import pytest

REPO = pathlib.Path(__file__).resolve().parents[1]
PKG = REPO / "comfyui-rdna35-attention_amd"
sys.path.insert(0, str(PKG))

import build_lib  # noqa: E402

HIPCC = next((c for c in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc") if c and pathlib.Path(c).exists()), None)
pytestmark = pytest.mark.skipif(HIPCC is None, reason="hipcc is not installed")


def _device_asm(source: pathlib.Path, out: pathlib.Path) -> str:
    cmd = [HIPCC, *build_lib.flags_for(source.name), f"-I{PKG / 'csrc'}", "-S", "--cuda-device-only", str(source),
           "-o", str(out)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    assert result.returncode == 0, result.stderr[-2000:]
    return out.read_text()


def _kernels(asm: str) -> dict[str, list[str]]:
    """Instruction lines of every kernel in a device assembly listing, by symbol."""
    kernels: dict[str, list[str]] = {}
    current = None
    for line in asm.splitlines():
        label = re.match(r"^(_Z\w+):", line)
        if label:
            current = label.group(1)
            kernels[current] = []
            continue
        if current is None:
            continue
        text = line.split(";")[0].strip()
        if not text or text.startswith(".") or text.endswith(":"):
            continue
        kernels[current].append(text)
        if text.startswith("s_endpgm"):
            current = None
    return kernels


def test_wait_immediates_assemble_to_the_waits_they_name(tmp_path):
    probe = tmp_path / "probe.hip"
    probe.write_text('#include "common.hpp"\n'
                     "__global__ void probe_vm0() { __builtin_amdgcn_s_waitcnt(pisa::kWaitVm0); }\n"
                     "__global__ void probe_lgkm0() { __builtin_amdgcn_s_waitcnt(pisa::kWaitLgkm0); }\n")
    kernels = _kernels(_device_asm(probe, tmp_path / "probe.s"))
    waits = {name: [i for i in body if i.startswith("s_waitcnt")] for name, body in kernels.items()}
    vm0 = next(w for name, w in waits.items() if "probe_vm0" in name)
    lgkm0 = next(w for name, w in waits.items() if "probe_lgkm0" in name)
    assert vm0 == ["s_waitcnt vmcnt(0)"], vm0
    assert lgkm0 == ["s_waitcnt lgkmcnt(0)"], lgkm0


@pytest.fixture(scope="module")
def device_asm(tmp_path_factory):
    """gfx950 assembly of every kernel source of the library, by file name."""
    out = tmp_path_factory.mktemp("asm")
    return {src.name: _device_asm(src, out / (src.stem + ".s")) for src in sorted((PKG / "csrc").glob("*.hip"))}


def test_no_kernel_spills_vector_registers(device_asm):
    spills, checked = [], 0
    for name, asm in device_asm.items():
        if "amdhsa.kernels:" not in asm:  # host-only source (api.hip)
            continue
        entries = asm.split("amdhsa.kernels:", 1)[1]
        for kernel, count in re.findall(r"\.name:\s+(\S+)[^-]*?\.vgpr_spill_count:\s+(\d+)", entries, re.S):
            checked += 1
            if int(count):
                spills.append(f"{name}: {kernel} spills {count} registers")
    assert checked >= 40, f"kernel metadata of only {checked} kernels found"
    assert not spills, "\n".join(spills)


def test_only_the_lds_copies_use_m0(device_asm):
    kernels = {**_kernels(device_asm["attention.hip"]), **_kernels(device_asm["attention_dense.hip"])}
    persistent = {n: b for n, b in kernels.items() if "attention_persistent_kernel" in n}
    assert persistent, "no persistent attention kernel in attention.hip"
    copies = 0
    for name, body in kernels.items():
        for index, instr in enumerate(body):
            if re.search(r"\bm0\b", instr):
                assert re.fullmatch(r"s_mov_b32 m0, s\d+", instr), f"{name}: M0 used by '{instr}'"
                assert index + 2 < len(body) and body[index + 1] == "s_nop 0" and \
                    body[index + 2].startswith("global_load_lds_dwordx4"), \
                    f"{name}: 's_mov_b32 m0' at instruction {index} is not followed by its copy: {body[index:index + 3]}"
            if instr.startswith("global_load_lds_dwordx4"):
                copies += 1
                assert index >= 2 and body[index - 2].startswith("s_mov_b32 m0"), \
                    f"{name}: copy at instruction {index} without its own 's_mov_b32 m0'"
    assert copies > 0
    for name, body in persistent.items():
        assert "s_waitcnt vmcnt(0)" in body, f"{name}: the wait that orders the copies is missing"
