"""The C ABI library loads on the CPU and exports exactly what include/pisa_hip.h declares.

No kernel is launched here: only metadata calls and argument validation that
returns before touching a device.
"""
from __future__ import annotations

import ctypes
import pathlib
import re
import subprocess

import pytest

REPO = pathlib.Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "pisa_hip.h"


def _declared() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"PISA_HIP_EXPORT\s+[\w\s\*]+?\b((?:pisa|attn)_hip_\w+)\s*\(", text))


@pytest.fixture(scope="module")
def lib():
    from mi355x_pisa import _lib

    return _lib


def test_header_declares_the_api():
    names = _declared()
    assert {"pisa_hip_forward", "pisa_hip_prepare", "pisa_hip_attend", "pisa_hip_block_stats",
            "pisa_hip_route_topk", "attn_hip_dense_forward", "attn_hip_fixed_block_forward",
            "pisa_hip_pack_spatial_qkv", "pisa_hip_unpack_spatial_output",
            "pisa_hip_fuse_spatial_epilogue"} <= names


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    declared = _declared()
    assert declared == exported, (declared ^ exported)
    assert declared == set(lib.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib.LIB, name)


def test_metadata_calls(lib):
    assert lib.LIB.pisa_hip_api_version() == 1
    info = lib.build_info_string()
    assert "architecture=gfx950" in info and "block_size=64" in info
    assert lib.LIB.pisa_hip_status_string(0) == b"ok"
    assert lib.LIB.pisa_hip_status_string(3) == b"workspace too small"
    small = ctypes.create_string_buffer(4)
    assert lib.LIB.pisa_hip_build_info(small, 4) == 1


def test_workspace_sizes(lib):
    c4 = lib.LIB.pisa_hip_forward_workspace_bytes(2, 16, 9216, 128, 23)
    # the packed K and V block tables alone are 2 x B*H*T*D bf16
    assert c4 > 2 * (2 * 16 * 9216 * 128 * 2)
    assert lib.LIB.pisa_hip_forward_workspace_bytes(0, 16, 9216, 128, 23) == 0
    assert lib.LIB.attn_hip_dense_workspace_bytes(2, 16, 512, 128) == 2 * (2 * 16 * 512 * 128 * 2)
    assert lib.LIB.attn_hip_dense_workspace_bytes(1, 1, 65, 64) == 2 * (128 * 64 * 2)
    # other head dims: packed tables at the padded width (40 -> 64, 80 -> 96, 160 -> 160, 200 -> 256)
    for d, dp in ((40, 64), (80, 96), (160, 160), (200, 256), (8, 64)):
        assert lib.LIB.attn_hip_dense_workspace_bytes(1, 2, 128, d) == 2 * (2 * 128 * dp * 2)
    # generic PISA off 128 has no H_sum partials: smaller than at 128 despite the padding of 80 -> 96
    assert lib.LIB.pisa_hip_forward_workspace_bytes(1, 4, 8192, 80, 32) < \
        lib.LIB.pisa_hip_forward_workspace_bytes(1, 4, 8192, 128, 32)
    assert lib.LIB.pisa_hip_forward_workspace_bytes(1, 4, 8192, 80, 32) > 2 * (4 * 8192 * 96 * 2)


def _views(lib):
    fake = lib.PisaView(0x1000, 9216 * 16 * 128, 128, 16 * 128)
    return fake, fake, fake, fake


def test_forward_validation_rejects_before_any_launch(lib):
    q, k, v, o = _views(lib)
    grid = lib.grid(1, 96, 96)
    args = dict(dtype=0, batch=2, heads=16, tokens=9216, head_dim=128, exact=23, scale=0.088, sink=-2, stats=1,
                route=0, first=1)

    def call(**over):
        a = {**args, **over}
        return lib.LIB.pisa_hip_forward(a["dtype"], a["batch"], a["heads"], a["tokens"], a["head_dim"], q, k, v, o,
                                        over.get("grid", grid), a["exact"], a["scale"], a["sink"], a["stats"],
                                        a["route"], a["first"], None, None, None, 0, None)

    assert call(head_dim=64) == 2                      # HYD statistics only at 128
    generic = dict(stats=lib.STATS_GENERIC, route=lib.ROUTE_CENTROID, first=0)
    assert call(head_dim=100, **generic) == 2          # not a multiple of 8
    assert call(head_dim=264, **generic) == 2          # above 256
    assert call(head_dim=64, **{**generic, "route": lib.ROUTE_HYD}) == 2
    assert call(head_dim=64, **generic) == 3           # supported: fails only for the missing workspace
    assert call(head_dim=64, **{**generic, "first": 1}) == 3   # first-order term at any width, as the reference's
    assert call(dtype=2) == 2                          # fp32 not supported by PISA
    assert call(exact=144) == 1                        # dense goes to attn_hip_dense_forward
    assert call(exact=0, sink=0) == 1                  # sink needs an exact block
    assert call(scale=0.0) == 1
    assert call(scale=float("inf")) == 1
    assert call(grid=lib.grid(1, 96, 90)) == 1         # width not a multiple of 8
    assert call(grid=lib.grid(2, 96, 96)) == 1         # grid does not match T
    assert call() == 3                                 # no workspace
    assert b"workspace" in lib.LIB.pisa_hip_last_error()


def test_other_entry_points_validate(lib):
    q, k, v, o = _views(lib)
    assert lib.LIB.attn_hip_dense_forward(0, 1, 1, 64, 64, 100, q, k, v, o, 0.1, None, 0, None) == 2
    assert lib.LIB.attn_hip_dense_forward(0, 1, 1, 64, 64, 264, q, k, v, o, 0.1, None, 0, None) == 2
    # one head's packed key table above 2 GiB (32-bit offsets in the kernel) is refused before any launch
    assert lib.LIB.attn_hip_dense_forward(0, 1, 1, 64, 1 << 23, 256, q, k, v, o, 0.1, None, 0, None) == 2
    assert b"above 2 GiB" in lib.LIB.pisa_hip_last_error()
    # B*H above 65535 or more than 2^24 - 1 blocks over all heads: refused before any launch, and the
    # int32 product B*H is never formed for them
    assert lib.LIB.attn_hip_dense_forward(0, 1 << 16, 1 << 16, 64, 64, 128, q, k, v, o, 0.1, None, 0, None) == 2
    assert b"B*H <= 65535" in lib.LIB.pisa_hip_last_error()
    assert lib.LIB.attn_hip_dense_forward(0, 4, 4096, 64, 1 << 16, 128, q, k, v, o, 0.1, None, 0, None) == 2
    assert lib.LIB.attn_hip_dense_workspace_bytes(4, 4096, 1 << 16, 128) == 0
    assert lib.LIB.attn_hip_fixed_block_forward(2, 1, 1, 1 << 30, 64, 64, q, k, v, o, 0.1, 0, None) == 2
    assert lib.LIB.pisa_hip_forward_workspace_bytes(70000, 1, 64, 128, 0) == 0
    assert lib.LIB.pisa_hip_block_stats_workspace_bytes(1, 70000, 64, 128) == 0
    assert lib.LIB.attn_hip_fixed_block_forward(0, 1, 1, 64, 48, 64, q, k, v, o, 0.1, 0, None) == 2
    assert lib.LIB.attn_hip_fixed_block_forward(0, 1, 1, 64, 64, 32, q, k, v, o, 0.1, 0, None) == 2
    assert lib.LIB.pisa_hip_route_topk(1, 2000, 128, None, None, None, 1, 0.1, -2, 3, None, None, None) == 2
    assert lib.LIB.pisa_hip_route_topk(1, 10, 128, None, None, None, 1, 0.1, 5, 3, None, None, None) == 1
    stats = lambda mode, out_dtype, head_dim=128: lib.LIB.pisa_hip_block_stats(  # noqa: E731
        0, out_dtype, 1, 1, 64, head_dim, q, k, v, lib.grid(), mode, None, None, None, None, None, None, 0, None)
    sums = lib.STATS_FLAG_VALUE_SUMS
    assert stats(lib.STATS_MEANS | sums, 2) == 1        # value sums need HYD / GENERIC statistics ...
    assert stats(lib.STATS_GENERIC | sums, 0) == 1      # ... and float32 outputs
    assert stats(lib.STATS_GENERIC | sums, 2) == 1      # accepted flag: fails only for the missing outputs
    assert b"centroid outputs" in lib.LIB.pisa_hip_last_error()
    assert stats(lib.STATS_HYD, 0, head_dim=264) == 2   # statistics: any 0 < D <= 256 ...
    assert b"head_dim <= 256" in lib.LIB.pisa_hip_last_error()
    assert stats(lib.STATS_HYD, 0, head_dim=0) == 2
    assert stats(lib.STATS_HYD, 0, head_dim=100) == 1   # ... odd widths accepted: fails only for the outputs
    assert b"centroid outputs" in lib.LIB.pisa_hip_last_error()
    misaligned = lib.PisaView(0x1002, 0, 0, 128)
    assert lib.LIB.pisa_hip_pack_spatial_qkv(0, 1, 1, 9216, 128, misaligned, k, v, lib.grid(1, 96, 96), None,
                                             None, None, None) == 1


def _reference_stats_choice(module, q, k, v, device_accepts: bool = False) -> str:
    """The reference's generic statistics choice (generic_pisa.py:119-128) restated against `module`.

    'hyd' when the module lists q's head dim and dtype among its HYD statistics and its block_stats_hyd
    accepts the call, else 'generic'.  device_accepts: on CPU tensors, a refusal that names only the
    device counts as acceptance (the shape and dtype checks come before the device check, as in
    __init__.py:216-230), so the decision is visible without a GPU.
    """
    try:
        caps = module.capabilities()
        if q.shape[-1] in caps.get("hyd_stats_head_dims", ()) and q.dtype in caps.get("hyd_stats_dtypes", ()):
            try:
                module.block_stats_hyd(q, k, v)
            except ValueError as exc:
                if not (device_accepts and "ROCm device" in str(exc)):
                    raise
            return "hyd"
    except (ImportError, OSError, RuntimeError, AttributeError, ValueError):
        pass
    return "generic"


def test_reference_module_name_keeps_the_reference_contract():
    """`import rdna35_pisa_ck` runs the mi355x_pisa kernels behind the reference's limits
    (native/rdna35_pisa_ck/rdna35_pisa_ck/__init__.py:27-29,216-230,455-474)."""
    import torch

    import mi355x_pisa
    import rdna35_pisa_ck

    assert rdna35_pisa_ck is not mi355x_pisa
    assert rdna35_pisa_ck.forward_spatial_bhtd is mi355x_pisa.forward_spatial_bhtd
    assert (rdna35_pisa_ck.MAX_BLOCKS, rdna35_pisa_ck.MAX_TOKENS) == (144, 9216)
    caps = rdna35_pisa_ck.capabilities()
    assert caps["architecture"] == "gfx950"
    assert caps["max_blocks"] == 144
    assert caps["hyd_stats_dtypes"] == (torch.bfloat16,)
    assert caps["hyd_stats_head_dims"] == (128,)
    assert rdna35_pisa_ck.SPATIAL_SPARSE_EXACT_BLOCKS == 23
    # the wider module agrees on the keys the reference's generic path reads
    wide = mi355x_pisa.capabilities()
    assert wide["hyd_stats_dtypes"] == caps["hyd_stats_dtypes"]
    assert wide["hyd_stats_head_dims"] == caps["hyd_stats_head_dims"]
    assert 256 in wide["block_stats_hyd_head_dims"] and torch.float16 in wide["block_stats_hyd_dtypes"]

    long = torch.zeros((1, 9280, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="0<T<=9216"):
        rdna35_pisa_ck.block_stats_hyd(long, long, long)
    with pytest.raises(ValueError, match="0<T<=9216"):
        rdna35_pisa_ck.forward(long, long, long, 23)
    with pytest.raises(RuntimeError, match="T<=9216"):
        rdna35_pisa_ck._C.block_stats_hyd(long, long, long)
    with pytest.raises(RuntimeError, match="T<=9216"):
        rdna35_pisa_ck._C.block_stats(long, long, long)
    # widths above 256 are refused with the limit named
    wide_d = torch.zeros((1, 64, 264), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="0<D<=256"):
        mi355x_pisa.block_stats_hyd(wide_d, wide_d, wide_d)


@pytest.mark.parametrize("dtype_name, tokens, head_dim", [
    ("bfloat16", 8192, 128), ("float16", 8192, 128), ("bfloat16", 32768, 128), ("bfloat16", 9216, 128),
    ("bfloat16", 9217, 128), ("bfloat16", 8192, 64), ("float16", 32768, 128),
])
def test_reference_stats_choice_through_the_alias_matches_generic_stats_mode(dtype_name, tokens, head_dim):
    """The reference's _block_stats rule run against `rdna35_pisa_ck` picks the regime that
    mi355x_pisa.generic_stats_mode (the HIP generic path's choice) picks."""
    import torch

    import mi355x_pisa
    import rdna35_pisa_ck

    dtype = getattr(torch, dtype_name)
    x = torch.zeros((1, tokens, head_dim), dtype=dtype)
    chosen = _reference_stats_choice(rdna35_pisa_ck, x, x, x, device_accepts=True)
    assert chosen == mi355x_pisa.generic_stats_mode(tokens, head_dim, dtype)
    expected = "hyd" if (dtype == torch.bfloat16 and head_dim == 128 and tokens <= 9216) else "generic"
    assert chosen == expected


def test_noalloc_scratch_size_holds_the_anima_profile(lib):
    """The header's PISA_NOALLOC_SCRATCH_BYTES, the binding's constant and the entry point's refusal agree,
    and the static scratch holds the Anima profile (B=2 H=16 T=9216) at every exact-block count."""
    define = re.search(r"#define\s+PISA_NOALLOC_SCRATCH_BYTES\s+\((\d+)LL\s*<<\s*(\d+)\)", HEADER.read_text())
    assert define, "PISA_NOALLOC_SCRATCH_BYTES not found in the header"
    scratch = int(define.group(1)) << int(define.group(2))
    assert scratch == lib.NOALLOC_SCRATCH_BYTES
    for exact in (0, 1, 23, 143):
        assert lib.LIB.pisa_hip_forward_workspace_bytes(2, 16, 9216, 128, exact) <= scratch
    assert lib.LIB.pisa_hip_forward_workspace_bytes(2, 17, 9216, 128, 23) > scratch
    q, k, v, o = _views(lib)
    # the size check comes before any device call: refused here, without a GPU
    status = lib.LIB.pisa_hip_forward_noalloc(0, 2, 17, 9216, 128, q, k, v, o, lib.grid(1, 96, 96), 23, 0.088, -2, 1,
                                              0, 1, None)
    assert status == 3
    assert b"static scratch" in lib.LIB.pisa_hip_last_error()
