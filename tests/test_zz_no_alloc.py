"""pisa_hip_forward_noalloc (static scratch, no allocation) against pisa_hip_forward (caller workspace).

Both run the same kernels on the same inputs, so the outputs must be equal bit
for bit: first at the Anima profile (B=2 H=16 T=9216, HYD, 23 exact blocks),
then right after with a smaller generic problem (the scratch still holds the
first call's tables), then an oversized problem is refused before any launch.
Everything goes through the C ABI (ctypes); torch only provides device memory
and the stream.
"""
from __future__ import annotations

import math

import pytest
import torch

pytestmark = pytest.mark.gpu
D = 128


@pytest.fixture(scope="module")
def lib():
    from mi355x_pisa import _lib

    return _lib


def _qkv(batch, heads, tokens, seed, dim=D):
    gen = torch.Generator().manual_seed(seed)
    storage = [(0.5 * torch.randn((batch, tokens, heads, dim), generator=gen)).to(torch.bfloat16).cuda()
               for _ in range(3)]
    return [t.permute(0, 2, 1, 3) for t in storage]  # BHTD views of [B,T,H,D] storage


def _args(lib, q, k, v, out, grid, exact, stats, route, first_order):
    batch, heads, tokens, dim = q.shape
    return (lib.DTYPE_BF16, batch, heads, tokens, dim, lib.view4(q), lib.view4(k), lib.view4(v), lib.view4(out),
            lib.grid(*grid), exact, 1.0 / math.sqrt(dim), lib.NO_SINK, stats, route, first_order)


def _both(lib, q, k, v, grid, exact, stats, route, first_order):
    batch, heads, tokens, dim = q.shape
    stream = torch.cuda.current_stream().cuda_stream
    out_ws = torch.empty((batch, heads, tokens, dim), dtype=torch.bfloat16, device="cuda")
    out_static = torch.full_like(out_ws, float("nan"))
    need = lib.LIB.pisa_hip_forward_workspace_bytes(batch, heads, tokens, dim, exact)
    workspace = torch.empty(need, dtype=torch.uint8, device="cuda")
    lib.check(lib.LIB.pisa_hip_forward(*_args(lib, q, k, v, out_ws, grid, exact, stats, route, first_order),
                                       None, None, workspace.data_ptr(), need, stream), "pisa_hip_forward")
    lib.check(lib.LIB.pisa_hip_forward_noalloc(*_args(lib, q, k, v, out_static, grid, exact, stats, route,
                                                      first_order), stream), "pisa_hip_forward_noalloc")
    torch.cuda.synchronize()
    return out_ws, out_static


def test_noalloc_equals_the_workspace_entry_point_on_two_calls(lib):
    # call 1: the Anima profile, 187.3 MiB of the 192 MiB scratch
    q, k, v = _qkv(2, 16, 9216, seed=7)
    ref, got = _both(lib, q, k, v, (1, 96, 96), 23, lib.STATS_HYD, lib.ROUTE_HYD, 1)
    assert torch.isfinite(ref).all()
    assert torch.equal(ref, got)
    # call 2: a smaller generic problem right after (the scratch holds call 1's tables)
    q, k, v = _qkv(1, 3, 4096, seed=8)
    ref, got = _both(lib, q, k, v, (1, 64, 64), 10, lib.STATS_GENERIC, lib.ROUTE_CENTROID, 1)
    assert torch.isfinite(ref).all()
    assert torch.equal(ref, got)
    # call 3: head dim 64 with the first-order term (H_sum partials of the covariance kernel in the scratch)
    q, k, v = _qkv(2, 2, 1000, seed=9, dim=64)
    ref, got = _both(lib, q, k, v, (0, 0, 0), 3, lib.STATS_GENERIC, lib.ROUTE_CENTROID, 1)
    assert torch.isfinite(ref).all()
    assert torch.equal(ref, got)


def test_noalloc_refuses_problems_beyond_the_scratch(lib):
    batch, heads, tokens = 3, 16, 9216
    need = lib.LIB.pisa_hip_forward_workspace_bytes(batch, heads, tokens, D, 23)
    assert need > lib.NOALLOC_SCRATCH_BYTES
    q = torch.zeros((1, 1, 1, D), dtype=torch.bfloat16, device="cuda").expand(batch, heads, tokens, D)
    out = torch.empty((batch, heads, tokens, D), dtype=torch.bfloat16, device="cuda")
    status = lib.LIB.pisa_hip_forward_noalloc(*_args(lib, q, q, q, out, (1, 96, 96), 23, lib.STATS_HYD,
                                                     lib.ROUTE_HYD, 1), torch.cuda.current_stream().cuda_stream)
    assert status == 3  # PISA_ERR_WORKSPACE, returned before any launch
    assert b"static scratch" in lib.LIB.pisa_hip_last_error()


def test_noalloc_call_replays_in_a_hip_graph(lib):
    """The callers this entry point serves are typically capturing: one call captured in a HIP graph
    replays to the eager result bit for bit, with eager calls of another problem (which overwrite the
    scratch) and synchronisations between the replays."""
    q, k, v = _qkv(1, 4, 9216, seed=21)
    eager = torch.empty((1, 4, 9216, D), dtype=torch.bfloat16, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    lib.check(lib.LIB.pisa_hip_forward_noalloc(*_args(lib, q, k, v, eager, (1, 96, 96), 23, lib.STATS_HYD,
                                                      lib.ROUTE_HYD, 1), stream), "pisa_hip_forward_noalloc")
    torch.cuda.synchronize()
    assert torch.isfinite(eager).all()
    replayed = torch.full_like(eager, float("nan"))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        status = lib.LIB.pisa_hip_forward_noalloc(
            *_args(lib, q, k, v, replayed, (1, 96, 96), 23, lib.STATS_HYD, lib.ROUTE_HYD, 1),
            torch.cuda.current_stream().cuda_stream)
    assert status == 0, lib.LIB.pisa_hip_last_error()
    q2, k2, v2 = _qkv(2, 2, 4096, seed=22)
    other = torch.empty((2, 2, 4096, D), dtype=torch.bfloat16, device="cuda")
    for replay in range(3):
        lib.check(lib.LIB.pisa_hip_forward_noalloc(*_args(lib, q2, k2, v2, other, (1, 64, 64), 10,
                                                          lib.STATS_GENERIC, lib.ROUTE_CENTROID, 1), stream),
                  "pisa_hip_forward_noalloc")
        torch.cuda.synchronize()
        replayed.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), f"replay {replay}"
