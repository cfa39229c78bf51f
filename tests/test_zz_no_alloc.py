"""The allocation-free int8 GEMM (hxm_gemm_i8_noalloc) against hxm_gemm_i8,
both called through the C ABI: bit-identical int32 results on two calls in a
row (the second smaller, so the shared static scratch holds the first call's
planes), with and without a K split, captured in a HIP graph and replayed,
plus the host-side refusals."""
import ctypes

import numpy as np
import pytest
import torch

import hxm
from hxm import search as S
from hxm._lib import B_NK, GemmConfig, lib
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

SCRATCH = 64 << 20


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _i8(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-127, 128, shape, generator=g, dtype=torch.int8)


def _cfg(split):
    c = S.gemm_configs(hxm.I8)[0]  # the 256x256 tile
    return GemmConfig(c.bm, c.bn, c.bk, c.waves_m, c.waves_n, c.stages, split)


def _call(fn, A, B, C, M, N, K, accumulate, cfg):
    return fn(A.data_ptr(), A.stride(0), B.data_ptr(), B.stride(0), C.data_ptr(),
              C.stride(0), M, N, K, int(accumulate), ctypes.byref(cfg) if cfg else None,
              _stream())


def _gemm_i8(A, B, C, M, N, K, accumulate, cfg):
    return lib.hxm_gemm_i8(A.data_ptr(), A.stride(0), B.data_ptr(), B.stride(0), B_NK,
                           C.data_ptr(), C.stride(0), M, N, K, int(accumulate),
                           ctypes.byref(cfg) if cfg else None, _stream())


@pytest.mark.parametrize("split", [8, 1, 0])
def test_noalloc_matches_gemm_i8_on_two_calls(dev, split):
    cfg = _cfg(split) if split else None
    for (M, N, K), seed in [((512, 512, 8192), 1), ((200, 264, 4112), 2)]:
        print(f"gemm_i8_noalloc split={split} M={M} N={N} K={K}", flush=True)
        A, B = _i8((M, K), seed), _i8((N, K), seed + 10)
        Ad, Bd = A.to(dev), B.to(dev)
        want = torch.empty(M, N, dtype=torch.int32, device=dev)
        got = torch.full((M, N), -7, dtype=torch.int32, device=dev)
        hxm.check(_gemm_i8(Ad, Bd, want, M, N, K, False, cfg), "hxm_gemm_i8")
        hxm.check(_call(lib.hxm_gemm_i8_noalloc, Ad, Bd, got, M, N, K, False, cfg),
                  "hxm_gemm_i8_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(got, want)
        assert np.array_equal(got.cpu().numpy(), orc.gemm_i8(A.numpy(), B.numpy(), b_nk=True))


def test_noalloc_accumulates_like_gemm_i8(dev):
    M, N, K = 96, 160, 2048
    A, B = _i8((M, K), 3), _i8((N, K), 4)
    Ad, Bd = A.to(dev), B.to(dev)
    base = torch.randint(-1000, 1000, (M, N), dtype=torch.int32).to(dev)
    want, got = base.clone(), base.clone()
    cfg = _cfg(4)
    print("gemm_i8_noalloc accumulate split=4", flush=True)
    hxm.check(_gemm_i8(Ad, Bd, want, M, N, K, True, cfg), "hxm_gemm_i8")
    hxm.check(_call(lib.hxm_gemm_i8_noalloc, Ad, Bd, got, M, N, K, True, cfg),
              "hxm_gemm_i8_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_noalloc_refuses_on_the_host(dev):
    """A split whose planes exceed the static scratch is refused before any
    launch: the output is left untouched."""
    M, N, K = 1024, 1024, 4096            # 16 planes of 4 MiB = 64 MiB + one stage over
    cfg = _cfg(16)
    assert 16 * M * N * 4 >= SCRATCH
    A = torch.zeros(M + 64, K, dtype=torch.int8, device=dev)
    B = torch.zeros(N, K, dtype=torch.int8, device=dev)
    C = torch.zeros(M + 64, N, dtype=torch.int32, device=dev)
    st = _call(lib.hxm_gemm_i8_noalloc, A, B, C, M + 64, N, K, False, cfg)
    assert st == hxm._lib.HXM_UNSUPPORTED_SHAPE and "workspace-budget" in hxm.last_error()
    torch.cuda.synchronize()
    assert int(C.abs().sum()) == 0


def test_noalloc_plan_reports_no_workspace(dev):
    M, N, K = 512, 512, 8192
    A, B = _i8((M, K), 5).to(dev), _i8((N, K), 6).to(dev)
    C = torch.empty(M, N, dtype=torch.int32, device=dev)
    hxm.check(_call(lib.hxm_gemm_i8_noalloc, A, B, C, M, N, K, False, _cfg(8)),
              "hxm_gemm_i8_noalloc")
    import hxm.ops as ops
    p = ops.last_plan()
    assert p["k_slices"] == 8 and p["workspace_bytes"] == 0
    hxm.check(_gemm_i8(A, B, C, M, N, K, False, _cfg(8)), "hxm_gemm_i8")
    assert ops.last_plan()["workspace_bytes"] == 8 * M * N * 4   # the library's own planes
    torch.cuda.synchronize()


def test_noalloc_split_captured_in_a_graph(dev):
    """With every library workspace released, the K-split call is captured on
    a fresh stream (it must not allocate there) and replayed three times, with
    eager work (inputs touched, output poisoned) and a synchronisation between
    replays; each replay equals the eager result bit for bit."""
    M, N, K = 512, 512, 8192
    A, B = _i8((M, K), 7), _i8((N, K), 8)
    Ad, Bd = A.to(dev), B.to(dev)
    cfg = _cfg(8)
    want = torch.empty(M, N, dtype=torch.int32, device=dev)
    got = torch.empty(M, N, dtype=torch.int32, device=dev)
    hxm.check(_gemm_i8(Ad, Bd, want, M, N, K, False, cfg), "hxm_gemm_i8")
    hxm.check(_call(lib.hxm_gemm_i8_noalloc, Ad, Bd, got, M, N, K, False, cfg),
              "hxm_gemm_i8_noalloc")            # eager, on this device first
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    hxm.check(lib.hxm_release_cache(), "hxm_release_cache")
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    print("capturing hxm_gemm_i8_noalloc split=8", flush=True)
    with torch.cuda.graph(graph, stream=s):
        st = _call(lib.hxm_gemm_i8_noalloc, Ad, Bd, got, M, N, K, False, cfg)
    assert st == 0, hxm.last_error()
    keep = Ad.clone()
    for rep in range(3):
        got.fill_(-7)
        Ad.mul_(2).copy_(keep)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {rep}"
    del graph
