"""Stream-K form of the W8A16 GEMMs (split_k = HXM_STREAM_K): the whole
rounds of tiles run one per workgroup, the remaining tiles' K stages are
shared by one workgroup per CU in the same launch, and a tile cut between
workgroups is summed from fp32 partial tiles in segment order by the
workgroup that arrives last.

Checked here: against the oracle at rtol 1e-2 / atol 1e-3 and against the
one-workgroup tiles at the same tolerance (they sum K in another grouping);
bit-identical results on repeated calls (the summation order is fixed, and
the arrival counters are left at zero for the next launch); the three
epilogues (per-channel scale, SwiGLU, residual); streams per XCD and the
global stream; K that ends inside a stage; ragged tiles; shapes with fewer
tiles than CUs (every tile cut) and the benchmark's partial third round; the
plan record; a shape with more arrival counters reusing the buffer an
earlier shape sized; and replays of a captured HIP graph."""
import numpy as np
import pytest
import torch

import hxm
import hxm.ops as ops
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-2, atol=1e-3)
SK = hxm.STREAM_K


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def f32(b):
    return orc.f16_bits_to_f32(b)


def w8_operands(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).half()
    W = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s = (torch.rand(N, generator=g) * 0.019 + 0.001).half().float()
    return x, W, s


def swiglu_operands(M, I, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).half()
    Wg = torch.randint(-127, 128, (I, K), generator=g, dtype=torch.int8)
    Wu = torch.randint(-127, 128, (I, K), generator=g, dtype=torch.int8)
    sc = 1.0 / np.sqrt(K * 127.0 ** 2 / 3.0)
    sg = ((torch.rand(I, generator=g) + 0.5) * sc).half().float()
    su = ((torch.rand(I, generator=g) + 0.5) * sc).half().float()
    return x, Wg, Wu, sg, su


# (M, N, K) on the tile that has a stream-K form: 256x256, 64 f16 of K per
# stage, 3 stages (the benchmark's gate/up tile).
#   512x4096x1024: 32 tiles < 256 CUs, all cut (8 segments each), per-XCD streams
#   300x520x656: 6 ragged tiles, K ends inside a stage, the global stream
#   768x768x2048: 9 tiles (not a multiple of 8), the global stream
#   2048x4608x512: 144 tiles; 2048x17408x512: 544 tiles = 2 rounds + 32
TILE = (256, 256, 64, 2, 2, 3)
CASES = [(512, 4096, 1024, TILE), (300, 520, 656, TILE), (768, 768, 2048, TILE),
         (2048, 4608, 512, TILE), (2048, 17408, 512, TILE)]


def _sample(M):
    return np.unique(np.linspace(0, M - 1, 12).astype(int))


@pytest.mark.parametrize("M,N,K,tile", CASES, ids=[f"{c[0]}x{c[1]}x{c[2]}" for c in CASES])
def test_stream_k_w8a16(dev, M, N, K, tile):
    print(f"stream-K w8a16 M={M} N={N} K={K} tile={tile}", flush=True)
    x, W, s = w8_operands(M, N, K, M + N + K)
    xd, Wd, sd = x.to(dev), W.to(dev), s.to(dev)
    y_sk = ops.gemm_w8a16(xd, Wd, sd, config=tile + (SK,))
    p = ops.last_plan()
    assert p["config"][6] == SK and p["k_slices"] >= 2 and p["workspace_bytes"] > 0
    y_dp = ops.gemm_w8a16(xd, Wd, sd, config=tile + (1,))
    np.testing.assert_allclose(y_sk.float().cpu().numpy(), y_dp.float().cpu().numpy(), **TOL)
    rows = _sample(M)
    ref = orc.gemm_w8a16(bits(x)[rows], W.numpy(), s.numpy())
    np.testing.assert_allclose(f32(bits(y_sk)[rows]), f32(ref), **TOL)
    for _ in range(2):  # fixed summation order, counters back at zero
        assert torch.equal(ops.gemm_w8a16(xd, Wd, sd, config=tile + (SK,)), y_sk)


def test_stream_k_residual(dev):
    M, N, K = 512, 4096, 1024
    print(f"stream-K w8a16 residual M={M} N={N} K={K}", flush=True)
    x, W, s = w8_operands(M, N, K, 3)
    r = torch.randn(M, N, generator=torch.Generator().manual_seed(4)).half()
    xd, Wd, sd, rd = x.to(dev), W.to(dev), s.to(dev), r.to(dev)
    tile = (256, 256, 64, 2, 2, 3)
    y = ops.gemm_w8a16(xd, Wd, sd, residual=rd, config=tile + (SK,))
    rows = _sample(M)
    ref = orc.gemm_w8a16_residual(bits(x)[rows], W.numpy(), s.numpy(), bits(r)[rows])
    np.testing.assert_allclose(f32(bits(y)[rows]), f32(ref), **TOL)
    assert torch.equal(ops.gemm_w8a16(xd, Wd, sd, residual=rd, config=tile + (SK,)), y)


@pytest.mark.parametrize("M,I,K", [(2048, 11008, 4096), (512, 704, 1024), (300, 200, 656)])
def test_stream_k_swiglu(dev, M, I, K):
    """The benchmark's gate/up GEMM (688 tiles: two whole rounds and 176
    tiles streamed by 32 workgroups per XCD), and small shapes where every
    tile is cut."""
    print(f"stream-K swiglu M={M} I={I} K={K}", flush=True)
    x, Wg, Wu, sg, su = swiglu_operands(M, I, K, M + I)
    Wgu, sgu = ops.swiglu_pack(Wg.to(dev), Wu.to(dev), sg.to(dev), su.to(dev))
    xd = x.to(dev)
    tile = (256, 256, 64, 2, 2, 3)
    h_sk = ops.gemm_w8a16_swiglu(xd, Wgu, sgu, I, config=tile + (SK,))
    h_dp = ops.gemm_w8a16_swiglu(xd, Wgu, sgu, I, config=tile + (1,))
    np.testing.assert_allclose(h_sk.float().cpu().numpy(), h_dp.float().cpu().numpy(), **TOL)
    rows = _sample(M)
    ref = orc.swiglu_gateup(bits(x)[rows], Wg.numpy(), Wu.numpy(), sg.numpy(), su.numpy())
    np.testing.assert_allclose(f32(bits(h_sk)[rows]), f32(ref), **TOL)
    assert torch.equal(ops.gemm_w8a16_swiglu(xd, Wgu, sgu, I, config=tile + (SK,)), h_sk)


def test_stream_k_counters_zero_across_shapes(dev):
    """A stream's stream-K buffer is reused by every shape that fits it.  The
    first shape (256x8448x256: 33 partial-round tiles cut in up to 4
    segments, a 34.6 MB buffer) sizes the buffer; the second (1280x3328x256:
    65 tiles of up to 2 segments, 34.1 MB) fits in it and has more arrival
    counters than the first.  Its counters must still start at zero, not
    in bytes the first shape used for partial tiles: every tile of the
    second call is written and equals the one-workgroup tiles' result."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    if cus != 256:
        pytest.skip(f"the shape pair is chosen for 256 CUs (this device has {cus})")
    tile = (256, 256, 64, 2, 2, 3)
    stream = torch.cuda.Stream()
    assert hxm.lib.hxm_release_cache() == 0  # no stream-K buffer yet
    outs = []
    for (M, N, K, seed) in [(256, 8448, 256, 11), (1280, 3328, 256, 12)]:
        print(f"stream-K counters M={M} N={N} K={K}", flush=True)
        x, W, s = w8_operands(M, N, K, seed)
        xd, Wd, sd = x.to(dev), W.to(dev), s.to(dev)
        y = torch.full((M, N), -7.0, dtype=torch.float16, device=dev)
        with torch.cuda.stream(stream):
            ops.gemm_w8a16(xd, Wd, sd, out=y, config=tile + (SK,))
            p = ops.last_plan()
        torch.cuda.synchronize()
        assert p["config"][6] == SK
        outs.append((p["workspace_bytes"], p["k_slices"]))
        want = ops.gemm_w8a16(xd, Wd, sd, config=tile + (1,))
        np.testing.assert_allclose(y.float().cpu().numpy(), want.float().cpu().numpy(), **TOL)
    assert outs[1][0] <= outs[0][0] and (outs[0][1], outs[1][1]) == (4, 2), outs


def test_stream_k_refused_where_not_compiled(dev):
    """Only the gate/up tile has a stream-K form: another tile asked for in
    that form is refused on the host with the lattice's no-kernel reason."""
    x, W, s = w8_operands(64, 256, 128, 9)
    with pytest.raises(Exception, match="no-kernel"):
        ops.gemm_w8a16(x.to(dev), W.to(dev), s.to(dev), config=(256, 128, 64, 2, 2, 3, SK))


def test_stream_k_whole_rounds_run_as_plain_tiles(dev):
    """Tiles that fill whole rounds leave nothing to stream: the call runs
    the one-workgroup tiles and the plan says split_k 1, bit for bit the same."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    M, N, K = 256, 256 * cus, 128
    x, W, s = w8_operands(M, N, K, 5)
    xd, Wd, sd = x.to(dev), W.to(dev), s.to(dev)
    tile = (256, 256, 64, 2, 2, 3)
    y_sk = ops.gemm_w8a16(xd, Wd, sd, config=tile + (SK,))
    assert ops.last_plan()["config"][6] == 1 and ops.last_plan()["workspace_bytes"] == 0
    assert torch.equal(y_sk, ops.gemm_w8a16(xd, Wd, sd, config=tile + (1,)))


def test_stream_k_graph_replays(dev):
    """Captured after one eager call (which sizes the stream's workspace),
    three replays with eager work between them equal the eager result."""
    M, N, K = 512, 4096, 1024
    x, W, s = w8_operands(M, N, K, 6)
    xd, Wd, sd = x.to(dev), W.to(dev), s.to(dev)
    tile = (256, 256, 64, 2, 2, 3, SK)
    stream = torch.cuda.Stream()
    y = torch.empty(M, N, dtype=torch.float16, device=dev)
    with torch.cuda.stream(stream):
        ops.gemm_w8a16(xd, Wd, sd, out=y, config=tile)
    torch.cuda.synchronize()
    want = y.clone()
    graph = torch.cuda.CUDAGraph()
    print("capturing stream-K w8a16", flush=True)
    with torch.cuda.graph(graph, stream=stream):
        ops.gemm_w8a16(xd, Wd, sd, out=y, config=tile)
    keep = xd.clone()
    for rep in range(3):
        y.fill_(-7.0)
        xd.mul_(2.0).copy_(keep)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want), f"replay {rep}"
    del graph


def test_tune_w8a16_measures_stream_k(dev):
    """The W8A16 tuner adds the stream-K form of the tile that has one when
    its tiles leave a partial round, verifies it within the float tolerance
    and may crown it; the cached winner then matches the oracle."""
    hxm.lib.hxm_tune_cache_clear()
    M, I, K = 2048, 2752, 1024
    x, Wg, Wu, sg, su = swiglu_operands(M, I, K, 8)
    Wgu, sgu = ops.swiglu_pack(Wg.to(dev), Wu.to(dev), sg.to(dev), su.to(dev))
    xd = x.to(dev)
    h = torch.empty(M, I, dtype=torch.float16, device=dev)
    best, rep = ops.tune_w8a16(xd, Wgu, sgu, h, swiglu=True, reps=3)
    sk = [c for c in rep["configs"] if c["split_k"] == SK]
    assert sk and all(c["verified"] for c in sk)
    h2 = ops.gemm_w8a16_swiglu(xd, Wgu, sgu, I)
    rows = _sample(M)
    ref = orc.swiglu_gateup(bits(x)[rows], Wg.numpy(), Wu.numpy(), sg.numpy(), su.numpy())
    np.testing.assert_allclose(f32(bits(h2)[rows]), f32(ref), **TOL)
    hxm.lib.hxm_tune_cache_clear()
