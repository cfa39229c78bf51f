"""GPU parity of the row reductions and the W8A16 GEMV against the CPU
oracle (rtol 1e-2 / atol 1e-3 for fp16 outputs; the reference's own test
tolerances, test_softmax.py:27-28 and test_rms_norm.py:24, are looser)."""
import numpy as np
import pytest
import torch

import hxm.ops as ops
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TDT = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


def host_bits(t, name):
    t = t.cpu()
    if name == "f32":
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def tol(name):
    return dict(rtol=1e-2, atol=1e-3) if name != "f32" else dict(rtol=1e-5, atol=1e-6)


# (33, 4096), (5, 2048) and (1, 4096): full rows of 8 vectors per lane for
# f16/bf16 and for f32, which every op splits over several waves (LayerNorm
# two, with an odd row count the last workgroup's second row is past the
# end; softmax and RMSNorm four, one row per workgroup).
ROW_SHAPES = [(128, 128), (127, 513), (8192, 4096), (27, 8192), (5, 1), (3, 20000), (64, 1000),
              (33, 4096), (5, 2048), (1, 4096)]


@pytest.mark.parametrize("rows,cols", ROW_SHAPES)
@pytest.mark.parametrize("name", ["f16", "bf16", "f32"])
def test_softmax(dev, rows, cols, name):
    print(f"softmax {name} {rows}x{cols}", flush=True)
    g = torch.Generator().manual_seed(rows * 7 + cols)
    x = (torch.randn(rows, cols, generator=g) * 2).to(TDT[name])
    y = ops.softmax(x.to(dev))
    ref = orc.to_f32(orc.softmax_rows(host_bits(x, name), name), name)
    got = y.float().cpu().numpy()
    np.testing.assert_allclose(got, ref, **tol(name))
    assert np.allclose(got.sum(axis=1), 1.0, atol=2e-2)


@pytest.mark.parametrize("r", range(8))
def test_softmax_row_order_covers_every_row(dev, r):
    """Softmax takes its row groups XCD-contiguously: for every grid size
    mod 8 = r (full f16 rows of 4096, one row per workgroup) each row is
    written once, with its own softmax (y starts as NaN)."""
    rows, cols = 8 * 9 + r, 4096
    g = torch.Generator().manual_seed(300 + r)
    x = (torch.randn(rows, cols, generator=g) * 2).half()
    y = torch.full((rows, cols), float("nan"), dtype=torch.float16, device=dev)
    ops.softmax(x.to(dev), out=y)
    ref = orc.to_f32(orc.softmax_rows(host_bits(x, "f16"), "f16"), "f16")
    got = y.float().cpu().numpy()
    assert np.isfinite(got).all()
    np.testing.assert_allclose(got, ref, **tol("f16"))


@pytest.mark.parametrize("rows,cols", ROW_SHAPES)
@pytest.mark.parametrize("name", ["f16", "bf16", "f32"])
def test_rmsnorm(dev, rows, cols, name):
    print(f"rmsnorm {name} {rows}x{cols}", flush=True)
    g = torch.Generator().manual_seed(rows * 11 + cols)
    x = (torch.randn(rows, cols, generator=g) * 2).to(TDT[name])
    w = (1 + 0.1 * torch.randn(cols, generator=g)).to(TDT[name])
    y = ops.rms_norm(x.to(dev), (cols,), weight=w.to(dev), eps=1e-6)
    ref = orc.to_f32(orc.rmsnorm_rows(host_bits(x, name), host_bits(w, name), 1e-6, name), name)
    np.testing.assert_allclose(y.float().cpu().numpy(), ref, **tol(name))


@pytest.mark.parametrize("rows,cols", [(27, 8192), (8192, 4096), (33, 300), (2, 17000),
                                       (33, 4096), (5, 2048), (1, 4096)])
@pytest.mark.parametrize("name", ["f32", "f16", "bf16"])
def test_layernorm(dev, rows, cols, name):
    print(f"layernorm {name} {rows}x{cols}", flush=True)
    g = torch.Generator().manual_seed(rows + cols)
    x = torch.rand(rows, cols, generator=g).to(TDT[name])
    w = torch.rand(cols, generator=g).to(TDT[name])
    b = torch.rand(cols, generator=g).to(TDT[name])
    y, mean, rstd = ops.layer_norm(x.to(dev), (cols,), w.to(dev), b.to(dev), eps=1e-5,
                                   return_stats=True)
    ry, rm, rr = orc.layernorm_rows(host_bits(x, name), host_bits(w, name), host_bits(b, name),
                                    1e-5, name)
    np.testing.assert_allclose(y.float().cpu().numpy(), orc.to_f32(ry, name), **tol(name))
    np.testing.assert_allclose(mean.cpu().numpy(), rm, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(rstd.cpu().numpy(), rr, rtol=1e-4)


@pytest.mark.parametrize("rows,cols", [(4, 4096), (5, 2048), (3, 300), (2, 1), (2, 17000)])
@pytest.mark.parametrize("name", ["f32", "f16"])
def test_layernorm_constant_rows_give_beta(dev, rows, cols, name):
    """Closed form: a constant row has x - mean = 0 exactly and variance 0,
    so LayerNorm returns beta exactly whatever gamma and the constant, with
    mean = the constant and rstd = 1/sqrt(eps).  The constants keep every
    partial sum exact in fp32, so no summation order can move the mean."""
    print(f"layernorm constant rows {name} {rows}x{cols}", flush=True)
    g = torch.Generator().manual_seed(rows * 3 + cols)
    consts = torch.tensor([1.5, -3.25, 96.0, 0.375, -7.0][:rows])
    x = consts[:, None].expand(rows, cols).contiguous().to(TDT[name])
    w = (1 + 0.1 * torch.randn(cols, generator=g)).to(TDT[name])
    b = torch.randn(cols, generator=g).to(TDT[name])
    y, mean, rstd = ops.layer_norm(x.to(dev), (cols,), w.to(dev), b.to(dev), eps=1e-5,
                                   return_stats=True)
    assert torch.equal(y.cpu(), b.expand(rows, cols)), "y must equal beta"
    assert torch.equal(mean.cpu(), consts)
    want = np.float32(1.0) / np.sqrt(np.float32(1e-5))
    np.testing.assert_allclose(rstd.cpu().numpy(), np.full(rows, want, np.float32), rtol=1e-6)


@pytest.mark.parametrize("rows,cols", [(62, 8384), (68, 1293), (40, 300), (4, 4096)])
def test_layernorm_f32_error_follows_the_conditioning(dev, rows, cols):
    """f32 rows far from zero mean (x = 3 + 0.01 z, |mean| / sigma = 300): any
    LayerNorm that holds the mean in fp32 shifts every x - mean by the mean's
    rounding, a few ulp(|mean|), and rstd = 1/sigma scales that shift into y.
    So y is held to 4 eps32 |mean| rstd max|gamma| on top of the 1e-5 that
    well-conditioned rows meet, and to no worse than three times a float32
    two-pass LayerNorm of the same rows (numpy, float32 throughout)."""
    print(f"layernorm f32 conditioning {rows}x{cols}", flush=True)
    g = torch.Generator().manual_seed(rows * cols)
    x = torch.randn(rows, cols, generator=g) * 0.01 + 3.0
    w = 1 + 0.1 * torch.randn(cols, generator=g)
    b = 0.1 * torch.randn(cols, generator=g)
    got = ops.layer_norm(x.to(dev), (cols,), w.to(dev), b.to(dev), eps=1e-5).cpu().numpy()
    ry, rm, rr = orc.layernorm_rows(x.numpy(), w.numpy(), b.numpy(), 1e-5, "f32")
    eps32 = float(np.finfo(np.float32).eps)
    shift = 4 * eps32 * np.abs(rm) * rr * float(w.abs().max())
    err = np.abs(got - ry)
    assert (err <= 1e-5 + 1e-5 * np.abs(ry) + shift[:, None]).all()
    xn = x.numpy()
    m = xn.sum(axis=1, dtype=np.float32) / np.float32(cols)
    c = xn - m[:, None]
    r = np.float32(1) / np.sqrt((c * c).sum(axis=1, dtype=np.float32) / np.float32(cols)
                                + np.float32(1e-5))
    np32 = (c * r[:, None]) * w.numpy() + b.numpy()
    assert err.max() <= 3 * np.abs(np32 - ry).max() + 2e-6


def test_rows_golden(dev, golden):
    g = golden("rows")
    xs = torch.from_numpy(g["softmax_x_bits"].view(np.float16)).to(dev)
    np.testing.assert_allclose(ops.softmax(xs).float().cpu().numpy(), g["softmax_y"],
                               rtol=1e-2, atol=1e-3)
    xr = torch.from_numpy(g["rms_x_bits"].view(np.float16)).to(dev)
    gr = torch.from_numpy(g["rms_gamma_bits"].view(np.float16)).to(dev)
    np.testing.assert_allclose(ops.rms_norm(xr, (513,), gr, eps=1e-6).float().cpu().numpy(),
                               g["rms_y"], rtol=1e-2, atol=1e-2)
    xl = torch.from_numpy(g["ln_x"]).to(dev)
    y = ops.layer_norm(xl, (8192,), torch.from_numpy(g["ln_w"]).to(dev),
                       torch.from_numpy(g["ln_b"]).to(dev), eps=1e-5)
    np.testing.assert_allclose(y.cpu().numpy(), g["ln_y"], rtol=1e-5, atol=1e-5)


def test_rows_strided_inplace_and_edge_values(dev):
    x = (torch.randn(16, 700) * 3).half()
    xd = torch.zeros(16, 704, dtype=torch.float16, device=dev)
    xd[:, :700] = x.to(dev)
    view = xd[:, :700]                      # ld 704: aligned rows
    ops.softmax(view, out=view)             # in place
    ref = orc.f16_bits_to_f32(orc.softmax_rows(host_bits(x, "f16")))
    np.testing.assert_allclose(view.float().cpu().numpy(), ref, rtol=1e-2, atol=1e-3)
    odd = torch.randn(9, 101).half()        # ld 101: unaligned rows
    od = odd.to(dev)
    np.testing.assert_allclose(ops.softmax(od).float().cpu().numpy(),
                               orc.f16_bits_to_f32(orc.softmax_rows(host_bits(odd, "f16"))),
                               rtol=1e-2, atol=1e-3)
    # a -inf entry gets probability 0; a constant row is uniform
    e = torch.zeros(2, 64, dtype=torch.float16)
    e[0, 5] = float("-inf")
    y = ops.softmax(e.to(dev)).cpu()
    assert y[0, 5] == 0 and torch.allclose(y[1].float(), torch.full((64,), 1 / 64), atol=1e-4)
    # zero row through RMSNorm stays 0 (eps inside the root)
    z = ops.rms_norm(torch.zeros(1, 256, dtype=torch.float16, device=dev), (256,), eps=1e-6)
    assert (z.cpu() == 0).all()
    assert ops.softmax(torch.empty(0, 32, dtype=torch.float16, device=dev)).shape == (0, 32)


def test_grid_beyond_the_launch_limit_is_refused(dev):
    """2^26 + 4 rows need 2^24 + 1 workgroups of 256 threads, more than 2^32
    work-items: refused before any launch, nothing written.  The buffers hold
    every row, so the test reads and writes in bounds whatever the launcher
    does."""
    import hxm
    from hxm import _lib
    rows = (1 << 26) + 4
    x = torch.zeros(rows, 8, dtype=torch.float16, device=dev)
    y = torch.full((rows, 8), 3.0, dtype=torch.float16, device=dev)
    st = hxm.lib.hxm_softmax_rows(x.data_ptr(), 8, y.data_ptr(), 8, rows, 8, hxm.F16,
                                  torch.cuda.current_stream().cuda_stream)
    assert st == _lib.HXM_UNSUPPORTED_SHAPE and "launch limit" in hxm.last_error()
    assert bool((y[-4:] == 3).all()) and bool((y[:4] == 3).all())
    del x, y
    torch.cuda.empty_cache()


@pytest.mark.parametrize("M", [1, 4, 16])
@pytest.mark.parametrize("packed", [True, False])
def test_gemv_baseline_shape(dev, M, packed):
    """The GEMV benchmark shapes: N=11008, K=4096, M in {1,4,16}; resident image and
    plain [N, K] weights."""
    print(f"gemv M={M} packed={packed}", flush=True)
    N, K = 11008, 4096
    g = torch.Generator().manual_seed(M)
    x = torch.randn(M, K, generator=g).half()
    W = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sc = (torch.rand(N, generator=g) * 0.019 + 0.001).half()
    Wd = W.to(dev)
    Wd = ops.prepack_w8a16(Wd) if packed else Wd
    y = ops.gemv_w8a16(x.to(dev), Wd, sc.to(dev)).cpu()
    ref = orc.f16_bits_to_f32(orc.gemv_w8a16(host_bits(x, "f16"), W.numpy(),
                                             host_bits(sc, "f16")))
    np.testing.assert_allclose(y.float().numpy(), ref, rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("M", [1, 4, 16])
@pytest.mark.parametrize("packed", [True, False])
def test_gemv_empty_k(dev, M, packed):
    """K == 0: every dot product is the empty sum, so y = f16(0.0 * scale)
    bit for bit (+0, and -0 where the scale is negative), whatever y held
    before; x and W may be null.  Called through the C ABI, since a torch
    tensor with no columns has no 8-aligned row stride."""
    import hxm
    N = 40
    sc = torch.linspace(-1.5, 1.5, N).half()
    sc[7] = -0.0
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
    st = hxm.lib.hxm_gemv_w8a16(None, 8, None, 16, hxm.W_PACKED if packed else hxm.W_NK,
                                sc.to(dev).data_ptr(), y.data_ptr(), N, M, N, 0,
                                torch.cuda.current_stream().cuda_stream)
    hxm.check(st, "hxm_gemv_w8a16")
    want = (torch.zeros(M, N) * sc.float()).half()
    assert np.array_equal(host_bits(y.cpu(), "f16"), host_bits(want, "f16"))
    assert (host_bits(want, "f16")[:, :20] == 0x8000).all()   # the negative scales give -0


@pytest.mark.parametrize("M,N,K", [(3, 100, 272), (33, 64, 512), (1, 17, 16), (16, 48, 256),
                                   (5, 40, 2064), (20, 31, 4160),
                                   # one GPU's share of an 8-way column split of config 3
                                   (1, 1376, 4096), (4, 1376, 4096), (16, 1376, 4096),
                                   # 322 channel groups: the pipelined kernels (three groups
                                   # per workgroup at M > 4, the last set partial), K of 33 slabs
                                   (3, 5140, 2064), (9, 5140, 2064)])
@pytest.mark.parametrize("packed", [True, False])
def test_gemv_ragged(dev, M, N, K, packed):
    g = torch.Generator().manual_seed(M * N + K)
    x = torch.randn(M, K, generator=g).half()
    W = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sc = (torch.rand(N, generator=g) * 0.019 + 0.001).half()
    Wd = W.to(dev)
    Wd = ops.prepack_w8a16(Wd) if packed else Wd
    y = ops.gemv_w8a16(x.to(dev), Wd, sc.to(dev)).cpu()
    ref = orc.f16_bits_to_f32(orc.gemv_w8a16(host_bits(x, "f16"), W.numpy(),
                                             host_bits(sc, "f16")))
    np.testing.assert_allclose(y.float().numpy(), ref, rtol=1e-2, atol=1e-3)


def test_w8a16_image_layout(dev):
    """The image is a permutation of W in offset binary (byte = w ^ 0x80)
    with zero-weight padding (0x80): block (g, s), lane l holds
    W[16g + l%16][64s + 16(l//16) ... +16] ^ 0x80."""
    N, K = 37, 208
    W = torch.randint(-127, 128, (N, K), dtype=torch.int8)
    img = ops.prepack_w8a16(W.to(dev)).cpu().numpy()
    ng, ns = (N + 15) // 16, (K + 63) // 64
    assert img.size == ng * ns * 1024
    exp = np.full((ng, ns, 64, 16), -128, dtype=np.int8)   # 0x80: a zero weight
    Wn = (W.numpy().view(np.uint8) ^ 0x80).view(np.int8)
    for gi in range(ng):
        for si in range(ns):
            for lane in range(64):
                n, k = gi * 16 + lane % 16, si * 64 + (lane // 16) * 16
                if n < N and k < K:
                    exp[gi, si, lane] = Wn[n, k:k + 16]
    assert np.array_equal(img.reshape(ng, ns, 64, 16), exp)


@pytest.mark.parametrize("packed", [True, False])
def test_gemv_golden_and_exact_small_ints(dev, golden, packed):
    gd = golden("gemv_w8a16")
    Wg = torch.from_numpy(gd["W"]).to(dev)
    y = ops.gemv_w8a16(torch.from_numpy(gd["x_bits"].view(np.float16)).to(dev),
                       ops.prepack_w8a16(Wg) if packed else Wg,
                       torch.from_numpy(gd["scale_bits"].view(np.float16)).to(dev))
    np.testing.assert_allclose(y.float().cpu().numpy(), gd["y_f64"], rtol=1e-2, atol=1e-3)
    # every int8 value -128..127 through the exact f16 conversion: x = e_k
    K = 256
    W = torch.arange(-128, 128, dtype=torch.int16).to(torch.int8).repeat(2, 1)  # [2, 256]
    x = torch.eye(K)[:16].half()                                                # picks k=0..15
    Wd = ops.prepack_w8a16(W.to(dev)) if packed else W.to(dev)
    y = ops.gemv_w8a16(x.to(dev), Wd, torch.ones(2).half().to(dev)).cpu()
    assert torch.equal(y.float(), W[:, :16].t().float())
    # M = 1 and 4 through the same rows (the one-chunk and pipelined kernels)
    for m in (1, 4):
        y = ops.gemv_w8a16(x[:m].to(dev), Wd, torch.ones(2).half().to(dev)).cpu()
        assert torch.equal(y.float(), W[:, :m].t().float())


def test_gemv_kernels_agree_bit_for_bit(dev):
    """Every GEMV kernel sums a row's products in one grouping: wave w of the
    8 takes the slabs w, w + 8, ..., two MFMAs per slab in K order, and the
    waves' partials are added in wave order.  So row 0 comes out the same
    bits from the one-chunk kernel (M = 1, packed and plain weights) and the
    pipelined kernels (M = 4 with one channel group per workgroup, M = 16
    with three), at the benchmark's N = 11008, K = 4096."""
    g = torch.Generator().manual_seed(17)
    N, K = 11008, 4096
    W = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
    sc = (torch.rand(N, generator=g) * 0.019 + 0.001).half().to(dev)
    x = torch.randn(16, K, generator=g).half().to(dev)
    Wp = ops.prepack_w8a16(W)
    y1 = ops.gemv_w8a16(x[:1], Wp, sc)
    assert torch.equal(ops.gemv_w8a16(x[:1], W, sc), y1)           # plain layout
    for M in (4, 16):
        assert torch.equal(ops.gemv_w8a16(x[:M], Wp, sc)[:1], y1), f"M={M}"


@pytest.mark.parametrize("r", range(8))
@pytest.mark.parametrize("M", [1, 16])
def test_gemv_group_order_covers_every_channel(dev, M, r):
    """The XCD-contiguous order of the channel groups (M = 1, and M > 4 with
    three groups per workgroup) maps the grid's G workgroups onto its G
    blocks one to one for every G mod 8 = r: every channel of y is written
    once, with its own row's dot product (y starts as NaN), packed and plain
    weights."""
    K = 128
    blocks = 8 * 41 + r                       # grid size: M = 1 one group each, M = 16 three
    N = 16 * blocks * (3 if M > 4 else 1) - 5  # the last group partial
    print(f"gemv order M={M} N={N} grid={blocks}", flush=True)
    g = torch.Generator().manual_seed(100 + 8 * M + r)
    x = torch.randn(M, K, generator=g).half()
    W = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sc = (torch.rand(N, generator=g) * 0.019 + 0.001).half()
    ref = orc.f16_bits_to_f32(orc.gemv_w8a16(host_bits(x, "f16"), W.numpy(),
                                             host_bits(sc, "f16")))
    Wd = W.to(dev)
    for Wx in (ops.prepack_w8a16(Wd), Wd):
        y = torch.full((M, N), float("nan"), dtype=torch.float16, device=dev)
        ops.gemv_w8a16(x.to(dev), Wx, sc.to(dev), out=y)
        yc = y.float().cpu().numpy()
        assert np.isfinite(yc).all()
        np.testing.assert_allclose(yc, ref, rtol=1e-2, atol=1e-3)
