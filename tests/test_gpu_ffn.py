"""GPU parity of the SwiGLU FFN block (tokens 2048, hidden 4096, intermediate 11008) against the CPU
oracle: the large-M W8A16 GEMM, the gate/up image, the fused gate/up GEMM
with SiLU * mul, and the whole block RMSNorm -> gate/up -> down.

fp16 outputs are held to rtol 1e-2 / atol 1e-3 (fp32 accumulation in MFMA
order vs the oracle's increasing-k fp32 sums); a small-integer case makes
every sum exact, so the W8A16 GEMM must match bit for bit.  At the benchmark
size (tokens 2048, hidden 4096, intermediate 11008) the oracle runs on a row
sample of the same inputs.  The block is checked stage by stage (each stage
fed the GPU's own input to it) and end to end, all at that tolerance."""
import numpy as np
import pytest
import torch

import hxm.ops as ops
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOL = dict(rtol=1e-2, atol=1e-3)


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def f32(b):
    return orc.f16_bits_to_f32(b)


def operands(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).half()
    W = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s = (torch.rand(N, generator=g) * 0.019 + 0.001).half().float()  # fp16-valued fp32
    return x, W, s


@pytest.mark.parametrize("M,N,K", [(256, 256, 512), (300, 260, 1024), (33, 96, 64),
                                   (1, 40, 16), (512, 4096, 1024)])
def test_gemm_w8a16(dev, M, N, K):
    print(f"gemm_w8a16 M={M} N={N} K={K}", flush=True)
    x, W, s = operands(M, N, K, M + N + K)
    y = ops.gemm_w8a16(x.to(dev), W.to(dev), s.to(dev))
    ref = orc.gemm_w8a16(bits(x), W.numpy(), s.numpy())
    np.testing.assert_allclose(y.float().cpu().numpy(), f32(ref), **TOL)


@pytest.mark.parametrize("K", [640, 656])  # K bytes a multiple of every stage depth / not
@pytest.mark.parametrize("cfg", ops.w8a16_configs(), ids=repr)
def test_gemm_w8a16_every_config(dev, cfg, K):
    print(f"gemm_w8a16 config {cfg} K={K}", flush=True)
    M, N = 300, 520
    x, W, s = operands(M, N, K, 7)
    xd, Wd, sd = x.to(dev), W.to(dev), s.to(dev)
    y = ops.gemm_w8a16(xd, Wd, sd, config=cfg)
    ref = orc.gemm_w8a16(bits(x), W.numpy(), s.numpy())
    np.testing.assert_allclose(y.float().cpu().numpy(), f32(ref), **TOL)
    # every tile groups K into the same k-steps: bit-identical to the default
    assert torch.equal(y, ops.gemm_w8a16(xd, Wd, sd))


def test_gemm_w8a16_small_integers_bit_exact(dev):
    """|x| <= 4, |W| <= 8, K = 256: every product and partial sum is an
    integer below 2^24, so every summation order gives the same fp32 sum and
    the f16 result must equal the oracle's bit for bit."""
    g = torch.Generator().manual_seed(3)
    M, N, K = 128, 256, 256
    x = torch.randint(-4, 5, (M, K), generator=g).half()
    W = torch.randint(-8, 9, (N, K), generator=g, dtype=torch.int8)
    s = torch.full((N,), 0.125)
    y = ops.gemm_w8a16(x.to(dev), W.to(dev), s.to(dev))
    assert np.array_equal(bits(y), orc.gemm_w8a16(bits(x), W.numpy(), s.numpy()))


def test_gemm_w8a16_strided_and_refusals(dev):
    x, W, s = operands(64, 128, 256, 11)
    xb = torch.zeros(64, 264, dtype=torch.float16, device=dev)
    xb[:, :256] = x.to(dev)
    Wb = torch.zeros(128, 272, dtype=torch.int8, device=dev)
    Wb[:, :256] = W.to(dev)
    yb = torch.full((64, 136), 7.0, dtype=torch.float16, device=dev)
    ops.gemm_w8a16(xb[:, :256], Wb[:, :256], s.to(dev), out=yb[:, :128])
    ref = orc.gemm_w8a16(bits(x), W.numpy(), s.numpy())
    np.testing.assert_allclose(yb[:, :128].float().cpu().numpy(), f32(ref), **TOL)
    assert (yb[:, 128:] == 7).all()                      # outside the view untouched
    with pytest.raises(Exception, match="tile-alignment"):
        ops.gemm_w8a16(x[:, :24].contiguous().to(dev), W[:, :24].contiguous().to(dev),
                       s.to(dev))


@pytest.mark.parametrize("M,N,K", [(256, 256, 512), (300, 260, 1024), (33, 96, 64),
                                   (1, 40, 16), (512, 4096, 1024)])
def test_gemm_w8a16_residual(dev, M, N, K):
    print(f"gemm_w8a16_residual M={M} N={N} K={K}", flush=True)
    x, W, s = operands(M, N, K, M + N + K + 1)
    r = (4 * torch.randn(M, N, generator=torch.Generator().manual_seed(M + N))).half()
    y = ops.gemm_w8a16(x.to(dev), W.to(dev), s.to(dev), residual=r.to(dev))
    ref = orc.gemm_w8a16_residual(bits(x), W.numpy(), s.numpy(), bits(r))
    np.testing.assert_allclose(y.float().cpu().numpy(), f32(ref), **TOL)


@pytest.mark.parametrize("cfg", ops.w8a16_configs(), ids=repr)
def test_gemm_w8a16_residual_every_config(dev, cfg):
    """Full tiles take the pipelined epilogue, edge tiles the general one."""
    print(f"gemm_w8a16_residual config {cfg}", flush=True)
    M, N, K = 520, 544, 640
    x, W, s = operands(M, N, K, 9)
    r = torch.randn(M, N, generator=torch.Generator().manual_seed(10)).half()
    y = ops.gemm_w8a16(x.to(dev), W.to(dev), s.to(dev), residual=r.to(dev), config=cfg)
    ref = orc.gemm_w8a16_residual(bits(x), W.numpy(), s.numpy(), bits(r))
    np.testing.assert_allclose(y.float().cpu().numpy(), f32(ref), **TOL)


def test_gemm_w8a16_residual_bit_exact_and_in_place(dev):
    """Small integers make every sum exact, so the result must equal the
    oracle bit for bit; the in-place form (out is the residual) gives the
    same bits; the KAT p = 1 + 2^-20, r = 2048 shows the fp32 sum is rounded
    before the f16 conversion (2048, not the single-rounding 2050)."""
    g = torch.Generator().manual_seed(12)
    M, N, K = 512, 512, 256
    x = torch.randint(-4, 5, (M, K), generator=g).half()
    W = torch.randint(-8, 9, (N, K), generator=g, dtype=torch.int8)
    s = torch.full((N,), 0.125)
    r = torch.randint(-64, 65, (M, N), generator=g).half()
    xd, Wd, sd = x.to(dev), W.to(dev), s.to(dev)
    y = ops.gemm_w8a16(xd, Wd, sd, residual=r.to(dev))
    ref = orc.gemm_w8a16_residual(bits(x), W.numpy(), s.numpy(), bits(r))
    assert np.array_equal(bits(y), ref)
    yi = r.to(dev)
    ops.gemm_w8a16(xd, Wd, sd, out=yi, residual=yi)
    assert np.array_equal(bits(yi), ref)
    xk = torch.zeros(256, 256).half()
    xk[:, 0] = 1
    Wk = torch.zeros(256, 256, dtype=torch.int8)
    Wk[:, 0] = 1
    sk = torch.full((256,), 1.0 + 2 ** -20)
    rk = torch.full((256, 256), 2048.0).half()
    yk = ops.gemm_w8a16(xk.to(dev), Wk.to(dev), sk.to(dev), residual=rk.to(dev))
    assert (yk.float().cpu() == 2048.0).all()


def test_gemm_w8a16_residual_refusals(dev):
    x, W, s = operands(64, 128, 256, 13)
    xd, Wd, sd = x.to(dev), W.to(dev), s.to(dev)
    buf = torch.zeros(66, 128, dtype=torch.float16, device=dev)
    with pytest.raises(Exception, match="overlaps"):
        ops.gemm_w8a16(xd, Wd, sd, out=buf[1:65], residual=buf[0:64])
    import hxm
    L = hxm.lib
    y = torch.empty(64, 128, dtype=torch.float16, device=dev)
    st = L.hxm_gemm_w8a16_residual(xd.data_ptr(), 256, Wd.data_ptr(), 256, sd.data_ptr(),
                                   buf.data_ptr(), 100, y.data_ptr(), 128, 64, 128, 256, None,
                                   None)
    assert st != 0 and "ldr" in hxm.last_error()


def test_swiglu_pack_layout(dev):
    """Image rows [128c, 128c+64) = gate channels [64c, 64c+64), the next 64
    rows the same up channels; channels >= I zero rows with zero scale.
    Weights are stored in offset binary: byte = w ^ 0x80 (zero -> 0x80)."""
    I, K = 100, 48
    g = torch.Generator().manual_seed(5)
    Wg = torch.randint(-127, 128, (I, K), generator=g, dtype=torch.int8)
    Wu = torch.randint(-127, 128, (I, K), generator=g, dtype=torch.int8)
    sg, su = torch.rand(I, generator=g), torch.rand(I, generator=g)
    Wgu, sgu = ops.swiglu_pack(Wg.to(dev), Wu.to(dev), sg.to(dev), su.to(dev))
    rows = 128 * ((I + 63) // 64)
    assert tuple(Wgu.shape) == (rows, K) and sgu.numel() == rows
    expW = np.full((rows, K), -128, np.int8)   # 0x80: a zero weight
    exps = np.zeros(rows, np.float32)
    for r in range(rows):
        ch = (r // 128) * 64 + r % 64
        if ch < I:
            src, ss = (Wu, su) if r % 128 >= 64 else (Wg, sg)
            expW[r] = (src[ch].numpy().view(np.uint8) ^ 0x80).view(np.int8)
            exps[r] = ss[ch].item()
    assert np.array_equal(Wgu.cpu().numpy(), expW)
    assert np.array_equal(sgu.cpu().numpy(), exps)


def swiglu_operands(M, I, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K, generator=g).half()
    Wg = torch.randint(-127, 128, (I, K), generator=g, dtype=torch.int8)
    Wu = torch.randint(-127, 128, (I, K), generator=g, dtype=torch.int8)
    # scales ~ 1/sqrt(K * 127^2 / 3) keep g and u near unit size
    sc = 1.0 / np.sqrt(K * 127.0 ** 2 / 3.0)
    sg = ((torch.rand(I, generator=g) + 0.5) * sc).half().float()
    su = ((torch.rand(I, generator=g) + 0.5) * sc).half().float()
    return x, Wg, Wu, sg, su


@pytest.mark.parametrize("M,I,K", [(256, 128, 512), (300, 100, 1024), (17, 64, 64),
                                   (512, 704, 1024),
                                   # K not a multiple of the 64-wide stage: the last stage's
                                   # zero-filled K (zero x against offset-binary zero bytes)
                                   (40, 96, 656), (9, 64, 48)])
def test_gemm_w8a16_swiglu(dev, M, I, K):
    print(f"swiglu M={M} I={I} K={K}", flush=True)
    x, Wg, Wu, sg, su = swiglu_operands(M, I, K, M + I)
    Wgu, sgu = ops.swiglu_pack(Wg.to(dev), Wu.to(dev), sg.to(dev), su.to(dev))
    h = ops.gemm_w8a16_swiglu(x.to(dev), Wgu, sgu, I)
    ref = orc.swiglu_gateup(bits(x), Wg.numpy(), Wu.numpy(), sg.numpy(), su.numpy())
    np.testing.assert_allclose(h.float().cpu().numpy(), f32(ref), **TOL)


@pytest.mark.parametrize("cfg", ops.w8a16_configs(swiglu=True), ids=repr)
def test_gemm_w8a16_swiglu_every_config(dev, cfg):
    print(f"swiglu config {cfg}", flush=True)
    M, I, K = 300, 200, 512
    x, Wg, Wu, sg, su = swiglu_operands(M, I, K, 9)
    Wgu, sgu = ops.swiglu_pack(Wg.to(dev), Wu.to(dev), sg.to(dev), su.to(dev))
    h = ops.gemm_w8a16_swiglu(x.to(dev), Wgu, sgu, I, config=cfg)
    ref = orc.swiglu_gateup(bits(x), Wg.numpy(), Wu.numpy(), sg.numpy(), su.numpy())
    np.testing.assert_allclose(h.float().cpu().numpy(), f32(ref), **TOL)


def ffn_operands(T, H, I, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).half()
    gamma = (1 + 0.1 * torch.randn(H, generator=g)).half()
    sc_h = 1.0 / np.sqrt(H * 127.0 ** 2 / 3.0)
    sc_i = 1.0 / np.sqrt(I * 127.0 ** 2 / 3.0)
    Wg = torch.randint(-127, 128, (I, H), generator=g, dtype=torch.int8)
    Wu = torch.randint(-127, 128, (I, H), generator=g, dtype=torch.int8)
    Wd = torch.randint(-127, 128, (H, I), generator=g, dtype=torch.int8)
    sg = ((torch.rand(I, generator=g) + 0.5) * sc_h).half().float()
    su = ((torch.rand(I, generator=g) + 0.5) * sc_h).half().float()
    sd = ((torch.rand(H, generator=g) + 0.5) * sc_i).half().float()
    return x, gamma, Wg, Wu, Wd, sg, su, sd


def run_ffn_stages(dev, x, gamma, Wg, Wu, Wd, sg, su, sd, residual=False):
    """The block on the GPU stage by stage -- RMSNorm, fused gate/up with
    SiLU * mul, down (with the residual in its epilogue) -- and, separately,
    through swiglu_ffn, which must launch exactly that composition (same
    bits).  Returns the f16 tensors xn, h, y on the host."""
    T, H = x.shape
    I = Wg.shape[0]
    Wgu, sgu = ops.swiglu_pack(Wg.to(dev), Wu.to(dev), sg.to(dev), su.to(dev))
    xd, gd, Wdd, sdd = x.to(dev), gamma.to(dev), Wd.to(dev), sd.to(dev)
    xn = ops.rms_norm(xd, (H,), gd, eps=1e-6)
    h = ops.gemm_w8a16_swiglu(xn, Wgu, sgu, I)
    y = ops.gemm_w8a16(h, Wdd, sdd, residual=xd if residual else None)
    y_block = ops.swiglu_ffn(xd, gd, Wgu, sgu, Wdd, sdd, I, residual=residual)
    assert torch.equal(y, y_block), "swiglu_ffn differs from its own stages"
    return xn.cpu(), h.cpu(), y.cpu()


def check_ffn_stages(ops_, xn, h, y, rows, residual=False):
    """Each stage against the oracle fed the GPU's own input to that stage,
    at rtol 1e-2 / atol 1e-3:
      1. xn = RMSNorm(x) against orc.rmsnorm_rows(x);
      2. h against orc.swiglu_gateup(GPU xn);
      3. y against the oracle's down projection of the GPU's h (with x as the
         residual when the block adds it);
    then the whole block against the oracle's own chain (x -> xn_o -> h_o ->
    y_o) at the same tolerance.  Stage by stage, a difference cannot hide
    behind a looser end-to-end bound: a one-ulp difference of an f16 h
    element between the two chains moves y by up to |Wd| * sd * ulp(h),
    which rtol does not absorb where y is near 0, and the stage checks show
    which stage such a difference would come from."""
    x, gamma, Wg, Wu, Wd, sg, su, sd = ops_
    xb = bits(x)[rows]
    xn_b, h_b, y_b = bits(xn)[rows], bits(h)[rows], bits(y)[rows]
    xn_ref = orc.rmsnorm_rows(xb, bits(gamma), 1e-6, "f16")
    np.testing.assert_allclose(f32(xn_b), f32(xn_ref), **TOL, err_msg="RMSNorm stage")
    h_ref = orc.swiglu_gateup(xn_b, Wg.numpy(), Wu.numpy(), sg.numpy(), su.numpy())
    np.testing.assert_allclose(f32(h_b), f32(h_ref), **TOL, err_msg="gate/up stage")
    if residual:
        y_ref = orc.gemm_w8a16_residual(h_b, Wd.numpy(), sd.numpy(), xb)
    else:
        y_ref = orc.gemm_w8a16(h_b, Wd.numpy(), sd.numpy())
    np.testing.assert_allclose(f32(y_b), f32(y_ref), **TOL, err_msg="down stage")
    y_o = orc.swiglu_ffn(xb, bits(gamma), Wg.numpy(), Wu.numpy(), sg.numpy(), su.numpy(),
                         Wd.numpy(), sd.numpy(), residual=residual)
    np.testing.assert_allclose(f32(y_b), f32(y_o), **TOL, err_msg="block end to end")


def test_swiglu_ffn_block(dev):
    T, H, I = 256, 512, 704
    ops_ = ffn_operands(T, H, I, 21)
    xn, h, y = run_ffn_stages(dev, *ops_)
    check_ffn_stages(ops_, xn, h, y, np.arange(T))


def test_swiglu_ffn_block_with_residual(dev):
    """x + FFN(x): the residual is added in the down GEMM's epilogue."""
    T, H, I = 256, 512, 704
    ops_ = ffn_operands(T, H, I, 22)
    xn, h, y = run_ffn_stages(dev, *ops_, residual=True)
    check_ffn_stages(ops_, xn, h, y, np.arange(T), residual=True)


SAMPLE_ROWS = np.array([0, 1, 255, 256, 511, 777, 1023, 1024, 1290, 1535, 1536, 1800, 2000,
                        2045, 2046, 2047])


def test_swiglu_ffn_baseline_size_stages(dev):
    """tokens 2048, hidden 4096, intermediate 11008: the whole block on the
    GPU, every stage checked against the oracle on 16 sampled token rows
    (rows are independent in every stage) at rtol 1e-2 / atol 1e-3, then the
    block end to end at the same tolerance."""
    T, H, I = 2048, 4096, 11008
    ops_ = ffn_operands(T, H, I, 31)
    xn, h, y = run_ffn_stages(dev, *ops_)
    assert torch.isfinite(y.float()).all()
    check_ffn_stages(ops_, xn, h, y, SAMPLE_ROWS)


def test_swiglu_gateup_baseline_size_alone(dev):
    """The gate/up + SiLU * mul stage alone at its benchmark size
    (2048 x 11008 x 4096, x ~ N(0, 1)) against the oracle on 16 sampled rows."""
    T, H, I = 2048, 4096, 11008
    x, Wg, Wu, sg, su = swiglu_operands(T, I, H, 33)
    Wgu, sgu = ops.swiglu_pack(Wg.to(dev), Wu.to(dev), sg.to(dev), su.to(dev))
    h = ops.gemm_w8a16_swiglu(x.to(dev), Wgu, sgu, I).cpu()
    ref = orc.swiglu_gateup(bits(x)[SAMPLE_ROWS], Wg.numpy(), Wu.numpy(), sg.numpy(),
                            su.numpy())
    np.testing.assert_allclose(f32(bits(h)[SAMPLE_ROWS]), f32(ref), **TOL)


def test_swiglu_ffn_tp8_shard_stages(dev):
    """One GPU's share of an 8-way tensor-parallel block: intermediate
    11008 / 8 = 1376 channels (not a multiple of the image's 64-channel
    blocks: the last block is half padding), gate/up column-parallel, down
    row-parallel over the same slice, so y is this GPU's partial sum of the
    block's output.  Stage checks on 16 sampled token rows."""
    T, H, I = 2048, 4096, 1376
    ops_ = ffn_operands(T, H, I, 37)
    xn, h, y = run_ffn_stages(dev, *ops_)
    assert torch.isfinite(y.float()).all()
    check_ffn_stages(ops_, xn, h, y, SAMPLE_ROWS)


def test_tune_w8a16_caches_a_verified_winner(dev):
    import hxm
    hxm.lib.hxm_tune_cache_clear()
    M, N, K = 512, 1024, 512
    x, W, s = operands(M, N, K, 41)
    xd, Wd, sd = x.to(dev), W.to(dev), s.to(dev)
    out = torch.empty(M, N, dtype=torch.float16, device=dev)
    best, rep = ops.tune_w8a16(xd, Wd, sd, out, reps=3)
    assert rep["kind"] == "hxm-search-champion" and rep["champion"] is not None
    assert any(c["verified"] for c in rep["configs"])
    y = ops.gemm_w8a16(xd, Wd, sd)                       # now runs the cached winner
    np.testing.assert_allclose(y.float().cpu().numpy(),
                               f32(orc.gemm_w8a16(bits(x), W.numpy(), s.numpy())), **TOL)
    I = 256
    xs, Wg, Wu, sg, su = swiglu_operands(M, I, K, 43)
    Wgu, sgu = ops.swiglu_pack(Wg.to(dev), Wu.to(dev), sg.to(dev), su.to(dev))
    h = torch.empty(M, I, dtype=torch.float16, device=dev)
    best, rep = ops.tune_w8a16(xs.to(dev), Wgu, sgu, h, swiglu=True, reps=3)
    assert rep["champion"] is not None and best.bn // best.waves_n == 128
    hxm.lib.hxm_tune_cache_clear()
