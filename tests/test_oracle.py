"""Pins the CPU oracle (oracle/oracle.c) before anything is compared with it.

Every check below uses an implementation independent of oracle.c: numpy's
IEEE casts and int64 matmul, torch's float64 softmax / rms_norm / layer_norm
/ matmul (the reference tests' own oracles), closed forms (identity,
small-integer exactness, shift/scale invariance) and the committed golden
fixtures.  Each would fail on a plausible oracle mistake: a wrong rounding
mode, a dropped eps, a transposed operand, a max not subtracted, a biased vs
unbiased variance, a missing scale.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc


def h(a):
    return np.asarray(a, dtype=np.float16).view(np.uint16)


# ---- conversions -----------------------------------------------------------

def test_f16_to_f32_all_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.f16_bits_to_f32(bits)
    exp = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), exp[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rne():
    rng = np.random.default_rng(1)
    r = [rng.standard_normal(1 << 20).astype(np.float32) * s for s in (1e-6, 1, 3e4)]
    # every f16 value, every halfway point between neighbours, +-1 f32 ulp
    hv = np.arange(0, 0x7c00, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    mid = ((hv[:-1].astype(np.float64) + hv[1:].astype(np.float64)) / 2).astype(np.float32)
    up = np.nextafter(mid, np.float32(np.inf))
    dn = np.nextafter(mid, np.float32(0))
    edge = np.array([65504, 65519.99, 65520, 65536, 1e30, np.inf, -np.inf, 0.0, -0.0,
                     2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 2.0 ** -26, 1e-45],
                    dtype=np.float32)
    x = np.concatenate(r + [hv, mid, up, dn, edge, -mid, -edge])
    got = orc.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        exp = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, exp)
    nanbits = orc.f32_to_f16_bits(np.array([np.nan], dtype=np.float32))
    assert np.isnan(nanbits.view(np.float16)).all()


def test_f32_to_bf16_matches_torch_rne():
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(1 << 20).astype(np.float32) * s
                        for s in (1e-30, 1, 1e30)])
    got = orc.f32_to_bf16_bits(x)
    exp = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, exp)


# ---- int8 GEMM ---------------------------------------------------------------

@pytest.mark.parametrize("M,N,K", [(1, 1, 16), (67, 45, 96), (33, 130, 272), (128, 64, 1024)])
@pytest.mark.parametrize("b_nk", [False, True])
def test_gemm_i8_matches_numpy_int64(M, N, K, b_nk):
    rng = np.random.default_rng(M * 1000 + N + K)
    A = rng.integers(-128, 128, size=(M, K)).astype(np.int8)
    B = rng.integers(-128, 128, size=(K, N)).astype(np.int8)
    exp = (A.astype(np.int64) @ B.astype(np.int64)).astype(np.int32)
    got = orc.gemm_i8(A, np.ascontiguousarray(B.T) if b_nk else B, b_nk=b_nk)
    assert np.array_equal(got, exp)


def test_gemm_i8_identity_and_extremes():
    K = 64
    I8 = np.eye(K, dtype=np.int8)
    B = np.random.default_rng(3).integers(-128, 128, size=(K, 40)).astype(np.int8)
    assert np.array_equal(orc.gemm_i8(I8, B), B.astype(np.int32))
    A = np.random.default_rng(4).integers(-128, 128, size=(40, K)).astype(np.int8)
    assert np.array_equal(orc.gemm_i8(A, I8), A.astype(np.int32))
    # all -128: every product is +16384, the largest magnitude
    M = np.full((3, 4096), -128, dtype=np.int8)
    assert (orc.gemm_i8(M, np.full((4096, 2), -128, dtype=np.int8)) == 4096 * 16384).all()


def test_gemm_i8_accumulate_wraps_like_int32():
    A = np.full((2, 16), 127, dtype=np.int8)
    B = np.full((16, 2), 127, dtype=np.int8)
    C0 = np.full((2, 2), 2 ** 31 - 10, dtype=np.int64).astype(np.int32)
    got = orc.gemm_i8(A, B, C=C0, accumulate=True)
    exp = ((C0.astype(np.int64) + 16 * 127 * 127 + 2 ** 31) % 2 ** 32 - 2 ** 31).astype(np.int32)
    assert np.array_equal(got, exp)


def test_gemm_i8_brute_force_tiny():
    rng = np.random.default_rng(5)
    A = rng.integers(-128, 128, size=(3, 16)).astype(np.int8)
    B = rng.integers(-128, 128, size=(16, 5)).astype(np.int8)
    got = orc.gemm_i8(A, B)
    for m in range(3):
        for n in range(5):
            assert got[m, n] == sum(int(A[m, k]) * int(B[k, n]) for k in range(16))


def test_gemm_i8_and_dequant_golden(golden):
    g = golden("gemm_i8")
    C = orc.gemm_i8(g["A"], g["B"])
    assert np.array_equal(C, g["C"])
    d = orc.dequant_f16(C, g["row_scale"], g["col_scale"])
    assert np.array_equal(d, g["dequant_f16_bits"])


def test_dequant_matches_numpy_spelling():
    rng = np.random.default_rng(6)
    acc = rng.integers(-66_000_000, 66_000_000, size=(512, 512)).astype(np.int32)
    rs = rng.uniform(0.001, 0.02, size=512).astype(np.float32)
    cs = rng.uniform(0.001, 0.02, size=512).astype(np.float32)
    exp = ((acc.astype(np.float32) * rs[:, None]) * cs[None, :]).astype(np.float16).view(np.uint16)
    assert np.array_equal(orc.dequant_f16(acc, rs, cs), exp)
    # The spelling is observable at this size: re-associating the scales or
    # computing in float64 changes some f16 results, so a wrong order fails.
    other = (acc.astype(np.float32) * (rs[:, None] * cs[None, :])).astype(np.float16)
    wide = (acc.astype(np.float64) * rs[:, None] * cs[None, :]).astype(np.float16)
    assert not np.array_equal(other.view(np.uint16), exp)
    assert not np.array_equal(wide.view(np.uint16), exp)


# ---- f16/bf16 matmul -----------------------------------------------------------

def test_matmul_golden(golden):
    g = golden("matmul_f16")
    got = orc.f16_bits_to_f32(orc.matmul(g["A_bits"], g["B_bits"]))
    np.testing.assert_allclose(got, g["C_f64"], rtol=1e-2, atol=1e-3)
    # small integers: every partial sum exact -> bit-exact result
    gi = orc.matmul(g["Ai_bits"], g["Bi_bits"])
    assert np.array_equal(gi, g["Ci_bits"])


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_matmul_vs_torch_f64(dt):
    g = torch.Generator().manual_seed(7)
    tdt = torch.float16 if dt == "f16" else torch.bfloat16
    a = (torch.rand(40, 96, generator=g) * 2 - 1).to(tdt)
    b = (torch.rand(96, 56, generator=g) * 2 - 1).to(tdt)
    bits = lambda t: t.view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    out = orc.matmul(bits(a), bits(b), ab_dtype=dt, c_dtype="f32")
    exp = (a.double() @ b.double()).numpy()
    np.testing.assert_allclose(out, exp, rtol=1e-5, atol=1e-5)
    # transposed operand layout gives the same numbers
    out_nk = orc.matmul(bits(a), bits(b.t().contiguous()), ab_dtype=dt, c_dtype="f32", b_nk=True)
    assert np.array_equal(out, out_nk)


def test_matmul_accumulate_adds_prior_c():
    a = h(np.ones((4, 16)))
    b = h(np.ones((16, 4)))
    C0 = np.full((4, 4), 0.5, dtype=np.float32)
    out = orc.matmul(a, b, c_dtype="f32", C=C0, accumulate=True)
    assert (out == 16.5).all()


# ---- W8A16 GEMV -----------------------------------------------------------------

def test_gemv_golden(golden):
    g = golden("gemv_w8a16")
    y = orc.f16_bits_to_f32(orc.gemv_w8a16(g["x_bits"], g["W"], g["scale_bits"]))
    np.testing.assert_allclose(y, g["y_f64"], rtol=1e-2, atol=1e-3)


def test_gemv_scale_is_per_output_channel():
    x = h(np.ones((1, 32)))
    W = np.ones((3, 32), dtype=np.int8)
    sc = h([1.0, 2.0, 0.5])
    y = orc.f16_bits_to_f32(orc.gemv_w8a16(x, W, sc))
    assert np.array_equal(y, np.array([[32.0, 64.0, 16.0]], dtype=np.float32))


def test_gemm_w8a16_vs_numpy_f64_and_small_integer_kat():
    rng = np.random.default_rng(4)
    x = h(rng.standard_normal((9, 80)))
    W = rng.integers(-127, 128, (13, 80)).astype(np.int8)
    sc = rng.uniform(0.001, 0.02, 13).astype(np.float32)
    y = orc.f16_bits_to_f32(orc.gemm_w8a16(x, W, sc))
    ref = (orc.f16_bits_to_f32(x).astype(np.float64) @ W.T.astype(np.float64)) * sc
    np.testing.assert_allclose(y, ref, rtol=2 ** -10, atol=1e-6)   # within ~1 f16 ulp
    # small integers: exact sums -> bit-exact against the float64 product
    xs = h(rng.integers(-4, 5, (6, 256)))
    Ws = rng.integers(-8, 9, (7, 256)).astype(np.int8)
    s8 = np.full(7, 0.125, np.float32)
    exact = (orc.f16_bits_to_f32(xs).astype(np.float64) @ Ws.T.astype(np.float64)) * 0.125
    assert np.array_equal(orc.f16_bits_to_f32(orc.gemm_w8a16(xs, Ws, s8)), exact)
    # the scale belongs to the output channel (a transposed scale fails this)
    y3 = orc.f16_bits_to_f32(orc.gemm_w8a16(h(np.ones((1, 32))), np.ones((3, 32), np.int8),
                                            np.array([1.0, 2.0, 0.5], np.float32)))
    assert np.array_equal(y3, np.array([[32.0, 64.0, 16.0]], np.float32))


def test_gemm_w8a16_residual_pins():
    rng = np.random.default_rng(8)
    x = h(rng.standard_normal((9, 80)))
    W = rng.integers(-127, 128, (13, 80)).astype(np.int8)
    sc = rng.uniform(0.001, 0.02, 13).astype(np.float32)
    r = h(4 * rng.standard_normal((9, 13)))
    y = orc.f16_bits_to_f32(orc.gemm_w8a16_residual(x, W, sc, r))
    p = (orc.f16_bits_to_f32(x).astype(np.float64) @ W.T.astype(np.float64)) * sc
    rf = orc.f16_bits_to_f32(r).astype(np.float64)
    # within ~1 f16 ulp of the float64 sum, measured against the magnitude of
    # its terms (the sum can cancel)
    assert np.all(np.abs(y - (p + rf)) <= 2 ** -10 * (np.abs(p) + np.abs(rf)) + 1e-6)
    # a -0 residual is the identity of fp32 addition: bit for bit gemm_w8a16
    mz = np.full((9, 13), 0x8000, np.uint16)
    assert np.array_equal(orc.gemm_w8a16_residual(x, W, sc, mz), orc.gemm_w8a16(x, W, sc))
    # zero weights leave the residual (0 * s + r = r exactly)
    assert np.array_equal(orc.f16_bits_to_f32(
        orc.gemm_w8a16_residual(x, np.zeros_like(W), sc, r)), orc.f16_bits_to_f32(r))
    # the residual is added after the per-channel scale, per output element
    y3 = orc.f16_bits_to_f32(orc.gemm_w8a16_residual(
        h(np.ones((1, 32))), np.ones((3, 32), np.int8), np.array([1.0, 2.0, 0.5], np.float32),
        h([[1.0, -2.0, 0.25]])))
    assert np.array_equal(y3, np.array([[33.0, 62.0, 16.25]], np.float32))
    # the sum rounds to fp32 before f16: p = 1 + 2^-20, r = 2048 -> fp32 2049,
    # an f16 tie that goes to even, 2048; one rounding of the exact sum
    # (a fused add-and-convert) gives 2050
    xk = np.zeros((1, 16)); xk[0, 0] = 1.0
    Wk = np.zeros((1, 16), np.int8); Wk[0, 0] = 1
    yk = orc.f16_bits_to_f32(orc.gemm_w8a16_residual(
        h(xk), Wk, np.array([1.0 + 2 ** -20], np.float32), h([[2048.0]])))
    assert yk[0, 0] == 2048.0
    assert np.float16(np.float64(1.0 + 2 ** -20) + 2048.0) == 2050.0


def test_swiglu_gateup_vs_numpy_f64_and_limits():
    rng = np.random.default_rng(5)
    K = 64
    x = h(rng.standard_normal((5, K)))
    Wg = rng.integers(-127, 128, (11, K)).astype(np.int8)
    Wu = rng.integers(-127, 128, (11, K)).astype(np.int8)
    sg = rng.uniform(0.001, 0.003, 11).astype(np.float32)
    su = rng.uniform(0.001, 0.003, 11).astype(np.float32)
    hh = orc.f16_bits_to_f32(orc.swiglu_gateup(x, Wg, Wu, sg, su))
    xf = orc.f16_bits_to_f32(x).astype(np.float64)
    g = (xf @ Wg.T.astype(np.float64)) * sg
    u = (xf @ Wu.T.astype(np.float64)) * su
    ref = g / (1.0 + np.exp(-g)) * u
    np.testing.assert_allclose(hh, ref, rtol=2 ** -9, atol=1e-6)
    # limits: g = 0 -> 0; g >> 0 -> g * u; g << 0 -> 0 (gate and up swapped fail these)
    one = h(np.ones((1, 16)))
    Wz = np.zeros((3, 16), np.int8)
    Wp = np.full((3, 16), 100, np.int8)
    Wun = np.ones((3, 16), np.int8)
    s1 = np.ones(3, np.float32)
    assert np.all(orc.f16_bits_to_f32(orc.swiglu_gateup(one, Wz, Wun, s1, s1)) == 0)
    big = orc.f16_bits_to_f32(orc.swiglu_gateup(one, Wp, Wun, s1, s1))
    assert np.array_equal(big, np.full((1, 3), 1600.0 * 16.0, np.float32))
    neg = orc.f16_bits_to_f32(orc.swiglu_gateup(one, -Wp, Wun, s1, s1))
    assert np.all(np.abs(neg) < 1e-30)


def test_swiglu_ffn_composes_the_stages():
    rng = np.random.default_rng(6)
    T, H, I = 4, 32, 48
    x = h(rng.standard_normal((T, H)))
    gamma = h(1 + 0.1 * rng.standard_normal(H))
    Wg = rng.integers(-127, 128, (I, H)).astype(np.int8)
    Wu = rng.integers(-127, 128, (I, H)).astype(np.int8)
    Wd = rng.integers(-127, 128, (H, I)).astype(np.int8)
    sg = np.full(I, 0.003, np.float32)
    su = np.full(I, 0.002, np.float32)
    sd = np.full(H, 0.004, np.float32)
    y = orc.swiglu_ffn(x, gamma, Wg, Wu, sg, su, Wd, sd)
    xn = orc.rmsnorm_rows(x, gamma, 1e-6, "f16")
    hh = orc.swiglu_gateup(xn, Wg, Wu, sg, su)
    assert np.array_equal(y, orc.gemm_w8a16(hh, Wd, sd))
    yr = orc.swiglu_ffn(x, gamma, Wg, Wu, sg, su, Wd, sd, residual=True)
    assert np.array_equal(yr, orc.gemm_w8a16_residual(hh, Wd, sd, x))


# ---- row reductions ----------------------------------------------------------------

def test_softmax_golden_and_invariants(golden):
    g = golden("rows")
    x = g["softmax_x_bits"]
    y = orc.f16_bits_to_f32(orc.softmax_rows(x))
    np.testing.assert_allclose(y, g["softmax_y"], rtol=1e-2, atol=1e-3)
    # the oracle is far tighter than the tolerance: within 1 f16 ulp
    np.testing.assert_allclose(y, g["softmax_y"], rtol=2 ** -10, atol=2 ** -24)
    assert np.allclose(y.sum(axis=1), 1.0, atol=1e-2)
    xf = orc.f16_bits_to_f32(x)
    assert np.array_equal(y.argmax(axis=1), xf.argmax(axis=1)) or np.all(
        np.take_along_axis(xf, y.argmax(axis=1)[:, None], 1)[:, 0] == xf.max(axis=1))
    # shift invariance: on multiples of 1/64 in (-8, 8), x + 8 is exact in f16
    small = h(np.round(np.clip(xf, -7.9, 7.9) * 64) / 64)
    shifted = h(orc.f16_bits_to_f32(small) + 8.0)
    assert np.array_equal(orc.softmax_rows(small), orc.softmax_rows(shifted))
    # constant row -> uniform 1/cols
    c = orc.f16_bits_to_f32(orc.softmax_rows(h(np.full((2, 64), 3.0))))
    assert np.array_equal(c, np.full((2, 64), np.float16(1 / 64), dtype=np.float32))


def test_softmax_vs_torch_f32_and_infinities():
    x = np.random.default_rng(8).standard_normal((16, 300)).astype(np.float32) * 4
    x[3, 7] = -np.inf
    y = orc.softmax_rows(x, dtype="f32")
    exp = torch.softmax(torch.from_numpy(x).double(), dim=-1).numpy()
    np.testing.assert_allclose(y, exp, rtol=1e-5, atol=1e-7)
    assert y[3, 7] == 0.0


def test_rmsnorm_golden_and_invariants(golden):
    g = golden("rows")
    y = orc.f16_bits_to_f32(orc.rmsnorm_rows(g["rms_x_bits"], g["rms_gamma_bits"], eps=1e-6))
    np.testing.assert_allclose(y, g["rms_y"], rtol=1e-2, atol=1e-2)
    np.testing.assert_allclose(y, g["rms_y"], rtol=2 ** -10, atol=2 ** -24)
    x = np.random.default_rng(9).standard_normal((8, 256)).astype(np.float32)
    y1 = orc.rmsnorm_rows(x, eps=0.0, dtype="f32")
    assert np.allclose((y1.astype(np.float64) ** 2).mean(axis=1), 1.0, atol=1e-5)
    y2 = orc.rmsnorm_rows(x * 4.0, eps=0.0, dtype="f32")
    np.testing.assert_allclose(y1, y2, rtol=1e-6, atol=1e-7)
    # eps is inside the square root: a zero row gives exactly 0, not NaN
    z = orc.rmsnorm_rows(np.zeros((1, 16), dtype=np.float32), eps=1e-6, dtype="f32")
    assert (z == 0).all()


def test_rmsnorm_vs_torch_reference_shape():
    """test_rms_norm.py: 127 x 513, eps 1e-5, f16 and f32."""
    x = np.random.default_rng(10).random((127, 513)).astype(np.float32)
    w = np.random.default_rng(11).random(513).astype(np.float32)
    y = orc.rmsnorm_rows(x, w, eps=1e-5, dtype="f32")
    exp = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (513,),
                                       weight=torch.from_numpy(w).double(), eps=1e-5).numpy()
    np.testing.assert_allclose(y, exp, rtol=1e-6, atol=1e-6)


def test_layernorm_golden(golden):
    g = golden("rows")
    y, mean, rstd = orc.layernorm_rows(g["ln_x"], g["ln_w"], g["ln_b"], eps=1e-5, dtype="f32")
    np.testing.assert_allclose(y, g["ln_y"], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(mean, g["ln_mean"], rtol=1e-6)
    np.testing.assert_allclose(rstd, g["ln_rstd"], rtol=1e-6)
    # gamma=1, beta=0: zero mean and (almost) unit biased variance
    y0, _, _ = orc.layernorm_rows(g["ln_x"], eps=0.0, dtype="f32")
    assert np.allclose(y0.mean(axis=1), 0.0, atol=1e-5)
    assert np.allclose(y0.var(axis=1), 1.0, atol=1e-4)
