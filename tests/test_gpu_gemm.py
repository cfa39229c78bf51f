"""GPU parity of the MFMA GEMMs against the CPU oracle.

int8 -> int32 and the dequant epilogue are bit-exact; f16/bf16 matmuls are
within rtol 1e-2 / atol 1e-3 (fp32 accumulate), the tolerance the target
states, plus a small-integer case that must be bit-exact.  At the full
4096^3 size the oracle runs on a row sample, and every element is covered
by exact int64 row- and column-checksums (sum_m C = (1^T A) B and
sum_n C = A (B 1), which a dropped tile, a transposed block or a wrong
offset all break)."""
import numpy as np
import pytest
import torch

import hxm
import hxm.ops as ops
import hxm.search as S
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def bits(t):
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def rand_i8(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-127, 128, shape, generator=g, dtype=torch.int8)


SHAPES = [(1, 1, 16), (67, 45, 96), (33, 130, 272), (128, 128, 256), (256, 256, 1024),
          (300, 260, 384), (1000, 520, 272), (5, 4096, 128)]


@pytest.mark.parametrize("M,N,K", SHAPES)
@pytest.mark.parametrize("layout", ["kn", "nk"])
def test_gemm_i8_bit_exact(dev, M, N, K, layout):
    print(f"gemm_i8 M={M} N={N} K={K} layout={layout}", flush=True)
    A = rand_i8((M, K), 1)
    B = rand_i8((K, N), 2)
    Bd = B.to(dev) if layout == "kn" else B.t().contiguous().to(dev)
    C = ops.gemm_i8(A.to(dev), Bd, b_layout=layout).cpu().numpy()
    assert np.array_equal(C, orc.gemm_i8(A.numpy(), B.numpy()))


def test_gemm_i8_golden(dev, golden):
    g = golden("gemm_i8")
    A = torch.from_numpy(g["A"]).to(dev)
    B = torch.from_numpy(g["B"]).to(dev)
    assert np.array_equal(ops.gemm_i8(A, B).cpu().numpy(), g["C"])
    d = ops.gemm_i8_dequant(A, B, torch.from_numpy(g["row_scale"]).to(dev),
                            torch.from_numpy(g["col_scale"]).to(dev))
    assert np.array_equal(bits(d), g["dequant_f16_bits"])


@pytest.mark.parametrize("K", [640, 656, 16])  # K bytes a multiple of every stage depth / not
@pytest.mark.parametrize("cfg", S.gemm_configs(hxm.I8), ids=repr)
def test_gemm_i8_every_config(dev, cfg, K):
    """Both main loops of every compiled tile: the one without the per-lane
    K test (K a multiple of the stage depth) and the one with it (K = 16 is
    a single partial stage)."""
    print(f"gemm_i8 config {cfg} K={K}", flush=True)
    M, N = 300, 260
    A = rand_i8((M, K), 3)
    B = rand_i8((N, K), 4)  # resident [N, K] image
    C = ops.gemm_i8(A.to(dev), B.to(dev), b_layout="nk", config=cfg).cpu().numpy()
    assert np.array_equal(C, orc.gemm_i8(A.numpy(), B.numpy(), b_nk=True))


@pytest.mark.parametrize("N", [264, 260])  # 8-element runs wholly inside C / straddling N
@pytest.mark.parametrize("cfg", S.gemm_configs(hxm.I8), ids=repr)
def test_gemm_i8_dequant_every_config_edges(dev, cfg, N):
    """Tiles crossing M and N in the dequant epilogue: with N a multiple of 8
    they take the pipelined path with a per-run predicate, otherwise the
    general path."""
    print(f"gemm_i8_dequant config {cfg} N={N}", flush=True)
    M, K = 300, 640
    A = rand_i8((M, K), 31)
    B = rand_i8((N, K), 32)
    g = torch.Generator().manual_seed(33)
    rs = (torch.rand(M, generator=g) * 0.019 + 0.001).float()
    cs = (torch.rand(N, generator=g) * 0.019 + 0.001).float()
    D = ops.gemm_i8_dequant(A.to(dev), B.to(dev), rs.to(dev), cs.to(dev), b_layout="nk",
                            config=cfg)
    acc = orc.gemm_i8(A.numpy(), B.numpy(), b_nk=True)
    assert np.array_equal(bits(D), orc.dequant_f16(acc, rs.numpy(), cs.numpy()))


def test_edge_tiles_write_only_inside_the_output_view(dev):
    """The edge-tile epilogues (N a multiple of the run length) store into a
    [300, 264] view of a [320, 272] buffer: the padding columns and the rows
    past the view keep their sentinel, for the int8 dequant, int32, f16 and
    W8A16 outputs."""
    M, N, K = 300, 264, 256
    A = rand_i8((M, K), 41).to(dev)
    B = rand_i8((N, K), 42).to(dev)
    g = torch.Generator().manual_seed(43)
    rs = (torch.rand(M, generator=g) * 0.019 + 0.001).float().to(dev)
    cs = (torch.rand(N, generator=g) * 0.019 + 0.001).float().to(dev)
    for dt, run in ((torch.float16, lambda o: ops.gemm_i8_dequant(A, B, rs, cs, out=o,
                                                                     b_layout="nk")),
                    (torch.int32, lambda o: ops.gemm_i8(A, B, out=o, b_layout="nk"))):
        buf = torch.full((320, 272), 7, dtype=dt, device=dev)
        ref = run(torch.empty(M, N, dtype=dt, device=dev))
        run(buf[:M, :N])
        assert torch.equal(buf[:M, :N], ref)
        assert bool((buf[:M, N:] == 7).all()) and bool((buf[M:] == 7).all())
    Af = (torch.rand(M, K, generator=g) * 2 - 1).half().to(dev)
    Bf = (torch.rand(N, K, generator=g) * 2 - 1).half().to(dev)
    buf = torch.full((320, 272), 7, dtype=torch.float16, device=dev)
    ref = ops.matmul(Af, Bf, b_layout="nk")
    ops.matmul(Af, Bf, out=buf[:M, :N], b_layout="nk")
    assert torch.equal(buf[:M, :N], ref)
    assert bool((buf[:M, N:] == 7).all()) and bool((buf[M:] == 7).all())
    W = rand_i8((N, K), 44).to(dev)
    sw = (torch.rand(N, generator=g) * 1e-3).float().to(dev)
    r = torch.randn(M, N, generator=g).half().to(dev)
    for res in (None, r):
        buf = torch.full((320, 272), 7, dtype=torch.float16, device=dev)
        ref = ops.gemm_w8a16(Af, W, sw, residual=res)
        ops.gemm_w8a16(Af, W, sw, out=buf[:M, :N], residual=res)
        assert torch.equal(buf[:M, :N], ref)
        assert bool((buf[:M, N:] == 7).all()) and bool((buf[M:] == 7).all())


def test_gemm_i8_accumulate_and_strides(dev):
    M, N, K = 96, 80, 256
    Afull = rand_i8((M, 320), 5)
    A = Afull[:, :K]
    Ad = Afull.to(dev)[:, :K]              # lda = 320 on the device
    assert Ad.stride(0) == 320
    B = rand_i8((N, K), 6)
    C0 = torch.randint(-2 ** 31, 2 ** 31 - 1, (M, 100), dtype=torch.int32)
    Cd = C0.to(dev)
    ops.gemm_i8(Ad, B.to(dev), out=Cd[:, :N], b_layout="nk", accumulate=True)
    exp = orc.gemm_i8(A.numpy(), B.numpy(), b_nk=True, C=C0[:, :N].numpy(), accumulate=True)
    got = Cd.cpu().numpy()
    assert np.array_equal(got[:, :N], exp)
    assert np.array_equal(got[:, N:], C0[:, N:].numpy()), "wrote outside the output view"


def test_gemm_i8_int32_is_modular(dev):
    """int32 results wrap in two's complement, as the oracle's int8
    linalg.matmul does: C += A.B past 2^31 in the epilogue (both B layouts)
    and in the split-K reduce, and the MFMA's own int32 accumulator past 2^31
    (K = 131088 products of -128 * -128 = 16384 sum to 2^31 + 262144), alone
    and split in two (each plane below 2^31, the sum wrapping in the reduce)."""
    A = torch.full((64, 1024), 127, dtype=torch.int8)
    B = torch.full((1024, 64), 127, dtype=torch.int8)
    C0 = torch.full((64, 64), 2 ** 31 - 1000000, dtype=torch.int64).to(torch.int32)
    ref = orc.gemm_i8(A.numpy(), B.numpy(), C=C0.numpy(), accumulate=True)
    assert (ref < 0).all()                      # the sum did wrap
    Ad, Bd = A.to(dev), B.to(dev)
    for lay, Bl in (("kn", Bd), ("nk", ops.prepack_weight(Bd))):
        for cfg in (None, hxm.GemmConfig(64, 64, 128, 2, 2, 2, 4)):
            C = C0.to(dev)
            ops.gemm_i8(Ad, Bl, out=C, b_layout=lay, accumulate=True, config=cfg)
            assert np.array_equal(C.cpu().numpy(), ref), f"{lay} {cfg}"
    K = 131088
    print(f"int8 accumulator wrap, K={K}", flush=True)
    A = torch.full((32, K), -128, dtype=torch.int8)
    B = torch.full((K, 32), -128, dtype=torch.int8)
    ref = orc.gemm_i8(A.numpy(), B.numpy())
    assert (ref == K * 16384 - 2 ** 32).all()
    Ad, Bp = A.to(dev), ops.prepack_weight(B.to(dev))
    for cfg in (None, hxm.GemmConfig(32, 32, 128, 1, 1, 2, 2)):
        got = ops.gemm_i8(Ad, Bp, b_layout="nk", config=cfg)
        assert np.array_equal(got.cpu().numpy(), ref), f"K={K} {cfg}"


def test_matmul_f16_overflow_and_subnormal_outputs(dev):
    """The fp32 -> f16 rounding at the edges of f16: sums past 65504 round to
    +-inf, and sums below the smallest normal (2^-14) come out as the
    subnormal the oracle's RNE conversion gives, bit for bit (every product
    and partial sum here is exact in fp32)."""
    M, N, K = 64, 64, 256                               # K <= 256: the small kernel too
    A = torch.full((M, K), 16.0).half()                 # 256 * 256 = 65536 -> +inf
    B = torch.full((K, N), 16.0).half()
    B[:, 1] = -16.0                                      # -> -inf
    tiny = torch.full((M, K), 2.0 ** -12).half()
    Bt = torch.full((K, N), 2.0 ** -12).half()           # 256 * 2^-24 = 2^-16
    Bt[:, 1] = 2.0 ** -15                                # 2^-19 = 32 subnormal ulps
    Bt[:, 2] = 3 * 2.0 ** -20                            # exactly 3 ulps
    Bt[:, 3] = 3 * 2.0 ** -21                            # 1.5 ulps: the tie rounds to 2
    for a, b in ((A, B), (tiny, Bt)):
        ref = orc.matmul(bits(a), bits(b))
        for cfg in (None, (256, 256, 64, 2, 2, 2, 1), (16, 16, 32, 1, 1, 0, 1)):
            got = ops.matmul(a.to(dev), b.to(dev), config=cfg)
            assert np.array_equal(bits(got), ref), cfg
    assert np.isinf(orc.f16_bits_to_f32(orc.matmul(bits(A), bits(B)))).all()
    sub = orc.matmul(bits(tiny), bits(Bt))
    assert (sub[:, :4] == [256, 32, 3, 2]).all()         # f16 bit patterns of the subnormals


def test_gemm_i8_4096_cube(dev):
    """The int8 4096^3 benchmark shape: int32 exact and the dequant epilogue."""
    n = 4096
    A = rand_i8((n, n), 11)
    B = rand_i8((n, n), 12)       # as [N, K]
    g = torch.Generator().manual_seed(13)
    rs = (torch.rand(n, generator=g) * 0.019 + 0.001).float()
    cs = (torch.rand(n, generator=g) * 0.019 + 0.001).float()
    Ad, Bd = A.to(dev), B.to(dev)
    C = ops.gemm_i8(Ad, Bd, b_layout="nk").cpu().numpy()
    a64, b64 = A.numpy().astype(np.int64), B.numpy().astype(np.int64)
    c64 = C.astype(np.int64)
    assert np.array_equal(c64.sum(axis=0), a64.sum(axis=0) @ b64.T)
    assert np.array_equal(c64.sum(axis=1), a64 @ b64.sum(axis=0))
    rows = np.random.default_rng(14).choice(n, 48, replace=False)
    ref = orc.gemm_i8(A.numpy()[rows], B.numpy(), b_nk=True)
    assert np.array_equal(C[rows], ref)
    D = ops.gemm_i8_dequant(Ad, Bd, rs.to(dev), cs.to(dev), b_layout="nk")
    assert np.array_equal(bits(D), orc.dequant_f16(C, rs.numpy(), cs.numpy()))


def test_gemm_i8_dequant_double_rounding(dev):
    """512 x 512 x 4096: at this size some outputs sit where a fused
    multiply-convert (one rounding) and the defined fp32-then-f16 spelling
    (two roundings) disagree, so the epilogue's spelling is observable."""
    A = rand_i8((512, 4096), 21)
    B = rand_i8((512, 4096), 22)
    g = torch.Generator().manual_seed(23)
    rs = (torch.rand(512, generator=g) * 0.019 + 0.001).float()
    cs = (torch.rand(512, generator=g) * 0.019 + 0.001).float()
    D = ops.gemm_i8_dequant(A.to(dev), B.to(dev), rs.to(dev), cs.to(dev), b_layout="nk")
    acc = orc.gemm_i8(A.numpy(), B.numpy(), b_nk=True)
    exp = orc.dequant_f16(acc, rs.numpy(), cs.numpy())
    fused = (acc.astype(np.float32) * rs.numpy()[:, None]).astype(np.float64) * \
        cs.numpy()[None, :].astype(np.float64)
    assert not np.array_equal(fused.astype(np.float16).view(np.uint16), exp)
    assert np.array_equal(bits(D), exp)


def test_prepack_is_the_transpose(dev):
    for dt, K, N in ((torch.int8, 300, 77), (torch.float16, 64, 1000)):
        B = torch.randn(K, N).to(dt) if dt != torch.int8 else rand_i8((K, N), 7)
        P = ops.prepack_weight(B.to(dev)).cpu()
        assert torch.equal(P, B.t().contiguous())


@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (64, 128, 64), (1024, 512, 64),
                                   (256, 64, 2048), (128, 128, 128), (77, 150, 200)])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_matmul_within_tolerance(dev, M, N, K, dt):
    """The fp16 256^3 benchmark shape and the reference's S1/S2/S3 shapes
    (ROADMAP.md:98-100), U[-1,1] inputs."""
    print(f"matmul {dt} M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(M + N + K)
    a = (torch.rand(M, K, generator=g) * 2 - 1).to(dt)
    b = (torch.rand(K, N, generator=g) * 2 - 1).to(dt)
    name = "f16" if dt == torch.float16 else "bf16"
    c = ops.matmul(a.to(dev), b.to(dev)).cpu()
    ref = orc.to_f32(orc.matmul(bits(a), bits(b), ab_dtype=name, c_dtype=name), name)
    np.testing.assert_allclose(c.float().numpy(), ref, rtol=1e-2, atol=1e-3)
    c32 = ops.matmul(a.to(dev), b.t().contiguous().to(dev), b_layout="nk",
                     out_dtype=torch.float32).cpu().numpy()
    ref32 = orc.matmul(bits(a), bits(b), ab_dtype=name, c_dtype="f32")
    np.testing.assert_allclose(c32, ref32, rtol=1e-4, atol=1e-4)


# K = 640: K bytes a multiple of every stage depth; 656: not, a whole number
# of 16-element k-steps; 648: ends in a partial k-step.
@pytest.mark.parametrize("K", [640, 656, 648])
@pytest.mark.parametrize("cfg", S.gemm_configs(hxm.F16), ids=repr)
def test_matmul_every_config(dev, cfg, K):
    """Every tile within tolerance of the oracle and bit-identical to the
    default tile: all tiles group K into the same 16-element k-steps."""
    print(f"matmul f16/bf16 config {cfg} K={K}", flush=True)
    M, N = 300, 260
    g = torch.Generator().manual_seed(K)
    for dt, name in ((torch.float16, "f16"), (torch.bfloat16, "bf16")):
        A = (torch.rand(M, K, generator=g) * 2 - 1).to(dt)
        B = (torch.rand(K, N, generator=g) * 2 - 1).to(dt)
        Ad, Bd = A.to(dev), B.t().contiguous().to(dev)
        C = ops.matmul(Ad, Bd, b_layout="nk", config=cfg)
        ref = orc.to_f32(orc.matmul(bits(A), bits(B), ab_dtype=name, c_dtype=name), name)
        np.testing.assert_allclose(C.float().cpu().numpy(), ref, rtol=1e-2, atol=1e-3)
        assert torch.equal(C, ops.matmul(Ad, Bd, b_layout="nk"))


def test_matmul_small_integers_bit_exact(dev, golden):
    g = golden("matmul_f16")
    a = torch.from_numpy(g["Ai_bits"].view(np.float16)).to(dev)
    b = torch.from_numpy(g["Bi_bits"].view(np.float16)).to(dev)
    assert np.array_equal(bits(ops.matmul(a, b)), g["Ci_bits"])
    ar = torch.from_numpy(g["A_bits"].view(np.float16)).to(dev)
    br = torch.from_numpy(g["B_bits"].view(np.float16)).to(dev)
    np.testing.assert_allclose(ops.matmul(ar, br).float().cpu().numpy(), g["C_f64"],
                               rtol=1e-2, atol=1e-3)


def test_matmul_identity_and_accumulate(dev):
    n = 128
    B = torch.randn(n, 96).half()
    I = torch.eye(n).half()
    assert torch.equal(ops.matmul(I.to(dev), B.to(dev)).cpu(), B)
    a = torch.randn(64, 128).half()
    b = torch.randn(128, 96).half()
    C0 = torch.randn(64, 96)
    Cd = C0.to(dev)
    ops.matmul(a.to(dev), b.to(dev), out=Cd, accumulate=True)
    ref = orc.matmul(bits(a), bits(b), c_dtype="f32", C=C0.numpy(), accumulate=True)
    np.testing.assert_allclose(Cd.cpu().numpy(), ref, rtol=1e-4, atol=1e-4)


def test_zero_k_and_empty(dev):
    A = torch.empty(8, 0, dtype=torch.float16, device=dev)
    B = torch.empty(0, 16, dtype=torch.float16, device=dev)
    C = ops.matmul(A, B)
    assert torch.equal(C.cpu(), torch.zeros(8, 16, dtype=torch.float16))
    E = ops.gemm_i8(torch.empty(0, 32, dtype=torch.int8, device=dev),
                    torch.empty(32, 8, dtype=torch.int8, device=dev))
    assert E.shape == (0, 8)


def test_refuses_misaligned_k(dev):
    A = torch.zeros(8, 24, dtype=torch.int8, device=dev)
    B = torch.zeros(24, 8, dtype=torch.int8, device=dev)
    with pytest.raises(hxm.HxmError, match="tile-alignment"):
        ops.gemm_i8(A, B)


def _split(cfg, s):
    t = list(cfg.as_tuple())
    t[6] = s
    return hxm.GemmConfig(*t)


@pytest.mark.parametrize("split", [2, 4, 16])
@pytest.mark.parametrize("cfg", S.gemm_configs(hxm.I8), ids=repr)
def test_gemm_i8_split_k_bit_exact(dev, cfg, split):
    """K split over workgroup rows: int32 partial planes summed in plane order
    are exact, so every split equals the oracle bit for bit -- with K not a
    multiple of the slice (a short last slice), with fewer stages than
    splits (fewer, non-empty slices) and with N = 33 (plane rows of 132
    bytes: the partial planes take the element-wise store path)."""
    for M, N, K in [(300, 260, 4112), (64, 96, 640), (40, 33 * 8, 16 * 9), (72, 33, 1024)]:
        print(f"gemm_i8 split_k={split} config {cfg} M={M} N={N} K={K}", flush=True)
        A = rand_i8((M, K), 41)
        B = rand_i8((N, K), 42)
        C = ops.gemm_i8(A.to(dev), B.to(dev), b_layout="nk", config=_split(cfg, split))
        assert np.array_equal(C.cpu().numpy(), orc.gemm_i8(A.numpy(), B.numpy(), b_nk=True))


def test_gemm_i8_split_k_accumulate_dequant_and_layout(dev):
    M, N, K = 200, 264, 2048
    A = rand_i8((M, K), 51)
    B = rand_i8((N, K), 52)
    acc = orc.gemm_i8(A.numpy(), B.numpy(), b_nk=True)
    cfg = _split(S.gemm_configs(hxm.I8)[0], 8)
    print(f"gemm_i8 split_k accumulate/dequant/kn {cfg}", flush=True)
    # accumulate into a strided int32 view: C += A.B
    base = torch.randint(-1000, 1000, (M, N + 8), dtype=torch.int32)
    Cd = base.clone().to(dev)
    ops.gemm_i8(A.to(dev), B.to(dev), Cd[:, :N], b_layout="nk", accumulate=True, config=cfg)
    got = Cd.cpu().numpy()
    assert np.array_equal(got[:, :N], base.numpy()[:, :N] + acc)
    assert np.array_equal(got[:, N:], base.numpy()[:, N:])
    # dequant epilogue, same spelling as the unsplit kernel
    g = torch.Generator().manual_seed(53)
    rs = (torch.rand(M, generator=g) * 0.019 + 0.001).float()
    cs = (torch.rand(N, generator=g) * 0.019 + 0.001).float()
    D = ops.gemm_i8_dequant(A.to(dev), B.to(dev), rs.to(dev), cs.to(dev), b_layout="nk",
                            config=cfg)
    assert np.array_equal(bits(D), orc.dequant_f16(acc, rs.numpy(), cs.numpy()))
    # B as a plain [K, N] operand (packed per call into the other workspace slot)
    Bkn = B.t().contiguous()
    C = ops.gemm_i8(A.to(dev), Bkn.to(dev), b_layout="kn", config=cfg)
    assert np.array_equal(C.cpu().numpy(), acc)


class _RawStream:
    """A HIP stream handle given by value (ops reads .cuda_stream)."""

    def __init__(self, handle):
        self.cuda_stream = handle


@pytest.mark.parametrize("handle", [1, 2], ids=["hipStreamLegacy", "hipStreamPerThread"])
def test_split_k_kn_layout_on_special_stream_handles(dev, handle):
    """The per-stream workspace keeps the per-call B pack and the split-K
    partial planes apart on every stream handle, including the small integer
    handles HIP reserves (hipStreamLegacy = 1, hipStreamPerThread = 2)."""
    M, N, K = 200, 264, 2048
    A = rand_i8((M, K), 61)
    B = rand_i8((N, K), 62)
    acc = orc.gemm_i8(A.numpy(), B.numpy(), b_nk=True)
    cfg = _split(S.gemm_configs(hxm.I8)[0], 8)
    print(f"gemm_i8 split_k=8 kn layout on stream handle {handle}", flush=True)
    Bkn = B.t().contiguous().to(dev)
    Ad = A.to(dev)
    torch.cuda.synchronize()
    C = ops.gemm_i8(Ad, Bkn, b_layout="kn", config=cfg, stream=_RawStream(handle))
    torch.cuda.synchronize()
    assert np.array_equal(C.cpu().numpy(), acc)


def test_graph_capture_needs_a_grown_workspace(dev):
    """Under HIP graph capture the per-stream workspace cannot grow: a [K,N]
    B, packed per call into the workspace, is refused with workspace-budget
    on a stream whose workspace is still empty, and the capture stays valid.
    One eager call of the shape grows the workspace; the same call then
    captures, and every replay (with eager work and a synchronisation in
    between) equals the eager result."""
    from hxm import _lib
    M, N, K = 192, 160, 512
    A = rand_i8((M, K), 81)
    B = rand_i8((N, K), 82)
    want = orc.gemm_i8(A.numpy(), B.numpy(), b_nk=True)
    Ad, Bkn = A.to(dev), B.t().contiguous().to(dev)
    C = torch.full((M, N), 7, dtype=torch.int32, device=dev)
    mark = torch.zeros(1, device=dev)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    assert hxm.lib.hxm_release_cache() == 0  # no workspace left from earlier tests

    def call():
        return hxm.lib.hxm_gemm_i8(Ad.data_ptr(), K, Bkn.data_ptr(), N, hxm.B_KN, C.data_ptr(),
                                   N, M, N, K, 0, None, s.cuda_stream)
    print("gemm_i8 kn layout under graph capture", flush=True)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        mark.add_(1)
        st = call()
    assert st == _lib.HXM_UNSUPPORTED_SHAPE
    assert hxm.last_error().startswith("workspace-budget")
    with torch.cuda.stream(s):
        assert call() == 0
    torch.cuda.synchronize()
    assert np.array_equal(C.cpu().numpy(), want)
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2, stream=s):
        assert call() == 0
    for _ in range(3):
        C.fill_(7)
        torch.cuda.synchronize()
        g2.replay()
        torch.cuda.synchronize()
        assert np.array_equal(C.cpu().numpy(), want)


def test_split_k_is_int8_only(dev):
    A = torch.zeros(64, 64, dtype=torch.float16, device=dev)
    B = torch.zeros(64, 64, dtype=torch.float16, device=dev)
    cfg = _split(S.gemm_configs(hxm.F16)[0], 2)
    with pytest.raises(hxm.HxmError):
        ops.matmul(A, B, b_layout="nk", config=cfg)


# ---- f32 operands: quantised to fp16 in the pack (HMXAPI.h:107-137) --------

def _f16_image(x):
    """The reference's f32 pack spelled in numpy: x + 0.0 (-0 -> +0), then
    IEEE round to nearest even (numpy's float16 cast)."""
    return (x.astype(np.float32) + np.float32(0.0)).astype(np.float16)


@pytest.mark.parametrize("layout", ["kn", "nk"])
@pytest.mark.parametrize("M,N,K", [(64, 96, 256), (100, 60, 36), (33, 17, 5)])
def test_matmul_f32_operands_against_the_oracle(dev, layout, M, N, K):
    print(f"matmul f32 {layout} M={M} N={N} K={K}", flush=True)
    g = torch.Generator().manual_seed(M * 7 + K)
    A = (torch.rand(M, K, generator=g) * 2 - 1).float().numpy()
    B = (torch.rand(K, N, generator=g) * 2 - 1).float().numpy()
    Bl = B if layout == "kn" else np.ascontiguousarray(B.T)
    for od in (torch.float32, torch.float16):
        C = ops.matmul(torch.from_numpy(A).to(dev), torch.from_numpy(Bl).to(dev),
                       b_layout=layout, out_dtype=od).float().cpu().numpy()
        a16 = _f16_image(A).view(np.uint16)
        b16 = _f16_image(B).view(np.uint16)
        ref = orc.f16_bits_to_f32(orc.matmul(a16, b16)) if od == torch.float16 else \
            orc.matmul(a16, b16, c_dtype="f32")
        np.testing.assert_allclose(C, ref, rtol=1e-2, atol=1e-3)


def test_matmul_f32_rounds_to_nearest_even_in_the_pack(dev):
    """Halfway points between fp16 neighbours: with B the identity, C is A's
    fp16 image itself (one product per output, the others exactly zero), so
    round-to-nearest-even is checked bit for bit (truncation or rounding half
    up would give the other neighbour)."""
    ulp = 2.0 ** -10
    vals = np.array([1 + ulp / 2, 1 + 1.5 * ulp, -(1 + 1.5 * ulp), 2048 + 1, 3 + 0.75 * ulp,
                     -0.0, 65504.0, 1e-8, -1e-8, 0.1, -0.3, 7.0], dtype=np.float32)
    K = 16
    A = np.zeros((8, K), dtype=np.float32)
    A.flat[:vals.size] = vals
    A[4:] = np.random.default_rng(5).uniform(-4, 4, (4, K)).astype(np.float32)
    eye = np.eye(K, dtype=np.float32)
    C = ops.matmul(torch.from_numpy(A).to(dev), torch.from_numpy(eye).to(dev),
                   out_dtype=torch.float16).cpu().numpy()
    want = _f16_image(A)
    # Exact bits wherever the image is nonzero; a zero's sign cannot survive
    # the fp32 sum (it starts at +0), so zeros are compared as values.
    nz = want.astype(np.float32) != 0
    assert np.array_equal(C.view(np.uint16)[nz], want.view(np.uint16)[nz])
    assert np.all(C[~nz] == 0)
    assert C[0, 0] == np.float16(1.0) and C[0, 1] == np.float16(1 + 2 * ulp)


def test_last_plan_records_each_call(dev):
    A = rand_i8((96, 256), 71).to(dev)
    B = rand_i8((80, 256), 72).to(dev)
    cfg = S.gemm_configs(hxm.I8)[1]
    ops.gemm_i8(A, B, b_layout="nk", config=cfg)
    p = ops.last_plan()
    assert p["op"] == hxm.I8 and p["source"] == "caller" and p["plan"] == "mfma-tail"
    assert p["config"][:6] == cfg.as_tuple()[:6] and p["shape"] == (96, 80, 256)
    with pytest.raises(hxm.HxmError, match="lds-budget"):
        ops.gemm_i8(A, B, b_layout="nk", config=(512, 512, 256, 2, 2, 2, 1))
    p = ops.last_plan()
    assert p["plan"] == "refused" and p["reason"] == "lds-budget"
    x = torch.randn(64, 256, device=dev).half()
    ops.gemm_w8a16(x, B, torch.rand(80, device=dev))
    p = ops.last_plan()
    assert p["op"] == hxm._lib.OP_W8A16 and p["plan"] == "mfma-tail" and p["threads"] > 0


def test_matmul_through_memref_descriptors(dev):
    """A caller holding the reference's memref descriptors (common.h:15-30):
    views with offsets into wider buffers, converted to (ptr, ld) by
    hxm.memref and run through hxm_matmul; checked against the oracle."""
    from hxm import memref as mr
    M, K, N = 40, 64, 24
    g = torch.Generator().manual_seed(81)
    big_a = (torch.rand(M + 3, K + 16, generator=g) * 2 - 1).half()
    big_b = (torch.rand(K + 1, N + 8, generator=g) * 2 - 1).half()
    big_c = torch.zeros(M, N + 8, dtype=torch.float32)
    da, db, dc = big_a.to(dev), big_b.to(dev), big_c.to(dev)
    A = mr.describe(da.data_ptr(), M, K, K + 16, offset=2 * (K + 16) + 8)
    B = mr.describe(db.data_ptr(), K, N, N + 8, offset=1 * (N + 8) + 0)
    C = mr.describe(dc.data_ptr(), M, N, N + 8, offset=8)
    mr.matmul(A, B, C, ab_dtype=hxm.F16, c_dtype=hxm.F32,
              stream=torch.cuda.current_stream().cuda_stream)
    got = dc.cpu()
    a = big_a[2:2 + M, 8:8 + K].contiguous()
    b = big_b[1:1 + K, :N].contiguous()
    bits = lambda t: t.view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    ref = orc.matmul(bits(a), bits(b), c_dtype="f32")
    np.testing.assert_allclose(got[:, 8:8 + N].numpy(), ref, rtol=1e-2, atol=1e-3)
    assert torch.count_nonzero(got[:, :8]) == 0


@pytest.mark.parametrize("M,N,K", [(256, 256, 256), (1, 1, 8), (17, 33, 40), (100, 70, 72),
                                   (300, 260, 200), (16, 512, 256)])
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_small_output_kernel(dev, M, N, K, dt):
    """The direct-load small-output kernel, the default for f16 / bf16 outputs
    of at most 512 16x16 tiles with K <= 256 (256^3 is 256 tiles):
    the plan names it, and its f16 / bf16 / f32 outputs, with and without
    accumulate, from [K, N] and [N, K] B, are within tolerance of the oracle.
    K = 8, 40, 72, 200 end inside a 32-wide k-step."""
    print(f"small kernel {dt} M={M} N={N} K={K}", flush=True)
    small = (16, 16, 32, 1, 1, 0, 1)
    name = "f16" if dt == torch.float16 else "bf16"
    g = torch.Generator().manual_seed(M * 7 + N + K)
    a = (torch.rand(M, K, generator=g) * 2 - 1).to(dt)
    b = (torch.rand(K, N, generator=g) * 2 - 1).to(dt)
    ad, bd = a.to(dev), b.to(dev)
    c = ops.matmul(ad, bd)
    assert ops.last_plan()["config"] == small
    ref = orc.to_f32(orc.matmul(bits(a), bits(b), ab_dtype=name, c_dtype=name), name)
    np.testing.assert_allclose(c.float().cpu().numpy(), ref, rtol=1e-2, atol=1e-3)
    c32 = ops.matmul(ad, b.t().contiguous().to(dev), b_layout="nk", out_dtype=torch.float32)
    assert ops.last_plan()["config"] == small
    ref32 = orc.matmul(bits(a), bits(b), ab_dtype=name, c_dtype="f32")
    np.testing.assert_allclose(c32.cpu().numpy(), ref32, rtol=1e-4, atol=1e-4)
    C0 = torch.randn(M, N, generator=g)
    acc32 = C0.to(dev)
    ops.matmul(ad, bd, out=acc32, accumulate=True)
    ref_acc = orc.matmul(bits(a), bits(b), ab_dtype=name, c_dtype="f32", C=C0.numpy(),
                         accumulate=True)
    np.testing.assert_allclose(acc32.cpu().numpy(), ref_acc, rtol=1e-4, atol=1e-4)
    C0h = C0.to(dt)
    acch = C0h.to(dev)
    ops.matmul(ad, bd, out=acch, accumulate=True)
    ref_acch = orc.to_f32(orc.matmul(bits(a), bits(b), ab_dtype=name, c_dtype=name,
                                     C=bits(C0h), accumulate=True), name)
    np.testing.assert_allclose(acch.float().cpu().numpy(), ref_acch, rtol=1e-2, atol=1e-3)
    # the same product on the LDS-staged 32x32 tile agrees within tolerance
    staged = ops.matmul(ad, bd, config=(32, 32, 64, 1, 1, 2, 1))
    np.testing.assert_allclose(staged.float().cpu().numpy(), c.float().cpu().numpy(),
                               rtol=1e-2, atol=1e-3)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_small_output_kernel_strided_operands(dev, dt):
    """The small-output kernel on row views of wider buffers: lda > K, an
    [N, K] image with ldb > K, and C inside a wider buffer whose columns past
    N must stay untouched (f16 / bf16 and f32 outputs, with accumulate)."""
    M, N, K, lda, ldb, ldc = 37, 45, 88, 104, 120, 64
    print(f"small kernel strided {dt} M={M} N={N} K={K} lda={lda} ldb={ldb} ldc={ldc}",
          flush=True)
    name = "f16" if dt == torch.float16 else "bf16"
    g = torch.Generator().manual_seed(77)
    abuf = (torch.rand(M, lda, generator=g) * 2 - 1).to(dt)
    bbuf = (torch.rand(N, ldb, generator=g) * 2 - 1).to(dt)
    a, b_nk = abuf[:, :K], bbuf[:, :K]
    ref = orc.to_f32(orc.matmul(bits(a.contiguous()), bits(b_nk.t().contiguous()),
                                ab_dtype=name, c_dtype=name), name)
    ad, bd = abuf.to(dev)[:, :K], bbuf.to(dev)[:, :K]
    cbuf = torch.full((M, ldc), 7.0, dtype=dt, device=dev)
    ops.matmul(ad, bd, out=cbuf[:, :N], b_layout="nk")
    assert ops.last_plan()["config"] == (16, 16, 32, 1, 1, 0, 1)
    got = cbuf.float().cpu().numpy()
    np.testing.assert_allclose(got[:, :N], ref, rtol=1e-2, atol=1e-3)
    assert (got[:, N:] == 7.0).all(), "wrote past N"
    C0 = torch.randn(M, N, generator=g)
    fbuf = torch.full((M, ldc), -3.0, dtype=torch.float32, device=dev)
    fbuf[:, :N] = C0.to(dev)
    ops.matmul(ad, bd, out=fbuf[:, :N], b_layout="nk", accumulate=True)
    ref_acc = orc.matmul(bits(a.contiguous()), bits(b_nk.t().contiguous()), ab_dtype=name,
                         c_dtype="f32", C=C0.numpy(), accumulate=True)
    got = fbuf.cpu().numpy()
    np.testing.assert_allclose(got[:, :N], ref_acc, rtol=1e-4, atol=1e-4)
    assert (got[:, N:] == -3.0).all(), "wrote past N"


def test_small_output_kernel_refusals(dev):
    small = (16, 16, 32, 1, 1, 0, 1)
    a = torch.randn(1024, 512, device=dev).half()
    b = torch.randn(512, 1024, device=dev).half()
    with pytest.raises(hxm.HxmError, match="no-kernel"):
        ops.matmul(a, b, config=small)                   # 4096 tiles, K = 512
    with pytest.raises(hxm.HxmError, match="no-kernel"):
        ops.gemm_i8(torch.zeros(64, 64, dtype=torch.int8, device=dev),
                    torch.zeros(64, 64, dtype=torch.int8, device=dev), config=small)


@pytest.mark.parametrize("dt,K,kp", [(torch.int8, 4000, 4096), (torch.int8, 128, 128),
                                     (torch.float16, 200, 256), (torch.bfloat16, 64, 64)])
def test_prepacked_rows_start_on_cache_lines(dev, dt, K, kp):
    """prepack_weight pads the image's rows to 128 bytes (a [N, K] view of
    [N, kp] storage) and the GEMMs read it through its row stride."""
    print(f"prepack rows {dt} K={K}", flush=True)
    N, M = 40, 24
    g = torch.Generator().manual_seed(K)
    if dt == torch.int8:
        A = torch.randint(-127, 128, (M, K), generator=g, dtype=dt)
        B = torch.randint(-127, 128, (K, N), generator=g, dtype=dt)
    else:
        A = (torch.rand(M, K, generator=g) * 2 - 1).to(dt)
        B = (torch.rand(K, N, generator=g) * 2 - 1).to(dt)
    img = ops.prepack_weight(B.to(dev))
    assert img.shape == (N, K) and img.stride() == (kp, 1)
    assert torch.equal(img.cpu(), B.t())
    if dt == torch.int8:
        C = ops.gemm_i8(A.to(dev), img, b_layout="nk").cpu().numpy()
        assert np.array_equal(C, orc.gemm_i8(A.numpy(), B.numpy()))
    else:
        name = "f16" if dt == torch.float16 else "bf16"
        ref = orc.to_f32(orc.matmul(bits(A), bits(B), ab_dtype=name, c_dtype=name), name)
        got = ops.matmul(A.to(dev), img, b_layout="nk").float().cpu().numpy()
        np.testing.assert_allclose(got, ref, rtol=1e-2, atol=1e-3)
