"""The torch-facing mirror refuses operands whose shape, dtype or device
the C entries could not check (they write rows x cols elements at the output
pointer): every refusal here is raised before any launch.  Also the
column-split calling pattern: one rank's slice of the W8A16 GEMV written
into its columns of the full output through ldy, checked against the
oracle."""
import numpy as np
import pytest
import torch

import hxm.ops as ops
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def bits(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def test_gemm_outputs_of_the_wrong_shape_or_dtype_are_refused(dev):
    A = torch.randint(-127, 128, (64, 96), dtype=torch.int8, device=dev)
    B = torch.randint(-127, 128, (96, 32), dtype=torch.int8, device=dev)
    sentinel = torch.full((64, 32), 7, dtype=torch.int32, device=dev)
    with pytest.raises(TypeError):
        ops.gemm_i8(A, B, out=torch.empty(64, 32, dtype=torch.float16, device=dev))
    with pytest.raises(ValueError):
        ops.gemm_i8(A, B, out=torch.empty(32, 32, dtype=torch.int32, device=dev))
    with pytest.raises(ValueError):                       # B's K is not A's
        ops.gemm_i8(A, B[:64], out=sentinel)
    with pytest.raises(TypeError):
        ops.gemm_i8(A.half(), B.half())
    with pytest.raises(ValueError):
        ops.gemm_i8(A, B, b_layout="kn ")
    assert (sentinel == 7).all()
    Ah = torch.randn(64, 96, device=dev).half()
    Bh = torch.randn(96, 32, device=dev).half()
    with pytest.raises(ValueError):
        ops.matmul(Ah, Bh, out=torch.empty(64, 16, dtype=torch.float16, device=dev))
    with pytest.raises(TypeError):
        ops.matmul(Ah, Bh, out=torch.empty(64, 32, dtype=torch.int32, device=dev))
    with pytest.raises(ValueError):
        ops.prepack_weight(Bh, out=torch.empty(96, 32, dtype=torch.float16, device=dev))


def test_w8a16_and_row_operands_are_checked(dev):
    x = torch.randn(4, 256, device=dev).half()
    W = torch.randint(-127, 128, (48, 256), dtype=torch.int8, device=dev)
    sc = torch.ones(48, dtype=torch.float16, device=dev)
    with pytest.raises(ValueError):
        ops.gemv_w8a16(x, W, sc, out=torch.empty(4, 32, dtype=torch.float16, device=dev))
    with pytest.raises(ValueError):
        ops.gemv_w8a16(x, W, sc[:40])
    with pytest.raises(ValueError):
        ops.gemv_w8a16(x, W, sc.float())
    with pytest.raises(TypeError):
        ops.gemv_w8a16(x.float(), W, sc)
    with pytest.raises(TypeError):
        ops.gemm_w8a16(x, W, sc.float(), out=torch.empty(4, 48, dtype=torch.float32, device=dev))
    r = torch.randn(8, 64, device=dev).half()
    with pytest.raises(ValueError):
        ops.softmax(r, out=torch.empty(8, 64, dtype=torch.float32, device=dev))
    with pytest.raises(ValueError):
        ops.softmax(r, out=torch.empty(8, 32, dtype=torch.float16, device=dev))
    with pytest.raises(ValueError):
        ops.rms_norm(r, (64,), torch.ones(32, dtype=torch.float16, device=dev))
    with pytest.raises(ValueError):
        ops.layer_norm(r, (64,), torch.ones(64, device=dev), None)       # f32 gamma for f16 x
    with pytest.raises(ValueError):                       # rows not evenly strided
        ops.softmax(r.view(2, 4, 64), out=torch.empty(4, 2, 64, dtype=torch.float16,
                                                      device=dev).transpose(0, 1))


@pytest.mark.parametrize("M", [1, 4, 16])
@pytest.mark.parametrize("packed", [True, False])
def test_gemv_column_split_writes_through_ldy(dev, M, packed):
    """Eight ranks' slices of W (176 channels each, each with its own packed
    image) write their columns of one y [M, 1408] (ldy = 1408); the whole y
    matches the oracle of the unsplit GEMV."""
    N, K, ranks = 1408, 1024, 8
    n = N // ranks
    g = torch.Generator().manual_seed(50 + M)
    x = torch.randn(M, K, generator=g).half()
    W = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    sc = (torch.rand(N, generator=g) * 0.019 + 0.001).half()
    xd, Wd, scd = x.to(dev), W.to(dev), sc.to(dev)
    y = torch.full((M, N), 3.0, dtype=torch.float16, device=dev)
    for r in range(ranks):
        Wr = Wd[r * n:(r + 1) * n]
        Wr = ops.prepack_w8a16(Wr) if packed else Wr
        ops.gemv_w8a16(xd, Wr, scd[r * n:(r + 1) * n], out=y[:, r * n:(r + 1) * n], N=n)
    ref = orc.f16_bits_to_f32(orc.gemv_w8a16(bits(x), W.numpy(), bits(sc)))
    np.testing.assert_allclose(y.float().cpu().numpy(), ref, rtol=1e-2, atol=1e-3)


def test_device_count_sees_the_gfx950(dev):
    """hxm_device_count counts the visible gfx950 devices: the box's MI355X."""
    import hxm
    assert hxm.lib.hxm_device_count() == torch.cuda.device_count() >= 1
