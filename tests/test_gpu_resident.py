"""GPU tests of the content-addressed resident weight images
(hxm_resident_weight), the counterpart of the reference's WeightPrepack.pack
(backend/hmx_weight_prepack.py:124-212): cache hits on equal content, misses
on any change, the f32 -> f16 image with -0 -> +0 and RNE, and the
dtype / shape contract refusals."""
import numpy as np
import pytest
import torch

import hxm
import hxm.ops as ops
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def test_resident_gemm_image_is_content_addressed(dev):
    hxm.lib.hxm_release_cache()
    g = torch.Generator().manual_seed(1)
    W = (torch.rand(256, 384, generator=g) * 2 - 1).half().to(dev)     # B [K, N]
    img = ops.resident_weight(W)
    assert tuple(img.shape) == (384, 256)
    assert torch.equal(img, W.t().contiguous())                          # the [N, K] image
    assert torch.equal(img, ops.prepack_weight(W))                       # same as the pre-pack
    # equal content at another address, and through a strided view: hits
    assert ops.resident_weight(W.clone()).data_ptr() == img.data_ptr()
    Wb = torch.zeros(256, 400, dtype=torch.float16, device=dev)
    Wb[:, :384] = W
    assert ops.resident_weight(Wb[:, :384]).data_ptr() == img.data_ptr()
    # one element changed: a different image
    W2 = W.clone()
    W2[17, 5] += 1
    img2 = ops.resident_weight(W2)
    assert img2.data_ptr() != img.data_ptr() and torch.equal(img2, W2.t().contiguous())
    # swapping two elements (same multiset of values) also misses: position is hashed
    W3 = W.clone()
    W3[0, 0], W3[0, 1] = W[0, 1].clone(), W[0, 0].clone()
    if not torch.equal(W3, W):
        assert ops.resident_weight(W3).data_ptr() != img.data_ptr()
    # the image feeds the matmul as a resident B
    A = (torch.rand(64, 256, generator=g) * 2 - 1).half()
    C = ops.matmul(A.to(dev), img, b_layout="nk")
    ref = orc.f16_bits_to_f32(orc.matmul(bits(A), bits(W)))
    np.testing.assert_allclose(C.float().cpu().numpy(), ref, rtol=1e-2, atol=1e-3)
    hxm.lib.hxm_release_cache()


def test_resident_f32_source_becomes_f16_image(dev):
    g = torch.Generator().manual_seed(2)
    W = torch.randn(64, 96, generator=g) * 3
    W[3, 7] = -0.0
    W[5, 1] = 1.0 + 2.0 ** -11          # halfway between two f16 values: RNE rounds to even
    W[6, 2] = 1.0 + 3 * 2.0 ** -11      # halfway, rounds up to even
    img = ops.resident_weight(W.to(dev))
    assert img.dtype == torch.float16 and tuple(img.shape) == (96, 64)
    ref = (W.t().contiguous() + 0.0).half()                  # -0 -> +0, then RNE (torch's cast)
    assert np.array_equal(bits(img), bits(ref))
    assert bits(img)[7, 3] == 0                              # +0, not 0x8000
    assert img[1, 5].item() == 1.0 and img[2, 6].item() == 1.0 + 2.0 ** -9
    hxm.lib.hxm_release_cache()


def test_resident_int8_and_bf16_images(dev):
    g = torch.Generator().manual_seed(3)
    Wi = torch.randint(-127, 128, (128, 64), generator=g, dtype=torch.int8).to(dev)
    assert torch.equal(ops.resident_weight(Wi), Wi.t().contiguous())
    Wb = torch.randn(64, 32, generator=g).bfloat16().to(dev)
    img = ops.resident_weight(Wb)
    assert img.dtype == torch.bfloat16 and torch.equal(img, Wb.t().contiguous())
    hxm.lib.hxm_release_cache()


def test_resident_w8a16_image_matches_prepack(dev):
    g = torch.Generator().manual_seed(4)
    N, K = 300, 512
    W = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
    img = ops.resident_weight(W, "w8a16")
    assert img.numel() == hxm.lib.hxm_w8a16_packed_bytes(N, K)
    assert torch.equal(img, ops.prepack_w8a16(W))
    assert ops.resident_weight(W.clone(), "w8a16").data_ptr() == img.data_ptr()
    x = torch.randn(4, K, generator=g).half()
    sc = (torch.rand(N, generator=g) * 0.019 + 0.001).half()
    y = ops.gemv_w8a16(x.to(dev), img, sc.to(dev))
    ref = orc.f16_bits_to_f32(orc.gemv_w8a16(bits(x), W.cpu().numpy(), bits(sc)))
    np.testing.assert_allclose(y.float().cpu().numpy(), ref, rtol=1e-2, atol=1e-3)
    hxm.lib.hxm_release_cache()


def test_resident_contract_refusals(dev):
    W = torch.randn(32, 48).half().to(dev)
    with pytest.raises(hxm.HxmError, match="unsupported-dtype"):
        ops.resident_weight(W, expect_dtype=torch.float32)
    with pytest.raises(hxm.HxmError, match=r"shape \[32, 48\], expected \[32, 40\]"):
        ops.resident_weight(W, expect_shape=(32, 40))
    with pytest.raises(hxm.HxmError, match="unsupported-dtype"):
        ops.resident_weight(W, "w8a16")                   # the W8A16 image takes int8 only
    assert ops.resident_weight(W, expect_dtype=torch.float16, expect_shape=(32, 48)) is not None
    hxm.lib.hxm_release_cache()
