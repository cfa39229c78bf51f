"""HIP graph capture of the compute entries: the one-chunk and pipelined
W8A16 GEMV kernels (full and small N), the row ops, the FFN's W8A16 GEMMs and
the MFMA GEMMs (int8 dequant, an int8 K split through the stream's
workspace, f16 on both kernels, f32 operands), captured once on a side
stream after an eager call of each has grown the workspace, then replayed three times with
eager work (inputs refreshed, outputs poisoned) and a synchronisation between
replays; every replay must equal the eager result bit for bit (same kernels,
same inputs), and the eager result itself matches the oracle elsewhere."""
import pytest
import torch

import hxm
import hxm.ops as ops

pytestmark = pytest.mark.gpu


def test_replays_equal_the_eager_results(dev):
    g = torch.Generator().manual_seed(90)
    K = 1024
    cases = []                                   # (name, fn(out), out, inputs to refresh)
    for M, N in ((1, 5136), (4, 5136), (16, 5136), (1, 1376), (4, 1376), (16, 1376)):
        x = torch.randn(M, K, generator=g).half().to(dev)
        W = ops.prepack_w8a16(torch.randint(-127, 128, (N, K), generator=g,
                                            dtype=torch.int8).to(dev))
        sc = (torch.rand(N, generator=g) * 0.02 + 0.001).half().to(dev)
        y = torch.empty(M, N, dtype=torch.float16, device=dev)
        cases.append((f"gemv M={M} N={N}",
                      lambda y, x=x, W=W, sc=sc, N=N: ops.gemv_w8a16(x, W, sc, out=y, N=N), y, x))
    r = (torch.randn(96, 4096, generator=g) * 2).half().to(dev)
    gam = (1 + 0.1 * torch.randn(4096, generator=g)).half().to(dev)
    for name, fn in (("softmax", lambda y: ops.softmax(r, out=y)),
                     ("rms_norm", lambda y: ops.rms_norm(r, (4096,), gam, eps=1e-6, out=y)),
                     ("layer_norm", lambda y: ops.layer_norm(r, (4096,), gam, None, out=y))):
        cases.append((name, fn, torch.empty_like(r), r))
    xs = torch.randn(256, 512, generator=g).half().to(dev)
    Wg, Wu = (torch.randint(-127, 128, (704, 512), generator=g, dtype=torch.int8).to(dev)
              for _ in range(2))
    sg, su = ((torch.rand(704, generator=g) * 0.004 + 0.001).to(dev) for _ in range(2))
    Wgu, sgu = ops.swiglu_pack(Wg, Wu, sg, su)
    cases.append(("swiglu gate/up", lambda h: ops.gemm_w8a16_swiglu(xs, Wgu, sgu, 704, out=h),
                  torch.empty(256, 704, dtype=torch.float16, device=dev), xs))
    # The MFMA GEMMs: int8 with the dequant epilogue on a resident B, an int8
    # K split over a [K, N] B (pack and partial planes in the stream's
    # workspace, grown by the eager call), f16 on the direct small-output
    # kernel and on the LDS-staged one, and f32 operands (fp16 images in the
    # workspace).
    A8 = torch.randint(-127, 128, (300, 2048), generator=g, dtype=torch.int8).to(dev)
    B8 = torch.randint(-127, 128, (2048, 200), generator=g, dtype=torch.int8).to(dev)
    B8p = ops.prepack_weight(B8)
    rs = (torch.rand(300, generator=g) * 0.02 + 0.001).to(dev)
    cs = (torch.rand(200, generator=g) * 0.02 + 0.001).to(dev)
    cases.append(("gemm_i8_dequant", lambda c: ops.gemm_i8_dequant(A8, B8p, rs, cs, out=c,
                                                                    b_layout="nk"),
                  torch.empty(300, 200, dtype=torch.float16, device=dev), A8))
    split = hxm.GemmConfig(256, 256, 128, 2, 2, 2, 4)
    cases.append(("gemm_i8 split 4", lambda c: ops.gemm_i8(A8, B8, out=c, config=split),
                  torch.empty(300, 200, dtype=torch.int32, device=dev), A8))
    a16, b16 = ((torch.rand(256, 256, generator=g) - 0.5).half().to(dev) for _ in range(2))
    cases.append(("matmul f16 256^3", lambda c: ops.matmul(a16, b16, out=c),
                  torch.empty(256, 256, dtype=torch.float16, device=dev), a16))
    a2 = (torch.rand(384, 1024, generator=g) - 0.5).half().to(dev)
    b2 = (torch.rand(1024, 640, generator=g) - 0.5).half().to(dev)
    cases.append(("matmul f16 384x640x1024", lambda c: ops.matmul(a2, b2, out=c),
                  torch.empty(384, 640, dtype=torch.float16, device=dev), a2))
    a32 = torch.randn(200, 300, generator=g).to(dev)
    b32 = torch.randn(300, 100, generator=g).to(dev)
    cases.append(("matmul f32 operands", lambda c: ops.matmul(a32, b32, out=c),
                  torch.empty(200, 100, dtype=torch.float32, device=dev), a32))

    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for _, fn, out, _ in cases:              # eager: the reference result of each
            fn(out)
    torch.cuda.synchronize()
    want = [out.clone() for _, _, out, _ in cases]
    print("capturing", len(cases), "entries", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=s):
        for _, fn, out, _ in cases:
            fn(out)
    saved = [inp.clone() for _, _, _, inp in cases]
    for rep in range(3):
        for (_, _, out, inp), keep in zip(cases, saved):
            out.fill_(-7.0)                      # eager work between replays
            inp.mul_(2).copy_(keep)              # touched and restored
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for (name, _, out, _), w in zip(cases, want):
            assert torch.equal(out, w), f"replay {rep}: {name}"
