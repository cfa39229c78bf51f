"""HIP graph capture of the memory-bound and FFN entries: the one-chunk and
pipelined W8A16 GEMV kernels (full and small N), the row ops and the FFN's
W8A16 GEMMs, captured once on a side stream, then replayed three times with
eager work (inputs refreshed, outputs poisoned) and a synchronisation between
replays; every replay must equal the eager result bit for bit (same kernels,
same inputs), and the eager result itself matches the oracle elsewhere."""
import pytest
import torch

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
            inp.mul_(2.0).copy_(keep)            # touched and restored
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for (name, _, out, _), w in zip(cases, want):
            assert torch.equal(out, w), f"replay {rep}: {name}"
