"""Host threads on their own streams: four threads call the entries that
use a per-stream workspace (int8 K split, the stream-K W8A16 GEMM, f32
operands packed to f16, the resident-weight cache) together with the GEMV
and the row kernels, each on its own stream and with workspaces growing
while the other threads run.  Every result must be bit-identical to the
same call made alone on one thread (every kernel here is deterministic)."""
import threading

import numpy as np
import pytest
import torch

import hxm
import hxm.ops as ops

pytestmark = pytest.mark.gpu


def _cases(dev):
    """(name, thunk) pairs; each thunk runs on the caller's current stream."""
    g = torch.Generator().manual_seed(31)
    cases = []
    for i, K in enumerate((2048, 4096, 8192)):      # growing K-split planes
        A = torch.randint(-127, 128, (96, K), generator=g, dtype=torch.int8).to(dev)
        B = torch.randint(-127, 128, (K, 160), generator=g, dtype=torch.int8).to(dev)
        cfg = hxm.GemmConfig(128, 128, 128, 2, 2, 2, 8)
        cases.append((f"int8 split-8 K={K}", lambda A=A, B=B, cfg=cfg: ops.gemm_i8(A, B, config=cfg)))
    for M, N, K in ((512, 4096, 1024), (300, 520, 656)):   # stream-K partial tiles
        x = torch.randn(M, K, generator=g).half().to(dev)
        W = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
        s = (torch.rand(N, generator=g) * 0.019 + 0.001).to(dev)
        cfg = (256, 256, 64, 2, 2, 3, hxm.STREAM_K)
        cases.append((f"stream-K {M}x{N}x{K}",
                      lambda x=x, W=W, s=s, cfg=cfg: ops.gemm_w8a16(x, W, s, config=cfg)))
    for n in (64, 200, 384):                        # f32 operands packed in the workspace
        A = torch.randn(n, n, generator=g).to(dev)
        B = torch.randn(n, n, generator=g).to(dev)
        cases.append((f"f32 matmul {n}", lambda A=A, B=B: ops.matmul(A, B)))
    W = torch.randint(-127, 128, (1376, 4096), generator=g, dtype=torch.int8).to(dev)
    xg = torch.randn(4, 4096, generator=g).half().to(dev)
    sc = (torch.rand(1376, generator=g) * 0.019 + 0.001).half().to(dev)
    cases.append(("resident gemv", lambda: ops.gemv_w8a16(xg, ops.resident_weight(W, "w8a16"), sc,
                                                           N=1376)))
    xr = (torch.randn(333, 4096, generator=g) * 2).half().to(dev)
    cases.append(("softmax", lambda: ops.softmax(xr)))
    return cases


def test_threads_on_own_streams_match_single_thread(dev):
    cases = _cases(dev)
    want = {}
    for name, fn in cases:                          # alone, on one thread
        want[name] = fn().clone()
    torch.cuda.synchronize()
    errors = []

    def worker(t):
        try:
            stream = torch.cuda.Stream()
            order = cases[t:] + cases[:t]           # each thread its own order
            for rep in range(3):
                with torch.cuda.stream(stream):
                    outs = [(name, fn()) for name, fn in order]
                stream.synchronize()
                for name, out in outs:
                    if not torch.equal(out, want[name]):
                        errors.append(f"thread {t} rep {rep}: {name} differs")
        except Exception as e:                      # reported by the main thread
            errors.append(f"thread {t}: {e!r}")

    print("4 threads x 3 reps", flush=True)
    hxm.lib.hxm_release_cache()                     # workspaces grow while threads run
    # Daemon threads: a worker stuck in a call fails the test below without
    # keeping the test process alive after it.
    threads = [threading.Thread(target=worker, args=(t,), daemon=True) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads), "a worker thread did not finish"
    torch.cuda.synchronize()
    assert not errors, errors
