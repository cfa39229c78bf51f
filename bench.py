#!/usr/bin/env python3
"""Benchmark of the MI355X hot path; prints ONE JSON line on stdout.

Headline: int8 GEMM M=N=K=4096, A,B ~ U{-127..127},
exact int32 accumulation, per-row x per-col fp32 scales dequantised to fp16
(hxm_gemm_i8_dequant).  B is the resident [N,K] image made once before the
timed region (the reference's weight-resident path).  One step = one GEMM
launch on inputs already resident in HBM.  value = 2*M*N*K / time, in
tera-ops/s (TFLOP/s slot of the schema, int8 ops counted like flops).

Also reported under "extra" (not the headline): W8A16 GEMV M in {1,4,16},
softmax / RMSNorm rows on f16 [8192 x 4096] (all HBM-bound, timed while
rotating buffer sets larger than the 256 MB Infinity Cache), the fp16 256^3
matmul (launch-bound) and the int32-output int8 GEMM.

cpu_baseline: the C restatement in oracle/ (OpenMP over the host cores)
timed on a bounded row sample of the same GEMM.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "hexagon-mlir_amd"))
sys.path.insert(0, ROOT)

PEAK_INT8_TOPS = 5000.0    # MI355X dense int8 MFMA
PEAK_F16_TFLOPS = 2500.0   # dense fp16/bf16 MFMA
PEAK_HBM_GBS = 8000.0      # HBM3E


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def event_time_ms(torch, fn, steps, warmup, rotate=1):
    """Average per-launch time over `steps` launches, HIP events on torch's
    current stream (the stream every launch here is issued on)."""
    for i in range(warmup):
        fn(i % rotate)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for i in range(steps):
        fn(i % rotate)
    e1.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return e0.elapsed_time(e1) / steps, wall


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="approximate CPU time budget of the cpu_baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the hot path here is a single-GPU kernel set "
              "and no multi-GPU path is built (see DESIGN.md, 'How the path would shard').",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import hxm
    import hxm.ops as ops

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    L = hxm.lib

    # ---------------- headline: int8 GEMM 4096^3 + dequant -----------------
    M = N = K = 4096
    g = torch.Generator().manual_seed(1)
    A = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(dev)
    g.manual_seed(2)
    B_kn = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int8).to(dev)
    g.manual_seed(3)
    rs = (torch.rand(M, generator=g) * 0.019 + 0.001).to(dev)
    g.manual_seed(4)
    cs = (torch.rand(N, generator=g) * 0.019 + 0.001).to(dev)
    Bp = ops.prepack_weight(B_kn)               # resident [N, K] image, once
    C16 = torch.empty(M, N, dtype=torch.float16, device=dev)
    C32 = torch.empty(M, N, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()

    a_p, b_p, rs_p, cs_p, c_p = (A.data_ptr(), Bp.data_ptr(), rs.data_ptr(), cs.data_ptr(),
                                 C16.data_ptr())

    def step_dequant(_):
        st = L.hxm_gemm_i8_dequant(a_p, K, b_p, K, hxm.B_NK, rs_p, cs_p, c_p, N, M, N, K,
                                   None, stream)
        if st:
            hxm.check(st, "hxm_gemm_i8_dequant")

    ms, wall_ms = event_time_ms(torch, step_dequant, args.steps, args.warmup)
    ops_per = 2.0 * M * N * K
    tops = ops_per / (ms * 1e-3) / 1e12
    log(f"int8 gemm+dequant 4096^3: {ms * 1e3:.1f} us/launch (wall {wall_ms * 1e3:.1f}), "
        f"{tops:.0f} TOPS")

    extra = {}
    if not args.no_extra:
        c32_p = C32.data_ptr()

        def step_i32(_):
            hxm.check(L.hxm_gemm_i8(a_p, K, b_p, K, hxm.B_NK, c32_p, N, M, N, K, 0, None,
                                    stream), "hxm_gemm_i8")
        ms32, _ = event_time_ms(torch, step_i32, args.steps, args.warmup)
        extra["int8_gemm_i32_out_4096"] = {"us": ms32 * 1e3,
                                           "TOPS": ops_per / (ms32 * 1e-3) / 1e12}
        del C32

        # fp16 matmul 256^3 (launch-bound).
        a16 = (torch.rand(256, 256, device=dev) * 2 - 1).half()
        b16 = ops.prepack_weight((torch.rand(256, 256, device=dev) * 2 - 1).half())
        c16 = torch.empty(256, 256, dtype=torch.float16, device=dev)
        pa, pb, pc = a16.data_ptr(), b16.data_ptr(), c16.data_ptr()

        def step_mm(_):
            hxm.check(L.hxm_matmul(pa, 256, pb, 256, hxm.B_NK, pc, 256, 256, 256, 256,
                                   hxm.F16, hxm.F16, 0, None, stream), "hxm_matmul")
        msm, _ = event_time_ms(torch, step_mm, args.steps, args.warmup)
        extra["f16_matmul_256"] = {"us": msm * 1e3,
                                   "TFLOPS": 2 * 256 ** 3 / (msm * 1e-3) / 1e12,
                                   "note": "launch-bound; roofline fraction not meaningful"}

        # W8A16 GEMV, N=11008, K=4096: rotate 12 weight copies (540 MB).
        Ng, Kg, R = 11008, 4096, 12
        Ws = [torch.randint(-127, 128, (Ng, Kg), dtype=torch.int8, device=dev)
              for _ in range(R)]
        scs = [(torch.rand(Ng, device=dev) * 0.019 + 0.001).half() for _ in range(R)]
        for Mg in (1, 4, 16):
            xs = torch.randn(Mg, Kg, device=dev).half()
            ys = torch.empty(Mg, Ng, dtype=torch.float16, device=dev)
            wp = [w.data_ptr() for w in Ws]
            sp = [s.data_ptr() for s in scs]
            px, py = xs.data_ptr(), ys.data_ptr()

            def step_gemv(i, Mg=Mg, wp=wp, sp=sp, px=px, py=py):
                hxm.check(L.hxm_gemv_w8a16(px, Kg, wp[i], Kg, sp[i], py, Ng, Mg, Ng, Kg,
                                           stream), "hxm_gemv_w8a16")
            msg, _ = event_time_ms(torch, step_gemv, 240, 24, rotate=R)
            nbytes = Ng * Kg + Ng * 2 + Mg * Kg * 2 + Mg * Ng * 2
            gbs = nbytes / (msg * 1e-3) / 1e9
            extra[f"w8a16_gemv_M{Mg}"] = {"us": msg * 1e3, "GB/s": gbs,
                                          "hbm_frac": gbs / PEAK_HBM_GBS, "bytes": nbytes}
        del Ws, scs

        # Row ops on f16 [8192, 4096], 4 buffer sets (536 MB).
        rows, cols, R2 = 8192, 4096, 4
        xs = [(torch.randn(rows, cols, device=dev) * 2).half() for _ in range(R2)]
        ys = [torch.empty_like(xs[0]) for _ in range(R2)]
        gam = (1 + 0.1 * torch.randn(cols, device=dev)).half()
        xp = [t.data_ptr() for t in xs]
        yp = [t.data_ptr() for t in ys]
        gp = gam.data_ptr()

        def step_softmax(i):
            hxm.check(L.hxm_softmax_rows(xp[i], cols, yp[i], cols, rows, cols, hxm.F16,
                                         stream), "hxm_softmax_rows")

        def step_rms(i):
            hxm.check(L.hxm_rmsnorm_rows(xp[i], cols, gp, yp[i], cols, rows, cols, 1e-6,
                                         hxm.F16, stream), "hxm_rmsnorm_rows")
        for name, fn, nbytes in (("softmax_f16_8192x4096", step_softmax, 2 * rows * cols * 2),
                                 ("rmsnorm_f16_8192x4096", step_rms,
                                  2 * rows * cols * 2 + cols * 2)):
            msr, _ = event_time_ms(torch, fn, 200, 20, rotate=R2)
            gbs = nbytes / (msr * 1e-3) / 1e9
            extra[name] = {"us": msr * 1e3, "GB/s": gbs, "hbm_frac": gbs / PEAK_HBM_GBS,
                           "bytes": nbytes}
        del xs, ys
        for k, v in extra.items():
            log(k, json.dumps(v))

    # ---------------- CPU baseline (oracle, bounded sample) -----------------
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import oracle as orc
        threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
        threads = max(1, min(threads, os.cpu_count() or 1))
        Ah = A.cpu().numpy()
        Bh = Bp.cpu().numpy()
        rows = 8
        t0 = time.perf_counter()
        orc.gemm_i8(Ah[:rows], Bh, b_nk=True, threads=threads)
        t_probe = time.perf_counter() - t0
        rows = int(min(M, max(rows, rows * args.cpu_seconds / max(t_probe, 1e-6))))
        times = []
        for _ in range(1 if rows * t_probe / 8 > 3 else 3):
            t0 = time.perf_counter()
            orc.gemm_i8(Ah[:rows], Bh, b_nk=True, threads=threads)
            times.append(time.perf_counter() - t0)
        t = statistics.median(times)
        cpu = {"value": 2.0 * rows * N * K / t / 1e12, "unit": "TOPS", "cores": threads,
               "kind": "port",
               "sample": f"int8 GEMM rows 0..{rows - 1} of A[4096,4096] x resident "
                         f"B[4096,4096] -> int32 (C restatement oracle/oracle.c, "
                         f"gcc -O3 OpenMP), median of {len(times)} run(s), {t:.2f} s each"}
        log("cpu baseline", json.dumps(cpu))

    out = {
        "metric": "int8 GEMM 4096^3 TOPS (int32 accumulate, fp16 dequant) + % MFMA peak",
        "value": tops,
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded U{-127..127} int8, U[0.001,0.02] fp32 scales)",
        "config": {"workload": "int8 GEMM M=N=K=4096, int32 accumulate, per-row x per-col "
                               "fp32 scales dequant to fp16; B resident [N,K] image",
                   "M": M, "N": N, "K": K, "parallelism": "single-gpu"},
        "roofline": {"bound": "mfma", "achieved": tops, "peak": PEAK_INT8_TOPS,
                     "unit": "TFLOP/s", "frac": tops / PEAK_INT8_TOPS, "traffic": None,
                     "kernel": "gemm_kernel<int8_t,...,kEpiDequant>",
                     "work_per_launch": ops_per, "avg_launch_us": ms * 1e3},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
