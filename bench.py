#!/usr/bin/env python3
"""Benchmark of the MI355X hot path; prints ONE JSON line on stdout.

Headline (the benchmark's metric and configuration): int8 GEMM M=N=K=4096, A,B ~ U{-127..127},
exact int32 accumulation, per-row x per-col fp32 scales dequantised to fp16
(hxm_gemm_i8_dequant).  B is the resident [N,K] image made once before the
timed region (the reference's weight-resident path).  One step = one GEMM
launch on inputs already resident in HBM.  value = 2*M*N*K / time in
tera-ops/s (int8 ops are counted like flops in the roofline's TFLOP/s slot).

Also reported under "extra" (not the headline): the int32-output int8 GEMM,
the fp16 256^3 matmul (launch-bound), a ragged int8 GEMM (M=N=K=4000: tail
tiles, a partial last K stage, C stored into a wider buffer), W8A16 GEMV M in
{1,4,16} and softmax /
RMSNorm rows on f16 [8192 x 4096] (HBM-bound: timed while rotating buffer
sets larger than the 256 MB Infinity Cache), the SwiGLU FFN block (tokens
2048, hidden 4096, intermediate 11008; tiles autotuned per GEMM; also with the
residual x + FFN(x) added in the down GEMM's epilogue), a plain
256 MiB device copy (the practical HBM copy rate next to the nominal peak),
and for context the vendor library (hipBLASLt via torch._int_mm /
torch.matmul) on the 4096^3 shapes next to this library's f16 4096^3 matmul.

Timing: a timed region is K back-to-back launches between one pair of HIP
events; the first region and ten more of the same launches give q20 / q50 /
q80 per launch, and every rate divides the algorithmic work by q50 (the
first region alone is reported as span_us).  HBM-bound results are also
given as a fraction of this library's streaming probes over the same bytes
(hxm_probe_copy for the row ops, hxm_probe_read for the GEMV): the measured
practical ceiling.

Output: one JSON line on stdout, kept well under 16 KB: the headline fields,
"configs" with one compact record per benchmark config (1: f16 256^3
matmul, 2: the headline, 3: W8A16 GEMV M=1/4/16, 4: softmax and RMSNorm
rows, 5: the SwiGLU FFN block), each with q20/q50/q80, rate, fraction of
the nominal peak, the HBM ceiling fraction where it applies and the CPU
figure, and "extra" with the context legs in a few numbers each.  Every
leg's full record (tuner tables, clock samples) goes to stderr.

CPU baselines: the C restatement in oracle/ built with -march=native on this
host (OpenMP, one thread count for every op) timed on a bounded sample of
each config's workload; the CPU model is recorded.

Warmup: the GPU's shader clock ramps up over the first ~60 ms of sustained
load (the headline kernel goes from ~66 to ~56 us per launch over its first
~1000 launches), so the default warmup is 2000 launches and the timed
region sees the steady-state clock.  The headline is also timed after the
"extra" legs, which keep the GPU busy for several seconds first: with a
short warmup (--warmup 5 --steps 20) it then reads the steady-state time as
well (one box: 57.5-57.9 us, against 58.0 us with 2000 warmup launches and
59.4 us when it was timed first, on a clock still ramping from idle).  It
still runs exactly W untimed launches and then exactly K timed ones.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
       python bench.py --only {int8,int8_i32,f16,ragged,gemv,rows,ffn,shard,copy,vendor,search,
                               ceilings}  (one workload, for rocprofv3 runs; prints its record)
"""
from __future__ import annotations

import argparse
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


class Ctx:
    def __init__(self, args):
        import torch

        import hxm
        import hxm.ops as ops
        self.args, self.torch, self.hxm, self.ops = args, torch, hxm, ops
        self.L = hxm.lib
        self.dev = torch.device("cuda:0")
        # Every launch and event goes to one created stream (default
        # priority), made torch's current stream, so that a HIP graph can
        # capture the same calls on it.
        self.s = torch.cuda.Stream()
        torch.cuda.set_stream(self.s)
        self.stream = self.s.cuda_stream

    def time_ms(self, fn, steps, warmup, rotate=1, reps=10):
        """Times `steps` launches after `warmup` untimed ones.

        The timed region: the launches back to back on torch's current stream
        (the stream every launch here is issued on) between one pair of HIP
        events, bracketed by device synchronisations; its time per launch is
        what every rate below divides by.  The spread: `reps` more reps of the
        same `steps` back-to-back launches, each between its own event pair;
        q20 / q50 / q80 are taken over the timed region and those reps (an
        event pair around every single launch would put a gap between
        launches, and the GPU's clock reacts to such gaps).  Returns a Timing
        in milliseconds per launch."""
        torch = self.torch
        for i in range(warmup):
            fn(i % rotate)
        torch.cuda.synchronize()

        def rep():
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(steps):
                fn(i % rotate)
            e1.record()
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) / steps
        t0 = time.perf_counter()
        span = rep()
        wall = (time.perf_counter() - t0) * 1e3 / steps
        return Timing([span] + [rep() for _ in range(reps)], span, wall)


    def graph_time(self, fn, launches, rotate=1, reps=5):
        """Per-launch time (ms, median of `reps`) of `launches` calls of fn(i %
        rotate) captured once into a HIP graph and replayed: the kernels back
        to back with no per-call host work, the rate a native caller's loop
        or a captured serving step sees.  The graph holds the kernel launches
        only."""
        torch = self.torch
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=self.s):
            for i in range(launches):
                fn(i % rotate)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            g.replay()
            e1.record()
            torch.cuda.synchronize()
            ts.append(e0.elapsed_time(e1) / launches)
        del g
        return sorted(ts)[len(ts) // 2]


class Timing:
    """One workload's times in ms per launch: `span`, the first timed region,
    and q20 / q50 / q80 over it and the extra reps (numpy's linear
    interpolation, the rule of hxm_quantile).  Every rate divides the work by
    the median, q50."""

    def __init__(self, per_rep, span, wall):
        import numpy as np
        self.per_rep = per_rep
        self.median, self.q20, self.q80 = (float(np.quantile(per_rep, q)) for q in (0.5, 0.2, 0.8))
        self.span, self.wall = span, wall

    def us(self):
        return {"us": self.median * 1e3, "q20_us": self.q20 * 1e3, "q50_us": self.median * 1e3,
                "q80_us": self.q80 * 1e3, "span_us": self.span * 1e3, "reps": len(self.per_rep)}


def int8_operands(c):
    torch, dev = c.torch, c.dev
    n = 4096
    g = torch.Generator().manual_seed(1)
    A = torch.randint(-127, 128, (n, n), generator=g, dtype=torch.int8).to(dev)
    g.manual_seed(2)
    B_kn = torch.randint(-127, 128, (n, n), generator=g, dtype=torch.int8).to(dev)
    g.manual_seed(3)
    rs = (torch.rand(n, generator=g) * 0.019 + 0.001).to(dev)
    g.manual_seed(4)
    cs = (torch.rand(n, generator=g) * 0.019 + 0.001).to(dev)
    Bp = c.ops.prepack_weight(B_kn)             # resident [N, K] image, once
    torch.cuda.synchronize()
    return A, Bp, rs, cs


def run_int8(c, A, Bp, rs, cs, out_i32=False):
    torch, hxm, L = c.torch, c.hxm, c.L
    M = N = K = 4096
    C = torch.empty(M, N, dtype=torch.int32 if out_i32 else torch.float16, device=c.dev)
    a, b, r, s, o, st = (A.data_ptr(), Bp.data_ptr(), rs.data_ptr(), cs.data_ptr(),
                         C.data_ptr(), c.stream)
    ldb = Bp.stride(0)                          # K: 4096-byte rows need no padding
    if out_i32:
        def step(_):
            hxm.check(L.hxm_gemm_i8(a, K, b, ldb, hxm.B_NK, o, N, M, N, K, 0, None, st),
                      "hxm_gemm_i8")
    else:
        def step(_):
            hxm.check(L.hxm_gemm_i8_dequant(a, K, b, ldb, hxm.B_NK, r, s, o, N, M, N, K, None,
                                            st), "hxm_gemm_i8_dequant")
    t = c.time_ms(step, c.args.steps, c.args.warmup)
    c.last_step = step
    ops_per = 2.0 * M * N * K
    return {**t.us(), "wall_us": t.wall * 1e3,
            "TOPS": ops_per / (t.median * 1e-3) / 1e12, "ops_per_launch": ops_per}


def run_f16(c):
    """The f16 256^3 matmul (a handful of workgroups: launch-bound).
    A Python loop of ctypes calls issues a launch every ~4 us, slower than
    the GPU runs them, so that loop times the host.  `us` comes from the
    launches replayed back to back from a HIP graph (50 per graph, captured
    once after the warmup; the graph holds the kernel launches only), which
    is the rate a native caller's loop sees; `host_loop_us` is the Python
    loop's figure.  Every replay's output is checked against the eager
    result."""
    torch, hxm, L = c.torch, c.hxm, c.L
    a16 = (torch.rand(256, 256, device=c.dev) * 2 - 1).half()
    b16 = c.ops.prepack_weight((torch.rand(256, 256, device=c.dev) * 2 - 1).half())
    c16 = torch.empty(256, 256, dtype=torch.float16, device=c.dev)
    pa, pb, pc = a16.data_ptr(), b16.data_ptr(), c16.data_ptr()

    def step(_=0):  # on torch's current stream (the capture stream while capturing)
        hxm.check(L.hxm_matmul(pa, 256, pb, 256, hxm.B_NK, pc, 256, 256, 256, 256, hxm.F16,
                               hxm.F16, 0, None, torch.cuda.current_stream().cuda_stream),
                  "hxm_matmul")
    host = c.time_ms(step, c.args.steps, c.args.warmup)
    want = c16.clone()
    per_graph = 50
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(per_graph):
            step()
    torch.cuda.synchronize()
    for _ in range(3):  # each replay, with eager work between, equals the eager result
        c16.zero_()
        g.replay()
        torch.cuda.synchronize()
        if not torch.equal(c16, want):
            raise RuntimeError("f16 256^3: a graph replay differs from the eager result")
    replays = max(1, c.args.steps // per_graph)

    def replay(_):
        c16.zero_()
        g.replay()
    t = c.time_ms(replay, replays, 2, reps=10)
    if not torch.equal(c16, want):
        raise RuntimeError("f16 256^3: a graph replay differs from the eager result")
    us = t.us()
    # per launch: the replay of 50 launches plus one small fill kernel
    graph = {k: (v / per_graph if k.endswith("us") else v) for k, v in us.items()}
    return {"f16_matmul_256": {**graph, "host_loop_us": host.median * 1e3,
                               "TFLOPS": 2 * 256 ** 3 / (graph["us"] * 1e-6) / 1e12,
                               "launches_per_graph": per_graph,
                               "note": "launch-bound; roofline fraction not meaningful"}}


def run_gemv(c):
    torch, hxm, L = c.torch, c.hxm, c.L
    N, K, R = 11008, 4096, 12            # 12 weight images = 540 MB rotated
    # Resident (pre-packed) images, made once outside the timed region.
    Ws = [c.ops.prepack_w8a16(torch.randint(-127, 128, (N, K), dtype=torch.int8,
                                            device=c.dev)) for _ in range(R)]
    scs = [(torch.rand(N, device=c.dev) * 0.019 + 0.001).half() for _ in range(R)]
    torch.cuda.synchronize()
    wp = [w.data_ptr() for w in Ws]
    sp = [s.data_ptr() for s in scs]
    out = {}
    for M in (1, 4, 16):
        xs = torch.randn(M, K, device=c.dev).half()
        ys = torch.empty(M, N, dtype=torch.float16, device=c.dev)
        px, py, st = xs.data_ptr(), ys.data_ptr(), c.stream

        def step(i, M=M, px=px, py=py):
            hxm.check(L.hxm_gemv_w8a16(px, K, wp[i], K, hxm.W_PACKED, sp[i], py, N, M, N, K,
                                       st), "hxm_gemv_w8a16")
        t = c.time_ms(step, 240, 24, rotate=R)
        nbytes = N * K + N * 2 + M * K * 2 + M * N * 2
        gbs = nbytes / (t.median * 1e-3) / 1e9
        out[f"w8a16_gemv_M{M}"] = {**t.us(), "GB/s": gbs, "hbm_frac": gbs / PEAK_HBM_GBS,
                                   "bytes": nbytes,
                                   "graph_us": c.graph_time(step, 240, rotate=R) * 1e3}
    # The practical ceiling: this library's streaming read of the same weight
    # bytes, over the same rotation of images.
    sink = torch.empty(8192, dtype=torch.int32, device=c.dev)  # HXM_PROBE_SINK_WORDS

    def read(i):
        hxm.check(L.hxm_probe_read(wp[i], N * K, sink.data_ptr(), c.stream), "hxm_probe_read")
    t = c.time_ms(read, 240, 24, rotate=R)
    gbs = N * K / (t.median * 1e-3) / 1e9
    read_graph_us = c.graph_time(read, 240, rotate=R) * 1e3
    out["hbm_ceiling_read_45MB"] = {**t.us(), "GB/s": gbs, "hbm_frac": gbs / PEAK_HBM_GBS,
                                    "bytes": N * K, "graph_us": read_graph_us,
                                    "what": "hxm_probe_read of one packed weight image "
                                            "(N*K bytes), 12 images rotated"}
    for M in (1, 4, 16):
        rec = out[f"w8a16_gemv_M{M}"]
        rec["ceiling_frac"] = rec["GB/s"] / gbs
        rec["graph_hbm_frac"] = rec["bytes"] / (rec["graph_us"] * 1e-6) / 1e9 / PEAK_HBM_GBS
        rec["graph_ceiling_frac"] = read_graph_us / rec["graph_us"] * N * K / rec["bytes"]
    return out


def run_rows(c):
    torch, hxm, L = c.torch, c.hxm, c.L
    rows, cols, R = 8192, 4096, 4        # 4 sets x 128 MiB rotated
    xs = [(torch.randn(rows, cols, device=c.dev) * 2).half() for _ in range(R)]
    ys = [torch.empty_like(xs[0]) for _ in range(R)]
    gam = (1 + 0.1 * torch.randn(cols, device=c.dev)).half()
    beta = (0.1 * torch.randn(cols, device=c.dev)).half()
    mean = torch.empty(rows, dtype=torch.float32, device=c.dev)
    rstd = torch.empty(rows, dtype=torch.float32, device=c.dev)
    xp = [t.data_ptr() for t in xs]
    yp = [t.data_ptr() for t in ys]
    gp, bp, st = gam.data_ptr(), beta.data_ptr(), c.stream

    def softmax(i):
        hxm.check(L.hxm_softmax_rows(xp[i], cols, yp[i], cols, rows, cols, hxm.F16, st),
                  "hxm_softmax_rows")

    def rms(i):
        hxm.check(L.hxm_rmsnorm_rows(xp[i], cols, gp, yp[i], cols, rows, cols, 1e-6, hxm.F16,
                                     st), "hxm_rmsnorm_rows")
    def layernorm(i):  # with the saved mean / rstd (layer_norm_fwd_kernel's outputs)
        hxm.check(L.hxm_layernorm_rows(xp[i], cols, gp, bp, yp[i], cols, mean.data_ptr(),
                                       rstd.data_ptr(), rows, cols, 1e-5, hxm.F16, st),
                  "hxm_layernorm_rows")
    def copy(i):  # the ceiling: this library's streaming copy of the same bytes
        hxm.check(L.hxm_probe_copy(xp[i], yp[i], rows * cols * 2, st), "hxm_probe_copy")
    out = {}
    t = c.time_ms(copy, 200, 20, rotate=R)
    ceil_gbs = 2 * rows * cols * 2 / (t.median * 1e-3) / 1e9
    copy_graph_us = c.graph_time(copy, 200, rotate=R) * 1e3
    out["hbm_ceiling_copy_64MiB"] = {**t.us(), "GB/s": ceil_gbs, "graph_us": copy_graph_us,
                                     "hbm_frac": ceil_gbs / PEAK_HBM_GBS,
                                     "bytes": 2 * rows * cols * 2,
                                     "what": "hxm_probe_copy of one 64 MiB row set (read + "
                                             "write), 4 sets rotated"}
    for name, fn, nbytes in (("softmax_f16_8192x4096", softmax, 2 * rows * cols * 2),
                             ("rmsnorm_f16_8192x4096", rms, 2 * rows * cols * 2 + cols * 2),
                             ("layernorm_f16_8192x4096", layernorm,
                              2 * rows * cols * 2 + 2 * cols * 2 + 2 * rows * 4)):
        t = c.time_ms(fn, 200, 20, rotate=R)
        gbs = nbytes / (t.median * 1e-3) / 1e9
        g_us = c.graph_time(fn, 200, rotate=R) * 1e3
        out[name] = {**t.us(), "GB/s": gbs, "hbm_frac": gbs / PEAK_HBM_GBS,
                     "ceiling_frac": gbs / ceil_gbs, "bytes": nbytes, "graph_us": g_us,
                     "graph_hbm_frac": nbytes / (g_us * 1e-6) / 1e9 / PEAK_HBM_GBS,
                     "graph_ceiling_frac": copy_graph_us / g_us * nbytes / (2 * rows * cols * 2)}
    return out


def run_ffn(c):
    """The SwiGLU FFN block, tokens 2048, hidden 4096,
    intermediate 11008.  RMSNorm (eps 1e-6) -> fused gate/up W8A16 GEMM with
    SiLU * mul -> down W8A16 GEMM; fp16 activations N(0,1), int8 weights
    U{-127..127} with per-channel scales.  Each GEMM's tile is autotuned on
    these operands first (outside the timed region); a step is the whole
    block."""
    import math
    torch, hxm, L, ops = c.torch, c.hxm, c.L, c.ops
    T, H, I = 2048, 4096, 11008
    x = torch.randn(T, H, device=c.dev).half()
    gamma = (1 + 0.1 * torch.randn(H, device=c.dev)).half()
    Wg = torch.randint(-127, 128, (I, H), dtype=torch.int8, device=c.dev)
    Wu = torch.randint(-127, 128, (I, H), dtype=torch.int8, device=c.dev)
    Wd = torch.randint(-127, 128, (H, I), dtype=torch.int8, device=c.dev)
    sc_h, sc_i = 1 / math.sqrt(H * 127 ** 2 / 3), 1 / math.sqrt(I * 127 ** 2 / 3)
    sg = ((torch.rand(I, device=c.dev) + 0.5) * sc_h).half().float()
    su = ((torch.rand(I, device=c.dev) + 0.5) * sc_h).half().float()
    sd = ((torch.rand(H, device=c.dev) + 0.5) * sc_i).half().float()
    Wgu, sgu = ops.swiglu_pack(Wg, Wu, sg, su)
    xn = torch.empty_like(x)
    h = torch.empty(T, I, dtype=torch.float16, device=c.dev)
    y = torch.empty(T, H, dtype=torch.float16, device=c.dev)
    ops.rms_norm(x, (H,), gamma, eps=1e-6, out=xn)
    cfg_gu, _ = ops.tune_w8a16(xn, Wgu, sgu, h, swiglu=True, reps=5)
    cfg_d, _ = ops.tune_w8a16(h, Wd, sd, y, reps=5)
    st = c.stream
    px, pg, pxn, ph, py = x.data_ptr(), gamma.data_ptr(), xn.data_ptr(), h.data_ptr(), y.data_ptr()
    pgu, psgu, pwd, psd = Wgu.data_ptr(), sgu.data_ptr(), Wd.data_ptr(), sd.data_ptr()

    def norm(_):
        hxm.check(L.hxm_rmsnorm_rows(px, H, pg, pxn, H, T, H, 1e-6, hxm.F16, st),
                  "hxm_rmsnorm_rows")

    def gateup(_):
        hxm.check(L.hxm_gemm_w8a16_swiglu(pxn, H, pgu, psgu, ph, I, T, I, H, None, st),
                  "hxm_gemm_w8a16_swiglu")

    def down(_):
        hxm.check(L.hxm_gemm_w8a16(ph, I, pwd, I, psd, py, H, T, H, I, None, st),
                  "hxm_gemm_w8a16")

    yr = torch.empty_like(y)

    def down_residual(_):  # y = x + down(h): the residual added in the down GEMM's epilogue
        hxm.check(L.hxm_gemm_w8a16_residual(ph, I, pwd, I, psd, px, H, yr.data_ptr(), H, T, H, I,
                                            None, st), "hxm_gemm_w8a16_residual")

    def block(i):
        norm(i), gateup(i), down(i)

    def block_residual(i):
        norm(i), gateup(i), down_residual(i)
    steps, warm = 50, 5
    tb = c.time_ms(block, steps, warm, reps=5)
    t_blk = tb.median
    t_norm = c.time_ms(norm, steps, warm, reps=2).median
    t_gu = c.time_ms(gateup, steps, warm, reps=2).median
    t_d = c.time_ms(down, steps, warm, reps=2).median
    t_dr = c.time_ms(down_residual, steps, warm, reps=2).median
    t_blkr = c.time_ms(block_residual, steps, warm, reps=2).median
    t_blk_graph = c.graph_time(block, 20)  # the three launches per block, 20 blocks per graph
    f_gu, f_d = 2.0 * T * H * (2 * I), 2.0 * T * I * H
    flops = f_gu + f_d
    tf = flops / (t_blk * 1e-3) / 1e12
    clk = sclk_under_load(c, block, what="the FFN block")
    return {"swiglu_ffn_2048x4096x11008": {
        **tb.us(), "TFLOPS": tf, "mfma_frac": tf / PEAK_F16_TFLOPS,
        "sclk_under_load": clk,
        "mfma_frac_at_measured_sclk": (tf / (PEAK_F16_TFLOPS * clk["median_mhz"] / 2400.0)
                                       if clk else None),
        "gemm_flops": flops,
        "stages_us": {"rmsnorm": t_norm * 1e3, "gate_up_swiglu": t_gu * 1e3, "down": t_d * 1e3,
                      "down_with_residual": t_dr * 1e3},
        "block_with_residual_us": t_blkr * 1e3,
        "graph_us": t_blk_graph * 1e3,
        "graph_TFLOPS": flops / (t_blk_graph * 1e-3) / 1e12,
        "stage_TFLOPS": {"gate_up_swiglu": f_gu / (t_gu * 1e-3) / 1e12,
                         "down": f_d / (t_d * 1e-3) / 1e12},
        "tuned": {"gate_up_swiglu": list(cfg_gu.as_tuple()), "down": list(cfg_d.as_tuple())}}}


def run_shard(c):
    """One GPU's share of an 8-way tensor-parallel split of configs 3 and 5
    (measured alone: no second GPU, and the all-reduce of the block's
    [2048, 4096] partial output is not built).  The GEMV keeps N / 8 = 1376
    output channels of W (5.6 MB per image, so 96 images rotate past the
    256 MB Infinity Cache); the FFN block keeps I / 8 = 1376 intermediate
    channels: gate/up column-parallel (its SwiGLU image interleaves 64-channel
    blocks, the last one half padding), down row-parallel over the same
    slice.  Tiles are tuned per GEMM at these shapes."""
    import math
    torch, hxm, L, ops = c.torch, c.hxm, c.L, c.ops
    out = {}
    N, K, R = 11008 // 8, 4096, 96
    Ws = [ops.prepack_w8a16(torch.randint(-127, 128, (N, K), dtype=torch.int8, device=c.dev))
          for _ in range(R)]
    scs = [(torch.rand(N, device=c.dev) * 0.019 + 0.001).half() for _ in range(R)]
    wp = [w.data_ptr() for w in Ws]
    sp = [s.data_ptr() for s in scs]
    for M in (1, 4, 16):
        xs = torch.randn(M, K, device=c.dev).half()
        ys = torch.empty(M, N, dtype=torch.float16, device=c.dev)
        px, py, st = xs.data_ptr(), ys.data_ptr(), c.stream

        def step(i, M=M, px=px, py=py):
            hxm.check(L.hxm_gemv_w8a16(px, K, wp[i], K, hxm.W_PACKED, sp[i], py, N, M, N, K,
                                       st), "hxm_gemv_w8a16")
        t = c.time_ms(step, 480, 48, rotate=R)
        nbytes = N * K + N * 2 + M * K * 2 + M * N * 2
        gbs = nbytes / (t.median * 1e-3) / 1e9
        out[f"tp8_shard_w8a16_gemv_M{M}"] = {
            **t.us(), "GB/s": gbs, "hbm_frac": gbs / PEAK_HBM_GBS, "bytes": nbytes,
            "graph_us": c.graph_time(step, 480, rotate=R) * 1e3,
            "shape": f"M={M} N={N} K={K} (config 3, N split 8 ways)",
            "note": "a kernel this short is shorter than one host launch: us is the host's "
                    "launch rate, graph_us the device time per launch"}
    del Ws, scs
    T, H, I = 2048, 4096, 11008 // 8
    x = torch.randn(T, H, device=c.dev).half()
    gamma = (1 + 0.1 * torch.randn(H, device=c.dev)).half()
    Wg = torch.randint(-127, 128, (I, H), dtype=torch.int8, device=c.dev)
    Wu = torch.randint(-127, 128, (I, H), dtype=torch.int8, device=c.dev)
    Wd = torch.randint(-127, 128, (H, I), dtype=torch.int8, device=c.dev)
    sc_h, sc_i = 1 / math.sqrt(H * 127 ** 2 / 3), 1 / math.sqrt(11008 * 127 ** 2 / 3)
    sg = ((torch.rand(I, device=c.dev) + 0.5) * sc_h).half().float()
    su = ((torch.rand(I, device=c.dev) + 0.5) * sc_h).half().float()
    sd = ((torch.rand(H, device=c.dev) + 0.5) * sc_i).half().float()
    Wgu, sgu = ops.swiglu_pack(Wg, Wu, sg, su)
    xn = torch.empty_like(x)
    h = torch.empty(T, I, dtype=torch.float16, device=c.dev)
    y = torch.empty(T, H, dtype=torch.float16, device=c.dev)
    ops.rms_norm(x, (H,), gamma, eps=1e-6, out=xn)
    cfg_gu, _ = ops.tune_w8a16(xn, Wgu, sgu, h, swiglu=True, reps=5)
    cfg_d, _ = ops.tune_w8a16(h, Wd, sd, y, reps=5)
    st = c.stream
    px, pg, pxn, ph, py = x.data_ptr(), gamma.data_ptr(), xn.data_ptr(), h.data_ptr(), y.data_ptr()
    pgu, psgu, pwd, psd = Wgu.data_ptr(), sgu.data_ptr(), Wd.data_ptr(), sd.data_ptr()

    def norm(_):
        hxm.check(L.hxm_rmsnorm_rows(px, H, pg, pxn, H, T, H, 1e-6, hxm.F16, st),
                  "hxm_rmsnorm_rows")

    def gateup(_):
        hxm.check(L.hxm_gemm_w8a16_swiglu(pxn, H, pgu, psgu, ph, I, T, I, H, None, st),
                  "hxm_gemm_w8a16_swiglu")

    def down(_):
        hxm.check(L.hxm_gemm_w8a16(ph, I, pwd, I, psd, py, H, T, H, I, None, st),
                  "hxm_gemm_w8a16")

    def block(i):
        norm(i), gateup(i), down(i)
    tb = c.time_ms(block, 100, 10, reps=5)
    t_gu = c.time_ms(gateup, 100, 10, reps=2).median
    t_d = c.time_ms(down, 100, 10, reps=2).median
    f_gu, f_d = 2.0 * T * H * (2 * I), 2.0 * T * I * H
    tf = (f_gu + f_d) / (tb.median * 1e-3) / 1e12
    out["tp8_shard_swiglu_ffn_2048x4096x1376"] = {
        **tb.us(), "TFLOPS": tf, "mfma_frac": tf / PEAK_F16_TFLOPS, "gemm_flops": f_gu + f_d,
        "stages_us": {"gate_up_swiglu": t_gu * 1e3, "down": t_d * 1e3},
        "stage_TFLOPS": {"gate_up_swiglu": f_gu / (t_gu * 1e-3) / 1e12,
                         "down": f_d / (t_d * 1e-3) / 1e12},
        "graph_us": c.graph_time(block, 20) * 1e3,
        "tuned": {"gate_up_swiglu": list(cfg_gu.as_tuple()), "down": list(cfg_d.as_tuple())},
        "shape": "tokens 2048, hidden 4096, intermediate 1376 (config 5, intermediate split 8 "
                 "ways; the all-reduce of the partial output is not built)"}
    return out


def run_ragged(c):
    """Tail tiles, a partial last K stage and an N-split store: int8 GEMM
    M=N=4000, K=4000 (K bytes not a multiple of the 128-byte stage) with
    dequant, C written into columns [0, 4000) of a [4000, 4096] buffer
    (ldc = 4096)."""
    torch, hxm, L = c.torch, c.hxm, c.L
    M = N = K = 4000
    A = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=c.dev)
    Bp = c.ops.prepack_weight(torch.randint(-127, 128, (K, N), dtype=torch.int8, device=c.dev))
    rs = torch.rand(M, device=c.dev) * 0.019 + 0.001
    cs = torch.rand(N, device=c.dev) * 0.019 + 0.001
    C = torch.empty(M, 4096, dtype=torch.float16, device=c.dev)
    a, b, r, s, o, st = A.data_ptr(), Bp.data_ptr(), rs.data_ptr(), cs.data_ptr(), C.data_ptr(), c.stream
    ldb = Bp.stride(0)                          # the image's rows are padded to 128 bytes

    def step(_):
        hxm.check(L.hxm_gemm_i8_dequant(a, K, b, ldb, hxm.B_NK, r, s, o, 4096, M, N, K, None, st),
                  "hxm_gemm_i8_dequant")
    t = c.time_ms(step, 200, 200)
    ops_per = 2.0 * M * N * K
    return {"int8_gemm_dequant_ragged_4000_ldc4096": {
        **t.us(), "TOPS": ops_per / (t.median * 1e-3) / 1e12,
        "mfma_frac": ops_per / (t.median * 1e-3) / 1e12 / PEAK_INT8_TOPS}}


def run_vendor(c):
    """Context, not the product: the vendor library (hipBLASLt behind
    torch._int_mm / torch.matmul) on the same shapes, next to this library's
    f16 4096^3 matmul with a resident B."""
    torch, hxm, L = c.torch, c.hxm, c.L
    n = 4096
    A = torch.randint(-127, 128, (n, n), dtype=torch.int8, device=c.dev)
    Bt = torch.randint(-127, 128, (n, n), dtype=torch.int8, device=c.dev).t()  # column-major
    Ah = (torch.rand(n, n, device=c.dev) * 2 - 1).half()
    Bh = (torch.rand(n, n, device=c.dev) * 2 - 1).half()
    Bnk = Bh.t().contiguous()                       # resident [N, K] image of B
    Ch = torch.empty(n, n, dtype=torch.float16, device=c.dev)
    out = {}
    ms = c.time_ms(lambda i: torch._int_mm(A, Bt), 100, 10).median
    out["vendor_int_mm_4096"] = {"us": ms * 1e3, "TOPS": 2 * n ** 3 / (ms * 1e-3) / 1e12,
                                 "what": "torch._int_mm (hipBLASLt), int8 -> int32, B column-major"}
    ms = c.time_ms(lambda i: torch.matmul(Ah, Bnk.t()), 100, 10).median
    out["vendor_f16_matmul_4096"] = {"us": ms * 1e3, "TFLOPS": 2 * n ** 3 / (ms * 1e-3) / 1e12,
                                     "what": "torch.matmul (hipBLASLt), f16, B = [N,K] transposed view"}
    pa, pb, pc, st = Ah.data_ptr(), Bnk.data_ptr(), Ch.data_ptr(), c.stream

    def f16(_):
        hxm.check(L.hxm_matmul(pa, n, pb, n, hxm.B_NK, pc, n, n, n, n, hxm.F16, hxm.F16, 0,
                               None, st), "hxm_matmul")
    ms = c.time_ms(f16, 100, 10).median
    tf = 2 * n ** 3 / (ms * 1e-3) / 1e12
    clk = sclk_under_load(c, f16, what="the f16 4096^3 matmul")
    out["f16_matmul_4096"] = {"us": ms * 1e3, "TFLOPS": tf, "mfma_frac": tf / PEAK_F16_TFLOPS,
                              "sclk_under_load": clk,
                              "mfma_frac_at_measured_sclk":
                                  tf / (PEAK_F16_TFLOPS * clk["median_mhz"] / 2400.0) if clk else None}
    return out


def run_search(c):
    """The measured tile search (hxm_tune_gemm) on the 4096^3 shapes: every
    compiled config -- both wave grids of the large tiles -- timed and checked
    against the control (the untuned default); then the winner and the
    default are timed with the headline's protocol (the int8 one with the
    dequant epilogue).  The tuning cache is cleared afterwards, so nothing
    else in this bench runs a tuned tile."""
    import ctypes
    torch, hxm, L, ops = c.torch, c.hxm, c.L, c.ops
    n = 4096
    out = {}
    A, Bp, rs, cs = int8_operands(c)
    Ah = (torch.rand(n, n, device=c.dev) * 2 - 1).half()
    Bh = ops.prepack_weight((torch.rand(n, n, device=c.dev) * 2 - 1).half())
    C32 = torch.empty(n, n, dtype=torch.int32, device=c.dev)
    C16 = torch.empty(n, n, dtype=torch.float16, device=c.dev)
    st = c.stream
    for name, a, b, cc in (("int8", A, Bp, C32), ("f16", Ah, Bh, C16)):
        best, rep = ops.tune_gemm(a, b, cc, reps=10)
        ctl = rep["configs"][rep["control"]]
        control = hxm.GemmConfig(*ctl["tiles"], *ctl["waves"], ctl["stages"], ctl["split_k"])

        def step(_, cfg=None):
            if name == "int8":
                hxm.check(L.hxm_gemm_i8_dequant(a.data_ptr(), n, b.data_ptr(), n, hxm.B_NK,
                                                rs.data_ptr(), cs.data_ptr(), C16.data_ptr(), n,
                                                n, n, n, ctypes.byref(cfg), st), "dequant")
            else:
                hxm.check(L.hxm_matmul(a.data_ptr(), n, b.data_ptr(), n, hxm.B_NK,
                                       C16.data_ptr(), n, n, n, n, hxm.F16, hxm.F16, 0,
                                       ctypes.byref(cfg), st), "matmul")
        t_best = c.time_ms(lambda i: step(i, best), 100, 200, reps=4)
        t_ctl = c.time_ms(lambda i: step(i, control), 100, 200, reps=4)
        work = 2.0 * n ** 3
        out[f"search_{name}_4096"] = {
            "winner": list(best.as_tuple()), "default": list(control.as_tuple()),
            "winner_us": t_best.median * 1e3, "default_us": t_ctl.median * 1e3,
            "winner_rate": work / (t_best.median * 1e-3) / 1e12,
            "default_rate": work / (t_ctl.median * 1e-3) / 1e12,
            "proof": rep.get("proof"), "start": rep.get("start"),
            "configs": [{"tiles": r["tiles"], "waves": r["waves"], "stages": r["stages"],
                         "q50_us": r["q50"], "verified": r["verified"]}
                        for r in rep["configs"]],
            "what": "hxm_tune_gemm over every compiled config (" + name + " -> " +
                    ("int32" if name == "int8" else "f16") + "); winner and default then "
                    "timed on the " + ("dequant GEMM" if name == "int8" else "f16 matmul")}
    L.hxm_tune_cache_clear()
    return out


def run_mfma_ceilings(c, A, Bp):
    """The practical MFMA ceiling of the MFMA-bound configs: hxm_probe_mfma
    runs the same number of 32x32 MFMAs as the GEMM, one workgroup of four
    waves per CU (the GEMM kernels' occupancy), on the GEMM's own operand
    bytes, with no staging and no epilogue.  The chip is power-limited, so
    with real data this is well below the nominal peak; each GEMM's
    ceiling_frac is probe time / GEMM time."""
    torch, hxm, L = c.torch, c.hxm, c.L
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    waves = 4 * cus
    sink = torch.empty(8192, dtype=torch.int32, device=c.dev)
    g = torch.Generator().manual_seed(11)
    xh = torch.randn(2048, 4096, generator=g).half().to(c.dev)     # FFN activations N(0, 1)
    wq = torch.randint(-127, 128, (11008, 4096), generator=g, dtype=torch.int8).to(c.dev)
    ah = (torch.rand(4096, 4096, generator=g) * 2 - 1).half().to(c.dev)
    bh = (torch.rand(4096, 4096, generator=g) * 2 - 1).half().to(c.dev)
    n = 4096
    cases = (
        ("int8_gemm_4096", A, Bp, hxm.I8, hxm.I8, 2.0 * n ** 3, 32 * 32 * 32 * 2, "TOPS"),
        ("f16_matmul_4096", ah, bh, hxm.F16, hxm.F16, 2.0 * n ** 3, 32 * 32 * 16 * 2, "TFLOPS"),
        ("swiglu_ffn_2048x4096x11008", xh, wq, hxm.F16, hxm.I8,
         2.0 * 2048 * 4096 * (2 * 11008) + 2.0 * 2048 * 11008 * 4096, 32 * 32 * 16 * 2, "TFLOPS"),
    )
    out = {}
    for name, a, b, adt, bdt, work, per_mfma, unit in cases:
        per_wave = int(-(-work // per_mfma // waves))
        per_wave = -(-per_wave // 32) * 32
        pa, pb, na, nb = a.data_ptr(), b.data_ptr(), a.numel() * a.element_size(), \
            b.numel() * b.element_size()

        def step(_, pa=pa, pb=pb, na=na, nb=nb, adt=adt, bdt=bdt, per_wave=per_wave):
            hxm.check(L.hxm_probe_mfma(pa, na, pb, nb, adt, bdt, per_wave, cus, sink.data_ptr(),
                                       c.stream), "hxm_probe_mfma")
        t = c.time_ms(step, 100 if work < 2e12 else 20, 200 if work < 2e12 else 20, reps=4)
        done = per_wave * waves * per_mfma
        out[f"mfma_ceiling_{name}"] = {
            **t.us(), unit: done / (t.median * 1e-3) / 1e12, "mfma_per_wave": per_wave,
            "workgroups": cus, "work": done,
            "what": "hxm_probe_mfma: the GEMM's MFMA count on its own operand bytes, nothing "
                    "else"}
    return out


def run_copy(c):
    """A plain 256 MiB device copy (torch's elementwise copy kernel): the
    known-size reference that scales rocprofv3 FETCH_SIZE / WRITE_SIZE."""
    torch = c.torch
    src = torch.empty(1 << 28, dtype=torch.uint8, device=c.dev).fill_(1)
    dst = torch.empty_like(src)
    ms = c.time_ms(lambda i: dst.copy_(src), c.args.steps, c.args.warmup).median
    return {"copy_256MiB": {"us": ms * 1e3, "bytes_read": 1 << 28, "bytes_written": 1 << 28,
                            "GB/s": 2 * (1 << 28) / (ms * 1e-3) / 1e9}}


def measured_traffic():
    """HBM bytes per launch of the headline kernel from its committed rocprofv3
    summary (FETCH_SIZE and WRITE_SIZE passes, scaled by the copy
    calibration); None when the summary is absent."""
    path = os.path.join(ROOT, "profiles", "int8_gemm_4096_dequant.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def cpu_model():
    """The host CPU's model name (what lscpu reports as "Model name") and the
    vector extensions it exposes that the int8 loop can use."""
    name, isa = None, []
    try:
        for line in open("/proc/cpuinfo"):
            key = line.split(":", 1)[0].strip().lower()
            if key == "model name" and name is None:
                name = line.split(":", 1)[1].strip()
            elif key == "flags" and not isa:
                flags = set(line.split(":", 1)[1].split())
                isa = [f for f in ("avx2", "avx512f", "avx512bw", "avx512_vnni", "avx_vnni")
                       if f in flags]
    except OSError:
        pass
    return name, isa


def cpu_baselines(A, Bp, seconds):
    """The C restatement (oracle/oracle.c) of every benchmark config (the five
    workloads of `configs` in the JSON line), timed on
    the host cores: one build of it for this host (gcc -O3 -march=native
    -fopenmp, `make native` in oracle/; the checker's portable build when
    that fails), one thread count for every op (OMP_NUM_THREADS, else the
    host's CPUs), each op on a bounded sample of its config's workload with
    the config's shapes and value distributions (seeded numpy data; the int8
    GEMM takes rows of the GPU run's own operands).  A sample's time is the
    median of a few runs after one untimed call.  Returns the common record
    (build, threads, CPU model) and one {value, unit, sample, s} per config."""
    import contextlib
    import numpy as np
    from oracle import oracle as orc
    native, why = orc.native_lib()
    march = "native" if native is not None else f"x86-64-v3 (native build failed: {why})"
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)
    threads = max(1, min(threads, os.cpu_count() or 1))
    model, isa = cpu_model()
    rng = np.random.default_rng(2024)
    budget = max(0.2, seconds / 8)          # seconds of timed CPU work per op

    def f16(a):
        return np.asarray(a, dtype=np.float32).astype(np.float16).view(np.uint16)

    def timed(fn, reps=3):
        fn()                                # untimed: page-in, thread pool
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    def rows_for(fn_rows, total, unit_work_s=None):
        """Rows of a row-independent op that take about `budget` seconds."""
        t0 = time.perf_counter()
        fn_rows(min(4, total))
        per_row = max(time.perf_counter() - t0, 1e-6) / min(4, total)
        return int(min(total, max(4, budget / per_row)))

    out = {}
    ctx = orc.using(native) if native is not None else contextlib.nullcontext()
    with ctx:
        # 2: int8 GEMM 4096^3 -> int32 (the dequant is elementwise and left out)
        Ah, Bh = A.cpu().numpy(), Bp.cpu().numpy()
        M, K = Ah.shape
        N = Bh.shape[0]
        r = rows_for(lambda n: orc.gemm_i8(Ah[:n], Bh, b_nk=True, threads=threads), M)
        t = timed(lambda: orc.gemm_i8(Ah[:r], Bh, b_nk=True, threads=threads))
        out[2] = {"value": 2.0 * r * N * K / t / 1e12, "unit": "TOPS", "s": t,
                  "sample": f"int8 GEMM rows 0..{r - 1} of A[{M},{K}] x resident B[{N},{K}] "
                            f"-> int32"}
        # 1: f16 matmul 256^3, the whole matmul
        a = f16(rng.uniform(-1, 1, (256, 256)))
        b = f16(rng.uniform(-1, 1, (256, 256)))
        t = timed(lambda: orc.matmul(a, b, threads=threads), reps=5)
        out[1] = {"value": 2.0 * 256 ** 3 / t / 1e12, "unit": "TFLOPS", "s": t,
                  "sample": "the whole f16 256^3 matmul (fp32 accumulate, f16 out)"}
        # 3: W8A16 GEMV, N=11008, K=4096, M in {1, 4, 16}: the whole GEMV
        Nw, Kw = 11008, 4096
        W = rng.integers(-127, 128, (Nw, Kw), dtype=np.int8)
        sc = f16(rng.uniform(0.001, 0.02, Nw))
        for Mv in (1, 4, 16):
            x = f16(rng.standard_normal((Mv, Kw)))
            t = timed(lambda: orc.gemv_w8a16(x, W, sc, threads=threads), reps=5)
            nbytes = Nw * Kw + Nw * 2 + Mv * Kw * 2 + Mv * Nw * 2
            out[f"3_M{Mv}"] = {"value": nbytes / t / 1e9, "unit": "GB/s", "s": t,
                               "sample": f"the whole GEMV M={Mv} N={Nw} K={Kw}"}
        del W
        # 4: softmax / RMSNorm rows, f16 [8192, 4096], values N(0, 2)
        R, C = 8192, 4096
        xr = f16(rng.standard_normal((R, C)) * 2)
        gam = f16(1 + 0.1 * rng.standard_normal(C))
        for name, fn in (("softmax", lambda n: orc.softmax_rows(xr[:n], "f16", threads)),
                         ("rmsnorm", lambda n: orc.rmsnorm_rows(xr[:n], gam, 1e-6, "f16",
                                                                threads))):
            r = rows_for(fn, R)
            t = timed(lambda: fn(r))
            out[f"4_{name}"] = {"value": 2.0 * r * C * 2 / t / 1e9, "unit": "GB/s", "s": t,
                                "sample": f"{name} rows 0..{r - 1} of f16 [{R}, {C}]"}
        del xr
        # 5: SwiGLU FFN block (tokens 2048, hidden 4096, intermediate 11008) on
        # a token-row sample, scaled per row (rows are independent)
        T, H, I = 2048, 4096, 11008
        x = f16(rng.standard_normal((T, H)))
        g5 = f16(1 + 0.1 * rng.standard_normal(H))
        Wg = rng.integers(-127, 128, (I, H), dtype=np.int8)
        Wu = rng.integers(-127, 128, (I, H), dtype=np.int8)
        Wd = rng.integers(-127, 128, (H, I), dtype=np.int8)
        sh, si = 1 / np.sqrt(H * 127 ** 2 / 3), 1 / np.sqrt(I * 127 ** 2 / 3)
        sg = ((rng.random(I) + 0.5) * sh).astype(np.float16).astype(np.float32)
        su = ((rng.random(I) + 0.5) * sh).astype(np.float16).astype(np.float32)
        sd = ((rng.random(H) + 0.5) * si).astype(np.float16).astype(np.float32)

        def ffn(n):
            return orc.swiglu_ffn(x[:n], g5, Wg, Wu, sg, su, Wd, sd, threads=threads)
        r = rows_for(ffn, T)
        t = timed(lambda: ffn(r))
        flops_row = 2.0 * H * 2 * I + 2.0 * I * H
        out[5] = {"value": flops_row * r / t / 1e12, "unit": "TFLOPS", "s": t,
                  "sample": f"the block on token rows 0..{r - 1} of {T}"}
    common = {"cores": threads, "kind": "port", "cpu_model": model, "cpu_isa": isa,
              "host_threads": os.cpu_count(), "march": march,
              "what": "oracle/oracle.c (the C restatement), gcc -O3 -march=" +
                      march.split()[0] + " -fopenmp"}
    return common, out


def sclk_under_load(c, fn, seconds=1.0, what="the headline GEMM"):
    """Shader clock (MHz) while `fn` runs back to back for about `seconds`:
    rocm-smi is sampled from a host thread during the loop.  Returns the
    median sample and the raw samples, or None when rocm-smi gives nothing.

    Under a profiler (rocprofv3 preloads its library into every child
    process, and that library initialises the GPU) rocm-smi is not started:
    its launcher script hands over to python3 by exec, which must not happen
    in a process that has initialised the GPU.  The record then says so."""
    import re
    import subprocess
    import threading
    if any(k.startswith("ROCPROF") for k in os.environ) or \
            "rocprofiler" in os.environ.get("LD_PRELOAD", ""):
        log(f"clock sampling skipped under a profiler ({what})")
        return None
    samples, stop = [], threading.Event()

    def sample():
        while not stop.is_set():
            try:
                out = subprocess.run(["rocm-smi", "--showclocks"], capture_output=True,
                                     text=True, timeout=5).stdout
            except (OSError, subprocess.SubprocessError):
                return
            m = re.search(r"sclk clock level:\s*\d+:\s*\(?(\d+)\s*Mhz", out, re.I)
            if m:
                samples.append(int(m.group(1)))
            time.sleep(0.05)

    fn(0)
    c.torch.cuda.synchronize()
    th = threading.Thread(target=sample, daemon=True)
    th.start()
    t0 = time.perf_counter()
    i = 0
    while time.perf_counter() - t0 < seconds:
        for _ in range(200):
            fn(i)
            i += 1
        c.torch.cuda.synchronize()
    stop.set()
    th.join(timeout=10)
    if not samples:
        return None
    steady = samples[len(samples) // 2:]  # the first samples still see the ramp from idle
    return {"median_mhz": statistics.median(steady), "samples_mhz": samples,
            "source": f"rocm-smi --showclocks sampled while {what} runs back to back"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # The shader clock ramps up over the first ~1000 back-to-back launches
    # (~60 ms) of the headline GEMM; 2000 untimed launches (~0.12 s) put the
    # timed region at the steady-state clock a continuously running
    # deployment sees.
    ap.add_argument("--warmup", type=int, default=2000)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="approximate CPU time of the cpu_baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--only", choices=["int8", "int8_i32", "f16", "ragged", "gemv", "rows", "ffn",
                                       "shard", "copy", "vendor", "search", "ceilings"])
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build is the single-GPU kernel set of the hot "
              "path and has no multi-GPU path; the design notes describe how it would shard.",
              file=sys.stderr)
        return 2
    c = Ctx(args)

    if args.only:
        if args.only in ("int8", "int8_i32"):
            rec = {args.only: run_int8(c, *int8_operands(c), out_i32=args.only == "int8_i32")}
        elif args.only == "ceilings":
            rec = run_mfma_ceilings(c, *int8_operands(c)[:2])
        else:
            rec = {"f16": run_f16, "ragged": run_ragged, "gemv": run_gemv, "rows": run_rows,
                   "ffn": run_ffn, "shard": run_shard, "copy": run_copy, "vendor": run_vendor,
                   "search": run_search}[
                args.only](c)
        print(json.dumps(rec), flush=True)
        return 0

    A, Bp, rs, cs = int8_operands(c)
    legs = {}
    if not args.no_extra:
        legs["int8_gemm_i32_out_4096"] = run_int8(c, A, Bp, rs, cs, out_i32=True)
        try:
            legs.update(run_mfma_ceilings(c, A, Bp))
        except Exception as e:
            log(f"run_mfma_ceilings failed: {e!r}")
            legs["run_mfma_ceilings"] = {"error": repr(e)}
        for fn in (run_f16, run_ragged, run_gemv, run_rows, run_ffn, run_shard, run_copy,
                   run_vendor, run_search):
            try:
                legs.update(fn(c))
            except Exception as e:  # a failed context leg is reported, the headline still runs
                log(f"{fn.__name__} failed: {e!r}")
                legs[fn.__name__] = {"error": repr(e)}
        for k, v in legs.items():   # every leg in full, on stderr
            log(k, json.dumps(v))
    # The headline last: the legs above have brought the clock to its
    # steady state under load (see the module docstring).
    head = run_int8(c, A, Bp, rs, cs)
    log("int8 gemm+dequant 4096^3:", json.dumps(head))
    clk = sclk_under_load(c, c.last_step)
    log("sclk under load:", json.dumps(clk))
    cpu_common, cpu = None, {}
    if not args.no_cpu_baseline:
        try:
            cpu_common, cpu = cpu_baselines(A, Bp, args.cpu_seconds)
        except Exception as e:  # the CPU baseline is reported, not required for the line
            log(f"cpu_baselines failed: {e!r}")
    log("cpu baselines", json.dumps([cpu_common, {str(k): v for k, v in cpu.items()}]))

    f16l, f16c = legs.get("f16_matmul_4096", {}), legs.get("mfma_ceiling_f16_matmul_4096", {})
    if "us" in f16l and "q50_us" in f16c:
        f16l["ceiling_frac"] = f16c["q50_us"] / f16l["us"]
    tops = head["TOPS"]
    cpu2 = cpu.get(2)
    out = {
        "metric": "int8 GEMM 4096^3 TOPS (int32 accumulate, fp16 dequant) + % MFMA peak",
        "value": tops,
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["q50_us"] / 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded U{-127..127} int8, U[0.001,0.02] fp32 scales)",
        "config": {"workload": "int8 GEMM M=N=K=4096, int32 accumulate, per-row x per-col "
                               "fp32 scales dequant to fp16; B resident [N,K] image",
                   "M": 4096, "N": 4096, "K": 4096, "parallelism": "single-gpu"},
        "roofline": {"bound": "mfma", "achieved": tops, "peak": PEAK_INT8_TOPS,
                     "unit": "TFLOP/s", "frac": tops / PEAK_INT8_TOPS,
                     "traffic": measured_traffic(),
                     "traffic_source": "profiles/int8_gemm_4096_dequant.md",
                     "kernel": "gemm_kernel<int8_t,256,256,128,2,2,2,kEpiDequant>",
                     "work_per_launch": head["ops_per_launch"],
                     "avg_launch_us": head["q50_us"], "span_us": head["span_us"],
                     "q20_us": head["q20_us"], "q50_us": head["q50_us"],
                     "q80_us": head["q80_us"], "reps": head["reps"],
                     "achieved_basis": "work / q50 of the time per launch over 1 + 10 timed "
                                       "regions of K back-to-back launches (one event pair "
                                       "each); span_us is the first region alone",
                     "sclk_mhz_under_load": clk["median_mhz"] if clk else None,
                     "frac_at_measured_sclk": (tops / (PEAK_INT8_TOPS * clk["median_mhz"] / 2400.0)
                                               if clk else None)},
        "cpu_baseline": ({**cpu_common, "value": cpu2["value"], "unit": cpu2["unit"],
                          "sample": cpu2["sample"]} if cpu2 else None),
        "configs": config_records(head, legs, cpu),
        "extra": compact_extra(legs),
    }
    line = json.dumps(out)
    log(f"result line: {len(line)} bytes")
    print(line, flush=True)
    return 0


def _r(v, nd=4):
    """Rounded for the compact record (None and strings pass through)."""
    return round(v, nd) if isinstance(v, float) else v


def config_records(head, legs, cpu):
    """One compact record per benchmark config (the reference's per-test
    Test_Info {Name, Result, Perf, Units}, test/utils/dsp/include/
    test_report.h:35-70): q20 / q50 / q80 microseconds per launch, the rate
    at q50, its fraction of the nominal peak, the fraction of this library's
    measured HBM ceiling where the op is HBM-bound, and the CPU restatement's
    rate on the same workload."""
    def base(leg, rate, unit, peak=None):
        r = {"us": _r(leg["q50_us"], 3), "q20_us": _r(leg["q20_us"], 3),
             "q80_us": _r(leg["q80_us"], 3), "rate": _r(leg[rate], 2), "unit": unit,
             "frac": _r(leg[rate] / peak) if peak else None}
        return r

    def cpu_of(key):
        v = cpu.get(key)
        return {"value": _r(v["value"], 4), "unit": v["unit"], "sample": v["sample"]} if v else None

    out = {}

    def put(name, make):
        """One config's record; a leg without the fields it needs is reported
        as an error in its own record, never by losing the line."""
        try:
            out[name] = make()
        except (KeyError, TypeError, ZeroDivisionError) as e:
            out[name] = {"error": f"incomplete leg record: {e!r}"}

    f = legs.get("f16_matmul_256")
    if f and "error" not in f:
        put("1_f16_matmul_256", lambda: {
            **base(f, "TFLOPS", "TFLOPS"),
            "note": "launch-bound: time per launch replayed from a HIP graph; no roofline fraction",
            "cpu": cpu_of(1)})
    ceil2 = legs.get("mfma_ceiling_int8_gemm_4096", {})
    put("2_int8_gemm_4096_dequant", lambda: {
        **base(head, "TOPS", "TOPS", PEAK_INT8_TOPS),
        "ceiling_frac": _r(ceil2["q50_us"] / head["q50_us"]) if "q50_us" in ceil2 else None,
        "cpu": cpu_of(2)})
    for M in (1, 4, 16):
        g = legs.get(f"w8a16_gemv_M{M}")
        if g:
            put(f"3_w8a16_gemv_M{M}", lambda g=g, M=M: {
                **base(g, "GB/s", "GB/s", PEAK_HBM_GBS),
                "ceiling_frac": _r(g["ceiling_frac"]), "graph_us": _r(g["graph_us"], 3),
                "graph_frac": _r(g["graph_hbm_frac"]), "cpu": cpu_of(f"3_M{M}")})
    for name, key in (("softmax", "softmax_f16_8192x4096"), ("rmsnorm", "rmsnorm_f16_8192x4096")):
        g = legs.get(key)
        if g:
            put(f"4_{key}", lambda g=g, name=name: {
                **base(g, "GB/s", "GB/s", PEAK_HBM_GBS),
                "ceiling_frac": _r(g["ceiling_frac"]), "graph_us": _r(g["graph_us"], 3),
                "cpu": cpu_of(f"4_{name}")})
    g = legs.get("swiglu_ffn_2048x4096x11008")
    if g:
        ceil5 = legs.get("mfma_ceiling_swiglu_ffn_2048x4096x11008", {})
        put("5_swiglu_ffn_2048x4096x11008", lambda: {
            **base(g, "TFLOPS", "TFLOPS", PEAK_F16_TFLOPS),
            "ceiling_frac": _r(ceil5["q50_us"] / g["q50_us"]) if "q50_us" in ceil5 else None,
            "stages_us": {k: _r(v, 2) for k, v in g["stages_us"].items()},
            "graph_us": _r(g["graph_us"], 2),
            "sclk_mhz": g["sclk_under_load"]["median_mhz"] if g.get("sclk_under_load") else None,
            "tuned": g["tuned"], "cpu": cpu_of(5)})
    return out


def compact_extra(legs):
    """The context legs in a few numbers each (their full records go to
    stderr)."""
    keep = ("us", "TOPS", "TFLOPS", "GB/s", "mfma_frac", "hbm_frac", "ceiling_frac", "graph_us",
            "winner", "default", "winner_us", "default_us", "proof", "mfma_per_wave", "error")
    out = {}
    for k, v in legs.items():
        if k in ("f16_matmul_256", "swiglu_ffn_2048x4096x11008", "softmax_f16_8192x4096",
                 "rmsnorm_f16_8192x4096") or k.startswith("w8a16_gemv_M"):
            continue                         # in "configs"
        out[k] = {f: _r(v[f], 4) for f in keep if f in v}
    return out


if __name__ == "__main__":
    sys.exit(main())
