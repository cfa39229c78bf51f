"""Writes the committed golden fixtures (tests/golden/*.npz).

Inputs are seeded; expected outputs come from library routines that are
independent of oracle/oracle.c -- numpy's int64 matmul and float32/float16
casts, torch's float64 softmax / rms_norm / layer_norm / matmul (the
functions the reference's own device tests compare against:
test/python/triton/test_matmul.py:86-88, test_softmax.py:91,
test_rms_norm.py:84, test_layer_norm.py).  The reference itself ships no
numeric golden files, and its Python test harness needs the Hexagon
Triton backend, so these fixtures are the committed known answers.

Run:  python tests/golden/make_golden.py   (rewrites the .npz files)
"""
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def f16_bits(a):
    return np.asarray(a, dtype=np.float16).view(np.uint16)


def main():
    rng = np.random.default_rng(20261201)

    # int8 GEMM (ragged M, N; K a multiple of 16) + dequant epilogue.
    A = rng.integers(-127, 128, size=(67, 96), dtype=np.int64).astype(np.int8)
    B = rng.integers(-127, 128, size=(96, 45), dtype=np.int64).astype(np.int8)
    C = (A.astype(np.int64) @ B.astype(np.int64)).astype(np.int32)
    rs = rng.uniform(0.001, 0.02, size=67).astype(np.float32)
    cs = rng.uniform(0.001, 0.02, size=45).astype(np.float32)
    deq = ((C.astype(np.float32) * rs[:, None]) * cs[None, :]).astype(np.float16)
    np.savez_compressed(os.path.join(HERE, "gemm_i8.npz"), A=A, B=B, C=C, row_scale=rs, col_scale=cs,
             dequant_f16_bits=deq.view(np.uint16))

    # f16 matmul: random U[-1,1] (expected in float64) and a small-integer
    # case whose every partial sum is exact in fp32 and whose result is exact
    # in fp16 (|C| <= 2048), so the expected f16 bits are exact.
    a = rng.uniform(-1, 1, size=(64, 128)).astype(np.float16)
    b = rng.uniform(-1, 1, size=(128, 48)).astype(np.float16)
    exp = (torch.from_numpy(a.astype(np.float64)) @ torch.from_numpy(b.astype(np.float64))).numpy()
    ai = rng.integers(-4, 5, size=(32, 64)).astype(np.float16)
    bi = rng.integers(-4, 5, size=(64, 32)).astype(np.float16)
    ci = (ai.astype(np.int64) @ bi.astype(np.int64)).astype(np.float16)
    np.savez_compressed(os.path.join(HERE, "matmul_f16.npz"), A_bits=f16_bits(a), B_bits=f16_bits(b),
             C_f64=exp, Ai_bits=f16_bits(ai), Bi_bits=f16_bits(bi), Ci_bits=f16_bits(ci))

    # W8A16 GEMV: y = (x @ W.T) * scale.
    x = rng.standard_normal((4, 256)).astype(np.float16)
    W = rng.integers(-127, 128, size=(48, 256), dtype=np.int64).astype(np.int8)
    sc = rng.uniform(0.001, 0.02, size=48).astype(np.float16)
    y = (x.astype(np.float64) @ W.astype(np.float64).T) * sc.astype(np.float64)[None, :]
    np.savez_compressed(os.path.join(HERE, "gemv_w8a16.npz"), x_bits=f16_bits(x), W=W,
             scale_bits=f16_bits(sc), y_f64=y)

    # Row ops (the reference test shapes: softmax 128x128, rms_norm 127x513;
    # layer_norm 8 of the reference's 27 rows x 8192 f32).
    xs = (rng.standard_normal((128, 128)) * 2).astype(np.float16)
    sm = torch.softmax(torch.from_numpy(xs.astype(np.float64)), dim=-1).numpy()
    xr = (rng.standard_normal((127, 513)) * 2).astype(np.float16)
    gr = (1 + 0.1 * rng.standard_normal(513)).astype(np.float16)
    rn = torch.nn.functional.rms_norm(torch.from_numpy(xr.astype(np.float64)), (513,),
                                      weight=torch.from_numpy(gr.astype(np.float64)),
                                      eps=1e-6).numpy()
    xl = rng.random((8, 8192)).astype(np.float32)
    wl = rng.random(8192).astype(np.float32)
    bl = rng.random(8192).astype(np.float32)
    xt = torch.from_numpy(xl.astype(np.float64))
    ln = torch.nn.functional.layer_norm(xt, (8192,), torch.from_numpy(wl.astype(np.float64)),
                                        torch.from_numpy(bl.astype(np.float64)), eps=1e-5).numpy()
    mean = xt.mean(dim=1).numpy()
    rstd = (1.0 / torch.sqrt(xt.var(dim=1, unbiased=False) + 1e-5)).numpy()
    # Expected values are computed in float64 and stored as float32 (far
    # below the f16/f32 output tolerances).
    f32 = lambda v: np.asarray(v, dtype=np.float32)  # noqa: E731
    np.savez_compressed(os.path.join(HERE, "rows.npz"), softmax_x_bits=f16_bits(xs),
                        softmax_y=f32(sm), rms_x_bits=f16_bits(xr),
                        rms_gamma_bits=f16_bits(gr), rms_y=f32(rn), ln_x=xl, ln_w=wl,
                        ln_b=bl, ln_y=f32(ln), ln_mean=f32(mean), ln_rstd=f32(rstd))


if __name__ == "__main__":
    main()
