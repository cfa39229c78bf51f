"""CPU oracle for the hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module, and only as the checker (or the
timed CPU baseline).  The product (``hexagon-mlir_amd/hxm``) never imports
it and has no CPU fallback.

Two layers:

* ``liboracle.so`` (``oracle.c``): the C restatement of the reference
  semantics, one function per hot-path operation, each citing the reference
  file:line it follows (see the header of ``oracle.c``).
* numpy wrappers that take/return numpy arrays (f16/bf16 as uint16 bit
  patterns where numpy has no dtype).

How each function is pinned (so that a plausible mistake fails a check):

=====================  ====================================================
function               pins (tests/test_oracle.py)
=====================  ====================================================
f16 <-> f32            all 65536 f16 patterns and 2M random f32 against
                       numpy's float16 cast (an independent IEEE-754
                       implementation); bf16 against torch's bfloat16 cast
gemm_i8                numpy int64 matmul (library routine), identity KATs
                       (A=I -> C=B), brute force on tiny shapes, golden
                       fixtures, wrap-around accumulate
dequant_f16            numpy float32 elementwise (a*rs)*cs then float16 cast
                       -- an independent spelling of the same two roundings
matmul (f16/bf16)      torch.matmul (the reference test's own oracle,
                       test_matmul.py:86-88) in float64; small-integer KAT
                       that makes every sum exact (bit-exact expectation)
gemv_w8a16             numpy float64 matmul of the dequantised weights
gemm_w8a16             numpy float64 matmul of the dequantised weights;
                       small-integer KAT (every fp32 sum exact -> bit-exact)
swiglu_gateup          numpy float64 silu(g)*u on numpy's float64 gate/up
                       products; g = 0 -> 0, g >> 0 -> g*u, g << 0 -> 0
softmax_rows           torch.softmax in float64 (test_softmax.py:91);
                       invariants: rows sum to 1, shift invariance, constant
                       row -> 1/cols, argmax preserved
rmsnorm_rows           torch rms_norm in float64 (test_rms_norm.py:84);
                       scale invariance, gamma = 1 -> mean(y^2) ~ 1
layernorm_rows         torch layer_norm in float64 (test_layer_norm.py);
                       y has zero mean / unit variance for gamma=1, beta=0
=====================  ====================================================

The reference's device numerics below the linalg level (the HMX 37-bit
accumulator cells, the qhmath exp/rsqrt routines, the fast inverse square
root) have no runnable implementation here: those are "parity unpinned" and
the oracle follows the linalg-level meaning with exact fp32/fp64 arithmetic.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

F16, BF16, F32 = 1, 2, 3

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float

_SIGS = {
    "hxo_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "hxo_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
    "hxo_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
    "hxo_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
    "hxo_f16_to_f32_array": (None, [_p, _p, _i64]),
    "hxo_f32_to_f16_array": (None, [_p, _p, _i64]),
    "hxo_f32_to_bf16_array": (None, [_p, _p, _i64]),
    "hxo_gemm_i8": (None, [_p, _i64, _p, _i64, _i32, _p, _i64, _i64, _i64, _i64, _i32, _i32]),
    "hxo_dequant_f16": (None, [_p, _i64, _p, _p, _p, _i64, _i64, _i64]),
    "hxo_matmul": (None, [_p, _i64, _p, _i64, _i32, _i32, _p, _i64, _i32, _i32,
                          _i64, _i64, _i64, _i32]),
    "hxo_gemv_w8a16": (None, [_p, _i64, _p, _i64, _p, _p, _i64, _i64, _i64, _i64, _i32]),
    "hxo_gemm_w8a16": (None, [_p, _i64, _p, _i64, _p, _p, _i64, _i64, _i64, _i64, _i32]),
    "hxo_gemm_w8a16_residual": (None, [_p, _i64, _p, _i64, _p, _p, _i64, _p, _i64, _i64, _i64,
                                       _i64, _i32]),
    "hxo_swiglu_gateup": (None, [_p, _i64, _p, _p, _i64, _p, _p, _p, _i64, _i64, _i64, _i64,
                                 _i32]),
    "hxo_softmax_rows": (None, [_p, _i64, _p, _i64, _i64, _i64, _i32, _i32]),
    "hxo_rmsnorm_rows": (None, [_p, _i64, _p, _p, _i64, _i64, _i64, _f32, _i32, _i32]),
    "hxo_layernorm_rows": (None, [_p, _i64, _p, _p, _p, _i64, _p, _p, _i64, _i64, _f32, _i32,
                                  _i32]),
    "hxo_max_threads": (ctypes.c_int, []),
}


def build() -> str:
    """Compiles liboracle.so with the committed Makefile (gcc, no GPU)."""
    subprocess.run(["make", "-s", "-B", "-C", _HERE], check=True)
    return _LIB_PATH


def _load(path):
    l = ctypes.CDLL(path)
    for name, (res, args) in _SIGS.items():
        fn = getattr(l, name)
        fn.restype = res
        fn.argtypes = args
    return l


def native_lib():
    """The same C source built for the host it runs on (-march=native), for
    bench.py's CPU baseline only.  Returns (library, None), or (None, reason)
    when it cannot be built here."""
    try:
        subprocess.run(["make", "-s", "-B", "-C", _HERE, "native"], check=True, capture_output=True,
                       timeout=120)
        return _load(os.path.join(_HERE, "_build", "liboracle_native.so")), None
    except (OSError, subprocess.SubprocessError) as e:
        return None, f"{type(e).__name__}: {e}"


_using = None


class using:
    """``with using(native_lib()[0]): ...`` runs every wrapper below on that
    build of the same source (bench.py's CPU baselines) instead of the
    checker build."""

    def __init__(self, l):
        self.l = l

    def __enter__(self):
        global _using
        self.prev, _using = _using, self.l
        return self.l

    def __exit__(self, *exc):
        global _using
        _using = self.prev
        return False


def lib():
    global _lib
    if _using is not None:
        return _using
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        l = _load(_LIB_PATH)
        _lib = l
    return _lib


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _dt(code_or_dtype) -> int:
    if isinstance(code_or_dtype, int):
        return code_or_dtype
    return {"f16": F16, "bf16": BF16, "f32": F32}[code_or_dtype]


# ---- conversions ----------------------------------------------------------

def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().hxo_f32_to_f16_array(_ptr(x), _ptr(out), x.size)
    return out


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().hxo_f16_to_f32_array(_ptr(h), _ptr(out), h.size)
    return out


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().hxo_f32_to_bf16_array(_ptr(x), _ptr(out), x.size)
    return out


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def to_f32(bits: np.ndarray, dtype) -> np.ndarray:
    dt = _dt(dtype)
    if dt == F16:
        return f16_bits_to_f32(bits)
    if dt == BF16:
        return bf16_bits_to_f32(bits)
    return np.asarray(bits, dtype=np.float32)


# ---- operations -----------------------------------------------------------

def gemm_i8(A: np.ndarray, B: np.ndarray, *, b_nk: bool = False,
            C: np.ndarray | None = None, accumulate: bool = False,
            threads: int = 0, using=None) -> np.ndarray:
    """int32 C = [C +] A[M,K] . B ([K,N], or [N,K] when b_nk).  ``using``: a
    library from native_lib() instead of the checker build."""
    A = np.ascontiguousarray(A, dtype=np.int8)
    B = np.ascontiguousarray(B, dtype=np.int8)
    M, K = A.shape
    N = B.shape[0] if b_nk else B.shape[1]
    assert (B.shape[1] if b_nk else B.shape[0]) == K
    if C is None:
        C = np.zeros((M, N), dtype=np.int32)
    else:
        C = np.ascontiguousarray(C, dtype=np.int32).copy()
    (using or lib()).hxo_gemm_i8(_ptr(A), K, _ptr(B), B.shape[1], int(b_nk), _ptr(C), N,
                                 M, N, K, int(accumulate), threads)
    return C


def dequant_f16(acc: np.ndarray, row_scale: np.ndarray, col_scale: np.ndarray) -> np.ndarray:
    """f16 bits of ((float)acc * rs[m]) * cs[n]."""
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    rs = np.ascontiguousarray(row_scale, dtype=np.float32)
    cs = np.ascontiguousarray(col_scale, dtype=np.float32)
    M, N = acc.shape
    out = np.empty((M, N), dtype=np.uint16)
    lib().hxo_dequant_f16(_ptr(acc), N, _ptr(rs), _ptr(cs), _ptr(out), N, M, N)
    return out


def matmul(A_bits: np.ndarray, B_bits: np.ndarray, *, ab_dtype="f16",
           c_dtype="f16", b_nk: bool = False, C: np.ndarray | None = None,
           accumulate: bool = False, threads: int = 0) -> np.ndarray:
    """C = [C +] A . B with fp32 accumulation, one rounding to c_dtype.

    A/B are uint16 bit patterns of ab_dtype; C is uint16 bits (f16/bf16) or
    float32."""
    A = np.ascontiguousarray(A_bits, dtype=np.uint16)
    B = np.ascontiguousarray(B_bits, dtype=np.uint16)
    M, K = A.shape
    N = B.shape[0] if b_nk else B.shape[1]
    cdt = _dt(c_dtype)
    if C is None:
        C = np.zeros((M, N), dtype=np.float32 if cdt == F32 else np.uint16)
    else:
        C = np.ascontiguousarray(C).copy()
    lib().hxo_matmul(_ptr(A), K, _ptr(B), B.shape[1], int(b_nk), _dt(ab_dtype),
                     _ptr(C), N, cdt, int(accumulate), M, N, K, threads)
    return C


def gemv_w8a16(x_bits: np.ndarray, W: np.ndarray, scale_bits: np.ndarray,
               threads: int = 0) -> np.ndarray:
    """f16 bits of y[m,n] = (sum_k x[m,k] * W[n,k]) * scale[n]."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    W = np.ascontiguousarray(W, dtype=np.int8)
    sc = np.ascontiguousarray(scale_bits, dtype=np.uint16)
    M, K = x.shape
    N = W.shape[0]
    y = np.empty((M, N), dtype=np.uint16)
    lib().hxo_gemv_w8a16(_ptr(x), K, _ptr(W), K, _ptr(sc), _ptr(y), N, M, N, K, threads)
    return y


def gemm_w8a16(x_bits: np.ndarray, W: np.ndarray, scale: np.ndarray,
               threads: int = 0) -> np.ndarray:
    """y = f16((x . W^T) * scale): x f16 bits [M,K], W int8 [N,K], scale fp32 [N]."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    W = np.ascontiguousarray(W, dtype=np.int8)
    sc = np.ascontiguousarray(scale, dtype=np.float32)
    M, K = x.shape
    N = W.shape[0]
    y = np.zeros((M, N), dtype=np.uint16)
    lib().hxo_gemm_w8a16(_ptr(x), K, _ptr(W), K, _ptr(sc), _ptr(y), N, M, N, K, threads)
    return y


def gemm_w8a16_residual(x_bits: np.ndarray, W: np.ndarray, scale: np.ndarray,
                        r_bits: np.ndarray, threads: int = 0) -> np.ndarray:
    """y = f16(f32((x . W^T) * scale) + r): x, r f16 bits [M,K] / [M,N], W int8 [N,K],
    scale fp32 [N] (oracle.c hxo_gemm_w8a16_residual)."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    W = np.ascontiguousarray(W, dtype=np.int8)
    sc = np.ascontiguousarray(scale, dtype=np.float32)
    r = np.ascontiguousarray(r_bits, dtype=np.uint16)
    M, K = x.shape
    N = W.shape[0]
    assert r.shape == (M, N)
    y = np.zeros((M, N), dtype=np.uint16)
    lib().hxo_gemm_w8a16_residual(_ptr(x), K, _ptr(W), K, _ptr(sc), _ptr(r), N, _ptr(y), N, M,
                                  N, K, threads)
    return y


def swiglu_gateup(x_bits: np.ndarray, Wg: np.ndarray, Wu: np.ndarray, sg: np.ndarray,
                  su: np.ndarray, threads: int = 0) -> np.ndarray:
    """h = f16(silu(g) * u) with g = (x . Wg^T) * sg, u = (x . Wu^T) * su."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    Wg = np.ascontiguousarray(Wg, dtype=np.int8)
    Wu = np.ascontiguousarray(Wu, dtype=np.int8)
    sg = np.ascontiguousarray(sg, dtype=np.float32)
    su = np.ascontiguousarray(su, dtype=np.float32)
    M, K = x.shape
    I = Wg.shape[0]
    h = np.zeros((M, I), dtype=np.uint16)
    lib().hxo_swiglu_gateup(_ptr(x), K, _ptr(Wg), _ptr(Wu), K, _ptr(sg), _ptr(su), _ptr(h), I,
                            M, I, K, threads)
    return h


def swiglu_ffn(x_bits: np.ndarray, gamma_bits: np.ndarray, Wg, Wu, sg, su, Wd, sd,
               eps: float = 1e-6, threads: int = 0, residual: bool = False) -> np.ndarray:
    """The SwiGLU FFN block with fp16 tensors between the stages:
    xn = rmsnorm(x) (f16), h = swiglu_gateup(xn) (f16), y = gemm_w8a16(h, Wd);
    with residual, y = gemm_w8a16_residual(h, Wd, r=x) = x + FFN(x)."""
    xn = rmsnorm_rows(x_bits, gamma_bits, eps, "f16")
    h = swiglu_gateup(xn, Wg, Wu, sg, su, threads)
    if residual:
        return gemm_w8a16_residual(h, Wd, sd, x_bits, threads)
    return gemm_w8a16(h, Wd, sd, threads)


def _rows_io(x, dtype):
    dt = _dt(dtype)
    x = np.ascontiguousarray(x, dtype=np.float32 if dt == F32 else np.uint16)
    return x, dt, np.empty_like(x)


def softmax_rows(x, dtype="f16", threads: int = 0) -> np.ndarray:
    x, dt, y = _rows_io(x, dtype)
    rows, cols = x.shape
    lib().hxo_softmax_rows(_ptr(x), cols, _ptr(y), cols, rows, cols, dt, threads)
    return y


def rmsnorm_rows(x, gamma=None, eps: float = 1e-6, dtype="f16",
                 threads: int = 0) -> np.ndarray:
    x, dt, y = _rows_io(x, dtype)
    rows, cols = x.shape
    g = None if gamma is None else np.ascontiguousarray(gamma, dtype=x.dtype)
    lib().hxo_rmsnorm_rows(_ptr(x), cols, _ptr(g), _ptr(y), cols, rows, cols, eps, dt,
                           threads)
    return y


def layernorm_rows(x, gamma=None, beta=None, eps: float = 1e-5, dtype="f16",
                   threads: int = 0):
    """Returns (y, mean, rstd) with mean/rstd fp32.  dtype defaults to f16
    (x as uint16 bit patterns), as for softmax_rows and rmsnorm_rows."""
    x, dt, y = _rows_io(x, dtype)
    rows, cols = x.shape
    g = None if gamma is None else np.ascontiguousarray(gamma, dtype=x.dtype)
    b = None if beta is None else np.ascontiguousarray(beta, dtype=x.dtype)
    mean = np.empty(rows, dtype=np.float32)
    rstd = np.empty(rows, dtype=np.float32)
    lib().hxo_layernorm_rows(_ptr(x), cols, _ptr(g), _ptr(b), _ptr(y), cols,
                             _ptr(mean), _ptr(rstd), rows, cols, eps, dt, threads)
    return y, mean, rstd


def max_threads() -> int:
    return int(lib().hxo_max_threads())
