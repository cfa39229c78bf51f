"""Torch-facing host mirror of the reference's operator surface for this path.

The reference launches Triton kernels whose meaning is ``linalg.matmul`` /
row reductions and checks them against torch (``torch.matmul``,
``F.softmax``, ``F.rms_norm``, ``F.layer_norm``: test/python/triton/
test_matmul.py:86-88, test_softmax.py:91, test_rms_norm.py:84,
test_layer_norm.py).  These functions keep those names and argument meanings
and run the gfx950 kernels through the C ABI.  Tensors must already live on
the GPU; a CPU tensor is an error, never a silent fallback.
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch

from ._lib import (B_KN, B_NK, BF16, F16, F32, I8, I32, IMAGE_GEMM, IMAGE_W8A16, OP_W8A16,
                   OP_W8A16_SWIGLU, W_NK, W_PACKED, GemmConfig, check, lib)

_DT = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32,
       torch.int8: I8, torch.int32: I32}


def _code(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}") from None


def _stream(stream=None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return s.cuda_stream


def _mat(t: torch.Tensor, name: str) -> torch.Tensor:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (got {t.device})")
    if t.dim() != 2:
        raise ValueError(f"{name} must be 2-D (got {tuple(t.shape)})")
    if t.stride(1) != 1:
        raise ValueError(f"{name} must have a contiguous last dimension")
    return t


def _out(out: torch.Tensor, shape, dtypes, like: torch.Tensor, name: str = "out") -> torch.Tensor:
    """A caller-supplied output: a GPU matrix of exactly ``shape``, one of
    ``dtypes``, on ``like``'s device.  The C entries write shape[0] rows of
    shape[1] elements at its pointer and cannot see the allocation, so a
    wrong shape or dtype here would be a write past the tensor."""
    _mat(out, name)
    if tuple(out.shape) != tuple(shape):
        raise ValueError(f"{name} must be {tuple(shape)} (got {tuple(out.shape)})")
    if out.dtype not in dtypes:
        raise TypeError(f"{name} must be {' or '.join(str(d) for d in dtypes)} (got {out.dtype})")
    if out.device != like.device:
        raise ValueError(f"{name} must be on {like.device} (got {out.device})")
    return out


def _dtype(t: torch.Tensor, dtypes, name: str) -> torch.Tensor:
    if t.dtype not in dtypes:
        raise TypeError(f"{name} must be {' or '.join(str(d) for d in dtypes)} (got {t.dtype})")
    return t


def _vec(t: torch.Tensor, n: int, dtype: torch.dtype, name: str) -> torch.Tensor:
    """A per-channel vector of n elements of dtype on the GPU, contiguous."""
    if not t.is_cuda or t.dtype != dtype or t.numel() != n:
        raise ValueError(f"{name} must be a GPU {dtype} tensor of {n} elements "
                         f"(got {t.dtype} {tuple(t.shape)} on {t.device})")
    return t.contiguous()


def _ld(t: torch.Tensor) -> int:
    return t.stride(0) if t.shape[0] > 1 else max(t.shape[1], t.stride(0))


def _b_extent(A: torch.Tensor, B: torch.Tensor, b_layout: str) -> int:
    """N of C = A @ B for B [K, N] (``"kn"``) or the [N, K] image (``"nk"``),
    after checking that B's K matches A's."""
    if b_layout not in ("kn", "nk"):
        raise ValueError(f"b_layout must be 'kn' or 'nk' (got {b_layout!r})")
    K = A.shape[1]
    kb, n = (B.shape[0], B.shape[1]) if b_layout == "kn" else (B.shape[1], B.shape[0])
    if kb != K:
        raise ValueError(f"shape mismatch A{tuple(A.shape)} B{tuple(B.shape)} ({b_layout})")
    return n


def _cfg(config) -> Optional[GemmConfig]:
    if config is None:
        return None
    if isinstance(config, GemmConfig):
        return config
    return GemmConfig(*config)


def _ptr_or_none(cfg):
    import ctypes
    return None if cfg is None else ctypes.byref(cfg)


def matmul(A: torch.Tensor, B: torch.Tensor, out: Optional[torch.Tensor] = None, *,
           b_layout: str = "kn", accumulate: bool = False,
           out_dtype: Optional[torch.dtype] = None, config=None, stream=None) -> torch.Tensor:
    """C = [C +] A @ B on f16/bf16/f32 with fp32 accumulation (linalg.matmul).
    f32 operands are quantised to fp16 by a pack pass (x + 0.0 then round to
    nearest even, the reference's f32 pack) and multiplied on the fp16 MFMA.

    ``b_layout="kn"``: B is [K, N] (packed per call); ``"nk"``: B is the
    resident [N, K] image from :func:`prepack_weight`."""
    _mat(A, "A"), _mat(B, "B")
    if A.dtype != B.dtype:
        raise TypeError(f"A and B must share a dtype (got {A.dtype} and {B.dtype})")
    M, K = A.shape
    N = _b_extent(A, B, b_layout)
    if out is None:
        if accumulate:
            raise ValueError("accumulate=True needs out")
        out = torch.empty((M, N), dtype=out_dtype or A.dtype, device=A.device)
    _out(out, (M, N), (torch.float16, torch.bfloat16, torch.float32), A)
    cfg = _cfg(config)
    st = lib.hxm_matmul(A.data_ptr(), _ld(A), B.data_ptr(), _ld(B),
                        B_KN if b_layout == "kn" else B_NK, out.data_ptr(), _ld(out),
                        M, N, K, _code(A), _code(out), int(accumulate), _ptr_or_none(cfg),
                        _stream(stream))
    check(st, "hxm_matmul")
    return out


_PLAN = {0: "mfma-full", 1: "mfma-tail", -1: "refused"}
_SOURCE = {0: "default", 1: "tuned", 2: "caller"}


def _plan_dict(p) -> dict:
    return {"op": p.op, "plan": _PLAN.get(p.plan, str(p.plan)),
            "reason": lib.hxm_reason_string(p.reason).decode(),
            "source": _SOURCE.get(p.source, str(p.source)), "config": p.config.as_tuple(),
            "k_slices": p.k_slices, "threads": p.threads, "tiles": p.tiles,
            "lds_bytes": p.lds_bytes, "workspace_bytes": p.workspace_bytes,
            "shape": (p.m, p.n, p.k)}


def plan_matmul(M: int, N: int, K: int, dtype: torch.dtype,
                out_dtype: Optional[torch.dtype] = None, *, b_layout: str = "nk",
                config=None) -> dict:
    """What a matmul call of this shape would run and why, without launching
    (hxm_plan_matmul): plan "mfma-full" / "mfma-tail" / "refused", the
    manifest-style reason, the config and where it came from, the K split,
    tiles, LDS and library workspace bytes.  A refusal is reported, not
    raised."""
    import ctypes
    from ._lib import Plan
    p = Plan()
    od = out_dtype or (torch.int32 if dtype == torch.int8 else dtype)
    cfg = _cfg(config)
    lib.hxm_plan_matmul(M, N, K, _DT[dtype], _DT[dtype], _DT[od],
                        B_KN if b_layout == "kn" else B_NK, _ptr_or_none(cfg), ctypes.byref(p))
    return _plan_dict(p)


def last_plan() -> Optional[dict]:
    """The plan of this thread's last matmul / GEMM call (hxm_last_plan)."""
    import ctypes
    from ._lib import Plan
    p = Plan()
    return _plan_dict(p) if lib.hxm_last_plan(ctypes.byref(p)) else None


def gemm_i8(A: torch.Tensor, B: torch.Tensor, out: Optional[torch.Tensor] = None, *,
            b_layout: str = "kn", accumulate: bool = False, config=None,
            stream=None) -> torch.Tensor:
    """int32 C = [C +] A @ B, exact (the reference's int8 linalg.matmul)."""
    _mat(A, "A"), _mat(B, "B")
    _dtype(A, (torch.int8,), "A"), _dtype(B, (torch.int8,), "B")
    M, K = A.shape
    N = _b_extent(A, B, b_layout)
    if out is None:
        if accumulate:
            raise ValueError("accumulate=True needs out")
        out = torch.empty((M, N), dtype=torch.int32, device=A.device)
    _out(out, (M, N), (torch.int32,), A)
    cfg = _cfg(config)
    st = lib.hxm_gemm_i8(A.data_ptr(), _ld(A), B.data_ptr(), _ld(B),
                         B_KN if b_layout == "kn" else B_NK, out.data_ptr(), _ld(out),
                         M, N, K, int(accumulate), _ptr_or_none(cfg), _stream(stream))
    check(st, "hxm_gemm_i8")
    return out


def gemm_i8_dequant(A: torch.Tensor, B: torch.Tensor, row_scale: torch.Tensor,
                    col_scale: torch.Tensor, out: Optional[torch.Tensor] = None, *,
                    b_layout: str = "kn", config=None, stream=None) -> torch.Tensor:
    """f16 C = f16(((float)(A @ B) * row_scale[:,None]) * col_scale[None,:])."""
    _mat(A, "A"), _mat(B, "B")
    _dtype(A, (torch.int8,), "A"), _dtype(B, (torch.int8,), "B")
    M, K = A.shape
    N = _b_extent(A, B, b_layout)
    if row_scale.dtype != torch.float32 or col_scale.dtype != torch.float32:
        raise TypeError("scales must be float32")
    if row_scale.numel() != M or col_scale.numel() != N:
        raise ValueError("scale lengths must be M and N")
    row_scale = _vec(row_scale, M, torch.float32, "row_scale")
    col_scale = _vec(col_scale, N, torch.float32, "col_scale")
    if out is None:
        out = torch.empty((M, N), dtype=torch.float16, device=A.device)
    _out(out, (M, N), (torch.float16,), A)
    cfg = _cfg(config)
    st = lib.hxm_gemm_i8_dequant(A.data_ptr(), _ld(A), B.data_ptr(), _ld(B),
                                 B_KN if b_layout == "kn" else B_NK,
                                 row_scale.contiguous().data_ptr(),
                                 col_scale.contiguous().data_ptr(), out.data_ptr(), _ld(out),
                                 M, N, K, _ptr_or_none(cfg), _stream(stream))
    check(st, "hxm_gemm_i8_dequant")
    return out


def prepack_weight(B: torch.Tensor, out: Optional[torch.Tensor] = None, *,
                   stream=None) -> torch.Tensor:
    """[K, N] -> resident [N, K] image (hmx_weight_prepack's role).  Without
    ``out`` the image is a [N, K] view of rows padded to 128 bytes (its
    stride(0) is the row stride to pass as ldb), so every row starts on a
    cache line: int8 4000^3 + dequant ran 59.5 us on 4000-byte rows and
    56.7 us on 4096-byte ones."""
    _mat(B, "B")
    K, N = B.shape
    if out is None:
        eb = B.element_size()
        kp = -(-K * eb // 128) * 128 // eb
        out = torch.empty((N, kp), dtype=B.dtype, device=B.device)[:, :K]
    _out(out, (N, K), (B.dtype,), B)
    st = lib.hxm_prepack_weight(B.data_ptr(), _ld(B), out.data_ptr(), _ld(out), K, N,
                                _code(B), _stream(stream))
    check(st, "hxm_prepack_weight")
    return out


def prepack_w8a16(W: torch.Tensor, *, stream=None) -> torch.Tensor:
    """int8 W [N, K] -> the resident GEMV image (flat int8 tensor; each
    weight in offset binary, byte = w ^ 0x80)."""
    _mat(W, "W")
    N, K = W.shape
    out = torch.empty(int(lib.hxm_w8a16_packed_bytes(N, K)), dtype=torch.int8, device=W.device)
    st = lib.hxm_prepack_w8a16(W.data_ptr(), _ld(W), N, K, out.data_ptr(), out.numel(),
                               _stream(stream))
    check(st, "hxm_prepack_w8a16")
    return out


def gemv_w8a16(x: torch.Tensor, W: torch.Tensor, scale: torch.Tensor,
               out: Optional[torch.Tensor] = None, *, N: Optional[int] = None,
               stream=None) -> torch.Tensor:
    """y = f16((x @ W.T in fp32) * scale) for int8 W [N, K] and f16 x [M, K].

    W may also be the flat image from :func:`prepack_w8a16`; then N is taken
    from ``scale`` (or passed explicitly)."""
    _mat(x, "x")
    _dtype(x, (torch.float16,), "x"), _dtype(W, (torch.int8,), "W")
    M, K = x.shape
    packed = W.dim() == 1
    if packed:
        if not W.is_cuda:
            raise ValueError(f"W must be a GPU tensor (got {W.device})")
        N = scale.numel() if N is None else N
        if W.numel() < lib.hxm_w8a16_packed_bytes(N, K):
            raise ValueError("packed image too small for [N, K]")
        ldw = K
    else:
        _mat(W, "W")
        N = W.shape[0]
        if W.shape[1] != K:
            raise ValueError("W must be [N, K]")
        ldw = _ld(W)
    scale = _vec(scale, N, torch.float16, "scale")
    if out is None:
        out = torch.empty((M, N), dtype=torch.float16, device=x.device)
    _out(out, (M, N), (torch.float16,), x)
    st = lib.hxm_gemv_w8a16(x.data_ptr(), _ld(x), W.data_ptr(), ldw,
                            W_PACKED if packed else W_NK, scale.data_ptr(),
                            out.data_ptr(), _ld(out), M, N, K, _stream(stream))
    check(st, "hxm_gemv_w8a16")
    return out


def _f32_vec(t: torch.Tensor, n: int, name: str) -> torch.Tensor:
    if not t.is_cuda or t.dtype != torch.float32 or t.numel() != n:
        raise ValueError(f"{name} must be a GPU float32 tensor of {n} elements")
    return t.contiguous()


def gemm_w8a16(x: torch.Tensor, W: torch.Tensor, scale: torch.Tensor,
               out: Optional[torch.Tensor] = None, *, residual: Optional[torch.Tensor] = None,
               config=None, stream=None) -> torch.Tensor:
    """y = f16((x @ W.T in fp32) * scale) for f16 x [M, K], int8 W [N, K] and
    fp32 per-channel scale [N] (the large-M W8A16 GEMM of the FFN).  With an
    f16 ``residual`` [M, N]: y = f16(fp32((x @ W.T) * scale) + residual)
    (hxm_gemm_w8a16_residual); ``out`` may be ``residual`` itself."""
    _mat(x, "x"), _mat(W, "W")
    _dtype(x, (torch.float16,), "x"), _dtype(W, (torch.int8,), "W")
    M, K = x.shape
    N = W.shape[0]
    if W.shape[1] != K:
        raise ValueError("W must be [N, K]")
    scale = _f32_vec(scale, N, "scale")
    if out is None:
        out = torch.empty((M, N), dtype=torch.float16, device=x.device)
    _out(out, (M, N), (torch.float16,), x)
    cfg = _cfg(config)
    if residual is not None:
        _mat(residual, "residual")
        if tuple(residual.shape) != (M, N) or residual.dtype != torch.float16:
            raise ValueError(f"residual must be f16 [{M}, {N}]")
        st = lib.hxm_gemm_w8a16_residual(x.data_ptr(), _ld(x), W.data_ptr(), _ld(W),
                                         scale.data_ptr(), residual.data_ptr(), _ld(residual),
                                         out.data_ptr(), _ld(out), M, N, K, _ptr_or_none(cfg),
                                         _stream(stream))
        check(st, "hxm_gemm_w8a16_residual")
        return out
    st = lib.hxm_gemm_w8a16(x.data_ptr(), _ld(x), W.data_ptr(), _ld(W), scale.data_ptr(),
                            out.data_ptr(), _ld(out), M, N, K, _ptr_or_none(cfg),
                            _stream(stream))
    check(st, "hxm_gemm_w8a16")
    return out


def swiglu_pack(Wg: torch.Tensor, Wu: torch.Tensor, gate_scale: torch.Tensor,
                up_scale: torch.Tensor, *, stream=None):
    """The fused gate/up image (int8 [128*ceil(I/64), K], each weight stored
    in offset binary, byte = w ^ 0x80) and its fp32 scales from gate/up
    weights int8 [I, K] and fp32 scales [I]; made once per weight pair."""
    _mat(Wg, "Wg"), _mat(Wu, "Wu")
    I, K = Wg.shape
    if tuple(Wu.shape) != (I, K) or _ld(Wu) != _ld(Wg):
        raise ValueError("Wg and Wu must both be [I, K] with the same row stride")
    sg = _f32_vec(gate_scale, I, "gate_scale")
    su = _f32_vec(up_scale, I, "up_scale")
    rows = lib.hxm_swiglu_packed_rows(I)
    Wgu = torch.empty((rows, K), dtype=torch.int8, device=Wg.device)
    sgu = torch.empty(rows, dtype=torch.float32, device=Wg.device)
    st = lib.hxm_swiglu_pack(Wg.data_ptr(), Wu.data_ptr(), _ld(Wg), sg.data_ptr(),
                             su.data_ptr(), I, K, Wgu.data_ptr(), sgu.data_ptr(),
                             _stream(stream))
    check(st, "hxm_swiglu_pack")
    return Wgu, sgu


def gemm_w8a16_swiglu(x: torch.Tensor, Wgu: torch.Tensor, sgu: torch.Tensor, I: int,
                      out: Optional[torch.Tensor] = None, *, config=None,
                      stream=None) -> torch.Tensor:
    """h = f16(silu(x @ Wg.T * sg) * (x @ Wu.T * su)) from the
    :func:`swiglu_pack` image; h is [M, I]."""
    _mat(x, "x"), _mat(Wgu, "Wgu")
    _dtype(x, (torch.float16,), "x"), _dtype(Wgu, (torch.int8,), "Wgu")
    M, K = x.shape
    rows = lib.hxm_swiglu_packed_rows(I)
    if tuple(Wgu.shape) != (rows, K) or _ld(Wgu) != K:
        raise ValueError(f"Wgu must be the contiguous [{rows}, {K}] swiglu_pack image")
    sgu = _f32_vec(sgu, rows, "sgu")
    if out is None:
        out = torch.empty((M, I), dtype=torch.float16, device=x.device)
    _out(out, (M, I), (torch.float16,), x)
    cfg = _cfg(config)
    st = lib.hxm_gemm_w8a16_swiglu(x.data_ptr(), _ld(x), Wgu.data_ptr(), sgu.data_ptr(),
                                   out.data_ptr(), _ld(out), M, I, K, _ptr_or_none(cfg),
                                   _stream(stream))
    check(st, "hxm_gemm_w8a16_swiglu")
    return out


def swiglu_ffn(x: torch.Tensor, gamma: torch.Tensor, Wgu: torch.Tensor, sgu: torch.Tensor,
               Wd: torch.Tensor, sd: torch.Tensor, I: int, *, eps: float = 1e-6,
               residual: bool = False, configs=(None, None), stream=None) -> torch.Tensor:
    """The Llama-style SwiGLU FFN block: RMSNorm -> fused gate/up GEMM with
    SiLU * mul -> down GEMM.  x f16 [T, H]; gamma f16 [H]; Wgu/sgu from
    :func:`swiglu_pack`; Wd int8 [H, I] with fp32 scales sd [H].  With
    ``residual`` the down GEMM's epilogue adds x: the block returns
    x + FFN(x)."""
    xn = rms_norm(x, (x.shape[-1],), gamma, eps=eps, stream=stream)
    h = gemm_w8a16_swiglu(xn, Wgu, sgu, I, config=configs[0], stream=stream)
    return gemm_w8a16(h, Wd, sd, residual=x if residual else None, config=configs[1],
                      stream=stream)


def w8a16_configs(swiglu: bool = False):
    """The compiled W8A16 GEMM configurations (bk in f16 elements)."""
    n = lib.hxm_w8a16_configs(int(swiglu), None, 0)
    arr = (GemmConfig * n)()
    lib.hxm_w8a16_configs(int(swiglu), arr, n)
    return list(arr)


def tune_w8a16(x: torch.Tensor, W: torch.Tensor, scale: torch.Tensor, out: torch.Tensor, *,
               swiglu: bool = False, reps: int = 5, stream=None):
    """Measured tile search for :func:`gemm_w8a16` (W [N, K], scale [N]) or,
    with swiglu=True, :func:`gemm_w8a16_swiglu` (W = Wgu, scale = sgu, out
    [M, I]).  The winner is cached for later calls; returns (GemmConfig,
    report dict).  reps=0 calibrates the repetitions per config as in
    :func:`tune_gemm`; the int8-weight configs are not priced, so all run."""
    import ctypes
    import json
    _mat(x, "x"), _mat(W, "W")
    _dtype(x, (torch.float16,), "x"), _dtype(W, (torch.int8,), "W")
    M, K = x.shape
    if swiglu:
        N = out.shape[1]
        rows = lib.hxm_swiglu_packed_rows(N)
        if tuple(W.shape) != (rows, K) or _ld(W) != K:
            raise ValueError(f"W must be the contiguous [{rows}, {K}] swiglu_pack image")
        scale = _f32_vec(scale, rows, "scale")
    else:
        N = W.shape[0]
        if W.shape[1] != K:
            raise ValueError("W must be [N, K]")
        scale = _f32_vec(scale, N, "scale")
    _out(out, (M, N), (torch.float16,), x)
    best = GemmConfig()
    buf = ctypes.create_string_buffer(1 << 16)
    st = lib.hxm_tune_w8a16(OP_W8A16_SWIGLU if swiglu else OP_W8A16, x.data_ptr(), _ld(x),
                            W.data_ptr(), _ld(W), scale.data_ptr(),
                            out.data_ptr(), _ld(out), M, N, K, reps, ctypes.byref(best), buf,
                            len(buf), _stream(stream))
    check(st, "hxm_tune_w8a16")
    return best, json.loads(buf.value.decode())


class _DeviceArray:
    """A non-owning view of library-owned device memory for torch.as_tensor
    (the CUDA array interface, which the ROCm build of torch accepts)."""

    _TYPESTR = {I8: "|i1", F16: "<f2", BF16: "<V2", F32: "<f4"}

    def __init__(self, ptr: int, shape, dtype_code: int):
        self.__cuda_array_interface__ = {"shape": tuple(shape), "data": (ptr, False),
                                         "typestr": self._TYPESTR[dtype_code], "version": 3,
                                         "strides": None}


def resident_weight(W: torch.Tensor, kind: str = "gemm", *, expect_dtype=None,
                    expect_shape=None, stream=None) -> torch.Tensor:
    """The content-addressed resident image of a weight, packed on first use
    (WeightPrepack.pack, hmx_weight_prepack.py:124-168).

    ``kind="gemm"``: W is B [K, N] (int8/f16/bf16, or f32 -> an f16 image);
    returns the [N, K] image for ``b_layout="nk"``.  ``kind="w8a16"``: W is
    int8 [N, K]; returns the flat packed GEMV image.  The returned tensor
    views library-owned memory that stays valid until ``hxm_release_cache``.
    ``expect_dtype`` / ``expect_shape`` are the contract: a mismatch raises."""
    import ctypes
    _mat(W, "W")
    rows, cols = W.shape
    k = {"gemm": IMAGE_GEMM, "w8a16": IMAGE_W8A16}[kind]
    exp_dt = -1 if expect_dtype is None else _DT[expect_dtype]
    shp = None if expect_shape is None else (ctypes.c_int64 * 2)(*expect_shape)
    img = ctypes.c_void_p()
    img_dt = ctypes.c_int32()
    st = lib.hxm_resident_weight(W.data_ptr(), _ld(W), rows, cols, _code(W), exp_dt, shp, k,
                                 ctypes.byref(img), ctypes.byref(img_dt), _stream(stream))
    check(st, "hxm_resident_weight")
    if k == IMAGE_GEMM:
        if img_dt.value == BF16:   # no bf16 typestr: view the bits, then reinterpret
            t = torch.as_tensor(_DeviceArray(img.value, (cols, rows), F16), device=W.device)
            return t.view(torch.bfloat16)
        return torch.as_tensor(_DeviceArray(img.value, (cols, rows), img_dt.value),
                               device=W.device)
    nbytes = lib.hxm_w8a16_packed_bytes(rows, cols)
    return torch.as_tensor(_DeviceArray(img.value, (nbytes,), I8), device=W.device)


def _rows(x: torch.Tensor):
    if not x.is_cuda:
        raise ValueError(f"x must be a GPU tensor (got {x.device})")
    if x.stride(-1) != 1:
        raise ValueError("x must have a contiguous last dimension")
    cols = x.shape[-1]
    x2 = x.reshape(-1, cols)
    return x2, x2.shape[0], cols


def _rows_out(out: Optional[torch.Tensor], x: torch.Tensor, cols: int):
    """The output of a row op: new, or the caller's of x's shape and dtype
    (rows of it may be strided, its last dimension contiguous)."""
    if out is None:
        out = torch.empty_like(x)
    elif tuple(out.shape) != tuple(x.shape) or out.dtype != x.dtype or out.device != x.device:
        raise ValueError(f"out must be {x.dtype} {tuple(x.shape)} on {x.device} "
                         f"(got {out.dtype} {tuple(out.shape)} on {out.device})")
    elif out.stride(-1) != 1:
        raise ValueError("out must have a contiguous last dimension")
    try:
        return out, out.view(-1, cols)   # a view: the kernel writes into out itself
    except RuntimeError:
        raise ValueError("out's rows must be evenly strided (viewable as [rows, cols])") from None


def _row_param(t: Optional[torch.Tensor], x: torch.Tensor, cols: int, name: str):
    """gamma / beta: None, or [cols] of x's dtype on x's device."""
    if t is None:
        return None
    if t.numel() != cols or t.dtype != x.dtype or t.device != x.device:
        raise ValueError(f"{name} must be {x.dtype} [{cols}] on {x.device} "
                         f"(got {t.dtype} {tuple(t.shape)} on {t.device})")
    return t.contiguous()


def softmax(x: torch.Tensor, dim: int = -1, out: Optional[torch.Tensor] = None, *,
            stream=None) -> torch.Tensor:
    """Row softmax over the last dimension (F.softmax(x, dim=-1))."""
    if dim not in (-1, x.dim() - 1):
        raise ValueError("only the last dimension is supported")
    x2, rows, cols = _rows(x)
    out, o2 = _rows_out(out, x, cols)
    st = lib.hxm_softmax_rows(x2.data_ptr(), _ld(x2), o2.data_ptr(), _ld(o2), rows, cols,
                              _code(x), _stream(stream))
    check(st, "hxm_softmax_rows")
    return out


def rms_norm(x: torch.Tensor, normalized_shape: Sequence[int],
             weight: Optional[torch.Tensor] = None, eps: Optional[float] = None,
             out: Optional[torch.Tensor] = None, *, stream=None) -> torch.Tensor:
    """F.rms_norm over the last dimension."""
    x2, rows, cols = _rows(x)
    if tuple(normalized_shape) != (cols,):
        raise ValueError("normalized_shape must be (x.shape[-1],)")
    if eps is None:
        eps = torch.finfo(x.dtype).eps
    out, o2 = _rows_out(out, x, cols)
    weight = _row_param(weight, x, cols, "weight")
    st = lib.hxm_rmsnorm_rows(x2.data_ptr(), _ld(x2),
                              None if weight is None else weight.data_ptr(), o2.data_ptr(), _ld(o2),
                              rows, cols, float(eps), _code(x), _stream(stream))
    check(st, "hxm_rmsnorm_rows")
    return out


def layer_norm(x: torch.Tensor, normalized_shape: Sequence[int],
               weight: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None,
               eps: float = 1e-5, out: Optional[torch.Tensor] = None, *,
               return_stats: bool = False, stream=None):
    """F.layer_norm over the last dimension; optionally returns (y, mean, rstd)."""
    x2, rows, cols = _rows(x)
    if tuple(normalized_shape) != (cols,):
        raise ValueError("normalized_shape must be (x.shape[-1],)")
    out, o2 = _rows_out(out, x, cols)
    weight = _row_param(weight, x, cols, "weight")
    bias = _row_param(bias, x, cols, "bias")
    mean = rstd = None
    if return_stats:
        mean = torch.empty(rows, dtype=torch.float32, device=x.device)
        rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
    st = lib.hxm_layernorm_rows(
        x2.data_ptr(), _ld(x2), None if weight is None else weight.data_ptr(),
        None if bias is None else bias.data_ptr(), o2.data_ptr(), _ld(o2),
        None if mean is None else mean.data_ptr(), None if rstd is None else rstd.data_ptr(),
        rows, cols, float(eps), _code(x), _stream(stream))
    check(st, "hxm_layernorm_rows")
    return (out, mean, rstd) if return_stats else out


def tune_gemm(A: torch.Tensor, B_nk: torch.Tensor, out: torch.Tensor, *, reps: int = 5,
              stream=None):
    """Measured tile search on these operands; returns (GemmConfig, report dict).
    reps=0 calibrates the repetitions per config (hxm_calibration_iters of the
    timed warm call against a 10 ms budget, 5 to 1000 launches).  Configs the
    cost model prices out of reach are not launched (``pruned`` in the
    report, with ``model_lb_us`` / ``model_ub_us`` for every config)."""
    import ctypes
    import json
    _mat(A, "A"), _mat(B_nk, "B")
    _dtype(A, (torch.int8, torch.float16, torch.bfloat16), "A")
    if B_nk.dtype != A.dtype:
        raise TypeError(f"A and B must share a dtype (got {A.dtype} and {B_nk.dtype})")
    M, K = A.shape
    N = _b_extent(A, B_nk, "nk")
    _out(out, (M, N), (torch.int32,) if A.dtype == torch.int8 else (A.dtype,), A)
    best = GemmConfig()
    buf = ctypes.create_string_buffer(1 << 16)
    st = lib.hxm_tune_gemm(_code(A), A.data_ptr(), _ld(A), B_nk.data_ptr(), _ld(B_nk),
                           out.data_ptr(), _ld(out), M, N, K, reps, ctypes.byref(best), buf,
                           len(buf), _stream(stream))
    check(st, "hxm_tune_gemm")
    return best, json.loads(buf.value.decode())
