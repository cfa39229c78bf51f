"""Memref descriptors at the C ABI.

The reference's compiled kernels take their tensors as
``MemRefDescriptor<T, R>*`` -- {allocated, aligned, offset, sizes[R],
strides[R]} (test/utils/dsp/include/common.h:15-30), passed by the generated
launcher (qcom_hexagon_backend/backend/hexagon_launcher_base.py:60-75).  The C
ABI here takes each rank-2 operand as (pointer, leading dimension) instead.
This module is the conversion a caller holding descriptors applies:

* data = aligned + offset * element bytes (``allocated`` is not used: the
  library never frees caller memory);
* ld = strides[0], rows = sizes[0], cols = sizes[1];
* strides[1] must be 1: the kernels stream contiguous rows, so a non-unit
  inner stride is refused ("tile-alignment") rather than copied;
* a negative offset, negative sizes, or rows that overlap (strides[0] <
  sizes[1] with more than one row) are refused ("invalid-argument").
"""
from __future__ import annotations

import ctypes
from typing import NamedTuple

from ._lib import (BF16, F16, F32, HXM_INVALID_ARG, HXM_UNSUPPORTED_SHAPE, I8, I32, HxmError,
                   check, lib)

_ELEM = {F16: 2, BF16: 2, F32: 4, I8: 1, I32: 4}


class MemRefDescriptor2D(ctypes.Structure):
    """MemRefDescriptor<T, 2> (common.h:15-21) with the element type erased."""
    _fields_ = [("allocated", ctypes.c_void_p), ("aligned", ctypes.c_void_p),
                ("offset", ctypes.c_int64), ("sizes", ctypes.c_int64 * 2),
                ("strides", ctypes.c_int64 * 2)]


class Operand(NamedTuple):
    ptr: int
    ld: int
    rows: int
    cols: int


def describe(base: int, rows: int, cols: int, ld: int, offset: int = 0,
             inner_stride: int = 1) -> MemRefDescriptor2D:
    """A descriptor over `base` (allocated == aligned) with the given view."""
    d = MemRefDescriptor2D()
    d.allocated = d.aligned = base
    d.offset = offset
    d.sizes[0], d.sizes[1] = rows, cols
    d.strides[0], d.strides[1] = ld, inner_stride
    return d


def operand(desc: MemRefDescriptor2D, dtype: int, name: str = "operand") -> Operand:
    """The (pointer, leading dimension, rows, cols) the C ABI takes for a
    rank-2 descriptor of element type `dtype` (an hxm dtype code)."""
    rows, cols = int(desc.sizes[0]), int(desc.sizes[1])
    if desc.strides[1] != 1:
        raise HxmError(HXM_UNSUPPORTED_SHAPE,
                       f"tile-alignment: {name} has inner stride {desc.strides[1]}; the "
                       "kernels read contiguous rows", "memref.operand")
    if desc.offset < 0 or rows < 0 or cols < 0 or (rows > 1 and desc.strides[0] < cols):
        raise HxmError(HXM_INVALID_ARG,
                       f"invalid-argument: {name} offset {desc.offset}, sizes "
                       f"[{rows}, {cols}], strides [{desc.strides[0]}, 1]", "memref.operand")
    ptr = (desc.aligned or 0) + desc.offset * _ELEM[dtype]
    return Operand(ptr, int(desc.strides[0]) if rows > 1 else max(cols, 1), rows, cols)


def matmul(A: MemRefDescriptor2D, B: MemRefDescriptor2D, C: MemRefDescriptor2D, *,
           ab_dtype: int, c_dtype: int, accumulate: bool = False, stream: int = 0) -> None:
    """linalg.matmul C = [C +] A . B on descriptors (A [M,K], B [K,N], C
    [M,N]) through hxm_matmul (f16 / bf16 / f32 operands)."""
    a, b, c = (operand(A, ab_dtype, "A"), operand(B, ab_dtype, "B"), operand(C, c_dtype, "C"))
    if a.cols != b.rows or c.rows != a.rows or c.cols != b.cols:
        raise HxmError(HXM_INVALID_ARG, f"invalid-argument: shapes A[{a.rows},{a.cols}] "
                       f"B[{b.rows},{b.cols}] C[{c.rows},{c.cols}]", "memref.matmul")
    from ._lib import B_KN
    check(lib.hxm_matmul(a.ptr, a.ld, b.ptr, b.ld, B_KN, c.ptr, c.ld, a.rows, b.cols, a.cols,
                         ab_dtype, c_dtype, int(accumulate), None, stream), "hxm_matmul")


def softmax_rows(X: MemRefDescriptor2D, Y: MemRefDescriptor2D, *, dtype: int,
                 stream: int = 0) -> None:
    """Row softmax on descriptors through hxm_softmax_rows."""
    x, y = operand(X, dtype, "X"), operand(Y, dtype, "Y")
    if (x.rows, x.cols) != (y.rows, y.cols):
        raise HxmError(HXM_INVALID_ARG, "invalid-argument: X and Y shapes differ",
                       "memref.softmax_rows")
    check(lib.hxm_softmax_rows(x.ptr, x.ld, y.ptr, y.ld, x.rows, x.cols, dtype, stream),
          "hxm_softmax_rows")
