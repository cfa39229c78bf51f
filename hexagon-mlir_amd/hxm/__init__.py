"""hxm -- the MI355X (gfx950) hot path of the Hexagon-MLIR matmul / row
reduction / tile-search pipeline, behind the C ABI of include/hxm.h.

``hxm.ops`` mirrors the operator surface (matmul, gemm_i8, gemv_w8a16,
softmax, rms_norm, layer_norm, prepack_weight, tune_gemm); ``hxm.search``
mirrors qcom_hexagon_backend/backend/hmx_search.py.  Importing this package
loads libhxm.so and fails if it has not been built.
"""
from ._lib import (B_KN, B_NK, BF16, F16, F32, I8, I32, LIB_PATH, STREAM_K, W_NK, W_PACKED,
                   GemmConfig, HxmError, check, last_error, lib, status_string)

__all__ = ["B_KN", "B_NK", "W_NK", "W_PACKED", "BF16", "F16", "F32", "I8", "I32", "LIB_PATH",
           "STREAM_K", "GemmConfig",
           "HxmError", "check", "last_error", "lib", "status_string", "version"]


def version() -> str:
    return lib.hxm_version().decode()
