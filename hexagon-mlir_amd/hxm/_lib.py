"""ctypes binding of libhxm.so (the C ABI declared in include/hxm.h).

The library is built in-tree by ``hexagon-mlir_amd/csrc/Makefile`` into this
directory.  There is no fallback: if the library is missing, importing
``hxm`` raises.
"""
from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libhxm.so")

HXM_OK = 0
HXM_INVALID_ARG = 1
HXM_UNSUPPORTED_DTYPE = 2
HXM_UNSUPPORTED_SHAPE = 3
HXM_HIP_ERROR = 4
HXM_OUT_OF_MEMORY = 5
HXM_NO_DEVICE = 6

F16, BF16, F32, I8, I32 = 1, 2, 3, 4, 5
B_KN, B_NK = 0, 1
W_NK, W_PACKED = 0, 1
OP_W8A16, OP_W8A16_SWIGLU = 16, 17
STREAM_K = 1024  # HXM_STREAM_K: split_k of a W8A16 config in stream-K form
IMAGE_GEMM, IMAGE_W8A16 = 0, 1


class HxmError(RuntimeError):
    """A non-OK hxm_status, carrying the library's reason string."""

    def __init__(self, status: int, reason: str, fn: str):
        self.status = status
        self.reason = reason
        super().__init__(f"{fn}: {status_string(status)} ({reason})")


class GemmConfig(ctypes.Structure):
    _fields_ = [("bm", ctypes.c_int32), ("bn", ctypes.c_int32), ("bk", ctypes.c_int32),
                ("waves_m", ctypes.c_int32), ("waves_n", ctypes.c_int32),
                ("stages", ctypes.c_int32), ("split_k", ctypes.c_int32)]

    def as_tuple(self):
        return (self.bm, self.bn, self.bk, self.waves_m, self.waves_n, self.stages,
                self.split_k)

    def __repr__(self):
        return ("GemmConfig(bm=%d, bn=%d, bk=%d, waves=%dx%d, stages=%d, split_k=%d)"
                % self.as_tuple())


class DeviceModel(ctypes.Structure):
    """hxm_device_model: the rates the cost model prices a config with."""
    _fields_ = [("cus", ctypes.c_int32), ("tier", ctypes.c_int32),
                ("sclk_mhz_peak", ctypes.c_double), ("sclk_mhz_sustained", ctypes.c_double),
                ("hbm_gbps_peak", ctypes.c_double), ("hbm_gbps_sustained", ctypes.c_double),
                ("lds_fill_peak", ctypes.c_double), ("lds_fill_sustained", ctypes.c_double),
                ("launch_us", ctypes.c_double), ("lds_bytes", ctypes.c_int64),
                ("cache_bytes", ctypes.c_int64)]


class TilePredictionC(ctypes.Structure):
    """hxm_tile_prediction: one config's modeled interval (microseconds)."""
    _fields_ = [("lb_us", ctypes.c_double), ("ub_us", ctypes.c_double),
                ("p50_us", ctypes.c_double), ("units", ctypes.c_int64 * 3),
                ("abstain", ctypes.c_int32), ("tier", ctypes.c_int32),
                ("heat", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class Plan(ctypes.Structure):
    """hxm_plan: one GEMM call's plan and reason."""
    _fields_ = [("op", ctypes.c_int32), ("plan", ctypes.c_int32), ("reason", ctypes.c_int32),
                ("source", ctypes.c_int32), ("config", GemmConfig),
                ("k_slices", ctypes.c_int32), ("threads", ctypes.c_int32),
                ("tiles", ctypes.c_int64), ("lds_bytes", ctypes.c_int64),
                ("workspace_bytes", ctypes.c_int64), ("m", ctypes.c_int64),
                ("n", ctypes.c_int64), ("k", ctypes.c_int64)]


class ArmQuantiles(ctypes.Structure):
    """hxm_arm_quantiles: one measured arm of a search round."""
    _fields_ = [("q20", ctypes.c_double), ("q50", ctypes.c_double), ("q80", ctypes.c_double)]


class RoundVerdict(ctypes.Structure):
    """hxm_round_verdict: a search round judged as a whole (codes only)."""
    _fields_ = [("canary", ctypes.c_int32), ("valid", ctypes.c_int32),
                ("start", ctypes.c_int32), ("champion", ctypes.c_int32),
                ("proof", ctypes.c_int32), ("measured", ctypes.c_int32),
                ("takeovers", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("canary_cv", ctypes.c_double), ("canary_delta", ctypes.c_double),
                ("canary_gate", ctypes.c_double), ("control_cv", ctypes.c_double),
                ("control_delta", ctypes.c_double), ("control_gate", ctypes.c_double)]


_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_f64 = ctypes.c_double
_st = ctypes.c_int  # hxm_status
_cfgp = ctypes.POINTER(GemmConfig)

# name -> (restype, argtypes); the exact list of include/hxm.h.
SIGNATURES = {
    "hxm_status_string": (ctypes.c_char_p, [_i32]),
    "hxm_last_error": (ctypes.c_char_p, []),
    "hxm_version": (ctypes.c_char_p, []),
    "hxm_device_count": (_i32, []),
    "hxm_release_cache": (_st, []),
    "hxm_query_contraction": (_st, [_i64, _i64, _i64, _i32, _i32, _i32, ctypes.POINTER(_i32)]),
    "hxm_plan_matmul": (_st, [_i64, _i64, _i64, _i32, _i32, _i32, _i32, _cfgp,
                              ctypes.POINTER(Plan)]),
    "hxm_last_plan": (_i32, [ctypes.POINTER(Plan)]),
    "hxm_matmul": (_st, [_p, _i64, _p, _i64, _i32, _p, _i64, _i64, _i64, _i64, _i32, _i32,
                         _i32, _cfgp, _p]),
    "hxm_gemm_i8": (_st, [_p, _i64, _p, _i64, _i32, _p, _i64, _i64, _i64, _i64, _i32, _cfgp, _p]),
    "hxm_gemm_i8_noalloc": (_st, [_p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _i32, _cfgp,
                                  _p]),
    "hxm_gemm_i8_dequant": (_st, [_p, _i64, _p, _i64, _i32, _p, _p, _p, _i64, _i64, _i64,
                                  _i64, _cfgp, _p]),
    "hxm_prepack_weight": (_st, [_p, _i64, _p, _i64, _i64, _i64, _i32, _p]),
    "hxm_gemv_w8a16": (_st, [_p, _i64, _p, _i64, _i32, _p, _p, _i64, _i64, _i64, _i64, _p]),
    "hxm_w8a16_packed_bytes": (_i64, [_i64, _i64]),
    "hxm_prepack_w8a16": (_st, [_p, _i64, _i64, _i64, _p, _i64, _p]),
    "hxm_gemm_w8a16": (_st, [_p, _i64, _p, _i64, _p, _p, _i64, _i64, _i64, _i64, _cfgp, _p]),
    "hxm_gemm_w8a16_residual": (_st, [_p, _i64, _p, _i64, _p, _p, _i64, _p, _i64, _i64, _i64,
                                      _i64, _cfgp, _p]),
    "hxm_swiglu_packed_rows": (_i64, [_i64]),
    "hxm_swiglu_pack": (_st, [_p, _p, _i64, _p, _p, _i64, _i64, _p, _p, _p]),
    "hxm_gemm_w8a16_swiglu": (_st, [_p, _i64, _p, _p, _p, _i64, _i64, _i64, _i64, _cfgp, _p]),
    "hxm_w8a16_configs": (_i32, [_i32, _cfgp, _i32]),
    "hxm_tune_w8a16": (_st, [_i32, _p, _i64, _p, _i64, _p, _p, _i64, _i64, _i64, _i64, _i32,
                             _cfgp, ctypes.c_char_p, _i64, _p]),
    "hxm_resident_weight": (_st, [_p, _i64, _i64, _i64, _i32, _i32, ctypes.POINTER(_i64), _i32,
                                  ctypes.POINTER(_p), ctypes.POINTER(_i32), _p]),
    "hxm_softmax_rows": (_st, [_p, _i64, _p, _i64, _i64, _i64, _i32, _p]),
    "hxm_rmsnorm_rows": (_st, [_p, _i64, _p, _p, _i64, _i64, _i64, _f32, _i32, _p]),
    "hxm_layernorm_rows": (_st, [_p, _i64, _p, _p, _p, _i64, _p, _p, _i64, _i64, _f32, _i32,
                                 _p]),
    "hxm_probe_copy": (_st, [_p, _p, _i64, _p]),
    "hxm_probe_read": (_st, [_p, _i64, _p, _p]),
    "hxm_probe_mfma": (_st, [_p, _i64, _p, _i64, _i32, _i32, _i64, _i32, _p, _p]),
    "hxm_reason_string": (ctypes.c_char_p, [_i32]),
    "hxm_tile_ladder": (_i32, [_i64, ctypes.POINTER(_i64), _i32]),
    "hxm_hmx_tile_verdict": (_i32, [_i64, _i64, _i64, _i64]),
    "hxm_gpu_tile_verdict": (_i32, [_cfgp, _i32, _i64]),
    "hxm_gemm_configs": (_i32, [_i32, _cfgp, _i32]),
    "hxm_champion_gate": (_f64, [_f64]),
    "hxm_quantile_spread_cv": (_f64, [_f64, _f64, _f64]),
    "hxm_quantile": (_f64, [ctypes.POINTER(_f64), _i32, _f64]),
    "hxm_calibration_iters": (_i32, [_f64, _f64, _i32, _i32]),
    "hxm_champion_walk": (_i32, [ctypes.POINTER(_f64), ctypes.POINTER(_f64),
                                 ctypes.POINTER(_f64), _i32, _i32, ctypes.POINTER(_i32),
                                 ctypes.POINTER(_f64), ctypes.POINTER(_f64)]),
    "hxm_canary_status": (_i32, [_i32, _f64, _f64, _f64, _f64, ctypes.POINTER(_f64),
                                 ctypes.POINTER(_f64)]),
    "hxm_judge_round": (_i32, [ctypes.POINTER(ArmQuantiles), _i32, _i32,
                               ctypes.POINTER(ArmQuantiles), _f64, ctypes.POINTER(RoundVerdict),
                               ctypes.POINTER(_i32), ctypes.POINTER(_i32), ctypes.POINTER(_f64),
                               ctypes.POINTER(_f64)]),
    "hxm_tune_gemm": (_st, [_i32, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _i32, _cfgp,
                            ctypes.c_char_p, _i64, _p]),
    "hxm_tune_cache_clear": (None, []),
    "hxm_tune_cache_lookup": (_i32, [_i32, _i64, _i64, _i64, _cfgp]),
    "hxm_tune_cache_save": (_st, [ctypes.c_char_p]),
    "hxm_tune_cache_load": (_st, [ctypes.c_char_p, ctypes.POINTER(_i32)]),
    "hxm_abstain_string": (ctypes.c_char_p, [_i32]),
    "hxm_device_model_nominal": (None, [ctypes.POINTER(DeviceModel)]),
    "hxm_device_model_query": (_st, [ctypes.POINTER(DeviceModel)]),
    "hxm_predict_tile_time": (_i32, [_i64, _i64, _i64, _cfgp, _i32, _i32,
                                     ctypes.POINTER(DeviceModel),
                                     ctypes.POINTER(TilePredictionC)]),
    "hxm_rank_tile_candidates": (_i32, [_i64, _i64, _i64, _i32, _i32, _cfgp, _i32,
                                        ctypes.POINTER(DeviceModel), ctypes.POINTER(_i32)]),
    "hxm_cost_prune": (_i32, [ctypes.POINTER(TilePredictionC), _cfgp, _i32, _i32,
                              ctypes.POINTER(_i32), _f64, _f64, _f64, ctypes.POINTER(_i32),
                              ctypes.POINTER(_f64)]),
}


def _load():
    # One HIP runtime per process: torch ships its own libamdhip64.so.7.  If
    # torch is importable it is loaded first, so that libhxm's dependency on
    # that soname binds to the runtime torch's tensors and streams live in.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"libhxm.so not found at {LIB_PATH}: build it first "
            "(python -c 'import __graft_entry__ as g; g.build()' or make -C "
            "hexagon-mlir_amd/csrc)")
    cdll = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(cdll, name)
        fn.restype = res
        fn.argtypes = args
    return _Lib(cdll)


class _Entry:
    """One entry of the C ABI with its argument count checked.  ctypes
    rejects too few arguments but passes surplus ones on as if the function
    were variadic: a call with one argument too many would hand the library
    every pointer after it shifted by one, so the count is checked first."""

    __slots__ = ("_fn", "_n", "__name__")

    def __init__(self, fn, name):
        self._fn, self._n, self.__name__ = fn, len(fn.argtypes), name

    def __call__(self, *args):
        if len(args) != self._n:
            raise TypeError(f"{self.__name__} takes {self._n} arguments ({len(args)} given)")
        return self._fn(*args)


class _Lib:
    """libhxm.so with every entry of SIGNATURES bound as an _Entry."""

    def __init__(self, cdll):
        self._cdll = cdll
        for name in SIGNATURES:
            setattr(self, name, _Entry(getattr(cdll, name), name))


lib = _load()


def status_string(st: int) -> str:
    return lib.hxm_status_string(int(st)).decode()


def last_error() -> str:
    return lib.hxm_last_error().decode()


def check(st: int, fn: str) -> None:
    if st != HXM_OK:
        raise HxmError(st, last_error(), fn)
