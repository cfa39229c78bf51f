"""The C ABI boundary on the CPU: libhxm.so loads, exports every symbol that
include/hxm.h declares, and refuses bad arguments on the host before any
launch -- with the manifest-style reason vocabulary -- without a GPU."""
import ctypes
import os
import re
import subprocess

import pytest

import hxm
from hxm import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hxm.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hxm_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", hxm.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (hxm_\w+)", out))
    missing = [s for s in declared_symbols() if s not in exported]
    assert not missing, missing
    for s in declared_symbols():
        assert getattr(hxm.lib, s) is not None


def test_binding_checks_the_argument_count():
    """ctypes would pass a surplus argument on, shifting every pointer after
    it; the binding refuses the call before it reaches the library."""
    import pytest as _pytest
    for name, (_, args) in _lib.SIGNATURES.items():
        fn = getattr(hxm.lib, name)
        with _pytest.raises(TypeError, match="takes"):
            fn(*([None] * (len(args) + 1)))
        if args:
            with _pytest.raises(TypeError):
                fn(*([None] * (len(args) - 1)))


def test_status_strings_and_version():
    assert hxm.status_string(0) == "ok"
    assert hxm.status_string(3) == "unsupported-shape"
    assert hxm.version().startswith("hxm ")


def _gpu_present():
    import torch
    return torch.cuda.is_available()


class _Fake:
    """Stand-in device addresses for a machine with no GPU: every call below
    must be refused on the host, so none of them is ever dereferenced."""

    def __call__(self, nbytes):
        return 16


class _Real:
    """Real device buffers of the declared sizes, for a machine with a GPU:
    should a refusal ever regress into a launch, it stays inside them."""

    def __init__(self):
        import torch
        self.torch, self.keep = torch, []

    def __call__(self, nbytes):
        t = self.torch.zeros(max(int(nbytes), 16), dtype=self.torch.uint8, device="cuda:0")
        self.keep.append(t)
        return t.data_ptr()


def _check_refusals(buf):
    L = hxm.lib
    # int8 GEMM with K not a multiple of 16 bytes -> tile-alignment
    st = L.hxm_gemm_i8(buf(8 * 24), 24, buf(8 * 24), 24, hxm.B_NK, buf(8 * 8 * 4), 8, 8, 8, 24,
                       0, None, None)
    assert st == _lib.HXM_UNSUPPORTED_SHAPE
    assert hxm.last_error().startswith("tile-alignment")
    # negative extent -> invalid argument
    st = L.hxm_gemm_i8(buf(256), 32, buf(256), 32, hxm.B_NK, buf(256), 8, -1, 8, 32, 0, None,
                       None)
    assert st == _lib.HXM_INVALID_ARG
    # int8 A/B with a float C is not an admitted matmul -> unsupported-dtype
    st = L.hxm_matmul(buf(4 * 32), 32, buf(32 * 4), 4, hxm.B_KN, buf(64), 4, 4, 4, 32, hxm.I8,
                      hxm.F16, 0, None, None)
    assert st == _lib.HXM_UNSUPPORTED_DTYPE
    assert hxm.last_error().startswith("unsupported-dtype")
    # leading dimension smaller than the row
    st = L.hxm_softmax_rows(buf(64), 4, buf(64), 8, 2, 8, hxm.F16, None)
    assert st == _lib.HXM_INVALID_ARG
    # int8 softmax is refused
    st = L.hxm_softmax_rows(buf(16), 8, buf(16), 8, 2, 8, hxm.I8, None)
    assert st == _lib.HXM_UNSUPPORTED_DTYPE
    # gemv: K not a multiple of 16
    st = L.hxm_gemv_w8a16(buf(48), 24, buf(8 * 24), 24, hxm.W_NK, buf(16), buf(16), 8, 1, 8, 24,
                          None)
    assert st == _lib.HXM_UNSUPPORTED_SHAPE
    # an unknown B layout
    st = L.hxm_gemm_i8(buf(256), 32, buf(256), 32, 7, buf(256), 8, 8, 8, 32, 0, None, None)
    assert st == _lib.HXM_INVALID_ARG
    # HBM probes: a length that is not a multiple of 16, overlapping buffers
    src = buf(64)
    assert L.hxm_probe_copy(src, buf(64), 24, None) == _lib.HXM_INVALID_ARG
    assert L.hxm_probe_copy(src, src + 16, 32, None) == _lib.HXM_INVALID_ARG
    assert "overlap" in hxm.last_error()
    assert L.hxm_probe_read(src, 32, None, None) == _lib.HXM_INVALID_ARG


def _span_refusals():
    """Rows 16 MiB apart: 256 rows of a tile would span 4 GiB of 32-bit
    offsets (checked with stand-in addresses only: the refusal precedes any
    use of them, and these sizes are not worth allocating)."""
    L = hxm.lib
    st = L.hxm_gemm_i8(16, 1 << 24, 16, 32, hxm.B_NK, 16, 8, 8, 8, 32, 0, None, None)
    assert st == _lib.HXM_UNSUPPORTED_SHAPE
    assert hxm.last_error().startswith("tile-alignment") and "2 GiB" in hxm.last_error()
    st = L.hxm_gemm_w8a16(16, 32, 16, 1 << 24, 16, 16, 8, 8, 8, 32, None, None)
    assert st == _lib.HXM_UNSUPPORTED_SHAPE and "2 GiB" in hxm.last_error()
    # A packed W8A16 image past 2^21 - 32 slabs: the GEMV's 32-bit buffer
    # offsets would wrap.  One slab fewer is admitted up to the device check.
    for slabs, refused in (((1 << 21) - 31, True), ((1 << 21) - 32, False)):
        K = slabs * 64
        st = L.hxm_gemv_w8a16(16, K, 16, K, hxm.W_PACKED, 16, 16, 8, 1, 8, K, None)
        if refused:
            assert st == _lib.HXM_UNSUPPORTED_SHAPE and "packed image" in hxm.last_error()
        else:
            assert st == _lib.HXM_NO_DEVICE
    # Resident images the pack would refuse are refused before the weight is
    # hashed: a GEMM image past the pack's grid (K > 65535 * 32), a W8A16
    # image past the GEMV's 32-bit extents.  At the limit the call goes on
    # to the device check.
    img, img_dt = ctypes.c_void_p(), ctypes.c_int32()

    def resident(rows, cols, kind):
        return L.hxm_resident_weight(16, cols, rows, cols, hxm.I8, -1, None, kind,
                                     ctypes.byref(img), ctypes.byref(img_dt), None)
    assert resident(65535 * 32 + 16, 16, _lib.IMAGE_GEMM) == _lib.HXM_UNSUPPORTED_SHAPE
    assert "launch grid" in hxm.last_error()
    assert resident(65535 * 32, 16, _lib.IMAGE_GEMM) == _lib.HXM_NO_DEVICE
    assert resident(2 ** 31 - 1, 16, _lib.IMAGE_W8A16) == _lib.HXM_UNSUPPORTED_SHAPE
    assert "beyond the pack's extents" in hxm.last_error()
    assert resident(16, 2 ** 31 - 64, _lib.IMAGE_W8A16) == _lib.HXM_UNSUPPORTED_SHAPE
    assert resident(1 << 16, 1 << 16, _lib.IMAGE_W8A16) == _lib.HXM_NO_DEVICE  # a 4 GiB image
    assert resident(1 << 20, 1 << 20, _lib.IMAGE_W8A16) == _lib.HXM_UNSUPPORTED_SHAPE  # 1 TiB
    # The MFMA probe's per-wave count is bounded (a launch stays short).
    assert L.hxm_probe_mfma(16, 64, 16, 64, hxm.I8, hxm.I8, (1 << 24) + 32, 1, 16,
                            None) == _lib.HXM_INVALID_ARG
    assert L.hxm_probe_mfma(16, 64, 16, 64, hxm.I8, hxm.I8, 1 << 24, 1, 16,
                            None) == _lib.HXM_NO_DEVICE


@pytest.mark.skipif("_gpu_present()", reason="a GPU box counts its gfx950 devices; "
                    "test_gpu_ops_contract.py covers it there")
def test_device_count_is_zero_without_a_gpu():
    assert hxm.lib.hxm_device_count() == 0


@pytest.mark.skipif("_gpu_present()", reason="stand-in addresses are for machines without a GPU; "
                    "test_refusals_with_device_buffers covers a GPU box")
def test_refusals_happen_before_launch():
    _check_refusals(_Fake())
    _span_refusals()


@pytest.mark.gpu
def test_refusals_with_device_buffers():
    _check_refusals(_Real())


@pytest.mark.skipif("_gpu_present()")
def test_valid_call_without_gpu_reports_no_device():
    st = hxm.lib.hxm_softmax_rows(16, 8, 16, 8, 2, 8, hxm.F16, None)
    assert st == _lib.HXM_NO_DEVICE
    assert hxm.last_error().startswith("no-device")


def test_query_contraction_plans():
    plan = ctypes.c_int32()
    L = hxm.lib
    assert L.hxm_query_contraction(256, 256, 256, hxm.F16, hxm.F16, hxm.F16,
                                   ctypes.byref(plan)) == 0 and plan.value == 0
    assert L.hxm_query_contraction(4096, 11000, 4096, hxm.I8, hxm.I8, hxm.I32,
                                   ctypes.byref(plan)) == 0 and plan.value == 1
    # int8 K not 16-byte aligned
    assert L.hxm_query_contraction(64, 64, 40, hxm.I8, hxm.I8, hxm.I32,
                                   ctypes.byref(plan)) == _lib.HXM_UNSUPPORTED_SHAPE
    assert plan.value == -1
    # f32 operands are admitted (quantised to fp16 by the pack, HMXAPI.h:107-137)
    assert L.hxm_query_contraction(64, 64, 64, hxm.F32, hxm.F32, hxm.F32,
                                   ctypes.byref(plan)) == 0 and plan.value == 0
    assert L.hxm_query_contraction(64, 64, 64, hxm.I8, hxm.F16, hxm.F32,
                                   ctypes.byref(plan)) == _lib.HXM_UNSUPPORTED_DTYPE


def test_product_has_no_oracle_dependency():
    """The product path never routes through the CPU oracle."""
    pkg = os.path.join(ROOT, "hexagon-mlir_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".py", ".hip", ".h", ".cpp")) or f == "Makefile":
                text = open(os.path.join(dirpath, f), errors="ignore").read()
                assert "oracle" not in text.lower().replace("oracle/oracle", ""), f


# ---- memref descriptors (test/utils/dsp/include/common.h:15-30) -> (ptr, ld) ----

def test_memref_descriptor_conversion():
    from hxm import memref as mr
    d = mr.describe(0x10000, rows=8, cols=24, ld=40, offset=3 * 40 + 8)
    op = mr.operand(d, hxm.F16)
    assert op == (0x10000 + (3 * 40 + 8) * 2, 40, 8, 24)
    assert mr.operand(mr.describe(0x10000, 1, 24, 0), hxm.F32) == (0x10000, 24, 1, 24)
    with pytest.raises(hxm.HxmError, match="tile-alignment"):
        mr.operand(mr.describe(0x10000, 8, 24, 48, inner_stride=2), hxm.F16)
    with pytest.raises(hxm.HxmError, match="invalid-argument"):
        mr.operand(mr.describe(0x10000, 8, 24, 16), hxm.F16)        # rows overlap
    with pytest.raises(hxm.HxmError, match="invalid-argument"):
        mr.operand(mr.describe(0x10000, 8, 24, 24, offset=-1), hxm.F16)
    assert ctypes.sizeof(mr.MemRefDescriptor2D) == 8 + 8 + 8 + 16 + 16


@pytest.mark.skipif("_gpu_present()", reason="stand-in addresses are for machines without a GPU")
def test_memref_call_reaches_the_abi_and_is_refused_there():
    """A descriptor-shaped call with K = 12 f16 (24 bytes, not a 16-byte
    multiple) is converted, handed to hxm_matmul and refused there."""
    from hxm import memref as mr
    A = mr.describe(0x10000, 8, 12, 12)
    B = mr.describe(0x20000, 12, 8, 8)
    C = mr.describe(0x30000, 8, 8, 8)
    with pytest.raises(hxm.HxmError, match="tile-alignment"):
        mr.matmul(A, B, C, ab_dtype=hxm.F16, c_dtype=hxm.F16)
    assert hxm.last_error().startswith("tile-alignment")
