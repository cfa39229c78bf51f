"""The admission planner on the CPU (hxm_plan_matmul / hxm_query_contraction
over csrc/gemm.hip): the plan / reason record of the reference's manifest
(qcom_hexagon_backend/include/hexagon/Dialect/Hmx/Transforms/HmxManifest.h
:78-100) and the refusal order of HmxTarget::queryContraction
(HmxTarget.h:195-218: dtype, then shape), extended by the GPU's config
lattice (frontend block limit, min-rows, tile alignment, LDS budget) and
its own limits (workspace budget, launch grid).  Planning touches no device."""
import pytest
import torch

import hxm
import hxm.search  # noqa: F401  (hxm.search.gemm_configs below)
from hxm import ops

I8, F16, BF16, F32 = torch.int8, torch.float16, torch.bfloat16, torch.float32


def plan(M, N, K, dt, od=None, **kw):
    return ops.plan_matmul(M, N, K, dt, od, **kw)


def test_admitted_plans_name_the_kernel_and_why():
    p = plan(4096, 4096, 4096, I8, torch.float16)
    assert p["plan"] == "mfma-full" and p["reason"] == "selected-aligned"
    assert p["source"] in ("default", "tuned") and p["k_slices"] == 1
    if p["source"] == "default":
        assert p["config"][:3] == (256, 256, 128) and p["tiles"] == 256
    assert p["threads"] == 256 and 0 < p["lds_bytes"] <= 160 * 1024
    assert p["workspace_bytes"] == 0          # resident [N, K] B: nothing to pack
    t = plan(4000, 4004, 4096, I8, torch.float16)   # N off the 32-wide edge
    assert t["plan"] == "mfma-tail" and t["reason"] == "selected-tail"
    kn = plan(512, 512, 512, F16, b_layout="kn")
    assert kn["workspace_bytes"] == 512 * 512 * 2   # the per-call [K, N] -> [N, K] pack


def test_f32_operands_plan_their_fp16_images():
    p = plan(100, 60, 36, F32)
    assert p["plan"] == "mfma-tail" and p["op"] == hxm.F32 and p["shape"] == (100, 60, 36)
    kp = 40                                        # K padded to a multiple of 8
    a_bytes = (100 * kp * 2 + 255) // 256 * 256
    assert p["workspace_bytes"] == a_bytes + 60 * kp * 2


@pytest.mark.parametrize("cfg,reason", [
    ((48, 32, 128, 1, 1, 2, 1), "frontend-block-limit"),
    ((2, 32, 128, 1, 1, 2, 1), "min-rows"),
    ((64, 64, 128, 4, 4, 2, 1), "tile-alignment"),
    ((512, 512, 256, 2, 2, 2, 1), "lds-budget"),
    ((512, 32, 32, 1, 1, 2, 1), "no-kernel"),
])
def test_a_callers_config_is_refused_with_the_lattices_reason(cfg, reason):
    p = plan(1024, 1024, 1024, I8, config=cfg)
    assert p["plan"] == "refused" and p["reason"] == reason and p["source"] == "caller"
    assert hxm.last_error().startswith(reason)


def test_refusal_order_dtype_then_arguments_then_shape():
    # dtype first, whatever the shape
    assert plan(0, 8, 24, I8, torch.float32)["reason"] == "unsupported-dtype"
    assert plan(0, 8, 24, I8)["reason"] == "invalid-argument"
    assert plan(8, 8, 24, I8)["reason"] == "tile-alignment"      # K bytes not 16-aligned
    assert plan(8, 8, 8, F16)["reason"] == "selected-tail"       # 16 bytes of fp16 K
    assert plan(8, 8, 4, F32)["plan"] == "mfma-tail"             # f32: K padded in the pack


def test_plan_class_uses_the_32_wide_edge_for_every_kernel():
    """The plan classes follow the 32-wide MFMA edge (the reference's
    queryContraction tileEdge) also where the direct small-output kernel,
    whose own tiles are 16 wide, takes the shape."""
    p = plan(48, 48, 64, F16)
    assert p["config"][:3] == (16, 16, 32)          # the small-output kernel
    assert p["plan"] == "mfma-tail" and p["reason"] == "selected-tail"
    q = plan(64, 96, 64, F16)
    assert q["config"][:3] == (16, 16, 32)
    assert q["plan"] == "mfma-full" and q["reason"] == "selected-aligned"


def test_split_k_limits():
    base = hxm.search.gemm_configs(hxm.I8)[0].as_tuple()[:6]
    ok = plan(512, 512, 16384, I8, config=base + (16,))
    assert ok["plan"] == "mfma-full" and ok["k_slices"] == 16
    assert ok["workspace_bytes"] == 16 * 512 * 512 * 4
    big = plan(4096, 4096, 4096, I8, config=base + (8,))           # 8 planes of 64 MiB
    assert big["plan"] == "refused" and big["reason"] == "workspace-budget"
    # The largest extents the planner admits: 16 planes of (2^30 - 1)^2 int32
    # would pass 2^63 bytes; the budget check must not form that product.
    huge = plan(2 ** 30 - 1, 2 ** 30 - 1, 4096, I8, config=base + (16,))
    assert huge["plan"] == "refused" and huge["reason"] == "workspace-budget"
    edge = plan(1024, 4096, 4096, I8, config=base + (16,))          # exactly 256 MiB
    assert edge["plan"] == "mfma-full" and edge["workspace_bytes"] == 16 * 1024 * 4096 * 4
    f16 = plan(512, 512, 512, F16, config=hxm.search.gemm_configs(hxm.F16)[0].as_tuple()[:6] + (2,))
    assert f16["reason"] == "no-kernel"


def test_query_contraction_agrees_with_the_planner():
    import ctypes
    out = ctypes.c_int32()
    for shape, dt in [((256, 256, 256), hxm.F16), ((300, 260, 4112), hxm.I8),
                      ((64, 64, 40), hxm.I8)]:
        st = hxm.lib.hxm_query_contraction(*shape, dt, dt, hxm.I32 if dt == hxm.I8 else dt,
                                           ctypes.byref(out))
        p = plan(*shape, {hxm.F16: F16, hxm.I8: I8}[dt])
        assert out.value == {"mfma-full": 0, "mfma-tail": 1, "refused": -1}[p["plan"]]
        assert (st == 0) == (p["plan"] != "refused")


def test_a_query_leaves_the_last_call_record_alone():
    before = ops.last_plan()
    plan(1024, 1024, 1024, I8, config=(2, 32, 128, 1, 1, 2, 1))
    assert ops.last_plan() == before


def test_small_outputs_plan_the_direct_kernel():
    """f16 / bf16 outputs of at most 512 16x16 tiles with 0 < K <= 256 default to
    the direct-load small kernel (one 64-thread wave per 16x16 tile, no LDS);
    larger outputs, larger K and int8 keep the LDS-staged tiles; a caller may
    name the small config, and is refused where it does not apply."""
    small = (16, 16, 32, 1, 1, 0, 1)
    for dt in (F16, BF16):
        p = plan(256, 256, 256, dt)                      # the fp16 256^3 benchmark shape
        assert p["config"] == small and p["source"] == "default"
        assert p["threads"] == 64 and p["tiles"] == 256 and p["lds_bytes"] == 0
        assert p["plan"] == "mfma-full" and p["workspace_bytes"] == 0
    t = plan(300, 260, 200, F16)
    assert t["config"] == small and t["plan"] == "mfma-tail" and t["tiles"] == 19 * 17
    assert plan(256, 256, 512, F16)["config"] != small                # K above 256
    assert plan(512, 512, 256, F16)["config"] != small                # 1024 tiles
    assert plan(256, 256, 256, I8)["config"] != small
    kn = plan(128, 128, 128, F16, b_layout="kn")
    assert kn["config"] == small and kn["workspace_bytes"] == 128 * 128 * 2
    named = plan(64, 64, 64, F16, config=small)
    assert named["config"] == small and named["source"] == "caller"
    refused = plan(1024, 1024, 1024, F16, config=small)
    assert refused["plan"] == "refused" and refused["reason"] == "no-kernel"
    assert plan(64, 64, 64, I8, config=small)["reason"] == "no-kernel"
