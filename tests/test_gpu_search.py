"""The measured tile search on the GPU: every candidate is launched, checked
bit-exact against the control config, timed; the winner is cached and used by
later calls (hmx_search.py's autotune sweep + hexagon_bench +
judge_champion_round)."""
import numpy as np
import pytest
import torch

import hxm.ops as ops
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype,M,N,K", [(torch.int8, 512, 512, 512),
                                         (torch.float16, 256, 256, 256),
                                         (torch.bfloat16, 256, 256, 256)])
def test_tune_gemm_picks_a_verified_winner(dev, dtype, M, N, K):
    g = torch.Generator().manual_seed(M)
    if dtype == torch.int8:
        A = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8)
        B = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
        out = torch.empty(M, N, dtype=torch.int32, device=dev)
    else:
        A = (torch.rand(M, K, generator=g) * 2 - 1).to(dtype)
        B = (torch.rand(N, K, generator=g) * 2 - 1).to(dtype)
        out = torch.empty(M, N, dtype=dtype, device=dev)     # C of the operands' dtype
    Ad, Bd = A.to(dev), B.to(dev)
    best, rep = ops.tune_gemm(Ad, Bd, out, reps=5)
    print(rep, flush=True)
    assert rep["round_verdict"] in ("valid", "invalid-canary")
    assert rep["champion"] is not None
    measured = [c for c in rep["configs"] if c["q50"] is not None]
    assert measured and all(c["verified"] for c in measured)
    win = rep["configs"][rep["champion"]]
    assert win["tiles"][:2] == [best.bm, best.bn]
    # the control arm is what an untuned call runs: the default tile, unsplit
    ctl = rep["configs"][rep["control"]]
    assert ctl["split_k"] == 1
    if dtype == torch.int8:
        assert ctl["tiles"][:2] == [64, 64]
    else:
        # 256 16x16 output tiles, K = 256: the direct-load small-output kernel,
        # against which the LDS-staged tiles are verified within tolerance
        assert ctl["tiles"] == [16, 16, 32] and ctl["stages"] == 0
        assert len(measured) > 1
    assert rep["start"] == "control" and rep["proof"] in (
        "proven", "control-held", "within-gate", "void")
    # later calls with no config use the cached winner and stay correct
    if dtype == torch.int8:
        C = ops.gemm_i8(Ad, Bd, b_layout="nk").cpu().numpy()
        assert np.array_equal(C, orc.gemm_i8(A.numpy(), B.numpy(), b_nk=True))
    else:
        C = ops.matmul(Ad, Bd, b_layout="nk").float().cpu().numpy()
        bits = lambda t: t.view(torch.int16).numpy().view(np.uint16)  # noqa: E731
        name = "f16" if dtype == torch.float16 else "bf16"
        ref = orc.to_f32(orc.matmul(bits(A), bits(B), ab_dtype=name, c_dtype=name, b_nk=True),
                         name)
        np.testing.assert_allclose(C, ref, rtol=1e-2, atol=1e-3)
        assert ops.last_plan()["config"] == best.as_tuple()


def test_tune_cache_save_load_round_trip(dev, tmp_path):
    """A tuned winner survives save -> clear -> load on the same build and
    device; entries naming a tile this build did not compile, out-of-range fields and
    over-long lines are skipped."""
    import hxm
    from hxm import search as S
    hxm.lib.hxm_tune_cache_clear()
    M = N = K = 512
    g = torch.Generator().manual_seed(5)
    A = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(dev)
    B = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
    out = torch.empty(M, N, dtype=torch.int32, device=dev)
    best, rep = ops.tune_gemm(A, B, out, reps=3)
    assert rep["champion"] is not None
    win = S.tune_cache_lookup(hxm.I8, M, N, K)
    assert win is not None and win.as_tuple() == best.as_tuple()
    p = tmp_path / "tune.txt"
    S.tune_cache_save(str(p))
    bm, bn, bk, wm, wn, st, sk = best.as_tuple()
    cfg = f"{bm} {bn} {bk} {wm} {wn} {st} {sk}"
    with open(p, "a") as f:
        f.write("4 1024 1024 1024 96 96 128 2 2 2 1 3\n")   # no such compiled tile
        f.write(f"4 1536 1536 1536 {bm + 2 ** 32} {bn} {bk} {wm} {wn} {st} {sk} 3\n")  # wraps
        f.write(f"4 1536 1536 1536 {cfg} 0\n")               # reps out of range
        f.write(f"4 -1 1536 1536 {cfg} 3\n")                 # negative extent
        # over-long line whose tail alone would read as a valid entry
        f.write("9" + " " * 254 + f"4 2048 2048 2048 {cfg} 3\n")
    hxm.lib.hxm_tune_cache_clear()
    assert S.tune_cache_lookup(hxm.I8, M, N, K) is None
    assert S.tune_cache_load(str(p)) == 1
    assert S.tune_cache_lookup(hxm.I8, M, N, K).as_tuple() == best.as_tuple()
    for n in (1024, 1536, 2048):
        assert S.tune_cache_lookup(hxm.I8, n, n, n) is None
    C = ops.gemm_i8(A, B, b_layout="nk").cpu().numpy()     # runs the reloaded winner
    assert np.array_equal(C, orc.gemm_i8(A.cpu().numpy(), B.cpu().numpy(), b_nk=True))
    hxm.lib.hxm_tune_cache_clear()


@pytest.mark.parametrize("M,N,K", [(4096, 4096, 4096), (512, 512, 16384)])
def test_cost_model_floor_holds_and_prune_keeps_the_measured_winner(dev, M, N, K):
    """predict_tile_pcyc / cost_prune (hmx_search.py:778-1027) priced by this
    device: every measured config time is at or above its modeled lower bound,
    and the conservative prune never drops the config measured fastest.  The
    under-filled 512x512x16384 shape brings in the K-split candidates, so the
    split terms of the model (S workgroup rows, K/S per slice, the partial
    planes and the second launch) are held against measured times too."""
    from hxm import search as S
    from hxm._lib import I8, I32
    model = S.device_model()
    assert model.tier == 1 and model.cus > 0 and model.sclk_mhz_peak > 0
    g = torch.Generator().manual_seed(11)
    A = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int8).to(dev)
    B = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8).to(dev)
    out = torch.empty(M, N, dtype=torch.int32, device=dev)
    _, rep = ops.tune_gemm(A, B, out, reps=5)
    assert rep["unit"] == "us"
    measured = {}
    for c in rep["configs"]:
        if c["q50"] is None or not c["verified"]:
            continue
        t = tuple(c["tiles"][:3])
        cfg = next(x for x in S.gemm_configs(I8) if (x.bm, x.bn, x.bk) == t
                   and x.stages == c["stages"])
        cfg.split_k = c["split_k"]
        measured[cfg.as_tuple()] = (cfg, c["q50"])
    assert len(measured) >= 3
    if M == 512:
        assert any(key[6] > 1 for key in measured), "no K-split candidate was measured"
    preds = {}
    for key, (cfg, q50) in measured.items():
        p = S.predict_tile_time(M, N, K, cfg, dtype=I8, out_dtype=I32, model=model)
        assert p.abstain is None, (key, p.abstain)
        print(f"{key}: measured {q50:.1f} us, model lb {p.lb:.1f} p50 {p.p50:.1f} "
              f"ub {p.ub:.1f}", flush=True)
        assert q50 >= p.lb, (key, q50, p.lb)
        preds[key] = p
    cands = [cfg for cfg, _ in measured.values()]
    kept, dropped, notes = S.cost_prune(cands, (M, N, K), predictions=preds)
    print(notes, flush=True)
    fastest = min(measured.values(), key=lambda v: v[1])[0]
    assert fastest.as_tuple() in [c.as_tuple() for c in kept]


def rand_i8(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-127, 128, shape, generator=g, dtype=torch.int8)


def test_tune_calibrated_repetitions_and_the_cost_model(dev):
    """reps=0: every launched config gets hxm_calibration_iters' count (5 to
    1000 timed launches) from its timed warm call; the cost model prices every
    candidate on this device, the control is never priced out, a priced-out
    config is not launched (no quantiles) and cannot win, and each measured
    time is at or above the config's modeled lower bound."""
    M = N = K = 1024
    A = rand_i8((M, K), 91).to(dev)
    B = rand_i8((N, K), 92).to(dev)
    out = torch.empty(M, N, dtype=torch.int32, device=dev)
    print("tune int8 1024^3 with calibrated repetitions", flush=True)
    best, rep = ops.tune_gemm(A, B, out, reps=0)
    assert rep["reps"] == "calibrated"
    assert rep["prune"]["priced"] is True
    cfgs = rep["configs"]
    assert rep["prune"]["dropped"] == sum(c["pruned"] for c in cfgs)
    assert not cfgs[rep["control"]]["pruned"]
    for c in cfgs:
        assert c["model_lb_us"] is not None and c["model_ub_us"] is not None
        if c["pruned"]:
            assert c["q50"] is None and c["samples"] == 0
        elif c["q50"] is not None:
            assert 5 <= c["samples"] <= 1000
            assert c["q50"] >= c["model_lb_us"]
    assert rep["champion"] is not None and not cfgs[rep["champion"]]["pruned"]
    C = ops.gemm_i8(A, B, b_layout="nk").cpu().numpy()
    assert np.array_equal(C, orc.gemm_i8(A.cpu().numpy(), B.cpu().numpy(), b_nk=True))
