"""Tile-search host logic (hxm.search over csrc/search.hip) against the
expectations the reference's own contract tests state:
qcom_hexagon_backend/test/test_hmx_search_loop_contract.py (:100-113 the
twelve shapes, :340-354 bench quantiles, :361-469 verdict oracle and known
answers) and test_hmx_champion_criterion_contract.py (:123-364 the gate, the
gated walk, the canary)."""
import math

import pytest

import hxm
from hxm import search as S

INF = float("inf")

TWELVE_SHAPES = [
    (1, 8192, 8192), (1, 8192, 4096), (1, 4096, 8192), (1, 4096, 16384), (1, 16384, 4096),
    (8192, 8192, 1), (8192, 4096, 1), (4096, 8192, 1), (4096, 16384, 1),
    (1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096),
]


def _rule_verdict(bm, bn, bk, budget=8 * 1024 * 1024):
    """HmxTarget's rules in pipeline order, one rule per line (an
    independent formulation, as the reference test keeps its own)."""
    def p2(x):
        return x > 0 and 2 ** int(round(math.log2(x))) == x
    if not all(p2(d) for d in (bm, bn, bk)) or max(bm * bk, bk * bn, bm * bn) > 1 << 20:
        return "frontend-block-limit"
    if bm <= 4:
        return "min-rows"
    if bm % 32 or bn % 32 or bk % 32:
        return "tile-alignment"
    if (bm * bk + bk * bn + bm * bn) * 2 >= budget:
        return "vtcm-budget"
    return "ok"


def test_ladder_shape():
    assert S.tile_ladder(4096) == (32, 64, 128, 256, 512, 1024, 2048, 4096)
    assert S.tile_ladder(1) == (1, 32)       # the degenerate whole extent
    assert S.tile_ladder(100) == (32, 64, 128)  # padded, 100 itself is not a power of 2
    assert S.tile_ladder(16) == (16, 32)


def test_ladder_and_verdict_at_the_int64_edge():
    """The reference's Python integers are unbounded; the C restatement takes
    int64.  Up to 2^62 the ladder is the reference's (every power of two from
    32, 57 rungs at 2^62); above it the padded power of two, 2^63, has no
    int64 form and the ladder is refused.  The verdict's block-size products
    of powers of two near 2^62 are decided without forming them."""
    top = 1 << 62
    assert S.tile_ladder(top) == tuple(1 << e for e in range(5, 63))
    assert S.tile_ladder(top - 1) == S.tile_ladder(top)
    assert S.tile_ladder((1 << 61) + 1)[-1] == top
    for bad in (top + 1, (1 << 63) - 1):
        with pytest.raises(ValueError):
            S.tile_ladder(bad)
    for dims in [(top, top, top), (top, 32, 32), (32, top, 32), (32, 32, top), (1 << 40, 1, 1),
                 (1 << 31, 1 << 31, 1), (1024, 1024, 1), (1024, 1, 1024), (2048, 512, 1)]:
        assert S.tile_verdict(*dims) == _rule_verdict(*dims), dims


def test_enumerator_matches_rules_on_the_twelve_shapes():
    verdicts = set()
    for m, n, k in TWELVE_SHAPES:
        configs = S.enumerate_tile_configs(m, n, k)
        assert configs and configs == sorted(configs)
        for cfg in configs:
            assert cfg.verdict == _rule_verdict(*cfg.tiles), (m, n, k, cfg)
            verdicts.add(cfg.verdict)
    assert {S.REASON_MIN_ROWS, S.REASON_TILE_ALIGNMENT, S.REASON_OK} <= verdicts
    assert S.tile_verdict(1, 128, 8192) == S.REASON_MIN_ROWS
    assert S.tile_verdict(128, 1, 8192) == S.REASON_TILE_ALIGNMENT
    assert S.tile_verdict(32, 32, 32) == S.REASON_OK
    assert S.TileConfig.tunables() == ("BM", "BN", "BK")


def test_budget_boundary_is_strict():
    assert S.tile_verdict(1024, 1024, 1024) == S.REASON_OK
    assert S.tile_verdict(1024, 1024, 1024, vtcm_budget=4 * 1024 * 1024) == S.REASON_VTCM_BUDGET
    cb = S.crouton_bytes(32, 32, 32)
    assert S.tile_verdict(32, 32, 32, vtcm_budget=cb) == S.REASON_VTCM_BUDGET
    assert S.tile_verdict(32, 32, 32, vtcm_budget=cb + 1) == S.REASON_OK


def test_calibration_box():
    assert S.calibration_iters(10.0) == 1000
    assert S.calibration_iters(2_600_000.0) == 5
    assert S.calibration_iters(0.0) == 1000
    # quotients past int64 (the reference's Python int() has no such limit)
    assert S.calibration_iters(1.0, target_us=1e300) == 1000
    assert S.calibration_iters(1.0, target_us=-1e300) == 5


def test_bench_quantiles_and_failures():
    t = iter([1000.0, 2000.0, 3000.0])
    assert S.hexagon_bench(lambda: next(t), reps=3, verify=lambda: True) == [2000.0, 1400.0, 2600.0]

    def boom():
        raise RuntimeError("lds overflow")
    assert S.hexagon_bench(boom, reps=3) == [INF, INF, INF]
    calls = []

    def once():
        calls.append(1)
        return 5.0
    assert S.hexagon_bench(once, reps=3, verify=lambda: False) == [INF, INF, INF]
    assert len(calls) == 1, "a failed verify scores inf on the first rep"
    assert S.hexagon_bench(lambda: float("nan"), reps=2) == [INF, INF, INF]


def _row(cfg, tiles, q50, spread=None):
    if spread is None:
        spread = 0.02 * q50
    return dict(cfg=cfg, tiles=list(tiles), q50_pcyc=q50, q20_pcyc=q50 - spread,
                q80_pcyc=q50 + spread)


def _canary(q50=5000.0, spread=100.0):
    return _row("canary-32x32x32", S.CANARY_TILES, q50, spread=spread)


def test_gate_and_tie_goes_to_incumbent():
    assert (S.CHAMPION_CV_FACTOR, S.CHAMPION_MARGIN_FLOOR) == (3.0, 0.15)
    assert S.champion_gate(0.0) == 0.15
    assert abs(S.champion_gate(0.05) - 0.15) < 1e-12
    assert abs(S.champion_gate(0.10) - 0.30) < 1e-12
    assert abs(S.champion_gate(1.0) - 3.0) < 1e-12
    assert S.champion_gate(None) == 0.15
    assert S.quantile_spread_cv(980, 1000, 1020) == 0.04
    assert S.quantile_spread_cv(None, 1000, 1020) == 0.0
    assert S.quantile_spread_cv(980, INF, 1020) == 0.0
    assert S.quantile_spread_cv(0, 0, 0) == 0.0
    rows = [_row("ctrl", (32, 32, 32), 1000.0), _row("edge", (64, 32, 32), 850.0)]
    rep = S.judge_champion_round(rows, control="ctrl", canary=_canary())
    assert rep["champion"] == "ctrl" and rep["changes"] == []
    assert rep["comparisons"][0]["outcome"] == "kept"
    assert rep["start"] == "control" and rep["proof"] == "control-held"


def test_challenger_takes_crown_only_past_gate():
    rows = [_row("ctrl", (32, 32, 32), 1000.0), _row("A", (64, 32, 32), 700.0),
            _row("B", (32, 64, 32), 900.0), _row("C", (128, 32, 32), 640.0)]
    rep = S.judge_champion_round(rows, control="ctrl", iters=300, canary=_canary())
    assert rep["round_verdict"] == S.ROUND_VALID
    assert rep["champion"] == "A" and rep["champion_tiles"] == [64, 32, 32]
    assert [c["challenger"] for c in rep["changes"]] == ["A"]
    tk = rep["changes"][0]
    assert tk["incumbent"] == "ctrl" and tk["outcome"] == "takeover"
    assert abs(tk["delta_pct"] - 30.0) < 1e-9 and abs(tk["gate_pct"] - 15.0) < 1e-9
    assert {c["challenger"]: c["outcome"] for c in rep["comparisons"]} == {
        "B": "kept", "A": "takeover", "C": "kept"}
    assert rep["beats_control"]["significant"] is True
    assert abs(rep["beats_control"]["delta_pct"] - 30.0) < 1e-9
    assert rep["champion_significant"] is True and rep["iters"] == 300
    assert rep["proof"] == "proven"
    noisy = [_row("ctrl", (32, 32, 32), 1000.0, spread=50.0),
             _row("A", (64, 32, 32), 700.0, spread=35.0)]
    rep = S.judge_champion_round(noisy, control="ctrl", canary=_canary())
    assert rep["champion"] == "ctrl"
    assert abs(rep["comparisons"][0]["gate_pct"] - 30.0) < 1e-9


def test_no_control_arm_is_named_not_proven():
    rows = [_row("x", (32, 32, 32), 900.0), _row("y", (64, 32, 32), 500.0)]
    rep = S.judge_champion_round(rows, canary=_canary())
    assert rep["champion"] == "y" and rep["beats_control"] is None
    assert rep["start"] == "nominal" and rep["proof"] == "no-control"
    assert rep["champion_significant"] is False
    dead = rows + [_row("ctrl", (128, 128, 128), INF)]
    rep = S.judge_champion_round(dead, control=(128, 128, 128), canary=_canary())
    assert rep["control"] is None and rep["beats_control"] is None
    assert rep["start"] == "control-unmeasured" and rep["champion"] is None
    assert rep["proof"] == "no-control"
    rep = S.judge_champion_round(rows, control="nobody", canary=_canary())
    assert rep["start"] == "control-absent" and rep["champion"] is None


def test_unmeasured_config_is_per_config_fact():
    rows = [_row("ctrl", (32, 32, 32), 1000.0), _row("dead", (64, 64, 64), INF),
            _row("alive", (128, 32, 32), 700.0)]
    rep = S.judge_champion_round(rows, control="ctrl", canary=_canary())
    assert rep["unmeasured"] == ["dead"] and rep["champion"] == "alive"
    assert rep["round_verdict"] == S.ROUND_VALID and rep["champion_significant"] is True
    empty = S.judge_champion_round([_row("only", (32, 32, 32), INF)], canary=_canary())
    assert empty["champion"] is None and empty["unmeasured"] == ["only"]


def test_canary_voids_round():
    assert S.tile_verdict(*S.CANARY_TILES) == S.REASON_OK
    assert S.canary_config()["tiles"] == [32, 32, 32]
    assert S.span_count(*S.CANARY_SHAPE, S.CANARY_TILES) == 1
    rows = [_row("ctrl", (32, 32, 32), 1000.0), _row("A", (64, 32, 32), 700.0)]
    good = S.judge_champion_round(rows, control="ctrl", canary=_canary())
    assert good["canary"]["status"] == S.CANARY_REFERENCE and good["canary"]["healthy"]
    judged = S.judge_champion_round(rows, control="ctrl", canary=_canary(),
                                    canary_reference=_canary())
    assert judged["canary"]["status"] == S.CANARY_OK
    for canary in (_row("canary", S.CANARY_TILES, INF), None):
        rep = S.judge_champion_round(rows, control="ctrl", canary=canary)
        assert rep["round_verdict"] == S.ROUND_INVALID_CANARY
        assert rep["champion"] == "A" and rep["champion_significant"] is False
        assert rep["beats_control"]["significant"] is False
        assert rep["proof"] == "void" and rep["start"] == "control"
    ref = _canary(5000.0)
    rep = S.judge_champion_round(rows, control="ctrl", canary=_canary(8000.0),
                                 canary_reference=ref)
    assert rep["canary"]["status"] == S.CANARY_DRIFT and not rep["canary"]["healthy"]
    assert abs(rep["canary"]["delta_pct"] - 60.0) < 1e-9
    assert rep["round_verdict"] == S.ROUND_INVALID_CANARY and rep["proof"] == "void"
    assert S.canary_verdict(_canary(3000.0), ref)["status"] == S.CANARY_DRIFT
    steady = S.canary_verdict(_canary(5400.0), ref)
    assert steady["status"] == S.CANARY_OK and abs(steady["delta_pct"] - 8.0) < 1e-9
    assert S.canary_verdict(_canary(), None)["status"] == S.CANARY_REFERENCE
    assert S.canary_verdict(_canary(), _row("ref", S.CANARY_TILES, INF))["status"] == \
        S.CANARY_REFERENCE


def test_report_is_json_ready():
    import json
    rows = [_row("ctrl", (32, 32, 32), 1000.0), _row("dead", (64, 32, 32), INF)]
    for canary in (_canary(), None):
        rep = S.judge_champion_round(rows, control="ctrl", canary=canary)
        json.loads(json.dumps(rep, allow_nan=False))


@pytest.mark.parametrize("dtype", [hxm.I8, hxm.F16, hxm.BF16])
def test_gpu_lattice_admits_exactly_the_compiled_configs(dtype):
    cfgs = S.gemm_configs(dtype)
    assert cfgs
    eb = 1 if dtype == hxm.I8 else 2
    for c in cfgs:
        assert S.gpu_tile_verdict(c, dtype) == S.REASON_OK, c
        assert c.bk * eb in (64, 128) and 2 <= c.stages <= 4
        assert c.stages * (c.bm + c.bn) * c.bk * eb <= S.DEFAULT_LDS_BUDGET
    assert S.gpu_tile_verdict((2, 32, 128, 1, 1, 2, 1), dtype) == "min-rows"
    assert S.gpu_tile_verdict((48, 32, 128, 1, 1, 2, 1), dtype) == "frontend-block-limit"
    assert S.gpu_tile_verdict((512, 512, 256, 2, 2, 2, 1), dtype) == "lds-budget"
    assert S.gpu_tile_verdict((256, 256, 128 // eb, 2, 2, 4, 1), dtype) == "lds-budget"
    assert S.gpu_tile_verdict((64, 64, 128, 4, 4, 2, 1), dtype) == "tile-alignment"
    assert S.gpu_tile_verdict((512, 32, 32, 1, 1, 2, 1), dtype) == "no-kernel"


# ---- persisted tuning winners: the file contract (the device-side round trip is in
# ---- test_gpu_search.py) ----------------------------------------------------------

def test_tune_cache_file_contract(tmp_path):
    """The file names this library build; a file of another build, a file that
    is not a cache and a missing file are refused -- after hmx_search.py:416-442,
    a result never crosses a rebuild."""
    hxm.lib.hxm_tune_cache_clear()
    assert S.tune_cache_lookup(hxm.I8, 64, 64, 64) is None
    p = tmp_path / "tune.txt"
    S.tune_cache_save(str(p))
    lines = p.read_text().splitlines()
    assert lines[0] == "hxm-tune-cache 1" and lines[1].startswith("build ")
    assert lines[2].startswith("cus ") and len(lines) == 3     # an empty cache
    other = tmp_path / "other.txt"
    bid = int(lines[1].split()[1], 16)
    other.write_text("\n".join([lines[0], "build %016x" % (bid ^ 1), lines[2],
                                "4 64 64 64 64 64 128 2 2 2 1 5"]) + "\n")
    with pytest.raises(hxm.HxmError, match="another build"):
        S.tune_cache_load(str(other))
    bad = tmp_path / "bad.txt"
    bad.write_text("not a cache\n")
    with pytest.raises(hxm.HxmError, match="not a tuning cache"):
        S.tune_cache_load(str(bad))
    with pytest.raises(hxm.HxmError, match="cannot open"):
        S.tune_cache_load(str(tmp_path / "missing.txt"))


def test_walk_and_round_refuse_missing_arrays():
    """The C walk and round judge take caller arrays: a NULL array with rows
    to read, or a negative row count, is refused (-2) rather than read."""
    import ctypes
    q = (ctypes.c_double * 2)(1.0, 2.0)
    L = hxm.lib
    assert L.hxm_champion_walk(None, q, q, 2, 0, None, None, None) == -2
    assert L.hxm_champion_walk(q, q, q, -1, 0, None, None, None) == -2
    assert L.hxm_champion_walk(q, q, q, 2, 0, None, None, None) == 0
    assert L.hxm_judge_round(None, 2, 0, None, 0.0, None, None, None, None, None) == -2
