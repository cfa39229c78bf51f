"""Host mirror of the reference's tile search (qcom_hexagon_backend/backend/
hmx_search.py) over the native implementation in libhxm.

Names, constants, argument meanings and report fields follow the reference
so that a caller of ``hmx_search`` finds the same surface.  The arithmetic
(ladder, verdicts, quantiles, the gate, the gated walk, the canary status)
lives once, in C++ behind the C ABI (csrc/search.hip); this module only
shapes the records.  On the GPU the legality budget is LDS instead of VTCM
(:func:`gpu_tile_verdict`) and the score is hipEvent microseconds instead of
pcycles; the record keys keep the reference's ``*_pcyc`` spelling where the
reference's own contract is mirrored.
"""
from __future__ import annotations

import ctypes
import math
from typing import Any, Mapping, NamedTuple, Optional, Sequence

from ._lib import GemmConfig, lib

# Constants (hmx_search.py:172-205, :1184-1214).
TILE_EDGE = 32
MIN_ROWS = 4
DEFAULT_VTCM_BUDGET = 8 * 1024 * 1024
CROUTON_ELEM_BYTES = 2
FRONTEND_MAX_BLOCK_NUMEL = 1048576
DEFAULT_LDS_BUDGET = 160 * 1024
CHAMPION_CV_FACTOR = 3.0
CHAMPION_MARGIN_FLOOR = 0.15

REASON_OK = "ok"
REASON_MIN_ROWS = "min-rows"
REASON_TILE_ALIGNMENT = "tile-alignment"
REASON_VTCM_BUDGET = "vtcm-budget"
REASON_FRONTEND_BLOCK_LIMIT = "frontend-block-limit"
REASON_LDS_BUDGET = "lds-budget"

CANARY_MISSING = "missing"
CANARY_UNMEASURED = "unmeasured"
CANARY_DRIFT = "drift"
CANARY_REFERENCE = "reference-established"
CANARY_OK = "ok"
ROUND_VALID = "valid"
ROUND_INVALID_CANARY = "invalid-canary"
CANARY_TILES = (32, 32, 32)
CANARY_SHAPE = (32, 32, 32)

_CANARY_STATUS = {0: CANARY_OK, 1: CANARY_MISSING, 2: CANARY_UNMEASURED, 3: CANARY_DRIFT,
                  4: CANARY_REFERENCE}


def _reason(code: int) -> str:
    return lib.hxm_reason_string(int(code)).decode()


def crouton_bytes(rows: int, n: int, k: int) -> int:
    """HmxTarget::croutonBytes (hmx_search.py:213-218)."""
    return (rows * k + k * n + rows * n) * CROUTON_ELEM_BYTES


def span_count(m: int, n: int, k: int, tiles) -> int:
    """ceil(M/BM)*ceil(N/BN)*ceil(K/BK) (hmx_search.py:221-232)."""
    bm, bn, bk = tiles
    return ((m + bm - 1) // bm) * ((n + bn - 1) // bn) * ((k + bk - 1) // bk)


def tile_ladder(extent: int) -> tuple:
    buf = (ctypes.c_int64 * 64)()
    n = lib.hxm_tile_ladder(int(extent), buf, 64)
    return tuple(int(buf[i]) for i in range(min(n, 64)))


def tile_verdict(bm: int, bn: int, bk: int, vtcm_budget: int = DEFAULT_VTCM_BUDGET) -> str:
    """The reference engine's legality predicate (hmx_search.py:269-292)."""
    return _reason(lib.hxm_hmx_tile_verdict(int(bm), int(bn), int(bk), int(vtcm_budget)))


def gpu_tile_verdict(config, dtype: int, lds_budget: int = DEFAULT_LDS_BUDGET) -> str:
    """The same lattice for a gfx950 kernel config (LDS budget, compiled list)."""
    cfg = config if isinstance(config, GemmConfig) else GemmConfig(*config)
    return _reason(lib.hxm_gpu_tile_verdict(ctypes.byref(cfg), int(dtype), int(lds_budget)))


class TileConfig(NamedTuple):
    tiles: tuple
    verdict: str

    @property
    def ok(self) -> bool:
        return self.verdict == REASON_OK

    @classmethod
    def tunables(cls) -> tuple:
        return ("BM", "BN", "BK")


def enumerate_tile_configs(m: int, n: int, k: int,
                           vtcm_budget: int = DEFAULT_VTCM_BUDGET) -> list:
    """hmx_search.py:315-332: the full ladder cross product with verdicts."""
    configs = [TileConfig(tiles=(bm, bn, bk), verdict=tile_verdict(bm, bn, bk, vtcm_budget))
               for bm in tile_ladder(m) for bn in tile_ladder(n) for bk in tile_ladder(k)]
    return sorted(configs)


def gemm_configs(dtype: int) -> list:
    """The compiled gfx950 GEMM configurations for an operand dtype."""
    buf = (GemmConfig * 64)()
    n = lib.hxm_gemm_configs(int(dtype), buf, 64)
    return [buf[i] for i in range(min(n, 64))]


def _is_finite(value) -> bool:
    if value is None:
        return False
    try:
        v = float(value)
    except (TypeError, ValueError):
        return False
    return math.isfinite(v)


def _f(value) -> float:
    return float(value) if _is_finite(value) else float("nan")


def _finite_or_none(value):
    return float(value) if _is_finite(value) else None


def _quantile(samples: Sequence[float], q: float) -> float:
    arr = (ctypes.c_double * max(1, len(samples)))(*[float(s) for s in samples])
    return float(lib.hxm_quantile(arr if samples else None, len(samples), float(q)))


def quantile_spread_cv(q20, q50, q80) -> float:
    return float(lib.hxm_quantile_spread_cv(_f(q20), _f(q50), _f(q80)))


def champion_gate(cv) -> float:
    return float(lib.hxm_champion_gate(_f(cv)))


def calibration_iters(perf_us: float, target_us: float = 2_000_000.0, lo: int = 5,
                      hi: int = 1000) -> int:
    return int(lib.hxm_calibration_iters(float(perf_us), float(target_us), int(lo), int(hi)))


def canary_config() -> dict:
    return {"cfg": "canary-32x32x32", "tiles": list(CANARY_TILES),
            "shape_mnk": list(CANARY_SHAPE)}


def _record_q50(record) -> Optional[float]:
    value = record.get("q50_pcyc") if isinstance(record, Mapping) else record
    return float(value) if _is_finite(value) else None


def canary_verdict(metrics, reference=None) -> dict:
    """hmx_search.canary_verdict (hmx_search.py:1292-1367)."""
    record = dict(status=CANARY_OK, healthy=True, q50_pcyc=None, cv=0.0,
                  reference_q50_pcyc=None, delta_pct=None, gate_pct=None, reason="")
    present = metrics is not None
    q50 = _record_q50(metrics) if present else None
    q20 = metrics.get("q20_pcyc") if isinstance(metrics, Mapping) else None
    q80 = metrics.get("q80_pcyc") if isinstance(metrics, Mapping) else None
    ref = _record_q50(reference)
    delta = ctypes.c_double()
    gate = ctypes.c_double()
    code = lib.hxm_canary_status(int(present), _f(q20), _f(q50), _f(q80), _f(ref),
                                 ctypes.byref(delta), ctypes.byref(gate))
    status = _CANARY_STATUS[code]
    if present and isinstance(metrics, Mapping):
        record["cv"] = quantile_spread_cv(q20, metrics.get("q50_pcyc"), q80)
    record["q50_pcyc"] = _finite_or_none(q50)
    if status == CANARY_MISSING:
        record.update(status=status, healthy=False,
                      reason=("no canary measurement rode with this round: without its "
                              "sentinel the round cannot tell a broken device from slow "
                              "configs, so it publishes no verdict"))
        return record
    if status == CANARY_UNMEASURED:
        record.update(status=status, healthy=False,
                      reason=("the canary config failed or printed no cycles: a "
                              "known-healthy config that cannot run indicts the device "
                              "or the launch path, not the config"))
        return record
    record["reference_q50_pcyc"] = _finite_or_none(ref)
    if status == CANARY_REFERENCE:
        record.update(status=status,
                      reason=("no healthy reference existed, so this run establishes it; "
                              "the round is valid and the next round can judge against "
                              "this median"))
        return record
    record["delta_pct"] = _finite_or_none(100.0 * delta.value)
    record["gate_pct"] = _finite_or_none(100.0 * gate.value)
    if status == CANARY_DRIFT:
        record.update(status=status, healthy=False,
                      reason=(f"the canary moved {100.0 * delta.value:+.1f}% from its "
                              f"reference, more than the {100.0 * gate.value:.1f}% gate: "
                              "same config, same build, same iteration count, so the "
                              "device state moved and every other number in this round "
                              "was taken under it"))
        return record
    record["reason"] = (f"the canary stayed within {100.0 * abs(delta.value):.1f}% of its "
                        f"reference (gate {100.0 * gate.value:.1f}%)")
    return record


def judge_champion_round(measurements, *, control=None, canary=None, canary_reference=None,
                         iters=None) -> dict:
    """hmx_search.judge_champion_round (hmx_search.py:1370-1571).

    The walk itself is hxm_champion_walk; this builds the same report."""
    canary_record = canary_verdict(canary, canary_reference)
    round_valid = bool(canary_record["healthy"])
    rows = []
    for entry in measurements:
        row = dict(entry)
        row["tiles_tuple"] = tuple(row.get("tiles") or ())
        rows.append(row)
    label_of = lambda r: str(r.get("cfg", ""))  # noqa: E731
    cv_of = lambda r: quantile_spread_cv(r.get("q20_pcyc"), r.get("q50_pcyc"),  # noqa: E731
                                         r.get("q80_pcyc"))
    measured = [r for r in rows if _record_q50(r) is not None]
    unmeasured = [label_of(r) for r in rows if _record_q50(r) is None]

    def as_control(row):
        if control is None:
            return False
        if str(control) == label_of(row):
            return True
        tiles = tuple(control) if not isinstance(control, str) else None
        return tiles is not None and tiles == row["tiles_tuple"]

    control_rows = [r for r in measured if as_control(r)]
    control_row = control_rows[0] if control_rows else None
    control_any = [r for r in rows if as_control(r)]
    ordered = sorted(measured, key=lambda r: (r["tiles_tuple"], label_of(r)))

    walk_note = ""
    start = -1
    if control_row is not None:
        start = next(i for i, r in enumerate(ordered) if r is control_row)
        walk_note = ("the incumbent starts at the manual control tile: the winner is judged "
                     "against it, so it defends the crown first")
    elif control_any:
        walk_note = ("the manual control tile was nominated but never measured (it scored "
                     "inf), so there is no arm to judge a win against")
    elif control is not None:
        walk_note = ("the nominated control arm is not among this round's measurements, so "
                     "there is no arm to judge a win against")
    elif ordered:
        start = 0
        walk_note = ("no control arm was nominated: the incumbent starts at the first "
                     "enumerated candidate, so the walk is deterministic but the starting "
                     "point is nominal")

    n = len(ordered)
    arr = lambda key: (ctypes.c_double * max(1, n))(*[_f(r.get(key)) for r in ordered])  # noqa
    outcome = (ctypes.c_int32 * max(1, n))()
    delta = (ctypes.c_double * max(1, n))()
    gate = (ctypes.c_double * max(1, n))()
    champ = -1
    comparisons, changes = [], []
    if start >= 0:
        champ = lib.hxm_champion_walk(arr("q20_pcyc"), arr("q50_pcyc"), arr("q80_pcyc"), n,
                                      start, outcome, delta, gate)
        # Replay the visit order to name the incumbent each challenger faced.
        inc = start
        step = 0
        for i in range(n):
            if i == start or outcome[i] < 0:
                continue
            ch, ic = ordered[i], ordered[inc]
            rec = dict(step=step, challenger=label_of(ch), incumbent=label_of(ic),
                       challenger_q50_pcyc=_finite_or_none(_record_q50(ch)),
                       incumbent_q50_pcyc=_finite_or_none(_record_q50(ic)),
                       delta_pct=_finite_or_none(100.0 * delta[i]),
                       cv=_finite_or_none(max(cv_of(ch), cv_of(ic))),
                       gate_pct=_finite_or_none(100.0 * gate[i]),
                       gate_form="max(3xCV, 15%)",
                       outcome="takeover" if outcome[i] == 1 else "kept")
            comparisons.append(rec)
            if outcome[i] == 1:
                changes.append(dict(rec))
                inc = i
            step += 1
    champion_row = ordered[champ] if champ >= 0 else None

    beats_control = None
    if control_row is not None and champion_row is not None:
        cv = max(cv_of(control_row), cv_of(champion_row))
        g = champion_gate(cv)
        if champion_row is control_row:
            beats_control = dict(delta_pct=0.0, cv=_finite_or_none(cv),
                                 gate_pct=_finite_or_none(100.0 * g),
                                 gate_form="max(3xCV, 15%)", significant=False,
                                 note=("the manual control tile kept the crown: no candidate "
                                       "beat it by the gate"))
        else:
            cq, wq = _record_q50(control_row), _record_q50(champion_row)
            d = (cq - wq) / cq
            beats_control = dict(
                delta_pct=_finite_or_none(100.0 * d), cv=_finite_or_none(cv),
                gate_pct=_finite_or_none(100.0 * g), gate_form="max(3xCV, 15%)",
                significant=bool(round_valid and d > g),
                note=("the champion beat the manual control tile by "
                      f"{100.0 * d:.1f}%, " + ("more than" if d > g else "not more than")
                      + f" the {100.0 * g:.1f}% gate"))
    significant = bool(round_valid and beats_control is not None
                       and beats_control["significant"])
    if not round_valid:
        note = ("the round is void (" + canary_record["status"] + "): "
                + canary_record["reason"] + ". The champion below is the walk's survivor, "
                "not a verdict.")
    elif beats_control is None:
        note = ("no control arm produced a measurement, so there is nothing to prove a win "
                "against: the champion is the walk's survivor (NOT-PROVEN, which is not the "
                "same as 'no effect')")
    elif beats_control["significant"]:
        note = f"the champion beat the manual control tile by more than the gate at iters={iters}"
    else:
        note = (f"the champion did not beat the manual control tile by more than the gate at "
                f"iters={iters}: NOT-PROVEN, which is not the same as 'no effect'")
    return dict(
        kind="hmx-search-champion",
        round_verdict=ROUND_VALID if round_valid else ROUND_INVALID_CANARY,
        iters=iters,
        gate=dict(form="max(3xCV, 15%)", cv_factor=CHAMPION_CV_FACTOR,
                  margin_floor=CHAMPION_MARGIN_FLOOR),
        canary=canary_record, walk_note=walk_note, measured_configs=len(measured),
        champion=label_of(champion_row) if champion_row is not None else None,
        champion_tiles=list(champion_row["tiles_tuple"]) if champion_row is not None else None,
        champion_q50_pcyc=(_finite_or_none(_record_q50(champion_row))
                           if champion_row is not None else None),
        control=label_of(control_row) if control_row is not None else None,
        control_tiles=list(control_row["tiles_tuple"]) if control_row is not None else None,
        beats_control=beats_control, champion_significant=significant,
        significance_note=note, changes=changes, comparisons=comparisons,
        unmeasured=unmeasured, cvs={label_of(r): _finite_or_none(cv_of(r)) for r in rows},
    )


def hexagon_bench(kernel_call, quantiles=(0.5, 0.2, 0.8), *, reps: int = 3,
                  verify=None) -> list:
    """hmx_search.hexagon_bench (:1109-1156) with a measured-time callable.

    ``kernel_call()`` returns one launch's time (any unit) or raises.  A bad
    config (exception or non-finite time) or a failed ``verify()`` scores
    inf on the first offending rep."""
    inf = [float("inf")] * len(quantiles)
    samples = []
    for _ in range(max(1, int(reps))):
        try:
            t = kernel_call()
        except (Exception, SystemExit):  # noqa: BLE001 - a bad config is inf
            return inf
        if not _is_finite(t):
            return inf
        if verify is not None:
            try:
                if not verify():
                    return inf
            except (Exception, SystemExit):  # noqa: BLE001
                return inf
        samples.append(float(t))
    return [_quantile(samples, q) for q in quantiles]


# ---- persisted tuning winners (C: hxm_tune_cache_save / _load / _lookup) ----

def tune_cache_lookup(op: int, m: int, n: int, k: int) -> Optional[GemmConfig]:
    """The cached tuning winner for (op, M, N, K), or None."""
    cfg = GemmConfig()
    return cfg if lib.hxm_tune_cache_lookup(int(op), m, n, k, ctypes.byref(cfg)) else None


def tune_cache_save(path: str) -> None:
    """Writes every cached winner to ``path``, keyed to this library build and
    device (backend/hmx_search.py:416-442 keys results on the build)."""
    from ._lib import check
    check(lib.hxm_tune_cache_save(str(path).encode()), "hxm_tune_cache_save")


def tune_cache_load(path: str) -> int:
    """Adds the winners saved in ``path`` to the cache; refuses a file of
    another build or device.  Returns how many entries were loaded."""
    from ._lib import check
    n = ctypes.c_int32(0)
    check(lib.hxm_tune_cache_load(str(path).encode(), ctypes.byref(n)), "hxm_tune_cache_load")
    return n.value


# ---- modeled cost: ordering and the conservative prune ---------------------
# hmx_search.predict_tile_pcyc (:778-887), rank_tile_candidates (:1030-1067),
# cost_prune (:916-1027), manifest_abstains (:895-913).  The arithmetic is C
# (hxm_predict_tile_time, hxm_rank_tile_candidates, hxm_cost_prune); this
# layer shapes the reference's records.  Times are microseconds, priced from
# a device model instead of a table of Hexagon leaf cells; the model's tier
# ("current" = read from this process's gfx950 device) plays the part of the
# reference's cell fingerprint tiers.

ABSTAIN_HEAT_BAND = "heat-band"
ABSTAIN_HEAT_CROSS = "heat-cross-boundary"
ABSTAIN_TAIL = "tail-blocks"
ABSTAIN_DTYPE = "dtype-no-cell"
ABSTAIN_MANIFEST = "manifest-strategy-unknown"
ABSTAIN_NO_CELL = "no-applicable-cell"
ABSTAIN_TABLE_MISSING = "table-missing"
_ABSTAIN_CODE = {None: 0, ABSTAIN_HEAT_BAND: 1, ABSTAIN_HEAT_CROSS: 2, ABSTAIN_TAIL: 3,
                 ABSTAIN_DTYPE: 4, ABSTAIN_MANIFEST: 5, ABSTAIN_NO_CELL: 6,
                 ABSTAIN_TABLE_MISSING: 7}

#: The modeled/measured band and the decision margin of the pruning rule
#: (hmx_search.py:731, :737): drop B only when lb(B) > 1.15 * 1.25/0.70 * ub(A).
COST_ENVELOPE = (0.70, 1.25)
PRUNE_MARGIN = 0.15

TIER_UNKNOWN, TIER_CURRENT, TIER_NOMINAL = "unknown", "current", "nominal"
_TIER = {0: TIER_UNKNOWN, 1: TIER_CURRENT, 2: TIER_NOMINAL}
_HEAT = {0: "cache", 1: "hbm", -1: "unknown"}
#: The priced items of one config: MFMA work, the L2 -> LDS fill, HBM bytes.
MODEL_ITEMS = ("mfma", "lds-fill", "hbm")

#: What a compiled config's "manifest" must say for cost_prune to act on it.
MANIFEST_VERDICT_OK = REASON_OK


class TilePrediction(NamedTuple):
    """One config's modeled interval (hmx_search.TilePrediction's fields;
    lb/ub/p50 in microseconds, NaN when abstaining)."""
    tiles: tuple
    lb: float
    ub: float
    p50: float
    heat: str
    units: tuple
    abstain: Optional[str]
    table_rev: str
    lb_tiers: tuple = ()


def nominal_model():
    """The spec-sheet gfx950 device model (tier "nominal": never drives a drop)."""
    from ._lib import DeviceModel
    m = DeviceModel()
    lib.hxm_device_model_nominal(ctypes.byref(m))
    return m


def device_model():
    """The model of this process's current device (needs a GPU)."""
    from ._lib import DeviceModel, check
    m = DeviceModel()
    check(lib.hxm_device_model_query(ctypes.byref(m)), "hxm_device_model_query")
    return m


def model_rev(model) -> str:
    """The model's version stamp: its tier and the rates it prices with."""
    return ("gpu-%s-%dcu-%.0f/%.0fmhz-%.0f/%.0fgbps-lds%.0f/%.0f-launch%.2f"
            % (_TIER.get(model.tier, TIER_UNKNOWN), model.cus, model.sclk_mhz_peak,
               model.sclk_mhz_sustained, model.hbm_gbps_peak, model.hbm_gbps_sustained,
               model.lds_fill_peak, model.lds_fill_sustained, model.launch_us))


def tiles_of(candidate) -> tuple:
    """A candidate's tile tuple: a GemmConfig, an object with ``.tiles`` or a
    bare tuple."""
    if isinstance(candidate, GemmConfig):
        return candidate.as_tuple()
    return tuple(candidate.tiles if hasattr(candidate, "tiles") else candidate)


def _config_of(candidate, dtype: int) -> GemmConfig:
    if isinstance(candidate, GemmConfig):
        return candidate
    t = tiles_of(candidate)
    if len(t) == 3:  # (BM, BN, BK): the compiled config with those tiles, if any
        for c in gemm_configs(dtype):
            if (c.bm, c.bn, c.bk) == t:
                return c
    return GemmConfig(*(list(t) + [0] * (7 - len(t)))[:7])


def _default_out(dtype: int) -> int:
    from ._lib import F16, I8, I32
    return I32 if dtype == I8 else F16


def predict_tile_time(m: int, n: int, k: int, config, *, dtype: int = 4,
                      out_dtype: Optional[int] = None, model=None) -> TilePrediction:
    """predict_tile_pcyc (hmx_search.py:778-887) for one compiled gfx950 config.

    ``dtype`` is the operand dtype code (``_lib.I8``, ``F16`` or ``BF16``);
    ``model`` defaults to :func:`nominal_model`."""
    from ._lib import TilePredictionC
    model = nominal_model() if model is None else model
    cfg = _config_of(config, dtype)
    out = TilePredictionC()
    od = _default_out(dtype) if out_dtype is None else out_dtype
    code = lib.hxm_predict_tile_time(int(m), int(n), int(k), ctypes.byref(cfg), int(dtype),
                                     int(od), ctypes.byref(model), ctypes.byref(out))
    abstain = None if code == 0 else lib.hxm_abstain_string(int(code)).decode()
    tier = _TIER.get(out.tier, TIER_UNKNOWN)
    return TilePrediction(tiles_of(config), out.lb_us, out.ub_us, out.p50_us,
                          _HEAT.get(out.heat, "unknown"), tuple(out.units), abstain,
                          model_rev(model), (tier,) * len(MODEL_ITEMS))


def rank_tile_candidates(shape, legal, *, dtype: int = 4, out_dtype: Optional[int] = None,
                         model=None) -> list:
    """rank_tile_candidates (hmx_search.py:1030-1067): a permutation of
    ``legal`` by (abstains last, modeled lower bound, span count, config)."""
    m, n, k = shape
    legal = list(legal)
    if not legal:
        return []
    model = nominal_model() if model is None else model
    cfgs = (GemmConfig * len(legal))(*[_config_of(c, dtype) for c in legal])
    order = (ctypes.c_int32 * len(legal))()
    od = _default_out(dtype) if out_dtype is None else out_dtype
    got = lib.hxm_rank_tile_candidates(int(m), int(n), int(k), int(dtype), int(od), cfgs,
                                       len(legal), ctypes.byref(model), order)
    assert got == len(legal)
    return [legal[order[i]] for i in range(len(legal))]


def manifest_record(config, dtype: int, lds_budget: int = DEFAULT_LDS_BUDGET) -> dict:
    """What the compiled-kernel table says about a config: the GPU's manifest."""
    return {"verdict": gpu_tile_verdict(_config_of(config, dtype), dtype, lds_budget)}


def manifest_abstains(record: Optional[Mapping[str, Any]]) -> Optional[str]:
    """manifest_abstains (hmx_search.py:895-913): a config no manifest vouches
    for (no record, or a verdict other than "ok") abstains."""
    if record is None or record.get("verdict") != MANIFEST_VERDICT_OK:
        return ABSTAIN_MANIFEST
    return None


def cost_prune(candidates, shape, *, control_tile=None, margin: float = PRUNE_MARGIN,
               envelope: tuple = COST_ENVELOPE, predictions: Optional[Mapping] = None,
               manifest_records: Optional[Mapping] = None, model=None, dtype: int = 4,
               out_dtype: Optional[int] = None):
    """cost_prune (hmx_search.py:916-1027): returns ``(kept, dropped, notes)``;
    ``kept`` keeps the caller's order, ``dropped`` holds (candidate, reason)."""
    from ._lib import TilePredictionC
    m, n, k = shape
    candidates = list(candidates)
    if predictions is None:
        predictions = {tiles_of(c): predict_tile_time(m, n, k, c, dtype=dtype,
                                                      out_dtype=out_dtype, model=model)
                       for c in candidates}
    count = len(candidates)
    preds = (TilePredictionC * max(1, count))()
    cfgs = (GemmConfig * max(1, count))()
    vouched = (ctypes.c_int32 * max(1, count))()
    control_tiles = tiles_of(control_tile) if control_tile is not None else None
    control = -1
    for i, cand in enumerate(candidates):
        t = tiles_of(cand)
        p = predictions[t]
        preds[i].lb_us, preds[i].ub_us, preds[i].p50_us = _f(p.lb), _f(p.ub), _f(p.p50)
        preds[i].abstain = _ABSTAIN_CODE.get(p.abstain, _ABSTAIN_CODE[ABSTAIN_NO_CELL])
        preds[i].tier = 1 if not any(tr != TIER_CURRENT for tr in p.lb_tiers) else 0
        cfgs[i] = GemmConfig(*(list(t) + [0] * 7)[:7])
        if manifest_records is not None:
            vouched[i] = 1 if manifest_abstains(manifest_records.get(t)) is None else 0
        if control < 0 and control_tiles is not None and t == control_tiles:
            control = i
    lo, hi = envelope
    kept_code = (ctypes.c_int32 * max(1, count))()
    threshold = ctypes.c_double(0.0)
    champ = lib.hxm_cost_prune(preds, cfgs, count, control,
                               vouched if manifest_records is not None else None,
                               float(margin), float(lo), float(hi), kept_code,
                               ctypes.byref(threshold))
    if champ == -2:
        raise ValueError("cost_prune: invalid margin or envelope")
    if champ < 0:
        return list(candidates), [], [
            "cost_prune: no priced candidate -- nothing compared, nothing dropped"]
    ch_t = tiles_of(candidates[champ])
    ch = predictions[ch_t]
    thr = threshold.value
    kept, dropped = [], []
    notes = [f"cost_prune: champion {ch_t} p50={ch.p50:.3f} lb={ch.lb:.3f} ub={ch.ub:.3f}; "
             f"drop when lb(B) > {thr:.3f} * ub(A)"]
    for i, cand in enumerate(candidates):
        t = tiles_of(cand)
        p = predictions[t]
        code = kept_code[i]
        if code == 0:
            dropped.append((cand, dict(tiles=list(t), lb=p.lb, ub=p.ub,
                                       champion_tiles=list(ch_t), champion_ub=ch.ub,
                                       ratio=p.lb / ch.ub, threshold=thr, margin=margin,
                                       envelope=list(envelope), table_rev=p.table_rev)))
            continue
        kept.append(cand)
        if code == 2:
            notes.append(f"cost_prune: {t} kept (control tile is the arm the winner is "
                         "judged against)")
        elif code == 3:
            notes.append(f"cost_prune: {t} kept (abstain {p.abstain})")
        elif code == 4:
            notes.append(f"cost_prune: {t} kept (abstain {ABSTAIN_MANIFEST})")
        elif code == 5:
            notes.append(f"cost_prune: {t} kept (lower bound rests on {p.lb_tiers} prices: "
                         "only a current-device model may drive a drop)")
    notes.append(f"cost_prune: kept {len(kept)}, dropped {len(dropped)}")
    return kept, dropped, notes
