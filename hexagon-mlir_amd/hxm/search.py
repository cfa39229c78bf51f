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

from ._lib import ArmQuantiles, GemmConfig, RoundVerdict, lib

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
    if n < 0:
        raise ValueError(f"extent {extent} is above 2^62: its padded power of two has no "
                         "64-bit form")
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


def _arm(record) -> ArmQuantiles:
    """A measurement record (``q20_pcyc`` / ``q50_pcyc`` / ``q80_pcyc``) as the
    C arm; missing or non-finite quantiles become NaN."""
    get = record.get if isinstance(record, Mapping) else (lambda _k: None)
    return ArmQuantiles(_f(get("q20_pcyc")), _f(get("q50_pcyc")), _f(get("q80_pcyc")))


#: hxm_judge_round's codes (include/hxm.h), by value.
START_CODES = ("control", "nominal", "control-unmeasured", "control-absent", "empty")
PROOF_CODES = ("proven", "within-gate", "control-held", "no-control", "void")
GATE_FORM = "max(3xCV, 15%)"


def canary_verdict(metrics, reference=None) -> dict:
    """The canary's status for one round (hmx_search.canary_verdict,
    hmx_search.py:1292-1367; decided by hxm_canary_status).  ``metrics`` is
    the canary's measurement record or None; ``reference`` the previous
    round's canary record (or its median)."""
    present = metrics is not None
    arm = _arm(metrics)
    ref = _record_q50(reference)
    delta, gate = ctypes.c_double(), ctypes.c_double()
    code = lib.hxm_canary_status(int(present), arm.q20, arm.q50, arm.q80, _f(ref),
                                 ctypes.byref(delta), ctypes.byref(gate))
    status = _CANARY_STATUS[code]
    return dict(status=status, healthy=status in (CANARY_OK, CANARY_REFERENCE),
                q50_pcyc=_finite_or_none(arm.q50),
                cv=quantile_spread_cv(arm.q20, arm.q50, arm.q80) if present else 0.0,
                reference_q50_pcyc=_finite_or_none(ref) if present else None,
                delta_pct=_finite_or_none(100.0 * delta.value),
                gate_pct=_finite_or_none(100.0 * gate.value))


def _matches(control, label: str, tiles: tuple) -> bool:
    if control is None:
        return False
    if isinstance(control, str):
        return control == label
    return tuple(control) == tiles


def judge_champion_round(measurements, *, control=None, canary=None, canary_reference=None,
                         iters=None) -> dict:
    """The verdict of one search round (the decision of
    hmx_search.judge_champion_round, hmx_search.py:1370-1571).

    ``measurements``: records with ``cfg`` (label), ``tiles`` and the
    ``q20_pcyc`` / ``q50_pcyc`` / ``q80_pcyc`` quantiles (a non-finite median
    means the config never ran).  ``control`` names the control arm by label
    or tiles.  The decision is hxm_judge_round's: the arms are handed over
    sorted by (tiles, label), which is the walk order.  ``start`` and
    ``proof`` carry its codes (START_CODES / PROOF_CODES)."""
    arms = sorted(({"label": str(m.get("cfg", "")), "tiles": tuple(m.get("tiles") or ()),
                    "rec": m} for m in measurements), key=lambda a: (a["tiles"], a["label"]))
    n = len(arms)
    hits = [i for i, a in enumerate(arms) if _matches(control, a["label"], a["tiles"])]
    if control is None:
        ctl = -1
    elif not hits:
        ctl = -2
    else:  # a measured match if there is one
        ctl = next((i for i in hits if _record_q50(arms[i]["rec"]) is not None), hits[0])

    c_arms = (ArmQuantiles * max(1, n))(*[_arm(a["rec"]) for a in arms])
    canary_arm = _arm(canary) if canary is not None else None
    ref = _record_q50(canary_reference)
    v = RoundVerdict()
    outcome, faced = (ctypes.c_int32 * max(1, n))(), (ctypes.c_int32 * max(1, n))()
    delta, gate = (ctypes.c_double * max(1, n))(), (ctypes.c_double * max(1, n))()
    lib.hxm_judge_round(c_arms, n, ctl, ctypes.byref(canary_arm) if canary_arm else None,
                        _f(ref), ctypes.byref(v), outcome, faced, delta, gate)

    def q50(i):
        return _finite_or_none(c_arms[i].q50)

    def cv(i):
        return quantile_spread_cv(c_arms[i].q20, c_arms[i].q50, c_arms[i].q80)

    comparisons = []
    for i in range(n):
        if outcome[i] < 0:
            continue
        j = faced[i]
        comparisons.append(dict(
            step=len(comparisons), challenger=arms[i]["label"], incumbent=arms[j]["label"],
            challenger_q50_pcyc=q50(i), incumbent_q50_pcyc=q50(j),
            delta_pct=_finite_or_none(100.0 * delta[i]), cv=_finite_or_none(max(cv(i), cv(j))),
            gate_pct=_finite_or_none(100.0 * gate[i]), gate_form=GATE_FORM,
            outcome="takeover" if outcome[i] == 1 else "kept"))

    champ = v.champion if v.champion >= 0 else None
    has_control = START_CODES[v.start] == "control"
    proof = PROOF_CODES[v.proof]
    versus = None
    if has_control and champ is not None:
        versus = dict(delta_pct=_finite_or_none(100.0 * v.control_delta),
                      cv=_finite_or_none(v.control_cv),
                      gate_pct=_finite_or_none(100.0 * v.control_gate), gate_form=GATE_FORM,
                      significant=proof == "proven")
    return dict(
        kind="hmx-search-champion",
        round_verdict=ROUND_VALID if v.valid else ROUND_INVALID_CANARY,
        iters=iters,
        gate=dict(form=GATE_FORM, cv_factor=CHAMPION_CV_FACTOR,
                  margin_floor=CHAMPION_MARGIN_FLOOR),
        canary=canary_verdict(canary, canary_reference),
        start=START_CODES[v.start], proof=proof, measured_configs=int(v.measured),
        champion=arms[champ]["label"] if champ is not None else None,
        champion_tiles=list(arms[champ]["tiles"]) if champ is not None else None,
        champion_q50_pcyc=q50(champ) if champ is not None else None,
        control=arms[ctl]["label"] if has_control else None,
        control_tiles=list(arms[ctl]["tiles"]) if has_control else None,
        beats_control=versus, champion_significant=proof == "proven",
        changes=[dict(c) for c in comparisons if c["outcome"] == "takeover"],
        comparisons=comparisons,
        unmeasured=[a["label"] for i, a in enumerate(arms) if q50(i) is None],
        cvs={a["label"]: _finite_or_none(cv(i)) for i, a in enumerate(arms)},
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


#: hxm_cost_prune's kept codes (include/hxm.h), by value.
KEPT_CODES = ("dropped", "band", "control", "abstains", "unvouched", "not-current",
              "nothing-priced")


def cost_prune(candidates, shape, *, control_tile=None, margin: float = PRUNE_MARGIN,
               envelope: tuple = COST_ENVELOPE, predictions: Optional[Mapping] = None,
               manifest_records: Optional[Mapping] = None, model=None, dtype: int = 4,
               out_dtype: Optional[int] = None):
    """The conservative prune (hmx_search.cost_prune, hmx_search.py:916-1027;
    decided by hxm_cost_prune).  Returns ``(kept, dropped, notes)``: ``kept``
    in the caller's order, ``dropped`` as (candidate, record) pairs, and
    ``notes`` as event records: ``{"event": "champion", ...}`` (or
    ``"nothing-priced"``) first, one ``{"event": "kept", "why": ...}`` per
    candidate kept for a reason other than lying inside the band, and a
    closing ``{"event": "summary", ...}``."""
    from ._lib import TilePredictionC
    m, n, k = shape
    candidates = list(candidates)
    if predictions is None:
        predictions = {tiles_of(c): predict_tile_time(m, n, k, c, dtype=dtype,
                                                      out_dtype=out_dtype, model=model)
                       for c in candidates}
    count = len(candidates)
    tiles = [tiles_of(c) for c in candidates]
    preds = (TilePredictionC * max(1, count))()
    cfgs = (GemmConfig * max(1, count))()
    vouched = (ctypes.c_int32 * max(1, count))()
    for i, t in enumerate(tiles):
        p = predictions[t]
        preds[i].lb_us, preds[i].ub_us, preds[i].p50_us = _f(p.lb), _f(p.ub), _f(p.p50)
        preds[i].abstain = _ABSTAIN_CODE.get(p.abstain, _ABSTAIN_CODE[ABSTAIN_NO_CELL])
        preds[i].tier = 1 if all(tr == TIER_CURRENT for tr in p.lb_tiers) else 0
        cfgs[i] = GemmConfig(*(list(t) + [0] * 7)[:7])
        if manifest_records is not None:
            vouched[i] = manifest_abstains(manifest_records.get(t)) is None
    wanted = tiles_of(control_tile) if control_tile is not None else None
    control = tiles.index(wanted) if wanted in tiles else -1
    lo, hi = envelope
    codes = (ctypes.c_int32 * max(1, count))()
    threshold = ctypes.c_double(0.0)
    champ = lib.hxm_cost_prune(preds, cfgs, count, control,
                               vouched if manifest_records is not None else None,
                               float(margin), float(lo), float(hi), codes,
                               ctypes.byref(threshold))
    if champ == -2:
        raise ValueError("cost_prune: invalid margin or envelope")
    if champ < 0:
        return candidates, [], [{"event": "nothing-priced", "candidates": count},
                                {"event": "summary", "kept": count, "dropped": 0}]
    best = predictions[tiles[champ]]
    notes = [{"event": "champion", "tiles": tiles[champ], "p50": best.p50, "lb": best.lb,
              "ub": best.ub, "threshold": threshold.value}]
    kept, dropped = [], []
    for i, cand in enumerate(candidates):
        p, why = predictions[tiles[i]], KEPT_CODES[codes[i]]
        if why == "dropped":
            dropped.append((cand, dict(tiles=list(tiles[i]), lb=p.lb, ub=p.ub,
                                       champion_tiles=list(tiles[champ]), champion_ub=best.ub,
                                       ratio=p.lb / best.ub, threshold=threshold.value,
                                       margin=margin, envelope=list(envelope),
                                       table_rev=p.table_rev)))
            continue
        kept.append(cand)
        if why != "band":
            note = {"event": "kept", "tiles": tiles[i], "why": why}
            if why == "abstains":
                note["abstain"] = p.abstain
            elif why == "not-current":
                note["lb_tiers"] = tuple(p.lb_tiers)
            notes.append(note)
    notes.append({"event": "summary", "kept": len(kept), "dropped": len(dropped)})
    return kept, dropped, notes
