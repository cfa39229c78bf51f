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
