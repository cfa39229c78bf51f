"""The modeled cost of a GEMM config (hxm.search over csrc/search.hip):
predict_tile_pcyc / rank_tile_candidates / cost_prune
(qcom_hexagon_backend/backend/hmx_search.py:778-1067), checked against the
expectations of the reference's contract test
qcom_hexagon_backend/test/test_hmx_cost_prune_contract.py (:348-403 the
ordering is a deterministic permutation with abstainers last, :415-575 the
pruning rule's arithmetic and every way it must refuse) and against the
device's published peaks (the lower bound never beats them)."""
import ctypes
import math

import pytest

import hxm
from hxm import search as S
from hxm._lib import BF16, F16, F32, I8, I32, GemmConfig, TilePredictionC

TWELVE_SHAPES = [
    (1, 8192, 8192), (1, 8192, 4096), (1, 4096, 8192), (1, 4096, 16384), (1, 16384, 4096),
    (8192, 8192, 1), (8192, 4096, 1), (4096, 8192, 1), (4096, 16384, 1),
    (1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096),
]


def _fake(tiles, lb, ub, abstain=None, lb_tiers=("current",) * 3):
    return S.TilePrediction(tiles=tiles, lb=lb, ub=ub, p50=0.5 * (lb + ub), heat="cache",
                            units=(0, 0, 0), abstain=abstain, table_rev="test",
                            lb_tiers=lb_tiers)


def _current_model():
    m = S.nominal_model()
    m.tier = 1  # as if read from this process's gfx950 device
    return m


def test_prune_arithmetic_and_refusals_match_the_reference_contract():
    close, pricey, control = (32, 32, 32), (64, 64, 64), (128, 128, 128)
    cands = [close, pricey, control]
    preds = {close: _fake(close, 10.0, 10.0), pricey: _fake(pricey, 10_000.0, 10_000.0),
             control: _fake(control, 5.0, 5.0)}
    shape = (1024, 1024, 1024)

    kept, dropped, notes = S.cost_prune(cands, shape, predictions=preds)
    assert kept == [close, control]
    assert [c for c, _ in dropped] == [pricey]
    reason = dropped[0][1]
    assert reason["ratio"] == 2000.0
    assert abs(reason["threshold"] - 2.0535714285714286) < 1e-9
    assert reason["table_rev"] == "test"
    assert notes[0]["event"] == "champion" and notes[0]["tiles"] == control
    assert notes[-1] == {"event": "summary", "kept": 2, "dropped": 1}

    # the control tile is immune even when it is the expensive one
    preds[control] = _fake(control, 900.0, 900.0)
    preds[close] = _fake(close, 5.0, 5.0)
    kept, dropped, _ = S.cost_prune(cands, shape, control_tile=control, predictions=preds)
    assert control in kept and [c for c, _ in dropped] == [pricey]

    # margin -> inf is the identity
    kept, dropped, _ = S.cost_prune(cands, shape, control_tile=control,
                                    margin=float("inf"), predictions=preds)
    assert dropped == [] and sorted(kept) == sorted(cands)

    # an abstaining candidate is never dropped
    preds[pricey] = _fake(pricey, 1e9, 1e9, abstain=S.ABSTAIN_HEAT_BAND)
    kept, dropped, _ = S.cost_prune(cands, shape, control_tile=control, predictions=preds)
    assert dropped == [] and pricey in kept

    # a lower bound priced by anything but a current-device model never drops
    preds[pricey] = _fake(pricey, 1e9, 1e9, lb_tiers=("current", "current", "nominal"))
    kept, dropped, _ = S.cost_prune(cands, shape, control_tile=control, predictions=preds)
    assert dropped == [] and pricey in kept

    # no manifest record for a candidate -> kept; every record clean -> dropped again
    preds[pricey] = _fake(pricey, 1e9, 1e9)
    kept, dropped, _ = S.cost_prune(cands, shape, control_tile=control, predictions=preds,
                                    manifest_records={close: {"verdict": "ok"}})
    assert dropped == []
    kept, dropped, _ = S.cost_prune(cands, shape, control_tile=control, predictions=preds,
                                    manifest_records={t: {"verdict": "ok"} for t in cands})
    assert [c for c, _ in dropped] == [pricey]
    # a record whose verdict is not "ok" does not vouch either
    kept, dropped, _ = S.cost_prune(
        cands, shape, control_tile=control, predictions=preds,
        manifest_records={**{t: {"verdict": "ok"} for t in cands},
                          pricey: {"verdict": "lds-budget"}})
    assert dropped == []

    # nothing priced -> nothing dropped, and the notes say so
    none = {t: _fake(t, 1.0, 1.0, abstain=S.ABSTAIN_TAIL) for t in cands}
    kept, dropped, notes = S.cost_prune(cands, shape, predictions=none)
    assert dropped == [] and kept == cands
    assert notes[0]["event"] == "nothing-priced"

    # the same partition whatever the input order; kept keeps the caller's order
    a = S.cost_prune(cands, shape, control_tile=control, predictions=preds)
    b = S.cost_prune(cands[::-1], shape, control_tile=control, predictions=preds)
    assert b[0] == a[0][::-1]
    assert [c for c, _ in a[1]] == [c for c, _ in b[1]]

    assert S.COST_ENVELOPE == (0.70, 1.25) and S.PRUNE_MARGIN == 0.15


def test_prune_champion_tie_breaks_on_the_config_not_the_order():
    a, b, far = (64, 64, 32), (32, 32, 32), (128, 128, 32)
    preds = {a: _fake(a, 5.0, 5.0), b: _fake(b, 5.0, 5.0), far: _fake(far, 100.0, 100.0)}
    for order in ([a, b, far], [far, b, a]):
        kept, dropped, notes = S.cost_prune(order, (1024, 1024, 1024), predictions=preds)
        assert notes[0]["event"] == "champion" and notes[0]["tiles"] == (32, 32, 32)
        assert [c for c, _ in dropped] == [far]


def test_prune_refuses_a_bad_envelope():
    t = (32, 32, 32)
    with pytest.raises(ValueError):
        S.cost_prune([t], (32, 32, 32), predictions={t: _fake(t, 1.0, 1.0)},
                     envelope=(0.0, 1.25))
    with pytest.raises(ValueError):
        S.cost_prune([t], (32, 32, 32), predictions={t: _fake(t, 1.0, 1.0)}, margin=-1.0)


@pytest.mark.parametrize("dtype", [I8, F16, BF16])
def test_ordering_is_a_deterministic_permutation_with_abstainers_last(dtype):
    legal = S.gemm_configs(dtype)
    assert legal
    changed = False
    for m, n, k in TWELVE_SHAPES:
        fwd = S.rank_tile_candidates((m, n, k), legal, dtype=dtype)
        again = S.rank_tile_candidates((m, n, k), list(legal), dtype=dtype)
        rev = S.rank_tile_candidates((m, n, k), legal[::-1], dtype=dtype)
        key = lambda cs: [c.as_tuple() for c in cs]  # noqa: E731
        assert key(fwd) == key(again) == key(rev)
        assert sorted(key(fwd)) == sorted(key(legal))
        preds = [S.predict_tile_time(m, n, k, c, dtype=dtype) for c in fwd]
        flags = [p.abstain is not None for p in preds]
        assert flags == sorted(flags), (m, n, k, "an abstainer sorts before a priced one")
        priced = [p for p in preds if p.abstain is None]
        assert [p.lb for p in priced] == sorted(p.lb for p in priced)
        for p, q, c, d in zip(priced, priced[1:], fwd, fwd[1:]):
            if p.lb == q.lb:  # ties: span count, then the config fields
                assert (S.span_count(m, n, k, c.as_tuple()[:3]), c.as_tuple()) <= (
                    S.span_count(m, n, k, d.as_tuple()[:3]), d.as_tuple())
        spans = sorted(legal, key=lambda c: (S.span_count(m, n, k, c.as_tuple()[:3]),
                                             c.as_tuple()))
        changed |= key(spans) != key(fwd)
    # the model changes something on a real shape (it is not a no-op)
    assert changed


def test_each_abstain_class():
    c = S.gemm_configs(I8)[0]  # 256 x 256 x 128
    assert S.predict_tile_time(4096, 4096, 4096, c, dtype=F32).abstain == S.ABSTAIN_DTYPE
    assert S.predict_tile_time(4096, 4096, 4096, c, dtype=I8,
                               out_dtype=I8).abstain == S.ABSTAIN_DTYPE
    out = TilePredictionC()
    code = hxm.lib.hxm_predict_tile_time(4096, 4096, 4096, ctypes.byref(c), I8, I32, None,
                                         ctypes.byref(out))
    assert hxm.lib.hxm_abstain_string(code).decode() == S.ABSTAIN_TABLE_MISSING
    assert math.isnan(out.lb_us) and math.isnan(out.ub_us)
    assert S.predict_tile_time(4000, 4096, 4096, c, dtype=I8).abstain == S.ABSTAIN_TAIL
    assert S.predict_tile_time(4096, 4096, 4000, c, dtype=I8).abstain == S.ABSTAIN_TAIL
    # operands (4096 + 16384) x 8192 int8 = 160 MiB: between half the 256 MiB
    # cache and all of it
    assert S.predict_tile_time(4096, 16384, 8192, c, dtype=I8).abstain == S.ABSTAIN_HEAT_BAND
    # operands 128 MiB (cache-resident), with the int32 C 384 MiB (HBM)
    assert S.predict_tile_time(8192, 8192, 8192, c, dtype=I8).abstain == S.ABSTAIN_HEAT_CROSS
    bad = S.nominal_model()
    bad.cus = 0
    assert S.predict_tile_time(4096, 4096, 4096, c, dtype=I8,
                               model=bad).abstain == S.ABSTAIN_NO_CELL
    bad = S.nominal_model()
    bad.hbm_gbps_sustained = float("nan")
    assert S.predict_tile_time(4096, 4096, 4096, c, dtype=I8,
                               model=bad).abstain == S.ABSTAIN_NO_CELL
    # a config with no compiled kernel has no price
    assert S.predict_tile_time(4096, 4096, 4096, GemmConfig(512, 512, 32, 2, 2, 2, 1),
                               dtype=I8).abstain == S.ABSTAIN_NO_CELL
    assert S.manifest_record(c, I8) == {"verdict": "ok"}
    assert S.manifest_abstains(None) == S.ABSTAIN_MANIFEST


def test_extents_past_int64_tile_counts():
    """The reference's Python integers are unbounded; the C restatement's
    extents are int64.  Shapes whose tile count passes int64 have no cell
    (HBM-bound by heat, so only the count refuses them), the largest count
    that fits is priced, and the ranking's span tiebreak takes any extent."""
    c = S.gemm_configs(I8)[0]  # 256 x 256 x 128
    big = 1 << 40               # (2^32 tiles)^2 = 2^64 > 2^63
    assert S.predict_tile_time(big, big, 128, c, dtype=I8).abstain == S.ABSTAIN_NO_CELL
    fits = S.predict_tile_time(1 << 38, 1 << 38, 128, c, dtype=I8)   # 2^60 tiles
    assert fits.abstain is None and fits.units[0] == 1 << 60
    huge = (2 ** 62, 2 ** 62, 2 ** 62)
    legal = S.gemm_configs(I8)[:4]
    order = S.rank_tile_candidates(huge, legal, dtype=I8)
    assert sorted(order, key=lambda x: x.as_tuple()) == sorted(legal, key=lambda x: x.as_tuple())


@pytest.mark.parametrize("dtype,peak_ops_per_clk_cu", [(I8, 8192), (F16, 4096), (BF16, 4096)])
def test_lower_bound_never_beats_the_published_peaks(dtype, peak_ops_per_clk_cu):
    """MI355X: 256 CUs at 2.4 GHz, dense int8 8192 and f16/bf16 4096 ops per
    clock per CU (5.0 POP/s, 2.5 PFLOP/s), HBM 8 TB/s."""
    model = S.nominal_model()
    peak = model.cus * peak_ops_per_clk_cu * model.sclk_mhz_peak * 1e6
    shapes = [(4096, 4096, 4096), (2048, 2048, 2048), (1024, 1024, 1024), (2048, 4096, 11008 - 1024),
              (4096, 8192, 2048), (8192, 2048, 4096), (16384, 16384, 256)]
    priced = 0
    for m, n, k in shapes:
        for c in S.gemm_configs(dtype):
            p = S.predict_tile_time(m, n, k, c, dtype=dtype, model=model)
            if p.abstain is not None:
                continue
            priced += 1
            assert p.lb * 1e-6 >= 2.0 * m * n * k / peak * (1 - 1e-12)
            assert p.ub >= p.lb and p.p50 == 0.5 * (p.lb + p.ub)
            assert p.ub * 1e-6 >= model.launch_us * 1e-6 + 2.0 * m * n * k / (
                peak * model.sclk_mhz_sustained / model.sclk_mhz_peak) * (1 - 1e-12)
            eb = 1 if dtype == I8 else 2
            ob = 4 if dtype == I8 else 2
            hbm_bytes = (m * k + k * n) * eb + m * n * ob
            if p.heat == "hbm":
                assert p.lb * 1e-6 >= hbm_bytes / (model.hbm_gbps_peak * 1e9) * (1 - 1e-12)
            tiles = (m // c.bm) * (n // c.bn)
            assert p.units == (tiles, -(-tiles // model.cus), k // c.bk)
    assert priced > 10


def test_one_full_round_is_priced_at_the_mfma_peak():
    """int8 4096^3 with 256 x 256 tiles is exactly one tile per CU: the lower
    bound is the chip's dense peak, 2*4096^3 / (256 * 8192 * 2.4e9) s."""
    c = S.gemm_configs(I8)[0]
    assert (c.bm, c.bn) == (256, 256)
    p = S.predict_tile_time(4096, 4096, 4096, c, dtype=I8, out_dtype=F16)
    assert p.abstain is None and p.heat == "cache"
    assert p.lb == pytest.approx(2 * 4096 ** 3 / (256 * 8192 * 2.4e9) * 1e6, rel=1e-12)
    # doubling K (still cache-resident, one round) doubles the compute floor
    p2 = S.predict_tile_time(4096, 4096, 8192, c, dtype=I8, out_dtype=F16)
    assert p2.lb == pytest.approx(2 * p.lb, rel=1e-12)


def test_live_prune_on_the_nominal_model_drops_nothing_and_a_current_one_may():
    legal = S.gemm_configs(I8)
    shape = (4096, 4096, 4096)
    kept, dropped, notes = S.cost_prune(legal, shape)
    assert dropped == [] and len(kept) == len(legal)
    kept, dropped, notes = S.cost_prune(legal, shape, model=_current_model())
    assert len(kept) + len(dropped) == len(legal)
    for cand, reason in dropped:
        assert reason["lb"] > reason["threshold"] * reason["champion_ub"]
        assert reason["envelope"] == [0.70, 1.25]
    assert any("kept" in n and "dropped" in n for n in notes)
    # the model's own best (lowest p50) is never dropped
    preds = [S.predict_tile_time(*shape, c, dtype=I8) for c in legal]
    best = min(range(len(legal)), key=lambda i: (preds[i].p50, legal[i].as_tuple()))
    assert legal[best] in kept


def test_split_k_configs_are_legal_for_int8_only_and_priced_per_slice():
    base = S.gemm_configs(I8)[0]
    t = list(base.as_tuple())
    for s, want in [(2, "ok"), (4, "ok"), (16, "ok"), (3, "no-kernel"), (32, "no-kernel")]:
        t[6] = s
        assert S.gpu_tile_verdict(GemmConfig(*t), I8) == want, s
    f = list(S.gemm_configs(F16)[0].as_tuple())
    f[6] = 2
    assert S.gpu_tile_verdict(GemmConfig(*f), F16) == "no-kernel"
    # 512^2 x 16384: 4 tiles of 256^2 leave 252 CUs idle; a 16-way K split
    # fills 64 of them, so its floor is 16x lower
    t[6] = 1
    one = S.predict_tile_time(512, 512, 16384, GemmConfig(*t), dtype=I8)
    t[6] = 16
    sixteen = S.predict_tile_time(512, 512, 16384, GemmConfig(*t), dtype=I8)
    assert one.abstain is None and sixteen.abstain is None
    assert one.units == (4, 1, 128) and sixteen.units == (64, 1, 128)
    assert sixteen.lb == pytest.approx(one.lb / 16, rel=1e-12)
