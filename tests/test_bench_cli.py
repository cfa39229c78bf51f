"""bench.py on the CPU: its command-line contract (more than one GPU, by flag
or by a launcher's WORLD_SIZE, is refused with a message and exit status 2
before anything touches torch or the GPU; this build measures one GPU) and
the per-config records of its result line, built from synthetic leg records."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(args, env_extra=None):
    env = dict(os.environ)
    env.update(env_extra or {})
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")] + args, cwd=ROOT,
                          env=env, capture_output=True, text=True, timeout=120)


def test_more_than_one_gpu_is_refused_by_flag():
    r = _run(["--gpus", "2", "--steps", "1", "--warmup", "0"])
    assert r.returncode == 2
    assert r.stdout == ""                       # no result line
    assert "one GPU" in r.stderr


def test_more_than_one_gpu_is_refused_by_world_size():
    r = _run(["--steps", "1"], {"WORLD_SIZE": "8", "RANK": "0", "LOCAL_RANK": "0"})
    assert r.returncode == 2 and r.stdout == "" and "one GPU" in r.stderr


def _bench():
    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    import bench                                 # stdlib imports only at module level
    return bench


def _timing(us, **extra):
    return {"q20_us": us * 0.99, "q50_us": us, "q80_us": us * 1.01, "us": us, **extra}


def _legs():
    return {
        "f16_matmul_256": _timing(2.2, TFLOPS=15.3),
        "mfma_ceiling_int8_gemm_4096": _timing(44.0, TOPS=3100.0),
        **{f"w8a16_gemv_M{M}": _timing(9.0 + M / 10, **{"GB/s": 5000.0, "ceiling_frac": 0.9,
                                                        "graph_us": 8.9, "graph_hbm_frac": 0.63})
           for M in (1, 4, 16)},
        "softmax_f16_8192x4096": _timing(20.0, **{"GB/s": 6700.0, "ceiling_frac": 1.0,
                                                   "graph_us": 20.1}),
        "rmsnorm_f16_8192x4096": _timing(20.0, **{"GB/s": 6700.0, "ceiling_frac": 1.0,
                                                   "graph_us": 20.0}),
        "mfma_ceiling_swiglu_ffn_2048x4096x11008": _timing(335.0),
        "swiglu_ffn_2048x4096x11008": _timing(460.0, TFLOPS=1200.0, graph_us=460.5,
                                              stages_us={"rmsnorm": 4.5, "gate_up_swiglu": 297.0},
                                              sclk_under_load={"median_mhz": 1700},
                                              tuned={"down": [256, 128, 64, 2, 2, 3, 1]}),
        "search_int8_4096": {"winner": [256, 256, 128, 2, 2, 2, 1], "winner_us": 56.5,
                             "proof": "control-held", "per_config": list(range(500))},
        "run_copy": {"error": "RuntimeError('x')"},
    }


def test_one_record_per_config_and_a_compact_line():
    """Every benchmark config gets its own record with q20/q50/q80, rate,
    peak fraction and ceiling fraction; the context legs keep a few fields
    each (bulk such as the tuner's per-config arrays stays out), so the
    printed line stays far below the driver's 16 KB tail."""
    import json
    b = _bench()
    head = _timing(56.0, TOPS=2450.0)
    cpu = {2: {"value": 1.0, "unit": "TOPS", "sample": "rows"}}
    rec = b.config_records(head, _legs(), cpu)
    assert sorted(rec) == ["1_f16_matmul_256", "2_int8_gemm_4096_dequant", "3_w8a16_gemv_M1",
                           "3_w8a16_gemv_M16", "3_w8a16_gemv_M4", "4_rmsnorm_f16_8192x4096",
                           "4_softmax_f16_8192x4096", "5_swiglu_ffn_2048x4096x11008"]
    r2 = rec["2_int8_gemm_4096_dequant"]
    assert r2["us"] == 56.0 and r2["frac"] == round(2450.0 / b.PEAK_INT8_TOPS, 4)
    assert r2["ceiling_frac"] == round(44.0 / 56.0, 4) and r2["cpu"]["unit"] == "TOPS"
    assert rec["1_f16_matmul_256"]["frac"] is None            # launch-bound: no roofline fraction
    assert rec["5_swiglu_ffn_2048x4096x11008"]["sclk_mhz"] == 1700
    extra = b.compact_extra(_legs())
    assert "per_config" not in extra["search_int8_4096"]
    assert "w8a16_gemv_M1" not in extra and extra["run_copy"] == {"error": "RuntimeError('x')"}
    assert len(json.dumps({"configs": rec, "extra": extra})) < 8000


def test_an_incomplete_leg_is_reported_in_its_own_record():
    """A leg that lacks a field its record needs becomes an error entry in
    that record; the headline and the other configs are still written."""
    b = _bench()
    legs = _legs()
    del legs["w8a16_gemv_M4"]["ceiling_frac"]
    del legs["swiglu_ffn_2048x4096x11008"]["stages_us"]
    rec = b.config_records(_timing(56.0, TOPS=2450.0), legs, {})
    assert "error" in rec["3_w8a16_gemv_M4"] and "error" in rec["5_swiglu_ffn_2048x4096x11008"]
    assert rec["3_w8a16_gemv_M1"]["us"] == 9.1 and rec["2_int8_gemm_4096_dequant"]["cpu"] is None
