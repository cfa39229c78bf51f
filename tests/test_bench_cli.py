"""bench.py's command-line contract on the CPU: more than one GPU (by flag or
by a launcher's WORLD_SIZE) is refused with a message and exit status 2
before anything touches torch or the GPU; this build measures one GPU."""
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
