"""CPU checks of bench.py's command line: a request for more than one GPU (or a launch under a
multi-rank world) exits with an explanation before anything touches a GPU, and unknown legs are
refused."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BENCH = os.path.join(ROOT, "bench.py")


def _run(args, env=None):
    e = dict(os.environ)
    e.update(env or {})
    return subprocess.run([sys.executable, BENCH] + args, capture_output=True, text=True, timeout=120, env=e)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _run(["--gpus", "2", "--steps", "1", "--warmup", "1"])
    assert r.returncode == 2, r.stdout + r.stderr
    assert "one GPU only" in r.stderr
    assert r.stdout.strip() == ""   # no JSON line


def test_a_multi_rank_launch_is_refused():
    r = _run(["--steps", "1"], env={"WORLD_SIZE": "8"})
    assert r.returncode == 2, r.stdout + r.stderr
    assert "one GPU only" in r.stderr


def test_unknown_legs_are_refused():
    r = _run(["--only", "prefill,nonsense"])
    assert r.returncode != 0
    assert "unknown legs" in r.stderr
