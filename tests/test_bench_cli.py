"""bench.py's command line, without a GPU: the refusals that come before any
device work."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _bench("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU only" in r.stderr and r.stdout == ""


def test_no_timed_steps_is_refused():
    r = _bench("--steps", "0")
    assert r.returncode == 2
    assert "--steps must be at least 1" in r.stderr


def test_every_single_part_mode_is_listed():
    r = _bench("--help")
    assert r.returncode == 0
    for flag in ("--pipeline-only", "--pipeline-layers", "--pipeline-step-sync", "--compaction-only",
                 "--decode-layouts", "--layout-launch", "--device-search-only", "--h2o-only"):
        assert flag in r.stdout, flag
