"""bench.py's command line on the host: the one-GPU contract and the
option list.  Nothing here touches a device (the GPU count is checked
before the library is loaded)."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=300, cwd=ROOT)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _bench("--gpus", "2")
    assert r.returncode != 0
    assert "one GPU" in r.stderr and "--gpus 2" in r.stderr
    assert r.stdout == ""  # no JSON line for a run that did not happen


def test_help_lists_the_driver_options():
    r = _bench("--help")
    assert r.returncode == 0
    for opt in ("--gpus", "--steps", "--warmup", "--suite", "--config", "--only"):
        assert opt in r.stdout
