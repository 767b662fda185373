"""bench.py's command line on the CPU: the cases that must stop before any device work -- a
request for more than one GPU and an unknown leg name -- exit with status 2 and a message."""
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def run(*args):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = run("--gpus", "2")
    assert r.returncode == 2
    assert "exactly one GPU" in r.stderr
    assert r.stdout == ""


def test_unknown_leg_is_refused():
    r = run("--legs", "gemv,c9")
    assert r.returncode == 2
    assert "unknown legs ['c9']" in r.stderr
