"""bench.py's command line: invalid runs are rejected before any device work (the reference's
tests/test_bench.py:35 rejects zero iterations the same way), and more than one GPU is refused
with the reason."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True,
                          text=True, timeout=120, cwd=ROOT)


@pytest.mark.parametrize("args,msg", [
    (["--steps", "0"], "--steps must be at least 1"),
    (["--warmup", "-1"], "--warmup must not be negative"),
    (["--ora", "--ora-rounds", "0"], "must be at least 1"),
    (["--ora-short", "-1"], "--ora-short must not be negative"),
    (["--serve", "--serve-action", "60", "--serve-steps", "48"], "--serve-action must be between"),
])
def test_invalid_runs_are_rejected(args, msg):
    p = _run(*args)
    assert p.returncode == 2 and msg in p.stderr


def test_more_than_one_gpu_is_refused_with_the_reason():
    p = _run("--gpus", "2")
    assert p.returncode == 2 and "one GPU only" in p.stderr
