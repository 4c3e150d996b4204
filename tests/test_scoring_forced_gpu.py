"""Both MFMA scoring kernels at every query-row count: the library picks one kernel per row
count, so each is also run forced (ACTKV_SCORE_KERNEL=qreg | kslice) over 32..512 rows, in a
child process (the choice is read once per process), against the oracle."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.parametrize("kernel", ["qreg", "kslice"])
def test_forced_kernel_matches_the_oracle_at_every_row_count(kernel):
    env = dict(os.environ, ACTKV_SCORE_KERNEL=kernel)
    p = subprocess.run([sys.executable, "-u", os.path.join(HERE, "_forced_scoring.py")], env=env,
                       capture_output=True, text=True, timeout=100)
    print(p.stdout[-3000:], p.stderr[-3000:])
    assert p.returncode == 0, f"{kernel}: child exited {p.returncode}"
    assert "cases match the oracle" in p.stdout
