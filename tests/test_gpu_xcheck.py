"""ZKH_XCHECK=1: with the opt-in convention cross-checks on, matmul, logUp and Hadamard
proofs of several shapes must pass their "folded terminal == multi_dim_me" guards
(zkob_fc.cu:337-345, zkob_rescale.cu:151-165, zkob_glu.cu:186-192, :254-260).  The switch is
read once per process, so the proofs run in one child process (tests/xcheck_driver.py)."""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def test_convention_crosschecks_pass():
    env = dict(os.environ, ZKH_XCHECK="1")
    r = subprocess.run([sys.executable, "-u", os.path.join(HERE, "xcheck_driver.py")], env=env,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-3000:]
    assert "xcheck all ok" in r.stdout
