"""Argument handling of the zkob_*-compatible drivers, checked without a GPU: every request
here is refused before a device context is made.  `--claims` needs its arguments
(zkob_fc.cu:1224-1228 takes three, zkob_rescale.cu:528-532 and the SwiGLU and RoPE drivers
two), the privacy modes and unknown flags answer exit status 2, and a bad mode prints usage
with status 2."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = {n: os.path.join(ROOT, "zk-hillclimb_amd", n) for n in
       ("zkh_fc", "zkh_rescale", "zkh_glu", "zkh_rope", "zkh_batchopen")}


def run(name, *args):
    if not os.path.exists(BIN[name]):
        pytest.skip("drivers not built")
    return subprocess.run([BIN[name]] + list(args), capture_output=True, text=True, timeout=60)


@pytest.mark.parametrize("name,nargs", [("zkh_fc", 3), ("zkh_rescale", 2), ("zkh_glu", 2), ("zkh_rope", 2)])
def test_claims_needs_its_arguments(name, nargs):
    r = run(name, "prove", "ob", "seed", "--claims", *["a"] * (nargs - 1))
    assert r.returncode == 1
    assert "--claims needs" in r.stderr


@pytest.mark.parametrize("name", ["zkh_fc", "zkh_rescale", "zkh_glu", "zkh_rope"])
def test_privacy_modes_and_unknown_flags_answer_2(name):
    for flag in ("--wpriv", "--apriv", "--hiding", "--frobnicate"):
        r = run(name, "prove", "ob", "seed", flag, "x")
        assert r.returncode == 2, (flag, r.stderr)
        assert flag in r.stderr


@pytest.mark.parametrize("name", sorted(BIN))
def test_bad_mode_prints_usage(name):
    r = run(name, "selftest")
    assert r.returncode == 2
    assert "usage" in r.stderr
