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


@pytest.mark.parametrize("spec,why", [("3=gen.bin", "power of two"), ("1=gen.bin", "power of two"),
                                      ("4x=gen.bin", "power of two"), ("=gen.bin", "power of two"),
                                      ("4", "power of two"), ("4=", "power of two"),
                                      ("99999999999=g", "power of two")])
def test_batchopen_rejects_bad_generator_spec(spec, why):
    """A generator spec is <G>=<file> with the whole of G a decimal power of two >= 2; anything
    else is refused by name before any file is read."""
    r = run("zkh_batchopen", "prove", "acc", "seed", "q.bin", "2=a.bin", spec)
    assert r.returncode == 1
    assert "generator spec '%s'" % spec in r.stderr and why in r.stderr


def test_batchopen_rejects_duplicate_domain():
    r = run("zkh_batchopen", "prove", "acc", "seed", "q.bin", "4=a.bin", "8=b.bin", "4=c.bin")
    assert r.returncode == 1
    assert "generator spec '4=c.bin': domain 4 given twice" in r.stderr


def test_serve_reads_long_request_lines_whole():
    """A request line longer than any fixed buffer is one request (zkob_serve.cuh reads lines
    with std::getline): one ZKW-RC answer, here usage (2) for an unknown mode."""
    if not os.path.exists(BIN["zkh_batchopen"]):
        pytest.skip("drivers not built")
    line = "selftest " + "x" * 200000
    r = subprocess.run([BIN["zkh_batchopen"], "serve"], input=line + "\n\n", capture_output=True, text=True,
                       timeout=60)
    assert r.returncode == 0
    assert r.stdout.splitlines() == ["ZKW-READY", "ZKW-RC 2"]
