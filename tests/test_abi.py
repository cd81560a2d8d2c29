"""CPU checks of the C-ABI library: it loads, exports every entry point include/zkh.h
declares, its host-side transcript matches the reference framing, and without a GPU the
context constructor fails cleanly (no CPU fallback)."""
import ctypes
import hashlib
import os
import re
import struct

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    src = open(os.path.join(ROOT, "include", "zkh.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(zkh_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_the_boundary():
    syms = declared_symbols()
    for s in ["zkh_ctx_create", "zkh_mm_prove", "zkh_lu_prove", "zkh_hp_prove", "zkh_me",
              "zkh_partial_me", "zkh_multi_dim_me", "zkh_lu_inverse", "zkh_lu_prep"]:
        assert s in syms


def test_library_exports_every_declared_symbol(zkh):
    lib = zkh.lib()
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_transcript_matches_reference_framing(zkh):
    st = zkh.transcript("run:ob1")
    ref = hashlib.sha256(b"run:ob1").digest()
    assert bytes(st) == ref
    zkh.absorb(st, "B", struct.pack("<I", 512))
    ref = hashlib.sha256(ref + struct.pack("<I", 1) + b"B" + struct.pack("<Q", 4) + struct.pack("<I", 512)).digest()
    assert bytes(st) == ref
    x = zkh.challenge(st)
    limbs = list(struct.unpack("<8I", hashlib.sha256(ref + b"chal").digest()))
    limbs[7] %= 1944954707
    assert list(x) == limbs


def test_transcript_matches_oracle(zkh):
    from oracle import coracle as C
    a, b = zkh.transcript("s"), C.tr_init("s")
    for i in range(20):
        data = bytes(range(i * 3 % 64))
        zkh.absorb(a, "p%d" % i, data)
        C.tr_absorb(b, "p%d" % i, data)
        assert np.array_equal(zkh.challenge(a), C.tr_challenge_fr(b))
    assert bytes(a) == bytes(b)


def test_transcript_long_absorbs(zkh):
    """Many-block absorbs (the SHA-NI path where the CPU has it) against hashlib."""
    rng = np.random.default_rng(5)
    st = zkh.transcript("long")
    ref = hashlib.sha256(b"long").digest()
    for n in [0, 1, 55, 56, 63, 64, 65, 119, 120, 128, 1000, 4096 * 3 + 17]:
        data = rng.integers(0, 256, size=n, dtype=np.uint8).tobytes()
        zkh.absorb(st, "x" * (n % 7), data)
        ref = hashlib.sha256(ref + struct.pack("<I", n % 7) + b"x" * (n % 7) + struct.pack("<Q", n) + data).digest()
        assert bytes(st) == ref, n


def test_sha256_matches_hashlib(zkh):
    """zkh_sha256 (bo_file_sha256, zkob_claims.cuh:311-318) on a fresh state per call, host
    only: block-boundary lengths and two calls in a row agree with hashlib."""
    rng = np.random.default_rng(9)
    for n in [0, 1, 55, 56, 63, 64, 65, 144, 1000, 65537, 3]:
        data = rng.integers(0, 256, size=n, dtype=np.uint8).tobytes()
        out = (ctypes.c_uint8 * 32)()
        assert zkh.lib().zkh_sha256(data, ctypes.c_size_t(n), out) == 0
        assert bytes(out) == hashlib.sha256(data).digest(), n


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present")
def test_no_gpu_fails_loudly(zkh):
    h = ctypes.c_void_p()
    rc = zkh.lib().zkh_ctx_create(0, ctypes.byref(h))
    assert rc == zkh.EDEV and not h.value
    with pytest.raises(zkh.ZkhError):
        zkh.Context(0)


def test_ints_to_fr_helper_vs_oracle():
    """The package's numpy int -> Fr conversion (used to bind field-element tensors) against
    the oracle's long_to_scalar, including the int64 extremes."""
    import numpy as np
    from conftest import load_zkh
    from oracle import coracle as C
    zkh = load_zkh()
    rng = np.random.default_rng(12)
    v = np.concatenate([rng.integers(-2**63, 2**63 - 1, size=5000, dtype=np.int64),
                        np.array([0, 1, -1, -2**63, 2**63 - 1, -2**31, 2**32], np.int64)])
    assert np.array_equal(zkh.ints_to_fr(v), C.ints_to_fr(v))
    assert np.array_equal(zkh.ints_to_fr(v[:100].astype(np.int32)), C.ints_to_fr(v[:100].astype(np.int32)))


def test_challenge_vec_is_sequential_draws(zkh):
    """zkh_transcript_challenge_vec (fs_challenge_vec) equals n single draws in sequence."""
    from oracle import coracle as C
    st, so = zkh.transcript("vec"), C.tr_init("vec")
    zkh.absorb(st, "x", b"abc")
    C.tr_absorb(so, "x", b"abc")
    got = zkh.challenges(st, 23)
    want = [C.tr_challenge_fr(so) for _ in range(23)]
    assert got.shape == (23, 8) and all((g == w).all() for g, w in zip(got, want))
    assert bytes(st) == bytes(so)
    assert zkh.challenges(st, 0).shape == (0, 8)


def test_absorb_trace_matches_reference_format(tmp_path):
    """P3_ABLOG=path (the reference's absorb trace, fs_transcript.hpp:135-148): one line per
    absorb with the label, the data length and the first 8 bytes of the new state in hex."""
    import os
    import subprocess
    import sys
    from oracle import coracle as C
    log = tmp_path / "ab.log"
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    prog = (
        "import sys; sys.path.insert(0, %r); sys.path.insert(0, %r)\n"
        "from conftest import load_zkh\n"
        "zkh = load_zkh()\n"
        "st = zkh.transcript('trace')\n"
        "zkh.absorb(st, 'B', b'\\x04\\x00\\x00\\x00')\n"
        "zkh.absorb(st, 'com_X', bytes(range(144)) * 3)\n"
        "zkh.challenge(st)\n"
        "zkh.absorb(st, 'p0', bytes(32))\n" % (root, os.path.join(root, "tests")))
    env = dict(os.environ, P3_ABLOG=str(log))
    subprocess.run([sys.executable, "-c", prog], check=True, env=env, timeout=120)
    st = C.tr_init("trace")
    want = []
    for label, data, chal in (("B", b"\x04\x00\x00\x00", False), ("com_X", bytes(range(144)) * 3, True),
                              ("p0", bytes(32), False)):
        C.tr_absorb(st, label, data)
        want.append("%s %d %s" % (label, len(data), bytes(st[:8]).hex()))
        if chal:
            C.tr_challenge_fr(st)
    assert log.read_text().splitlines() == want


R_MOD = 0x73EDA753299D7D483339D80809A1D80553BDA402FFFE5BFEFFFFFFFF00000001


def _limbs(x):
    return (ctypes.c_uint32 * 8)(*[(x >> (32 * i)) & 0xFFFFFFFF for i in range(8)])


def _int(l):
    return sum(int(l[i]) << (32 * i) for i in range(8))


def test_host_scalar_ops_match_big_integers(zkh):
    """zkh_fr_scalar (the host field arithmetic of the round logic): add, sub, mul and the
    inverse (the optimized binary GCD: 31-step updates from 64-bit approximations) against
    Python integers mod r, with the inverse pinned by Fermat's little theorem (x^(r-2)) and
    x * x^-1 = 1, and inverse(0) = 0; powers of two and their negatives, whose GCD runs are
    the longest and most lopsided, are among the inputs."""
    lib = zkh.lib()
    f = lib.zkh_fr_scalar
    f.restype = ctypes.c_int
    rng = np.random.default_rng(5)
    vals = [0, 1, 2, 3, R_MOD - 1, R_MOD - 2, (R_MOD + 1) // 2, 1 << 200, (1 << 255) % R_MOD]
    vals += [int.from_bytes(rng.bytes(32), "little") % R_MOD for _ in range(300)]
    vals += [1 << k for k in range(0, 255, 5)] + [R_MOD - (1 << k) for k in range(0, 254, 9)]
    vals += [int.from_bytes(rng.bytes(8), "little") for _ in range(40)]
    out = (ctypes.c_uint32 * 8)()
    for i, a in enumerate(vals):
        b = vals[(7 * i + 3) % len(vals)]
        for op, want in ((0, (a + b) % R_MOD), (1, (a - b) % R_MOD), (2, a * b % R_MOD),
                         (3, pow(a, R_MOD - 2, R_MOD))):
            assert f(_limbs(a), _limbs(b), op, out) == 0
            assert _int(out) == want, (op, hex(a))
        if a:
            assert _int(out) * a % R_MOD == 1
    assert f(_limbs(R_MOD), _limbs(1), 0, out) != 0  # non-canonical input is refused
