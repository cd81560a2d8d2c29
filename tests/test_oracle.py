"""Pins the C oracle (oracle/zkh_oracle.c) before it is trusted as the GPU checker.

Every oracle function is checked against something a plausible mistake would break:
textbook modular arithmetic (Python integers), the published BLS12-381 parameter, FIPS
180-4 SHA-256 answers and hashlib, MLEs by their defining sums, brute-force counting, the
witness-free verifier algebra of the reference (zkob_fc.cu:489-712,
zkob_rescale.cu:256-316, zkob_rope.cu:29), forgeries that must be rejected, and an
independently written restatement (oracle/pyref.py).
"""
import hashlib
import random
import struct

import numpy as np
import pytest

from oracle import coracle as C
from oracle import pyref as P

R = P.R


def L(x):
    return P.to_limbs(x % R)


def I(a):
    return P.from_limbs(a)


def rnd(rng, n):
    return [rng.randrange(R) for _ in range(n)]


EDGE = [0, 1, 2, R - 1, R - 2, (R - 1) // 2, (R + 1) // 2, 1944954706 << 224, (1 << 255) % R,
        (1 << 224) - 1, 0xFFFFFFFF, 1 << 32]


# ------------------------------------------------------------------ field
def test_modulus_is_bls12_381_r():
    z = -0xD201000000010000  # BLS12-381 curve parameter
    assert R == z**4 - z**2 + 1
    assert R.bit_length() == 255
    assert P.to_limbs(R)[7] == 1944954707  # the challenge reduction constant (vrf_common.cuh:242)


def test_field_ops_vs_integers():
    rng = random.Random(1)
    vals = EDGE + rnd(rng, 300)
    rinv = pow(1 << 256, -1, R)
    for a, b in zip(vals, reversed(vals)):
        A, B = L(a), L(b)
        assert I(C.fr_op("add", A, B)) == (a + b) % R
        assert I(C.fr_op("sub", A, B)) == (a - b) % R
        assert I(C.fr_op("montmul", A, B)) == a * b * rinv % R
        assert I(C.fr_op("mul", A, B)) == a * b % R
    for a in vals:
        got = I(C.fr_op("inv", L(a)))
        assert got == (0 if a == 0 else pow(a, -1, R))
        if a:
            assert got * a % R == 1
    assert I(C.fr_op("mul", L(2), L(P.INV2))) == 1  # vrf_selfcheck (vrf_common.cuh:374-377)


def test_from_i64():
    for v in [0, 1, -1, 2**31 - 1, -2**31, 2**62, -2**62, 2**63 - 1, -2**63]:
        out = np.zeros(8, np.uint32)
        C.lib().or_fr_from_i64(C.ctypes.c_int64(v), C._p(out))
        assert I(out) == v % R


# ------------------------------------------------------------------ SHA-256 / transcript
FIPS = [(b"abc", "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"),
        (b"", "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"),
        (b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq",
         "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1"),
        (b"a" * 1000000, "cdc76e5c9914fb9281a1c7e284d73e67f1809a48a497200e046d39ccc7112cd0")]


@pytest.mark.parametrize("msg,hexd", FIPS)
def test_sha256_fips(msg, hexd):
    assert C.sha256(msg).hex() == hexd


def test_sha256_lengths_vs_hashlib():
    rng = random.Random(2)
    for n in list(range(0, 140)) + [1000, 4095, 4096, 4097]:
        m = bytes(rng.randrange(256) for _ in range(n))
        assert C.sha256(m) == hashlib.sha256(m).digest()


def test_transcript_framing():
    st = C.tr_init("seed:x")
    ref = hashlib.sha256(b"seed:x").digest()
    assert bytes(st) == ref
    data = bytes(range(40))
    C.tr_absorb(st, "label", data)
    ref = hashlib.sha256(ref + struct.pack("<I", 5) + b"label" + struct.pack("<Q", 40) + data).digest()
    assert bytes(st) == ref
    x = C.tr_challenge_fr(st)
    out = hashlib.sha256(ref + b"chal").digest()
    limbs = list(struct.unpack("<8I", out))
    limbs[7] %= 1944954707
    assert list(x) == limbs
    assert bytes(st) == hashlib.sha256(ref + b"rtch").digest()
    assert I(x) < R


# ------------------------------------------------------------------ MLE primitives
def test_me_vs_definition():
    rng = random.Random(3)
    for n, k in [(1, 0), (2, 1), (3, 2), (4, 2), (5, 3), (7, 3), (8, 3), (9, 4), (33, 6)]:
        t = rnd(rng, n)
        u = rnd(rng, k)
        rc, out = C.me(C.ints_to_fr(t), C.ints_to_fr(u) if k else np.zeros((0, 8), np.uint32))
        assert rc == 0
        assert I(out) == P.mle(t, u), (n, k)
    rc, _ = C.me(C.ints_to_fr([1, 2, 3]), C.ints_to_fr([5, 6, 7]))  # 3 <= 2^3/2
    assert rc == 1


def test_partial_me_vs_definition():
    rng = random.Random(4)
    for O, Cd, W in [(1, 5, 1), (3, 4, 2), (2, 7, 3), (1, 1, 4), (4, 3, 1)]:
        t = rnd(rng, O * Cd * W)
        k = P.ceil_log2(Cd)
        u = rnd(rng, k)
        rc, out = C.partial_me(C.ints_to_fr(t), C.ints_to_fr(u) if k else np.zeros((0, 8), np.uint32), Cd, W)
        assert rc == 0
        want = [sum(P.eq_weight(c, u) * t[(o * Cd + c) * W + w] for c in range(Cd)) % R
                for o in range(O) for w in range(W)]
        assert C.fr_to_ints(out) == want, (O, Cd, W)


def test_partial_me_window_vs_definition():
    rng = random.Random(5)
    for n, W, k in [(12, 3, 2), (10, 2, 3), (16, 4, 2), (7, 1, 3)]:
        t = rnd(rng, n)
        u = rnd(rng, k)
        out = C.frs(n)
        on = C.ctypes.c_uint32(0)
        tt = np.ascontiguousarray(C.ints_to_fr(t))
        uu = np.ascontiguousarray(C.ints_to_fr(u))
        rc = C.lib().or_partial_me_window(C._p(tt), n, C._p(uu), k, W, C._p(out), C.ctypes.byref(on))
        assert rc == 0
        rows = (n + W - 1) // W
        want = [sum(P.eq_weight(r, u) * (t[r * W + j] if r * W + j < n else 0)
                    for r in range(rows)) % R for j in range(W)]
        got = C.fr_to_ints(out[:on.value])
        assert got[:W] == want and all(v == 0 for v in got[W:]), (n, W, k)


def test_multi_dim_me_vs_definition():
    rng = random.Random(6)
    for rows, cols in [(4, 8), (3, 5), (1, 6), (7, 1), (5, 9)]:
        t = rnd(rng, rows * cols)
        ur, uc = rnd(rng, P.ceil_log2(rows)), rnd(rng, P.ceil_log2(cols))
        rc, out = C.multi_dim_me(C.ints_to_fr(t), [C.ints_to_fr(ur) if ur else np.zeros((0, 8), np.uint32),
                                                   C.ints_to_fr(uc) if uc else np.zeros((0, 8), np.uint32)],
                                 [rows, cols])
        assert rc == 0
        assert I(out) == P.mle2(t, rows, cols, ur, uc), (rows, cols)


def test_pad_and_eq_table():
    rng = random.Random(7)
    shape = [3, 5, 6]
    t = rnd(rng, 90)
    out = C.frs(256)
    on = C.ctypes.c_uint32(0)
    tt = np.ascontiguousarray(C.ints_to_fr(t))
    C.lib().or_pad(C._p(tt), C._p(np.array(shape, np.uint32)), 3, C._p(out), C.ctypes.byref(on))
    got = C.fr_to_ints(out[:on.value])
    for i in range(4):
        for j in range(8):
            for k in range(8):
                v = t[(i * 5 + j) * 6 + k] if (i < 3 and j < 5 and k < 6) else 0
                assert got[(i * 8 + j) * 8 + k] == v
    u = rnd(rng, 5)
    assert C.fr_to_ints(C.build_eq(C.ints_to_fr(u))) == P.eq_table(u)
    assert sum(P.eq_table(u)) % R == 1


def test_lagrange():
    rng = random.Random(8)
    for deg, fn, npts in [(2, "or_lagrange3", 3), (3, "or_lagrange4", 4)]:
        coef = rnd(rng, deg + 1)
        pts = [sum(c * pow(t, i, R) for i, c in enumerate(coef)) % R for t in range(npts)]
        x = rng.randrange(R)
        out = np.zeros(8, np.uint32)
        getattr(C.lib(), fn)(C._p(np.ascontiguousarray(C.ints_to_fr(pts))), C._p(np.array(L(x), np.uint32)), C._p(out))
        assert I(out) == sum(c * pow(x, i, R) for i, c in enumerate(coef)) % R


# ------------------------------------------------------------------ matmul sumcheck
@pytest.mark.parametrize("shape", [(4, 8, 4), (4, 6, 3), (2, 8, 3), (8, 16, 16), (16, 12, 5), (1, 4, 2),
                                   (3, 5, 7), (5, 1, 3)])
def test_mm_oracle_pins(shape):
    B, IN, OUT = shape
    rng = np.random.default_rng(sum(shape))
    X = rng.integers(-300, 300, size=(B, IN))
    W = rng.integers(-300, 300, size=(IN, OUT))
    Y = X @ W
    st = C.tr_init("pin")
    rc, d = C.mm_prove(st, X, W, Y, B, IN, OUT)
    assert rc == 0
    ev = C.fr_to_ints(d["ev"])
    claim, cx, cw = C.fr_to_ints(d["claims"])
    ub, uo, ui = (C.fr_to_ints(d[k]) for k in ("u_batch", "u_output", "u_input"))
    Xl, Wl, Yl = [int(v) for v in X.ravel()], [int(v) for v in W.ravel()], [int(v) for v in Y.ravel()]
    # claims by their definitions
    assert claim == P.mle2([v % R for v in Yl], B, OUT, ub, uo)
    assert cx == P.mle2([v % R for v in Xl], B, IN, ub, ui)
    assert cw == P.mle2([v % R for v in Wl], IN, OUT, ui, uo)
    # the verifier's algebra accepts and replays the same transcript
    tv = P.Transcript("pin")
    ok, ub2, uo2, ui2 = P.mm_verify(tv, B, IN, OUT, ev, claim, cx, cw)
    assert ok and bytes(st) == tv.state and ui2 == ui
    # independent restatement agrees
    tp = P.Transcript("pin")
    pr = P.mm_prove(tp, Xl, Wl, Yl, B, IN, OUT)
    assert pr["ev"] == ev and tp.state == bytes(st)
    # forgeries: a tampered round message or claim is rejected
    if ev:
        bad = list(ev)
        bad[0] = (bad[0] + 1) % R
        assert not P.mm_verify(P.Transcript("pin"), B, IN, OUT, bad, claim, cx, cw)[0]
    assert not P.mm_verify(P.Transcript("pin"), B, IN, OUT, ev, claim, (cx + 1) % R, cw)[0]


def test_mm_oracle_rejects_wrong_witness():
    X = np.arange(8 * 16).reshape(8, 16) % 7 - 3
    W = np.arange(16 * 4).reshape(16, 4) % 5 - 2
    Y = X @ W
    Y[1, 1] += 1
    rc, _ = C.mm_prove(C.tr_init("bad"), X, W, Y, 8, 16, 4)
    assert rc == 2


# ------------------------------------------------------------------ logUp
LU = [(32, 8, -3, 5), (16, 16, 0, 16), (64, 4, -2, 3), (32, 4, -2, 4), (8, 4, -2, 4), (64, 16, -8, 16)]


@pytest.mark.parametrize("low,ln,N", [(2**31 - 4, 8, 8), (2**31 - 2, 3, 4), (-2**31, 4, 8)])
def test_range_table_int32_arithmetic(low, ln, N):
    """tlookuprange_init_kernel adds in C++ int (tlookup.cu:376): past 2^31 - 1 the entries
    wrap, as numpy's int32 addition does."""
    want = (np.int32(low) + np.minimum(np.arange(N), ln - 1).astype(np.int32)).astype(np.int64)
    assert C.fr_to_ints(C.range_table(low, ln, N)) == [int(v) % R for v in want]


@pytest.mark.parametrize("shape", LU)
def test_lu_oracle_pins(shape):
    D, N, low, ln = shape
    rng = np.random.default_rng(D * 7 + N)
    vals = [int(v) for v in rng.integers(low, low + ln, size=D)]
    S = C.ints_to_fr(vals)
    T = C.range_table(low, ln, N)
    assert C.fr_to_ints(T) == [(low + i if i < ln else low + ln - 1) % R for i in range(N)]
    rc, m = C.lu_prep(S, low, N)
    assert rc == 0
    assert C.fr_to_ints(m) == [sum(1 for v in vals if v - low == j) for j in range(N)]
    st = C.tr_init("lu")
    beta = C.tr_challenge_fr(st)
    A = C.lu_inverse(S, beta)
    b = I(beta)
    assert all(a * ((v + b) % R) % R == 1 for a, v in zip(C.fr_to_ints(A), vals))
    alpha = C.tr_challenge_fr(st)
    logD = P.ceil_log2(D)
    u = np.array([C.tr_challenge_fr(st) for _ in range(logD)])
    st_pre = bytes(st)
    rc, d = C.lu_prove(st, A, S, T, m, alpha, beta, u)
    assert rc == 0
    ev = C.fr_to_ints(d["ev"])
    A_f, S_f, B_f, T_f, m_f = C.fr_to_ints(d["term"])
    ui = C.fr_to_ints(u)
    ok, ws = P.lu_verify(P.Transcript(state=st_pre), D, N, C.fr_to_ints(T), ev, A_f, S_f, m_f, I(alpha), b, ui)
    assert ok
    assert ws == C.fr_to_ints(d["ws"])
    tp = P.Transcript(state=st_pre)
    ev2, term2, _ = P.lu_prove(tp, C.fr_to_ints(A), [v % R for v in vals], C.fr_to_ints(T),
                               C.fr_to_ints(m), I(alpha), b, ui)
    assert ev2 == ev and tp.state == bytes(st)
    # terminals are the MLEs of the tables at the reversed round challenges (zkob_rescale.cu:151-165)
    pt = ws[::-1]
    assert A_f == P.mle(C.fr_to_ints(A), pt) and S_f == P.mle([v % R for v in vals], pt)
    assert m_f == P.mle(C.fr_to_ints(m), pt[:P.ceil_log2(N)])
    # forgery: tampered terminal is rejected
    assert not P.lu_verify(P.Transcript(state=st_pre), D, N, C.fr_to_ints(T), ev, (A_f + 1) % R, S_f,
                           m_f, I(alpha), b, ui)[0]


def test_lu_out_of_range_witness():
    """zkob_rescale's evil_idx forgery: a witness outside the table.  The honest-procedure
    proof (non-strict) is rejected by the verifier; the strict prover reports it."""
    D, N, low = 16, 8, 0
    vals = [i % 8 for i in range(D)]
    S = C.ints_to_fr(vals)
    rc, m = C.lu_prep(S, low, N)
    assert rc == 0
    vals[3] = 9  # out of range: limb0 index 9 >= N
    rc2, _ = C.lu_prep(C.ints_to_fr(vals), low, N)
    assert rc2 == 1
    S = C.ints_to_fr(vals)
    T = C.range_table(low, 8, N)
    st = C.tr_init("evil")
    beta, alpha = C.tr_challenge_fr(st), C.tr_challenge_fr(st)
    u = np.array([C.tr_challenge_fr(st) for _ in range(4)])
    A = C.lu_inverse(S, beta)
    pre = bytes(st)
    rc, _ = C.lu_prove(st.copy(), A, S, T, m, alpha, beta, u, strict=True)
    assert rc == 2
    rc, d = C.lu_prove(st, A, S, T, m, alpha, beta, u, strict=False)
    A_f, S_f, _, _, m_f = C.fr_to_ints(d["term"])
    assert not P.lu_verify(P.Transcript(state=pre), D, N, C.fr_to_ints(T), C.fr_to_ints(d["ev"]),
                           A_f, S_f, m_f, I(alpha), I(beta), C.fr_to_ints(u))[0]


def test_lu_inverse_of_zero():
    S = C.ints_to_fr([5, 7, R - 9, 11])
    A = C.lu_inverse(S, np.array(L(9), np.uint32))
    assert C.fr_to_ints(A) == [pow(14, -1, R), pow(16, -1, R), 0, pow(20, -1, R)]


# ------------------------------------------------------------------ Hadamard
@pytest.mark.parametrize("k", [1, 2, 3, 5])
def test_hp_oracle_pins(k):
    rng = random.Random(k)
    n = 1 << k
    u = rnd(rng, k)
    E, S, U = P.eq_table(u), rnd(rng, n), rnd(rng, n)
    claim = sum(e * s * x for e, s, x in zip(E, S, U)) % R
    assert claim == P.mle([s * x % R for s, x in zip(S, U)], u)
    st = C.tr_init("hp")
    rc, d = C.hp_prove(st, L(claim), C.ints_to_fr(E), C.ints_to_fr(S), C.ints_to_fr(U))
    assert rc == 0
    ev = C.fr_to_ints(d["ev"])
    S_f, U_f, E_f = C.fr_to_ints(d["term"])
    ws = C.fr_to_ints(d["ws"])
    # replay: p(0)+p(1) chain with Lagrange-4, terminal E_f*S_f*U_f (zkob_rope.cu:29)
    tv = P.Transcript("hp")
    cur = claim
    for r in range(k):
        e = ev[4 * r:4 * r + 4]
        assert (e[0] + e[1]) % R == cur
        for lab, v in zip(("hp0", "hp1", "hp2", "hp3"), e):
            tv.absorb_fr(lab, v)
        w = tv.challenge_fr()
        assert w == ws[r]
        cur = P.lagrange(e, w)
    assert cur == E_f * S_f * U_f % R and tv.state == bytes(st)
    pt = ws[::-1]
    assert S_f == P.mle(S, pt) and U_f == P.mle(U, pt)
    assert E_f == np.prod([P.eq2(a, b) for a, b in zip(u, pt)], dtype=object) % R
    tp = P.Transcript("hp")
    ev2, _, _ = P.hp_prove(tp, claim, E, S, U)
    assert ev2 == ev
    rc, _ = C.hp_prove(C.tr_init("hp"), L(claim + 1), C.ints_to_fr(E), C.ints_to_fr(S), C.ints_to_fr(U))
    assert rc == 2
