"""Pins the oracle's G1 routines (oracle/zkh_g1_oracle.c) -- Fp Montgomery arithmetic,
doubling, addition, scalar multiplication and the Pippenger commitment -- against:

- the reference's own constants (tests/golden/g1/constants.json: the generator and one in
  Montgomery form, -p^-1 mod 2^32), which fix p, R and the Montgomery layout;
- Python big-integer arithmetic (a*b*2^-384 mod p) for Fp;
- textbook affine group arithmetic (oracle/pyg1.py) for every group element produced;
- closed forms that fix the Jacobian representative, which is what the transcript absorbs:
  dbl-2009-l gives Z3 = 2 Y1 Z1; add-2007-bl gives Z3 = 2 Z1 Z2 H with H = X2 Z1^2 - X1 Z2^2,
  and for P + (-P) the point (r^2, -r^3, 0) with r = 2 (S2 - S1); with Z fixed, projective
  equality fixes X and Y;
- the commitment schedule on inputs whose result follows from it by hand: a zero row is
  exactly {0, ONE, 0}; a single digit d in window w of one generator gives
  dbl^(4w)(G, 2G, ...) (the running sum adds the bucket d times); two generators sharing a
  digit enter their bucket in index order.
"""
import json
import os
import random

import numpy as np
import pytest

from oracle import coracle as C
from oracle import pyg1 as G
from oracle import pyref

P = G.P
GOLD = os.path.join(os.path.dirname(__file__), "golden", "g1", "constants.json")


def rand_point(rng, k=None, z=None):
    """a random subgroup point as a Jacobian point with a random Z."""
    k = rng.randrange(1, G.ORDER) if k is None else k
    z = rng.randrange(1, P) if z is None else z
    a = G.aff_mul((G.GX, G.GY), k)
    return a, G.aff_to_jac(a, z)


def test_constants_match_reference():
    g = json.load(open(GOLD))
    assert list(G.limbs12(G.to_mont(G.GX))) == g["g1_generator_x_mont"]
    assert list(G.limbs12(G.to_mont(G.GY))) == g["g1_generator_y_mont"]
    assert list(G.limbs12(G.to_mont(1))) == g["g1_one"]
    assert (-pow(P, -1, 1 << 32)) % (1 << 32) == g["fp_inv"]
    assert (G.GY ** 2 - G.GX ** 3 - 4) % P == 0
    assert G.aff_mul((G.GX, G.GY), G.ORDER) is None
    assert G.ORDER == pyref.R


def test_fp_ops_against_big_ints():
    rng = random.Random(1)
    edge = [0, 1, 2, P - 1, P - 2, (P - 1) // 2, 1 << 380, (1 << 381) - 1 - ((1 << 381) - P)]
    vals = edge + [rng.randrange(P) for _ in range(60)]
    for a in vals[:40]:
        for b in vals[20:60:3]:
            la, lb = G.limbs12(a), G.limbs12(b)
            assert G.from_limbs12(C.fp_op("mul", la, lb)) == a * b * G.MONT_INV % P
            assert G.from_limbs12(C.fp_op("add", la, lb)) == (a + b) % P
            assert G.from_limbs12(C.fp_op("sub", la, lb)) == (a - b) % P


def test_dbl_group_and_representative():
    rng = random.Random(2)
    for _ in range(12):
        a, pt = rand_point(rng)
        out = C.g1_dbl(pt)
        assert G.on_curve_jac(out)
        assert G.to_affine(out) == G.aff_add(a, a)
        X, Y, Z = G.jac_ints(pt)
        assert G.jac_ints(out)[2] == 2 * Y * Z % P
    inf = G.jac_point(5, 7, 0)
    assert np.array_equal(C.g1_dbl(inf), inf)


def test_add_group_and_representative():
    rng = random.Random(3)
    for _ in range(12):
        a, pa = rand_point(rng)
        b, pb = rand_point(rng)
        out = C.g1_add(pa, pb)
        assert G.on_curve_jac(out)
        assert G.to_affine(out) == G.aff_add(a, b)
        X1, Y1, Z1 = G.jac_ints(pa)
        X2, Y2, Z2 = G.jac_ints(pb)
        H = (X2 * Z1 * Z1 - X1 * Z2 * Z2) % P
        assert G.jac_ints(out)[2] == 2 * Z1 * Z2 * H % P


def test_add_special_cases():
    rng = random.Random(4)
    a, pa = rand_point(rng)
    _, pa2 = rand_point(rng, k=None, z=None)
    zero = G.g1_zero()
    odd_inf = G.jac_point(3, 9, 0)
    # an operand at infinity returns the other one unchanged
    assert np.array_equal(C.g1_add(zero, pa), pa)
    assert np.array_equal(C.g1_add(pa, odd_inf), pa)
    assert np.array_equal(C.g1_add(odd_inf, zero), zero)
    # the same point under another Z doubles the first operand
    k = rng.randrange(1, G.ORDER)
    a, p1 = rand_point(rng, k=k)
    _, p2 = rand_point(rng, k=k)
    assert np.array_equal(C.g1_add(p1, p2), C.g1_dbl(p1))
    # P + (-P): general formula with H = 0 -> (r^2, -r^3, 0), r = 2 (S2 - S1)
    X1, Y1, Z1 = G.jac_ints(p1)
    z = rng.randrange(1, P)
    neg = G.aff_to_jac((a[0], (-a[1]) % P), z)
    X2, Y2, Z2 = G.jac_ints(neg)
    S1 = Y1 * Z2 * Z2 * Z2 % P
    S2 = Y2 * Z1 * Z1 * Z1 % P
    r = 2 * (S2 - S1) % P
    assert G.jac_ints(C.g1_add(p1, neg)) == (r * r % P, (-r * r * r) % P, 0)


def test_scalar_mul_raw_bits():
    rng = random.Random(5)
    base = G.aff_to_jac((G.GX, G.GY))
    for k in [1, 2, 3, 5, 16, 255, rng.randrange(G.ORDER), G.ORDER - 1]:
        out = C.g1_mul(base, np.array(pyref.to_limbs(k), np.uint32))
        assert G.to_affine(out) == G.aff_mul((G.GX, G.GY), k)
    out = C.g1_mul(base, np.array(pyref.to_limbs(G.ORDER), np.uint32))
    assert G.jac_ints(out)[2] == 0


def _gens(rng, n):
    pts = [rand_point(rng) for _ in range(n)]
    return [a for a, _ in pts], np.stack([p for _, p in pts])


def test_commit_group_element():
    rng = random.Random(6)
    n, m = 5, 3
    aff, gens = _gens(rng, n)
    ints = [rng.choice([rng.randrange(-(1 << 17), 1 << 17), rng.randrange(pyref.R)])
            for _ in range(m * n)]
    sc = C.ints_to_fr(ints)
    rc, out = C.g1_commit(gens, sc, n)
    assert rc == 0
    for row in range(m):
        want = None
        for i in range(n):
            want = G.aff_add(want, G.aff_mul(aff[i], ints[row * n + i] % pyref.R))
        assert G.to_affine(out[row]) == want
        assert G.on_curve_jac(out[row])


def test_commit_zero_row_is_canonical_infinity():
    rng = random.Random(7)
    _, gens = _gens(rng, 4)
    rc, out = C.g1_commit(gens, np.zeros((8, 8), np.uint32), 4)
    assert rc == 0
    assert np.array_equal(out[0], G.g1_zero()) and np.array_equal(out[1], G.g1_zero())


def _chain(b, d):
    run = b
    for _ in range(d - 1):
        run = C.g1_add(run, b)
    return run


@pytest.mark.parametrize("w,d", [(0, 1), (0, 15), (1, 2), (7, 9), (8, 3), (33, 12), (63, 7)])
def test_commit_single_digit(w, d):
    rng = random.Random(100 + w)
    _, gens = _gens(rng, 3)
    s = d << (4 * w)
    sc = np.zeros((3, 8), np.uint32)
    sc[1] = pyref.to_limbs(s)
    rc, out = C.g1_commit(gens, sc, 3)
    want = _chain(gens[1], d)
    for _ in range(4 * w):
        want = C.g1_dbl(want)
    assert np.array_equal(out[0], want)


def test_commit_bucket_order():
    rng = random.Random(8)
    _, gens = _gens(rng, 2)
    w, d = 5, 6
    sc = np.zeros((2, 8), np.uint32)
    sc[0] = sc[1] = pyref.to_limbs(d << (4 * w))
    rc, out = C.g1_commit(gens, sc, 2)
    bucket = C.g1_add(gens[0], gens[1])
    assert not np.array_equal(bucket, C.g1_add(gens[1], gens[0]))
    want = _chain(bucket, d)
    for _ in range(4 * w):
        want = C.g1_dbl(want)
    assert np.array_equal(out[0], want)


# ---- inner-product argument (ipa_prove, vrf_common.cuh:302-336) ----
def ipa_verify(state, g_aff, Q_aff, a, b, L, R, a_final):
    """Witness-free IPA check written from the argument's algebra (the reference's
    ipa_verify, vrf_common.cuh:338-371): P0 = <a, g> + <a, b> Q; per round P <- x^2 L + P +
    x^-2 R and b folds to x^-1 b_lo + x b_hi; the final generator is sum_i s_i g_i with
    s_i = prod_r (bit (rounds-1-r) of i ? x_r : x_r^-1); accept iff P = a_f g_f + a_f b_f Q.
    Affine big-integer arithmetic; returns (accepted, final transcript state)."""
    RR = pyref.R
    n = len(g_aff)
    P = None
    for i in range(n):
        P = G.aff_add(P, G.aff_mul(g_aff[i], a[i]))
    P = G.aff_add(P, G.aff_mul(Q_aff, sum(x * y for x, y in zip(a, b)) % RR))
    tr = pyref.Transcript(state=bytes(state))
    xs = []
    bb = list(b)
    for r in range(len(L)):
        tr.absorb("L", bytes(np.asarray(L[r], np.uint32).tobytes()))
        tr.absorb("R", bytes(np.asarray(R[r], np.uint32).tobytes()))
        x = tr.challenge_fr()
        xi = pow(x, RR - 2, RR)
        xs.append((x, xi))
        P = G.aff_add(G.aff_add(G.aff_mul(G.to_affine(L[r]), x * x % RR), P),
                      G.aff_mul(G.to_affine(R[r]), xi * xi % RR))
        h = len(bb) // 2
        bb = [(xi * bb[k] + x * bb[k + h]) % RR for k in range(h)]
    rounds = len(L)
    gf = None
    for i in range(n):
        s = 1
        for r in range(rounds):
            s = s * (xs[r][0] if (i >> (rounds - 1 - r)) & 1 else xs[r][1]) % RR
        gf = G.aff_add(gf, G.aff_mul(g_aff[i], s))
    want = G.aff_add(G.aff_mul(gf, a_final), G.aff_mul(Q_aff, a_final * bb[0] % RR))
    return P == want, tr.state


@pytest.mark.parametrize("n", [1, 2, 8])
def test_ipa_oracle_accepted_by_verifier(n):
    rng = random.Random(200 + n)
    pts = [rand_point(rng) for _ in range(n + 1)]
    g_aff = [p[0] for p in pts[:n]]
    g = np.stack([p[1] for p in pts[:n]])
    Q_aff, Q = pts[n]
    a = [rng.randrange(pyref.R) for _ in range(n)]
    u = [rng.randrange(pyref.R) for _ in range(max(n.bit_length() - 1, 0))]
    b = [pyref.eq_weight(k, u) if u else 1 for k in range(n)]
    st = C.tr_init("ipa-test")
    st0 = st.copy()
    rc, L, R, af = C.ipa_prove(st, C.ints_to_fr(a), C.ints_to_fr(b), g, Q, n)
    assert rc == 0 and len(L) == n.bit_length() - 1
    ok, st_v = ipa_verify(st0, g_aff, Q_aff, a, b, L, R, pyref.from_limbs(af))
    assert ok
    assert bytes(st_v) == bytes(st)
    if n > 1:
        # a wrong final scalar and a swapped L/R pair must both fail
        bad, _ = ipa_verify(st0, g_aff, Q_aff, a, b, L, R, (pyref.from_limbs(af) + 1) % pyref.R)
        assert not bad
        bad, _ = ipa_verify(st0, g_aff, Q_aff, a, b, R, L, pyref.from_limbs(af))
        assert not bad


def test_ipa_round_points_by_definition():
    """L and R of the first round are, as group elements, <g_hi, a_lo> + <a_lo, b_hi> Q and
    <g_lo, a_hi> + <a_hi, b_lo> Q."""
    rng = random.Random(210)
    n = 4
    pts = [rand_point(rng) for _ in range(n + 1)]
    g = np.stack([p[1] for p in pts[:n]])
    Q_aff, Q = pts[n]
    a = [rng.randrange(pyref.R) for _ in range(n)]
    b = [rng.randrange(pyref.R) for _ in range(n)]
    rc, L, R, af = C.ipa_prove(C.tr_init("ipa-def"), C.ints_to_fr(a), C.ints_to_fr(b), g, Q, n)
    h = n // 2
    wantL = G.aff_mul(Q_aff, sum(a[i] * b[h + i] for i in range(h)) % pyref.R)
    wantR = G.aff_mul(Q_aff, sum(a[h + i] * b[i] for i in range(h)) % pyref.R)
    for i in range(h):
        wantL = G.aff_add(wantL, G.aff_mul(pts[h + i][0], a[i]))
        wantR = G.aff_add(wantR, G.aff_mul(pts[i][0], a[h + i]))
    assert G.to_affine(L[0]) == wantL and G.to_affine(R[0]) == wantR
