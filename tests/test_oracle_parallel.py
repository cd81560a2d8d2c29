"""Pins the oracle additions used by the config-scale checks and the all-cores CPU baseline.

- The OpenMP table loops: a proof computed on 1 thread equals the same proof on 4 threads
  at sizes where every parallel loop engages (field addition is exact, so the order of the
  per-thread partial sums cannot change a result; a data race or a lost partial would).
- The C int -> Fr conversion against Python integers, including the int64 extremes.
- Elementwise axpy / Hadamard against Python integers; the inverse-identity checker on a
  correct inverse, a planted error and the inverse(0) = 0 convention (tlookup.cu:50-62).
- The field-input matmul segment: on the field images of integer inputs it equals the
  integer-input oracle (which the other oracle tests pin); on full-width field tables its
  claims equal their defining MLE sums and the witness-free verifier accepts the proof.
"""
import random

import numpy as np
import pytest

from oracle import coracle as C
from oracle import pyref as P

R = P.R


@pytest.fixture
def threads():
    before = C.get_threads()
    yield C.set_threads
    C.set_threads(before)


def test_ints_to_fr_vs_integers():
    rng = np.random.default_rng(5)
    vals = np.concatenate([rng.integers(-2**63, 2**63 - 1, size=500, dtype=np.int64),
                           np.array([0, 1, -1, 2**63 - 1, -2**63, -2**31, 2**31 - 1], np.int64)])
    got = C.fr_to_ints(C.ints_to_fr(vals))
    assert got == [int(v) % R for v in vals]
    small = rng.integers(-2**20, 2**20, size=100).astype(np.int32)
    assert C.fr_to_ints(C.ints_to_fr(small)) == [int(v) % R for v in small]


def test_axpy_hadamard_vs_integers():
    rng = random.Random(3)
    n = 9000  # above the parallel threshold
    a = [rng.randrange(R) for _ in range(n)]
    b = [rng.randrange(R) for _ in range(n)]
    c = rng.randrange(R)
    A, B = C.ints_to_fr(a), C.ints_to_fr(b)
    assert C.fr_to_ints(C.axpy(A, P.to_limbs(c), B)) == [(x + c * y) % R for x, y in zip(a, b)]
    assert C.fr_to_ints(C.hadamard(A, B)) == [x * y % R for x, y in zip(a, b)]


def test_check_inverse():
    rng = random.Random(4)
    s = [rng.randrange(R) for _ in range(10000)]
    beta = rng.randrange(R)
    s[17] = (R - beta) % R  # S + beta = 0 -> inverse 0
    S = C.ints_to_fr(s)
    bl = np.array(P.to_limbs(beta), np.uint32)
    A = C.lu_inverse(S, bl)
    assert C.check_inverse(S, A, bl) == 0
    A2 = A.copy()
    A2[5] = C.ints_to_fr([(C.fr_to_ints(A[5:6])[0] + 1) % R])[0]
    assert C.check_inverse(S, A2, bl) == 1
    A3 = A.copy()
    A3[17] = C.ints_to_fr([1])[0]  # must be 0 where S + beta = 0
    assert C.check_inverse(S, A3, bl) == 1


def _mm_both(X, W, Y, B, IN, OUT, seed):
    st = C.tr_init(seed)
    rc, d = C.mm_prove(st, X, W, Y, B, IN, OUT)
    st2 = C.tr_init(seed)
    rc2, d2 = C.mm_prove_fr(st2, C.ints_to_fr(X.ravel()), C.ints_to_fr(W.ravel()), C.ints_to_fr(Y.ravel()),
                            B, IN, OUT)
    return (rc, d, st), (rc2, d2, st2)


@pytest.mark.parametrize("shape", [(4, 8, 4), (3, 5, 7), (16, 12, 5), (1, 1, 1)])
def test_mm_prove_fr_equals_int_oracle(shape):
    B, IN, OUT = shape
    rng = np.random.default_rng(sum(shape))
    X = rng.integers(-2**24, 2**24, size=(B, IN))
    W = rng.integers(-2**24, 2**24, size=(IN, OUT))
    Y = X @ W
    (rc, d, st), (rc2, d2, st2) = _mm_both(X, W, Y, B, IN, OUT, "fr:%d" % B)
    assert rc == 0 and rc2 == 0
    for k in ("ev", "claims", "u_batch", "u_output", "u_input"):
        assert np.array_equal(d[k], d2[k]), k
    assert bytes(st) == bytes(st2)


@pytest.mark.parametrize("shape", [(4, 8, 4), (3, 6, 5), (2, 16, 3)])
def test_mm_prove_fr_full_width(shape):
    B, IN, OUT = shape
    rng = random.Random(sum(shape) * 3)
    x = [rng.randrange(R) for _ in range(B * IN)]
    w = [rng.randrange(R) for _ in range(IN * OUT)]
    y = [sum(x[b * IN + i] * w[i * OUT + o] for i in range(IN)) % R for b in range(B) for o in range(OUT)]
    rc, Yc = C.matmul_fr(C.ints_to_fr(x), C.ints_to_fr(w), B, IN, OUT)
    assert rc == 0 and C.fr_to_ints(Yc) == y
    st = C.tr_init("frw")
    rc, d = C.mm_prove_fr(st, C.ints_to_fr(x), C.ints_to_fr(w), Yc, B, IN, OUT)
    assert rc == 0
    claim, cx, cw = C.fr_to_ints(d["claims"])
    ub, uo, ui = (C.fr_to_ints(d[k]) for k in ("u_batch", "u_output", "u_input"))
    assert claim == P.mle2(y, B, OUT, ub, uo)
    assert cx == P.mle2(x, B, IN, ub, ui)
    assert cw == P.mle2(w, IN, OUT, ui, uo)
    ok, _, _, ui2 = P.mm_verify(P.Transcript("frw"), B, IN, OUT, C.fr_to_ints(d["ev"]), claim, cx, cw)
    assert ok and ui2 == ui
    # a wrong product entry fails the prover's own round check
    bad = Yc.copy()
    bad[0] = C.ints_to_fr([(y[0] + 1) % R])[0]
    rc, _ = C.mm_prove_fr(C.tr_init("frw"), C.ints_to_fr(x), C.ints_to_fr(w), bad, B, IN, OUT)
    assert rc == 2


def test_thread_count_invariance(threads):
    rng = np.random.default_rng(8)
    # matmul: IN = 20000 puts the zkip rounds and partial_me passes above the threshold
    B, IN, OUT = 2, 20000, 3
    X = rng.integers(-2**15, 2**15, size=(B, IN))
    W = rng.integers(-2**17, 2**17, size=(IN, OUT))
    Y = X @ W
    # logUp: D = 2^15 against 2^12 (phase 1 and phase 2 loops above the threshold)
    D, N, low = 1 << 15, 1 << 12, -(1 << 11)
    vals = rng.integers(low, low + N, size=D)
    S = C.ints_to_fr(vals)
    T = C.range_table(low, N, N)
    _, m = C.lu_prep(S, low, N)
    # Hadamard 2^14
    k = 14
    u = C.ints_to_fr([int(v) for v in rng.integers(0, 2**62, size=k)])
    E = C.build_eq(u)
    Sh = C.ints_to_fr(rng.integers(-2**20, 2**20, size=1 << k))
    Uh = C.ints_to_fr(rng.integers(-2**20, 2**20, size=1 << k))
    H = C.hadamard(Sh, Uh)
    _, claim_h = C.me(H, u)

    def run():
        out = []
        st = C.tr_init("inv")
        rc, d = C.mm_prove(st, X, W, Y, B, IN, OUT)
        assert rc == 0
        out += [d[k].tobytes() for k in sorted(d)] + [bytes(st)]
        st = C.tr_init("inv-lu")
        beta, alpha = C.tr_challenge_fr(st), C.tr_challenge_fr(st)
        uu = np.array([C.tr_challenge_fr(st) for _ in range(15)])
        A = C.lu_inverse(S, beta)
        rc, d = C.lu_prove(st, A, S, T, m, alpha, beta, uu)
        assert rc == 0
        out += [A.tobytes()] + [d[k].tobytes() for k in sorted(d)] + [bytes(st)]
        st = C.tr_init("inv-hp")
        rc, d = C.hp_prove(st, claim_h, E, Sh, Uh)
        assert rc == 0
        out += [d[k].tobytes() for k in sorted(d)] + [bytes(st)]
        return out

    threads(1)
    one = run()
    threads(4)
    assert run() == one
