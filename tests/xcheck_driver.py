"""Runs matmul, logUp and Hadamard proofs through libzkh.so in a process started with
ZKH_XCHECK=1, so that every proof also re-evaluates its folded terminals as MLEs of its
input tables at the opening point (the reference's "terminal != multi_dim_me" guards,
zkob_fc.cu:337-345, zkob_rescale.cu:151-165, zkob_glu.cu:186-192 and :254-260), and the
logUp and Hadamard round kernels compute every round's sums at 1, so that each round's
p(0) + p(1) = claim is checked on device sums (zkob_lookup.cuh:155, :183, :303).  A
mismatch fails the call with ZKH_EROUND; the script prints one line per case and exits
non-zero on the first failure.  Called by tests/test_gpu_xcheck.py; not a test module."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

from conftest import load_zkh  # noqa: E402
from oracle import coracle as C  # noqa: E402
from oracle import pyref as P  # noqa: E402


def main():
    assert os.environ.get("ZKH_XCHECK") == "1"
    zkh = load_zkh()
    ctx = zkh.Context(0)
    rng = np.random.default_rng(7)

    def say(*a):
        print(*a, flush=True)

    # matmuls: int and FR witnesses, power-of-two and ragged shapes, one persistent launch
    # group and the per-round path
    shapes = [(8, 16, 4), (5, 12, 3), (128, 768, 64), (64, 4096, 32)]
    for no_persist in (False, True):
        if no_persist:
            os.environ["ZKH_NO_PERSIST"] = "1"
        items = []
        for i, (B, IN, OUT) in enumerate(shapes):
            X = rng.integers(-2**15, 2**15, size=(B, IN)).astype(np.int32)
            W = rng.integers(-2**17, 2**17, size=(IN, OUT)).astype(np.int32)
            Y = (X.astype(np.int64) @ W.astype(np.int64))
            st = zkh.transcript("xc:mm:%d" % i)
            if i % 2:
                tX, tW, tY = (ctx.from_fr(C.ints_to_fr(a.ravel())) for a in (X, W, Y))
            else:
                tX, tW, tY = ctx.from_i32(X.ravel()), ctx.from_i32(W.ravel()), ctx.from_i64(Y.ravel())
            items.append((st, tX, tW, tY, B, IN, OUT))
        outs, status = ctx.mm_prove_batch(items)
        assert all(s == 0 for s in status), status
        say("mm ok", "per-round" if no_persist else "persistent", shapes)
        os.environ.pop("ZKH_NO_PERSIST", None)

    # logUp: D > N (several sizes) and D == N
    for D, N, low in [(1 << 12, 1 << 8, -128), (1 << 14, 1 << 14, -(1 << 13)), (32, 8, -3)]:
        vals = rng.integers(low, low + N, size=D).astype(np.int32)
        Sg = ctx.from_i32(vals)
        mg = ctx.lu_prep(Sg, low, N)
        Tg = ctx.range_table(low, N, N)
        st = zkh.transcript("xc:lu:%d:%d" % (D, N))
        beta = zkh.challenge(st)
        Ag = ctx.lu_inverse(Sg, beta)
        alpha = zkh.challenge(st)
        u = np.array([zkh.challenge(st) for _ in range(P.ceil_log2(D))])
        ctx.lu_prove(st, Ag, Sg, Tg, mg, alpha, beta, u)
        say("lu ok", D, N)

    # Hadamard: explicit E table and the eq(u, .) form
    for k in (3, 13):
        n = 1 << k
        u = np.array([zkh.challenge(zkh.transcript("xc:u:%d:%d" % (k, i))) for i in range(k)])
        E = C.build_eq(u)
        S = C.ints_to_fr(rng.integers(-2**20, 2**20, size=n))
        U = C.ints_to_fr(rng.integers(-2**20, 2**20, size=n))
        Ei, Si, Ui = C.fr_to_ints(E), C.fr_to_ints(S), C.fr_to_ints(U)
        claim = C.ints_to_fr([sum(a * b % P.R * c for a, b, c in zip(Ei, Si, Ui)) % P.R])[0]
        ctx.hp_prove(zkh.transcript("xc:hp:%d" % k), claim, ctx.from_fr(E), ctx.from_fr(S), ctx.from_fr(U))
        ctx.hp_prove_eq(zkh.transcript("xc:hp:%d" % k), claim, u, ctx.from_fr(S), ctx.from_fr(U))
        say("hp ok", k)

    # per-round checks: tables large enough for the round kernels (above the persistent
    # loops' 8192 entries), whose folding rounds then compute their sums at 1 instead of
    # deriving them; each call checks p(0) + p(1) = claim every round, and the proofs
    # must equal the oracle's (which checks the same identity per round)
    D = N = 1 << 16
    low = -(1 << 15)
    vals = rng.integers(low, low + N, size=D).astype(np.int32)
    Sf = C.ints_to_fr(vals)
    Sg = ctx.from_i32(vals)
    Tg = ctx.range_table(low, N, N)
    st, st_o = zkh.transcript("xc:lu:rounds"), C.tr_init("xc:lu:rounds")
    beta = zkh.challenge(st)
    assert np.array_equal(C.tr_challenge_fr(st_o), beta)
    Ag = ctx.lu_range_inverse(Sg, low, Tg, beta)
    alpha = zkh.challenge(st)
    C.tr_challenge_fr(st_o)
    u = np.array([zkh.challenge(st) for _ in range(16)])
    for _ in range(16):
        C.tr_challenge_fr(st_o)
    got = ctx.lu_prove(st, Ag, Sg, Tg, ctx.lu_prep(Sg, low, N), alpha, beta, u)
    rc, m = C.lu_prep(Sf, low, N)
    rc, want = C.lu_prove(st_o, C.lu_inverse(Sf, beta), Sf, C.range_table(low, N, N), m, alpha, beta, u)
    assert rc == 0
    for key in ("ev", "term", "ws"):
        assert np.array_equal(got[key], want[key]), key
    assert bytes(st) == bytes(st_o)
    say("lu per-round ok", D)
    k = 16
    n = 1 << k
    S_i = rng.integers(-2**15, 2**15, size=n).astype(np.int32)
    U_i = rng.integers(-2**15, 2**15, size=n).astype(np.int32)
    Sf, Uf = C.ints_to_fr(S_i), C.ints_to_fr(U_i)
    st, st_o = zkh.transcript("xc:hp:rounds"), C.tr_init("xc:hp:rounds")
    u = np.array([zkh.challenge(st) for _ in range(k)])
    for _ in range(k):
        C.tr_challenge_fr(st_o)
    got = ctx.hp_prove_eq_claim(st, "claim_H", u, ctx.from_i32(S_i), ctx.from_i32(U_i))
    rc, claim = C.me(C.hadamard(Sf, Uf), u)
    C.tr_absorb(st_o, "claim_H", claim.tobytes())
    rc, want = C.hp_prove(st_o, claim, C.build_eq(u), Sf, Uf)
    assert rc == 0 and np.array_equal(got["claim"], claim)
    for key in ("ev", "term", "ws"):
        assert np.array_equal(got[key], want[key]), key
    assert bytes(st) == bytes(st_o)
    E = C.build_eq(u)
    got = ctx.hp_prove(zkh.transcript("xc:hpE"), claim, ctx.from_fr(E), ctx.from_fr(Sf), ctx.from_fr(Uf))
    rc, want = C.hp_prove(C.tr_init("xc:hpE"), claim, E, Sf, Uf)
    for key in ("ev", "term", "ws"):
        assert np.array_equal(got[key], want[key]), key
    say("hp per-round ok", k)
    ctx.close()
    say("xcheck all ok")


if __name__ == "__main__":
    main()
