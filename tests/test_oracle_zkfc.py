"""Pins the oracle's zkip / zkip_stacked / zkFCStacked::prove, window partial_me, pad with a
pad value and the rescaling witness (zkllm-src/zkfc.cu:94-307, fr-tensor.cu:612-641,
:800-828, :935-945, rescaling.cu:8-21) against their mathematical definitions:

- zkip: the claim is sum a_i b_i; the final claim is the product of the zero-padded MLEs
  at the round challenges (u[0] on the least significant index bit), or, with fewer rounds
  than variables, the inner product of the tables with their top bits bound by eq sums;
- zkip_stacked: claim = sum_n eq(uN, n) sum_d A[n,d] B[n,d]; final = A~(uD; vN) B~(uD; vN);
- zkFCStacked::prove: the claim is the 3-D MLE of Y less the broadcast bias term and the
  final claim the product of the 3-D MLEs of X and W (all by their defining sums);
- rescaling: x = sf*q + rem with rem in [-sf/2, sf - sf/2), which fixes (q, rem) uniquely;
  scalar_to_long by hand-derived answers at the branch edges.
"""
import itertools
import random

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


def fr(vals):
    return C.ints_to_fr(vals) if len(vals) else np.zeros((0, 8), np.uint32)


def mle_nd(t, shape, us):
    """sum over all indices of t[idx] * prod_d eq(idx_d, us[d]) (row-major t)."""
    acc = 0
    for idx in itertools.product(*[range(s) for s in shape]):
        flat = 0
        for d, i in enumerate(idx):
            flat = flat * shape[d] + i
        w = 1
        for d, i in enumerate(idx):
            w = w * P.eq_weight(i, us[d]) % R
        acc = (acc + w * t[flat]) % R
    return acc


# ------------------------------------------------------------------ window partial_me
@pytest.mark.parametrize("n,W,k", [(40, 3, 2), (33, 4, 1), (64, 4, 3), (17, 5, 1), (9, 1, 3)])
def test_partial_me_window_multi_row(n, W, k):
    rng = random.Random(n * 31 + W)
    t, u = rnd(rng, n), rnd(rng, k)
    rc, out = C.partial_me_window(C.ints_to_fr(t), C.ints_to_fr(u), W)
    assert rc == 0
    rows = (n + W - 1) // W
    orows = -(-rows // (1 << k))
    assert len(out) == orows * W
    want = [sum(P.eq_weight(b, u) * (t[(w * (1 << k) + b) * W + j] if (w * (1 << k) + b) * W + j < n else 0)
                for b in range(1 << k)) % R for w in range(orows) for j in range(W)]
    assert C.fr_to_ints(out) == want
    # size rule of FrTensor::partial_me(u, window) (fr-tensor.cu:512-516)
    rc, _ = C.partial_me_window(C.ints_to_fr(t[:W * (1 << (k - 1))]), C.ints_to_fr(u), W)
    assert rc == 1


def test_pad_with_value():
    rng = random.Random(3)
    shape, pv = [3, 5, 2], rng.randrange(R)
    t = rnd(rng, 30)
    rc, out = C.pad_val(C.ints_to_fr(t), shape, L(pv))
    assert rc == 0 and len(out) == 4 * 8 * 2
    got = C.fr_to_ints(out)
    for i, j, k in itertools.product(range(4), range(8), range(2)):
        want = t[(i * 5 + j) * 2 + k] if i < 3 and j < 5 else pv
        assert got[(i * 8 + j) * 2 + k] == want
    rc0, out0 = C.pad_val(C.ints_to_fr(t), shape, L(0))
    assert rc0 == 0
    in_shape = [(g // 16) < 3 and (g // 2) % 8 < 5 for g in range(64)]
    assert C.fr_to_ints(out0) == [v if ins else 0 for v, ins in zip(got, in_shape)]


# ------------------------------------------------------------------ zkip
@pytest.mark.parametrize("n", [1, 2, 3, 5, 8, 13, 16, 37])
def test_zkip_pins(n):
    rng = random.Random(100 + n)
    a, b = rnd(rng, n), rnd(rng, n)
    Lv = P.ceil_log2(n)
    u = rnd(rng, Lv)
    claim = sum(x * y for x, y in zip(a, b)) % R
    rc, proof, fin = C.zkip(L(claim), C.ints_to_fr(a), C.ints_to_fr(b), fr(u))
    assert rc == 0 and len(proof) == 3 * Lv
    assert I(fin) == P.mle(a, u) * P.mle(b, u) % R
    # the proof chain: p(0)+p(1) = running claim, next claim p(u_last)
    cur = claim
    for r in range(Lv):
        c0, c1, c2 = C.fr_to_ints(proof[3 * r:3 * r + 3])
        assert (2 * c0 + c1 + c2) % R == cur
        x = u[Lv - 1 - r]
        cur = (c0 + c1 * x + c2 * x * x) % R
    assert cur == I(fin)
    if n > 1:
        rc, _, _ = C.zkip(L(claim + 1), C.ints_to_fr(a), C.ints_to_fr(b), fr(u))
        assert rc == 2


@pytest.mark.parametrize("n,k", [(16, 2), (13, 1), (37, 3)])
def test_zkip_partial_rounds(n, k):
    """k < ceilLog2(n) rounds bind the top k index bits: the final claim is
    sum_j a'_j b'_j with a'_j = sum_h eq(h, u) a[j + h 2^(L-k)] (zero padding)."""
    rng = random.Random(200 + n)
    a, b = rnd(rng, n), rnd(rng, n)
    Lv = P.ceil_log2(n)
    u = rnd(rng, k)
    claim = sum(x * y for x, y in zip(a, b)) % R
    rc, proof, fin = C.zkip(L(claim), C.ints_to_fr(a), C.ints_to_fr(b), fr(u))
    assert rc == 0
    lo = 1 << (Lv - k)
    ext = lambda t, i: t[i] if i < n else 0
    ap = [sum(P.eq_weight(h, u) * ext(a, j + h * lo) for h in range(1 << k)) % R for j in range(lo)]
    bp = [sum(P.eq_weight(h, u) * ext(b, j + h * lo) for h in range(1 << k)) % R for j in range(lo)]
    assert I(fin) == sum(x * y for x, y in zip(ap, bp)) % R
    rc, _, _ = C.zkip(L(claim), C.ints_to_fr(a), C.ints_to_fr(b), fr(rnd(rng, Lv + 1)))
    assert rc == 1


@pytest.mark.parametrize("N,D", [(1, 4), (2, 3), (3, 5), (4, 8), (7, 6), (8, 1), (5, 13)])
def test_zkip_stacked_pins(N, D):
    rng = random.Random(300 + 17 * N + D)
    A, B = rnd(rng, N * D), rnd(rng, N * D)
    kN, kD = P.ceil_log2(N), P.ceil_log2(D)
    uN, vN, uD = rnd(rng, kN), rnd(rng, kN), rnd(rng, kD)
    claim = sum(P.eq_weight(n, uN) * A[n * D + d] * B[n * D + d] for n in range(N) for d in range(D)) % R
    rc, proof, fin = C.zkip_stacked(L(claim), C.ints_to_fr(A), C.ints_to_fr(B), fr(uN), fr(uD), fr(vN), N, D)
    assert rc == 0 and len(proof) == 3 * (kN + kD)
    assert I(fin) == P.mle2(A, N, D, vN, uD) * P.mle2(B, N, D, vN, uD) % R
    # stacked rounds: claim = (1-u) p(0) + u p(1) with u = uN.back(); then p(v)
    cur = claim
    for r in range(kN):
        c0, c1, c2 = C.fr_to_ints(proof[3 * r:3 * r + 3])
        ul = uN[kN - 1 - r]
        assert ((1 - ul) * c0 + ul * (c0 + c1 + c2)) % R == cur
        v = vN[kN - 1 - r]
        cur = (c0 + c1 * v + c2 * v * v) % R
    rc, _, _ = C.zkip_stacked(L(claim + 1), C.ints_to_fr(A), C.ints_to_fr(B), fr(uN), fr(uD), fr(vN), N, D)
    assert rc == 2
    rc, _, _ = C.zkip_stacked(L(claim), C.ints_to_fr(A), C.ints_to_fr(B), fr(uN + [1]), fr(uD), fr(vN + [1]), N, D)
    assert rc == 1


@pytest.mark.parametrize("num,B,IN,OUT,bias", [(2, 4, 8, 4, False), (3, 5, 6, 3, True), (1, 2, 3, 2, True),
                                               (4, 1, 4, 5, False)])
def test_fc_stacked_pins(num, B, IN, OUT, bias):
    rng = random.Random(400 + num * 100 + B * 10 + IN)
    X = [rng.randrange(-999, 1000) for _ in range(num * B * IN)]
    W = [rng.randrange(-999, 1000) for _ in range(num * IN * OUT)]
    bv = [rng.randrange(-99, 100) for _ in range(num * OUT)] if bias else None
    Y = []
    for s in range(num):
        for i in range(B):
            for o in range(OUT):
                y = sum(X[(s * B + i) * IN + j] * W[(s * IN + j) * OUT + o] for j in range(IN))
                Y.append(y + (bv[s * OUT + o] if bias else 0))
    kn, kb, ki, ko = (P.ceil_log2(x) for x in (num, B, IN, OUT))
    un, vn, ub, ui, uo = rnd(rng, kn), rnd(rng, kn), rnd(rng, kb), rnd(rng, ki), rnd(rng, ko)
    Xf, Wf, Yf = (C.ints_to_fr(v) for v in (X, W, Y))
    bf = C.ints_to_fr(bv) if bias else None
    rc, proof, claims = C.fc_stacked_prove(Xf, Wf, Yf, bf, num, B, IN, OUT, fr(un), fr(vn), fr(ub), fr(ui), fr(uo))
    assert rc == 0 and len(proof) == 3 * (kn + ki)
    Xm, Wm, Ym = ([v % R for v in t] for t in (X, W, Y))
    want = mle_nd(Ym, [num, B, OUT], [un, ub, uo])
    if bias:
        ones = P.mle([1] * B, ub)
        want = (want - ones * mle_nd([v % R for v in bv], [num, OUT], [un, uo])) % R
    assert I(claims[0]) == want
    assert I(claims[1]) == mle_nd(Xm, [num, B, IN], [vn, ub, ui]) * mle_nd(Wm, [num, IN, OUT], [vn, ui, uo]) % R
    Y2 = list(Y)
    Y2[-1] += 1
    rc, _, _ = C.fc_stacked_prove(Xf, Wf, C.ints_to_fr(Y2), bf, num, B, IN, OUT, fr(un), fr(vn), fr(ub), fr(ui),
                                  fr(uo))
    assert rc == 2


# ------------------------------------------------------------------ rescaling
def test_scalar_to_long_known_answers():
    for v in [0, 1, -1, 12345, -12345, (1 << 62), -(1 << 62), (1 << 63) - 1, -((1 << 63) - 1)]:
        assert C.scalar_to_long(L(v)) == v
    assert C.scalar_to_long(L(1 << 63)) == 0            # bit 63 set: r - x is wide -> 0
    assert C.scalar_to_long(L(R - (1 << 63))) == -(1 << 63)  # r - x = 2^63 -> -(long)2^63
    assert C.scalar_to_long(L(1 << 64)) == 0
    assert C.scalar_to_long(L(R - (1 << 64))) == 0      # r - x = 2^64 has limb 2 set
    assert C.scalar_to_long(L(R - 5)) == -5


@pytest.mark.parametrize("sf", [1, 2, 3, 7, 256, 1 << 16])
def test_rescale_identity(sf):
    rng = random.Random(sf)
    xs = [0, 1, -1, sf, -sf, sf // 2, -(sf // 2), sf // 2 - 1, -(sf // 2) - 1, (1 << 40) + 3, -(1 << 40) - 3]
    xs += [rng.randrange(-(1 << 50), 1 << 50) for _ in range(200)]
    hsf = sf >> 1
    for rc, q, r in [C.rescale(np.array(xs, np.int64), sf), C.rescale(C.ints_to_fr(xs), sf)]:
        assert rc == 0
        for x, qq, rr in zip(xs, q.tolist(), r.tolist()):
            assert qq * sf + rr == x and -hsf <= rr < sf - hsf, (x, sf, qq, rr)
    assert C.rescale(np.array([5], np.int64), 0)[0] == 1


# ------------------------------------------------------------------ witness GEMM
@pytest.mark.parametrize("M,N,Pc", [(1, 1, 1), (3, 5, 4), (7, 2, 9)])
def test_matmul_fr_definition(M, N, Pc):
    """The oracle's field matmul (Montgomery accumulation, fr-tensor.cu:862-872) against
    sum_k A[i][k] B[k][j] mod r on full-size field elements and on small signed integers
    (where it is the integer product reduced mod r), with and without a bias."""
    rng = random.Random(M * 100 + N * 10 + Pc)
    for full in (True, False):
        A = rnd(rng, M * N) if full else [rng.randrange(-2**20, 2**20) for _ in range(M * N)]
        B = rnd(rng, N * Pc) if full else [rng.randrange(-2**20, 2**20) for _ in range(N * Pc)]
        bias = rnd(rng, Pc)
        for bv in (None, bias):
            rc, got = C.matmul_fr(C.ints_to_fr(A), C.ints_to_fr(B), M, N, Pc, C.ints_to_fr(bv) if bv else None)
            assert rc == 0
            want = [(sum(A[i * N + k] * B[k * Pc + j] for k in range(N)) + (bv[j] if bv else 0)) % R
                    for i in range(M) for j in range(Pc)]
            assert [I(x) for x in got] == want
    assert C.matmul_fr(C.ints_to_fr([1]), C.ints_to_fr([1]), 0, 1, 1)[0] == 1
