"""GPU parity for the MLE helpers and the transcript-free inner-product sumchecks:
window partial_me (fr-tensor.cu:612-641), pad with a pad value (fr-tensor.cu:800-828), the
range table (tlookup.cu:372-391), zkip / zkip_stacked / zkFCStacked::prove
(zkfc.cu:94-307) and the rescaling witness (rescaling.cu:8-21) -- libzkh.so on the GPU
against the C oracle on the same seeded inputs, bit-exact."""
import numpy as np
import pytest

from oracle import coracle as C
from oracle import pyref as P

pytestmark = pytest.mark.gpu


def rand_fr(rng, n):
    return C.ints_to_fr([int.from_bytes(rng.bytes(32), "little") % P.R for _ in range(n)]) if n else \
        np.zeros((0, 8), np.uint32)


def fr_eq(a, b):
    return np.array_equal(np.asarray(a, np.uint32).reshape(-1, 8), np.asarray(b, np.uint32).reshape(-1, 8))


@pytest.mark.parametrize("n,W,k", [(40, 3, 2), (33, 4, 1), (64, 4, 3), (17, 5, 1), (9, 1, 3), (100000, 64, 4)])
@pytest.mark.parametrize("kind", ["fr", "i32", "i64"])
def test_partial_me_window(zkh, ctx, n, W, k, kind):
    rng = np.random.default_rng(n + W + k)
    vals = rng.integers(-2**30, 2**30, size=n)
    t = rand_fr(rng, n) if kind == "fr" else C.ints_to_fr(vals)
    u = rand_fr(rng, k)
    rc, want = C.partial_me_window(t, u, W)
    assert rc == 0
    tg = ctx.from_fr(t) if kind == "fr" else ctx.from_i32(vals) if kind == "i32" else ctx.from_i64(vals)
    assert fr_eq(ctx.partial_me_window(tg, u, W).to_fr(), want)


def test_partial_me_window_size_rule(zkh, ctx):
    rng = np.random.default_rng(1)
    with pytest.raises(zkh.ZkhError) as e:
        ctx.partial_me_window(ctx.from_fr(rand_fr(rng, 8)), rand_fr(rng, 3), 2)
    assert e.value.code == zkh.EARG


@pytest.mark.parametrize("shape", [[3, 5, 6], [7], [1, 1], [5, 1, 3], [33, 65]])
def test_pad(zkh, ctx, shape):
    rng = np.random.default_rng(len(shape) * 10 + shape[0])
    n = int(np.prod(shape))
    x = rand_fr(rng, n)
    pv = rand_fr(rng, 1)
    for val in (None, pv):
        rc, want = C.pad_val(x, shape, np.zeros(8, np.uint32) if val is None else val[0])
        assert rc == 0
        assert fr_eq(ctx.pad(ctx.from_fr(x), shape, val).to_fr(), want)
    ints = rng.integers(-50, 50, size=n)
    rc, want = C.pad_val(C.ints_to_fr(ints), shape, pv[0])
    assert fr_eq(ctx.pad(ctx.from_i32(ints), shape, pv).to_fr(), want)
    with pytest.raises(zkh.ZkhError):
        ctx.pad(ctx.from_fr(x), shape + [2])


@pytest.mark.parametrize("low,length,N", [(-8, 16, 16), (-32768, 65536, 65536), (5, 3, 8), (-(1 << 21), 1 << 22, 1 << 22),
                                           (2**31 - 4, 8, 8), (-2**31, 4, 8)])
def test_range_table(zkh, ctx, low, length, N):
    """tLookupRange's table (int32 entries, the reference's 32-bit arithmetic wrapping past
    2^31 - 1) against the oracle, with padding past len."""
    assert fr_eq(ctx.range_table(low, length, N).to_fr(), C.range_table(low, length, N))


# ---------------------------------------------------------------- zkip / zkip_stacked
@pytest.mark.parametrize("n,k", [(1, 0), (2, 1), (3, 2), (13, 4), (16, 2), (1000, 10), (5000, 13), (70000, 17),
                                 (70000, 5)])
def test_zkip(zkh, ctx, n, k):
    rng = np.random.default_rng(n * 7 + k)
    a, b = rand_fr(rng, n), rand_fr(rng, n)
    u = rand_fr(rng, k)
    claim = np.zeros(8, np.uint32)
    for x, y in zip(C.fr_to_ints(a), C.fr_to_ints(b)):  # sum a_i b_i
        claim = C.fr_op("add", claim, C.fr_op("mul", P.to_limbs(x), P.to_limbs(y)))
    rc, pw, fw = C.zkip(claim, a, b, u)
    assert rc == 0
    pg, fg = ctx.zkip(claim, ctx.from_fr(a), ctx.from_fr(b), u)
    assert fr_eq(pg, pw) and fr_eq(fg, fw)
    if k:
        bad = C.fr_op("add", claim, P.to_limbs(1))
        with pytest.raises(zkh.ZkhError) as e:
            ctx.zkip(bad, ctx.from_fr(a), ctx.from_fr(b), u)
        assert e.value.code == zkh.EROUND


def _stacked_claim(A, B, uN, N, D):
    Ai, Bi, ui = C.fr_to_ints(A), C.fr_to_ints(B), C.fr_to_ints(uN)
    s = sum(P.eq_weight(n, ui) * Ai[n * D + d] * Bi[n * D + d] for n in range(N) for d in range(D)) % P.R
    return np.array(P.to_limbs(s), np.uint32)


@pytest.mark.parametrize("N,D", [(1, 4), (2, 3), (3, 5), (4, 8), (7, 6), (8, 1), (16, 100), (7, 2048)])
def test_zkip_stacked(zkh, ctx, N, D):
    rng = np.random.default_rng(N * 1000 + D)
    A, B = rand_fr(rng, N * D), rand_fr(rng, N * D)
    kN, kD = P.ceil_log2(N), P.ceil_log2(D)
    uN, vN, uD = rand_fr(rng, kN), rand_fr(rng, kN), rand_fr(rng, kD)
    claim = _stacked_claim(A, B, uN, N, D)
    rc, pw, fw = C.zkip_stacked(claim, A, B, uN, uD, vN, N, D)
    assert rc == 0
    pg, fg = ctx.zkip_stacked(claim, ctx.from_fr(A), ctx.from_fr(B), uN, uD, vN, N, D)
    assert fr_eq(pg, pw) and fr_eq(fg, fw)
    with pytest.raises(zkh.ZkhError) as e:
        ctx.zkip_stacked(C.fr_op("add", claim, P.to_limbs(1)), ctx.from_fr(A), ctx.from_fr(B), uN, uD, vN, N, D)
    assert e.value.code == zkh.EROUND


@pytest.mark.parametrize("num,B,IN,OUT,bias", [(2, 4, 8, 4, False), (3, 5, 6, 3, True), (1, 2, 3, 2, True),
                                               (4, 1, 4, 5, False), (7, 64, 256, 96, True)])
def test_fc_stacked_prove(zkh, ctx, num, B, IN, OUT, bias):
    rng = np.random.default_rng(num * 100 + B + IN)
    X = rng.integers(-300, 300, size=(num, B, IN)).astype(np.int64)
    W = rng.integers(-300, 300, size=(num, IN, OUT)).astype(np.int64)
    bv = rng.integers(-99, 100, size=(num, OUT)).astype(np.int64)
    Y = np.einsum("sbi,sio->sbo", X, W) + (bv[:, None, :] if bias else 0)
    kn, kb, ki, ko = (P.ceil_log2(x) for x in (num, B, IN, OUT))
    un, vn, ub, ui, uo = (rand_fr(rng, k) for k in (kn, kn, kb, ki, ko))
    Xf, Wf, Yf = (C.ints_to_fr(v.reshape(-1).tolist()) for v in (X, W, Y))
    bf = C.ints_to_fr(bv.reshape(-1).tolist()) if bias else None
    rc, pw, cw = C.fc_stacked_prove(Xf, Wf, Yf, bf, num, B, IN, OUT, un, vn, ub, ui, uo)
    assert rc == 0
    bg = ctx.from_i64(bv) if bias else None
    for tx, tw, ty in [(ctx.from_i32(X), ctx.from_i32(W), ctx.from_i64(Y)),
                       (ctx.from_fr(Xf), ctx.from_fr(Wf), ctx.from_fr(Yf))]:
        pg, cg = ctx.fc_stacked_prove(tx, tw, ty, bg, num, B, IN, OUT, un, vn, ub, ui, uo)
        assert fr_eq(pg, pw) and fr_eq(cg, cw)
    Y2 = Y.copy()
    Y2[0, 0, 0] += 1
    with pytest.raises(zkh.ZkhError) as e:
        ctx.fc_stacked_prove(ctx.from_i32(X), ctx.from_i32(W), ctx.from_i64(Y2), bg, num, B, IN, OUT,
                             un, vn, ub, ui, uo)
    assert e.value.code == zkh.EROUND


# ---------------------------------------------------------------- rescaling witness
@pytest.mark.parametrize("sf", [1, 2, 3, 256, 1 << 16])
def test_rescale(zkh, ctx, sf):
    rng = np.random.default_rng(sf)
    x = np.concatenate([rng.integers(-(1 << 40), 1 << 40, size=5000),
                        np.array([0, 1, -1, sf, -sf, sf // 2, -(sf // 2), sf // 2 - 1, -(sf // 2) - 1])])
    rc, qw, rw = C.rescale(x.astype(np.int64), sf)
    assert rc == 0
    q, r = ctx.rescale(ctx.from_i64(x), sf)
    assert q.kind == zkh.KIND_I64 and r.kind == zkh.KIND_I64
    assert fr_eq(q.to_fr(), C.ints_to_fr(qw.tolist())) and fr_eq(r.to_fr(), C.ints_to_fr(rw.tolist()))
    small = (x % (1 << 20)).astype(np.int32) - (1 << 19)
    rc, qs, rs = C.rescale(small.astype(np.int64), sf)
    q, r = ctx.rescale(ctx.from_i32(small), sf)
    assert fr_eq(q.to_fr(), C.ints_to_fr(qs.tolist())) and fr_eq(r.to_fr(), C.ints_to_fr(rs.tolist()))
    # FR input read through scalar_to_long, including values outside the long range
    xf = np.concatenate([C.ints_to_fr(x[:100].tolist()), rand_fr(rng, 50)])
    rc, qf, rf = C.rescale(xf, sf)
    q, r = ctx.rescale(ctx.from_fr(xf), sf)
    assert fr_eq(q.to_fr(), C.ints_to_fr(qf.tolist())) and fr_eq(r.to_fr(), C.ints_to_fr(rf.tolist()))
