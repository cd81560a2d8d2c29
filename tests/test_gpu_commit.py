"""GPU parity for the Pedersen commitment (zkh_commit): Commitment::commit = commit_pippenger
(commitment.cu:47-108).  Every output point is compared byte for byte with the C oracle,
whose G1 arithmetic and schedule tests/test_oracle_g1.py pins: the Jacobian bytes are what
the reference's transcript absorbs (zkob_fc.cu:256-258), so equal group elements are not
enough.  Generators are G1Jacobian_mul(G, random) as Commitment::random makes them
(commitment.cu:3-8), with Z != 1.  Covered: every tensor kind (FR, int32, int64, registered
weights), rows that are not a multiple of the 64-row wave, zero rows and zero columns,
repeated and opposite generators (the doubling and P + (-P) branches of the addition),
a generator at infinity, and the dimension errors; at a matmul's real shape (X of a
TinyLlama projection, 512 x 2048) sampled rows are checked against the oracle."""
import numpy as np
import pytest

from oracle import coracle as C
from oracle import pyg1 as G
from oracle import pyref as P

pytestmark = pytest.mark.gpu

_BASE = G.aff_to_jac((G.GX, G.GY))


def gens_for(seed, n):
    rng = np.random.default_rng(seed)
    out = np.zeros((n, 36), np.uint32)
    for i in range(n):
        k = int.from_bytes(rng.bytes(32), "little") % P.R
        out[i] = C.g1_mul(_BASE, np.array(P.to_limbs(k), np.uint32))
    return out


def scalars_mixed(rng, count):
    """small signed ints (the witness tables) mixed with full-width field elements."""
    small = rng.integers(-229376, 229377, size=count)
    full = [int.from_bytes(rng.bytes(32), "little") % P.R for _ in range(count)]
    pick = rng.random(count) < 0.25
    return [full[i] if pick[i] else int(small[i]) for i in range(count)]


def check(ctx, gens, t, sc_fr, n, rows=None):
    g = ctx.g1_from_host(gens)
    got = ctx.commit(g, t).to_host()
    m = sc_fr.shape[0] // n
    assert got.shape == (m, 36)
    rows = range(m) if rows is None else rows
    for r in rows:
        rc, want = C.g1_commit(gens, sc_fr[r * n:(r + 1) * n], n)
        assert rc == 0
        assert np.array_equal(got[r], want[0]), "row %d" % r


@pytest.mark.parametrize("m,n", [(1, 1), (3, 5), (2, 64), (70, 16), (5, 257)])
def test_commit_fr_vs_oracle(ctx, m, n):
    rng = np.random.default_rng(m * 1000 + n)
    gens = gens_for(n, n)
    sc = C.ints_to_fr(scalars_mixed(rng, m * n))
    check(ctx, gens, ctx.from_fr(sc), sc, n)


@pytest.mark.parametrize("kind", ["i32", "i64", "weights"])
def test_commit_int_kinds(ctx, kind):
    rng = np.random.default_rng(11)
    m, n = 9, 24
    gens = gens_for(3, n)
    if kind == "i64":
        v = rng.integers(-2**40, 2**40, size=m * n).astype(np.int64)
        t = ctx.from_i64(v)
    else:
        v = rng.integers(-2**17, 2**17, size=m * n).astype(np.int32)
        t = ctx.weights_i32(v, m, n) if kind == "weights" else ctx.from_i32(v)
    check(ctx, gens, t, C.ints_to_fr(v), n)


def test_commit_zero_rows_and_columns(ctx):
    rng = np.random.default_rng(12)
    m, n = 6, 8
    v = rng.integers(-1000, 1000, size=(m, n)).astype(np.int32)
    v[2] = 0
    v[:, 5] = 0
    gens = gens_for(4, n)
    check(ctx, gens, ctx.from_i32(v.reshape(-1)), C.ints_to_fr(v.reshape(-1)), n)
    got = ctx.commit(ctx.g1_from_host(gens), ctx.from_i32(v.reshape(-1))).to_host()
    assert np.array_equal(got[2], G.g1_zero())


def test_commit_special_generators(ctx):
    """equal generators (U1 = U2, S1 = S2: doubling), a generator and its negation
    (P + (-P) = a Z = 0 point that later additions skip) and a generator at infinity."""
    n = 6
    gens = gens_for(5, n)
    gens[1] = gens[0]
    neg = gens[0].copy()
    y = G.from_limbs12(neg[12:24])
    neg[12:24] = G.limbs12((G.P - y) % G.P)
    gens[2] = neg
    gens[4] = G.jac_point(0, 1, 0)
    rng = np.random.default_rng(13)
    v = rng.integers(-50, 50, size=(40, n)).astype(np.int32)
    v[0] = [3, 3, 3, 0, 7, 1]      # same digits for 0, 1 and 2 in window 0
    v[1] = [-5, -5, -5, 2, 2, -5]  # negatives: every high window sees all three
    check(ctx, gens, ctx.from_i32(v.reshape(-1)), C.ints_to_fr(v.reshape(-1)), n)


def test_commit_dimension_errors(zkh, ctx):
    gens = ctx.g1_from_host(gens_for(6, 4))
    with pytest.raises(zkh.ZkhError) as e:
        ctx.commit(gens, ctx.from_i32(np.arange(10, dtype=np.int32)))
    assert e.value.code == zkh.EARG
    many = ctx.g1_from_host(np.tile(G.g1_zero(), (65537, 1)))
    with pytest.raises(zkh.ZkhError) as e:
        ctx.commit(many, ctx.from_i32(np.zeros(65537, np.int32)))
    assert e.value.code == zkh.EARG


def test_commit_real_shape_sampled_rows(ctx):
    """X of a TinyLlama projection: 512 rows of 2048 (int16-range activations)."""
    rng = np.random.default_rng(14)
    m, n = 512, 2048
    gens = gens_for(7, n)
    v = rng.integers(-2**15, 2**15, size=m * n).astype(np.int32)
    sc = C.ints_to_fr(v[:3 * n])
    g = ctx.g1_from_host(gens)
    got = ctx.commit(g, ctx.from_i32(v)).to_host()
    for r in (0, 1, 2):
        rc, want = C.g1_commit(gens, sc[r * n:(r + 1) * n], n)
        assert np.array_equal(got[r], want[0]), "row %d" % r
    for r in (200, 511):
        rc, want = C.g1_commit(gens, C.ints_to_fr(v[r * n:(r + 1) * n]), n)
        assert np.array_equal(got[r], want[0]), "row %d" % r


def test_commit_shared_chain_edges(ctx):
    """values whose high digits break the shared-list pattern in some windows only: -1
    (digits of r itself), -2 and 2 (one above / below), magnitudes at window boundaries
    (2^k - 1, 2^k), int32 extremes; rows mixing them with ordinary small negatives, so
    that equal fingerprints must be confirmed and near-equal lists must stay apart."""
    rng = np.random.default_rng(15)
    edge = [-1, -2, 2, 1, 0, -(2**20), 2**20, -(2**20) + 1, 2**31 - 1, -(2**31), 15, -15, 16, -16]
    m, n = 66, 40
    v = rng.integers(-300, 300, size=(m, n)).astype(np.int64)
    for r in range(m):
        k = rng.integers(0, 4)
        v[r, rng.integers(0, n, size=k)] = rng.choice(edge, size=k)
    v[0] = -1
    v[1] = -5
    v[2, ::2] = -1
    v[3] = np.where(np.arange(n) % 3 == 0, -(2**20), -7)
    v = v.astype(np.int32)
    gens = gens_for(8, n)
    check(ctx, gens, ctx.from_i32(v.reshape(-1)), C.ints_to_fr(v.reshape(-1)), n)


def test_g1_generator_matches_reference_constant(zkh):
    assert np.array_equal(zkh.g1_generator(), G.aff_to_jac((G.GX, G.GY)))


def test_g1_mul_vs_oracle(zkh, ctx):
    """G1Jacobian_mul elementwise with a broadcast base (Commitment::random's step)."""
    rng = np.random.default_rng(16)
    n = 70
    ks = [int.from_bytes(rng.bytes(32), "little") % P.R for _ in range(n - 6)] + [0, 1, 2, P.R - 1, 2**255 - 1, 2**128]
    sc = np.zeros((n, 8), np.uint32)
    for i, k in enumerate(ks):
        sc[i] = P.to_limbs(k)   # raw bits, as G1Jacobian_mul reads them (2^255 - 1 is not reduced)
    bases = gens_for(9, 3)
    # from_fr takes canonical values only
    canon = [i for i, k in enumerate(ks) if k < P.R]
    g = ctx.g1_mul(ctx.g1_from_host(bases), ctx.from_fr(sc[canon])).to_host()
    for j, i in enumerate(canon):
        want = C.g1_mul(bases[j % 3], sc[i])
        assert np.array_equal(g[j], want), i
    one = ctx.g1_mul(ctx.g1_from_host(zkh.g1_generator()[None, :]), ctx.from_i32(np.array([3, -1, 0], np.int32))).to_host()
    base = zkh.g1_generator()
    assert np.array_equal(one[0], C.g1_mul(base, np.array(P.to_limbs(3), np.uint32)))
    assert np.array_equal(one[1], C.g1_mul(base, np.array(P.to_limbs(P.R - 1), np.uint32)))
    assert np.array_equal(one[2], G.g1_zero())


def test_g1_addmul_vs_oracle(zkh, ctx):
    """hb_addmul, mul_first false (zkob_fastg1.cuh:56-88): out[i] = b[i] + a[i] * s, row by
    row, with the addition's special cases: b[i] the point at infinity, b[i] equal to a[i] s
    (the doubling branch), b[i] its negative (infinity), and s = 0."""
    rng = np.random.default_rng(23)
    n = 40
    a = gens_for(31, n)
    for s in [int.from_bytes(rng.bytes(32), "little") % P.R, 0, 1, P.R - 1]:
        sl = np.array(P.to_limbs(s), np.uint32)
        b = gens_for(32, n)
        b[0] = G.g1_zero()
        b[1] = C.g1_mul(a[1], sl)
        b[2] = C.g1_mul(a[2], np.array(P.to_limbs((P.R - s) % P.R), np.uint32))
        got = ctx.g1_addmul(ctx.g1_from_host(a), sl, ctx.g1_from_host(b)).to_host()
        for i in range(n):
            assert np.array_equal(got[i], C.g1_add(b[i], C.g1_mul(a[i], sl))), (s, i)
        # the group element: b + s a, by affine arithmetic
        assert G.to_affine(got[3]) == G.aff_add(G.to_affine(b[3]), G.aff_mul(G.to_affine(a[3]), s))
        assert G.to_affine(got[2]) is None and G.to_affine(got[0]) == G.aff_mul(G.to_affine(a[0]), s)
    with pytest.raises(zkh.ZkhError) as e:
        ctx.g1_addmul(ctx.g1_from_host(a), np.zeros(8, np.uint32), ctx.g1_from_host(a[:3]))
    assert e.value.code == zkh.EARG


@pytest.mark.parametrize("n", [1, 2, 4, 32, 256])
def test_ipa_prove_vs_oracle(zkh, ctx, n):
    """ipa_prove (vrf_common.cuh:302-336): L, R (absorbed, so byte-exact), a_final and the
    transcript state equal the oracle's, with b = me_weights(u) as the drivers pass it."""
    rng = np.random.default_rng(300 + n)
    gens = gens_for(20 + n, n + 1)
    g, Q = gens[:n], gens[n]
    a = [int.from_bytes(rng.bytes(32), "little") % P.R for _ in range(n)]
    u = [int.from_bytes(rng.bytes(32), "little") % P.R for _ in range(max(n.bit_length() - 1, 0))]
    b = [P.eq_weight(k, u) if u else 1 for k in range(n)]
    st_g = zkh.transcript("ipa-%d" % n)
    st_o = C.tr_init("ipa-%d" % n)
    got = ctx.ipa_prove(st_g, ctx.from_fr(C.ints_to_fr(a)), ctx.from_fr(C.ints_to_fr(b)), ctx.g1_from_host(g), Q)
    rc, L, R, af = C.ipa_prove(st_o, C.ints_to_fr(a), C.ints_to_fr(b), g, Q, n)
    assert rc == 0
    assert np.array_equal(got["L"], L) and np.array_equal(got["R"], R)
    assert np.array_equal(got["a_final"], af)
    assert bytes(st_g) == bytes(st_o)


def test_ipa_prove_int_witness_and_errors(zkh, ctx):
    """a from an int32 tensor (a folded weight row is small until it is folded); sizes that
    are not a power of two or disagree are ZKH_EARG."""
    n = 16
    rng = np.random.default_rng(310)
    v = rng.integers(-229376, 229377, size=n).astype(np.int32)
    gens = gens_for(40, n + 1)
    u = [int.from_bytes(rng.bytes(32), "little") % P.R for _ in range(4)]
    b = C.ints_to_fr([P.eq_weight(k, u) for k in range(n)])
    st_g, st_o = zkh.transcript("ipa-int"), C.tr_init("ipa-int")
    got = ctx.ipa_prove(st_g, ctx.from_i32(v), ctx.from_fr(b), ctx.g1_from_host(gens[:n]), gens[n])
    rc, L, R, af = C.ipa_prove(st_o, C.ints_to_fr(v), b, gens[:n], gens[n], n)
    assert np.array_equal(got["L"], L) and np.array_equal(got["R"], R) and np.array_equal(got["a_final"], af)
    with pytest.raises(zkh.ZkhError) as e:
        ctx.ipa_prove(zkh.transcript("x"), ctx.from_i32(v[:12]), ctx.from_fr(b[:12]), ctx.g1_from_host(gens[:12]), gens[n])
    assert e.value.code == zkh.EARG
    with pytest.raises(zkh.ZkhError) as e:
        ctx.ipa_prove(zkh.transcript("x"), ctx.from_i32(v[:8]), ctx.from_fr(b), ctx.g1_from_host(gens[:n]), gens[n])
    assert e.value.code == zkh.EARG


def test_ipa_prove_batch_vs_oracle(zkh, ctx):
    """zkh_ipa_prove_batch: jobs of different n (1, 2, 8, 32, 64: 0 to 6 rounds, so jobs drop
    out of the lockstep rounds at different points) and transcripts, each job byte-identical
    to the oracle's ipa_prove on its own transcript; 0 or 9 jobs are ZKH_EARG."""
    rng = np.random.default_rng(330)
    jobs, want = [], []
    for t, n in enumerate((32, 1, 8, 64, 2)):
        gens = gens_for(60 + t, n + 1)
        a = C.ints_to_fr([int.from_bytes(rng.bytes(32), "little") % P.R for _ in range(n)])
        u = [int.from_bytes(rng.bytes(32), "little") % P.R for _ in range(max(n.bit_length() - 1, 0))]
        b = C.ints_to_fr([P.eq_weight(k, u) if u else 1 for k in range(n)])
        st_o = C.tr_init("ipab-%d" % t)
        rc, L, R, af = C.ipa_prove(st_o, a, b, gens[:n], gens[n], n)
        assert rc == 0
        want.append((L, R, af, bytes(st_o)))
        jobs.append((zkh.transcript("ipab-%d" % t), ctx.from_fr(a), ctx.from_fr(b), ctx.g1_from_host(gens[:n]), gens[n]))
    got = ctx.ipa_prove_batch(jobs)
    for (st, *_), g, (L, R, af, st_o) in zip(jobs, got, want):
        assert np.array_equal(g["L"], L) and np.array_equal(g["R"], R)
        assert np.array_equal(g["a_final"], af)
        assert bytes(st) == st_o
    with pytest.raises(zkh.ZkhError) as e:
        ctx.ipa_prove_batch([(zkh.transcript("x"),) + j[1:] for j in jobs[:1] * 9])
    assert e.value.code == zkh.EARG
    with pytest.raises(zkh.ZkhError) as e:
        ctx._chk(zkh.lib().zkh_ipa_prove_batch(ctx.h, 0, None, None, None, None, None, None, None, None))
    assert e.value.code == zkh.EARG


def test_from_fr_rejects_non_canonical(zkh, ctx):
    """zkh_tensor_from_fr checks canonical form on the device: r itself, r + 1 and 2^256 - 1
    anywhere in the array are rejected; r - 1 and 0 round-trip."""
    rng = np.random.default_rng(41)
    n = 5000
    good = np.array([P.to_limbs(int.from_bytes(rng.bytes(32), "little") % P.R) for _ in range(n)], np.uint32)
    good[0], good[n - 1] = P.to_limbs(P.R - 1), P.to_limbs(0)
    assert np.array_equal(ctx.from_fr(good).to_fr(), good)
    for pos, v in ((0, P.R), (n // 2, P.R + 1), (n - 1, 2**256 - 1)):
        bad = good.copy()
        bad[pos] = P.to_limbs(v)
        with pytest.raises(zkh.ZkhError) as e:
            ctx.from_fr(bad)
        assert e.value.code == zkh.EARG, (pos, v)
