"""GPU parity: libzkh.so (HIP, gfx950) against the C oracle on the same seeded inputs.

Bar: bit-exact field elements, identical transcript states.  Shapes are the reference's
own test shapes (vrf_toy_matmul.cu:249-260, vrf_toy_lookup.cu:323-335,
zkob_fc.cu:1246-1248, zkob_rescale.cu:539-541, zkob_glu.cu:711-713) plus BASELINE.json
config 1 and medium sizes that exercise multi-block reductions, odd/non-pow2 dimensions
and the eq split (>= 2^11 pairs).
"""
import numpy as np
import pytest

from oracle import coracle as C
from oracle import pyref as P

pytestmark = pytest.mark.gpu


def rand_fr(rng, n):
    return C.ints_to_fr([int(x) for x in rng.integers(0, 2**63, size=n)] if n else [])


def rand_fr_full(rng, n):
    vals = [int.from_bytes(rng.bytes(32), "little") % P.R for _ in range(n)]
    return C.ints_to_fr(vals)


def fr_eq(a, b):
    return np.array_equal(np.asarray(a, np.uint32).reshape(-1, 8), np.asarray(b, np.uint32).reshape(-1, 8))


def seed_transcript(zkh, label):
    st_g = zkh.transcript(label)
    st_o = C.tr_init(label)
    assert bytes(st_g) == bytes(st_o)
    return st_g, st_o


# ---------------------------------------------------------------- MLE primitives
@pytest.mark.parametrize("n,k", [(1, 0), (5, 3), (8, 3), (1000, 10), (1024, 10), (3000, 12), (70000, 17)])
def test_me(zkh, ctx, n, k):
    rng = np.random.default_rng(n * 31 + k)
    t = rand_fr_full(rng, n)
    u = rand_fr_full(rng, k) if k else np.zeros((0, 8), np.uint32)
    rc, want = C.me(t, u)
    assert rc == 0
    got = ctx.me(ctx.from_fr(t), u)
    assert fr_eq(got, want)


@pytest.mark.parametrize("n,k", [(5, 3), (1000, 10), (70001, 17), (1 << 20, 20)])
def test_me_integer_tensors(zkh, ctx, n, k):
    """FrTensor::operator()(u) of int32 and int64 tensors read as integers (the field x int64
    weighting, its 2^256 removed on the host), with the ends of both ranges and a partial last
    chunk of 1024; and of H = S (.) U over int32 S and U, which comes back as the exact int64
    products.  Against the oracle's evaluation of the same field values."""
    rng = np.random.default_rng(n + k)
    u = rand_fr_full(rng, k)
    v32 = rng.integers(-2**31, 2**31, size=n, dtype=np.int64)
    v32[:4] = [-2**31, 2**31 - 1, -1, 0][: min(4, n)]
    v64 = rng.integers(-2**63, 2**63, size=n, dtype=np.int64)
    v64[:4] = [-2**63, 2**63 - 1, -1, 0][: min(4, n)]
    for vals, t in ((v32, ctx.from_i32(v32.astype(np.int32))), (v64, ctx.from_i64(v64))):
        rc, want = C.me(C.ints_to_fr([int(x) for x in vals]), u)
        assert rc == 0
        assert fr_eq(ctx.me(t, u), want)
    s = rng.integers(-2**31, 2**31, size=n, dtype=np.int64)
    s[:2] = [-2**31, 2**31 - 1][: min(2, n)]
    uu = rng.integers(-2**31, 2**31, size=n, dtype=np.int64)
    uu[:2] = [-2**31, -2**31][: min(2, n)]
    H = ctx.hadamard(ctx.from_i32(s.astype(np.int32)), ctx.from_i32(uu.astype(np.int32)))
    assert zkh.lib().zkh_tensor_kind(H.h) == zkh.KIND_I64
    prod = [int(a) * int(b) for a, b in zip(s, uu)]
    assert fr_eq(H.to_fr(), C.ints_to_fr(prod))
    rc, want = C.me(C.ints_to_fr(prod), u)
    assert fr_eq(ctx.me(H, u), want)


@pytest.mark.parametrize("n,k", [(8, 3), (1000, 10), (70000, 17)])
def test_me_boolean_and_one_coordinates(zkh, ctx, n, k):
    """FrTensor::operator()(u) at points with coordinates 0 and 1: at a Boolean point the MLE
    is the table entry itself; a coordinate 1 among random ones matches the oracle."""
    rng = np.random.default_rng(n + k)
    t = rand_fr_full(rng, n)
    tt = ctx.from_fr(t)
    for idx in (0, n - 1, n // 3):
        u = C.ints_to_fr([(idx >> b) & 1 for b in range(k)])
        assert fr_eq(ctx.me(tt, u), t[idx])
    u = rand_fr_full(rng, k)
    u[k // 2] = C.ints_to_fr([1])[0]
    rc, want = C.me(t, u)
    assert rc == 0
    assert fr_eq(ctx.me(tt, u), want)


@pytest.mark.parametrize("shape", [(6, 5, 3), (4, 8, 1), (1, 7, 2), (3, 64, 5)])
def test_partial_me(zkh, ctx, shape):
    O, Cd, Wd = shape
    rng = np.random.default_rng(sum(shape))
    t = rand_fr_full(rng, O * Cd * Wd)
    k = P.ceil_log2(Cd)
    u = rand_fr_full(rng, k)
    rc, want = C.partial_me(t, u, Cd, Wd)
    assert rc == 0
    got = ctx.partial_me(ctx.from_fr(t), u, Cd, Wd).to_fr()
    assert fr_eq(got, want)


@pytest.mark.parametrize("shape", [(4, 8), (3, 5), (16, 12), (64, 128)])
def test_multi_dim_me_int(zkh, ctx, shape):
    rng = np.random.default_rng(7 + shape[0])
    vals = rng.integers(-2**20, 2**20, size=shape[0] * shape[1])
    us = [rand_fr_full(rng, P.ceil_log2(s)) for s in shape]
    rc, want = C.multi_dim_me(C.ints_to_fr(vals), us, list(shape))
    assert rc == 0
    got = ctx.multi_dim_me(ctx.from_i32(vals), us, list(shape))
    assert fr_eq(got, want)
    got64 = ctx.multi_dim_me(ctx.from_i64(vals.astype(np.int64) * (1 << 20)), us, list(shape))
    rc, want64 = C.multi_dim_me(C.ints_to_fr([int(v) << 20 for v in vals]), us, list(shape))
    assert fr_eq(got64, want64)


def test_eq_table_sum_pad_fold(zkh, ctx):
    rng = np.random.default_rng(11)
    u = rand_fr_full(rng, 6)
    assert fr_eq(ctx.eq_table(u).to_fr(), C.build_eq(u))
    t = rand_fr_full(rng, 777)
    want = np.zeros(8, np.uint32)
    C.lib().or_sum(C._p(np.ascontiguousarray(t)), 777, C._p(want))
    assert fr_eq(ctx.sum(ctx.from_fr(t)), want)
    # pad (3,5,6) -> (4,8,8)
    x = rand_fr_full(rng, 90)
    out = C.frs(256)
    on = C.ctypes.c_uint32(0)
    shp = np.array([3, 5, 6], np.uint32)
    C.lib().or_pad(C._p(np.ascontiguousarray(x)), C._p(shp), 3, C._p(out), C.ctypes.byref(on))
    assert on.value == 256
    assert fr_eq(ctx.pad(ctx.from_fr(x), [3, 5, 6]).to_fr(), out)
    # fold: MSB halving with v
    f = rand_fr_full(rng, 64)
    v = rand_fr_full(rng, 1)
    tf = ctx.from_fr(f)
    ctx.fold(tf, v)
    fi, vi = C.fr_to_ints(f), C.fr_to_ints(v)[0]
    assert C.fr_to_ints(tf.to_fr()) == [(fi[i] + vi * (fi[i + 32] - fi[i])) % P.R for i in range(32)]


# ---------------------------------------------------------------- matmul sumcheck
MM_SHAPES = [(4, 8, 4), (4, 6, 3), (2, 8, 3), (8, 16, 16),  # vrf_toy_matmul.cu:249-260
             (8, 8, 8), (16, 12, 5),                          # zkob_fc.cu:1246-1248
             (1, 4, 2), (3, 5, 7), (1, 1, 1), (5, 1, 3),     # edge: B=1, IN=1
             (64, 128, 64),
             (33, 700, 129), (128, 3000, 64)]                 # multi-block, non-pow2


def _mm_inputs(shape, seed):
    from zkh_synth import fp8_e4m3_ints, gaussian_int16, matmul_exact
    B, IN, OUT = shape
    rng = np.random.default_rng(seed)
    X = fp8_e4m3_ints(rng, (B, IN)) if seed % 2 else gaussian_int16(rng, (B, IN))
    W = fp8_e4m3_ints(rng, (IN, OUT))
    return X, W, matmul_exact(X, W)


@pytest.fixture(scope="module", autouse=True)
def _synth_alias():
    import importlib.util
    import os
    import sys
    if "zkh_synth" not in sys.modules:
        path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                            "zk-hillclimb_amd", "synth.py")
        spec = importlib.util.spec_from_file_location("zkh_synth", path)
        mod = importlib.util.module_from_spec(spec)
        sys.modules["zkh_synth"] = mod
        spec.loader.exec_module(mod)
    yield


@pytest.mark.parametrize("shape", MM_SHAPES)
@pytest.mark.parametrize("weights", [True, False])
def test_mm_prove(zkh, ctx, shape, weights):
    B, IN, OUT = shape
    X, W, Y = _mm_inputs(shape, B * 1000 + IN + OUT)
    st_g, st_o = seed_transcript(zkh, "mm:%d:%d:%d" % shape)
    rc, want = C.mm_prove(st_o, X, W, Y, B, IN, OUT)
    assert rc == 0
    Wt = ctx.weights_i32(W, IN, OUT) if weights else ctx.from_i32(W)
    got = ctx.mm_prove(st_g, ctx.from_i32(X), Wt, ctx.from_i64(Y), B, IN, OUT)
    for key in ("ev", "claims", "u_batch", "u_output", "u_input"):
        assert fr_eq(got[key], want[key]), key
    assert bytes(st_g) == bytes(st_o)


def test_mm_prove_batch(zkh, ctx):
    """All MM_SHAPES proven in one batched call; each job equals its own oracle run."""
    items, wants, sts = [], [], []
    keep = []
    for idx, shape in enumerate(MM_SHAPES):
        B, IN, OUT = shape
        X, W, Y = _mm_inputs(shape, 77 + idx)
        st_g, st_o = seed_transcript(zkh, "batch:%d" % idx)
        rc, want = C.mm_prove(st_o, X, W, Y, B, IN, OUT)
        assert rc == 0
        t = (ctx.from_i32(X), ctx.weights_i32(W, IN, OUT) if idx % 2 else ctx.from_i32(W), ctx.from_i64(Y))
        keep.append(t)
        items.append((st_g, t[0], t[1], t[2], B, IN, OUT))
        wants.append(want)
        sts.append((st_g, st_o))
    outs, status = ctx.mm_prove_batch(items)
    assert status == [0] * len(items)
    for got, want, (st_g, st_o) in zip(outs, wants, sts):
        for key in ("ev", "claims", "u_batch", "u_output", "u_input"):
            assert fr_eq(got[key], want[key]), key
        assert bytes(st_g) == bytes(st_o)


def test_mm_batch_isolates_a_bad_job(zkh, ctx):
    good = _mm_inputs((8, 16, 4), 5)
    X, W, Y = _mm_inputs((8, 16, 4), 6)
    Y = Y.copy()
    Y[0, 0] += 1
    ta = [ctx.from_i32(good[0]), ctx.from_i32(good[1]), ctx.from_i64(good[2])]
    tb = [ctx.from_i32(X), ctx.from_i32(W), ctx.from_i64(Y)]
    st_a, st_o = seed_transcript(zkh, "iso")
    st_b = zkh.transcript("iso2")
    with pytest.raises(zkh.ZkhError) as e:
        ctx.mm_prove_batch([(st_a, *ta, 8, 16, 4), (st_b, *tb, 8, 16, 4)])
    assert e.value.code == zkh.EROUND
    rc, _ = C.mm_prove(st_o, *good, 8, 16, 4)
    assert bytes(st_a) == bytes(st_o)  # the good job completed normally


def test_mm_wrong_witness_rejected(zkh, ctx):
    X, W, Y = _mm_inputs((8, 16, 4), 5)
    Y = Y.copy()
    Y[3, 2] += 1
    st = zkh.transcript("bad")
    with pytest.raises(zkh.ZkhError) as e:
        ctx.mm_prove(st, ctx.from_i32(X), ctx.from_i32(W), ctx.from_i64(Y), 8, 16, 4)
    assert e.value.code == zkh.EROUND


def _mm_check_batch(zkh, ctx, shapes, tag):
    items, wants, sts, keep = [], [], [], []
    for idx, shape in enumerate(shapes):
        B, IN, OUT = shape
        X, W, Y = _mm_inputs(shape, 300 + idx)
        st_g, st_o = seed_transcript(zkh, "%s:%d" % (tag, idx))
        rc, want = C.mm_prove(st_o, X, W, Y, B, IN, OUT)
        assert rc == 0
        t = (ctx.from_i32(X), ctx.from_i32(W), ctx.from_i64(Y))
        keep.append(t)
        items.append((st_g, t[0], t[1], t[2], B, IN, OUT))
        wants.append(want)
        sts.append((st_g, st_o))
    outs, status = ctx.mm_prove_batch(items)
    assert status == [0] * len(items)
    for got, want, (st_g, st_o) in zip(outs, wants, sts):
        for key in ("ev", "claims", "u_batch", "u_output", "u_input"):
            assert fr_eq(got[key], want[key]), key
        assert bytes(st_g) == bytes(st_o)


@pytest.mark.parametrize("shape", [(2, 40000, 3),   # 2^16 entries: 128 blocks in LDS
                                   (2, 70000, 2)])  # 2^17: beyond LDS, one launch per round
def test_mm_prove_large_in(zkh, ctx, shape):
    _mm_check_batch(zkh, ctx, [shape], "large")


def test_mm_prove_batch_several_launch_groups(zkh, ctx):
    """3 x 128 + 4 blocks exceed one 256-block launch: the jobs run in two groups."""
    _mm_check_batch(zkh, ctx, [(2, 40000, 2), (3, 2048, 4), (2, 33000, 2), (1, 60000, 1)], "groups")


def test_mm_prove_per_round_launch_path(zkh, ctx, monkeypatch):
    """The one-launch-per-round path (used beyond the LDS sizes), forced for small shapes."""
    monkeypatch.setenv("ZKH_NO_PERSIST", "1")
    _mm_check_batch(zkh, ctx, [(4, 8, 4), (1, 1, 1), (33, 700, 129), (8, 2048, 8)], "perround")


# Wide integer operands: the eq-weighted reductions switch from one 20-bit piece per int32
# (|v| < 2^19) and two 22-bit pieces per int64 (|Y| < 2^43) to two / three 22-bit pieces.
# Each case names which operands take the wide layout.
def _wide_inputs(case, B, IN, OUT, seed):
    rng = np.random.default_rng(seed)
    if case == "all":  # X, W near +-2^24, |Y| ~ 2^54: every reduction wide
        X = rng.integers(-2**24, 2**24, size=(B, IN), dtype=np.int64)
        W = rng.integers(-2**24, 2**24, size=(IN, OUT), dtype=np.int64)
        X[0, :] = 2**24 - 1
        W[:, 0] = -(2**24 - 1)
    elif case == "y":  # X, W narrow (|v| < 2^19) but |Y| >= 2^43
        X = rng.integers(-(2**19 - 1), 2**19, size=(B, IN), dtype=np.int64)
        W = rng.integers(-(2**19 - 1), 2**19, size=(IN, OUT), dtype=np.int64)
        X[0, :] = 2**19 - 1
        W[:, 0] = 2**19 - 1
    else:  # "x": only X wide (int32 needing 2 pieces), W and Y narrow
        X = rng.integers(-2**19, 2**19, size=(B, IN), dtype=np.int64)
        X[1, 2] = -(2**30)
        W = rng.integers(-2, 3, size=(IN, OUT), dtype=np.int64)
    Y = X @ W  # exact int64 (|Y| < 2^63)
    return X.astype(np.int32), W.astype(np.int32), Y


WIDE_CASES = [("all", (8, 64, 16)), ("all", (3, 100, 5)), ("y", (4, 64, 8)), ("y", (33, 128, 7)),
              ("x", (5, 40, 6))]


@pytest.mark.parametrize("case,shape", WIDE_CASES)
@pytest.mark.parametrize("weights", [True, False])
def test_mm_prove_wide(zkh, ctx, case, shape, weights):
    B, IN, OUT = shape
    X, W, Y = _wide_inputs(case, B, IN, OUT, B * 7 + IN + OUT)
    if case == "y":
        assert np.abs(Y).max() >= 2**43 and np.abs(X).max() < 2**19 and np.abs(W).max() < 2**19
    st_g, st_o = seed_transcript(zkh, "wide:%s:%d:%d:%d" % ((case,) + shape))
    rc, want = C.mm_prove(st_o, X, W, Y, B, IN, OUT)
    assert rc == 0
    Wt = ctx.weights_i32(W, IN, OUT) if weights else ctx.from_i32(W)
    got = ctx.mm_prove(st_g, ctx.from_i32(X), Wt, ctx.from_i64(Y), B, IN, OUT)
    for key in ("ev", "claims", "u_batch", "u_output", "u_input"):
        assert fr_eq(got[key], want[key]), key
    assert bytes(st_g) == bytes(st_o)


def test_mm_prove_batch_mixed_widths(zkh, ctx):
    """Narrow and wide jobs in one batch: two eqdot launch groups in one call."""
    items, wants, sts, keep = [], [], [], []
    for idx, (case, shape) in enumerate(WIDE_CASES + [("narrow", (16, 12, 5)), ("narrow", (64, 128, 64))]):
        B, IN, OUT = shape
        if case == "narrow":
            X, W, Y = _mm_inputs(shape, 900 + idx)
        else:
            X, W, Y = _wide_inputs(case, B, IN, OUT, 900 + idx)
        st_g, st_o = seed_transcript(zkh, "mixed:%d" % idx)
        rc, want = C.mm_prove(st_o, X, W, Y, B, IN, OUT)
        assert rc == 0
        t = (ctx.from_i32(X), ctx.weights_i32(W, IN, OUT) if idx % 2 else ctx.from_i32(W), ctx.from_i64(Y))
        keep.append(t)
        items.append((st_g, t[0], t[1], t[2], B, IN, OUT))
        wants.append(want)
        sts.append((st_g, st_o))
    outs, status = ctx.mm_prove_batch(items)
    assert status == [0] * len(items)
    for got, want, (st_g, st_o) in zip(outs, wants, sts):
        for key in ("ev", "claims", "u_batch", "u_output", "u_input"):
            assert fr_eq(got[key], want[key]), key
        assert bytes(st_g) == bytes(st_o)


# Field-element operands: the FrTensors zkob_fc binds (zkob_fc.cu:276-277, :337-338).
FR_SHAPES = [(4, 8, 4), (3, 5, 7), (1, 1, 1), (5, 1, 3), (16, 12, 5), (64, 128, 64), (33, 700, 129),
             (128, 3000, 64), (2, 40000, 3)]


def _fr_inputs(shape, seed):
    B, IN, OUT = shape
    rng = np.random.default_rng(seed)
    X = rand_fr_full(rng, B * IN)
    W = rand_fr_full(rng, IN * OUT)
    rc, Y = C.matmul_fr(X, W, B, IN, OUT)
    assert rc == 0
    return X, W, Y


@pytest.mark.parametrize("shape", FR_SHAPES)
def test_mm_prove_fr(zkh, ctx, shape):
    B, IN, OUT = shape
    X, W, Y = _fr_inputs(shape, sum(shape) + 5)
    st_g, st_o = seed_transcript(zkh, "mmfr:%d:%d:%d" % shape)
    rc, want = C.mm_prove_fr(st_o, X, W, Y, B, IN, OUT)
    assert rc == 0
    got = ctx.mm_prove(st_g, ctx.from_fr(X), ctx.from_fr(W), ctx.from_fr(Y), B, IN, OUT)
    for key in ("ev", "claims", "u_batch", "u_output", "u_input"):
        assert fr_eq(got[key], want[key]), key
    assert bytes(st_g) == bytes(st_o)


@pytest.mark.parametrize("kinds", ["fii", "ifi", "iif", "ffi", "fif", "iff"])
def test_mm_prove_mixed_kinds(zkh, ctx, kinds):
    """Each of X, W, Y as an integer tensor (f: field-element tensor of the same values)."""
    shape = (33, 700, 129)
    B, IN, OUT = shape
    X, W, Y = _mm_inputs(shape, 4242)
    st_g, st_o = seed_transcript(zkh, "mixed-kinds:" + kinds)
    rc, want = C.mm_prove(st_o, X, W, Y, B, IN, OUT)
    assert rc == 0
    tX = ctx.from_fr(C.ints_to_fr(X.ravel())) if kinds[0] == "f" else ctx.from_i32(X)
    tW = ctx.from_fr(C.ints_to_fr(W.ravel())) if kinds[1] == "f" else ctx.weights_i32(W, IN, OUT)
    tY = ctx.from_fr(C.ints_to_fr(Y.ravel())) if kinds[2] == "f" else ctx.from_i64(Y)
    got = ctx.mm_prove(st_g, tX, tW, tY, B, IN, OUT)
    for key in ("ev", "claims", "u_batch", "u_output", "u_input"):
        assert fr_eq(got[key], want[key]), key
    assert bytes(st_g) == bytes(st_o)


def test_mm_prove_fr_batch_with_int_jobs(zkh, ctx):
    items, wants, sts, keep = [], [], [], []
    for idx, shape in enumerate(FR_SHAPES[:7]):
        B, IN, OUT = shape
        st_g, st_o = seed_transcript(zkh, "frbatch:%d" % idx)
        if idx % 2:
            X, W, Y = _mm_inputs(shape, 500 + idx)
            rc, want = C.mm_prove(st_o, X, W, Y, B, IN, OUT)
            t = (ctx.from_i32(X), ctx.weights_i32(W, IN, OUT), ctx.from_i64(Y))
        else:
            X, W, Y = _fr_inputs(shape, 500 + idx)
            rc, want = C.mm_prove_fr(st_o, X, W, Y, B, IN, OUT)
            t = (ctx.from_fr(X), ctx.from_fr(W), ctx.from_fr(Y))
        assert rc == 0
        keep.append(t)
        items.append((st_g, t[0], t[1], t[2], B, IN, OUT))
        wants.append(want)
        sts.append((st_g, st_o))
    outs, status = ctx.mm_prove_batch(items)
    assert status == [0] * len(items)
    for got, want, (st_g, st_o) in zip(outs, wants, sts):
        for key in ("ev", "claims", "u_batch", "u_output", "u_input"):
            assert fr_eq(got[key], want[key]), key
        assert bytes(st_g) == bytes(st_o)


def test_mm_prove_fr_wrong_witness(zkh, ctx):
    X, W, Y = _fr_inputs((8, 16, 4), 77)
    Y = Y.copy()
    Y[5] = C.fr_op("add", Y[5], C.ints_to_fr([1])[0])
    with pytest.raises(zkh.ZkhError) as e:
        ctx.mm_prove(zkh.transcript("frbad"), ctx.from_fr(X), ctx.from_fr(W), ctx.from_fr(Y), 8, 16, 4)
    assert e.value.code == zkh.EROUND


def test_mm_prove_fr_tinyllama_layer_equals_int_path(zkh, ctx):
    """The 7 TinyLlama matmuls with X, W, Y bound as field-element tensors: every proof equals
    the integer-input proof of the same values (which test_gpu_configs checks against the
    oracle at this size)."""
    from zkh_synth import CONFIGS, matmul_inputs, rng_for
    c = CONFIGS["C4"]
    B = c["B"]
    rng = rng_for(4)
    items_i, items_f, keep = [], [], []
    for name, IN, OUT in c["matmuls"]:
        X, W, Y = matmul_inputs(rng, B, IN, OUT)
        ti = (ctx.from_i32(X), ctx.weights_i32(W, IN, OUT), ctx.from_i64(Y))
        tf = (ctx.from_fr(C.ints_to_fr(X.ravel())), ctx.from_fr(C.ints_to_fr(W.ravel())),
              ctx.from_fr(C.ints_to_fr(Y.ravel())))
        keep += [ti, tf]
        items_i.append((zkh.transcript("frl:" + name), *ti, B, IN, OUT))
        items_f.append((zkh.transcript("frl:" + name), *tf, B, IN, OUT))
    outs_i, st_i = ctx.mm_prove_batch(items_i)
    outs_f, st_f = ctx.mm_prove_batch(items_f)
    assert st_i == [0] * 7 and st_f == [0] * 7
    for a, b, ia, ib in zip(outs_i, outs_f, items_i, items_f):
        for key in ("ev", "claims", "u_batch", "u_output", "u_input"):
            assert fr_eq(a[key], b[key]), key
        assert bytes(ia[0]) == bytes(ib[0])


# ---------------------------------------------------------------- logUp
LU_SHAPES = [(32, 8, -3, 5), (16, 16, 0, 16), (64, 4, -2, 3),  # vrf_toy_lookup.cu:323-335
             (32, 4, -2, 4), (64, 16, -8, 16), (48 * 0 + 64, 64, -32, 64),
             (1 << 12, 1 << 8, -128, 256), (1 << 14, 1 << 14, -(1 << 13), 1 << 14)]


@pytest.mark.parametrize("shape", LU_SHAPES)
def test_lu_prove(zkh, ctx, shape):
    D, N, low, ln = shape
    rng = np.random.default_rng(D + N)
    vals = rng.integers(low, low + ln, size=D).astype(np.int32)
    S = C.ints_to_fr(vals)
    T = C.range_table(low, ln, N)
    st_g, st_o = seed_transcript(zkh, "lu:%d:%d" % (D, N))
    rc, m = C.lu_prep(S, low, N)
    assert rc == 0
    Sg = ctx.from_i32(vals)
    mg = ctx.lu_prep(Sg, low, N)
    assert fr_eq(mg.to_fr(), m)
    Tg = ctx.range_table(low, ln, N)
    assert fr_eq(Tg.to_fr(), T)
    beta = C.tr_challenge_fr(st_o)
    assert fr_eq(zkh.challenge(st_g), beta)
    A = C.lu_inverse(S, beta)
    Ag = ctx.lu_inverse(Sg, beta)
    assert fr_eq(Ag.to_fr(), A)
    alpha = C.tr_challenge_fr(st_o)
    assert fr_eq(zkh.challenge(st_g), alpha)
    logD = P.ceil_log2(D)
    u = np.array([C.tr_challenge_fr(st_o) for _ in range(logD)])
    ug = np.array([zkh.challenge(st_g) for _ in range(logD)])
    assert fr_eq(u, ug)
    st_g2 = st_g.copy()
    rc, want = C.lu_prove(st_o, A, S, T, m, alpha, beta, u)
    assert rc == 0
    # FR-kind witness (not the int view) must give the same proof
    got = ctx.lu_prove(st_g, Ag, ctx.from_fr(S), Tg, mg, alpha, beta, u)
    for key in ("ev", "term", "ws"):
        assert fr_eq(got[key], want[key]), key
    assert bytes(st_g) == bytes(st_o)
    # with the tensor that zkh_lu_inverse inverted, the first round takes A (S + beta) = 1
    # (the closed-form sums) and must give the same proof
    got = ctx.lu_prove(st_g2, Ag, Sg, Tg, mg, alpha, beta, u)
    for key in ("ev", "term", "ws"):
        assert fr_eq(got[key], want[key]), ("closed form", key)
    assert bytes(st_g2) == bytes(st_o)


@pytest.mark.parametrize("D,N,zeros", [(1 << 16, 1 << 16, ()), (1 << 16, 1 << 12, ()),
                                        (1 << 16, 1 << 16, (14, 13)), (1 << 16, 1 << 12, (15, 11, 3))])
def test_lu_prove_derived_rounds(zkh, ctx, D, N, zeros):
    """Tables above the persistent loop's size: the folding rounds leave their sums at 1 to the
    pieces' claims (phase 1, the phase-1 -> 2 round, phase 2).  Coordinates of u set to 0 make
    those rounds compute every sum instead.  Proofs and terminals equal the oracle's."""
    low, ln = -(N // 2), N
    rng = np.random.default_rng(D + N + len(zeros))
    vals = rng.integers(low, low + ln, size=D).astype(np.int32)
    S = C.ints_to_fr(vals)
    T = C.range_table(low, ln, N)
    rc, m = C.lu_prep(S, low, N)
    assert rc == 0
    beta, alpha = rand_fr_full(rng, 2)
    logD = P.ceil_log2(D)
    u = rand_fr_full(rng, logD)
    for z in zeros:
        u[z] = 0
    A = C.lu_inverse(S, beta)
    st_g, st_o = seed_transcript(zkh, "lud:%d:%d:%d" % (D, N, len(zeros)))
    rc, want = C.lu_prove(st_o, A, S, T, m, alpha, beta, u)
    assert rc == 0
    Sg = ctx.from_i32(vals)
    got = ctx.lu_prove(st_g, ctx.lu_inverse(Sg, beta), Sg, ctx.range_table(low, ln, N), ctx.from_fr(m),
                       alpha, beta, u)
    for key in ("ev", "term", "ws"):
        assert fr_eq(got[key], want[key]), key
    assert bytes(st_g) == bytes(st_o)


@pytest.mark.parametrize("D,N,skew", [(1000, 64, 0), (70000, 16384, 1), (1 << 17, 40000, 1), (1 << 17, 40000, 0),
                                       (300000, 1 << 16, 1), (1 << 18, 1 << 24, 1)])
def test_lu_prep_histogram(zkh, ctx, D, N, skew):
    """Multiplicities against brute-force counting, through the LDS histogram's direct mode
    (N <= 16384) and its partitioned mode (several buckets, a partial last bucket, up to the
    1024-bucket maximum), with a skewed witness (a quarter of the entries on one index, as
    zero padding makes) and FR-kind witnesses."""
    rng = np.random.default_rng(D + N)
    low = -(N // 2)
    vals = rng.integers(low, low + N, size=D).astype(np.int32)
    if skew:
        vals[: D // 4] = 0
    want = np.bincount((vals.astype(np.int64) - low), minlength=N)
    got = ctx.lu_prep(ctx.from_i32(vals), low, N).to_fr()
    assert np.array_equal(got[:, 0], want.astype(np.uint32)) and not got[:, 1:].any()
    if D <= (1 << 17):
        got_fr = ctx.lu_prep(ctx.from_fr(C.ints_to_fr(vals)), low, N).to_fr()
        assert fr_eq(got_fr, got)


@pytest.mark.parametrize("N", [64, 40000])
def test_lu_prep_out_of_range_partitioned(zkh, ctx, N):
    vals = np.zeros(50000, np.int32)
    vals[4321] = N  # low = 0: index N is one past the table
    with pytest.raises(zkh.ZkhError) as e:
        ctx.lu_prep(ctx.from_i32(vals), 0, N)
    assert e.value.code == zkh.EARG
    # limb 0 of r - 2 (the field image of -2) is 2^32 - 1: outside; -1 (limb 0 of r - 1 is
    # 0) aliases into bin 0 as the reference's limb-0 index does (tlookup.cu:419)
    vals[4321] = -2
    with pytest.raises(zkh.ZkhError):
        ctx.lu_prep(ctx.from_i32(vals), 0, N)
    vals[4321] = -1
    got = ctx.lu_prep(ctx.from_i32(vals), 0, N).to_fr()
    assert got[0, 0] == 50000 and not got[1:].any()


def test_lu_out_of_range_rejected(zkh, ctx):
    S = ctx.from_i32(np.array([0, 1, 2, 40], np.int32))
    with pytest.raises(zkh.ZkhError) as e:
        ctx.lu_prep(S, 0, 16)
    assert e.value.code == zkh.EARG


def test_lu_inverse_zero(zkh, ctx):
    rng = np.random.default_rng(3)
    S = rand_fr_full(rng, 5000)
    beta = C.fr_op("sub", np.zeros(8, np.uint32), S[1234])  # S[1234] + beta = 0
    want = C.lu_inverse(S, beta)
    assert not want[1234].any()
    got = ctx.lu_inverse(ctx.from_fr(S), beta).to_fr()
    assert fr_eq(got, want)


@pytest.mark.parametrize("D,N", [(1 << 15, 1 << 15), (1 << 16, 1 << 14)])
def test_lu_prove_zero_inverse(zkh, ctx, D, N):
    """beta = -(a table value v): A and B have zero entries (inverse of zero is zero), so
    a (s + beta) = 0 where S = v and the first round may not take sum eq a (s + beta) = 1;
    the logUp relation then fails and, as in the oracle, the proof stops at its first
    round's consistency check.  With a random beta (no zero) the same tensors prove and
    equal the oracle's proof (phase 2 alone, and phase 1 first)."""
    low = -(N // 2)
    rng = np.random.default_rng(D + 3 * N)
    vals = rng.integers(low, low + N, size=D).astype(np.int32)
    v = int(vals[7])
    S = C.ints_to_fr(vals)
    T = C.range_table(low, N, N)
    rc, m = C.lu_prep(S, low, N)
    assert rc == 0
    alpha = rand_fr_full(rng, 1)[0]
    u = rand_fr_full(rng, P.ceil_log2(D))
    Sg, Tg = ctx.from_i32(vals), ctx.range_table(low, N, N)
    mg = ctx.lu_prep(Sg, low, N)
    for shift in (0, 1):
        beta = C.ints_to_fr([-v % P.R])[0] if not shift else rand_fr_full(rng, 1)[0]
        A = C.lu_inverse(S, beta)
        assert A[7].any() == bool(shift)
        st_g, st_o = seed_transcript(zkh, "luz:%d:%d:%d" % (D, N, shift))
        rc, want = C.lu_prove(st_o, A, S, T, m, alpha, beta, u)
        Ag = ctx.lu_inverse(Sg, beta)
        if not shift:
            assert rc != 0
            with pytest.raises(zkh.ZkhError) as e:
                ctx.lu_prove(st_g, Ag, Sg, Tg, mg, alpha, beta, u)
            assert e.value.code == zkh.EROUND and "round 0" in str(e.value)
            # the same through the range gather (A read off the table inverse)
            Ar = ctx.lu_range_inverse(Sg, low, Tg, beta)
            with pytest.raises(zkh.ZkhError) as e:
                ctx.lu_prove(seed_transcript(zkh, "luz")[0], Ar, Sg, Tg, mg, alpha, beta, u)
            assert e.value.code == zkh.EROUND and "round 0" in str(e.value)
        else:
            assert rc == 0
            got = ctx.lu_prove(st_g, Ag, Sg, Tg, mg, alpha, beta, u)
            for key in ("ev", "term", "ws"):
                assert fr_eq(got[key], want[key]), key
            assert bytes(st_g) == bytes(st_o)


def test_lu_mapping(zkh, ctx):
    rng = np.random.default_rng(9)
    low, N = -16, 32
    mapped_vals = rng.integers(-1000, 1000, size=N)
    vals = rng.integers(low, low + N, size=256).astype(np.int32)
    Sout, m = ctx.lu_mapping(ctx.from_i32(vals), low, ctx.from_fr(C.ints_to_fr(mapped_vals)))
    want = C.ints_to_fr([int(mapped_vals[v - low]) for v in vals])
    assert fr_eq(Sout.to_fr(), want)
    rc, mw = C.lu_prep(C.ints_to_fr(vals), low, N)
    assert fr_eq(m.to_fr(), mw)


@pytest.mark.parametrize("n", [3 * (1 << 20) + 17, 1 << 21, (1 << 23) + 3])
def test_lu_inverse_sizes(zkh, ctx, n):
    """Batched inversion at sizes whose block products take the one-block stage's register
    path (up to 8 per thread, a partial last group) and its loop path (more than 8):
    A (S + beta) = 1 on every entry, against the oracle, with one entry S = -beta (inverse
    of zero is zero)."""
    rng = np.random.default_rng(n)
    S = rng.integers(0, 2**32, size=(n, 8), dtype=np.uint64).astype(np.uint32)
    S[:, 7] %= 0x73EDA753  # below r
    beta = rand_fr_full(rng, 1)[0]
    S[5] = C.ints_to_fr([(P.R - C.fr_to_ints(beta.reshape(1, 8))[0]) % P.R])[0]
    A = ctx.lu_inverse(ctx.from_fr(S), beta).to_fr()
    assert C.check_inverse(S, A, beta) == 0
    assert not np.asarray(A).reshape(-1, 8)[5].any()


def tuple_case(D, N, ln, seed):
    """A SwiGLU-style tuple lookup: witness G in the table's domain with zero padding in its
    last eighth, a mapped table with int32 extremes, and where the table is padded (ln < N)
    a few witnesses past ln, whose table entry (low + ln - 1) is not the witness."""
    rng = np.random.default_rng(seed)
    low = -(N // 2)
    mapped = rng.integers(-2**31, 2**31, size=N, dtype=np.int64)
    mapped[:4] = [2**31 - 1, -2**31, -1, 0]
    mapped[-low] = 0
    mapped = mapped.astype(np.int32)
    G = rng.integers(low, low + min(ln, N), size=D).astype(np.int32)
    G[-(D // 8):] = 0
    if ln < N:
        G[:7] = low + ln + np.arange(7) % (N - ln)
    r, beta = rand_fr_full(rng, 2)
    # the reference's steps on the oracle (zkob_glu.cu:155-160, :168-170)
    S = C.ints_to_fr([int(mapped[g - low]) for g in G])
    comb = C.axpy(C.ints_to_fr([int(g) for g in G]), r, S)
    Tcomb = C.axpy(C.range_table(low, ln, N), r, C.ints_to_fr([int(v) for v in mapped]))
    return dict(low=low, mapped=mapped, G=G, r=r, beta=beta, comb=comb, Tcomb=Tcomb)


@pytest.mark.parametrize("D,N,ln,gkind", [(4096, 4096, 4096, "i32"), (1 << 14, 1 << 12, 1 << 12, "fr"),
                                           (4096, 1024, 1000, "i32"), (4096, 1024, 1000, "fr"),
                                           (1 << 20, 1 << 18, 1 << 18, "i32")])
def test_lu_tuple_inverse(zkh, ctx, D, N, ln, gkind):
    """comb = G + r mapped[G - low], T_comb = T + r mapped and A = 1/(comb + beta) in one call
    equal the reference's separate steps on the oracle: A read off the table inverse (every
    G[i] the table's entry at its index), or, with a padded table and witnesses past ln, by
    the direct inversion of comb; int32- and field-kind witnesses.  A is also checked against
    the definition (A (comb + beta) = 1)."""
    t = tuple_case(D, N, ln, D + N + ln)
    G = ctx.from_i32(t["G"]) if gkind == "i32" else ctx.from_fr(C.ints_to_fr([int(g) for g in t["G"]]))
    mapped = ctx.from_i32(t["mapped"])
    S, _ = ctx.lu_mapping(G, t["low"], mapped)
    for s_in in (None, S):  # comb from mapped[j], or from the mapping's S read in order
        comb, Tcomb, A = ctx.lu_tuple_inverse(G, t["low"], ctx.range_table(t["low"], ln, N), mapped, t["r"], t["beta"],
                                              S=s_in)
        assert fr_eq(comb.to_fr(), t["comb"])
        assert fr_eq(Tcomb.to_fr(), t["Tcomb"])
        got = A.to_fr()
        assert C.check_inverse(t["comb"], got, t["beta"]) == 0
        if D <= 1 << 14:
            assert fr_eq(got, C.lu_inverse(t["comb"], t["beta"]))


def test_lu_tuple_inverse_rejects_other_s(zkh, ctx):
    """S must be zkh_lu_mapping's output for the same G, low and mapped."""
    t = tuple_case(4096, 1024, 1024, 77)
    G, mapped = ctx.from_i32(t["G"]), ctx.from_i32(t["mapped"])
    T = ctx.range_table(t["low"], 1024, 1024)
    S, _ = ctx.lu_mapping(G, t["low"], mapped)
    G2 = ctx.from_i32(t["G"])  # same values, another tensor
    for args in ((G2, t["low"], S), (G, t["low"] + 1, S), (G, t["low"], ctx.from_i32(np.zeros(4096, np.int32)))):
        with pytest.raises(zkh.ZkhError) as e:
            ctx.lu_tuple_inverse(args[0], args[1], T, mapped, t["r"], t["beta"], S=args[2])
        assert e.value.code == zkh.EARG


@pytest.mark.parametrize("D,N", [(1 << 16, 1 << 16), (1 << 16, 1 << 14)])
def test_lu_prove_takes_table_inverse(zkh, ctx, D, N):
    """The SwiGLU lookup through zkh_lu_tuple_inverse: the proof that takes its table inverse
    over equals the oracle's from the separate steps; a second proof on the same tensors (the
    table inverse then folded and gone) inverts T_comb itself and equals it too."""
    t = tuple_case(D, N, N, D * 3 + N)
    rng = np.random.default_rng(D + 5 * N)
    alpha = rand_fr_full(rng, 1)
    u = rand_fr_full(rng, P.ceil_log2(D))
    rc, m = C.lu_prep(C.ints_to_fr([int(g) for g in t["G"]]), t["low"], N)
    assert rc == 0
    A_o = C.lu_inverse(t["comb"], t["beta"])
    Gg = ctx.from_i32(t["G"])
    _, mg = ctx.lu_mapping(Gg, t["low"], ctx.from_i32(t["mapped"]))
    assert fr_eq(mg.to_fr(), m)
    comb, Tcomb, A = ctx.lu_tuple_inverse(Gg, t["low"], ctx.range_table(t["low"], N, N), ctx.from_i32(t["mapped"]),
                                          t["r"], t["beta"])
    for k in range(2):
        st_g, st_o = seed_transcript(zkh, "lut:%d:%d:%d" % (D, N, k))
        rc, want = C.lu_prove(st_o, A_o, t["comb"], t["Tcomb"], m, alpha, t["beta"], u)
        assert rc == 0
        got = ctx.lu_prove(st_g, A, comb, Tcomb, mg, alpha, t["beta"], u)
        for key in ("ev", "term", "ws"):
            assert fr_eq(got[key], want[key]), (k, key)
        assert bytes(st_g) == bytes(st_o)


@pytest.mark.parametrize("D,N,ln,skind", [(1 << 16, 1 << 12, 1 << 12, "i32"), (1 << 14, 1 << 12, 3000, "fr"),
                                           (1 << 14, 1 << 12, 3000, "i32"), (4096, 4096, 4096, "fr")])
def test_lu_range_inverse(zkh, ctx, D, N, ln, skind):
    """zkh_lu_range_inverse's A (read off the table inverse) equals zkh_lu_inverse's and the
    oracle's 1/(S + beta): witnesses in the table's domain with zero padding, and with a padded
    table (ln < N) witnesses past ln and one outside the domain (the direct inversion);
    int32- and field-kind witnesses."""
    rng = np.random.default_rng(D + N + ln)
    low = -(N // 2)
    vals = rng.integers(low, low + ln, size=D).astype(np.int64)
    vals[-(D // 8):] = 0
    if ln < N:
        vals[:5] = low + ln + np.arange(5) % (N - ln)
        vals[5] = low + N + 7
    ints = [int(v) for v in vals]
    beta = rand_fr_full(rng, 1)[0]
    S = ctx.from_i32(vals.astype(np.int32)) if skind == "i32" else ctx.from_fr(C.ints_to_fr(ints))
    want = C.lu_inverse(C.ints_to_fr(ints), beta)
    assert fr_eq(ctx.lu_range_inverse(S, low, ctx.range_table(low, ln, N), beta).to_fr(), want)
    assert fr_eq(ctx.lu_inverse(S, beta).to_fr(), want)


@pytest.mark.parametrize("D,N", [(1 << 16, 1 << 12), (1 << 15, 1 << 15)])
def test_lu_prove_takes_range_table_inverse(zkh, ctx, D, N):
    """The rescale lookup through zkh_lu_range_inverse (phase 1 and phase 2, and phase 2
    alone): the proof that takes the table inverse over, and a second proof on the same
    tensors, equal the oracle's."""
    low = -(N // 2)
    rng = np.random.default_rng(7 * D + N)
    vals = rng.integers(low, low + N, size=D).astype(np.int32)
    Sf = C.ints_to_fr([int(v) for v in vals])
    rc, m = C.lu_prep(Sf, low, N)
    assert rc == 0
    beta, alpha = rand_fr_full(rng, 2)
    u = rand_fr_full(rng, P.ceil_log2(D))
    A_o = C.lu_inverse(Sf, beta)
    Sg, Tg = ctx.from_i32(vals), ctx.range_table(low, N, N)
    A, mg = ctx.lu_range_inverse(Sg, low, Tg, beta), ctx.from_fr(m)
    for k in range(2):
        st_g, st_o = seed_transcript(zkh, "lur:%d:%d:%d" % (D, N, k))
        rc, want = C.lu_prove(st_o, A_o, Sf, C.range_table(low, N, N), m, alpha, beta, u)
        assert rc == 0
        got = ctx.lu_prove(st_g, A, Sg, Tg, mg, alpha, beta, u)
        for key in ("ev", "term", "ws"):
            assert fr_eq(got[key], want[key]), (k, key)
        assert bytes(st_g) == bytes(st_o)


def test_lu_tuple_inverse_out_of_range(zkh, ctx):
    """A witness outside the table's domain fails as zkh_lu_mapping does."""
    low, N = -8, 16
    G = np.array([0, 3, low + N, -2], np.int32)
    with pytest.raises(zkh.ZkhError) as e:
        ctx.lu_tuple_inverse(ctx.from_i32(G), low, ctx.range_table(low, N, N), ctx.from_i32(np.zeros(N, np.int32)),
                             C.ints_to_fr([5]), C.ints_to_fr([7]))
    assert e.value.code == zkh.EARG


@pytest.mark.parametrize("gkind", ["i32", "fr"])
def test_range_inverses_table_past_int32_max(zkh, ctx, gkind):
    """A range table whose entries wrap past 2^31 - 1 (low + j computed in 32-bit int, as
    tlookup.cu:376 builds it): witnesses low + j are the table's entry only below the wrap.
    A field-kind witness above 2^31 - 1 is no table entry, so its A must be its own inverse
    1/(G + beta) (the direct inversion), for both gathers; int32 witnesses cover the entries
    below the wrap."""
    N = 64
    low = 2**31 - 1 - 40  # entries j <= 40 are low + j, j >= 41 wrap to negative values
    js = np.array(list(range(N)) * 3, np.int64)
    rng = np.random.default_rng(41)
    rng.shuffle(js)
    if gkind == "i32":
        js = js[js <= 40]
    vals = [low + int(j) for j in js]  # the true integers, past 2^31 - 1 for j > 40
    D = len(vals)
    beta, r = rand_fr_full(rng, 2)
    mapped = rng.integers(-2**20, 2**20, size=N).astype(np.int32)
    Gf = C.ints_to_fr(vals)
    G = ctx.from_i32(np.array(vals, np.int64).astype(np.int32)) if gkind == "i32" else ctx.from_fr(Gf)
    T = ctx.range_table(low, N, N)
    T_o = C.range_table(low, N, N)
    assert fr_eq(T.to_fr(), T_o)
    # plain range lookup: A = 1/(G + beta)
    want = C.lu_inverse(Gf, beta)
    assert fr_eq(ctx.lu_range_inverse(G, low, T, beta).to_fr(), want)
    # SwiGLU combiner: comb = G + r mapped[(G - low).limb0], A = 1/(comb + beta)
    S_o = C.ints_to_fr([int(mapped[int(j)]) for j in js])
    comb_o = C.axpy(Gf, r, S_o)
    comb, Tcomb, A = ctx.lu_tuple_inverse(G, low, T, ctx.from_i32(mapped), r, beta)
    assert fr_eq(comb.to_fr(), comb_o)
    assert fr_eq(Tcomb.to_fr(), C.axpy(T_o, r, C.ints_to_fr(mapped)))
    assert fr_eq(A.to_fr(), C.lu_inverse(comb_o, beta))


# ---------------------------------------------------------------- elementwise with int32 operands
def test_hadamard_axpy_int32_edges(zkh, ctx):
    """Elementwise products and axpy with int32 operands take the 32-bit multiply (quotient
    estimated in double precision, one correction): every kind pairing against the field
    definition, with field values 0, 1, r-1, r-2, (r-1)/2 and random ones against int32
    values 0, +-1, +-2^30, -2^31, 2^31-1 and random ones, plus a long random tail that goes
    through the grid-stride loops."""
    rng = np.random.default_rng(7)
    fv = [0, 1, P.R - 1, P.R - 2, (P.R - 1) // 2] + [int.from_bytes(rng.bytes(32), "little") % P.R for _ in range(27)]
    iv = [0, 1, -1, 2**30, -2**30, -2**31, 2**31 - 1] + [int(x) for x in rng.integers(-2**31, 2**31, size=25)]
    F = [f for f in fv for _ in iv] + [int.from_bytes(rng.bytes(32), "little") % P.R for _ in range(70000)]
    I = [i for _ in fv for i in iv] + [int(x) for x in rng.integers(-2**31, 2**31, size=70000)]
    I2 = I[1:] + I[:1]
    A, B, B2 = ctx.from_fr(C.ints_to_fr(F)), ctx.from_i32(np.array(I, np.int32)), ctx.from_i32(np.array(I2, np.int32))
    ints = lambda t: C.fr_to_ints(t.to_fr())
    assert ints(ctx.hadamard(A, B)) == [f * i % P.R for f, i in zip(F, I)]
    assert ints(ctx.hadamard(B, A)) == [f * i % P.R for f, i in zip(F, I)]
    assert ints(ctx.hadamard(B2, B)) == [i * j % P.R for i, j in zip(I2, I)]
    for c in (0, 1, P.R - 1, int.from_bytes(rng.bytes(32), "little") % P.R):
        cf = C.ints_to_fr([c])[0]
        assert ints(ctx.axpy(A, cf, B)) == [(f + c * i) % P.R for f, i in zip(F, I)], c
        assert ints(ctx.axpy(B2, cf, B)) == [(j + c * i) % P.R for j, i in zip(I2, I)], c


# ---------------------------------------------------------------- Hadamard
@pytest.mark.parametrize("k", [1, 2, 5, 11, 13, 14])
def test_hp_prove(zkh, ctx, k):
    n = 1 << k
    rng = np.random.default_rng(k)
    u = rand_fr_full(rng, k)
    E = C.build_eq(u)
    S = C.ints_to_fr(rng.integers(-2**20, 2**20, size=n))
    U = rand_fr_full(rng, n)
    Ei, Si, Ui = C.fr_to_ints(E), C.fr_to_ints(S), C.fr_to_ints(U)
    claim = C.ints_to_fr([sum(a * b % P.R * c for a, b, c in zip(Ei, Si, Ui)) % P.R])[0]
    for eqform in (False, True):
        st_g, st_o = seed_transcript(zkh, "hp:%d" % k)
        rc, want = C.hp_prove(st_o, claim, E, S, U)
        assert rc == 0
        if eqform:
            got = ctx.hp_prove_eq(st_g, claim, u, ctx.from_fr(S), ctx.from_fr(U))
        else:
            got = ctx.hp_prove(st_g, claim, ctx.from_fr(E), ctx.from_fr(S), ctx.from_fr(U))
        for key in ("ev", "term", "ws"):
            assert fr_eq(got[key], want[key]), (key, eqform)
        assert bytes(st_g) == bytes(st_o)


def test_persistent_loops_queued_on_fresh_context(zkh):
    """The persistent loops are queued behind a relay while the round before them runs; on a
    fresh context their first use allocates the pinned slot memory, which waits for the
    stream, so the relay has to go in after that allocation.  A logUp proof whose loop starts
    after two round kernels (D = 32 > N = 8) and a Hadamard proof whose loop starts after one
    (2^14 entries), each on a new context, equal the oracle's."""
    rng = np.random.default_rng(77)
    D, N, low, ln = 32, 8, -3, 5
    vals = rng.integers(low, low + ln, size=D).astype(np.int32)
    S = C.ints_to_fr(vals)
    T = C.range_table(low, ln, N)
    rc, m = C.lu_prep(S, low, N)
    assert rc == 0
    beta, alpha = rand_fr_full(rng, 2)
    u = rand_fr_full(rng, P.ceil_log2(D))
    st_g, st_o = seed_transcript(zkh, "fresh:lu")
    rc, want = C.lu_prove(st_o, C.lu_inverse(S, beta), S, T, m, alpha, beta, u)
    assert rc == 0
    c1 = zkh.Context(0)
    try:
        Sg = c1.from_i32(vals)
        got = c1.lu_prove(st_g, c1.lu_inverse(Sg, beta), Sg, c1.range_table(low, ln, N), c1.from_fr(m), alpha,
                          beta, u)
    finally:
        c1.close()
    for key in ("ev", "term", "ws"):
        assert fr_eq(got[key], want[key]), key
    assert bytes(st_g) == bytes(st_o)
    k = 14
    n = 1 << k
    uh = rand_fr_full(rng, k)
    E = C.build_eq(uh)
    Sv, U = C.ints_to_fr(rng.integers(-2**20, 2**20, size=n)), rand_fr_full(rng, n)
    Ei, Si, Ui = C.fr_to_ints(E), C.fr_to_ints(Sv), C.fr_to_ints(U)
    claim = C.ints_to_fr([sum(a * b % P.R * c for a, b, c in zip(Ei, Si, Ui)) % P.R])[0]
    st_g, st_o = seed_transcript(zkh, "fresh:hp")
    rc, want = C.hp_prove(st_o, claim, E, Sv, U)
    assert rc == 0
    c2 = zkh.Context(0)
    try:
        got = c2.hp_prove_eq(st_g, claim, uh, c2.from_fr(Sv), c2.from_fr(U))
    finally:
        c2.close()
    for key in ("ev", "term", "ws"):
        assert fr_eq(got[key], want[key]), key
    assert bytes(st_g) == bytes(st_o)


@pytest.mark.parametrize("k,zeros", [(16, ()), (16, (14, 13)), (17, (15,))])
def test_hp_prove_derived_rounds(zkh, ctx, k, zeros):
    """Tables above the persistent loop's size (explicit E and eq form): the folding rounds leave
    their sum at 1 to the host (claim - p(0), or the inner claim of the eq form); a coordinate
    of u set to 0 makes the eq form's round compute all three sums.  Proofs equal the oracle's."""
    n = 1 << k
    rng = np.random.default_rng(300 + k + len(zeros))
    u = rand_fr_full(rng, k)
    for z in zeros:
        u[z] = 0
    E = C.build_eq(u)
    S = rand_fr_full(rng, n)
    U = rand_fr_full(rng, n)
    Ei, Si, Ui = C.fr_to_ints(E), C.fr_to_ints(S), C.fr_to_ints(U)
    claim = C.ints_to_fr([sum(a * b % P.R * c for a, b, c in zip(Ei, Si, Ui)) % P.R])[0]
    for eqform in (False, True):
        st_g, st_o = seed_transcript(zkh, "hpd:%d:%d" % (k, len(zeros)))
        rc, want = C.hp_prove(st_o, claim, E, S, U)
        assert rc == 0
        if eqform:
            got = ctx.hp_prove_eq(st_g, claim, u, ctx.from_fr(S), ctx.from_fr(U))
        else:
            got = ctx.hp_prove(st_g, claim, ctx.from_fr(E), ctx.from_fr(S), ctx.from_fr(U))
        for key in ("ev", "term", "ws"):
            assert fr_eq(got[key], want[key]), (key, eqform)
        assert bytes(st_g) == bytes(st_o)


@pytest.mark.parametrize("k", [3, 11])
def test_hp_prove_eq_wrong_claim_stops(zkh, ctx, k):
    """A claim off by one fails the first round inside the persistent round loop (eq and
    explicit-E forms): the call returns ZKH_EROUND (2), the blocks exit on the quit command,
    and the context stays usable (the next proof is bit-exact against the oracle)."""
    n = 1 << k
    rng = np.random.default_rng(100 + k)
    u = rand_fr_full(rng, k)
    S = C.ints_to_fr(rng.integers(-2**20, 2**20, size=n))
    U = rand_fr_full(rng, n)
    E = C.build_eq(u)
    Ei, Si, Ui = C.fr_to_ints(E), C.fr_to_ints(S), C.fr_to_ints(U)
    good = sum(a * b % P.R * c for a, b, c in zip(Ei, Si, Ui)) % P.R
    bad = C.ints_to_fr([(good + 1) % P.R])[0]
    for eqform in (True, False):
        st_g, _ = seed_transcript(zkh, "hpbad:%d" % k)
        with pytest.raises(zkh.ZkhError) as e:
            if eqform:
                ctx.hp_prove_eq(st_g, bad, u, ctx.from_fr(S), ctx.from_fr(U))
            else:
                ctx.hp_prove(st_g, bad, ctx.from_fr(E), ctx.from_fr(S), ctx.from_fr(U))
        assert e.value.code == 2
    st_g, st_o = seed_transcript(zkh, "hpgood:%d" % k)
    claim = C.ints_to_fr([good])[0]
    rc, want = C.hp_prove(st_o, claim, E, S, U)
    got = ctx.hp_prove_eq(st_g, claim, u, ctx.from_fr(S), ctx.from_fr(U))
    for key in ("ev", "term", "ws"):
        assert fr_eq(got[key], want[key]), key
    assert bytes(st_g) == bytes(st_o)


@pytest.mark.parametrize("mode", ["per_round", "one_round"])
def test_lu_hp_per_round_launch_path(zkh, ctx, mode, monkeypatch):
    """per_round: every round of the lookup and Hadamard sumchecks as its own launch (the
    persistent loops off): the folding rounds derive their sums at 1 down to 2-entry tables,
    the terminals come from the folded tables.  one_round: the persistent loops with one
    round per message, in both of their phases (the blocks' own rounds, then the block that
    gathers every block's entry).  The proofs equal the oracle's (phase 1 and 2, explicit E,
    eq form, U all ones over an int32 S)."""
    monkeypatch.setenv("ZKH_NO_PERSIST" if mode == "per_round" else "ZKH_PERSIST_ONE", "1")
    rng = np.random.default_rng(41)
    for D, N, low in [(1 << 10, 1 << 10, -512), (1 << 12, 1 << 8, -128)]:
        vals = rng.integers(low, low + N, size=D).astype(np.int32)
        S = C.ints_to_fr(vals)
        T = C.range_table(low, N, N)
        rc, m = C.lu_prep(S, low, N)
        assert rc == 0
        beta, alpha = rand_fr_full(rng, 2)
        u = rand_fr_full(rng, P.ceil_log2(D))
        st_g, st_o = seed_transcript(zkh, "lupr:%d:%d" % (D, N))
        rc, want = C.lu_prove(st_o, C.lu_inverse(S, beta), S, T, m, alpha, beta, u)
        assert rc == 0
        Sg = ctx.from_i32(vals)
        got = ctx.lu_prove(st_g, ctx.lu_inverse(Sg, beta), Sg, ctx.range_table(low, N, N), ctx.from_fr(m),
                           alpha, beta, u)
        for key in ("ev", "term", "ws"):
            assert fr_eq(got[key], want[key]), (D, N, key)
        assert bytes(st_g) == bytes(st_o)
    k = 11
    n = 1 << k
    u = rand_fr_full(rng, k)
    E = C.build_eq(u)
    Sv = rng.integers(-2**31, 2**31, size=n)
    S, U = C.ints_to_fr(Sv), rand_fr_full(rng, n)
    Ei, Si, Ui = C.fr_to_ints(E), C.fr_to_ints(S), C.fr_to_ints(U)
    claim = C.ints_to_fr([sum(a * b % P.R * c for a, b, c in zip(Ei, Si, Ui)) % P.R])[0]
    ones = np.ones(n, np.int64)
    claim1 = C.ints_to_fr([sum(a * b for a, b in zip(Ei, Si)) % P.R])[0]
    for form in ("E", "eq", "ones"):
        st_g, st_o = seed_transcript(zkh, "hppr:" + form)
        if form == "ones":
            rc, want = C.hp_prove(st_o, claim1, E, S, C.ints_to_fr(ones))
            got = ctx.hp_prove(st_g, claim1, ctx.from_fr(E), ctx.from_i32(Sv.astype(np.int32)),
                               ctx.from_i32(ones.astype(np.int32)))
        else:
            rc, want = C.hp_prove(st_o, claim, E, S, U)
            got = (ctx.hp_prove_eq(st_g, claim, u, ctx.from_fr(S), ctx.from_fr(U)) if form == "eq"
                   else ctx.hp_prove(st_g, claim, ctx.from_fr(E), ctx.from_fr(S), ctx.from_fr(U)))
        assert rc == 0
        for key in ("ev", "term", "ws"):
            assert fr_eq(got[key], want[key]), (form, key)
        assert bytes(st_g) == bytes(st_o)


def test_calib_fr_mul(zkh, ctx):
    """The multiply-rate probe runs and reports a plausible device-wide rate; zero
    iterations are refused."""
    rate = ctx.calib_fr_mul(64)
    assert 1e9 < rate < 1e13, rate
    with pytest.raises(zkh.ZkhError):
        ctx.calib_fr_mul(0)


@pytest.mark.parametrize("k,extreme", [(4, False), (14, False), (16, False), (15, True)])
def test_hp_prove_u_all_ones(zkh, ctx, k, extreme):
    """U = 1 everywhere as an int32 tensor (the RoPE obligations' U, zkob_rope.cu:215-281): the
    per-round kernels skip U (E_t S_t from three products per pair) and must give the oracle's
    proof of the generic E, S, U sumcheck.  With an int32 S (extreme) the first round forms its
    sums exactly with the 32-bit multiply, here at the ends of the int32 range."""
    n = 1 << k
    rng = np.random.default_rng(100 + k)
    E = rand_fr_full(rng, n)
    Sv = rng.integers(-2**31 if extreme else -2**20, 2**31 if extreme else 2**20, size=n)
    if extreme:  # the first round's 32-bit multiply at the ends of the int32 range
        Sv[:6] = [-2**31, 2**31 - 1, 0, -1, 2**31 - 1, -2**31]
    S = C.ints_to_fr(Sv)
    ones = np.ones(n, np.int64)
    Ei, Si = C.fr_to_ints(E), C.fr_to_ints(S)
    claim = C.ints_to_fr([sum(a * b for a, b in zip(Ei, Si)) % P.R])[0]
    st_g, st_o = seed_transcript(zkh, "hp1:%d" % k)
    rc, want = C.hp_prove(st_o, claim, E, S, C.ints_to_fr(ones))
    assert rc == 0
    got = ctx.hp_prove(st_g, claim, ctx.from_fr(E), ctx.from_i32(Sv.astype(np.int32)) if extreme else ctx.from_fr(S),
                       ctx.from_i32(ones.astype(np.int32)))
    for key in ("ev", "term", "ws"):
        assert fr_eq(got[key], want[key]), key
    assert bytes(st_g) == bytes(st_o)


@pytest.mark.parametrize("k,bits", [(15, 20), (16, 29), (15, 31)])
def test_hp_prove_eq_small_ints(zkh, ctx, k, bits):
    """Eq-form Hadamard on int32 witnesses (the SwiGLU segment's S and U): the first round forms
    the products as 64-bit integers while every value is within (-2^30, 2^30) and as field
    products otherwise (bits = 31 mixes both within one round); proofs equal the oracle's."""
    n = 1 << k
    rng = np.random.default_rng(200 + k + bits)
    u = rand_fr_full(rng, k)
    Si = rng.integers(-(1 << bits), 1 << bits, size=n)
    Ui = rng.integers(-(1 << 15), 1 << 15, size=n)
    Si[:4] = [-(1 << 30), (1 << 30) - 1, -(1 << 31), (1 << 31) - 1]
    E = C.build_eq(u)
    S, U = C.ints_to_fr(Si), C.ints_to_fr(Ui)
    Ei = C.fr_to_ints(E)
    claim = C.ints_to_fr([sum(a * int(b) % P.R * int(c) for a, b, c in zip(Ei, Si, Ui)) % P.R])[0]
    st_g, st_o = seed_transcript(zkh, "hpeq:%d:%d" % (k, bits))
    rc, want = C.hp_prove(st_o, claim, E, S, U)
    assert rc == 0
    got = ctx.hp_prove_eq(st_g, claim, u, ctx.from_i32(Si.astype(np.int32)), ctx.from_i32(Ui.astype(np.int32)))
    for key in ("ev", "term", "ws"):
        assert fr_eq(got[key], want[key]), key
    assert bytes(st_g) == bytes(st_o)


@pytest.mark.parametrize("k,form,no_persist", [(0, "ones", False), (5, "ones", False), (13, "gen", False),
                                               (14, "ones", False), (14, "gen", False), (15, "ones_i32", False),
                                               (14, "ones", True), (17, "ones_i32", False)])
def test_hp_prove_claim(zkh, ctx, k, form, no_persist, monkeypatch):
    """c = (E * S * U).sum(), its absorb, then fs_hadamard in one call (zkob_rope.cu:230-238):
    the claim from the first round's sums (k >= 14, or every k with no persistent loop) or the
    products' sum ahead of the persistent loop (k <= 13).  U all ones as an int32 tensor (the
    RoPE form, S as field elements or int32 at the ends of its range) or a general U.  Claim,
    proof and transcript equal the separate steps' (hadamard, sum, absorb, hp_prove) and, up
    to 2^15, the oracle's."""
    n = 1 << k
    rng = np.random.default_rng(900 + k + 7 * len(form))
    if no_persist:
        monkeypatch.setenv("ZKH_NO_PERSIST", "1")
    E = rand_fr_full(rng, n)
    if form == "ones_i32":
        Sv = rng.integers(-2**31, 2**31, size=n)
        Sv[:4] = [-2**31, 2**31 - 1, 0, -1][:n]
        S_f = C.ints_to_fr(Sv)
        S_t = ctx.from_i32(Sv.astype(np.int32))
    else:
        S_f = rand_fr_full(rng, n)
        S_t = ctx.from_fr(S_f)
    if form == "gen":
        U_f = rand_fr_full(rng, n)
        U_t = ctx.from_fr(U_f)
    else:
        U_f = C.ints_to_fr(np.ones(n, np.int64))
        U_t = ctx.from_i32(np.ones(n, np.int32))
    E_t = ctx.from_fr(E)
    st1, st_o = seed_transcript(zkh, "hpc:%d:%s" % (k, form))
    st2 = st1.copy()
    got = ctx.hp_prove_claim(st1, "c1", E_t, S_t, U_t)
    claim = ctx.sum(ctx.hadamard(E_t, ctx.hadamard(S_t, U_t)))
    zkh.absorb(st2, "c1", claim.tobytes())
    want = ctx.hp_prove(st2, claim, E_t, S_t, U_t)
    assert fr_eq(got["claim"], claim)
    for key in ("ev", "term", "ws"):
        assert fr_eq(got[key], want[key]), key
    assert bytes(st1) == bytes(st2)
    if k <= 15:
        Ei, Si, Ui = C.fr_to_ints(E), C.fr_to_ints(S_f), C.fr_to_ints(U_f)
        oc = C.ints_to_fr([sum(a * b % P.R * c for a, b, c in zip(Ei, Si, Ui)) % P.R])[0]
        assert fr_eq(got["claim"], oc)
        C.tr_absorb(st_o, "c1", oc.tobytes())
        rc, hp = C.hp_prove(st_o, oc, E, S_f, U_f)
        assert rc == 0
        assert fr_eq(got["ev"], hp["ev"]) and fr_eq(got["term"], hp["term"])
        assert bytes(st1) == bytes(st_o)


@pytest.mark.parametrize("k,kind,no_persist", [(0, "i32", False), (0, "i32", True), (6, "i32", False),
                                               (13, "i32", False), (14, "i32", False), (14, "fr", False),
                                               (18, "i32", False)])
def test_hp_prove_eq_claim(zkh, ctx, k, kind, no_persist, monkeypatch):
    """claim_H = H(u) of H = S (.) U, its absorb, then the eq-form Hadamard sumcheck in one call
    (zkob_glu.cu:231-247): the claim from the first round's sums (k >= 14) or from the
    eq-weighted sum ahead of the persistent loop (k <= 13).  Claim, proof and transcript equal
    the separate steps' (me of the hadamard, absorb, hp_prove_eq) and, up to 2^14, the oracle's."""
    n = 1 << k
    rng = np.random.default_rng(500 + k + (kind == "fr"))
    s = rng.integers(-2**15, 2**15, size=n, dtype=np.int64)
    uu = rng.integers(-2**15, 2**15, size=n, dtype=np.int64)
    s[:3] = [-2**31, 2**31 - 1, 0][:n]  # beyond the first round's small-integer range
    uu[:3] = [-2**31, -2**31, 5][:n]
    if no_persist:  # every round a round kernel (k = 0: none at all, the sum first)
        monkeypatch.setenv("ZKH_NO_PERSIST", "1")
    Sf, Uf = C.ints_to_fr([int(x) for x in s]), C.ints_to_fr([int(x) for x in uu])
    if kind == "i32":
        S, U = ctx.from_i32(s.astype(np.int32)), ctx.from_i32(uu.astype(np.int32))
    else:
        S, U = ctx.from_fr(Sf), ctx.from_fr(Uf)
    u = rand_fr_full(rng, k)
    st1, st_o = seed_transcript(zkh, "hpclaim%d" % k)
    st2 = st1.copy()
    got = ctx.hp_prove_eq_claim(st1, "claim_H", u, S, U)
    claim = ctx.me(ctx.hadamard(S, U), u)
    zkh.absorb(st2, "claim_H", claim.tobytes())
    want = ctx.hp_prove_eq(st2, claim, u, S, U)
    assert fr_eq(got["claim"], claim)
    for key in ("ev", "term", "ws"):
        assert fr_eq(got[key], want[key]), key
    assert bytes(st1) == bytes(st2)
    if k <= 14:
        rc, oc = C.me(C.hadamard(Sf, Uf), u)
        assert rc == 0
        C.tr_absorb(st_o, "claim_H", oc.tobytes())
        rc, hp = C.hp_prove(st_o, oc, C.build_eq(u), Sf, Uf)
        assert rc == 0
        assert fr_eq(got["claim"], oc)
        assert fr_eq(got["ev"], hp["ev"]) and fr_eq(got["term"], hp["term"])
        assert bytes(st1) == bytes(st_o)
