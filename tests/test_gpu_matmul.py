"""GPU parity for the witness GEMM (zkh_matmul_i32): Y = X W (+ bias) over the integers, the
zkFC::operator() / FrTensor::matmul step of zkob_fc prove (zkob_fc.cu:212, zkfc.cu:44-58,
fr-tensor.cu:831-878).  Small shapes are checked against the C oracle's field matmul (the
reference's Montgomery accumulation), larger ones against numpy's exact int64 product; both
paths (fp64 matrix cores and int64 VALU) and the overflow rule are covered, and a matmul
sumcheck proven from the GPU's Y equals the one proven from numpy's."""
import numpy as np
import pytest

from oracle import coracle as C
from oracle import pyref as P

pytestmark = pytest.mark.gpu


def fr_eq(a, b):
    return np.array_equal(np.asarray(a, np.uint32).reshape(-1, 8), np.asarray(b, np.uint32).reshape(-1, 8))


def as_fr(v):
    return C.ints_to_fr(np.asarray(v, np.int64).reshape(-1))


SMALL = [(1, 1, 1), (5, 7, 3), (16, 16, 16), (33, 100, 70), (64, 128, 64), (3, 257, 5)]


@pytest.mark.parametrize("B,IN,OUT", SMALL)
@pytest.mark.parametrize("registered", [False, True])
@pytest.mark.parametrize("bias", [None, "i32", "i64"])
def test_matmul_small_vs_oracle(zkh, ctx, B, IN, OUT, registered, bias):
    rng = np.random.default_rng(B * 1000 + IN * 10 + OUT)
    X = rng.integers(-2**15, 2**15, size=(B, IN)).astype(np.int32)
    W = rng.integers(-229376, 229377, size=(IN, OUT)).astype(np.int32)
    b = rng.integers(-2**20, 2**20, size=OUT) if bias else None
    rc, want = C.matmul_fr(as_fr(X), as_fr(W), B, IN, OUT, as_fr(b) if bias else None)
    assert rc == 0
    Wg = ctx.weights_i32(W, IN, OUT) if registered else ctx.from_i32(W.reshape(-1))
    bg = None if not bias else ctx.from_i32(b.astype(np.int32)) if bias == "i32" else ctx.from_i64(b.astype(np.int64))
    Y = ctx.matmul_i32(ctx.from_i32(X.reshape(-1)), Wg, B, IN, OUT, bg)
    assert fr_eq(Y.to_fr(), want)


@pytest.mark.parametrize("B,IN,OUT,bx,bw", [
    (512, 2048, 256, 15, 18),     # TinyLlama K/V shape, fp64 path
    (128, 3001, 97, 16, 19),      # odd sizes, IN not a multiple of 4
    (64, 64, 64, 24, 24),         # 24 + 24 + 6 = 54 bits: int64 path
    (40, 1000, 30, 26, 25),       # int64 path, non-multiple tiles
    (8, 4, 8, 31, 31),            # 31 + 31 + 2 = 64 > 63: rejected
])
def test_matmul_paths_vs_numpy(zkh, ctx, B, IN, OUT, bx, bw):
    rng = np.random.default_rng(B + IN + OUT + bx)
    X = rng.integers(-(2**bx - 1), 2**bx, size=(B, IN)).astype(np.int64)
    W = rng.integers(-(2**bw - 1), 2**bw, size=(IN, OUT)).astype(np.int64)
    X[0, 0], W[0, 0] = 2**bx - 1, 2**bw - 1  # the bounds are reached
    Xg, Wg = ctx.from_i32(X.astype(np.int32).reshape(-1)), ctx.weights_i32(W.astype(np.int32), IN, OUT)
    if bx + bw + P.ceil_log2(IN) + 1 > 63:
        with pytest.raises(zkh.ZkhError) as e:
            ctx.matmul_i32(Xg, Wg, B, IN, OUT)
        assert e.value.code == zkh.EARG
        return
    want = X @ W  # exact: |sum| < 2^63
    Y = ctx.matmul_i32(Xg, Wg, B, IN, OUT)
    assert fr_eq(Y.to_fr(), as_fr(want))


def test_matmul_shape_rules(zkh, ctx):
    X = ctx.from_i32(np.zeros(12, np.int32))
    W = ctx.from_i32(np.zeros(12, np.int32))
    with pytest.raises(zkh.ZkhError) as e:
        ctx.matmul_i32(X, W, 3, 5, 4)  # X holds 12 entries, not 15
    assert e.value.code == zkh.EARG
    Wr = ctx.weights_i32(np.zeros((4, 3), np.int32), 4, 3)
    with pytest.raises(zkh.ZkhError) as e:
        ctx.matmul_i32(X, Wr, 4, 3, 4)  # registered as 4 x 3, used as 3 x 4
    assert e.value.code == zkh.EARG


def test_matmul_feeds_mm_prove(zkh, ctx):
    """Y from the GPU witness GEMM gives the same matmul sumcheck as numpy's Y."""
    rng = np.random.default_rng(7)
    B, IN, OUT = 64, 200, 48
    X = rng.integers(-2**15, 2**15, size=(B, IN)).astype(np.int32)
    W = rng.integers(-229376, 229377, size=(IN, OUT)).astype(np.int32)
    Xg, Wg = ctx.from_i32(X.reshape(-1)), ctx.weights_i32(W, IN, OUT)
    Yg = ctx.matmul_i32(Xg, Wg, B, IN, OUT)
    Yn = ctx.from_i64((X.astype(np.int64) @ W.astype(np.int64)).reshape(-1))
    outs = []
    for Y in (Yg, Yn):
        st = zkh.transcript("witness-gemm")
        outs.append((ctx.mm_prove(st, Xg, Wg, Y, B, IN, OUT), bytes(st)))
    for k in ("ev", "claims", "u_input"):
        assert np.array_equal(outs[0][0][k], outs[1][0][k]), k
    assert outs[0][1] == outs[1][1]
