"""zkh_me_static (the allocation-free MLE evaluation) against zkh_me and the oracle, through
the C ABI: two calls in a row, the second on a smaller input, then a third larger again,
Boolean points, the rejections (too many variables, integer tensor), and that the calls
leave the device's free memory unchanged."""
import ctypes

import numpy as np
import pytest

from oracle import coracle as C
from oracle import pyref as P

pytestmark = pytest.mark.gpu


def rand_fr_full(rng, n):
    return C.ints_to_fr([int.from_bytes(rng.bytes(32), "little") % P.R for _ in range(n)])


def fr_eq(a, b):
    return np.array_equal(np.asarray(a, np.uint32).reshape(-1, 8), np.asarray(b, np.uint32).reshape(-1, 8))


@pytest.fixture(scope="module")
def sctx(zkh):
    c = zkh.Context(0)
    yield c
    c.close()


def _check(zkh, ctx, n, k, seed):
    rng = np.random.default_rng(seed)
    t = rand_fr_full(rng, n)
    u = rand_fr_full(rng, k) if k else np.zeros((0, 8), np.uint32)
    tt = ctx.from_fr(t)
    got = ctx.me_static(tt, u)
    assert fr_eq(got, ctx.me(tt, u))
    rc, want = C.me(t, u)
    assert rc == 0 and fr_eq(got, want)


def test_me_static_two_calls_second_smaller(zkh, sctx):
    _check(zkh, sctx, 70000, 17, 1)
    _check(zkh, sctx, 1000, 10, 2)   # smaller: the scratch keeps the first call's contents
    _check(zkh, sctx, 5, 3, 3)
    _check(zkh, sctx, 1, 0, 4)
    _check(zkh, sctx, 300000, 19, 5)


def test_me_static_max_vars(zkh, sctx):
    n = (1 << 23) + 12345  # k = 24, the static scratch's limit
    rng = np.random.default_rng(6)
    t = C.ints_to_fr(rng.integers(-2**40, 2**40, size=n))
    u = rand_fr_full(rng, 24)
    tt = sctx.from_fr(t)
    got = sctx.me_static(tt, u)
    assert fr_eq(got, sctx.me(tt, u))
    rc, want = C.me(t, u)
    assert fr_eq(got, want)


def test_me_static_boolean_point(zkh, sctx):
    rng = np.random.default_rng(7)
    t = rand_fr_full(rng, 3000)
    tt = sctx.from_fr(t)
    for idx in (0, 2999, 1234):
        u = C.ints_to_fr([(idx >> b) & 1 for b in range(12)])
        assert fr_eq(sctx.me_static(tt, u), t[idx])


def test_me_static_rejections(zkh, sctx):
    n = (1 << 24) + 1  # needs k = 25
    tt = sctx.from_fr(np.zeros((n, 8), np.uint32))
    with pytest.raises(zkh.ZkhError) as e:
        sctx.me_static(tt, np.zeros((25, 8), np.uint32))
    assert e.value.code == zkh.EARG and "static scratch" in str(e.value)
    ti = sctx.from_i32(np.arange(16, dtype=np.int32))
    with pytest.raises(zkh.ZkhError) as e:
        sctx.me_static(ti, np.zeros((4, 8), np.uint32))
    assert e.value.code == zkh.EARG
    # the context still works afterwards
    _check(zkh, sctx, 100, 7, 8)


def _device_free_bytes():
    """hipMemGetInfo's free bytes of the current device, from the HIP runtime libzkh.so uses."""
    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_me_static_allocates_nothing(zkh):
    """A fresh context: after its tensors exist and one zkh_me has run the same kernels once
    (the runtime's first launches may set up the code object), several zkh_me_static calls
    of different sizes must not change the device's free memory."""
    ctx = zkh.Context(0)
    try:
        rng = np.random.default_rng(9)
        big = ctx.from_fr(rand_fr_full(rng, 1 << 16))
        small = ctx.from_fr(rand_fr_full(rng, 300))
        u16, u9 = rand_fr_full(rng, 16), rand_fr_full(rng, 9)
        want_big, want_small = ctx.me(big, u16), ctx.me(small, u9)
        ctx.sync()
        before = _device_free_bytes()
        for _ in range(3):
            assert fr_eq(ctx.me_static(big, u16), want_big)
            assert fr_eq(ctx.me_static(small, u9), want_small)
        ctx.sync()
        assert _device_free_bytes() == before
    finally:
        ctx.close()
