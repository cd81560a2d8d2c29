"""ctypes binding of the C oracle (libzkh_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker or the timed CPU baseline.  Field elements are passed
as numpy uint32 arrays of shape (n, 8) (the reference's Fr_t layout).
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "libzkh_oracle.so")
        if not os.path.exists(path):
            raise RuntimeError("oracle not built: run `make -C oracle`")
        _LIB = ctypes.CDLL(path)
    return _LIB


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def frs(n):
    return np.zeros((n, 8), dtype=np.uint32)


def set_threads(n):
    """OpenMP threads of the oracle's table loops (1: the scalar CPU baseline)."""
    lib().or_set_threads(ctypes.c_int(int(n)))


def get_threads():
    return int(lib().or_get_threads())


def ints_to_fr(vals):
    """Integers (any sign) -> (n,8) uint32, reduced mod r."""
    arr = np.asarray(vals)
    if arr.dtype.kind in "iu" and (arr.dtype.itemsize < 8 or arr.dtype.kind == "i"):
        v = np.ascontiguousarray(arr.reshape(-1), dtype=np.int64)
        out = frs(len(v))
        lib().or_ints_to_fr(_p(v), ctypes.c_size_t(len(v)), _p(out))
        return out
    from .pyref import R, to_limbs
    out = frs(len(vals))
    for i, v in enumerate(vals):
        out[i] = to_limbs(int(v) % R)
    return out


def fr_to_ints(a):
    a = np.asarray(a, dtype=np.uint64).reshape(-1, 8)
    return [sum(int(row[i]) << (32 * i) for i in range(8)) for row in a]


def tr_init(seed):
    st = np.zeros(32, dtype=np.uint8)
    b = seed.encode()
    lib().or_tr_init(_p(st), b, ctypes.c_size_t(len(b)))
    return st


def tr_absorb(st, label, data):
    lb = label.encode()
    buf = np.frombuffer(bytes(data), dtype=np.uint8).copy()
    lib().or_tr_absorb(_p(st), lb, ctypes.c_size_t(len(lb)), _p(buf), ctypes.c_size_t(len(buf)))


def tr_challenge_fr(st):
    out = np.zeros(8, dtype=np.uint32)
    lib().or_tr_challenge_fr(_p(st), _p(out))
    return out


def sha256(data):
    buf = np.frombuffer(bytes(data), dtype=np.uint8).copy()
    out = np.zeros(32, dtype=np.uint8)
    lib().or_sha256(_p(buf), ctypes.c_size_t(len(buf)), _p(out))
    return bytes(out)


def fr_op(name, a, b=None):
    out = np.zeros(8, dtype=np.uint32)
    a = np.ascontiguousarray(a, dtype=np.uint32)
    if b is None:
        getattr(lib(), "or_fr_" + name)(_p(a), _p(out))
    else:
        b = np.ascontiguousarray(b, dtype=np.uint32)
        getattr(lib(), "or_fr_" + name)(_p(a), _p(b), _p(out))
    return out


def me(t, u):
    t = np.ascontiguousarray(t, dtype=np.uint32)
    u = np.ascontiguousarray(u, dtype=np.uint32).reshape(-1, 8)
    out = np.zeros(8, dtype=np.uint32)
    rc = lib().or_me(_p(t), ctypes.c_uint32(len(t)), _p(u), ctypes.c_uint32(len(u)), _p(out))
    return rc, out


def partial_me(t, u, cur_dim, window):
    t = np.ascontiguousarray(t, dtype=np.uint32)
    u = np.ascontiguousarray(u, dtype=np.uint32).reshape(-1, 8)
    out = frs(len(t))
    on = ctypes.c_uint32(0)
    rc = lib().or_partial_me(_p(t), ctypes.c_uint32(len(t)), _p(u), ctypes.c_uint32(len(u)),
                             ctypes.c_uint32(cur_dim), ctypes.c_uint32(window), _p(out),
                             ctypes.byref(on))
    return rc, out[:on.value]


def multi_dim_me(t, us, shape):
    t = np.ascontiguousarray(t, dtype=np.uint32)
    ks = np.array([len(u) for u in us], dtype=np.uint32)
    cat = np.concatenate([np.asarray(u, dtype=np.uint32).reshape(-1, 8) for u in us] +
                         [frs(0)]) if us else frs(1)
    cat = np.ascontiguousarray(cat)
    shp = np.array(shape, dtype=np.uint32)
    out = np.zeros(8, dtype=np.uint32)
    rc = lib().or_multi_dim_me(_p(t), ctypes.c_uint32(len(t)), _p(cat), _p(ks), _p(shp),
                               ctypes.c_uint32(len(shape)), _p(out))
    return rc, out


def build_eq(u):
    u = np.ascontiguousarray(u, dtype=np.uint32).reshape(-1, 8)
    out = frs(1 << len(u))
    lib().or_build_eq(_p(u), ctypes.c_uint32(len(u)), _p(out))
    return out


def mm_prove(st, X, W, Y, B, IN, OUT):
    """Returns (rc, dict) for the zkob_fc.cu:259-440 segment on int inputs."""
    from .pyref import ceil_log2
    X = np.ascontiguousarray(X, dtype=np.int32)
    W = np.ascontiguousarray(W, dtype=np.int32)
    Y = np.ascontiguousarray(Y, dtype=np.int64)
    L, lb, lo = ceil_log2(IN), ceil_log2(B), ceil_log2(OUT)
    ev, cl = frs(3 * L + 1), frs(3)
    ub, uo, ui = frs(lb + 1), frs(lo + 1), frs(L + 1)
    rc = lib().or_mm_prove(_p(st), _p(X), _p(W), _p(Y), ctypes.c_uint32(B), ctypes.c_uint32(IN),
                           ctypes.c_uint32(OUT), _p(ev), _p(cl), _p(ub), _p(uo), _p(ui))
    return rc, dict(ev=ev[:3 * L], claims=cl, u_batch=ub[:lb], u_output=uo[:lo], u_input=ui[:L])


def mm_prove_fr(st, X, W, Y, B, IN, OUT):
    """The same segment on field-element tables: X (B*IN, 8), W (IN*OUT, 8), Y (B*OUT, 8)."""
    from .pyref import ceil_log2
    X, W, Y = (np.ascontiguousarray(a, dtype=np.uint32) for a in (X, W, Y))
    L, lb, lo = ceil_log2(IN), ceil_log2(B), ceil_log2(OUT)
    ev, cl = frs(3 * L + 1), frs(3)
    ub, uo, ui = frs(lb + 1), frs(lo + 1), frs(L + 1)
    rc = lib().or_mm_prove_fr(_p(st), _p(X), _p(W), _p(Y), ctypes.c_uint32(B), ctypes.c_uint32(IN),
                              ctypes.c_uint32(OUT), _p(ev), _p(cl), _p(ub), _p(uo), _p(ui))
    return rc, dict(ev=ev[:3 * L], claims=cl, u_batch=ub[:lb], u_output=uo[:lo], u_input=ui[:L])


def axpy(a, c, b):
    a, b = (np.ascontiguousarray(x, dtype=np.uint32).reshape(-1, 8) for x in (a, b))
    out = frs(len(a))
    lib().or_axpy(_p(a), _p(np.ascontiguousarray(c, dtype=np.uint32)), _p(b), ctypes.c_size_t(len(a)), _p(out))
    return out


def hadamard(a, b):
    a, b = (np.ascontiguousarray(x, dtype=np.uint32).reshape(-1, 8) for x in (a, b))
    out = frs(len(a))
    lib().or_hadamard(_p(a), _p(b), ctypes.c_size_t(len(a)), _p(out))
    return out


def check_inverse(S, A, beta):
    """Entries of A that are not 1/(S + beta) (0 where S + beta = 0)."""
    S, A = (np.ascontiguousarray(x, dtype=np.uint32).reshape(-1, 8) for x in (S, A))
    lib().or_check_inverse.restype = ctypes.c_size_t
    return int(lib().or_check_inverse(_p(S), _p(A), ctypes.c_size_t(len(S)),
                                      _p(np.ascontiguousarray(beta, dtype=np.uint32))))


def range_table(low, length, size):
    T = frs(size)
    lib().or_range_table(ctypes.c_int32(low), ctypes.c_uint32(length), ctypes.c_uint32(size), _p(T))
    return T


def lu_prep(S, low, N):
    S = np.ascontiguousarray(S, dtype=np.uint32)
    m = frs(N)
    rc = lib().or_lu_prep(_p(S), ctypes.c_uint32(len(S)), ctypes.c_int32(low), ctypes.c_uint32(N),
                          _p(m))
    return rc, m


def lu_inverse(S, beta):
    S = np.ascontiguousarray(S, dtype=np.uint32)
    beta = np.ascontiguousarray(beta, dtype=np.uint32)
    A = frs(len(S))
    lib().or_lu_inverse(_p(S), ctypes.c_uint32(len(S)), _p(beta), _p(A))
    return A


def lu_prove(st, A, S, T, m, alpha, beta, u, strict=True):
    from .pyref import ceil_log2
    D, N = len(A), len(T)
    logD = ceil_log2(D)
    arrs = [np.ascontiguousarray(x, dtype=np.uint32) for x in (A, S, T, m, alpha, beta, u)]
    ev, term, ws = frs(4 * logD + 1), frs(5), frs(logD + 1)
    rc = lib().or_lu_prove(_p(st), *[_p(x) for x in arrs[:4]], ctypes.c_uint32(D),
                           ctypes.c_uint32(N), _p(arrs[4]), _p(arrs[5]), _p(arrs[6]),
                           ctypes.c_int(1 if strict else 0), _p(ev), _p(term), _p(ws))
    return rc, dict(ev=ev[:4 * logD], term=term, ws=ws[:logD])


def hp_prove(st, claim, E, S, U, strict=True):
    n = len(E)
    k = n.bit_length() - 1
    arrs = [np.ascontiguousarray(x, dtype=np.uint32) for x in (claim, E, S, U)]
    ev, term, ws = frs(4 * k + 1), frs(3), frs(k + 1)
    rc = lib().or_hp_prove(_p(st), _p(arrs[0]), _p(arrs[1]), _p(arrs[2]), _p(arrs[3]),
                           ctypes.c_uint32(n), ctypes.c_int(1 if strict else 0), _p(ev),
                           _p(term), _p(ws))
    return rc, dict(ev=ev[:4 * k], term=term, ws=ws[:k])


def pad_val(t, shape, pad):
    t = np.ascontiguousarray(t, dtype=np.uint32)
    shp = np.array(shape, dtype=np.uint32)
    total = 1
    for s in shape:
        total *= 1 << (int(s) - 1).bit_length() if s > 1 else 1
    out = frs(total)
    on = ctypes.c_uint32(0)
    pv = np.ascontiguousarray(pad, dtype=np.uint32)
    rc = lib().or_pad_val(_p(t), _p(shp), ctypes.c_uint32(len(shape)), _p(pv), _p(out), ctypes.byref(on))
    return rc, out[:on.value]


def partial_me_window(t, u, window):
    t = np.ascontiguousarray(t, dtype=np.uint32)
    u = np.ascontiguousarray(u, dtype=np.uint32).reshape(-1, 8)
    out = frs(len(t) + window)
    on = ctypes.c_uint32(0)
    rc = lib().or_partial_me_window(_p(t), ctypes.c_uint32(len(t)), _p(u), ctypes.c_uint32(len(u)),
                                    ctypes.c_uint32(window), _p(out), ctypes.byref(on))
    return rc, out[:on.value]


def _u(u):
    u = np.ascontiguousarray(u, dtype=np.uint32).reshape(-1, 8)
    return u if len(u) else frs(1)


def zkip(claim, a, b, u):
    k = len(u)
    a, b = (np.ascontiguousarray(x, dtype=np.uint32) for x in (a, b))
    proof, fin = frs(3 * k + 1), np.zeros(8, np.uint32)
    rc = lib().or_zkip(_p(np.ascontiguousarray(claim, dtype=np.uint32)), _p(a), _p(b),
                       ctypes.c_uint32(len(a)), _p(_u(u)), ctypes.c_uint32(k), _p(proof), _p(fin))
    return rc, proof[:3 * k], fin


def zkip_stacked(claim, A, B, uN, uD, vN, N, D):
    kN, kD = len(uN), len(uD)
    A, B = (np.ascontiguousarray(x, dtype=np.uint32) for x in (A, B))
    proof, fin = frs(3 * (kN + kD) + 1), np.zeros(8, np.uint32)
    rc = lib().or_zkip_stacked(_p(np.ascontiguousarray(claim, dtype=np.uint32)), _p(A), _p(B),
                               _p(_u(uN)), ctypes.c_uint32(kN), _p(_u(uD)), ctypes.c_uint32(kD),
                               _p(_u(vN)), ctypes.c_uint32(N), ctypes.c_uint32(D), _p(proof), _p(fin))
    return rc, proof[:3 * (kN + kD)], fin


def fc_stacked_prove(X, W, Y, bias, num, B, IN, OUT, u_num, v_num, u_batch, u_input, u_output):
    X, W, Y = (np.ascontiguousarray(x, dtype=np.uint32) for x in (X, W, Y))
    bp = None if bias is None else _p(np.ascontiguousarray(bias, dtype=np.uint32))
    nr = len(u_num) + len(u_input)
    proof, claims = frs(3 * nr + 1), frs(2)
    rc = lib().or_fc_stacked_prove(_p(X), _p(W), _p(Y), bp, ctypes.c_uint32(num), ctypes.c_uint32(B),
                                   ctypes.c_uint32(IN), ctypes.c_uint32(OUT),
                                   *[_p(_u(x)) for x in (u_num, v_num, u_batch, u_input, u_output)],
                                   _p(proof), _p(claims))
    return rc, proof[:3 * nr], claims


def scalar_to_long(x):
    lib().or_scalar_to_long.restype = ctypes.c_int64
    return lib().or_scalar_to_long(_p(np.ascontiguousarray(x, dtype=np.uint32)))


def rescale(x, sf):
    """x: int64 array or (n, 8) Fr array -> (rc, q, rem) as int64 arrays."""
    x = np.asarray(x)
    if x.dtype == np.uint32 and x.ndim == 2:
        n = len(x)
        q, r = np.zeros(n, np.int64), np.zeros(n, np.int64)
        rc = lib().or_rescale_fr(_p(np.ascontiguousarray(x)), ctypes.c_uint32(n), ctypes.c_uint32(sf), _p(q), _p(r))
    else:
        x = np.ascontiguousarray(x, dtype=np.int64).reshape(-1)
        n = len(x)
        q, r = np.zeros(n, np.int64), np.zeros(n, np.int64)
        rc = lib().or_rescale_i64(_p(x), ctypes.c_uint32(n), ctypes.c_uint32(sf), _p(q), _p(r))
    return rc, q, r


def matmul_fr(A, B, M, N, Pc, bias=None):
    """FrTensor::matmul (+ zkFC bias): A (M*N, 8), B (N*Pc, 8) Fr arrays -> (rc, C (M*Pc, 8))."""
    A = np.ascontiguousarray(A, dtype=np.uint32)
    B = np.ascontiguousarray(B, dtype=np.uint32)
    C = np.zeros((M * Pc, 8), np.uint32)
    bp = _p(np.ascontiguousarray(bias, dtype=np.uint32)) if bias is not None else None
    rc = lib().or_matmul_fr(_p(A), _p(B), bp, ctypes.c_uint32(M), ctypes.c_uint32(N), ctypes.c_uint32(Pc), _p(C))
    return rc, C


# ---- G1 over Fp (zkh_g1_oracle.c): Fp as (12,) uint32, points as (36,) uint32 ----
def fp_op(name, a, b):
    out = np.zeros(12, dtype=np.uint32)
    getattr(lib(), "or_fp_" + name)(_p(np.ascontiguousarray(a, np.uint32)),
                                     _p(np.ascontiguousarray(b, np.uint32)), _p(out))
    return out


def g1_dbl(p):
    out = np.zeros(36, dtype=np.uint32)
    lib().or_g1_dbl(_p(np.ascontiguousarray(p, np.uint32)), _p(out))
    return out


def g1_add(a, b):
    out = np.zeros(36, dtype=np.uint32)
    lib().or_g1_add(_p(np.ascontiguousarray(a, np.uint32)), _p(np.ascontiguousarray(b, np.uint32)),
                    _p(out))
    return out


def g1_mul(a, s):
    out = np.zeros(36, dtype=np.uint32)
    lib().or_g1_mul(_p(np.ascontiguousarray(a, np.uint32)), _p(np.ascontiguousarray(s, np.uint32)),
                    _p(out))
    return out


def g1_commit(gens, scalars, n):
    """gens (n, 36) uint32; scalars (m*n, 8) plain Fr -> (m, 36) points."""
    gens = np.ascontiguousarray(gens, np.uint32).reshape(n, 36)
    sc = np.ascontiguousarray(scalars, np.uint32).reshape(-1, 8)
    m = sc.shape[0] // n
    out = np.zeros((m, 36), dtype=np.uint32)
    rc = lib().or_g1_commit(_p(gens), ctypes.c_uint32(n), _p(sc), ctypes.c_uint32(m), _p(out))
    return rc, out


def ipa_prove(st, a, b, g, Q, n):
    """ipa_prove: a, b (n, 8) plain Fr; g (n, 36); Q (36,).  Returns (rc, L, R, a_final)."""
    rounds = max(n.bit_length() - 1, 0)
    L = np.zeros((rounds, 36), np.uint32)
    R = np.zeros((rounds, 36), np.uint32)
    af = np.zeros(8, np.uint32)
    rc = lib().or_ipa_prove(_p(st), _p(np.ascontiguousarray(a, np.uint32)), _p(np.ascontiguousarray(b, np.uint32)),
                            _p(np.ascontiguousarray(g, np.uint32)), _p(np.ascontiguousarray(Q, np.uint32)),
                            ctypes.c_uint32(n), _p(L), _p(R), _p(af))
    return rc, L, R, af
