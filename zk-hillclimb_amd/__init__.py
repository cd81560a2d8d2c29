"""Python binding of libzkh.so, the C-ABI MI355X prover hot path (include/zkh.h).

This is a thin ctypes layer for tests, the smoke check and bench.py; the product is the
shared library.  Field elements are numpy uint32 arrays of shape (n, 8) in the reference's
Fr_t layout (8 little-endian limbs, canonical, plain).  Every call raises ZkhError on a
non-zero return code; there is no CPU fallback: without the built library or a GPU the
calls fail.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libzkh.so")

OK, EARG, EROUND, EDEV = 0, 1, 2, 3
KIND_FR, KIND_I32, KIND_I64 = 0, 1, 2

_lib = None


class MmJob(ctypes.Structure):
    _fields_ = [("X", ctypes.c_void_p), ("W", ctypes.c_void_p), ("Y", ctypes.c_void_p),
                ("B", ctypes.c_uint32), ("IN", ctypes.c_uint32), ("OUT", ctypes.c_uint32),
                ("transcript", ctypes.c_void_p), ("ev_out", ctypes.c_void_p),
                ("claims_out", ctypes.c_void_p), ("u_batch_out", ctypes.c_void_p),
                ("u_output_out", ctypes.c_void_p), ("u_input_out", ctypes.c_void_p),
                ("status", ctypes.c_int)]


class ZkhError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__("zkh error %d: %s" % (code, msg))
        self.code = code


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError("libzkh.so is not built (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        vp, u32, i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int32
        L.zkh_last_error.restype = ctypes.c_char_p
        L.zkh_last_error.argtypes = [vp]
        L.zkh_tensor_size.restype = u32
        L.zkh_tensor_size.argtypes = [vp]
        L.zkh_tensor_kind.argtypes = [vp]
        for name in ["zkh_ctx_destroy", "zkh_ctx_sync", "zkh_tensor_free"]:
            getattr(L, name).argtypes = [vp]
        L.zkh_ctx_create.argtypes = [ctypes.c_int, ctypes.POINTER(vp)]
        L.zkh_tensor_from_fr.argtypes = [vp, vp, u32, ctypes.POINTER(vp)]
        L.zkh_tensor_from_i32.argtypes = [vp, vp, u32, ctypes.POINTER(vp)]
        L.zkh_tensor_from_i64.argtypes = [vp, vp, u32, ctypes.POINTER(vp)]
        L.zkh_tensor_from_i32_device.argtypes = [vp, vp, u32, ctypes.POINTER(vp)]
        L.zkh_tensor_from_i64_device.argtypes = [vp, vp, u32, ctypes.POINTER(vp)]
        L.zkh_tensor_weights_i32.argtypes = [vp, vp, u32, u32, ctypes.POINTER(vp)]
        L.zkh_tensor_to_fr.argtypes = [vp, vp, vp]
        L.zkh_sum.argtypes = [vp, vp, vp]
        L.zkh_me.argtypes = [vp, vp, vp, u32, vp]
        L.zkh_me_static.argtypes = [vp, vp, vp, u32, vp]
        L.zkh_partial_me.argtypes = [vp, vp, vp, u32, u32, u32, ctypes.POINTER(vp)]
        L.zkh_multi_dim_me.argtypes = [vp, vp, vp, vp, vp, u32, vp]
        L.zkh_eq_table.argtypes = [vp, vp, u32, ctypes.POINTER(vp)]
        L.zkh_pad.argtypes = [vp, vp, vp, u32, vp, ctypes.POINTER(vp)]
        L.zkh_partial_me_window.argtypes = [vp, vp, vp, u32, u32, ctypes.POINTER(vp)]
        L.zkh_zkip.argtypes = [vp, vp, vp, vp, vp, u32, vp, vp]
        L.zkh_zkip_stacked.argtypes = [vp, vp, vp, vp, vp, u32, vp, u32, vp, u32, u32, vp, vp]
        L.zkh_fc_stacked_prove.argtypes = [vp, vp, vp, vp, vp, u32, u32, u32, u32, vp, vp, vp, vp, vp,
                                           vp, vp]
        L.zkh_rescale.argtypes = [vp, vp, u32, ctypes.POINTER(vp), ctypes.POINTER(vp)]
        L.zkh_matmul_i32.argtypes = [vp, vp, vp, vp, u32, u32, u32, ctypes.POINTER(vp)]
        L.zkh_fold.argtypes = [vp, vp, vp]
        L.zkh_axpy.argtypes = [vp, vp, vp, vp, ctypes.POINTER(vp)]
        L.zkh_hadamard.argtypes = [vp, vp, vp, ctypes.POINTER(vp)]
        L.zkh_transcript_init.argtypes = [vp, ctypes.c_char_p, ctypes.c_size_t]
        L.zkh_transcript_absorb.argtypes = [vp, ctypes.c_char_p, ctypes.c_size_t, vp, ctypes.c_size_t]
        L.zkh_transcript_challenge_fr.argtypes = [vp, vp]
        L.zkh_transcript_challenge_vec.argtypes = [vp, u32, vp]
        L.zkh_mm_prove.argtypes = [vp, vp, vp, vp, vp, u32, u32, u32, vp, vp, vp, vp, vp]
        L.zkh_lu_range_table.argtypes = [vp, i32, u32, u32, ctypes.POINTER(vp)]
        L.zkh_lu_prep.argtypes = [vp, vp, i32, u32, ctypes.POINTER(vp)]
        L.zkh_lu_mapping.argtypes = [vp, vp, i32, vp, ctypes.POINTER(vp), ctypes.POINTER(vp)]
        L.zkh_lu_inverse.argtypes = [vp, vp, vp, ctypes.POINTER(vp)]
        L.zkh_lu_range_inverse.argtypes = [vp, vp, i32, vp, vp, ctypes.POINTER(vp)]
        L.zkh_lu_tuple_inverse.argtypes = [vp, vp, i32, vp, vp, vp, vp, vp, ctypes.POINTER(vp), ctypes.POINTER(vp),
                                           ctypes.POINTER(vp)]
        L.zkh_lu_prove.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
        L.zkh_hp_prove.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, vp]
        L.zkh_hp_prove_eq.argtypes = [vp, vp, vp, vp, u32, vp, vp, vp, vp, vp]
        L.zkh_hp_prove_eq_claim.argtypes = [vp, vp, ctypes.c_char_p, vp, u32, vp, vp, vp, vp, vp, vp]
        L.zkh_hp_prove_claim.argtypes = [vp, vp, ctypes.c_char_p, vp, vp, vp, vp, vp, vp, vp]
        L.zkh_mm_prove_batch.argtypes = [vp, vp, u32]
        L.zkh_prof_enable.argtypes = [vp, ctypes.c_int]
        L.zkh_prof_get.argtypes = [vp, ctypes.c_char_p, vp, vp, vp]
        L.zkh_calib_fr_mul.argtypes = [vp, u32, ctypes.POINTER(ctypes.c_double)]
        L.zkh_prof_names.argtypes = [vp, ctypes.c_char_p, ctypes.c_size_t]
        L.zkh_g1_from_host.argtypes = [vp, vp, u32, ctypes.POINTER(vp)]
        L.zkh_g1_to_host.argtypes = [vp, vp, vp]
        L.zkh_g1_free.argtypes = [vp]
        L.zkh_g1_size.restype = u32
        L.zkh_g1_size.argtypes = [vp]
        L.zkh_commit.argtypes = [vp, vp, vp, ctypes.POINTER(vp)]
        L.zkh_g1_generator.restype = None
        L.zkh_g1_generator.argtypes = [vp]
        L.zkh_g1_mul.argtypes = [vp, vp, vp, ctypes.POINTER(vp)]
        L.zkh_g1_addmul.argtypes = [vp, vp, vp, vp, ctypes.POINTER(vp)]
        L.zkh_ipa_prove.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, vp]
        L.zkh_ipa_prove_batch.argtypes = [vp, ctypes.c_uint32, vp, vp, vp, vp, vp, vp, vp, vp]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _frs(a, n=None):
    a = np.ascontiguousarray(a, dtype=np.uint32).reshape(-1, 8)
    if n is not None:
        assert a.shape[0] == n
    return a


def ceil_log2(n):
    return 0 if n <= 1 else (int(n) - 1).bit_length()


# r, the BLS12-381 scalar field modulus, as 8 little-endian uint32 limbs (bls12-381.cu:4)
R_LIMBS = np.array([0x00000001, 0xFFFFFFFF, 0xFFFE5BFE, 0x53BDA402, 0x09A1D805, 0x3339D808,
                    0x299D7D48, 0x73EDA753], dtype=np.int64)


def ints_to_fr(v):
    """int_to_scalar / long_to_scalar on an integer array (fr-tensor.cu:701-717): v >= 0 -> v,
    v < 0 -> r - |v|, as an (n, 8) uint32 Fr array."""
    v = np.ascontiguousarray(v).reshape(-1).astype(np.int64)
    neg = v < 0
    mag = np.where(neg, -(v + 1), v).astype(np.uint64) + neg.astype(np.uint64)  # |v|, also for -2^63
    out = np.zeros((len(v), 8), dtype=np.int64)
    m = [(mag & np.uint64(0xFFFFFFFF)).astype(np.int64), (mag >> np.uint64(32)).astype(np.int64)]
    borrow = np.zeros(len(v), dtype=np.int64)
    for k in range(8):
        d = R_LIMBS[k] - (m[k] if k < 2 else 0) - borrow
        borrow = (d < 0).astype(np.int64)
        out[:, k] = np.where(neg, d + (borrow << 32), m[k] if k < 2 else 0)
    return out.astype(np.uint32)


# ---------------- transcript ----------------
def transcript(seed):
    st = np.zeros(32, dtype=np.uint8)
    b = seed.encode()
    lib().zkh_transcript_init(_p(st), b, len(b))
    return st


def absorb(st, label, data):
    lb = label.encode()
    buf = np.frombuffer(bytes(data), dtype=np.uint8).copy()
    lib().zkh_transcript_absorb(_p(st), lb, len(lb), _p(buf), len(buf))


def challenge(st):
    out = np.zeros(8, dtype=np.uint32)
    lib().zkh_transcript_challenge_fr(_p(st), _p(out))
    return out


def challenges(st, n):
    """fs_challenge_vec: n challenges in sequence, as an (n, 8) array (one C call)."""
    out = np.zeros((max(n, 1), 8), dtype=np.uint32)
    lib().zkh_transcript_challenge_vec(_p(st), n, _p(out))
    return out[:n]


class Tensor:
    def __init__(self, ctx, handle):
        self.ctx, self.h = ctx, handle

    def __del__(self):
        if getattr(self, "h", None) and lib is not None:
            try:
                lib().zkh_tensor_free(self.h)
            except Exception:
                pass
            self.h = None

    @property
    def n(self):
        return lib().zkh_tensor_size(self.h)

    @property
    def kind(self):
        return lib().zkh_tensor_kind(self.h)

    def to_fr(self):
        out = np.zeros((self.n, 8), dtype=np.uint32)
        self.ctx._chk(lib().zkh_tensor_to_fr(self.ctx.h, self.h, _p(out)))
        return out


def g1_generator():
    """the standard G1 generator as the reference stores it (36 uint32, Montgomery form)."""
    out = np.zeros(36, dtype=np.uint32)
    lib().zkh_g1_generator(_p(out))
    return out


class G1:
    """Device array of G1 points (the reference's 144-byte G1Jacobian_t)."""

    def __init__(self, ctx, handle):
        self.ctx, self.h = ctx, handle

    def __del__(self):
        if getattr(self, "h", None) and lib is not None:
            try:
                lib().zkh_g1_free(self.h)
            except Exception:
                pass
            self.h = None

    @property
    def n(self):
        return lib().zkh_g1_size(self.h)

    def to_host(self):
        out = np.zeros((self.n, 36), dtype=np.uint32)
        self.ctx._chk(lib().zkh_g1_to_host(self.ctx.h, self.h, _p(out)))
        return out


class Context:
    """One device context (one HIP stream).  Use one per host thread."""

    def __init__(self, device=0):
        h = ctypes.c_void_p()
        rc = lib().zkh_ctx_create(device, ctypes.byref(h))
        if rc:
            raise ZkhError(rc, "zkh_ctx_create(%d) failed" % device)
        self.h = h

    def close(self):
        if self.h:
            lib().zkh_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _chk(self, rc):
        if rc:
            raise ZkhError(rc, lib().zkh_last_error(self.h).decode(errors="replace"))

    def _new(self, fn, *args):
        h = ctypes.c_void_p()
        self._chk(fn(self.h, *args, ctypes.byref(h)))
        return Tensor(self, h)

    def sync(self):
        self._chk(lib().zkh_ctx_sync(self.h))

    # tensors
    def from_fr(self, a):
        a = _frs(a)
        return self._new(lib().zkh_tensor_from_fr, _p(a), a.shape[0])

    def from_i32(self, v):
        v = np.ascontiguousarray(v, dtype=np.int32).reshape(-1)
        return self._new(lib().zkh_tensor_from_i32, _p(v), v.size)

    def from_i64(self, v):
        v = np.ascontiguousarray(v, dtype=np.int64).reshape(-1)
        return self._new(lib().zkh_tensor_from_i64, _p(v), v.size)

    def from_i32_device(self, ptr, n):
        return self._new(lib().zkh_tensor_from_i32_device, ctypes.c_void_p(ptr), n)

    def from_i64_device(self, ptr, n):
        return self._new(lib().zkh_tensor_from_i64_device, ctypes.c_void_p(ptr), n)

    def weights_i32(self, W, IN, OUT):
        W = np.ascontiguousarray(W, dtype=np.int32).reshape(-1)
        assert W.size == IN * OUT
        return self._new(lib().zkh_tensor_weights_i32, _p(W), IN, OUT)

    # MLE primitives
    def calib_fr_mul(self, iters=256):
        """Montgomery products per second of the library's multiply on this device."""
        r = ctypes.c_double(0)
        self._chk(lib().zkh_calib_fr_mul(self.h, iters, ctypes.byref(r)))
        return r.value

    def sum(self, t):
        out = np.zeros(8, dtype=np.uint32)
        self._chk(lib().zkh_sum(self.h, t.h, _p(out)))
        return out

    def me(self, t, u):
        u = _frs(u)
        out = np.zeros(8, dtype=np.uint32)
        self._chk(lib().zkh_me(self.h, t.h, _p(u), u.shape[0], _p(out)))
        return out

    def me_static(self, t, u):
        """zkh_me without device allocation (static per-device scratch)."""
        u = _frs(u)
        out = np.zeros(8, dtype=np.uint32)
        self._chk(lib().zkh_me_static(self.h, t.h, _p(u), u.shape[0], _p(out)))
        return out

    def partial_me(self, t, u, cur_dim, window):
        u = _frs(u)
        return self._new(lib().zkh_partial_me, t.h, _p(u), u.shape[0], cur_dim, window)

    def multi_dim_me(self, t, us, shape):
        ks = np.array([len(u) for u in us], dtype=np.uint32)
        cat = np.concatenate([_frs(u) for u in us] + [np.zeros((1, 8), np.uint32)])
        shp = np.array(shape, dtype=np.uint32)
        out = np.zeros(8, dtype=np.uint32)
        self._chk(lib().zkh_multi_dim_me(self.h, t.h, _p(cat), _p(ks), _p(shp), len(shape), _p(out)))
        return out

    def eq_table(self, u):
        u = _frs(u)
        return self._new(lib().zkh_eq_table, _p(u), u.shape[0])

    def pad(self, t, shape, pad_val=None):
        shp = np.array(shape, dtype=np.uint32)
        pv = None if pad_val is None else _frs(pad_val, 1)
        return self._new(lib().zkh_pad, t.h, _p(shp), len(shape), _p(pv))

    def partial_me_window(self, t, u, window):
        u = _frs(u)
        return self._new(lib().zkh_partial_me_window, t.h, _p(u), u.shape[0], window)

    # inner-product sumchecks without a transcript (zkfc.cu)
    def zkip(self, claim, a, b, u):
        k = len(u)
        u = _frs(u) if k else np.zeros((1, 8), np.uint32)
        proof = np.zeros((3 * k + 1, 8), np.uint32)
        fin = np.zeros(8, np.uint32)
        self._chk(lib().zkh_zkip(self.h, _p(_frs(claim, 1)), a.h, b.h, _p(u), k, _p(proof), _p(fin)))
        return proof[:3 * k], fin

    def zkip_stacked(self, claim, A, B, uN, uD, vN, N, D):
        kN, kD = len(uN), len(uD)
        z = np.zeros((1, 8), np.uint32)
        uN, vN = (_frs(x) if kN else z for x in (uN, vN))
        uD = _frs(uD) if kD else z
        proof = np.zeros((3 * (kN + kD) + 1, 8), np.uint32)
        fin = np.zeros(8, np.uint32)
        self._chk(lib().zkh_zkip_stacked(self.h, _p(_frs(claim, 1)), A.h, B.h, _p(uN), kN, _p(uD), kD,
                                         _p(vN), N, D, _p(proof), _p(fin)))
        return proof[:3 * (kN + kD)], fin

    def fc_stacked_prove(self, X, W, Y, bias, num, B, IN, OUT, u_num, v_num, u_batch, u_input, u_output):
        z = np.zeros((1, 8), np.uint32)
        us = [_frs(x) if len(x) else z for x in (u_num, v_num, u_batch, u_input, u_output)]
        nr = len(u_num) + len(u_input)
        proof = np.zeros((3 * nr + 1, 8), np.uint32)
        claims = np.zeros((2, 8), np.uint32)
        self._chk(lib().zkh_fc_stacked_prove(self.h, X.h, W.h, Y.h, None if bias is None else bias.h, num, B,
                                             IN, OUT, *[_p(x) for x in us], _p(proof), _p(claims)))
        return proof[:3 * nr], claims

    def rescale(self, X, sf):
        q, r = ctypes.c_void_p(), ctypes.c_void_p()
        self._chk(lib().zkh_rescale(self.h, X.h, sf, ctypes.byref(q), ctypes.byref(r)))
        return Tensor(self, q), Tensor(self, r)

    def matmul_i32(self, X, W, B, IN, OUT, bias=None):
        """Y = X W (+ bias), exact int64 (zkh_matmul_i32); X, W int32 tensors (W row-major or
        registered weights), bias None or an int tensor of OUT entries."""
        y = ctypes.c_void_p()
        self._chk(lib().zkh_matmul_i32(self.h, X.h, W.h, bias.h if bias is not None else None, B, IN, OUT,
                                       ctypes.byref(y)))
        return Tensor(self, y)

    def g1_from_host(self, pts):
        """(n, 36) uint32 points -> device G1 array."""
        pts = np.ascontiguousarray(pts, dtype=np.uint32).reshape(-1, 36)
        h = ctypes.c_void_p()
        self._chk(lib().zkh_g1_from_host(self.h, _p(pts), pts.shape[0], ctypes.byref(h)))
        return G1(self, h)

    def g1_mul(self, base, t):
        """out[i] = base[i % base.n] * t[i] (G1Jacobian_mul)."""
        h = ctypes.c_void_p()
        self._chk(lib().zkh_g1_mul(self.h, base.h, t.h, ctypes.byref(h)))
        return G1(self, h)

    def g1_addmul(self, a, s, b):
        """out[i] = b[i] + a[i] * s, s one plain scalar (8 uint32): hb_addmul, mul_first false."""
        sc = np.ascontiguousarray(s, dtype=np.uint32).reshape(8)
        h = ctypes.c_void_p()
        self._chk(lib().zkh_g1_addmul(self.h, a.h, _p(sc), b.h, ctypes.byref(h)))
        return G1(self, h)

    def ipa_prove(self, st, a, b, g, Q):
        """ipa_prove over n = g.n: returns {"L": (log n, 36), "R": (log n, 36), "a_final": (8,)};
        st (32 uint8) is advanced in place."""
        n = g.n
        rounds = max(n.bit_length() - 1, 0)
        L = np.zeros((max(rounds, 1), 36), np.uint32)
        R = np.zeros((max(rounds, 1), 36), np.uint32)
        af = np.zeros(8, np.uint32)
        Q = np.ascontiguousarray(Q, np.uint32)
        self._chk(lib().zkh_ipa_prove(self.h, _p(st), a.h, b.h, g.h, _p(Q), _p(L), _p(R), _p(af)))
        return {"L": L[:rounds], "R": R[:rounds], "a_final": af}

    def ipa_prove_batch(self, jobs):
        """zkh_ipa_prove_batch over jobs [(st, a, b, g, Q), ...]: one ipa_prove result per job, as
        ipa_prove returns it; each st (32 uint8) is advanced in place."""
        nj = len(jobs)
        arr = lambda vals: (ctypes.c_void_p * nj)(*vals)
        outs, keep = [], []
        for st, a, b, g, Q in jobs:
            rounds = max(g.n.bit_length() - 1, 0)
            o = {"L": np.zeros((max(rounds, 1), 36), np.uint32), "R": np.zeros((max(rounds, 1), 36), np.uint32),
                 "a_final": np.zeros(8, np.uint32), "rounds": rounds}
            keep.append(np.ascontiguousarray(Q, np.uint32))
            outs.append(o)
        self._chk(lib().zkh_ipa_prove_batch(
            self.h, nj, arr([_p(j[0]) for j in jobs]), arr([j[1].h for j in jobs]), arr([j[2].h for j in jobs]),
            arr([j[3].h for j in jobs]), arr([_p(q) for q in keep]), arr([_p(o["L"]) for o in outs]),
            arr([_p(o["R"]) for o in outs]), arr([_p(o["a_final"]) for o in outs])))
        return [{"L": o["L"][:o["rounds"]], "R": o["R"][:o["rounds"]], "a_final": o["a_final"]} for o in outs]

    def commit(self, gens, t):
        """Commitment::commit: rows of n = gens.n scalars of tensor t -> one point per row."""
        h = ctypes.c_void_p()
        self._chk(lib().zkh_commit(self.h, gens.h, t.h, ctypes.byref(h)))
        return G1(self, h)

    def fold(self, t, v):
        v = _frs(v, 1)
        self._chk(lib().zkh_fold(self.h, t.h, _p(v)))

    def axpy(self, a, c, b):
        c = _frs(c, 1)
        return self._new(lib().zkh_axpy, a.h, _p(c), b.h)

    def hadamard(self, a, b):
        return self._new(lib().zkh_hadamard, a.h, b.h)

    # provers
    def mm_prove(self, st, X, W, Y, B, IN, OUT):
        L, lb, lo = ceil_log2(IN), ceil_log2(B), ceil_log2(OUT)
        ev = np.zeros((3 * L + 1, 8), np.uint32)
        cl = np.zeros((3, 8), np.uint32)
        ub, uo, ui = (np.zeros((x + 1, 8), np.uint32) for x in (lb, lo, L))
        self._chk(lib().zkh_mm_prove(self.h, _p(st), X.h, W.h, Y.h, B, IN, OUT, _p(ev), _p(cl),
                                     _p(ub), _p(uo), _p(ui)))
        return dict(ev=ev[:3 * L], claims=cl, u_batch=ub[:lb], u_output=uo[:lo], u_input=ui[:L])

    def mm_prove_batch(self, items):
        """items: list of (transcript, X, W, Y, B, IN, OUT); returns (outputs, statuses);
        raises on any failing job (statuses still filled)."""
        b = MmBatch(self, items)
        status = b.run(check=False)
        outs = [dict(o) for o in b.outs]
        self._chk(b.rc)
        return outs, status

    def range_table(self, low, length, N):
        return self._new(lib().zkh_lu_range_table, low, length, N)

    def lu_prep(self, S, low, N):
        return self._new(lib().zkh_lu_prep, S.h, low, N)

    def lu_mapping(self, S, low, mapped):
        so, m = ctypes.c_void_p(), ctypes.c_void_p()
        self._chk(lib().zkh_lu_mapping(self.h, S.h, low, mapped.h, ctypes.byref(so), ctypes.byref(m)))
        return Tensor(self, so), Tensor(self, m)

    def lu_inverse(self, S, beta):
        beta = _frs(beta, 1)
        return self._new(lib().zkh_lu_inverse, S.h, _p(beta))

    def lu_range_inverse(self, S, low, T, beta):
        """1/(S + beta) as lu_inverse, read off the table inverse of T (a range lookup); the
        table inverse goes on to the lu_prove on T and beta."""
        beta = _frs(beta, 1)
        return self._new(lib().zkh_lu_range_inverse, S.h, int(low), T.h, _p(beta))

    def lu_tuple_inverse(self, G, low, T, mapped, r, beta, S=None):
        """(comb, T_comb, A) = (G + r mapped[G - low], T + r mapped, 1/(comb + beta)) for int32
        G, T, mapped; the table inverse goes on to the lu_prove on T_comb and beta.  S: the
        lu_mapping output for this G (comb then reads it in order)."""
        r, beta = _frs(r, 1), _frs(beta, 1)
        hs = [ctypes.c_void_p() for _ in range(3)]
        self._chk(lib().zkh_lu_tuple_inverse(self.h, G.h, int(low), T.h, mapped.h, S.h if S is not None else None,
                                             _p(r), _p(beta), *[ctypes.byref(h) for h in hs]))
        return tuple(Tensor(self, h) for h in hs)

    def lu_prove(self, st, A, S, T, m, alpha, beta, u):
        D = A.n
        logD = ceil_log2(D)
        alpha, beta = _frs(alpha, 1), _frs(beta, 1)
        u = _frs(u) if logD else np.zeros((1, 8), np.uint32)
        ev = np.zeros((4 * logD + 1, 8), np.uint32)
        term = np.zeros((5, 8), np.uint32)
        ws = np.zeros((logD + 1, 8), np.uint32)
        self._chk(lib().zkh_lu_prove(self.h, _p(st), A.h, S.h, T.h, m.h, _p(alpha), _p(beta), _p(u),
                                     _p(ev), _p(term), _p(ws)))
        return dict(ev=ev[:4 * logD], term=term, ws=ws[:logD])

    def hp_prove(self, st, claim, E, S, U):
        k = ceil_log2(S.n)
        claim = _frs(claim, 1)
        ev = np.zeros((4 * k + 1, 8), np.uint32)
        term = np.zeros((3, 8), np.uint32)
        ws = np.zeros((k + 1, 8), np.uint32)
        self._chk(lib().zkh_hp_prove(self.h, _p(st), _p(claim), E.h, S.h, U.h, _p(ev), _p(term), _p(ws)))
        return dict(ev=ev[:4 * k], term=term, ws=ws[:k])

    def hp_prove_eq(self, st, claim, u, S, U):
        u = _frs(u)
        k = u.shape[0]
        claim = _frs(claim, 1)
        ev = np.zeros((4 * k + 1, 8), np.uint32)
        term = np.zeros((3, 8), np.uint32)
        ws = np.zeros((k + 1, 8), np.uint32)
        self._chk(lib().zkh_hp_prove_eq(self.h, _p(st), _p(claim), _p(u), k, S.h, U.h, _p(ev),
                                        _p(term), _p(ws)))
        return dict(ev=ev[:4 * k], term=term, ws=ws[:k])

    def hp_prove_claim(self, st, label, E, S, U):
        """claim = sum E[i] S[i] U[i] absorbed under label, then hp_prove, in one call (the claim
        from the first round's sums; zkob_rope.cu:230-238)."""
        k = ceil_log2(S.n)
        claim = np.zeros(8, np.uint32)
        ev = np.zeros((4 * k + 1, 8), np.uint32)
        term = np.zeros((3, 8), np.uint32)
        ws = np.zeros((k + 1, 8), np.uint32)
        self._chk(lib().zkh_hp_prove_claim(self.h, _p(st), label.encode(), E.h, S.h, U.h, _p(claim), _p(ev),
                                           _p(term), _p(ws)))
        return dict(claim=claim, ev=ev[:4 * k], term=term, ws=ws[:k])

    def hp_prove_eq_claim(self, st, label, u, S, U):
        """claim = sum eq(u, i) S[i] U[i] absorbed under label, then hp_prove_eq, in one call
        (the claim from the first round's sums; zkob_glu.cu:231-247)."""
        u = _frs(u)
        k = u.shape[0]
        claim = np.zeros(8, np.uint32)
        ev = np.zeros((4 * k + 1, 8), np.uint32)
        term = np.zeros((3, 8), np.uint32)
        ws = np.zeros((k + 1, 8), np.uint32)
        self._chk(lib().zkh_hp_prove_eq_claim(self.h, _p(st), label.encode(), _p(u), k, S.h, U.h, _p(claim),
                                              _p(ev), _p(term), _p(ws)))
        return dict(claim=claim, ev=ev[:4 * k], term=term, ws=ws[:k])


class MmBatch:
    """A prepared zkh_mm_prove_batch call (the zkob_fc prove runs of several matmuls): the
    zkh_mm_job array and the output buffers are built once, so run() is one C call that
    proves every job again from the transcripts' current states."""

    def __init__(self, ctx, items):
        self.ctx = ctx
        n = len(items)
        self.arr = (MmJob * n)()
        self.outs = []
        self._keep = items
        for k, (st, X, W, Y, B, IN, OUT) in enumerate(items):
            L, lb, lo = ceil_log2(IN), ceil_log2(B), ceil_log2(OUT)
            full = dict(ev=np.zeros((3 * L + 1, 8), np.uint32), claims=np.zeros((3, 8), np.uint32),
                        u_batch=np.zeros((lb + 1, 8), np.uint32), u_output=np.zeros((lo + 1, 8), np.uint32),
                        u_input=np.zeros((L + 1, 8), np.uint32))
            self.arr[k] = MmJob(X.h, W.h, Y.h, B, IN, OUT, st.ctypes.data, _p(full["ev"]), _p(full["claims"]),
                                _p(full["u_batch"]), _p(full["u_output"]), _p(full["u_input"]), 0)
            self.outs.append(dict(ev=full["ev"][:3 * L], claims=full["claims"], u_batch=full["u_batch"][:lb],
                                  u_output=full["u_output"][:lo], u_input=full["u_input"][:L]))
        self._ptr = ctypes.cast(self.arr, ctypes.c_void_p)
        self.rc = 0

    def run(self, check=True):
        self.rc = lib().zkh_mm_prove_batch(self.ctx.h, self._ptr, len(self.arr))
        if check:
            self.ctx._chk(self.rc)
        return [self.arr[k].status for k in range(len(self.arr))]
