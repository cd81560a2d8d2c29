"""The zkob_fc-compatible driver zk-hillclimb_amd/zkh_fc (zkob_fc.cu:1207-1330,
zkob_serve.cuh): `prove` in the reference's plain mode must write the same obligation files
as the reference, byte for byte -- com_X.bin, com_Y.bin, dims.bin, sumcheck.bin, ipa_W.bin,
ipa_X.bin, ipa_Y.bin and the int64 Y -- which this test restates from the C oracle: the
commitments (commit_pippenger), the transcript absorbs (zkob_fc.cu:254-258), the matmul
sumcheck (:259-440), write_sumcheck (:105-112), the IPA openings in the order W, X, Y
(:473-483) and write_ipa (vrf_common.cuh:284-289).  Shapes: the reference's own selftest
cases (zkob_fc.cu:1246-1248) and a non-power-of-two B.  `commit` (weight registration) and
`serve` (ZKW-READY / ZKW-RC) are covered too.  zkh_rescale (zkob_rescale.cu:70-197) is
checked the same way: rescaling witness, multiplicities, five commitments, the logUp proof
(write_lookup, zkob_lookup.cuh:80-87) and the openings of A, rem and m (open_prove,
zkob_lookup.cuh:116-127), on the reference's rescale selftest shapes (zkob_rescale.cu:539-541)."""
import os
import struct
import subprocess

import numpy as np
import pytest

from oracle import coracle as C
from oracle import pyg1 as G
from oracle import pyref as P

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "zk-hillclimb_amd", "zkh_fc")
RESCALE = os.path.join(ROOT, "zk-hillclimb_amd", "zkh_rescale")
BASE = G.aff_to_jac((G.GX, G.GY))


@pytest.fixture(autouse=True)
def _convention_crosschecks(monkeypatch):
    """The drivers run with ZKH_XCHECK=1: every proof also checks its folded terminals against
    multi_dim_me at the opening point, as the reference's drivers do."""
    monkeypatch.setenv("ZKH_XCHECK", "1")


def points(seed, n):
    rng = np.random.default_rng(seed)
    out = np.zeros((n, 36), np.uint32)
    for i in range(n):
        k = int.from_bytes(rng.bytes(32), "little") % P.R
        out[i] = C.g1_mul(BASE, np.array(P.to_limbs(k), np.uint32))
    return out


def pow2(n):
    return 1 << max(n - 1, 0).bit_length()


def padded(M):
    r, c = M.shape
    out = np.zeros((pow2(r), pow2(c)), np.int64)
    out[:r, :c] = M
    return out


def pod(arr, words):
    a = np.ascontiguousarray(arr, np.uint32).reshape(-1, words)
    return struct.pack("<I", a.shape[0]) + a.tobytes()


def expected(seed, X, W, gin, gout, Q):
    """the obligation directory's files, restated from the oracle"""
    B, IN = X.shape
    OUT = W.shape[1]
    Y = X.astype(np.int64) @ W.astype(np.int64)
    Xp, Wp, Yp = padded(X), padded(W), padded(Y)
    files = {}
    coms = {}
    for name, T, g in (("X", Xp, gin), ("W", Wp, gout), ("Y", Yp, gout)):
        rc, c = C.g1_commit(g, C.ints_to_fr(T.reshape(-1)), T.shape[1])
        assert rc == 0
        coms[name] = c
    files["com_X.bin"] = coms["X"].tobytes()
    files["com_Y.bin"] = coms["Y"].tobytes()
    files["dims.bin"] = struct.pack("<III", B, IN, OUT)
    st = C.tr_init(seed)
    for lab, v in (("B", B), ("IN", IN), ("OUT", OUT)):
        C.tr_absorb(st, lab, struct.pack("<I", v))
    for lab in ("X", "W", "Y"):
        C.tr_absorb(st, "com_" + lab, coms[lab].tobytes())
    rc, mm = C.mm_prove(st, X, W, Y, B, IN, OUT)
    assert rc == 0
    files["sumcheck.bin"] = pod(mm["ev"], 8) + mm["claims"].tobytes()
    bW = C.build_eq(mm["u_output"])
    for name, T, u, b, g, win in (("W", Wp, mm["u_input"], bW, gout, Wp.shape[1]),
                                  ("X", Xp, mm["u_batch"], C.build_eq(mm["u_input"]), gin, Xp.shape[1]),
                                  ("Y", Yp, mm["u_batch"], bW, gout, Yp.shape[1])):
        rc, a = C.partial_me_window(C.ints_to_fr(T.reshape(-1)), u, win)
        assert rc == 0 and len(a) == win
        rc, L, R, af = C.ipa_prove(st, a, b, g, Q, win)
        assert rc == 0
        files["ipa_%s.bin" % name] = pod(L, 36) + pod(R, 36) + af.tobytes()
    return files, Y


def write_inputs(d, X, W, gin, gout, q):
    paths = {}
    for name, arr in (("X.bin", X.astype(np.int32)), ("W.bin", W.astype(np.int32)), ("gen_in.bin", gin),
                      ("gen_out.bin", gout), ("q.bin", q)):
        paths[name] = os.path.join(d, name)
        np.ascontiguousarray(arr).tofile(paths[name])
    return paths


@pytest.mark.parametrize("B,IN,OUT", [(4, 6, 3), (8, 8, 8), (16, 12, 5), (3, 16, 2)])
def test_prove_files_match_reference_format(tmp_path, B, IN, OUT):
    rng = np.random.default_rng(B * 100 + IN * 10 + OUT)
    X = rng.integers(-2**15, 2**15, size=(B, IN)).astype(np.int32)
    W = rng.integers(-229376, 229377, size=(IN, OUT)).astype(np.int32)
    gin, gout, q = points(1, pow2(IN)), points(2, pow2(OUT)), points(3, 2)
    p = write_inputs(str(tmp_path), X, W, gin, gout, q)
    ob = tmp_path / "ob"
    ob.mkdir()
    yout = str(tmp_path / "Y.i64")
    seed = "run7:layer0.q_proj.matmul"
    r = subprocess.run([CLI, "prove", str(ob), seed, p["X.bin"], p["W.bin"], str(B), str(IN), str(OUT),
                        p["gen_in.bin"], p["gen_out.bin"], p["q.bin"], yout], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    assert "PROVED matmul obligation" in r.stdout
    want, Y = expected(seed, X, W, gin, gout, q[0])
    for name, data in want.items():
        assert (ob / name).read_bytes() == data, name
    assert open(yout, "rb").read() == Y.astype(np.int64).tobytes()


def test_commit_registration_and_errors(tmp_path):
    rng = np.random.default_rng(5)
    IN, OUT = 6, 5
    W = rng.integers(-1000, 1000, size=(IN, OUT)).astype(np.int32)
    gout = points(4, pow2(OUT))
    p = write_inputs(str(tmp_path), W[:1], W, gout, gout, gout[:1])
    out = str(tmp_path / "com_W.bin")
    r = subprocess.run([CLI, "commit", p["W.bin"], str(IN), str(OUT), p["gen_out.bin"], out],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    rc, want = C.g1_commit(gout, C.ints_to_fr(padded(W).reshape(-1)), pow2(OUT))
    assert open(out, "rb").read() == want.tobytes()
    # a generator file of the wrong size, a short input file, an unsupported mode flag
    r = subprocess.run([CLI, "commit", p["W.bin"], str(IN), str(OUT * 2), p["gen_out.bin"], out],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 1
    r = subprocess.run([CLI, "commit", p["X.bin"], str(IN), str(OUT), p["gen_out.bin"], out],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 1 and "short read" in r.stderr
    r = subprocess.run([CLI, "prove", "x", "y", "--claims", "a", "b", "c"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2


def test_serve_mode(tmp_path):
    rng = np.random.default_rng(6)
    B, IN, OUT = 4, 6, 3
    X = rng.integers(-100, 100, size=(B, IN)).astype(np.int32)
    W = rng.integers(-100, 100, size=(IN, OUT)).astype(np.int32)
    gin, gout, q = points(7, pow2(IN)), points(8, pow2(OUT)), points(9, 1)
    p = write_inputs(str(tmp_path), X, W, gin, gout, q)
    obs = [tmp_path / "a", tmp_path / "b"]
    for o in obs:
        o.mkdir()
    lines = ["prove %s s%d %s %s %d %d %d %s %s %s" % (o, i, p["X.bin"], p["W.bin"], B, IN, OUT, p["gen_in.bin"],
                                                       p["gen_out.bin"], p["q.bin"]) for i, o in enumerate(obs)]
    lines.append("prove %s s --wpriv a b" % obs[0])
    r = subprocess.run([CLI, "serve"], input="\n".join(lines) + "\n", capture_output=True, text=True, timeout=120)
    assert r.returncode == 0
    out = r.stdout.splitlines()
    assert out[0] == "ZKW-READY"
    rcs = [l for l in out if l.startswith("ZKW-RC ")]
    assert rcs == ["ZKW-RC 0", "ZKW-RC 0", "ZKW-RC 3"]
    for i, o in enumerate(obs):
        want, _ = expected("s%d" % i, X, W, gin, gout, q[0])
        for name, data in want.items():
            assert (o / name).read_bytes() == data, (i, name)


def log2(n):
    return n.bit_length() - 1


def expected_rescale(seed, X, B, Cc, log_sf, gen, Q):
    sf = 1 << log_sf
    Bp, Cp = pow2(B), pow2(Cc)
    D, N = Bp * Cp, sf
    logD, n1, logG = log2(D), log2(D // N), log2(Cp)
    rc, q, rem = C.rescale(X.reshape(-1), sf)
    assert rc == 0
    Xp, Xrp, remp = padded(X.reshape(B, Cc)), padded(q.reshape(B, Cc)), padded(rem.reshape(B, Cc))
    low = -(sf >> 1)
    T = C.range_table(low, sf, N)
    S = C.ints_to_fr(remp.reshape(-1))
    rc, m = C.lu_prep(S, low, N)
    assert rc == 0
    files, coms = {}, {}
    for name, t in (("X", C.ints_to_fr(Xp.reshape(-1))), ("Xr", C.ints_to_fr(Xrp.reshape(-1))), ("rem", S), ("m", m)):
        rc, coms[name] = C.g1_commit(gen, t, Cp)
        files["com_%s.bin" % name] = coms[name].tobytes()
    files["dims.bin"] = struct.pack("<III", B, Cc, log_sf)
    st = C.tr_init(seed)
    for lab, v in (("B", B), ("C", Cc), ("LOG_SF", log_sf)):
        C.tr_absorb(st, lab, struct.pack("<I", v))
    for name in ("X", "Xr", "rem", "m"):
        C.tr_absorb(st, "com_" + name, coms[name].tobytes())
    beta = C.tr_challenge_fr(st)
    A = C.lu_inverse(S, beta)
    rc, comA = C.g1_commit(gen, A, Cp)
    files["com_A.bin"] = comA.tobytes()
    C.tr_absorb(st, "com_A", comA.tobytes())
    alpha = C.tr_challenge_fr(st)
    u = np.array([C.tr_challenge_fr(st) for _ in range(logD)])
    rc, lk = C.lu_prove(st, A, S, T, m, alpha, beta, u)
    assert rc == 0
    files["lookup.bin"] = pod(lk["ev"], 8) + lk["term"][0].tobytes() + lk["term"][1].tobytes() + lk["term"][4].tobytes()
    u_pt = lk["ws"][::-1]
    for name, t, pt in (("A", A, u_pt), ("rem", S, u_pt), ("m", m, u_pt[:logD - n1])):
        a = t if len(pt) == logG else C.partial_me_window(t, pt[logG:], Cp)[1]
        rc, L, R, af = C.ipa_prove(st, a, C.build_eq(pt[:logG]), gen, Q, Cp)
        assert rc == 0
        files["ipa_%s.bin" % name] = pod(L, 36) + pod(R, 36) + af.tobytes()
    return files, q


@pytest.mark.parametrize("B,Cc,log_sf", [(8, 4, 4), (4, 16, 4), (8, 6, 6)])
def test_rescale_prove_files_match_reference_format(tmp_path, B, Cc, log_sf):
    rng = np.random.default_rng(B * 100 + Cc * 10 + log_sf)
    X = rng.integers(-(1 << 12), 1 << 12, size=(B, Cc)).astype(np.int64) * 37
    gen, q = points(11, pow2(Cc)), points(12, 1)
    xp, gp, qp = (str(tmp_path / n) for n in ("X.i64", "gen.bin", "q.bin"))
    X.tofile(xp)
    gen.tofile(gp)
    q.tofile(qp)
    ob = tmp_path / "ob"
    ob.mkdir()
    xr = str(tmp_path / "Xr.i32")
    seed = "selftest:rescale"
    r = subprocess.run([RESCALE, "prove", str(ob), seed, xp, str(B), str(Cc), str(log_sf), gp, qp, xr],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "PROVED rescaling obligation" in r.stdout
    want, Xr = expected_rescale(seed, X, B, Cc, log_sf, gen, q[0])
    for name, data in want.items():
        assert (ob / name).read_bytes() == data, name
    assert open(xr, "rb").read() == Xr.astype(np.int32).tobytes()
    # a layout the reference rejects (N > D) and a generator of the wrong size
    r = subprocess.run([RESCALE, "prove", str(ob), seed, xp, str(B), str(Cc), str(10), gp, qp],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 1


GLU = os.path.join(ROOT, "zk-hillclimb_amd", "zkh_glu")


def fr_of(vals):
    return C.ints_to_fr([int(v) % P.R for v in np.asarray(vals, dtype=object).reshape(-1)])


def open_ipa(st, t, pt, Cp, gen, Q):
    logG = log2(Cp)
    a = t if len(pt) == logG else C.partial_me_window(t, pt[logG:], Cp)[1]
    rc, L, R, af = C.ipa_prove(st, a, C.build_eq(pt[:logG]), gen, Q, Cp)
    assert rc == 0
    return pod(L, 36) + pod(R, 36) + af.tobytes()


def expected_glu(seed, Gm, Um, low, ln, mapped, gen, Q):
    """zkob_glu.cu:86-247 (plain mode) restated from the oracle and the definitions of the
    mapping lookup (S = mapped[G - low], m = counts)"""
    B, Cc = Gm.shape
    Bp, Cp = pow2(B), pow2(Cc)
    D, N = Bp * Cp, ln
    logD, n1 = log2(D), log2(D // N)
    Gp, Up = padded(Gm), padded(Um)
    idx = (Gp - low).reshape(-1)
    S = np.asarray(mapped, np.int64)[idx].reshape(Gp.shape)
    m = np.bincount(idx, minlength=N).astype(np.int64)
    H = S * Up
    files, coms = {}, {}
    for name, t in (("G", Gp), ("S", S), ("U", Up), ("H", H), ("m", m)):
        rc, coms[name] = C.g1_commit(gen, fr_of(t), Cp)
        files["com_%s.bin" % name] = coms[name].tobytes()
    files["dims.bin"] = struct.pack("<iiii", B, Cc, low, ln)
    st = C.tr_init(seed)
    for lab, v in (("B", B), ("C", Cc), ("LOW", low & 0xFFFFFFFF), ("LEN", ln)):
        C.tr_absorb(st, lab, struct.pack("<I", v))
    for name in ("G", "S", "U", "H", "m"):
        C.tr_absorb(st, "com_" + name, coms[name].tobytes())
    r = P.from_limbs(C.tr_challenge_fr(st))
    beta = C.tr_challenge_fr(st)
    comb = fr_of([(int(g) + r * int(s)) % P.R for g, s in zip(Gp.reshape(-1), S.reshape(-1))])
    Tcomb = fr_of([(low + i + r * int(mapped[i])) % P.R for i in range(N)])
    A = C.lu_inverse(comb, beta)
    rc, comA = C.g1_commit(gen, A, Cp)
    files["com_A.bin"] = comA.tobytes()
    C.tr_absorb(st, "com_A", comA.tobytes())
    alpha = C.tr_challenge_fr(st)
    u = np.array([C.tr_challenge_fr(st) for _ in range(logD)])
    rc, lk = C.lu_prove(st, A, comb, Tcomb, fr_of(m), alpha, beta, u)
    assert rc == 0
    files["lookup.bin"] = pod(lk["ev"], 8) + lk["term"][0].tobytes() + lk["term"][1].tobytes() + lk["term"][4].tobytes()
    u_pt = lk["ws"][::-1]
    files["ipa_A.bin"] = open_ipa(st, A, u_pt, Cp, gen, Q)
    files["ipa_comb.bin"] = open_ipa(st, comb, u_pt, Cp, gen, Q)
    files["ipa_m.bin"] = open_ipa(st, fr_of(m), u_pt[:logD - n1], Cp, gen, Q)
    uh = np.array([C.tr_challenge_fr(st) for _ in range(logD)])
    rc, claimH = C.me(fr_of(H), uh)
    assert rc == 0
    C.tr_absorb(st, "claim_H", claimH.tobytes())
    rc, hp = C.hp_prove(st, claimH, C.build_eq(uh), fr_of(S), fr_of(Up))
    assert rc == 0
    C.tr_absorb(st, "S_f2", hp["term"][0].tobytes())
    C.tr_absorb(st, "U_f2", hp["term"][1].tobytes())
    files["hp.bin"] = claimH.tobytes() + pod(hp["ev"], 8) + hp["term"][0].tobytes() + hp["term"][1].tobytes()
    u_pt2 = hp["ws"][::-1]
    files["ipa_H.bin"] = open_ipa(st, fr_of(H), uh, Cp, gen, Q)
    files["ipa_S.bin"] = open_ipa(st, fr_of(S), u_pt2, Cp, gen, Q)
    files["ipa_U.bin"] = open_ipa(st, fr_of(Up), u_pt2, Cp, gen, Q)
    return files, H[:B, :Cc]


@pytest.mark.parametrize("B,Cc,low,ln", [(8, 4, -8, 16), (4, 4, -8, 16), (8, 6, -16, 32)])
def test_glu_prove_files_match_reference_format(tmp_path, B, Cc, low, ln):
    rng = np.random.default_rng(B * 1000 + Cc * 10 + ln)
    mapped = np.array([(i + low) ** 2 for i in range(ln)], np.int32)  # the reference selftest's table
    Gm = rng.integers(low, low + ln, size=(B, Cc)).astype(np.int32)
    Um = rng.integers(-300, 300, size=(B, Cc)).astype(np.int32)
    gen, q = points(21, pow2(Cc)), points(22, 1)
    paths = {}
    for name, arr in (("G", Gm), ("U", Um), ("map", mapped), ("gen", gen), ("q", q)):
        paths[name] = str(tmp_path / (name + ".bin"))
        np.ascontiguousarray(arr).tofile(paths[name])
    ob = tmp_path / "ob"
    ob.mkdir()
    hout = str(tmp_path / "H.i64")
    seed = "selftest:glu"
    r = subprocess.run([GLU, "prove", str(ob), seed, paths["G"], paths["U"], str(B), str(Cc), str(low), str(ln),
                        paths["map"], paths["gen"], paths["q"], hout], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "PROVED swiglu obligation" in r.stdout
    want, H = expected_glu(seed, Gm, Um, low, ln, mapped, gen, q[0])
    for name, data in want.items():
        assert (ob / name).read_bytes() == data, name
    assert open(hout, "rb").read() == H.astype(np.int64).tobytes()
    # a table without (0, 0) is refused, as load_mapped refuses it
    bad = mapped.copy()
    bad[-low] = 5
    bad.tofile(paths["map"])
    r = subprocess.run([GLU, "prove", str(ob), seed, paths["G"], paths["U"], str(B), str(Cc), str(low), str(ln),
                        paths["map"], paths["gen"], paths["q"]], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1 and "mapped(0)" in r.stderr


ROPE = os.path.join(ROOT, "zk-hillclimb_amd", "zkh_rope")


def ints_of(fr):
    return [P.from_limbs(x) for x in np.asarray(fr, np.uint32).reshape(-1, 8)]


def expected_rope(seed, Th, HD, cosT, sinT, gen, Q):
    """zkob_rope.cu prove (plain mode) restated: weights and the flipped T by their
    definitions, then the oracle for commitments, MLEs, both Hadamard sumchecks and IPAs"""
    B, Cc = Th.shape
    Cp = pow2(Cc)
    logCp, logD = log2(Cp), log2(B) + log2(Cp)
    flipv, fb = HD // 2, log2(HD) - 1
    W1 = np.zeros((B, Cp), np.int64)
    W2 = np.zeros((B, Cp), np.int64)
    Tg = np.zeros((B, Cp), np.int64)
    for t in range(B):
        for e in range(Cc):
            W1[t, e] = cosT[t, e % HD]
            W2[t, e] = (1 if e & flipv else -1) * sinT[t, e % HD]
            Tg[t, e] = Th[t, e]
    Txg = Tg[:, [e ^ flipv for e in range(Cp)]]
    Y = Tg * W1 + Txg * W2
    T_fr, Tx_fr, Y_fr, ones = fr_of(Tg), fr_of(Txg), fr_of(Y), fr_of(np.ones(B * Cp, np.int64))
    files = {}
    rc, comT = C.g1_commit(gen, T_fr, Cp)
    rc, comY = C.g1_commit(gen, Y_fr, Cp)
    files["com_T.bin"], files["com_Y64.bin"] = comT.tobytes(), comY.tobytes()
    files["dims.bin"] = struct.pack("<IIII", B, Cc, HD, 16)
    st = C.tr_init(seed)
    for lab, v in (("B", B), ("C", Cc), ("HD", HD), ("SCALE_R", 16)):
        C.tr_absorb(st, lab, struct.pack("<I", v))
    C.tr_absorb(st, "com_T", comT.tobytes())
    C.tr_absorb(st, "com_Y64", comY.tobytes())
    u = np.array([C.tr_challenge_fr(st) for _ in range(logD)])
    rc, ev = C.me(Y_fr, u)
    C.tr_absorb(st, "ev", ev.tobytes())
    files["ev.bin"] = ev.tobytes()
    Eu = ints_of(C.build_eq(u))
    for k, (W, S_fr, S_int) in enumerate(((W1, T_fr, Tg), (W2, Tx_fr, Txg)), start=1):
        E = [e * int(w) % P.R for e, w in zip(Eu, W.reshape(-1))]
        c = sum(e * int(s) for e, s in zip(E, S_int.reshape(-1))) % P.R
        cl = np.array(P.to_limbs(c), np.uint32)
        C.tr_absorb(st, "c%d" % k, cl.tobytes())
        rc, hp = C.hp_prove(st, cl, fr_of(E), S_fr, ones)
        assert rc == 0
        C.tr_absorb(st, "S_f2", hp["term"][0].tobytes())
        C.tr_absorb(st, "U_f2", hp["term"][1].tobytes())
        files["hp%d.bin" % k] = cl.tobytes() + pod(hp["ev"], 8) + hp["term"][0].tobytes() + hp["term"][1].tobytes()
        pt = hp["ws"][::-1].copy()
        if k == 2:
            pt[fb] = P.to_limbs((1 - P.from_limbs(pt[fb])) % P.R)
        files["ipa_T%d.bin" % k] = open_ipa(st, T_fr, pt, Cp, gen, Q)
    files["ipa_Y.bin"] = open_ipa(st, Y_fr, u, Cp, gen, Q)
    return files, Y[:, :Cc]


@pytest.mark.parametrize("B,Cc,HD", [(8, 6, 2), (4, 8, 4), (16, 12, 4)])
def test_rope_prove_files_match_reference_format(tmp_path, B, Cc, HD):
    rng = np.random.default_rng(2026 + B * 100 + Cc * 10 + HD)
    cosT = rng.integers(-128, 129, size=(B, HD)).astype(np.int32)
    sinT = rng.integers(-128, 129, size=(B, HD)).astype(np.int32)
    Th = rng.integers(-128, 129, size=(B, Cc)).astype(np.int32)
    gen, q = points(31, pow2(Cc)), points(32, 1)
    paths = {}
    for name, arr in (("T", Th), ("cos", cosT), ("sin", sinT), ("gen", gen), ("q", q)):
        paths[name] = str(tmp_path / (name + ".bin"))
        np.ascontiguousarray(arr).tofile(paths[name])
    ob = tmp_path / "ob"
    ob.mkdir()
    yout = str(tmp_path / "Y64.i64")
    seed = "selftest:rope"
    r = subprocess.run([ROPE, "prove", str(ob), seed, paths["T"], str(B), str(Cc), str(HD), paths["cos"],
                        paths["sin"], paths["gen"], paths["q"], yout], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "PROVED rope obligation" in r.stdout
    want, Y = expected_rope(seed, Th, HD, cosT, sinT, gen, q[0])
    for name, data in want.items():
        assert (ob / name).read_bytes() == data, name
    assert open(yout, "rb").read() == Y.astype(np.int64).tobytes()
    # a layout the reference refuses: HD not dividing C
    r = subprocess.run([ROPE, "prove", str(ob), seed, paths["T"], str(B), str(Cc), str(8 if Cc % 8 else 16),
                        paths["cos"], paths["sin"], paths["gen"], paths["q"]], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 1
