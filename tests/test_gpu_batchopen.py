"""The claims accumulator and its batch opening: zkh_fc's claim mode (`--claims <accdir>
<obid> <com_W>`, zkob_fc.cu:449-470) and zkh_batchopen (zkob_batchopen.cu:695-755, batch_prove
zkob_claims.cuh:832-1066).

The claim mode must append the same claims.bin records (claim_blob, zkob_claims.cuh:104-116),
witness files, witrefs.txt lines and drvstates.bin entries as the reference; the batch opening
must write the same batch_sumcheck.bin, batch_vfin.bin and ipa_batch_<G>.bin, byte for byte.
Both are restated here from the oracle's primitives (transcript, SHA-256, commitments, matmul
sumcheck, eq tables, row folds, IPA) with the batch rounds written out in Python integers.
The restatement is pinned by the protocol's own identities, checked as it runs: every round
satisfies p(0) + p(1) = the running claim, the terminals satisfy
sum_j M_j(r) kappa_j v_j = the final claim (bo_Mj_at_r, bo_kappa, zkob_claims.cuh:758-778),
and every domain's IPA vectors satisfy <a, b> = sum_j rho'^j kappa_j v_j.
Cases: two obligations of different shapes (two generator domains, tensors of 3 to 5
variables, so the constant-S rounds run), a weight shared by two obligations (two claims on
one tensor), and the error paths (no witref, no generator file, a false claim, a committed
claim)."""
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
FC = os.path.join(ROOT, "zk-hillclimb_amd", "zkh_fc")
BO = os.path.join(ROOT, "zk-hillclimb_amd", "zkh_batchopen")
BASE = G.aff_to_jac((G.GX, G.GY))
R = P.R


@pytest.fixture(autouse=True)
def _convention_crosschecks(monkeypatch):
    """The drivers run with ZKH_XCHECK=1: every proof also checks its folded terminals against
    multi_dim_me at the opening point, as the reference's drivers do; the batch opening also
    runs its commitment-side self-check (ZKOB_BATCH_SELFCHECK, zkob_claims.cuh:1038-1052)."""
    monkeypatch.setenv("ZKH_XCHECK", "1")
    monkeypatch.setenv("ZKOB_BATCH_SELFCHECK", "1")


def points(seed, n):
    rng = np.random.default_rng(seed)
    out = np.zeros((n, 36), np.uint32)
    for i in range(n):
        k = int.from_bytes(rng.bytes(32), "little") % R
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


def ints(fr):
    return C.fr_to_ints(fr)


def fr_bytes(x):
    return P.to_bytes(x % R)


def challenge(st):
    return P.from_limbs(C.tr_challenge_fr(st))


def blob(c):
    """claim_blob (zkob_claims.cuh:104-116)"""
    pid, ref = c["id"].encode(), c["comref"].encode()
    return (struct.pack("<I", len(pid)) + pid + struct.pack("<I", len(ref)) + ref +
            struct.pack("<III", c["domain"], c["n_rows"], len(c["point"])) +
            b"".join(fr_bytes(x) for x in c["point"]) + b"\x00" + fr_bytes(c["eval"]))


def claims_file(cs):
    return b"ZKCL" + struct.pack("<II", 1, len(cs)) + b"".join(blob(c) for c in cs)


def drvstates_file(ds):
    return b"ZKDS" + struct.pack("<II", 1, len(ds)) + b"".join(
        struct.pack("<I", len(i)) + i.encode() + s for i, s in ds)


def fc_claims(seed, obid, obdir, comW, X, W, gin, gout):
    """zkob_fc claim mode restated: the three claims, the padded witnesses, the commitments
    and the driver's final transcript state."""
    B, IN = X.shape
    OUT = W.shape[1]
    Y = X.astype(np.int64) @ W.astype(np.int64)
    Xp, Wp, Yp = padded(X), padded(W), padded(Y)
    coms = {}
    for name, T, g in (("X", Xp, gin), ("W", Wp, gout), ("Y", Yp, gout)):
        rc, c = C.g1_commit(g, C.ints_to_fr(T.reshape(-1)), T.shape[1])
        assert rc == 0
        coms[name] = c.tobytes()
    st = C.tr_init(seed)
    for lab, v in (("B", B), ("IN", IN), ("OUT", OUT)):
        C.tr_absorb(st, lab, struct.pack("<I", v))
    for lab in ("X", "W", "Y"):
        C.tr_absorb(st, "com_" + lab, coms[lab])
    rc, mm = C.mm_prove(st, X, W, Y, B, IN, OUT)
    assert rc == 0
    claim, claim_X, claim_W = ints(mm["claims"])
    uo, ui, ub = ints(mm["u_output"]), ints(mm["u_input"]), ints(mm["u_batch"])
    refX, refY = os.path.join(obdir, "com_X.bin"), os.path.join(obdir, "com_Y.bin")
    cs = [dict(id=obid + ":W", comref=comW, domain=Wp.shape[1], n_rows=Wp.shape[0], point=uo + ui, eval=claim_W),
          dict(id=obid + ":X", comref=refX, domain=Xp.shape[1], n_rows=Xp.shape[0], point=ui + ub, eval=claim_X),
          dict(id=obid + ":Y", comref=refY, domain=Yp.shape[1], n_rows=Yp.shape[0], point=uo + ub, eval=claim)]
    wit = {comW: Wp.reshape(-1), refX: Xp.reshape(-1), refY: Yp.reshape(-1)}
    return cs, wit, coms, bytes(st)


def batch_expected(cs, ds, wit, comfiles, run_seed, gens, Q):
    """batch_prove (zkob_claims.cuh:832-1066) restated: returns the three kinds of files."""
    tensors, key = [], {}
    for i, c in enumerate(cs):  # derive_tensors (zkob_claims.cuh:280-308)
        if c["comref"] not in key:
            key[c["comref"]] = len(tensors)
            tensors.append(dict(comref=c["comref"], domain=c["domain"], vars=len(c["point"]),
                                logG=P.ceil_log2(c["domain"]), idx=[]))
        tensors[key[c["comref"]]]["idx"].append(i)
    m_max = max(t["vars"] for t in tensors)
    st = C.tr_init(run_seed + ":opening_batch")
    C.tr_absorb(st, "n_claims", struct.pack("<I", len(cs)))
    for c in cs:
        C.tr_absorb(st, "claim", blob(c))
    for t in tensors:
        ref = t["comref"].encode()
        C.tr_absorb(st, "comref", struct.pack("<I", len(ref)) + ref + C.sha256(comfiles[t["comref"]]))
    for i, s in ds:
        C.tr_absorb(st, "drvstate", struct.pack("<I", len(i)) + i.encode() + s)
    rho = challenge(st)
    rp = [pow(rho, i, R) for i in range(len(cs))]
    M, Pt, S, c2 = [], [], [], []
    for t in tensors:
        m = [sum(rp[i] * P.eq_weight(b, cs[i]["point"]) for i in t["idx"]) % R for b in range(1 << t["vars"])]
        p = [int(v) % R for v in wit[t["comref"]]]
        M.append(m)
        Pt.append(p)
        S.append(sum(x * y for x, y in zip(m, p)) % R)
        c2.append(1)
    cur = sum(rp[i] * c["eval"] for i, c in enumerate(cs)) % R
    r, ev = [0] * m_max, []
    for t in range(m_max):
        v = m_max - 1 - t
        p = [0, 0, 0]
        for j, tj in enumerate(tensors):
            if tj["vars"] <= v:
                p[0] = (p[0] + c2[j] * S[j]) % R
                p[2] = (p[2] + c2[j] * S[j]) % R
                continue
            h = len(M[j]) // 2
            for k in range(3):
                q = sum((M[j][i] + k * (M[j][i + h] - M[j][i])) * (Pt[j][i] + k * (Pt[j][i + h] - Pt[j][i]))
                        for i in range(h))
                p[k] = (p[k] + c2[j] * q) % R
        assert (p[0] + p[1]) % R == cur, "round %d" % t
        for k in range(3):
            C.tr_absorb(st, "bp%d" % k, fr_bytes(p[k]))
        x = challenge(st)
        r[v] = x
        ev += p
        cur = P.lagrange(p, x)
        for j, tj in enumerate(tensors):
            if tj["vars"] <= v:
                c2[j] = c2[j] * (1 - x) ** 2 % R
            else:
                h = len(M[j]) // 2
                M[j] = [(M[j][i] + x * (M[j][i + h] - M[j][i])) % R for i in range(h)]
                Pt[j] = [(Pt[j][i] + x * (Pt[j][i + h] - Pt[j][i])) % R for i in range(h)]
    files = {"batch_sumcheck.bin": b"ZKBS" + struct.pack("<III", len(cs), m_max, len(ev)) +
             b"".join(fr_bytes(e) for e in ev)}
    vfin = [p[0] for p in Pt]
    for x in vfin:
        C.tr_absorb(st, "vfin", fr_bytes(x))
    files["batch_vfin.bin"] = b"ZKBV" + struct.pack("<I", len(vfin)) + b"".join(fr_bytes(x) for x in vfin)

    def kappa(vars_):
        k = 1
        for v in range(vars_, m_max):
            k = k * (1 - r[v]) % R
        return k
    total = 0
    for j, tj in enumerate(tensors):
        kap = kappa(tj["vars"])
        mj = sum(rp[i] * kap * _eqprod(cs[i]["point"], r) for i in tj["idx"]) % R
        total += mj * kap * vfin[j]
    assert total % R == cur, "terminal identity"
    rhop = challenge(st)
    for Gd in sorted({t["domain"] for t in tensors}):
        logG = P.ceil_log2(Gd)
        a, vstar = [0] * Gd, 0
        for j, tj in enumerate(tensors):
            if tj["domain"] != Gd:
                continue
            coef = pow(rhop, j, R) * kappa(tj["vars"]) % R
            w = C.ints_to_fr(wit[tj["comref"]])
            if tj["vars"] > logG:
                rc, w = C.partial_me_window(w, C.ints_to_fr(r[logG:tj["vars"]]), Gd)
                assert rc == 0
            a = [(x + coef * y) % R for x, y in zip(a, ints(w))]
            vstar += coef * vfin[j]
        b = C.build_eq(C.ints_to_fr(r[:logG]))
        assert sum(x * y for x, y in zip(a, ints(b))) % R == vstar % R, "group %d" % Gd
        rc, L, Rr, af = C.ipa_prove(st, C.ints_to_fr(a), b, gens[Gd], Q, Gd)
        assert rc == 0
        files["ipa_batch_%d.bin" % Gd] = pod(L, 36) + pod(Rr, 36) + af.tobytes()
    return files


def _eqprod(point, r):
    e = 1
    for v, u in enumerate(point):
        e = e * P.eq2(u, r[v]) % R
    return e


GENS = {G_: points(40 + G_, G_) for G_ in (2, 4, 8)}
Q2 = points(99, 2)


def run_fc(tmp, obid, X, W, comW, accdir):
    B, IN = X.shape
    OUT = W.shape[1]
    obdir = os.path.join(tmp, obid)
    os.makedirs(obdir, exist_ok=True)
    paths = {}
    for name, arr in (("X", X.astype(np.int32)), ("W", W.astype(np.int32))):
        paths[name] = os.path.join(obdir, name + ".in")
        np.ascontiguousarray(arr).tofile(paths[name])
    gin, gout = os.path.join(tmp, "gen_%d.bin" % pow2(IN)), os.path.join(tmp, "gen_%d.bin" % pow2(OUT))
    seed = "run3:" + obid
    r = subprocess.run([FC, "prove", obdir, seed, paths["X"], paths["W"], str(B), str(IN), str(OUT), gin, gout,
                        os.path.join(tmp, "q.bin"), "--claims", accdir, obid, comW],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "claim mode, 3 claims emitted" in r.stdout
    assert not os.path.exists(os.path.join(obdir, "ipa_W.bin"))
    return obdir, seed


def setup_dirs(tmp):
    for G_, g in GENS.items():
        g.tofile(os.path.join(tmp, "gen_%d.bin" % G_))
    Q2.tofile(os.path.join(tmp, "q.bin"))
    acc = os.path.join(tmp, "acc")
    os.makedirs(acc)
    return acc


def accumulate(tmp, obligations, acc=None, cs=None, ds=None, wit=None, comfiles=None):
    """run zkh_fc --claims for each (obid, X, W, comW-name) and restate what it must emit"""
    if acc is None:
        acc = setup_dirs(tmp)
        cs, ds, wit, comfiles = [], [], {}, {}
    for obid, X, W, wname in obligations:
        comW = os.path.join(tmp, wname)
        obdir = os.path.join(tmp, obid)
        gin, gout = GENS[pow2(X.shape[1])], GENS[pow2(W.shape[1])]
        ccs, cwit, coms, state = fc_claims("run3:" + obid, obid, obdir, comW, X, W, gin, gout)
        if not os.path.exists(comW):  # the registered weight commitment
            open(comW, "wb").write(coms["W"])
        run_fc(tmp, obid, X, W, comW, acc)
        cs += ccs
        ds.append((obid, state))
        for k, v in cwit.items():
            wit.setdefault(k, v)
        comfiles.update({comW: coms["W"], ccs[1]["comref"]: coms["X"], ccs[2]["comref"]: coms["Y"]})
    return acc, cs, ds, wit, comfiles


def check_accumulator(acc, cs, ds, wit, obligations):
    assert open(os.path.join(acc, "claims.bin"), "rb").read() == claims_file(cs)
    assert open(os.path.join(acc, "drvstates.bin"), "rb").read() == drvstates_file(ds)
    lines, seen = [], set()
    for obid in [o[0] for o in obligations]:
        for c in cs:
            if c["id"].startswith(obid + ":") and c["comref"] not in seen:
                seen.add(c["comref"])
                t = c["id"].split(":")[-1]
                wpath = os.path.join(acc, "wit_%s_%s.fr" % (obid, t))
                lines.append("%s\t%s\n" % (c["comref"], wpath))
                assert open(wpath, "rb").read() == C.ints_to_fr(wit[c["comref"]]).tobytes()
    assert open(os.path.join(acc, "witrefs.txt")).read() == "".join(lines)


def run_bo(acc, tmp, seed, domains):
    return subprocess.run([BO, "prove", acc, seed, os.path.join(tmp, "q.bin")] +
                          ["%d=%s" % (d, os.path.join(tmp, "gen_%d.bin" % d)) for d in domains],
                          capture_output=True, text=True, timeout=120)


def rng_mats(seed, B, IN, OUT):
    rng = np.random.default_rng(seed)
    return (rng.integers(-2**15, 2**15, size=(B, IN)).astype(np.int32),
            rng.integers(-229376, 229377, size=(IN, OUT)).astype(np.int32))


def test_two_obligations_two_domains(tmp_path):
    tmp = str(tmp_path)
    X1, W1 = rng_mats(1, 4, 8, 4)
    X2, W2 = rng_mats(2, 2, 3, 7)
    obs = [("L0.fc1", X1, W1, "comW1.bin"), ("L0.fc2", X2, W2, "comW2.bin")]
    acc, cs, ds, wit, comfiles = accumulate(tmp, obs)
    check_accumulator(acc, cs, ds, wit, obs)
    r = run_bo(acc, tmp, "run3", (4, 8))
    assert r.returncode == 0, r.stderr
    assert "PROVED opening_batch (6 claims, 6 tensors, 2 domains)" in r.stdout
    want = batch_expected(cs, ds, wit, comfiles, "run3", GENS, Q2[0])
    assert sorted(want) == sorted(f for f in os.listdir(acc) if f.startswith(("batch_", "ipa_batch_")))
    for name, data in want.items():
        assert open(os.path.join(acc, name), "rb").read() == data, name


def test_shared_weight_two_claims_one_tensor(tmp_path):
    tmp = str(tmp_path)
    Xa, W = rng_mats(3, 4, 4, 8)
    Xb, _ = rng_mats(4, 2, 4, 8)
    obs = [("L1.a", Xa, W, "comW.bin"), ("L1.b", Xb, W, "comW.bin")]
    acc, cs, ds, wit, comfiles = accumulate(tmp, obs)
    check_accumulator(acc, cs, ds, wit, obs)
    r = run_bo(acc, tmp, "run9", (4, 8))
    assert r.returncode == 0, r.stderr
    assert "(6 claims, 5 tensors, 2 domains)" in r.stdout
    want = batch_expected(cs, ds, wit, comfiles, "run9", GENS, Q2[0])
    for name, data in want.items():
        assert open(os.path.join(acc, name), "rb").read() == data, name


def test_batch_open_errors(tmp_path):
    tmp = str(tmp_path)
    X, W = rng_mats(5, 2, 4, 2)
    obs = [("L2.fc", X, W, "comW.bin")]
    acc, cs, ds, wit, comfiles = accumulate(tmp, obs)
    r = run_bo(acc, tmp, "run1", (4,))  # no generator file for domain 2
    assert r.returncode == 1 and "no generator file for domain 2" in r.stderr
    r = run_bo(acc, tmp, "run1", (2, 4))
    assert r.returncode == 0, r.stderr
    good = open(os.path.join(acc, "claims.bin"), "rb").read()
    bad = dict(cs[0], eval=(cs[0]["eval"] + 1) % R)  # a false claim
    open(os.path.join(acc, "claims.bin"), "wb").write(claims_file([bad] + cs[1:]))
    r = run_bo(acc, tmp, "run1", (2, 4))
    assert r.returncode == 1 and "round 0 inconsistency" in r.stderr
    committed = claims_file(cs).replace(blob(cs[0]), blob(cs[0])[:-33] + b"\x01" + blob(cs[0])[-32:])
    open(os.path.join(acc, "claims.bin"), "wb").write(committed)
    r = run_bo(acc, tmp, "run1", (2, 4))
    assert r.returncode == 2, r.stderr
    open(os.path.join(acc, "claims.bin"), "wb").write(good)
    wr = open(os.path.join(acc, "witrefs.txt")).read().splitlines(True)
    open(os.path.join(acc, "witrefs.txt"), "w").write("".join(wr[1:]))
    r = run_bo(acc, tmp, "run1", (2, 4))
    assert r.returncode == 1 and "no witref" in r.stderr
    r = subprocess.run([FC, "prove", "--claims", acc], capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and "--claims needs" in r.stderr


RESCALE = os.path.join(ROOT, "zk-hillclimb_amd", "zkh_rescale")


def rescale_claims(seed, obid, obdir, X, log_sf, gen):
    """zkob_rescale claim mode restated (zkob_rescale.cu:70-190): the claims on A, rem and m
    at the logUp proof's terminal points, their witnesses and commitments, the final state."""
    B, Cc = X.shape
    sf = 1 << log_sf
    Bp, Cp = pow2(B), pow2(Cc)
    D, N = Bp * Cp, sf
    logD, n1 = P.ceil_log2(D), P.ceil_log2(D // N)
    rc, q, rem = C.rescale(X.reshape(-1), sf)
    assert rc == 0
    Xp, Xrp, remp = padded(X), padded(q.reshape(B, Cc)), padded(rem.reshape(B, Cc))
    low = -(sf >> 1)
    S = C.ints_to_fr(remp.reshape(-1))
    rc, m = C.lu_prep(S, low, N)
    assert rc == 0
    coms = {}
    for name, t in (("X", C.ints_to_fr(Xp.reshape(-1))), ("Xr", C.ints_to_fr(Xrp.reshape(-1))), ("rem", S),
                    ("m", m)):
        rc, c = C.g1_commit(gen, t, Cp)
        coms[name] = c.tobytes()
    st = C.tr_init(seed)
    for lab, v in (("B", B), ("C", Cc), ("LOG_SF", log_sf)):
        C.tr_absorb(st, lab, struct.pack("<I", v))
    for name in ("X", "Xr", "rem", "m"):
        C.tr_absorb(st, "com_" + name, coms[name])
    beta = C.tr_challenge_fr(st)
    A = C.lu_inverse(S, beta)
    rc, c = C.g1_commit(gen, A, Cp)
    coms["A"] = c.tobytes()
    C.tr_absorb(st, "com_A", coms["A"])
    alpha = C.tr_challenge_fr(st)
    u = np.array([C.tr_challenge_fr(st) for _ in range(logD)])
    rc, lk = C.lu_prove(st, A, S, C.range_table(low, sf, N), m, alpha, beta, u)
    assert rc == 0
    u_pt = ints(lk["ws"][::-1])
    A_f, S_f, _, _, m_f = ints(lk["term"])
    ref = {t: os.path.join(obdir, "com_%s.bin" % t) for t in ("A", "rem", "m")}
    cs = [dict(id=obid + ":A", comref=ref["A"], domain=Cp, n_rows=Bp, point=u_pt, eval=A_f),
          dict(id=obid + ":rem", comref=ref["rem"], domain=Cp, n_rows=Bp, point=u_pt, eval=S_f),
          dict(id=obid + ":m", comref=ref["m"], domain=Cp, n_rows=N // Cp, point=u_pt[:logD - n1], eval=m_f)]
    wit = {ref["A"]: ints(A), ref["rem"]: ints(S), ref["m"]: ints(m)}
    return cs, wit, {ref[t]: coms[t] for t in ref}, bytes(st)


@pytest.mark.parametrize("B,Cc,log_sf", [(8, 4, 4), (4, 8, 5)])
def test_rescale_and_fc_claims_in_one_batch(tmp_path, B, Cc, log_sf):
    """lookup-derived claims (A, rem, m of a rescaling, zkob_rescale.cu:165-190) and a
    matmul's claims accumulated together, then opened in one batch"""
    tmp = str(tmp_path)
    acc = setup_dirs(tmp)
    rng = np.random.default_rng(B + Cc + log_sf)
    X = rng.integers(-(1 << 12), 1 << 12, size=(B, Cc)).astype(np.int64) * 37
    obid, obdir = "L3.rescale", os.path.join(tmp, "L3.rescale")
    os.makedirs(obdir)
    xp = os.path.join(obdir, "X.i64")
    X.tofile(xp)
    seed = "run5:" + obid
    r = subprocess.run([RESCALE, "prove", obdir, seed, xp, str(B), str(Cc), str(log_sf),
                        os.path.join(tmp, "gen_%d.bin" % pow2(Cc)), os.path.join(tmp, "q.bin"), "--claims", acc, obid],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "claim mode, 3 claims emitted" in r.stdout
    assert not os.path.exists(os.path.join(obdir, "ipa_A.bin"))
    cs, wit, comfiles, state = rescale_claims(seed, obid, obdir, X, log_sf, GENS[pow2(Cc)])
    ds = [(obid, state)]
    X1, W1 = rng_mats(6, 4, 8, 4)
    obs = [("L3.fc", X1, W1, "comW.bin")]
    acc, cs, ds, wit, comfiles = accumulate(tmp, obs, acc, cs, ds, wit, comfiles)
    check_accumulator(acc, cs, ds, wit, [(obid,)] + obs)
    r = run_bo(acc, tmp, "run5", (4, 8))
    assert r.returncode == 0, r.stderr
    assert "(6 claims, 6 tensors, 2 domains)" in r.stdout
    want = batch_expected(cs, ds, wit, comfiles, "run5", GENS, Q2[0])
    for name, data in want.items():
        assert open(os.path.join(acc, name), "rb").read() == data, name


ROPE = os.path.join(ROOT, "zk-hillclimb_amd", "zkh_rope")


def rope_claims(seed, obid, obdir, Th, HD, cosT, sinT, gen):
    """zkob_rope claim mode restated (zkob_rope.cu:102-304): the weights and the flipped T by
    their definitions, the two Hadamard sumchecks from the oracle, and the claims T1 (at the
    first terminal point), T2 (at the second, its coordinate log2(HD)-1 complemented) and Y
    (at u), both T claims on the one tensor com_T.bin."""
    B, Cc = Th.shape
    Cp = pow2(Cc)
    logD = P.ceil_log2(B) + P.ceil_log2(Cp)
    flipv, fb = HD // 2, P.ceil_log2(HD) - 1
    W1, W2, Tg = (np.zeros((B, Cp), np.int64) for _ in range(3))
    for t in range(B):
        for e in range(Cc):
            W1[t, e] = cosT[t, e % HD]
            W2[t, e] = (1 if e & flipv else -1) * sinT[t, e % HD]
            Tg[t, e] = Th[t, e]
    Txg = Tg[:, [e ^ flipv for e in range(Cp)]]
    Y = Tg * W1 + Txg * W2
    T_fr, Tx_fr, Y_fr = (C.ints_to_fr(M.reshape(-1)) for M in (Tg, Txg, Y))
    ones = C.ints_to_fr([1] * (B * Cp))
    comT, comY = (C.g1_commit(gen, t, Cp)[1].tobytes() for t in (T_fr, Y_fr))
    st = C.tr_init(seed)
    for lab, v in (("B", B), ("C", Cc), ("HD", HD), ("SCALE_R", 16)):
        C.tr_absorb(st, lab, struct.pack("<I", v))
    C.tr_absorb(st, "com_T", comT)
    C.tr_absorb(st, "com_Y64", comY)
    u = np.array([C.tr_challenge_fr(st) for _ in range(logD)])
    rc, ev = C.me(Y_fr, u)
    C.tr_absorb(st, "ev", ev.tobytes())
    Eu = ints(C.build_eq(u))
    refT, refY = os.path.join(obdir, "com_T.bin"), os.path.join(obdir, "com_Y64.bin")
    cs = []
    for k, (W, S_fr, S_int) in enumerate(((W1, T_fr, Tg), (W2, Tx_fr, Txg)), start=1):
        E = [e * int(w) % R for e, w in zip(Eu, W.reshape(-1))]
        c = sum(e * int(s) for e, s in zip(E, S_int.reshape(-1))) % R
        C.tr_absorb(st, "c%d" % k, fr_bytes(c))
        rc, hp = C.hp_prove(st, np.array(P.to_limbs(c), np.uint32), C.ints_to_fr(E), S_fr, ones)
        assert rc == 0
        C.tr_absorb(st, "S_f2", hp["term"][0].tobytes())
        C.tr_absorb(st, "U_f2", hp["term"][1].tobytes())
        pt = ints(hp["ws"][::-1])
        if k == 2:
            pt[fb] = (1 - pt[fb]) % R
        cs.append(dict(id="%s:T%d" % (obid, k), comref=refT, domain=Cp, n_rows=B, point=pt,
                       eval=ints(hp["term"][0])[0]))
    cs.append(dict(id=obid + ":Y", comref=refY, domain=Cp, n_rows=B, point=ints(u), eval=ints(ev)[0]))
    wit = {refT: Tg.reshape(-1), refY: Y.reshape(-1)}
    return cs, wit, {refT: comT, refY: comY}, bytes(st)


@pytest.mark.parametrize("B,Cc,HD", [(8, 6, 2), (4, 8, 4)])
def test_rope_and_fc_claims_in_one_batch(tmp_path, B, Cc, HD):
    """a RoPE obligation's three claims (two on one tensor, zkob_rope.cu:250-304) and a
    matmul's accumulated together, then opened in one batch"""
    tmp = str(tmp_path)
    acc = setup_dirs(tmp)
    rng = np.random.default_rng(2027 + B * 100 + Cc * 10 + HD)
    cosT = rng.integers(-128, 129, size=(B, HD)).astype(np.int32)
    sinT = rng.integers(-128, 129, size=(B, HD)).astype(np.int32)
    Th = rng.integers(-128, 129, size=(B, Cc)).astype(np.int32)
    obid, obdir = "L4.rope_q", os.path.join(tmp, "L4.rope_q")
    os.makedirs(obdir)
    paths = {}
    for name, arr in (("T", Th), ("cos", cosT), ("sin", sinT)):
        paths[name] = os.path.join(obdir, name + ".in")
        np.ascontiguousarray(arr).tofile(paths[name])
    seed = "run6:" + obid
    r = subprocess.run([ROPE, "prove", obdir, seed, paths["T"], str(B), str(Cc), str(HD), paths["cos"], paths["sin"],
                        os.path.join(tmp, "gen_%d.bin" % pow2(Cc)), os.path.join(tmp, "q.bin"), "--claims", acc, obid],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "claim mode, 3 claims emitted" in r.stdout
    assert not os.path.exists(os.path.join(obdir, "ipa_T1.bin"))
    cs, wit, comfiles, state = rope_claims(seed, obid, obdir, Th, HD, cosT, sinT, GENS[pow2(Cc)])
    ds = [(obid, state)]
    X1, W1 = rng_mats(7, 2, 4, 8)
    obs = [("L4.fc", X1, W1, "comW.bin")]
    acc, cs, ds, wit, comfiles = accumulate(tmp, obs, acc, cs, ds, wit, comfiles)
    assert open(os.path.join(acc, "claims.bin"), "rb").read() == claims_file(cs)
    assert open(os.path.join(acc, "drvstates.bin"), "rb").read() == drvstates_file(ds)
    for t, ref in (("T", cs[0]["comref"]), ("Y", cs[2]["comref"])):
        wpath = os.path.join(acc, "wit_%s_%s.fr" % (obid, t))
        assert open(wpath, "rb").read() == C.ints_to_fr(wit[ref]).tobytes()
    r = run_bo(acc, tmp, "run6", (4, 8))
    assert r.returncode == 0, r.stderr
    assert "(6 claims, 5 tensors, 2 domains)" in r.stdout
    want = batch_expected(cs, ds, wit, comfiles, "run6", GENS, Q2[0])
    for name, data in want.items():
        assert open(os.path.join(acc, name), "rb").read() == data, name


GLU = os.path.join(ROOT, "zk-hillclimb_amd", "zkh_glu")


def glu_claims(seed, obid, obdir, Gm, Um, low, ln, mapped, gen):
    """zkob_glu claim mode restated (zkob_glu.cu:86-275): the mapping lookup by its
    definition, com_comb = com_G + r com_S row by row (hb_addmul, zkob_fastg1.cuh:56-88), and
    the six claims A, comb, m (lookup terminals) and H, S, U (Hadamard)."""
    B, Cc = Gm.shape
    Bp, Cp = pow2(B), pow2(Cc)
    D, N = Bp * Cp, ln
    logD, n1 = P.ceil_log2(D), P.ceil_log2(D // N)
    Gp, Up = padded(Gm), padded(Um)
    idx = (Gp - low).reshape(-1)
    S = np.asarray(mapped, np.int64)[idx].reshape(Gp.shape)
    m = np.bincount(idx, minlength=N).astype(np.int64)
    H = S * Up
    coms = {}
    for name, t in (("G", Gp), ("S", S), ("U", Up), ("H", H), ("m", m)):
        coms[name] = C.g1_commit(gen, C.ints_to_fr(t.reshape(-1)), Cp)[1]
    st = C.tr_init(seed)
    for lab, v in (("B", B), ("C", Cc), ("LOW", low & 0xFFFFFFFF), ("LEN", ln)):
        C.tr_absorb(st, lab, struct.pack("<I", v))
    for name in ("G", "S", "U", "H", "m"):
        C.tr_absorb(st, "com_" + name, coms[name].tobytes())
    r = challenge(st)
    beta = C.tr_challenge_fr(st)
    comb = [(int(g) + r * int(s)) % R for g, s in zip(Gp.reshape(-1), S.reshape(-1))]
    Tcomb = C.ints_to_fr([(low + i + r * int(mapped[i])) % R for i in range(N)])
    A = C.lu_inverse(C.ints_to_fr(comb), beta)
    coms["A"] = C.g1_commit(gen, A, Cp)[1]
    C.tr_absorb(st, "com_A", coms["A"].tobytes())
    alpha = C.tr_challenge_fr(st)
    u = np.array([C.tr_challenge_fr(st) for _ in range(logD)])
    rc, lk = C.lu_prove(st, A, C.ints_to_fr(comb), Tcomb, C.ints_to_fr(m), alpha, beta, u)
    assert rc == 0
    rl = np.array(P.to_limbs(r), np.uint32)
    coms["comb"] = np.array([C.g1_add(coms["G"][j], C.g1_mul(coms["S"][j], rl)) for j in range(Bp)])
    # pin: com_comb row j is the commitment of comb row j as a group element
    for j in (0, Bp - 1):
        want = C.g1_commit(gen, C.ints_to_fr(comb[j * Cp:(j + 1) * Cp]), Cp)[1][0]
        assert G.to_affine(coms["comb"][j]) == G.to_affine(want)
    u_pt = ints(lk["ws"][::-1])
    A_f, S_f, _, _, m_f = ints(lk["term"])
    uh = np.array([C.tr_challenge_fr(st) for _ in range(logD)])
    rc, claimH = C.me(C.ints_to_fr(H.reshape(-1)), uh)
    C.tr_absorb(st, "claim_H", claimH.tobytes())
    rc, hp = C.hp_prove(st, claimH, C.build_eq(uh), C.ints_to_fr(S.reshape(-1)), C.ints_to_fr(Up.reshape(-1)))
    assert rc == 0
    C.tr_absorb(st, "S_f2", hp["term"][0].tobytes())
    C.tr_absorb(st, "U_f2", hp["term"][1].tobytes())
    u_pt2 = ints(hp["ws"][::-1])
    S_f2, U_f2 = ints(hp["term"][:2])
    ref = {t: os.path.join(obdir, "com_%s.bin" % t) for t in ("A", "comb", "m", "H", "S", "U")}
    rows = dict(A=Bp, comb=Bp, m=N // Cp, H=Bp, S=Bp, U=Bp)
    pts = dict(A=u_pt, comb=u_pt, m=u_pt[:logD - n1], H=ints(uh), S=u_pt2, U=u_pt2)
    evs = dict(A=A_f, comb=S_f, m=m_f, H=ints(claimH)[0], S=S_f2, U=U_f2)
    cs = [dict(id="%s:%s" % (obid, t), comref=ref[t], domain=Cp, n_rows=rows[t], point=pts[t], eval=evs[t])
          for t in ("A", "comb", "m", "H", "S", "U")]
    wit = {ref["A"]: ints(A), ref["comb"]: comb, ref["m"]: m.reshape(-1), ref["H"]: H.reshape(-1),
           ref["S"]: S.reshape(-1), ref["U"]: Up.reshape(-1)}
    return cs, wit, {ref[t]: coms[t].tobytes() for t in ref}, bytes(st)


@pytest.mark.parametrize("B,Cc,low,ln", [(8, 4, -8, 16), (8, 6, -16, 32)])
def test_glu_and_fc_claims_in_one_batch(tmp_path, B, Cc, low, ln):
    """a SwiGLU obligation's six claims (zkob_glu.cu:204-275, com_comb.bin included) and a
    matmul's accumulated together, then opened in one batch"""
    tmp = str(tmp_path)
    acc = setup_dirs(tmp)
    rng = np.random.default_rng(B * 1000 + Cc * 10 + ln + 1)
    mapped = np.array([(i + low) ** 2 for i in range(ln)], np.int32)
    Gm = rng.integers(low, low + ln, size=(B, Cc)).astype(np.int32)
    Um = rng.integers(-300, 300, size=(B, Cc)).astype(np.int32)
    obid, obdir = "L5.glu", os.path.join(tmp, "L5.glu")
    os.makedirs(obdir)
    paths = {}
    for name, arr in (("G", Gm), ("U", Um), ("mapped", mapped)):
        paths[name] = os.path.join(obdir, name + ".in")
        np.ascontiguousarray(arr).tofile(paths[name])
    seed = "run8:" + obid
    r = subprocess.run([GLU, "prove", obdir, seed, paths["G"], paths["U"], str(B), str(Cc), str(low), str(ln),
                        paths["mapped"], os.path.join(tmp, "gen_%d.bin" % pow2(Cc)), os.path.join(tmp, "q.bin"),
                        "--claims", acc, obid], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "claim mode, 6 claims emitted" in r.stdout
    assert not os.path.exists(os.path.join(obdir, "ipa_A.bin"))
    cs, wit, comfiles, state = glu_claims(seed, obid, obdir, Gm, Um, low, ln, mapped, GENS[pow2(Cc)])
    assert open(os.path.join(obdir, "com_comb.bin"), "rb").read() == comfiles[cs[1]["comref"]]
    ds = [(obid, state)]
    X1, W1 = rng_mats(8, 4, 8, 4)
    obs = [("L5.fc", X1, W1, "comW.bin")]
    acc, cs, ds, wit, comfiles = accumulate(tmp, obs, acc, cs, ds, wit, comfiles)
    check_accumulator(acc, cs, ds, wit, [(obid,)] + obs)
    r = run_bo(acc, tmp, "run8", (4, 8))
    assert r.returncode == 0, r.stderr
    assert "(9 claims, 9 tensors, 2 domains)" in r.stdout
    want = batch_expected(cs, ds, wit, comfiles, "run8", GENS, Q2[0])
    for name, data in want.items():
        assert open(os.path.join(acc, name), "rb").read() == data, name
