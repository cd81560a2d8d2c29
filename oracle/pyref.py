"""Independent pure-Python restatement of the Fr hot path (small cases only).

TEST INFRASTRUCTURE ONLY: used by tests/ and tests/golden/make_golden.py as a second,
independently written restatement to pin the C oracle (zkh_oracle.c), and as the
witness-free verifier whose algebra follows the reference's verify paths
(zkllm-src/zkob_fc.cu:489-712, zkob_rescale.cu:198-316, vrf_toy_lookup.cu:177-240).

It deliberately uses different methods from the C oracle where the mathematics allows:
Python big integers instead of Montgomery limbs, hashlib instead of a hand-written
SHA-256, and MLE evaluation by the definition sum_b f[b]*prod_i eq(b_i, u_i) instead of
the reference's pairwise folding.  Field values are canonical ints in [0, r).
"""
import hashlib
import struct

R = 0x73EDA753299D7D483339D80809A1D80553BDA402FFFE5BFEFFFFFFFF00000001
INV2 = (R + 1) // 2
MONT_R = 1 << 256


def fr(v):
    return v % R


def inv(a):
    # Fermat inverse with the reference's 0 -> 0 convention (tlookup.cu:50-62)
    return pow(a, R - 2, R)


def montmul(a, b):
    """Raw Montgomery product a*b*2^-256 mod r (bls12-381.cu:499-531)."""
    return a * b * pow(MONT_R, -1, R) % R


def to_limbs(x):
    return [(x >> (32 * i)) & 0xFFFFFFFF for i in range(8)]


def from_limbs(v):
    return sum(int(v[i]) << (32 * i) for i in range(8))


def to_bytes(x):
    return x.to_bytes(32, "little")


def ceil_log2(n):
    return 0 if n <= 1 else (n - 1).bit_length()


# ---------------- transcript (fs_transcript.hpp:115-166) ----------------
class Transcript:
    def __init__(self, seed=None, state=None):
        self.state = bytes(state) if state is not None else hashlib.sha256(seed.encode()).digest()

    def absorb(self, label, data):
        lb = label.encode()
        msg = self.state + struct.pack("<I", len(lb)) + lb + struct.pack("<Q", len(data)) + data
        self.state = hashlib.sha256(msg).digest()

    def absorb_fr(self, label, x):
        self.absorb(label, to_bytes(x))

    def absorb_u32(self, label, v):
        self.absorb(label, struct.pack("<I", v & 0xFFFFFFFF))

    def challenge_bytes(self):
        out = hashlib.sha256(self.state + b"chal").digest()
        self.state = hashlib.sha256(self.state + b"rtch").digest()
        return out

    def challenge_fr(self):
        # vrf_common.cuh:235-245: LE limbs, top limb %= 1944954707, redraw on zero
        while True:
            b = self.challenge_bytes()
            limbs = list(struct.unpack("<8I", b))
            limbs[7] %= 1944954707
            x = from_limbs(limbs)
            if x:
                return x

    def challenge_vec(self, n):
        return [self.challenge_fr() for _ in range(n)]


# ---------------- MLE by definition ----------------
def eq_weight(b, u):
    """prod_i (bit_i(b) ? u_i : 1-u_i), u[0] on the least significant bit."""
    w = 1
    for i, ui in enumerate(u):
        w = w * (ui if (b >> i) & 1 else (1 - ui)) % R
    return w


def mle(t, u):
    """sum_b t[b]*eq(b,u) over b < len(t) (entries beyond len(t) are zero)."""
    return sum(t[b] * eq_weight(b, u) for b in range(len(t))) % R


def eq_table(u):
    return [eq_weight(b, u) for b in range(1 << len(u))]


def mle2(mat, rows, cols, u_row, u_col):
    """2-D MLE of a row-major rows x cols matrix: row index bits bound by u_row, column
    bits by u_col (what multi_dim_me({u_row,u_col},{rows,cols}) evaluates)."""
    er = [eq_weight(i, u_row) for i in range(rows)]
    ec = [eq_weight(j, u_col) for j in range(cols)]
    return sum(er[i] * ec[j] * mat[i * cols + j] for i in range(rows) for j in range(cols)) % R


def lagrange(evals, x):
    """Evaluate the polynomial through (t, evals[t]), t = 0..k-1, at x."""
    k = len(evals)
    acc = 0
    for i in range(k):
        num, den = 1, 1
        for j in range(k):
            if j != i:
                num = num * (x - j) % R
                den = den * (i - j) % R
        acc = (acc + evals[i] * num * inv(den % R)) % R
    return acc


def eq2(u, v):
    return (2 * u * v - u - v + 1) % R


# ---------------- matmul sumcheck prover (zkob_fc.cu:259-440) ----------------
def mm_prove(tr, X, W, Y, B, IN, OUT):
    lb, lo, L = ceil_log2(B), ceil_log2(OUT), ceil_log2(IN)
    ub = tr.challenge_vec(lb)
    uo = tr.challenge_vec(lo)
    Xf = [fr(v) for v in X]
    Wf = [fr(v) for v in W]
    Yf = [fr(v) for v in Y]
    claim = mle2(Yf, B, OUT, ub, uo)
    tr.absorb_fr("claim", claim)
    eb = [eq_weight(i, ub) for i in range(B)]
    eo = [eq_weight(j, uo) for j in range(OUT)]
    a = [sum(eb[i] * Xf[i * IN + j] for i in range(B)) % R for j in range(IN)]
    b = [sum(Wf[j * OUT + o] * eo[o] for o in range(OUT)) % R for j in range(IN)]
    cur, xs, ev = claim, [], []
    sz = IN
    for _ in range(L):
        no = (1 << ceil_log2(sz)) >> 1
        a += [0] * (2 * no - len(a))
        b += [0] * (2 * no - len(b))
        # p(t) = sum_i (a0 + t da)(b0 + t db)
        p = [sum((a[i] + t * (a[i + no] - a[i])) * (b[i] + t * (b[i + no] - b[i]))
                 for i in range(no)) % R for t in range(3)]
        assert (p[0] + p[1]) % R == cur, "round inconsistency"
        for lab, v in zip(("p0", "p1", "p2"), p):
            tr.absorb_fr(lab, v)
        x = tr.challenge_fr()
        xs.append(x)
        ev += p
        cur = lagrange(p, x)
        a = [(a[i] + x * (a[i + no] - a[i])) % R for i in range(no)]
        b = [(b[i] + x * (b[i + no] - b[i])) % R for i in range(no)]
        sz = no
    ui = xs[::-1]
    cx = mle2(Xf, B, IN, ub, ui)
    cw = mle2(Wf, IN, OUT, ui, uo)
    tr.absorb_fr("claim_X", cx)
    tr.absorb_fr("claim_W", cw)
    return dict(ev=ev, claim=claim, claim_X=cx, claim_W=cw, u_batch=ub, u_output=uo,
                u_input=ui, a_fin=a[0], b_fin=b[0], cur=cur)


def mm_verify(tr, B, IN, OUT, ev, claim, claim_X, claim_W):
    """Witness-free replay (zkob_fc.cu:489-712 shape): round sums, Lagrange chain,
    terminal product.  Returns (ok, u_batch, u_output, u_input)."""
    ub = tr.challenge_vec(ceil_log2(B))
    uo = tr.challenge_vec(ceil_log2(OUT))
    tr.absorb_fr("claim", claim)
    cur, xs = claim, []
    L = ceil_log2(IN)
    for r in range(L):
        p = ev[3 * r:3 * r + 3]
        if (p[0] + p[1]) % R != cur:
            return False, ub, uo, None
        for lab, v in zip(("p0", "p1", "p2"), p):
            tr.absorb_fr(lab, v)
        x = tr.challenge_fr()
        xs.append(x)
        cur = lagrange(p, x)
    ok = cur == claim_X * claim_W % R
    tr.absorb_fr("claim_X", claim_X)
    tr.absorb_fr("claim_W", claim_W)
    return ok, ub, uo, xs[::-1]


# ---------------- logUp (tlookup.cu, zkob_lookup.cuh, zkob_rescale.cu) ----------------
def range_table(low, length, size):
    return [fr(low + i) if i < length else fr(low + length - 1) for i in range(size)]


def lu_prep(S, low, N):
    m = [0] * N
    for s in S:
        idx = ((s - fr(low)) % R) & 0xFFFFFFFF
        assert idx < N, "witness outside the table"
        m[idx] += 1
    return m


def lu_prove(tr, A, S, T, m, alpha, beta, u):
    """Round polynomials of fs_phase1/fs_phase2, computed from their defining sums:
    phase 1 p(X) = eq(u_last,X) sum_b eq(b,u_) alpha(A_X)(S_X+beta) + sum A_X + C/2,
    phase 2 adds (N/D) alpha^2 B_X (T_X+beta) inside the eq term and subtracts
    (N/D) sum m_X B_X."""
    D, N = len(A), len(T)
    Bv = [inv((t + beta) % R) for t in T]
    alpha_sq = alpha * alpha % R
    C = (alpha_sq - sum(b * mm for b, mm in zip(Bv, m))) % R
    claim = (alpha + alpha_sq) % R
    ratio = N * inv(D) % R
    A, S, Bv, T, m, u = list(A), list(S), list(Bv), list(T), list(m), list(u)
    ev, ws = [], []
    while u:
        sz = len(A)
        h = sz // 2
        ul, ur = u[-1], u[:-1]
        e_ = eq_table(ur)
        p = []
        for t in range(4):
            def lin(tab, i):
                return tab[i] + t * (tab[i + h] - tab[i])
            qa = sum(e_[i] * alpha * lin(A, i) * (lin(S, i) + beta) for i in range(h))
            sa = sum(lin(A, i) for i in range(h))
            val = eq2(ul, t) * qa + sa
            if sz > N:
                val += C * INV2
            else:
                qb = sum(e_[i] * ratio * alpha_sq * lin(Bv, i) * (lin(T, i) + beta)
                         for i in range(h))
                smb = sum(lin(m, i) * lin(Bv, i) for i in range(h))
                val += eq2(ul, t) * qb - ratio * smb
            p.append(val % R)
        assert (p[0] + p[1]) % R == claim, "lookup round inconsistency at round %d (sz %d)" % (len(ws), sz)
        for lab, v in zip(("p0", "p1", "p2", "p3"), p):
            tr.absorb_fr(lab, v)
        v = tr.challenge_fr()
        ws.append(v)
        ev += p
        claim = lagrange(p, v)
        eqv = eq2(ul, v)

        def fold(tab):
            return [(tab[i] + v * (tab[i + h] - tab[i])) % R for i in range(h)]
        A, S = fold(A), fold(S)
        if sz <= N:
            Bv, T, m = fold(Bv), fold(T), fold(m)
            alpha_sq = alpha_sq * eqv % R
        else:
            C = C * INV2 % R
        alpha = alpha * eqv % R
        u = ur
    term = dict(A_f=A[0], S_f=S[0], B_f=Bv[0], T_f=T[0], m_f=m[0])
    tr.absorb_fr("A_f", A[0])
    tr.absorb_fr("S_f", S[0])
    tr.absorb_fr("m_f", m[0])
    return ev, term, ws


def lu_verify(tr, D, N, T_public, ev, A_f, S_f, m_f, alpha, beta, u):
    """Witness-free verifier algebra (zkob_rescale.cu:282-316): Lagrange-4 chain with
    alpha/alpha^2 eq accumulators, B_f/T_f recomputed from the public table, terminal
    identity."""
    logD, n1 = ceil_log2(D), ceil_log2(D // N)
    cur = (alpha + alpha * alpha) % R
    aacc, a2acc = alpha, alpha * alpha % R
    ws = []
    for k in range(logD):
        e = ev[4 * k:4 * k + 4]
        if (e[0] + e[1]) % R != cur:
            return False, ws
        for lab, v in zip(("p0", "p1", "p2", "p3"), e):
            tr.absorb_fr(lab, v)
        w = tr.challenge_fr()
        ws.append(w)
        cur = lagrange(e, w)
        eqv = eq2(u[logD - 1 - k], w)
        aacc = aacc * eqv % R
        if k >= n1:
            a2acc = a2acc * eqv % R
    B = [inv((t + beta) % R) for t in T_public]
    T = list(T_public)
    for k in range(ceil_log2(N)):
        w = ws[n1 + k]
        h = len(B) // 2
        B = [(B[i] + w * (B[i + h] - B[i])) % R for i in range(h)]
        T = [(T[i] + w * (T[i + h] - T[i])) % R for i in range(h)]
    ratio = N * inv(D) % R
    rhs = (aacc * A_f * (S_f + beta) + ratio * a2acc * B[0] * (T[0] + beta) + A_f
           - ratio * m_f * B[0]) % R
    tr.absorb_fr("A_f", A_f)
    tr.absorb_fr("S_f", S_f)
    tr.absorb_fr("m_f", m_f)
    return cur == rhs, ws


# ---------------- Hadamard sumcheck (zkob_lookup.cuh:212-315) ----------------
def hp_prove(tr, claim, E, S, U):
    E, S, U = list(E), list(S), list(U)
    ev, ws = [], []
    while len(E) > 1:
        h = len(E) // 2
        p = [sum((E[i] + t * (E[i + h] - E[i])) * (S[i] + t * (S[i + h] - S[i]))
                 * (U[i] + t * (U[i + h] - U[i])) for i in range(h)) % R for t in range(4)]
        assert (p[0] + p[1]) % R == claim, "hadamard round inconsistency"
        for lab, v in zip(("hp0", "hp1", "hp2", "hp3"), p):
            tr.absorb_fr(lab, v)
        w = tr.challenge_fr()
        ws.append(w)
        ev += p
        claim = lagrange(p, w)

        def fold(tab):
            return [(tab[i] + w * (tab[i + h] - tab[i])) % R for i in range(h)]
        E, S, U = fold(E), fold(S), fold(U)
    return ev, dict(S_f2=S[0], U_f2=U[0], E_f=E[0], cur=claim), ws
