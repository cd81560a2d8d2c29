"""GPU parity at BASELINE.json's own configurations (C2-C5), full size, against the C oracle.

Bar: bit-exact field elements and identical transcript states, as in test_gpu_parity.py.
The oracle follows the reference's schedule (zkob_fc.cu:254-345, zkob_rescale.cu:110-150,
zkob_glu.cu:146-247, zkob_rope.cu:215-281) on all host cores.  One shortcut keeps the
2^22 / 2^25 lookups to seconds: the GPU's batched inverse A = 1/(S + beta) is checked
entry by entry against the identity A (S + beta) = 1 (inverse(0) = 0), which fixes A
uniquely, and that A then enters the oracle's lookup proof; everything else (the mapping,
the combiner, multiplicities, the table inverse inside the proof, every round) is the
oracle's own computation.

- C2: llama-68m FFN matmuls at seq 128 (768 -> 3072 -> 768).
- C3: logUp, 2^20 witnesses uniform in [-2^15, 2^15) against the 2^16 range table.
- C4: TinyLlama-1.1B layer at seq 512: the 7 matmuls; the SwiGLU mapping lookup (D = N =
  2^22) with its Hadamard sumcheck; the RoPE q / k Hadamard sumchecks (2^20, 2^17).
- C5: OpenLLaMA-3B layer at seq 2048: the 7 matmuls (3200 / 8640, non-power-of-two zero
  fill); the SwiGLU lookup on the 2048 x 16384 grid (2^25 witnesses) against a 2^22 table
  (three phase-1 rounds, then phase 2) with its 2^25 Hadamard sumcheck.
"""
import importlib.util
import os
import struct
import sys

import numpy as np
import pytest

from oracle import coracle as C
from oracle import pyref as P

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _synth():
    if "zkh_synth" not in sys.modules:
        spec = importlib.util.spec_from_file_location("zkh_synth", os.path.join(ROOT, "zk-hillclimb_amd", "synth.py"))
        mod = importlib.util.module_from_spec(spec)
        sys.modules["zkh_synth"] = mod
        spec.loader.exec_module(mod)
    return sys.modules["zkh_synth"]


S = _synth()


def fr_eq(a, b):
    return np.array_equal(np.asarray(a, np.uint32).reshape(-1, 8), np.asarray(b, np.uint32).reshape(-1, 8))


def both(zkh, label):
    st_g, st_o = zkh.transcript(label), C.tr_init(label)
    assert bytes(st_g) == bytes(st_o)
    return st_g, st_o


def absorb_both(zkh, st_g, st_o, label, data):
    zkh.absorb(st_g, label, data)
    C.tr_absorb(st_o, label, data)


def chal_both(zkh, st_g, st_o, n=None):
    if n is None:
        a, b = zkh.challenge(st_g), C.tr_challenge_fr(st_o)
        assert fr_eq(a, b)
        return b
    return np.array([chal_both(zkh, st_g, st_o) for _ in range(n)]).reshape(-1, 8)


def log(msg):
    print("[configs] " + msg, flush=True)


# ------------------------------------------------------------------ matmul sumchecks
def _matmuls(zkh, ctx, cfg, names, seed):
    c = S.CONFIGS[cfg]
    B = c["B"]
    rng = S.rng_for(seed)
    items, wants, sts, keep = [], [], [], []
    for name, IN, OUT in c["matmuls"]:
        X, W, Y = S.matmul_inputs(rng, B, IN, OUT)  # drawn for every matmul: fixed inputs per name
        if name not in names:
            continue
        st_g, st_o = both(zkh, "%s:%s" % (cfg, name))
        for lab, v in (("B", B), ("IN", IN), ("OUT", OUT)):
            absorb_both(zkh, st_g, st_o, lab, struct.pack("<I", v))
        log("%s %s (%d, %d, %d): oracle" % (cfg, name, B, IN, OUT))
        rc, want = C.mm_prove(st_o, X, W, Y, B, IN, OUT)
        assert rc == 0
        t = (ctx.from_i32(X), ctx.weights_i32(W, IN, OUT), ctx.from_i64(Y))
        keep.append(t)
        items.append((st_g, t[0], t[1], t[2], B, IN, OUT))
        wants.append((name, want))
        sts.append((st_g, st_o))
    log("%s %s: GPU batch" % (cfg, ",".join(names)))
    outs, status = ctx.mm_prove_batch(items)
    assert status == [0] * len(items)
    for got, (name, want), (st_g, st_o) in zip(outs, wants, sts):
        for key in ("ev", "claims", "u_batch", "u_output", "u_input"):
            assert fr_eq(got[key], want[key]), (name, key)
        assert bytes(st_g) == bytes(st_o), name


def test_c2_ffn_matmuls(zkh, ctx):
    _matmuls(zkh, ctx, "C2", ("up", "down"), 2)


def test_c4_matmuls(zkh, ctx):
    _matmuls(zkh, ctx, "C4", ("q", "k", "v", "o", "gate", "up", "down"), 4)


def test_c5_attention_matmuls(zkh, ctx):
    _matmuls(zkh, ctx, "C5", ("q", "k", "v", "o"), 5)


def test_c5_ffn_matmuls(zkh, ctx):
    _matmuls(zkh, ctx, "C5", ("gate", "up", "down"), 5)


# ------------------------------------------------------------------ logUp (C3)
def test_c3_logup(zkh, ctx):
    c = S.CONFIGS["C3"]
    D, N, low = c["D"], c["N"], c["low"]
    rng = S.rng_for(3)
    vals = rng.integers(low, low + N, size=D).astype(np.int32)
    Sf = C.ints_to_fr(vals)
    T = C.range_table(low, N, N)
    st_g, st_o = both(zkh, "C3:rescale")
    rc, m = C.lu_prep(Sf, low, N)
    assert rc == 0
    Sg = ctx.from_i32(vals)
    mg = ctx.lu_prep(Sg, low, N)
    assert fr_eq(mg.to_fr(), m)
    Tg = ctx.range_table(low, N, N)
    assert fr_eq(Tg.to_fr(), T)
    beta = chal_both(zkh, st_g, st_o)
    log("C3: oracle inverse (Fermat, 2^20)")
    A = C.lu_inverse(Sf, beta)
    Ag = ctx.lu_inverse(Sg, beta)
    assert fr_eq(Ag.to_fr(), A)
    alpha = chal_both(zkh, st_g, st_o)
    u = chal_both(zkh, st_g, st_o, P.ceil_log2(D))
    log("C3: oracle proof")
    rc, want = C.lu_prove(st_o, A, Sf, T, m, alpha, beta, u)
    assert rc == 0
    got = ctx.lu_prove(st_g, Ag, Sg, Tg, mg, alpha, beta, u)
    for key in ("ev", "term", "ws"):
        assert fr_eq(got[key], want[key]), key
    assert bytes(st_g) == bytes(st_o)


def test_c3_logup_range_inverse(zkh, ctx):
    """C3 through the entry point the bench times: zkh_lu_range_inverse (A read off the
    table inverse, which zkh_lu_prove then takes over; zkob_rescale.cu:119-146), the whole
    proof against the oracle's separate steps (Fermat inverses of S and of T)."""
    c = S.CONFIGS["C3"]
    D, N, low = c["D"], c["N"], c["low"]
    rng = S.rng_for(3)
    vals = rng.integers(low, low + N, size=D).astype(np.int32)
    Sf = C.ints_to_fr(vals)
    T = C.range_table(low, N, N)
    st_g, st_o = both(zkh, "C3:rescale:fused")
    rc, m = C.lu_prep(Sf, low, N)
    assert rc == 0
    Sg = ctx.from_i32(vals)
    mg = ctx.lu_prep(Sg, low, N)
    Tg = ctx.range_table(low, N, N)
    beta = chal_both(zkh, st_g, st_o)
    log("C3 fused: oracle inverse (Fermat, 2^20)")
    A = C.lu_inverse(Sf, beta)
    Ag = ctx.lu_range_inverse(Sg, low, Tg, beta)
    assert fr_eq(Ag.to_fr(), A)
    alpha = chal_both(zkh, st_g, st_o)
    u = chal_both(zkh, st_g, st_o, P.ceil_log2(D))
    log("C3 fused: oracle proof")
    rc, want = C.lu_prove(st_o, A, Sf, T, m, alpha, beta, u)
    assert rc == 0
    got = ctx.lu_prove(st_g, Ag, Sg, Tg, mg, alpha, beta, u)
    for key in ("ev", "term", "ws"):
        assert fr_eq(got[key], want[key]), key
    assert bytes(st_g) == bytes(st_o)


# ------------------------------------------------------------------ SwiGLU (C4, C5)
def _glu(zkh, ctx, cfg, seed, parts=("lookup", "hadamard"), fused=False):
    """zkob_glu.cu:146-247: mapping lookup of G into the silu table, combiner
    comb = G + r S against T_comb = T + r silu, logUp proof, then the eq-weighted Hadamard
    sumcheck of H = S (.) U, on the GPU and on the oracle side by side.  With parts =
    ("hadamard",) the lookup runs on the GPU only (its challenges advance both transcripts
    identically: the oracle replays the same absorbs from the GPU's round polynomials).
    fused: the GPU side runs the entry points the bench times, zkh_lu_tuple_inverse (comb,
    T_comb and A in one call, A read off the table inverse that zkh_lu_prove takes over) and
    zkh_hp_prove_eq_claim (claim_H from the Hadamard prover's first round, absorbed inside),
    against the oracle's separate steps (zkob_glu.cu:155-170, :231-247)."""
    c = S.CONFIGS[cfg]
    inp = S.glu_inputs(S.rng_for(seed), c["B"], c["ffn"], N=c["glu_table"])
    D, N, low = inp["D"], inp["N"], inp["low"]
    logD = P.ceil_log2(D)
    G = inp["G"].ravel()
    U = inp["U"].ravel()
    silu = inp["silu"]
    st_g, st_o = both(zkh, "%s:swiglu" % cfg)
    for lab, v in (("B", c["B"]), ("C", c["ffn"]), ("LOW", low & 0xFFFFFFFF), ("LEN", N)):
        absorb_both(zkh, st_g, st_o, lab, struct.pack("<I", v))
    log("%s SwiGLU: D = 2^%d, N = 2^%d" % (cfg, logD, P.ceil_log2(N)))
    # GPU: mapping, challenges, combiner, inverse
    Gg, Ug, mapped = ctx.from_i32(G), ctx.from_i32(U), ctx.from_i32(silu)
    Tg = ctx.range_table(low, N, N)
    Sg, mg = ctx.lu_mapping(Gg, low, mapped)
    # oracle: the mapped witness and multiplicities
    s_vals = silu[G.astype(np.int64) - low]
    Sf = C.ints_to_fr(s_vals)
    Gf = C.ints_to_fr(G)
    rc, m = C.lu_prep(Gf, low, N)
    assert rc == 0
    assert fr_eq(Sg.to_fr(), Sf)
    assert fr_eq(mg.to_fr(), m)
    r = chal_both(zkh, st_g, st_o)
    beta = chal_both(zkh, st_g, st_o)
    if fused:
        comb_g, tcomb_g, Ag = ctx.lu_tuple_inverse(Gg, low, Tg, mapped, r, beta, S=Sg)
    else:
        comb_g = ctx.axpy(Gg, r, Sg)
        tcomb_g = ctx.axpy(Tg, r, mapped)
    comb = C.axpy(Gf, r, Sf)
    tcomb = C.axpy(C.range_table(low, N, N), r, C.ints_to_fr(silu))
    assert fr_eq(comb_g.to_fr(), comb)
    assert fr_eq(tcomb_g.to_fr(), tcomb)
    if not fused:
        Ag = ctx.lu_inverse(comb_g, beta)
    A = Ag.to_fr()
    assert C.check_inverse(comb, A, beta) == 0  # fixes A = 1/(comb + beta) entry by entry
    absorb_both(zkh, st_g, st_o, "com_A", bytes(range(144)))
    alpha = chal_both(zkh, st_g, st_o)
    u = chal_both(zkh, st_g, st_o, logD)
    got = ctx.lu_prove(st_g, Ag, comb_g, tcomb_g, mg, alpha, beta, u)
    if "lookup" in parts:
        log("%s SwiGLU: oracle lookup proof" % cfg)
        rc, want = C.lu_prove(st_o, A, comb, tcomb, m, alpha, beta, u)
        assert rc == 0
        for key in ("ev", "term", "ws"):
            assert fr_eq(got[key], want[key]), key
    else:  # the lookup's transcript effects, from the GPU's proof
        for k in range(logD):
            for t, lab in enumerate(("p0", "p1", "p2", "p3")):
                C.tr_absorb(st_o, lab, got["ev"][4 * k + t].tobytes())
            assert fr_eq(C.tr_challenge_fr(st_o), got["ws"][k])
        for lab, i in (("A_f", 0), ("S_f", 1), ("m_f", 4)):
            C.tr_absorb(st_o, lab, got["term"][i].tobytes())
    assert bytes(st_g) == bytes(st_o)
    del A, comb, tcomb, Gf
    if "hadamard" not in parts:
        return
    # Hadamard sumcheck of H = S (.) U at the fresh point u_h (zkob_glu.cu:236-247)
    u_h = chal_both(zkh, st_g, st_o, logD)
    Uf = C.ints_to_fr(U)
    H = C.hadamard(Sf, Uf)
    rc, claim = C.me(H, u_h)
    assert rc == 0
    del H
    if fused:
        # the claim absorbed inside the call, before the first round's evaluations
        C.tr_absorb(st_o, "claim_H", claim.tobytes())
    else:
        claim_g = ctx.me(ctx.hadamard(Sg, Ug), u_h)
        assert fr_eq(claim_g, claim)
        absorb_both(zkh, st_g, st_o, "claim_H", claim.tobytes())
    log("%s SwiGLU: oracle Hadamard proof" % cfg)
    E = C.build_eq(u_h)
    rc, want = C.hp_prove(st_o, claim, E, Sf, Uf)
    assert rc == 0
    if fused:
        got = ctx.hp_prove_eq_claim(st_g, "claim_H", u_h, Sg, Ug)
        assert fr_eq(got["claim"], claim)
    else:
        got = ctx.hp_prove_eq(st_g, claim_g, u_h, Sg, Ug)
    for key in ("ev", "term", "ws"):
        assert fr_eq(got[key], want[key]), key
    assert bytes(st_g) == bytes(st_o)


def test_c4_swiglu(zkh, ctx):
    _glu(zkh, ctx, "C4", 4)


def test_c5_swiglu_lookup(zkh, ctx):
    _glu(zkh, ctx, "C5", 5, parts=("lookup",))


def test_c5_swiglu_hadamard(zkh, ctx):
    _glu(zkh, ctx, "C5", 5, parts=("hadamard",))


def test_c4_swiglu_fused(zkh, ctx):
    _glu(zkh, ctx, "C4", 4, fused=True)


def test_c5_swiglu_lookup_fused(zkh, ctx):
    """2^25 witnesses against the 2^22 table: A gathered from the table inverse, which the
    proof takes over and folds through its three phase-1 rounds into phase 2."""
    _glu(zkh, ctx, "C5", 5, parts=("lookup",), fused=True)


def test_c5_swiglu_hadamard_fused(zkh, ctx):
    _glu(zkh, ctx, "C5", 5, parts=("hadamard",), fused=True)


# ------------------------------------------------------------------ RoPE (C4)
@pytest.mark.parametrize("which", ["q", "k"])
def test_c4_rope(zkh, ctx, which):
    """zkob_rope.cu:215-281: c1 = sum eq(u,b) W1(b) T(b), c2 = sum eq(u,b) W2(b) Tx(b), each
    proven by the explicit-E Hadamard sumcheck with U = 1."""
    c = S.CONFIGS["C4"]
    cols = dict(c["rope"])[which]
    inp = S.rope_inputs(S.rng_for(40 + len(which) + cols), c["B"], cols, c["hd"])
    D = inp["D"]
    logD = P.ceil_log2(D)
    st_g, st_o = both(zkh, "C4:rope:" + which)
    u = chal_both(zkh, st_g, st_o, logD)
    Eu = C.build_eq(u)
    Eu_g = ctx.eq_table(u)
    assert fr_eq(Eu_g.to_fr(), Eu)
    ONE = C.ints_to_fr(np.ones(D, np.int64))
    ONE_g = ctx.from_i32(np.ones(D, np.int32))
    for lab, Wk, Sk in (("c1", "W1", "T"), ("c2", "W2", "Tx")):
        Wf, Sv = C.ints_to_fr(inp[Wk].ravel()), C.ints_to_fr(inp[Sk].ravel())
        E = C.hadamard(Eu, Wf)
        claim = np.zeros(8, np.uint32)
        C.lib().or_sum(C._p(np.ascontiguousarray(C.hadamard(E, Sv))), D, C._p(claim))
        E_g = ctx.hadamard(Eu_g, ctx.from_i32(inp[Wk].ravel()))
        S_g = ctx.from_i32(inp[Sk].ravel())
        claim_g = ctx.sum(ctx.hadamard(E_g, S_g))
        assert fr_eq(claim_g, claim)
        absorb_both(zkh, st_g, st_o, lab, claim.tobytes())
        rc, want = C.hp_prove(st_o, claim, E, Sv, ONE)
        assert rc == 0
        got = ctx.hp_prove(st_g, claim_g, E_g, S_g, ONE_g)
        for key in ("ev", "term", "ws"):
            assert fr_eq(got[key], want[key]), (lab, key)
        absorb_both(zkh, st_g, st_o, "S_f2", want["term"][0].tobytes())
        absorb_both(zkh, st_g, st_o, "U_f2", want["term"][1].tobytes())
        assert bytes(st_g) == bytes(st_o)
