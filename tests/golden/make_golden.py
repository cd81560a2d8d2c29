"""Write the golden fixtures under tests/golden/ from oracle/pyref.py.

pyref is the independent pure-Python restatement (big integers, hashlib, MLEs by their
defining sums); the fixtures pin the C oracle (zkh_oracle.c) and, through it, the GPU
library.  Shapes are the reference's own test shapes (vrf_toy_matmul.cu:249-260,
zkob_fc.cu:1246-1248, vrf_toy_lookup.cu:323-335, zkob_rescale.cu:539-541) plus
BASELINE.json config 1 (64x128 times 128x64 fp8-e4m3 scaled ints, seeded).
The reference has no golden vectors for this path (its tests pin relations with random
challenges), so these are the builder's vectors; nothing from the reference is run.

Usage: python tests/golden/make_golden.py
"""
import importlib.util
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
from oracle import pyref as P  # noqa: E402

spec = importlib.util.spec_from_file_location("zkh_synth", os.path.join(ROOT, "zk-hillclimb_amd", "synth.py"))
synth = importlib.util.module_from_spec(spec)
spec.loader.exec_module(synth)


def hx(x):
    return "%064x" % x


def mm_case(name, B, IN, OUT, seed, fp8_x):
    rng = np.random.default_rng(seed)
    X = synth.fp8_e4m3_ints(rng, (B, IN)) if fp8_x else synth.gaussian_int16(rng, (B, IN))
    W = synth.fp8_e4m3_ints(rng, (IN, OUT))
    Y = synth.matmul_exact(X, W)
    tr = P.Transcript("golden:" + name)
    for lab, v in (("B", B), ("IN", IN), ("OUT", OUT)):
        tr.absorb_u32(lab, v)
    st0 = tr.state
    out = P.mm_prove(tr, [int(v) for v in X.ravel()], [int(v) for v in W.ravel()],
                     [int(v) for v in Y.ravel()], B, IN, OUT)
    return {"kind": "mm", "name": name, "B": B, "IN": IN, "OUT": OUT,
            "X": X.ravel().tolist(), "W": W.ravel().tolist(), "Y": Y.ravel().tolist(),
            "state_in": st0.hex(), "state_out": tr.state.hex(),
            "ev": [hx(v) for v in out["ev"]],
            "claims": [hx(out[k]) for k in ("claim", "claim_X", "claim_W")],
            "u_batch": [hx(v) for v in out["u_batch"]], "u_output": [hx(v) for v in out["u_output"]],
            "u_input": [hx(v) for v in out["u_input"]]}


def lu_case(name, D, N, low, ln, seed):
    rng = np.random.default_rng(seed)
    vals = [int(v) for v in rng.integers(low, low + ln, size=D)]
    S = [v % P.R for v in vals]
    T = P.range_table(low, ln, N)
    m = P.lu_prep(S, low, N)
    tr = P.Transcript("golden:" + name)
    beta = tr.challenge_fr()
    A = [P.inv((s + beta) % P.R) for s in S]
    alpha = tr.challenge_fr()
    u = tr.challenge_vec(P.ceil_log2(D))
    st0 = tr.state
    ev, term, ws = P.lu_prove(tr, A, S, T, m, alpha, beta, u)
    return {"kind": "lu", "name": name, "D": D, "N": N, "low": low, "len": ln, "S": vals,
            "state_in": st0.hex(), "state_out": tr.state.hex(), "alpha": hx(alpha),
            "beta": hx(beta), "u": [hx(v) for v in u], "m": m, "A": [hx(v) for v in A],
            "ev": [hx(v) for v in ev],
            "term": [hx(term[k]) for k in ("A_f", "S_f", "B_f", "T_f", "m_f")],
            "ws": [hx(v) for v in ws]}


def hp_case(name, k, seed):
    rng = np.random.default_rng(seed)
    n = 1 << k
    tr = P.Transcript("golden:" + name)
    u = tr.challenge_vec(k)
    E = P.eq_table(u)
    S = [int(v) % P.R for v in rng.integers(-2**31, 2**31, size=n)]
    U = [int(v) % P.R for v in rng.integers(-2**31, 2**31, size=n)]
    claim = sum(e * s * x for e, s, x in zip(E, S, U)) % P.R
    tr.absorb_fr("claim_H", claim)
    st0 = tr.state
    ev, term, ws = P.hp_prove(tr, claim, E, S, U)
    return {"kind": "hp", "name": name, "k": k, "S": [hx(v) for v in S], "U": [hx(v) for v in U],
            "u": [hx(v) for v in u], "claim": hx(claim), "state_in": st0.hex(),
            "state_out": tr.state.hex(), "ev": [hx(v) for v in ev],
            "term": [hx(term["S_f2"]), hx(term["U_f2"]), hx(term["E_f"])], "ws": [hx(v) for v in ws]}


def main():
    cases = [
        mm_case("toy_4_8_4", 4, 8, 4, 1, True),
        mm_case("toy_4_6_3", 4, 6, 3, 2, True),
        mm_case("toy_2_8_3", 2, 8, 3, 3, False),
        mm_case("toy_8_16_16", 8, 16, 16, 4, False),
        mm_case("fc_16_12_5", 16, 12, 5, 5, True),
        mm_case("cfg1_64_128_64", 64, 128, 64, 0x5EED0001, True),
        lu_case("toy_32_8", 32, 8, -3, 5, 11),
        lu_case("toy_16_16", 16, 16, 0, 16, 12),
        lu_case("toy_64_4", 64, 4, -2, 3, 13),
        lu_case("rescale_32_4", 32, 4, -2, 4, 14),
        hp_case("hp_k3", 3, 21),
        hp_case("hp_k5", 5, 22),
    ]
    for c in cases:
        with open(os.path.join(HERE, c["name"] + ".json"), "w") as f:
            json.dump(c, f, separators=(",", ":"))
    print("wrote %d fixtures" % len(cases))


if __name__ == "__main__":
    main()
