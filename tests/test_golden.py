"""The C oracle reproduces every golden fixture under tests/golden/ (written by
tests/golden/make_golden.py from the independent Python restatement)."""
import glob
import json
import os

import numpy as np
import pytest

from oracle import coracle as C
from oracle import pyref as P

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "*.json")))


def H(xs):
    return [int(x, 16) for x in xs]


def st_from(hexs):
    return np.frombuffer(bytes.fromhex(hexs), dtype=np.uint8).copy()


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_oracle_matches_golden(path):
    g = json.load(open(path))
    st = st_from(g["state_in"])
    if g["kind"] == "mm":
        B, IN, OUT = g["B"], g["IN"], g["OUT"]
        X = np.array(g["X"]).reshape(B, IN)
        W = np.array(g["W"]).reshape(IN, OUT)
        Y = np.array(g["Y"], dtype=np.int64).reshape(B, OUT)
        rc, d = C.mm_prove(st, X, W, Y, B, IN, OUT)
        assert rc == 0
        assert C.fr_to_ints(d["ev"]) == H(g["ev"])
        assert C.fr_to_ints(d["claims"]) == H(g["claims"])
        for k in ("u_batch", "u_output", "u_input"):
            assert C.fr_to_ints(d[k]) == H(g[k])
    elif g["kind"] == "lu":
        D, N, low, ln = g["D"], g["N"], g["low"], g["len"]
        S = C.ints_to_fr(g["S"])
        rc, m = C.lu_prep(S, low, N)
        assert rc == 0 and C.fr_to_ints(m) == g["m"]
        A = C.lu_inverse(S, np.array(P.to_limbs(int(g["beta"], 16)), np.uint32))
        assert C.fr_to_ints(A) == H(g["A"])
        T = C.range_table(low, ln, N)
        rc, d = C.lu_prove(st, A, S, T, m, C.ints_to_fr([int(g["alpha"], 16)])[0],
                           C.ints_to_fr([int(g["beta"], 16)])[0], C.ints_to_fr(H(g["u"])))
        assert rc == 0
        assert C.fr_to_ints(d["ev"]) == H(g["ev"])
        assert C.fr_to_ints(d["term"]) == H(g["term"])
        assert C.fr_to_ints(d["ws"]) == H(g["ws"])
    else:
        u = C.ints_to_fr(H(g["u"]))
        E = C.build_eq(u)
        rc, d = C.hp_prove(st, C.ints_to_fr([int(g["claim"], 16)])[0], E, C.ints_to_fr(H(g["S"])),
                           C.ints_to_fr(H(g["U"])))
        assert rc == 0
        assert C.fr_to_ints(d["ev"]) == H(g["ev"])
        assert C.fr_to_ints(d["term"]) == H(g["term"])
        assert C.fr_to_ints(d["ws"]) == H(g["ws"])
    assert bytes(st).hex() == g["state_out"]
