#!/usr/bin/env python3
"""Benchmark: the Fr sumcheck hot path on a TinyLlama-1.1B-shaped layer (seq 512), one MI355X.

Metric: "Fr elements bound/sec in matmul sumcheck; prove s/layer at
TinyLlama-1.1B".

- A *step* is the 7 matmul (zkip) sumchecks of one layer -- Q, K, V, O (d=2048, 4 KV heads
  x 64 = 256), gate/up (2048 -> 5632), down (5632 -> 2048) at B = 512 -- each the
  zkob_fc.cu:259-440 segment with its own transcript, proven in one batched call
  (zkh_mm_prove_batch: one launch and one host synchronisation per round for all 7).
  value = elements bound per second, with elements bound E = B*IN + IN*OUT + B*OUT + 2*IN
  per matmul (every input table entry bound once).
- prove_s_per_layer additionally runs the layer's other hot-path segments concurrently:
  the SwiGLU mapping lookup (logUp, D = N = 2^22) with its Hadamard sumcheck (2^22), and
  the RoPE eq-weighted Hadamard sumchecks (q: 2 x 2^20, k: 2 x 2^17).
  Excluded, as in the reference's accounting: Pedersen commitments (their transcript
  absorbs use fixed synthetic blobs), IPA openings, the witness GEMM Y = X*W (computed
  in setup), process init.
- commitments: the layer's com_X, com_W, com_Y (zkob_fc.cu:215-230) with zkh_commit,
  byte-identical to the reference's commit_pippenger, reported beside the metric (not part
  of it) with their own CPU baseline (the C oracle on one row each of X, W, Y); openings:
  the layer's 21 IPA openings (zkob_fc.cu:473-483, zkh_ipa_prove) after the sumchecks, with
  the oracle's time for one of them as CPU baseline.
- Inputs are seeded synthetic tensors (fp8-e4m3 weights as scaled ints, Gaussian int16
  activations), resident in HBM before the timed region.
- The throughput steps carry no timing events (stamping them costs the host ~20 us per
  step).  roofline: the dominant kernel's algorithmic bytes over its duration in a second
  live pass of the same steps, from HIP events that the launch itself stamps at its start
  and end (hipExtLaunchKernel on the library's stream, read through the zkh_prof_* hooks),
  so the figure is the kernel's execution time as a kernel trace reports it.
- layer_roofline: the same for the dominant kernel class of the SwiGLU segment, and (valu)
  its Montgomery products per second against fr_mul_peak, the device-wide rate of the
  library's multiply measured by zkh_calib_fr_mul in the same run.
- fr_inputs: the 7 matmuls with X, W, Y bound as field-element tensors (32 B per entry).
- configs: BASELINE configs C2 (llama-68m FFN matmuls), C3 (logUp 2^20 vs 2^16) and C5
  (OpenLLaMA-3B layer at seq 2048: matmuls, SwiGLU lookup 2^25 vs 2^22 + Hadamard).
- cpu_baseline: the C oracle (scalar port of the reference schedule) on the Q, K, V, O
  matmuls on one thread and on all cores, on the GPU proofs' own transcripts, each proof
  asserted byte-identical to the GPU's; layer.cpu_baseline: the whole layer hot path the
  same way (all cores; one thread estimated from bounded samples); C3 likewise.
"""
import argparse
import concurrent.futures
import gc
import hashlib
import importlib.util
import json
import os
import struct
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
HBM_PEAK_GBS = 8000.0
LATENCY_BOUND = {"zkip_rounds"}
# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE runs: the
# counters of a 256 MiB device copy read 0.500x (FETCH) and 1.000x (WRITE) of its bytes, so
# FETCH is scaled by 2.  eqdot: profiles/eqdot_hbm_traffic_tinyllama.txt (one launch per
# matmul step); lu_phase2: profiles/swiglu_counters_tinyllama.txt (the 9 launches of the class
# in one SwiGLU segment, 2450.0 MB, averaged per launch like bytes_per_launch).
TRAFFIC = {"eqdot": 315.4e6, "lu_phase2": 272.2e6}


def load_pkg():
    path = os.path.join(ROOT, "zk-hillclimb_amd", "__init__.py")
    spec = importlib.util.spec_from_file_location("zkh", path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules["zkh"] = mod
    spec.loader.exec_module(mod)
    spec = importlib.util.spec_from_file_location("zkh_synth", os.path.join(ROOT, "zk-hillclimb_amd", "synth.py"))
    synth = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(synth)
    return mod, synth


def blob(label, nbytes):
    """Deterministic stand-in bytes for a commitment tensor (commitments are outside the path)."""
    out = bytearray()
    ctr = 0
    while len(out) < nbytes:
        out += hashlib.sha256(b"%s:%d" % (label.encode(), ctr)).digest()
        ctr += 1
    return bytes(out[:nbytes])


def pow2(n):
    return 1 << ((n - 1).bit_length()) if n > 1 else 1


LAYER = dict(B=512, d=2048, kv=256, ffn=5632, heads=32, hd=64)


def _oracle():
    """The C oracle, imported only by the CPU-baseline legs (test infrastructure)."""
    sys.path.insert(0, ROOT)
    from oracle import coracle
    return coracle


class MatmulJob:
    """One zkob_fc sumcheck segment (zkob_fc.cu:254-345) with its own transcript; fr=True binds
    X, W, Y as field-element tensors (the FrTensors of zkob_fc.cu:276-277) instead of ints."""

    def __init__(self, zkh, synth, rng, name, B, IN, OUT, tag="cfg4:layer0", fr=False, inputs=None):
        self.zkh, self.name, self.B, self.IN, self.OUT = zkh, name, B, IN, OUT
        X, W, Y = inputs if inputs is not None else synth.matmul_inputs(rng, B, IN, OUT)
        self.ctx = zkh.Context(0)
        if fr:
            self.X = self.ctx.from_fr(zkh.ints_to_fr(X))
            self.W = self.ctx.from_fr(zkh.ints_to_fr(W))
            self.Y = self.ctx.from_fr(zkh.ints_to_fr(Y))
        else:
            self.X = self.ctx.from_i32(X)
            self.W = self.ctx.weights_i32(W, IN, OUT)
            self.Y = self.ctx.from_i64(Y)
        st = zkh.transcript("%s.%s" % (tag, name))
        for lab, v in (("B", B), ("IN", IN), ("OUT", OUT)):
            zkh.absorb(st, lab, struct.pack("<I", v))
        zkh.absorb(st, "com_X", blob(name + "X", pow2(B) * 144))
        zkh.absorb(st, "com_W", blob(name + "W", pow2(IN) * 144))
        zkh.absorb(st, "com_Y", blob(name + "Y", pow2(B) * 144))
        self.st0 = st
        self.elements = synth.mm_elements(B, IN, OUT)
        self.inputs = (X, W, Y)

    def run(self):
        st = self.st0.copy()
        out = self.ctx.mm_prove(st, self.X, self.W, self.Y, self.B, self.IN, self.OUT)
        return out["claims"].tobytes() + st.tobytes()

    @staticmethod
    def result(out, st):
        """Bytes that identify a proof: round evaluations, claims, challenges, transcript."""
        return b"".join(out[k].tobytes() for k in ("ev", "claims", "u_batch", "u_output", "u_input")) + st.tobytes()

    def cpu_run(self):
        C = _oracle()
        st = self.st0.copy()
        rc, out = C.mm_prove(st, *self.inputs, self.B, self.IN, self.OUT)
        assert rc == 0
        return self.result(out, st)


class GluJob:
    """SwiGLU obligation hot path (zkob_glu.cu:146-247): mapping lookup of G into the silu
    table, combiner comb = G + r S against T_comb = T + r silu, the logUp proof, and the
    eq-weighted Hadamard sumcheck of H = S (.) U."""

    def __init__(self, zkh, synth, rng, B, C, N=None, tag="cfg4:layer0", inputs=None):
        self.zkh = zkh
        inp = inputs if inputs is not None else synth.glu_inputs(rng, B, C, N=N)
        self.inp = inp
        self.D, self.N, self.low = inp["D"], inp["N"], inp["low"]
        self.ctx = zkh.Context(0)
        self.G = self.ctx.from_i32(inp["G"].ravel())
        self.U = self.ctx.from_i32(inp["U"].ravel())
        self.mapped = self.ctx.from_i32(inp["silu"])
        self.T = self.ctx.range_table(self.low, self.N, self.N)
        st = zkh.transcript(tag + ".swiglu")
        for lab, v in (("B", B), ("C", C), ("LOW", self.low & 0xFFFFFFFF), ("LEN", self.N)):
            zkh.absorb(st, lab, struct.pack("<I", v))
        for lab in ("com_G", "com_S", "com_U", "com_H", "com_m"):
            zkh.absorb(st, lab, blob("glu" + lab, inp["Bp"] * 144))
        self.st0 = st
        self.comA = blob("gluA", inp["Bp"] * 144)
        self.logD = self.D.bit_length() - 1

    def run(self):
        zkh, c = self.zkh, self.ctx
        st = self.st0.copy()
        S, m = c.lu_mapping(self.G, self.low, self.mapped)
        r = zkh.challenge(st)
        beta = zkh.challenge(st)
        comb, Tcomb, A = c.lu_tuple_inverse(self.G, self.low, self.T, self.mapped, r, beta, S=S)
        zkh.absorb(st, "com_A", self.comA)
        alpha = zkh.challenge(st)
        u = zkh.challenges(st, self.logD)
        lu = c.lu_prove(st, A, comb, Tcomb, m, alpha, beta, u)
        u_h = zkh.challenges(st, self.logD)
        # claim_H = H(u_h) of H = S (.) U, absorbed, then the Hadamard sumcheck: one call that
        # takes the claim from the first round's sums (same transcript bytes as forming H,
        # evaluating it and absorbing the claim before zkh_hp_prove_eq)
        hp = c.hp_prove_eq_claim(st, "claim_H", u_h, S, self.U)
        zkh.absorb(st, "S_f2", hp["term"][0].tobytes())
        zkh.absorb(st, "U_f2", hp["term"][1].tobytes())
        return lu["ev"].tobytes() + lu["term"].tobytes() + hp["ev"].tobytes() + hp["term"].tobytes() + st.tobytes()

    def cpu_run(self):
        """The same segment on the C oracle (the reference's schedule: per-element Fermat
        inverses, per-round MLE re-evaluation), on the same transcript."""
        C = _oracle()
        inp, low, N = self.inp, self.low, self.N
        G = inp["G"].ravel()
        st = self.st0.copy()
        Gf = C.ints_to_fr(G)
        Sf = C.ints_to_fr(inp["silu"][G.astype(np.int64) - low])
        Uf = C.ints_to_fr(inp["U"].ravel())
        rc, m = C.lu_prep(Gf, low, N)
        assert rc == 0
        r = C.tr_challenge_fr(st)
        beta = C.tr_challenge_fr(st)
        comb = C.axpy(Gf, r, Sf)
        Tcomb = C.axpy(C.range_table(low, N, N), r, C.ints_to_fr(inp["silu"]))
        A = C.lu_inverse(comb, beta)
        C.tr_absorb(st, "com_A", self.comA)
        alpha = C.tr_challenge_fr(st)
        u = np.array([C.tr_challenge_fr(st) for _ in range(self.logD)])
        rc, lu = C.lu_prove(st, A, comb, Tcomb, m, alpha, beta, u)
        assert rc == 0
        u_h = np.array([C.tr_challenge_fr(st) for _ in range(self.logD)])
        rc, claim = C.me(C.hadamard(Sf, Uf), u_h)
        C.tr_absorb(st, "claim_H", claim.tobytes())
        rc, hp = C.hp_prove(st, claim, C.build_eq(u_h), Sf, Uf)
        assert rc == 0
        C.tr_absorb(st, "S_f2", hp["term"][0].tobytes())
        C.tr_absorb(st, "U_f2", hp["term"][1].tobytes())
        return lu["ev"].tobytes() + lu["term"].tobytes() + hp["ev"].tobytes() + hp["term"].tobytes() + st.tobytes()


class RopeJob:
    """One RoPE obligation (zkob_rope.cu:215-281): two eq-weighted Hadamard sumchecks
    c1 = sum eq(u,b) W1(b) T(b) and c2 = sum eq(u,b) W2(b) Tx(b), with U = 1."""

    def __init__(self, zkh, synth, rng, name, B, C, HD=64, tag="cfg4:layer0"):
        self.zkh = zkh
        self.inp = inp = synth.rope_inputs(rng, B, C, HD)
        self.D = inp["D"]
        self.logD = self.D.bit_length() - 1
        self.ctx = c = zkh.Context(0)
        self.T, self.Tx = c.from_i32(inp["T"].ravel()), c.from_i32(inp["Tx"].ravel())
        self.W1, self.W2 = c.from_i32(inp["W1"].ravel()), c.from_i32(inp["W2"].ravel())
        self.ONE = c.from_i32(np.ones(self.D, np.int32))
        st = zkh.transcript(tag + ".rope." + name)
        for lab, v in (("B", B), ("C", C), ("HD", HD), ("SCALE_R", 16)):
            zkh.absorb(st, lab, struct.pack("<I", v))
        zkh.absorb(st, "com_T", blob("rope" + name + "T", inp["Bp"] * 144))
        zkh.absorb(st, "com_Y64", blob("rope" + name + "Y", inp["Bp"] * 144))
        self.st0 = st

    def run(self):
        zkh, c = self.zkh, self.ctx
        st = self.st0.copy()
        u = zkh.challenges(st, self.logD)
        Eu = c.eq_table(u)
        outs = []
        for lab, W, S in (("c1", self.W1, self.T), ("c2", self.W2, self.Tx)):
            E = c.hadamard(Eu, W)
            # the claim sum(E S U) and its absorb inside the call, taken from the first round's
            # sums (same transcript bytes as the product, its sum and the absorb before hp_prove)
            hp = c.hp_prove_claim(st, lab, E, S, self.ONE)
            zkh.absorb(st, "S_f2", hp["term"][0].tobytes())
            zkh.absorb(st, "U_f2", hp["term"][1].tobytes())
            outs.append(hp["ev"].tobytes() + hp["term"].tobytes())
        return b"".join(outs) + st.tobytes()

    def cpu_run(self):
        C = _oracle()
        st = self.st0.copy()
        u = np.array([C.tr_challenge_fr(st) for _ in range(self.logD)])
        Eu = C.build_eq(u)
        one = C.ints_to_fr(np.ones(self.D, np.int64))
        outs = []
        for lab, Wk, Sk in (("c1", "W1", "T"), ("c2", "W2", "Tx")):
            Sf = C.ints_to_fr(self.inp[Sk].ravel())
            E = C.hadamard(Eu, C.ints_to_fr(self.inp[Wk].ravel()))
            claim = np.zeros(8, np.uint32)
            C.lib().or_sum(C._p(np.ascontiguousarray(C.hadamard(E, Sf))), self.D, C._p(claim))
            C.tr_absorb(st, lab, claim.tobytes())
            rc, hp = C.hp_prove(st, claim, E, Sf, one)
            assert rc == 0
            C.tr_absorb(st, "S_f2", hp["term"][0].tobytes())
            C.tr_absorb(st, "U_f2", hp["term"][1].tobytes())
            outs.append(hp["ev"].tobytes() + hp["term"].tobytes())
        return b"".join(outs) + st.tobytes()


class LookupJob:
    """BASELINE config 3 / zkob_rescale's lookup (zkob_rescale.cu:110-150): 2^20 witnesses
    uniform in [-2^15, 2^15) against tLookupRange(-2^15, 2^16): multiplicities, the batched
    inverse 1/(S + beta) and the logUp sumcheck."""

    def __init__(self, zkh, rng, D, N, low, tag="cfg3"):
        self.zkh, self.D, self.N, self.low = zkh, D, N, low
        self.vals = rng.integers(low, low + N, size=D).astype(np.int32)
        self.ctx = c = zkh.Context(0)
        self.S = c.from_i32(self.vals)
        self.T = c.range_table(low, N, N)
        st = zkh.transcript(tag + ".rescale")
        zkh.absorb(st, "com_rem", blob("c3rem", 1024 * 144))
        self.st0 = st
        self.logD = D.bit_length() - 1

    def run(self):
        zkh, c = self.zkh, self.ctx
        st = self.st0.copy()
        m = c.lu_prep(self.S, self.low, self.N)
        beta = zkh.challenge(st)
        A = c.lu_range_inverse(self.S, self.low, self.T, beta)
        alpha = zkh.challenge(st)
        u = zkh.challenges(st, self.logD)
        lu = c.lu_prove(st, A, self.S, self.T, m, alpha, beta, u)
        return lu["ev"].tobytes() + lu["term"].tobytes() + st.tobytes()

    def cpu_run(self, sample=None):
        """The oracle on the same transcript; sample = D' < D runs the first D' witnesses
        against the same table instead (a bounded single-thread sample, not compared)."""
        C = _oracle()
        vals = self.vals if sample is None else self.vals[:sample]
        D = len(vals)
        st = self.st0.copy()
        Sf = C.ints_to_fr(vals)
        rc, m = C.lu_prep(Sf, self.low, self.N)
        beta = C.tr_challenge_fr(st)
        A = C.lu_inverse(Sf, beta)
        alpha = C.tr_challenge_fr(st)
        u = np.array([C.tr_challenge_fr(st) for _ in range(D.bit_length() - 1)])
        rc, lu = C.lu_prove(st, A, Sf, C.range_table(self.low, self.N, self.N), m, alpha, beta, u)
        assert rc == 0
        return lu["ev"].tobytes() + lu["term"].tobytes() + st.tobytes()


def witness_gemm(zkh, jobs, reps=5):
    """The layer's witness GEMMs Y = X W (zkh_matmul_i32, zkob_fc.cu:212), outside the prove
    time as in the reference's accounting: kernel time from the launch-stamped events, the
    fp64 matrix-core path (the operands' bounds keep every partial sum below 2^53)."""
    import ctypes
    flops = sum(2.0 * j.B * j.IN * j.OUT for j in jobs)
    for j in jobs:
        j.ctx.matmul_i32(j.X, j.W, j.B, j.IN, j.OUT)  # warm
        zkh.lib().zkh_prof_enable(j.ctx.h, 1)
    t = time.perf_counter()
    for _ in range(reps):
        for j in jobs:
            j.ctx.matmul_i32(j.X, j.W, j.B, j.IN, j.OUT)
    wall = (time.perf_counter() - t) / reps
    kern, paths = 0.0, set()
    for j in jobs:
        for name in ("matmul_f64", "matmul_i64"):
            ms, la, by = ctypes.c_double(), ctypes.c_uint64(), ctypes.c_double()
            zkh.lib().zkh_prof_get(j.ctx.h, name.encode(), ctypes.byref(ms), ctypes.byref(la), ctypes.byref(by))
            if la.value:
                kern += ms.value / reps
                paths.add(name)
        zkh.lib().zkh_prof_enable(j.ctx.h, 0)
    tf = flops / (kern / 1000.0) / 1e12
    return {"kernel_ms_per_layer": round(kern, 4), "wall_ms_per_layer": round(wall * 1000.0, 4),
            "TFLOPs": round(tf, 2), "frac_fp64_matrix_peak": round(tf / 78.6, 4), "paths": sorted(paths),
            "scope": "Y = X W for the 7 matmuls (exact int64), not part of prove_s_per_layer"}


def commit_setup(zkh, jobs, seed=0x5EED0004):
    """Commitment keys and padded tensors for the layer's matmuls (zkob_fc.cu:215-230): one
    pool of random generators made as Commitment::random makes them (the generator times
    random field elements, commitment.cu:3-8, here zkh_g1_mul), of which gen_in takes the
    first IN_pad points and gen_out the first OUT_pad; X, W, Y padded per dimension to
    powers of two."""
    rng = np.random.default_rng(seed)
    G = zkh.g1_generator()[None, :]
    c0 = jobs[0].ctx
    npool = max(max(pow2(j.IN), pow2(j.OUT)) for j in jobs)
    a = rng.integers(0, 2**32, size=(npool + 1, 8), dtype=np.uint64).astype(np.uint32)
    a[:, 7] %= 0x73EDA753  # below r's top limb: canonical
    pool = c0.g1_mul(c0.g1_from_host(G), c0.from_fr(a)).to_host()
    for j in jobs:
        c = j.ctx
        j.Q = pool[npool]  # the IPA's Q (the first point of the reference's q.bin)
        j.gen_in = c.g1_from_host(pool[:pow2(j.IN)])
        j.gen_out = c.g1_from_host(pool[:pow2(j.OUT)])
        j.Xp = c.pad(j.X, (j.B, j.IN))
        j.Wp = c.pad(j.W, (j.IN, j.OUT))
        j.Yp = c.pad(j.Y, (j.B, j.OUT))
        j.commit_scalars = j.Xp.n + j.Wp.n + j.Yp.n
    return pool


def commit_job(j):
    """com_X, com_W, com_Y of one matmul (zkob_fc.cu:219-230), as digests of the points."""
    c = j.ctx
    outs = [c.commit(j.gen_in, j.Xp), c.commit(j.gen_out, j.Wp), c.commit(j.gen_out, j.Yp)]
    return b"".join(hashlib.sha256(o.to_host().tobytes()).digest() for o in outs)


PIP_KERNELS = ("pip_sort", "pip_alias", "pip_bucket", "pip_window", "pip_combine")


def commitments(zkh, jobs, pool, reps=3, cpu=True):
    """Pedersen commitments of the layer's 7 matmuls: com_X, com_W, com_Y each (the reference
    recomputes com_W on every proof, zkob_fc.cu:220), byte-identical to commit_pippenger.
    Timed with the 7 matmuls' commitments issued concurrently (one context and stream per
    matmul), and sequentially; kernel times from the launch-stamped events."""
    import ctypes
    commit_setup(zkh, jobs)
    ref = [commit_job(j) for j in jobs]
    for j in jobs:
        zkh.lib().zkh_prof_enable(j.ctx.h, 1)
    t = time.perf_counter()
    for j in jobs:
        assert commit_job(j) == ref[jobs.index(j)]
    seq = time.perf_counter() - t
    kern = {}
    for j in jobs:
        for name in PIP_KERNELS:
            ms, la, by = ctypes.c_double(), ctypes.c_uint64(), ctypes.c_double()
            zkh.lib().zkh_prof_get(j.ctx.h, name.encode(), ctypes.byref(ms), ctypes.byref(la), ctypes.byref(by))
            kern[name] = kern.get(name, 0.0) + ms.value
        zkh.lib().zkh_prof_enable(j.ctx.h, 0)
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        futs = [pool.submit(commit_job, j) for j in jobs]
        assert [f.result() for f in futs] == ref, "non-deterministic commitments"
        times.append(time.perf_counter() - t)
    scalars = sum(j.commit_scalars for j in jobs)
    best = min(times)
    res = {"commit_s_per_layer": round(best, 4), "commit_s_per_layer_sequential": round(seq, 4),
           "scalars_committed": scalars, "scalars_per_s": round(scalars / best),
           "kernel_ms_sequential": {k: round(v, 3) for k, v in kern.items()},
           "scope": "com_X, com_W, com_Y of Q,K,V,O,gate,up,down (padded tensors, zkob_fc.cu:215-230), "
                    "7 matmuls concurrent on 7 streams; byte-identical to commit_pippenger"}
    if cpu:
        res["cpu_baseline"] = commit_cpu_baseline(jobs[0])
    return res


def open_job(j, out):
    """The IPA openings that end zkob_fc's prove (zkob_fc.cu:473-483), order W, X, Y, each
    continuing the matmul's transcript after its sumcheck: a = the padded tensor folded over
    its rows by the proof's challenges (partial_me), b = me_weights of the other point."""
    c = j.ctx
    st = j.st.copy()
    ub, uo, ui = out["u_batch"], out["u_output"], out["u_input"]
    bW = c.eq_table(uo)
    r = [c.ipa_prove(st, c.partial_me_window(j.Wp, ui, pow2(j.OUT)), bW, j.gen_out, j.Q),
         c.ipa_prove(st, c.partial_me_window(j.Xp, ub, pow2(j.IN)), c.eq_table(ui), j.gen_in, j.Q),
         c.ipa_prove(st, c.partial_me_window(j.Yp, ub, pow2(j.OUT)), bW, j.gen_out, j.Q)]
    return b"".join(x["L"].tobytes() + x["R"].tobytes() + x["a_final"].tobytes() for x in r) + st.tobytes()


def open_batched(jobs, outs):
    """The same 21 openings through zkh_ipa_prove_batch: the openings' inputs formed on each
    matmul's context, then three batched calls on one context (all W openings, all X, all Y:
    each matmul's transcript runs W, X, Y in order as in open_job)."""
    ins = []
    for j, o in zip(jobs, outs):
        c = j.ctx
        ub, ui = o["u_batch"], o["u_input"]
        bW = c.eq_table(o["u_output"])
        ins.append((j.st.copy(), [(c.partial_me_window(j.Wp, ui, pow2(j.OUT)), bW, j.gen_out),
                                  (c.partial_me_window(j.Xp, ub, pow2(j.IN)), c.eq_table(ui), j.gen_in),
                                  (c.partial_me_window(j.Yp, ub, pow2(j.OUT)), bW, j.gen_out)]))
        c.sync()
    res = [[] for _ in jobs]
    for k in range(3):
        got = jobs[0].ctx.ipa_prove_batch([(st, t[k][0], t[k][1], t[k][2], j.Q) for j, (st, t) in zip(jobs, ins)])
        for r, g in zip(res, got):
            r.append(g)
    return [b"".join(x["L"].tobytes() + x["R"].tobytes() + x["a_final"].tobytes() for x in r) + st.tobytes()
            for r, (st, _) in zip(res, ins)]


def openings(zkh, jobs, outs, pool, reps=2, cpu=True):
    """The layer's 21 IPA openings (3 per matmul) through zkh_ipa_prove_batch; every pass must
    reproduce, byte for byte, the proofs of one zkh_ipa_prove call per opening.  Also timed:
    the 7 matmuls' openings concurrent on their own contexts, one call per opening."""
    ref = [open_job(j, o) for j, o in zip(jobs, outs)]
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        assert open_batched(jobs, outs) == ref, "batched openings differ from the single-call ones"
        times.append(time.perf_counter() - t)
    t = time.perf_counter()
    futs = [pool.submit(open_job, j, o) for j, o in zip(jobs, outs)]
    assert [f.result() for f in futs] == ref, "non-deterministic openings"
    t_ctx = time.perf_counter() - t
    res = {"ipa_s_per_layer": round(min(times), 4), "ipas": 3 * len(jobs),
           "ipa_s_per_layer_contexts": round(t_ctx, 4),
           "scope": "ipa_W, ipa_X, ipa_Y of the 7 matmuls (vrf_common.cuh:302-336) in three zkh_ipa_prove_batch "
                    "calls, byte-identical to one zkh_ipa_prove per opening; _contexts: one call per opening, the 7 "
                    "matmuls concurrent on their own contexts"}
    if cpu:
        sys.path.insert(0, ROOT)
        from oracle import coracle
        j, o = jobs[0], outs[0]
        st = coracle.tr_init("cpu-ipa")
        a = j.ctx.partial_me_window(j.Xp, o["u_batch"], pow2(j.IN)).to_fr()
        b = j.ctx.eq_table(o["u_input"]).to_fr()
        t0 = time.perf_counter()
        rc, _, _, _ = coracle.ipa_prove(st, a, b, j.gen_in.to_host(), j.Q, pow2(j.IN))
        secs = time.perf_counter() - t0
        assert rc == 0
        res["cpu_baseline"] = {"value": round(secs, 3), "unit": "s per IPA (n = %d)" % pow2(j.IN), "cores": 1,
                               "kind": "port", "sample": "C oracle ipa_prove of the Q projection's X opening"}
    return res


def batch_open(zkh, jobs, reps=2):
    """The layer's 21 matmul claims opened in one batch, as the reference's claim-mode walk
    does: zkh_fc commit registers each W (zkob_fc.cu commit), zkh_fc prove --claims runs each
    matmul's commitments and sumcheck and appends its claims on W, X and Y with the padded
    witnesses (zkob_fc.cu:449-470), then zkh_batchopen prove (batch_prove,
    zkob_claims.cuh:832-1066) opens all of them: witness loads and the rho-weighted eq tables
    (setup), the batch-evaluation rounds, the terminals, and one IPA per generator domain.
    Timed by the driver's own ZKOB_PROF laps (BoTimer), so process start and HIP
    initialisation are outside; the witness files are read from the page cache."""
    import shutil
    import subprocess
    import tempfile
    here = os.path.dirname(os.path.abspath(__file__))
    fc, bo = (os.path.join(here, "zk-hillclimb_amd", n) for n in ("zkh_fc", "zkh_batchopen"))
    pool = commit_setup(zkh, jobs)
    tmp = tempfile.mkdtemp(prefix="zkh_batchopen_")
    try:
        sizes = sorted({pow2(j.IN) for j in jobs} | {pow2(j.OUT) for j in jobs})
        for G in sizes:
            pool[:G].tofile(os.path.join(tmp, "gen_%d.bin" % G))
        q = os.path.join(tmp, "q.bin")
        pool[len(pool) - 1:].tofile(q)
        acc = os.path.join(tmp, "acc")
        os.makedirs(acc)
        t_claims, wit_bytes = 0.0, 0
        for j in jobs:
            X, W, _ = j.inputs
            d = os.path.join(tmp, j.name)
            os.makedirs(d)
            X.astype(np.int32).tofile(os.path.join(d, "X.i32"))
            W.astype(np.int32).tofile(os.path.join(d, "W.i32"))
            gi, go = (os.path.join(tmp, "gen_%d.bin" % pow2(n)) for n in (j.IN, j.OUT))
            dims = [str(j.B), str(j.IN), str(j.OUT)]
            subprocess.run([fc, "commit", os.path.join(d, "W.i32"), str(j.IN), str(j.OUT), go,
                            os.path.join(d, "com_W.bin")], check=True, capture_output=True, timeout=300)
            t = time.perf_counter()
            subprocess.run([fc, "prove", d, "cfg4:layer0." + j.name, os.path.join(d, "X.i32"),
                            os.path.join(d, "W.i32")] + dims + [gi, go, q, "--claims", acc, "layer0." + j.name,
                                                               os.path.join(d, "com_W.bin")],
                           check=True, capture_output=True, timeout=300)
            t_claims += time.perf_counter() - t
            wit_bytes += 32 * (j.Xp.n + j.Wp.n + j.Yp.n)
            print("batchopen: claims of %s emitted" % j.name, file=sys.stderr, flush=True)
        runs = []
        for _ in range(reps):
            r = subprocess.run([bo, "prove", acc, "cfg4", q] + ["%d=%s" % (G, os.path.join(tmp, "gen_%d.bin" % G))
                                                               for G in sizes],
                               env=dict(os.environ, ZKOB_PROF="1"), capture_output=True, text=True, timeout=600)
            if r.returncode:
                raise RuntimeError("zkh_batchopen failed: " + r.stderr)
            laps = {ln.split()[1].split(".", 1)[1]: float(ln.split()[2])
                    for ln in r.stdout.splitlines() if ln.startswith("PROF ")}
            runs.append(laps)
            print("batchopen: %s" % r.stdout.strip().splitlines()[-1], file=sys.stderr, flush=True)
        best = min(runs, key=lambda x: sum(x.values()))
        return {"batch_open_s_per_layer": round(sum(best.values()), 4),
                "laps_s": best,
                "claims": 3 * len(jobs),
                "domains": sizes,
                "witness_bytes": wit_bytes,
                "claim_mode_prove_wall_s": round(t_claims, 3),
                "scope": "one batch opening of the 7 matmuls' 21 claims (W, X, Y each) of a TinyLlama layer, "
                         "replacing their 21 inline IPAs; the drivers' claim-mode runs are timed separately "
                         "(wall, process start included)"}
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def commit_cpu_baseline(j, rows=1):
    """The C oracle's commit_pippenger (scalar, one thread) on one row each of the Q
    projection's X, W and Y (the same generators and padded values as the GPU run)."""
    sys.path.insert(0, ROOT)
    from oracle import coracle
    total, secs = 0, 0.0
    for t, g in ((j.Xp, j.gen_in), (j.Wp, j.gen_out), (j.Yp, j.gen_out)):
        gens = g.to_host()
        n = g.n
        sc = t.to_fr()[: rows * n]
        t0 = time.perf_counter()
        rc, _ = coracle.g1_commit(gens, sc, n)
        secs += time.perf_counter() - t0
        assert rc == 0
        total += rows * n
    return {"value": round(total / secs, 1), "unit": "scalars committed/s", "cores": 1, "kind": "port",
            "sample": "C oracle commit_pippenger on %d row(s) each of the Q projection's padded X, W, Y "
                      "(%d scalars, %.1f s, 1 thread)" % (rows, total, secs)}


def host_info():
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)), "cpu_model": model}


def timed(fn):
    t = time.perf_counter()
    out = fn()
    return out, time.perf_counter() - t


def cpu_baseline(jobs, outs, names=("q", "k", "v", "o")):
    """The C oracle (the reference's algorithmic schedule: partial_me + multi_dim_me passes,
    per-round zkip kernels) on the Q, K, V, O matmuls of the same layer, on the GPU proofs'
    own transcripts: each CPU proof must equal the GPU's byte for byte.  Timed on one thread
    and on all the host cores the process may use."""
    C = _oracle()
    host = host_info()
    sel = [(j, o) for j, o in zip(jobs, outs) if j.name in names]
    E = sum(j.elements for j, _ in sel)
    res = {}
    for label, thr in (("single_thread", 1), ("all_cores", host["affinity"])):
        C.set_threads(thr)
        t = 0.0
        for j, (out, st) in sel:
            got, secs = timed(j.cpu_run)
            assert got == MatmulJob.result(out, st), "CPU proof differs from the GPU's (%s)" % j.name
            t += secs
        res[label] = {"value": E / t, "cores": thr, "s": round(t, 3)}
    best = res["all_cores"]
    return {"value": best["value"], "unit": "Fr elements/s", "cores": best["cores"], "kind": "port",
            "sample": "C oracle (reference schedule: partial_me + multi_dim_me passes, per-round zkip "
                      "kernels) on the Q,K,V,O matmul sumchecks of the same layer (%d elements) on the GPU "
                      "proofs' transcripts, every proof byte-identical to the GPU's; %d threads %.2f s, "
                      "1 thread %.2f s" % (E, best["cores"], best["s"], res["single_thread"]["s"]),
            "single_thread": {"value": res["single_thread"]["value"], "cores": 1, "s": res["single_thread"]["s"]},
            **host}


def layer_cpu_baseline(jobs, mm_outs, others, others_ref, glu, rope_k, synth):
    """The whole layer hot path on the C oracle, all cores, on the GPU's transcripts (every
    segment byte-identical to the GPU's): the 7 matmuls, the SwiGLU lookup + Hadamard and
    the RoPE Hadamards.  One thread is estimated from bounded samples: the Q,K,V,O matmuls
    (scaled by elements to the 7), the SwiGLU segment at 2^16 entries (scaled by 2^22 / 2^16)
    and the RoPE k obligation (2^17, scaled by entries to q + k)."""
    C = _oracle()
    host = host_info()
    C.set_threads(host["affinity"])
    t_mm = 0.0
    for j, (out, st) in zip(jobs, mm_outs):
        got, secs = timed(j.cpu_run)
        assert got == MatmulJob.result(out, st), "CPU proof differs from the GPU's (%s)" % j.name
        t_mm += secs
    seg = {}
    for j, ref in zip(others, others_ref):
        got, secs = timed(j.cpu_run)
        assert got == ref, "CPU segment differs from the GPU's (%s)" % type(j).__name__
        seg[type(j).__name__ + ":2^%d" % j.logD] = round(secs, 3)
    all_cores = t_mm + sum(seg.values())
    # one thread, bounded samples
    C.set_threads(1)
    E_all = sum(j.elements for j in jobs)
    qkvo = [j for j in jobs if j.name in ("q", "k", "v", "o")]
    t1_qkvo = sum(timed(j.cpu_run)[1] for j in qkvo)
    small = GluJob(glu.zkh, synth, synth.rng_for(99), 64, 1024)  # D = N = 2^16
    t1_glu = timed(small.cpu_run)[1] * (glu.D / small.D)
    t1_rope = timed(rope_k.cpu_run)[1] * (sum(o.D for o in others if isinstance(o, RopeJob)) / rope_k.D)
    C.set_threads(host["affinity"])
    one = t1_qkvo * E_all / sum(j.elements for j in qkvo) + t1_glu + t1_rope
    return {"value": all_cores, "unit": "s per layer", "cores": host["affinity"], "kind": "port",
            "sample": "the whole TinyLlama layer hot path on the C oracle (reference schedule, per-element "
                      "Fermat inverses), all cores, every output byte-identical to the GPU's: 7 matmuls %.2f s, "
                      "segments %s" % (t_mm, seg),
            "single_thread_estimate_s": round(one, 2),
            "single_thread_basis": "Q,K,V,O matmuls on 1 thread scaled by elements to the 7 (%.2f s); SwiGLU "
                                   "segment at D = N = 2^16 on 1 thread scaled to 2^22 (%.2f s); RoPE k on 1 "
                                   "thread scaled to q + k (%.2f s)" % (t1_qkvo, t1_glu, t1_rope),
            **host}


def prof_kernels(zkh, ctx, reps=1):
    """Per-kernel-class device time (ms per run), launches and algorithmic bytes of the
    launch-stamped records on one context."""
    import ctypes
    kern = {}
    buf = ctypes.create_string_buffer(4096)
    zkh.lib().zkh_prof_names(ctx.h, buf, 4096)
    for name in filter(None, buf.value.decode().split(",")):
        ms, la, by = ctypes.c_double(), ctypes.c_uint64(), ctypes.c_double()
        zkh.lib().zkh_prof_get(ctx.h, name.encode(), ctypes.byref(ms), ctypes.byref(la), ctypes.byref(by))
        kern[name] = [ms.value / reps, la.value / reps, by.value / reps]
    return kern


def mm_batch_rate(zkh, jobs, steps, warmup):
    """Elements bound per second of one batched call over the jobs (inputs resident)."""
    ctx = jobs[0].ctx
    for j in jobs:
        j.st = j.st0.copy()
    mb = zkh.MmBatch(ctx, [(j.st, j.X, j.W, j.Y, j.B, j.IN, j.OUT) for j in jobs])

    def step():
        for j in jobs:
            np.copyto(j.st, j.st0)
        mb.run()
    for _ in range(warmup):
        step()
    ref = [MatmulJob.result(o, j.st) for o, j in zip(mb.outs, jobs)]
    gc.collect()
    gc.disable()
    t = time.perf_counter()
    for _ in range(steps):
        step()
    ms = (time.perf_counter() - t) * 1000.0 / steps
    gc.enable()
    assert [MatmulJob.result(o, j.st) for o, j in zip(mb.outs, jobs)] == ref
    E = sum(j.elements for j in jobs)
    return {"value": E / (ms / 1000.0), "unit": "Fr elements/s", "ms_per_step": round(ms, 4),
            "elements_bound_per_step": E}, mb, ref


def seg_time(job, reps):
    ref = job.run()
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        assert job.run() == ref
        times.append((time.perf_counter() - t) * 1000.0)
    return min(times), ref


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--layer-steps", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-layer", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip the C2, C3, C5 and field-input keys")
    ap.add_argument("--no-commit", action="store_true", help="skip the Pedersen commitments")
    ap.add_argument("--no-batchopen", action="store_true", help="skip the claim-mode batch opening")
    ap.add_argument("--no-prof", action="store_true", help="skip the profiled pass (no kernel times)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run one 256 MiB device-to-device copy (the known-size kernel that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--segment", choices=["glu", "rope", "ropek", "commit", "batchopen", "c3", "c5glu", "mmfr", "frmul"],
                    default=None, help="only run one segment repeatedly (for profiling), then exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "; run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch

    zkh, synth = load_pkg()
    if args.calibrate_copy:
        src = torch.ones(64 << 20, dtype=torch.int32, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    rng = synth.rng_for(4)
    L = LAYER
    C4 = synth.CONFIGS["C4"]
    MATMULS = C4["matmuls"]
    if args.segment == "frmul":  # the Montgomery-multiply rate probe alone (for profiling)
        ctx = zkh.Context(0)
        rates = [ctx.calib_fr_mul(256) for _ in range(max(args.steps, 1))]
        print(json.dumps({"segment": "frmul", "mul_per_s": rates}))
        return
    if args.segment == "commit":
        jobs = [MatmulJob(zkh, synth, rng, n, L["B"], i, o) for n, i, o in MATMULS]
        pool = concurrent.futures.ThreadPoolExecutor(max_workers=16)
        print(json.dumps({"segment": "commit", **commitments(zkh, jobs, pool, reps=args.steps, cpu=False)}))
        pool.shutdown()
        return
    if args.segment == "batchopen":
        jobs = [MatmulJob(zkh, synth, rng, n, L["B"], i, o) for n, i, o in MATMULS]
        print(json.dumps({"segment": "batchopen", **batch_open(zkh, jobs, reps=max(1, min(args.steps, 3)))}))
        return
    if args.segment == "mmfr":
        jobs = [MatmulJob(zkh, synth, rng, n, L["B"], i, o, fr=True) for n, i, o in MATMULS]
        r, _, _ = mm_batch_rate(zkh, jobs, args.steps, args.warmup)
        print(json.dumps({"segment": "mmfr", **r}))
        return
    if args.segment:
        if args.segment == "glu":
            job = GluJob(zkh, synth, rng, L["B"], L["ffn"])
        elif args.segment == "c5glu":
            C5 = synth.CONFIGS["C5"]
            job = GluJob(zkh, synth, synth.rng_for(5), C5["B"], C5["ffn"], N=C5["glu_table"], tag="cfg5:layer0")
        elif args.segment == "c3":
            c3 = synth.CONFIGS["C3"]
            job = LookupJob(zkh, synth.rng_for(3), c3["D"], c3["N"], c3["low"])
        elif args.segment == "ropek":
            job = RopeJob(zkh, synth, rng, "k", L["B"], L["kv"])
        else:
            job = RopeJob(zkh, synth, rng, "q", L["B"], L["d"])
        ref = job.run()
        gc.collect()
        gc.disable()
        times = []
        for _ in range(args.steps):
            t = time.perf_counter()
            assert job.run() == ref
            times.append((time.perf_counter() - t) * 1000.0)
        print(json.dumps({"segment": args.segment, "ms": times}))
        return
    t_setup = time.perf_counter()
    jobs = [MatmulJob(zkh, synth, rng, n, L["B"], i, o) for n, i, o in MATMULS]
    E_total = sum(j.elements for j in jobs)
    pool = concurrent.futures.ThreadPoolExecutor(max_workers=16)

    mctx = zkh.Context(0)
    # the Montgomery-multiply rate of this build (the VALU roofline of the field kernels)
    fr_peak = max(mctx.calib_fr_mul(256) for _ in range(3))

    # one prepared zkh_mm_prove_batch call (job array and output buffers built once); a
    # step resets each transcript to its pre-proof state and proves all seven matmuls
    for j in jobs:
        j.st = j.st0.copy()
    mbatch = zkh.MmBatch(mctx, [(j.st, j.X, j.W, j.Y, j.B, j.IN, j.OUT) for j in jobs])

    def mm_step():
        for j in jobs:
            np.copyto(j.st, j.st0)
        mbatch.run()

    def mm_result():
        return [o["claims"].tobytes() + j.st.tobytes() for o, j in zip(mbatch.outs, jobs)]

    mm_step()  # the reference proofs (every timed step must reproduce them)
    ref = mm_result()
    mm_outs = [({k: v.copy() for k, v in o.items()}, j.st.copy()) for o, j in zip(mbatch.outs, jobs)]
    print("setup %.1fs; matmul step warm" % (time.perf_counter() - t_setup), file=sys.stderr, flush=True)
    # the interpreter's cyclic GC (millions of objects once torch is imported) would stall
    # a step for tens of ms at fixed allocation counts; it stays off while timing.  The W
    # warmup steps run right before the timed ones, after the collection: a step that follows
    # an idle pause (the collection, the device and the host workers going idle) takes
    # several times as long as the next ones, and the first ~200 steps after the jobs' setup
    # (the large uploads and allocations) run at ~0.205 ms against ~0.18 after them; W
    # defaults to 300 steps (~60 ms).
    def timed_steps(prof=False):
        gc.collect()
        gc.disable()
        for _ in range(args.warmup):
            mm_step()
        if prof:  # launch records of the K timed steps only (enabling clears the records)
            zkh.lib().zkh_prof_enable(mctx.h, 1)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        step_ms = []
        for _ in range(args.steps):
            ts = time.perf_counter()
            mm_step()
            step_ms.append((time.perf_counter() - ts) * 1000.0)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        out = mm_result()
        gc.enable()
        assert out == ref, "non-deterministic proof output"
        return (t1 - t0) * 1000.0 / args.steps, step_ms

    # Timed steps without kernel-timing events: a launch that stamps HIP events costs the host
    # ~20 us per step here, so the throughput steps carry none.  A second, live pass of the
    # same steps stamps the kernels' own launches (hipExtLaunchKernel start/stop events on
    # the library's stream) for the per-kernel times and the roofline; its own step time is
    # reported beside it.
    ms_step, step_ms = timed_steps()
    print("per-step ms: " + " ".join("%.2f" % x for x in step_ms), file=sys.stderr, flush=True)
    value = E_total / (ms_step / 1000.0)
    print("matmul step %.3f ms -> %.3g elements/s" % (ms_step, value), file=sys.stderr, flush=True)
    prof_ms_step = None
    if not args.no_prof:
        prof_ms_step, _ = timed_steps(prof=True)

    # per-kernel device time, launches and bytes over the profiled pass's K timed steps
    kern = prof_kernels(zkh, mctx)
    zkh.lib().zkh_prof_enable(mctx.h, 0)
    # The roofline object covers the dominant HBM-bound kernel.  The persistent round loop
    # (zkip_rounds) runs one host round trip per round (Fiat-Shamir challenge) and moves
    # ~1 MB per step: it is bounded by that latency, not by HBM or the integer VALU, and is
    # listed under "kernels" with its own time.
    hbm = {n: v for n, v in kern.items() if n not in LATENCY_BOUND}
    dom = max(hbm, key=lambda n: hbm[n][0]) if hbm else None
    dms, dla, dby = hbm[dom] if hbm else (1.0, 1, 0.0)
    achieved = dby / (dms / 1000.0) / 1e9
    roofline = {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": TRAFFIC.get(dom),
                "bytes_per_launch": dby / max(dla, 1), "avg_launch_us": dms * 1000.0 / max(dla, 1),
                "launches_per_step": dla / args.steps,
                "bytes_basis": "stored integer widths of X, W (int32) and Y (int64), each read once",
                "timing": "events stamped by the kernel's own launch, over a second live pass of the "
                          "same %d steps (ms_per_step %s)" % (args.steps, None if prof_ms_step is None
                                                               else round(prof_ms_step, 4))}
    kernels = {n: {"ms_per_step": round(v[0] / args.steps, 4), "launches_per_step": v[1] / args.steps,
                   "GBps": round(v[2] / (v[0] / 1000.0) / 1e9, 1) if v[0] else None,
                   "bound": "latency" if n in LATENCY_BOUND else "hbm"}
               for n, v in sorted(kern.items(), key=lambda kv: -kv[1][0])}

    layer = None
    glu = ropes = others = lref_others = None
    if not args.no_layer:
        glu = GluJob(zkh, synth, rng, L["B"], L["ffn"])
        ropes = [RopeJob(zkh, synth, rng, "q", L["B"], L["d"]), RopeJob(zkh, synth, rng, "k", L["B"], L["kv"])]
        others = [glu] + ropes

        def layer_step():
            futs = [pool.submit(j.run) for j in others]
            mm_step()
            return [mm_result()] + [f.result() for f in futs]

        lref = layer_step()
        lref_others = lref[1:]
        seg = {}
        for j in others:  # isolated segment times (sequential, for the breakdown)
            t = time.perf_counter()
            j.run()
            seg[type(j).__name__ + ":2^%d" % j.logD] = round((time.perf_counter() - t) * 1000.0, 2)
        gc.collect()
        gc.disable()
        torch.cuda.synchronize()
        ta = time.perf_counter()
        for _ in range(args.layer_steps):
            lout = layer_step()
        torch.cuda.synchronize()
        tb = time.perf_counter()
        gc.enable()
        assert lout == lref, "non-deterministic layer output"
        # kernel classes of the SwiGLU segment (the layer's largest) in one profiled run
        zkh.lib().zkh_prof_enable(glu.ctx.h, 1)
        assert glu.run() == lref_others[0]
        gk = prof_kernels(zkh, glu.ctx)
        zkh.lib().zkh_prof_enable(glu.ctx.h, 0)
        gdom = max(gk, key=lambda n: gk[n][0])
        gms, gla, gby = gk[gdom]
        layer = {"prove_s_per_layer": (tb - ta) / args.layer_steps,
                 "segments_isolated_ms": seg,
                 "swiglu_kernels": {n: {"ms": round(v[0], 4), "launches": int(v[1]),
                                        "GBps": round(v[2] / (v[0] / 1000.0) / 1e9, 1) if v[0] else None}
                                    for n, v in sorted(gk.items(), key=lambda kv: -kv[1][0])},
                 "scope": "7 matmul sumchecks + SwiGLU logUp (D=N=2^22) + its Hadamard (2^22) + "
                          "RoPE q/k Hadamards (2x2^20, 2x2^17), concurrent; commitments, IPA "
                          "openings and the witness GEMM excluded"}
        layer_roofline = {"bound": "hbm", "kernel": gdom, "achieved": round(gby / (gms / 1000.0) / 1e9, 1),
                          "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(gby / (gms / 1000.0) / 1e9 / HBM_PEAK_GBS, 4),
                          "traffic": TRAFFIC.get(gdom),
                          "bytes_per_launch": gby / max(gla, 1), "avg_launch_us": gms * 1000.0 / max(gla, 1),
                          "launches_per_segment": gla,
                          "scope": "dominant kernel class of the SwiGLU segment (the layer's largest), "
                                   "algorithmic bytes over launch-stamped time"}
        if gdom == "lu_phase2":
            # the same launches against the Montgomery-multiply peak: per pair 6 Montgomery
            # products in the first round (A = 1/(comb + beta) and B = 1/(T_comb + beta) take
            # the closed form: 3 per group, eq weights included; the three multiplicity
            # products there are 32-bit multiplies, not counted) and 22 after it (the sums at 1
            # derived on the host: 5 + 7, and the owed folds of A, S, B, T, m, 2 per table)
            pairs = [(glu.D >> r) // 2 for r in range(int(gla))]
            prods = sum(p * (6 if r == 0 else 22) for r, p in enumerate(pairs))
            rate = prods / (gms / 1000.0)
            layer_roofline["valu"] = {
                "products_per_segment": prods, "achieved_Gmul_s": round(rate / 1e9, 1),
                "peak_Gmul_s": round(fr_peak / 1e9, 1), "frac": round(rate / fr_peak, 4),
                "basis": "Montgomery products of the %d lu_phase2 launches (n = 2^%d .. 2^%d) over their "
                         "launch-stamped time, against zkh_calib_fr_mul's device-wide rate"
                         % (gla, glu.logD, glu.logD - int(gla) + 1)}
        print("layer %.3f s" % layer["prove_s_per_layer"], file=sys.stderr, flush=True)

    configs = None
    fr_key = None
    if not args.no_configs:
        configs = {}
        # field-element inputs: the same 7 matmuls with X, W, Y bound as FrTensors
        fr_jobs = [MatmulJob(zkh, synth, None, j.name, j.B, j.IN, j.OUT, fr=True, inputs=j.inputs) for j in jobs]
        r, fb, fref = mm_batch_rate(zkh, fr_jobs, args.steps, args.warmup)
        assert [MatmulJob.result(o, st) for o, st in mm_outs] == fref, "FR-input proofs differ from the int ones"
        zkh.lib().zkh_prof_enable(fr_jobs[0].ctx.h, 1)
        fb.run()
        fk = prof_kernels(zkh, fr_jobs[0].ctx)
        zkh.lib().zkh_prof_enable(fr_jobs[0].ctx.h, 0)
        fms, fla, fby = fk.get("eqdot_fr", (1.0, 1, 0.0))
        fr_key = dict(r, roofline={"bound": "hbm", "kernel": "eqdot_fr",
                                   "achieved": round(fby / (fms / 1000.0) / 1e9, 1), "peak": HBM_PEAK_GBS,
                                   "unit": "GB/s", "frac": round(fby / (fms / 1000.0) / 1e9 / HBM_PEAK_GBS, 4),
                                   "bytes_per_launch": fby, "avg_launch_us": fms * 1000.0},
                      kernels_ms={n: round(v[0], 4) for n, v in fk.items()},
                      scope="the TinyLlama layer's 7 matmuls with X, W, Y as field-element tensors (32 B "
                            "per entry); proofs byte-identical to the integer-input ones")
        del fr_jobs, fb
        print("FR-input matmul step %.3f ms" % fr_key["ms_per_step"], file=sys.stderr, flush=True)
        # C2: llama-68m FFN matmuls at seq 128
        c2 = synth.CONFIGS["C2"]
        c2_jobs = [MatmulJob(zkh, synth, synth.rng_for(2), n, c2["B"], i, o, tag="cfg2") for n, i, o in c2["matmuls"]]
        r, _, _ = mm_batch_rate(zkh, c2_jobs, args.steps, args.warmup)
        configs["C2"] = dict(r, workload="llama-68m FFN matmul sumchecks, X 128x768, W_up 768x3072, W_down 3072x768")
        del c2_jobs
        # C3: the logUp range proof (zkob_rescale's shape; 2.19 s on an RTX 4090 for the whole
        # zkob_rescale prove incl. commitments, INT_BASELINE.md:176)
        c3 = synth.CONFIGS["C3"]
        lj = LookupJob(zkh, synth.rng_for(3), c3["D"], c3["N"], c3["low"])
        ms3, ref3 = seg_time(lj, 5)
        configs["C3"] = {"ms": round(ms3, 3), "witness_per_s": round(lj.D / (ms3 / 1000.0)),
                         "workload": "logUp: 2^20 witnesses in [-2^15, 2^15) vs the 2^16 range table "
                                     "(multiplicities, batched inverse, 20 rounds)"}
        # C5: OpenLLaMA-3B layer at seq 2048: 7 matmuls, SwiGLU 2^25 vs 2^22
        c5 = synth.CONFIGS["C5"]
        c5rng = synth.rng_for(5)
        c5_jobs = [MatmulJob(zkh, synth, c5rng, n, c5["B"], i, o, tag="cfg5:layer0") for n, i, o in c5["matmuls"]]
        r5, _, _ = mm_batch_rate(zkh, c5_jobs, max(5, args.steps // 2), 2)
        del c5_jobs
        g5 = GluJob(zkh, synth, synth.rng_for(5), c5["B"], c5["ffn"], N=c5["glu_table"], tag="cfg5:layer0")
        ms5, _ = seg_time(g5, 3)
        del g5
        configs["C5"] = {"matmuls": r5, "swiglu_ms": round(ms5, 3),
                         "workload": "OpenLLaMA-3B layer, seq 2048: 7 matmul sumchecks (d 3200, ffn 8640) and the "
                                     "SwiGLU lookup on the 2048x16384 grid (2^25 witnesses) vs a 2^22 table with its "
                                     "2^25 Hadamard"}
        print("configs: C2 %.3f ms, C3 %.2f ms, C5 matmuls %.3f ms, C5 SwiGLU %.1f ms" %
              (configs["C2"]["ms_per_step"], ms3, r5["ms_per_step"], ms5), file=sys.stderr, flush=True)
        if not args.no_cpu:
            C = _oracle()
            C.set_threads(len(os.sched_getaffinity(0)))
            got, secs = timed(lj.cpu_run)
            assert got == ref3, "C3 CPU proof differs from the GPU's"
            C.set_threads(1)
            sample = 1 << 16
            _, secs1 = timed(lambda: lj.cpu_run(sample))
            C.set_threads(len(os.sched_getaffinity(0)))
            configs["C3"]["cpu_baseline"] = {
                "value": round(secs, 3), "unit": "s", "cores": len(os.sched_getaffinity(0)), "kind": "port",
                "sample": "the C oracle on the same lookup and transcript (byte-identical proof), all cores",
                "single_thread_estimate_s": round(secs1 * lj.D / sample, 2),
                "single_thread_basis": "the first 2^16 witnesses against the same table on 1 thread, scaled by 2^4"}

    wg = None if args.no_layer else witness_gemm(zkh, jobs)
    com = None if args.no_commit else commitments(zkh, jobs, pool, cpu=not args.no_cpu)
    ope = None
    if com:
        print("commitments %.3f s per layer" % com["commit_s_per_layer"], file=sys.stderr, flush=True)
        ope = openings(zkh, jobs, mbatch.outs, pool, cpu=not args.no_cpu)
        print("openings %.3f s per layer" % ope["ipa_s_per_layer"], file=sys.stderr, flush=True)
    bo = None
    if com and not args.no_batchopen:
        bo = batch_open(zkh, jobs, reps=2)
        print("batch opening %.3f s per layer" % bo["batch_open_s_per_layer"], file=sys.stderr, flush=True)
    cpu = lcpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(jobs, mm_outs)
        print("cpu baseline (Q,K,V,O): %.3g elements/s on %d threads" % (cpu["value"], cpu["cores"]),
              file=sys.stderr, flush=True)
        if layer:
            lcpu = layer_cpu_baseline(jobs, mm_outs, others, lref_others, glu, ropes[1], synth)
            print("cpu baseline layer: %.2f s on %d threads" % (lcpu["value"], lcpu["cores"]),
                  file=sys.stderr, flush=True)
    res = {
        "metric": "Fr elements bound/sec in matmul sumcheck; prove s/layer at TinyLlama-1.1B",
        "value": value, "unit": "Fr elements/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_step, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "u32", "data": "synthetic",
        "config": {"workload": "TinyLlama-1.1B layer (BASELINE config 4), seq 512: Q,K,V,O,gate,up,down "
                               "matmul sumchecks", "B": L["B"], "d": L["d"], "kv": L["kv"],
                   "ffn": L["ffn"], "elements_bound_per_step": E_total, "field": "BLS12-381 Fr",
                   "inputs": "X, W int32 and Y int64 tensors (zkob_fc's int input files); the field-element "
                             "input rate is under fr_inputs"},
        "roofline": roofline, "kernels": kernels, "cpu_baseline": cpu,
        "fr_mul_peak": {"value": fr_peak, "unit": "Montgomery products/s",
                        "probe": "zkh_calib_fr_mul: 2048 blocks x 256 threads, 4 independent chains of 256 "
                                 "products per thread, device time of the launch (best of 3)"},
    }
    if layer:
        res["prove_s_per_layer"] = layer["prove_s_per_layer"]
        res["layer"] = layer
        res["layer_roofline"] = layer_roofline
        if lcpu:
            res["layer"]["cpu_baseline"] = lcpu
    if fr_key:
        res["fr_inputs"] = fr_key
    if configs:
        res["configs"] = configs
    if wg:
        res["witness_gemm"] = wg
    if com:
        res["commitments"] = com
    if ope:
        res["openings"] = ope
    if bo:
        res["batch_opening"] = bo
    print(json.dumps(res))
    pool.shutdown()


if __name__ == "__main__":
    main()
