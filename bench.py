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
  so the figure is the kernel's execution time as a kernel trace reports it; cpu_baseline:
  the C oracle (scalar port of the reference schedule) on the Q, K, V and O matmuls, one
  thread.
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
# HBM bytes per step measured with rocprofv3 --pmc FETCH_SIZE and --pmc WRITE_SIZE runs
# (profiles/eqdot_hbm_traffic_tinyllama.txt): the counters of a 256 MiB device copy read
# 0.500x (FETCH) and 1.000x (WRITE) of its bytes, so FETCH is scaled by 2.
TRAFFIC = {"eqdot": 315.4e6}


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
MATMULS = [("q", 2048, 2048), ("k", 2048, 256), ("v", 2048, 256), ("o", 2048, 2048),
           ("gate", 2048, 5632), ("up", 2048, 5632), ("down", 5632, 2048)]


def mm_elements(B, IN, OUT):
    return B * IN + IN * OUT + B * OUT + 2 * IN


class MatmulJob:
    def __init__(self, zkh, synth, rng, name, B, IN, OUT):
        self.zkh, self.name, self.B, self.IN, self.OUT = zkh, name, B, IN, OUT
        X = synth.gaussian_int16(rng, (B, IN))
        W = synth.fp8_e4m3_ints(rng, (IN, OUT))
        Y = synth.matmul_exact(X, W)
        self.ctx = zkh.Context(0)
        self.X = self.ctx.from_i32(X)
        self.W = self.ctx.weights_i32(W, IN, OUT)
        self.Y = self.ctx.from_i64(Y)
        st = zkh.transcript("cfg4:layer0.%s" % name)
        for lab, v in (("B", B), ("IN", IN), ("OUT", OUT)):
            zkh.absorb(st, lab, struct.pack("<I", v))
        zkh.absorb(st, "com_X", blob(name + "X", pow2(B) * 144))
        zkh.absorb(st, "com_W", blob(name + "W", pow2(IN) * 144))
        zkh.absorb(st, "com_Y", blob(name + "Y", pow2(B) * 144))
        self.st0 = st
        self.elements = mm_elements(B, IN, OUT)
        self.inputs = (X, W, Y)

    def run(self):
        st = self.st0.copy()
        out = self.ctx.mm_prove(st, self.X, self.W, self.Y, self.B, self.IN, self.OUT)
        return out["claims"].tobytes() + st.tobytes()


class GluJob:
    """SwiGLU obligation hot path (zkob_glu.cu:146-247): mapping lookup + Hadamard."""

    def __init__(self, zkh, synth, rng, B, C, scale_bits=12):
        self.zkh = zkh
        Cp, Bp = pow2(C), pow2(B)
        self.D = D = Bp * Cp
        self.N = N = D
        self.low = low = -(N // 2)
        self.ctx = zkh.Context(0)
        G = np.zeros((Bp, Cp), np.int32)
        G[:B, :C] = rng.integers(low, low + N, size=(B, C))
        U = np.zeros((Bp, Cp), np.int32)
        U[:B, :C] = synth.gaussian_int16(rng, (B, C))
        x = (np.arange(N, dtype=np.float64) + low) / (1 << scale_bits)
        silu = np.rint(x / (1.0 + np.exp(-x)) * (1 << scale_bits)).astype(np.int32)
        assert silu[-low] == 0  # the table holds (0, 0), so zero padding is a valid row
        self.G = self.ctx.from_i32(G)
        self.U = self.ctx.from_i32(U)
        self.mapped = self.ctx.from_i32(silu)
        self.T = self.ctx.range_table(low, N, N)
        st = zkh.transcript("cfg4:layer0.swiglu")
        for lab, v in (("B", B), ("C", C), ("LOW", low & 0xFFFFFFFF), ("LEN", N)):
            zkh.absorb(st, lab, struct.pack("<I", v))
        for lab in ("com_G", "com_S", "com_U", "com_H", "com_m"):
            zkh.absorb(st, lab, blob("glu" + lab, Bp * 144))
        self.st0 = st
        self.comA = blob("gluA", Bp * 144)
        self.logD = D.bit_length() - 1

    def run(self):
        zkh, c = self.zkh, self.ctx
        st = self.st0.copy()
        S, m = c.lu_mapping(self.G, self.low, self.mapped)
        r = zkh.challenge(st)
        beta = zkh.challenge(st)
        comb = c.axpy(self.G, r, S)
        Tcomb = c.axpy(self.T, r, self.mapped)
        A = c.lu_inverse(comb, beta)
        zkh.absorb(st, "com_A", self.comA)
        alpha = zkh.challenge(st)
        u = np.array([zkh.challenge(st) for _ in range(self.logD)])
        lu = c.lu_prove(st, A, comb, Tcomb, m, alpha, beta, u)
        u_h = np.array([zkh.challenge(st) for _ in range(self.logD)])
        H = c.hadamard(S, self.U)
        claim_H = c.me(H, u_h)
        zkh.absorb(st, "claim_H", claim_H.tobytes())
        hp = c.hp_prove_eq(st, claim_H, u_h, S, self.U)
        zkh.absorb(st, "S_f2", hp["term"][0].tobytes())
        zkh.absorb(st, "U_f2", hp["term"][1].tobytes())
        return lu["term"].tobytes() + hp["term"].tobytes() + st.tobytes()


class RopeJob:
    """One RoPE obligation (zkob_rope.cu:215-281): two eq-weighted Hadamard sumchecks
    c1 = sum eq(u,b) W1(b) T(b) and c2 = sum eq(u,b) W2(b) Tx(b), with U = 1."""

    def __init__(self, zkh, rng, name, B, C, HD=64):
        self.zkh = zkh
        Bp, Cp = pow2(B), pow2(C)
        self.D = Bp * Cp
        self.logD = self.D.bit_length() - 1
        self.ctx = c = zkh.Context(0)
        T = np.zeros((Bp, Cp), np.int32)
        T[:B, :C] = rng.integers(-(1 << 15), 1 << 15, size=(B, C))
        e = np.arange(Cp)
        flip = e ^ (HD // 2)
        Tx = T[:, np.minimum(flip, Cp - 1)] * (flip < Cp)
        t = np.arange(Bp)[:, None]
        ang = t / (10000.0 ** ((2 * ((e % HD) // 2)) / HD))[None, :]
        sigma = np.where(e & (HD // 2), 1, -1)[None, :]
        W1 = np.where(e[None, :] < C, np.rint(np.cos(ang) * 65536), 0).astype(np.int32)
        W2 = np.where(e[None, :] < C, sigma * np.rint(np.sin(ang) * 65536), 0).astype(np.int32)
        self.T, self.Tx = c.from_i32(T), c.from_i32(Tx.astype(np.int32))
        self.W1, self.W2 = c.from_i32(W1), c.from_i32(W2)
        self.ONE = c.from_i32(np.ones(self.D, np.int32))
        st = zkh.transcript("cfg4:layer0.rope." + name)
        for lab, v in (("B", B), ("C", C), ("HD", HD), ("SCALE_R", 16)):
            zkh.absorb(st, lab, struct.pack("<I", v))
        zkh.absorb(st, "com_T", blob("rope" + name + "T", Bp * 144))
        zkh.absorb(st, "com_Y64", blob("rope" + name + "Y", Bp * 144))
        self.st0 = st

    def run(self):
        zkh, c = self.zkh, self.ctx
        st = self.st0.copy()
        u = np.array([zkh.challenge(st) for _ in range(self.logD)])
        Eu = c.eq_table(u)
        outs = []
        for lab, W, S in (("c1", self.W1, self.T), ("c2", self.W2, self.Tx)):
            E = c.hadamard(Eu, W)
            claim = c.sum(c.hadamard(E, S))
            zkh.absorb(st, lab, claim.tobytes())
            hp = c.hp_prove(st, claim, E, S, self.ONE)
            zkh.absorb(st, "S_f2", hp["term"][0].tobytes())
            zkh.absorb(st, "U_f2", hp["term"][1].tobytes())
            outs.append(hp["term"].tobytes())
        return b"".join(outs) + st.tobytes()


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


def openings(zkh, jobs, outs, pool, reps=2, cpu=True):
    """The layer's 21 IPA openings (3 per matmul), the 7 matmuls concurrent on their own
    contexts; every pass must reproduce the first pass's proofs."""
    ref = [open_job(j, o) for j, o in zip(jobs, outs)]
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        futs = [pool.submit(open_job, j, o) for j, o in zip(jobs, outs)]
        assert [f.result() for f in futs] == ref, "non-deterministic openings"
        times.append(time.perf_counter() - t)
    res = {"ipa_s_per_layer": round(min(times), 4), "ipas": 3 * len(jobs),
           "scope": "ipa_W, ipa_X, ipa_Y of the 7 matmuls (vrf_common.cuh:302-336), byte-identical round points"}
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


def cpu_baseline(jobs, budget_names=("q", "k", "v", "o")):
    """The C oracle (reference algorithmic schedule, scalar, one thread) on a bounded
    sample: the four attention projections of the same layer."""
    sys.path.insert(0, ROOT)
    from oracle import coracle
    total_e, total_t = 0, 0.0
    for j in jobs:
        if j.name not in budget_names:
            continue
        X, W, Y = j.inputs
        st = coracle.tr_init("cpu")
        t0 = time.perf_counter()
        rc, _ = coracle.mm_prove(st, X, W, Y, j.B, j.IN, j.OUT)
        total_t += time.perf_counter() - t0
        assert rc == 0
        total_e += j.elements
    return {"value": total_e / total_t, "unit": "Fr elements/s", "cores": 1, "kind": "port",
            "sample": "C oracle (reference schedule: partial_me + multi_dim_me passes, per-round "
                      "zkip kernels) on the Q,K,V,O matmul sumchecks of the same layer "
                      "(%d elements, %.1f s, 1 thread)" % (total_e, total_t)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layer-steps", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-layer", action="store_true")
    ap.add_argument("--no-commit", action="store_true", help="skip the Pedersen commitments")
    ap.add_argument("--no-batchopen", action="store_true", help="skip the claim-mode batch opening")
    ap.add_argument("--no-prof", action="store_true", help="skip the profiled pass (no kernel times)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run one 256 MiB device-to-device copy (the known-size kernel that "
                         "scales rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--segment", choices=["glu", "rope", "commit", "batchopen"], default=None,
                    help="only run one non-matmul segment repeatedly (for profiling), then exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(see DESIGN.md for how the path would shard); run with --gpus 1", file=sys.stderr)
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
    if args.segment:
        job = GluJob(zkh, synth, rng, L["B"], L["ffn"]) if args.segment == "glu" else \
            RopeJob(zkh, rng, "q", L["B"], L["d"])
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

    ref = None
    for _ in range(args.warmup):
        mm_step()
        ref = mm_result()
    print("setup %.1fs; matmul step warm" % (time.perf_counter() - t_setup), file=sys.stderr, flush=True)
    # the interpreter's cyclic GC (millions of objects once torch is imported) would stall
    # a step for tens of ms at fixed allocation counts; it stays off while timing
    def timed_steps():
        gc.collect()
        gc.disable()
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
        assert ref is None or out == ref, "non-deterministic proof output"
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
        zkh.lib().zkh_prof_enable(mctx.h, 1)
        prof_ms_step, _ = timed_steps()

    # per-kernel device time over the profiled pass's steps (all contexts)
    import ctypes
    kern = {}
    buf = ctypes.create_string_buffer(4096)
    zkh.lib().zkh_prof_names(mctx.h, buf, 4096)
    for name in filter(None, buf.value.decode().split(",")):
        ms, la, by = ctypes.c_double(), ctypes.c_uint64(), ctypes.c_double()
        zkh.lib().zkh_prof_get(mctx.h, name.encode(), ctypes.byref(ms), ctypes.byref(la), ctypes.byref(by))
        kern[name] = [ms.value, la.value, by.value]
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
    if not args.no_layer:
        glu = GluJob(zkh, synth, rng, L["B"], L["ffn"])
        ropes = [RopeJob(zkh, rng, "q", L["B"], L["d"]), RopeJob(zkh, rng, "k", L["B"], L["kv"])]
        others = [glu] + ropes

        def layer_step():
            futs = [pool.submit(j.run) for j in others]
            mm_step()
            return [mm_result()] + [f.result() for f in futs]

        lref = layer_step()
        seg = {}
        for j in others:  # isolated segment times (sequential, for the breakdown)
            t = time.perf_counter()
            j.run()
            seg[type(j).__name__ + ("" if not hasattr(j, "logD") else ":2^%d" % j.logD)] = \
                round((time.perf_counter() - t) * 1000.0, 2)
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
        layer = {"prove_s_per_layer": (tb - ta) / args.layer_steps,
                 "segments_isolated_ms": seg,
                 "scope": "7 matmul sumchecks + SwiGLU logUp (D=N=2^22) + its Hadamard (2^22) + "
                          "RoPE q/k Hadamards (2x2^20, 2x2^17), concurrent; commitments, IPA "
                          "openings and the witness GEMM excluded"}
        print("layer %.3f s" % layer["prove_s_per_layer"], file=sys.stderr, flush=True)

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
    cpu = None if args.no_cpu else cpu_baseline(jobs)
    res = {
        "metric": "Fr elements bound/sec in matmul sumcheck; prove s/layer at TinyLlama-1.1B",
        "value": value, "unit": "Fr elements/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_step, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "u32", "data": "synthetic",
        "config": {"workload": "TinyLlama-1.1B layer (BASELINE config 4), seq 512: Q,K,V,O,gate,up,down "
                               "matmul sumchecks", "B": L["B"], "d": L["d"], "kv": L["kv"],
                   "ffn": L["ffn"], "elements_bound_per_step": E_total, "field": "BLS12-381 Fr"},
        "roofline": roofline, "kernels": kernels, "cpu_baseline": cpu,
    }
    if layer:
        res["prove_s_per_layer"] = layer["prove_s_per_layer"]
        res["layer"] = layer
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
