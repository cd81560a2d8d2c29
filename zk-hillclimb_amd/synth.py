"""Seeded synthetic inputs shaped like the reference's workloads (no datasets, no weights).

- fp8-e4m3 weights as exact scaled integers: a uniform byte code among the 254 non-NaN
  codes, decoded to v = value * 2^9 (subnormal E=0: v = M; normal: v = (8+M)*2^(E-1)),
  so |v| <= 229376 (the reference's fp8-exact convention, FP8_EXACT_PLAN.md:53-55).
- "Gaussian int16" activations: round(N(0,1) * 2^12) clamped to [-2^15, 2^15).
- PRNG: numpy PCG64 seeded per config (0x5EED0000 + config number).
"""
import numpy as np


def fp8_e4m3_ints(rng, shape):
    codes = rng.integers(0, 254, size=shape)
    # skip the two NaN codes 0x7f and 0xff: map [0,254) onto the 256 codes minus NaNs
    codes = codes + (codes >= 0x7F)          # 0x7f -> 0x80 ...
    codes = codes + (codes >= 0xFF)
    s = (codes >> 7) & 1
    e = (codes >> 3) & 0xF
    m = codes & 7
    mag = np.where(e == 0, m, (8 + m) << np.maximum(e - 1, 0))
    return np.where(s == 1, -mag, mag).astype(np.int32)


def gaussian_int16(rng, shape, scale_bits=12):
    x = np.rint(rng.standard_normal(shape) * (1 << scale_bits))
    return np.clip(x, -(1 << 15), (1 << 15) - 1).astype(np.int32)


def matmul_exact(X, W):
    """Y = X @ W exactly (int64).  |X| < 2^15, |W| < 2^18 and IN < 2^20 keep every partial
    sum below 2^53, so float64 products and sums are exact."""
    Y = X.astype(np.float64) @ W.astype(np.float64)
    return np.rint(Y).astype(np.int64)


def rng_for(config):
    return np.random.default_rng(0x5EED0000 + config)


def pow2(n):
    return 1 << ((n - 1).bit_length()) if n > 1 else 1


# BASELINE.json configurations (shapes of the reference's workloads).  Matmuls are
# (name, IN, OUT) at batch B; `glu` is the SwiGLU lookup grid (rows B, columns ffn) with its
# table size; `rope` the RoPE Hadamard obligations (name, columns) at head_dim hd.
CONFIGS = {
    "C1": dict(B=64, matmuls=[("fc", 128, 64)]),
    "C2": dict(B=128, matmuls=[("up", 768, 3072), ("down", 3072, 768)]),
    "C3": dict(D=1 << 20, N=1 << 16, low=-(1 << 15)),
    "C4": dict(B=512, d=2048, kv=256, ffn=5632, hd=64,
               matmuls=[("q", 2048, 2048), ("k", 2048, 256), ("v", 2048, 256), ("o", 2048, 2048),
                        ("gate", 2048, 5632), ("up", 2048, 5632), ("down", 5632, 2048)],
               glu_table=1 << 22, rope=[("q", 2048), ("k", 256)]),
    "C5": dict(B=2048, d=3200, kv=3200, ffn=8640, hd=100,
               matmuls=[("q", 3200, 3200), ("k", 3200, 3200), ("v", 3200, 3200), ("o", 3200, 3200),
                        ("gate", 3200, 8640), ("up", 3200, 8640), ("down", 8640, 3200)],
               glu_table=1 << 22),
}


def mm_elements(B, IN, OUT):
    """Fr entries bound by one matmul sumcheck: X, W, Y and the two folded IN-vectors."""
    return B * IN + IN * OUT + B * OUT + 2 * IN


def matmul_inputs(rng, B, IN, OUT):
    """Gaussian int16 activations X (B x IN), fp8-e4m3 weights W (IN x OUT), Y = X W."""
    X = gaussian_int16(rng, (B, IN))
    W = fp8_e4m3_ints(rng, (IN, OUT))
    return X, W, matmul_exact(X, W)


def silu_table(N, low, scale_bits=12):
    """silu(x) at x = (low + i) / 2^scale_bits, rounded to the same fixed point; N entries."""
    x = (np.arange(N, dtype=np.float64) + low) / (1 << scale_bits)
    return np.rint(x / (1.0 + np.exp(-x)) * (1 << scale_bits)).astype(np.int32)


def glu_inputs(rng, B, C, N=None, scale_bits=12):
    """SwiGLU obligation inputs (zkob_glu.cu:83-156) on the padded grid Bp x Cp: G uniform in
    the table domain [low, low + N), U Gaussian int16, zero padding; N defaults to the grid
    size (the reference's D = N case).  The table contains (0, 0), so padding rows are valid."""
    Bp, Cp = pow2(B), pow2(C)
    D = Bp * Cp
    N = D if N is None else N
    low = -(N // 2)
    G = np.zeros((Bp, Cp), np.int32)
    G[:B, :C] = rng.integers(low, low + N, size=(B, C))
    U = np.zeros((Bp, Cp), np.int32)
    U[:B, :C] = gaussian_int16(rng, (B, C))
    silu = silu_table(N, low, scale_bits)
    assert silu[-low] == 0
    return dict(G=G, U=U, silu=silu, low=low, N=N, D=D, Bp=Bp, Cp=Cp)


def rope_inputs(rng, B, C, HD=64):
    """RoPE obligation inputs (zkob_rope.cu:72-114): T (B x C int16-range activations), its
    rotate-half partner Tx and the fixed-point cos / signed sin weights W1, W2 (scale 2^16),
    all zero-padded to Bp x Cp."""
    Bp, Cp = pow2(B), pow2(C)
    T = np.zeros((Bp, Cp), np.int32)
    T[:B, :C] = rng.integers(-(1 << 15), 1 << 15, size=(B, C))
    e = np.arange(Cp)
    flip = e ^ (HD // 2)
    Tx = (T[:, np.minimum(flip, Cp - 1)] * (flip < Cp)).astype(np.int32)
    t = np.arange(Bp)[:, None]
    ang = t / (10000.0 ** ((2 * ((e % HD) // 2)) / HD))[None, :]
    sigma = np.where(e & (HD // 2), 1, -1)[None, :]
    W1 = np.where(e[None, :] < C, np.rint(np.cos(ang) * 65536), 0).astype(np.int32)
    W2 = np.where(e[None, :] < C, sigma * np.rint(np.sin(ang) * 65536), 0).astype(np.int32)
    return dict(T=T, Tx=Tx, W1=W1, W2=W2, Bp=Bp, Cp=Cp, D=Bp * Cp)
