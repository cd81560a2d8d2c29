"""Textbook BLS12-381 G1 arithmetic with Python big integers (small cases only).

TEST INFRASTRUCTURE ONLY: pins the C oracle's G1 routines (zkh_g1_oracle.c) and, through
it, the GPU commitment path.  It is written from the curve's definition, not from the
reference's formulas: affine chord-and-tangent addition on y^2 = x^3 + 4 over Fp with
field inversion by pow(), so a mistake in the Montgomery limbs or in the Jacobian
formulas shows up as a different group element.  Points cross as the reference's
144-byte G1Jacobian_t (g1-tensor.cuh:63): x, y, z each 12 little-endian uint32 limbs in
Montgomery form (R = 2^384); affine points here are (x, y) ints or None for infinity.
"""
import numpy as np

P = 0x1A0111EA397FE69A4B1BA7B6434BACD764774B84F38512BF6730D2A0F6B0F6241EABFFFEB153FFFFB9FEFFFFFFFFAAAB
MONT = 1 << 384
MONT_INV = pow(MONT, -1, P)
B = 4
# standard generator (affine, plain)
GX = 0x17F1D3A73197D7942695638C4FA9AC0FC3688C4F9774B905A14E3A3F171BAC586C55E83FF97A1AEFFB3AF00ADB22C6BB
GY = 0x08B3F481E3AAA0F1A09E30ED741D8AE4FCF5E095D5D00AF600DB18CB2C04B3EDD03CC744A2888AE40CAA232946C5E7E1
# subgroup order = the scalar field modulus r
ORDER = 0x73EDA753299D7D483339D80809A1D80553BDA402FFFE5BFEFFFFFFFF00000001


def limbs12(x):
    return np.array([(x >> (32 * i)) & 0xFFFFFFFF for i in range(12)], dtype=np.uint32)


def from_limbs12(v):
    return sum(int(v[i]) << (32 * i) for i in range(12))


def to_mont(x):
    return x * MONT % P


def from_mont(x):
    return x * MONT_INV % P


def jac_ints(pt):
    """(36,) uint32 Jacobian point -> plain (X, Y, Z) ints."""
    pt = np.asarray(pt, dtype=np.uint32)
    return tuple(from_mont(from_limbs12(pt[12 * k:12 * k + 12])) for k in range(3))


def jac_point(X, Y, Z):
    """plain (X, Y, Z) ints -> (36,) uint32 in the reference's Montgomery layout."""
    return np.concatenate([limbs12(to_mont(v % P)) for v in (X, Y, Z)])


def to_affine(pt):
    X, Y, Z = jac_ints(pt)
    if Z == 0:
        return None
    zi = pow(Z, -1, P)
    return (X * zi * zi % P, Y * zi * zi * zi % P)


def on_curve_jac(pt):
    """Y^2 = X^3 + 4 Z^6 (holds for Z = 0 only if Y^2 = X^3)."""
    X, Y, Z = jac_ints(pt)
    return (Y * Y - X * X * X - B * pow(Z, 6, P)) % P == 0


def aff_add(a, b):
    if a is None:
        return b
    if b is None:
        return a
    (x1, y1), (x2, y2) = a, b
    if x1 == x2:
        if (y1 + y2) % P == 0:
            return None
        lam = 3 * x1 * x1 * pow(2 * y1, -1, P) % P
    else:
        lam = (y2 - y1) * pow(x2 - x1, -1, P) % P
    x3 = (lam * lam - x1 - x2) % P
    return (x3, (lam * (x1 - x3) - y1) % P)


def aff_mul(a, k):
    out, acc = None, a
    while k:
        if k & 1:
            out = aff_add(out, acc)
        acc = aff_add(acc, acc)
        k >>= 1
    return out


def aff_to_jac(a, z=1):
    """affine point -> Jacobian (x z^2, y z^3, z) for a chosen z != 0."""
    if a is None:
        return jac_point(0, 1, 0)
    x, y = a
    return jac_point(x * z * z, y * z * z * z, z)


def g1_zero():
    """blstrs__g1__G1Affine_ZERO = {0, ONE, 0} (bls12-381.cuh:422)."""
    return jac_point(0, 1, 0)
