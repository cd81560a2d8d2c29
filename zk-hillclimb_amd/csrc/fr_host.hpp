// fr_host.hpp -- host-side BLS12-381 Fr scalar arithmetic for the round-by-round
// Fiat-Shamir logic (round polynomials, Lagrange interpolation, eq factors).
//
// The reference performs these few-per-round scalar operations as one-thread GPU kernels
// with a cudaMalloc + memcpy each (polynomial.cu:9-150, vrf_common.cuh:100-104); here they
// run on the host in 4 x 64-bit limbs (CIOS Montgomery with unsigned __int128).  Values
// are canonical, plain (integer view) unless a name says _m (Montgomery form x*2^256).
#pragma once
#include <stdint.h>
#include <string.h>

namespace zkh {

typedef unsigned __int128 u128;

struct Fr {
    uint64_t v[4];
};

static const Fr kP = {{0xffffffff00000001ULL, 0x53bda402fffe5bfeULL, 0x3339d80809a1d805ULL,
                       0x73eda753299d7d48ULL}};
static const Fr kR2 = {{0xc999e990f3f29c6dULL, 0x2b6cedcb87925c23ULL, 0x05d314967254398fULL,
                        0x0748d9d99f59ff11ULL}};
static const uint64_t kInv = 0xfffffffeffffffffULL;  // -r^-1 mod 2^64
static const Fr kZero = {{0, 0, 0, 0}};
static const Fr kOne = {{1, 0, 0, 0}};

inline Fr fr_u64(uint64_t x) { return Fr{{x, 0, 0, 0}}; }
inline bool fr_eq(const Fr& a, const Fr& b) { return memcmp(a.v, b.v, 32) == 0; }
inline bool fr_geq(const Fr& a, const Fr& b) {
    for (int i = 3; i >= 0; i--) {
        if (a.v[i] != b.v[i]) return a.v[i] > b.v[i];
    }
    return true;
}
inline Fr raw_sub(const Fr& a, const Fr& b) {
    Fr r;
    uint64_t br = 0;
    for (int i = 0; i < 4; i++) {
        u128 d = (u128)a.v[i] - b.v[i] - br;
        r.v[i] = (uint64_t)d;
        br = (uint64_t)(d >> 64) & 1;
    }
    return r;
}
inline Fr raw_add(const Fr& a, const Fr& b, uint64_t* carry) {
    Fr r;
    uint64_t c = 0;
    for (int i = 0; i < 4; i++) {
        u128 s = (u128)a.v[i] + b.v[i] + c;
        r.v[i] = (uint64_t)s;
        c = (uint64_t)(s >> 64);
    }
    *carry = c;
    return r;
}
inline Fr fr_add(const Fr& a, const Fr& b) {
    uint64_t c;
    Fr s = raw_add(a, b, &c);
    if (c || fr_geq(s, kP)) s = raw_sub(s, kP);
    return s;
}
inline Fr fr_sub(const Fr& a, const Fr& b) {
    Fr d = raw_sub(a, b);
    if (!fr_geq(a, b)) {
        uint64_t c;
        d = raw_add(d, kP, &c);
    }
    return d;
}
inline Fr fr_neg(const Fr& a) { return fr_sub(kZero, a); }
inline Fr fr_mont_mul(const Fr& a, const Fr& b) {
    uint64_t t[6] = {0, 0, 0, 0, 0, 0};
    for (int i = 0; i < 4; i++) {
        u128 c = 0;
        for (int j = 0; j < 4; j++) {
            c = (u128)a.v[j] * b.v[i] + t[j] + (uint64_t)(c >> 64);
            t[j] = (uint64_t)c;
        }
        c = (u128)t[4] + (uint64_t)(c >> 64);
        t[4] = (uint64_t)c;
        t[5] = (uint64_t)(c >> 64);
        uint64_t m = t[0] * kInv;
        c = (u128)m * kP.v[0] + t[0];
        for (int j = 1; j < 4; j++) {
            c = (u128)m * kP.v[j] + t[j] + (uint64_t)(c >> 64);
            t[j - 1] = (uint64_t)c;
        }
        c = (u128)t[4] + (uint64_t)(c >> 64);
        t[3] = (uint64_t)c;
        t[4] = t[5] + (uint64_t)(c >> 64);
    }
    Fr r = {{t[0], t[1], t[2], t[3]}};
    if (t[4] || fr_geq(r, kP)) r = raw_sub(r, kP);
    return r;
}
inline Fr fr_to_mont(const Fr& a) { return fr_mont_mul(a, kR2); }
inline const Fr& fr_one_m() {  // 1 in Montgomery form (2^256 mod r)
    static const Fr v = fr_to_mont(kOne);
    return v;
}
inline Fr fr_from_mont(const Fr& a) { return fr_mont_mul(a, kOne); }
inline Fr fr_mul(const Fr& a, const Fr& b) { return fr_mont_mul(fr_to_mont(a), b); }
// a^e for a plain a and a 256-bit exponent
inline Fr fr_pow(const Fr& a, const Fr& e) {
    Fr base = fr_to_mont(a), acc = fr_to_mont(kOne);
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 64; j++) {
            if ((e.v[i] >> j) & 1) acc = fr_mont_mul(acc, base);
            base = fr_mont_mul(base, base);
        }
    return fr_from_mont(acc);
}
// a^(r-2) (Fermat): the inverse, inverse(0) = 0 (the reference's convention, tlookup.cu:50-62)
inline Fr fr_inv_fermat(const Fr& a) { return fr_pow(a, raw_sub(kP, fr_u64(2))); }
inline Fr raw_shr1(const Fr& a) {
    Fr r;
    for (int i = 0; i < 3; i++) r.v[i] = (a.v[i] >> 1) | (a.v[i + 1] << 63);
    r.v[3] = a.v[3] >> 1;
    return r;
}
// x / 2 mod r for x < r: x >> 1, or (x + r) >> 1 for odd x (x + r < 2^256 as r < 2^255)
inline Fr fr_half(const Fr& x) {
    if (!(x.v[0] & 1)) return raw_shr1(x);
    uint64_t c;
    return raw_shr1(raw_add(x, kP, &c));
}
// The inverse by the binary extended Euclidean algorithm (Knuth, TAOCP vol. 2, 4.5.2,
// Algorithm B with the cofactors kept mod r): u = x1 a, v = x2 a (mod r) hold throughout,
// and gcd(a, r) = 1 ends the loop at u = 1 or v = 1.  Same value as fr_inv_fermat, about 1
// shift or subtraction per bit instead of some 380 Montgomery products; inverse(0) = 0.
inline Fr fr_inv(const Fr& a) {
    if (fr_eq(a, kZero)) return kZero;
    Fr u = a, v = kP, x1 = kOne, x2 = kZero;
    while (!fr_eq(u, kOne) && !fr_eq(v, kOne)) {
        while (!(u.v[0] & 1)) {
            u = raw_shr1(u);
            x1 = fr_half(x1);
        }
        while (!(v.v[0] & 1)) {
            v = raw_shr1(v);
            x2 = fr_half(x2);
        }
        if (fr_geq(u, v)) {
            u = raw_sub(u, v);
            x1 = fr_sub(x1, x2);
        } else {
            v = raw_sub(v, u);
            x2 = fr_sub(x2, x1);
        }
    }
    return fr_eq(u, kOne) ? x1 : x2;
}
inline Fr fr_from_i64(int64_t v) {
    if (v >= 0) return fr_u64((uint64_t)v);
    uint64_t mag = (uint64_t)(-(v + 1)) + 1;
    return fr_sub(kZero, fr_u64(mag));
}
// 2^256k mod r, i.e. the factor that undoes k Montgomery reductions
inline Fr fr_rpow(int k) {
    Fr x = kOne;
    for (int i = 0; i < k; i++) x = fr_mont_mul(x, kR2);  // x * 2^256
    return x;
}
inline void fr_store(const Fr& x, uint32_t* p) {
    for (int i = 0; i < 4; i++) {
        p[2 * i] = (uint32_t)x.v[i];
        p[2 * i + 1] = (uint32_t)(x.v[i] >> 32);
    }
}
inline Fr fr_load(const uint32_t* p) {
    Fr x;
    for (int i = 0; i < 4; i++) x.v[i] = (uint64_t)p[2 * i] | ((uint64_t)p[2 * i + 1] << 32);
    return x;
}
inline bool fr_is_canonical(const uint32_t* p) { return !fr_geq(fr_load(p), kP); }
// eq(u,v) = 2uv - u - v + 1 (polynomial.cu:355-372)
inline Fr fr_eq2(const Fr& u, const Fr& v) {
    Fr uv = fr_mul(u, v);
    return fr_add(fr_sub(fr_add(uv, uv), fr_add(u, v)), kOne);
}
// Lagrange interpolation through (t, p[t]), t = 0..2 (vrf_common.cuh:130-140)
inline Fr fr_lagrange3(const Fr p[3], const Fr& u) {
    static const Fr inv2 = {{0x7fffffff80000001ULL, 0xa9ded2017fff2dffULL,
                             0x199cec0404d0ec02ULL, 0x39f6d3a994cebea4ULL}};
    Fr two = fr_u64(2), um1 = fr_sub(u, kOne), um2 = fr_sub(u, two);
    Fr l0 = fr_mul(fr_mul(um1, um2), inv2);
    Fr l1 = fr_mul(u, fr_sub(two, u));
    Fr l2 = fr_mul(fr_mul(u, um1), inv2);
    return fr_add(fr_add(fr_mul(p[0], l0), fr_mul(p[1], l1)), fr_mul(p[2], l2));
}
// coefficient-form evaluation
inline Fr fr_poly_eval(const Fr* c, int deg, const Fr& x) {
    Fr acc = c[deg];
    for (int i = deg - 1; i >= 0; i--) acc = fr_add(fr_mul(acc, x), c[i]);
    return acc;
}
// (r+1)/2
inline Fr fr_inv2() {
    return Fr{{0x7fffffff80000001ULL, 0xa9ded2017fff2dffULL, 0x199cec0404d0ec02ULL,
               0x39f6d3a994cebea4ULL}};
}

}  // namespace zkh
