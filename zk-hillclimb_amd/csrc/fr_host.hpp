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
inline Fr fr_inv_bin(const Fr& a) {
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
namespace inv_detail {
// five-limb two's complement values (the products of a 256-bit value and a signed factor)
inline void neg5(uint64_t r[5]) {
    uint64_t c = 1;
    for (int i = 0; i < 5; i++) {
        const u128 s = (u128)(~r[i]) + c;
        r[i] = (uint64_t)s;
        c = (uint64_t)(s >> 64);
    }
}
// r = x f for x < 2^256 and |f| < 2^63
inline void mul_s64(const uint64_t x[4], int64_t f, uint64_t r[5]) {
    const uint64_t af = f < 0 ? 0 - (uint64_t)f : (uint64_t)f;
    u128 c = 0;
    for (int i = 0; i < 4; i++) {
        c = (u128)x[i] * af + (uint64_t)(c >> 64);
        r[i] = (uint64_t)c;
    }
    r[4] = (uint64_t)(c >> 64);
    if (f < 0) neg5(r);
}
inline void add5(uint64_t r[5], const uint64_t b[5]) {
    uint64_t c = 0;
    for (int i = 0; i < 5; i++) {
        const u128 s = (u128)r[i] + b[i] + c;
        r[i] = (uint64_t)s;
        c = (uint64_t)(s >> 64);
    }
}
inline void sar31(uint64_t r[5]) {  // arithmetic shift right by 31
    for (int i = 0; i < 4; i++) r[i] = (r[i] >> 31) | (r[i + 1] << 33);
    r[4] = (uint64_t)((int64_t)r[4] >> 31);
}
inline bool is_neg(const uint64_t r[5]) { return (int64_t)r[4] < 0; }
// x f + y g for x, y < 2^256, |f|, |g| <= 2^31
inline void lin(const uint64_t x[4], int64_t f, const uint64_t y[4], int64_t g, uint64_t r[5]) {
    uint64_t t[5];
    mul_s64(x, f, r);
    mul_s64(y, g, t);
    add5(r, t);
}
inline uint32_t bitlen(const uint64_t x[4]) {
    for (int i = 3; i >= 0; i--)
        if (x[i]) return 64 * i + 64 - (uint32_t)__builtin_clzll(x[i]);
    return 0;
}
inline uint64_t bits_at(const uint64_t x[4], uint32_t s) {  // (x >> s) mod 2^64, s < 256
    const uint32_t l = s >> 6, o = s & 63;
    const uint64_t lo = x[l] >> o;
    return o && l < 3 ? lo | (x[l + 1] << (64 - o)) : lo;
}
// (u f + v g) / 2^31 mod r for canonical u, v: one 31-bit Montgomery step, then 0 <= . < r
inline Fr lin_div31(const Fr& u, int64_t f, const Fr& v, int64_t g) {
    uint64_t t[5], qr[5];
    lin(u.v, f, v.v, g, t);
    const int64_t q = (int64_t)((t[0] * kInv) & 0x7fffffffULL);  // t + q r = 0 mod 2^31
    mul_s64(kP.v, q, qr);
    add5(t, qr);
    sar31(t);  // now in (-2r, 3r)
    uint64_t p5[5] = {kP.v[0], kP.v[1], kP.v[2], kP.v[3], 0};
    while (is_neg(t)) add5(t, p5);
    Fr x = {{t[0], t[1], t[2], t[3]}};
    while (t[4] || fr_geq(x, kP)) {
        uint64_t m5[5] = {kP.v[0], kP.v[1], kP.v[2], kP.v[3], 0};
        neg5(m5);
        add5(t, m5);
        x = Fr{{t[0], t[1], t[2], t[3]}};
    }
    return x;
}
}  // namespace inv_detail
// The inverse by Pornin's optimized binary GCD (T. Pornin, "Optimized Binary GCD for Modular
// Inversion", IACR ePrint 2020/972, Algorithm 2 with k = 32).  Each outer step runs 31
// binary-GCD iterations on 64-bit approximations of a and b (their low 31 bits and their top
// 33 bits at the length of the longer one), collecting the update (f0 g0; f1 g1); then a, b
// become (a f0 + b g0) / 2^31, (a f1 + b g1) / 2^31 (made nonnegative by flipping the row's
// signs) and the cofactors u, v the same combinations divided by 2^31 mod r.  a = u y and
// b = v y (mod r) hold throughout; with gcd(y, r) = 1 the loop ends at a = 0, b = 1, v = 1/y,
// after about 17 outer steps for this 255-bit r instead of some 500 bit-by-bit iterations.
// A run that does not end at b = 1 (it cannot for prime r and y != 0) falls back to
// fr_inv_bin; inverse(0) = 0.
inline Fr fr_inv(const Fr& y) {
    using namespace inv_detail;
    if (fr_eq(y, kZero)) return kZero;
    uint64_t a[4], b[4];
    memcpy(a, y.v, 32);
    memcpy(b, kP.v, 32);
    Fr u = kOne, v = kZero;
    for (int it = 0; it < 64 && (a[0] | a[1] | a[2] | a[3]); it++) {
        uint32_t n = bitlen(a) > bitlen(b) ? bitlen(a) : bitlen(b);
        if (n < 64) n = 64;
        uint64_t ab = (a[0] & 0x7fffffffULL) | (bits_at(a, n - 33) << 31);
        uint64_t bb = (b[0] & 0x7fffffffULL) | (bits_at(b, n - 33) << 31);
        int64_t f0 = 1, g0 = 0, f1 = 0, g1 = 1;
        for (int j = 0; j < 31; j++) {  // branch-free: odd a swaps when a < b, then subtracts
            const uint64_t odd = 0 - (ab & 1), sw = odd & (0 - (uint64_t)(ab < bb));
            const uint64_t tx = (ab ^ bb) & sw;
            ab ^= tx;
            bb ^= tx;
            const int64_t tf = (f0 ^ f1) & (int64_t)sw, tg = (g0 ^ g1) & (int64_t)sw;
            f0 ^= tf;
            f1 ^= tf;
            g0 ^= tg;
            g1 ^= tg;
            ab = (ab - (bb & odd)) >> 1;
            f0 -= f1 & (int64_t)odd;
            g0 -= g1 & (int64_t)odd;
            f1 *= 2;
            g1 *= 2;
        }
        uint64_t na[5], nb[5];
        lin(a, f0, b, g0, na);
        lin(a, f1, b, g1, nb);
        sar31(na);
        sar31(nb);
        if (is_neg(na)) {
            neg5(na);
            f0 = -f0;
            g0 = -g0;
        }
        if (is_neg(nb)) {
            neg5(nb);
            f1 = -f1;
            g1 = -g1;
        }
        if (na[4] || nb[4]) return fr_inv_bin(y);  // cannot happen: |a'|, |b'| <= max(a, b)
        memcpy(a, na, 32);
        memcpy(b, nb, 32);
        const Fr nu = lin_div31(u, f0, v, g0), nv = lin_div31(u, f1, v, g1);
        u = nu;
        v = nv;
    }
    if (a[0] | a[1] | a[2] | a[3] || b[0] != 1 || b[1] | b[2] | b[3]) return fr_inv_bin(y);
    return v;
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
