// fr_dev.hpp -- BLS12-381 scalar-field arithmetic for gfx950 (CDNA4) integer VALU.
//
// Elements are 8 x 32-bit limbs, little-endian, canonical in [0, r).  The Montgomery
// product (R = 2^256, so mont_mul(a, b) = a*b*2^-256 mod r) is product scanning with the
// reduction interleaved per column (Koc, Acar, Kaliski, "Analyzing and comparing Montgomery
// multiplication algorithms", 1996), generated straight-line by gen_mont_mul.py: each of
// the 120 32x32 products is one v_mad_u64_u32 whose carry-out feeds a v_addc_co_u32 into
// a 96-bit column sum.  Since -r^-1 mod 2^32 = 0xffffffff, the reduction multiplier of a
// column is minus its low word.
//
// Tables in HBM use a structure-of-limb-quads layout: limbs 0-3 of element i in plane 0
// at lo[i] (uint4), limbs 4-7 in plane 1 at hi[i], so every wave load reads 1 KiB
// contiguous per plane.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define ZDEV __device__ __forceinline__

struct fr_t {
    uint32_t v[8];
};

// r (bls12-381.cu:4)
#define ZKH_P0 0x00000001u
#define ZKH_P1 0xffffffffu
#define ZKH_P2 0xfffe5bfeu
#define ZKH_P3 0x53bda402u
#define ZKH_P4 0x09a1d805u
#define ZKH_P5 0x3339d808u
#define ZKH_P6 0x299d7d48u
#define ZKH_P7 0x73eda753u

ZDEV uint32_t fr_p(int i) {
    switch (i) {
        case 0: return ZKH_P0;
        case 1: return ZKH_P1;
        case 2: return ZKH_P2;
        case 3: return ZKH_P3;
        case 4: return ZKH_P4;
        case 5: return ZKH_P5;
        case 6: return ZKH_P6;
        default: return ZKH_P7;
    }
}

ZDEV fr_t fr_zero() {
    fr_t r;
#pragma unroll
    for (int i = 0; i < 8; i++) r.v[i] = 0;
    return r;
}

// Multi-limb carries go through __builtin_addc / __builtin_subc, which lower to
// v_add_co_u32 / v_addc_co_u32 (v_sub_co / v_subb) chains on VCC: about a third of the
// instructions of the same arithmetic written with 64-bit intermediates.

// r if x >= r else x, for x < 2r (single correction, as bls12-381.cu:295-300)
ZDEV fr_t fr_reduce_once(const fr_t& x, uint32_t carry_in) {
    fr_t d;
    unsigned br = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) d.v[i] = __builtin_subc(x.v[i], fr_p(i), br, &br);
    // keep x when it borrowed (x < r) and there was no carry out of limb 7
    const bool keep = (br != 0) && (carry_in == 0);
    fr_t r;
#pragma unroll
    for (int i = 0; i < 8; i++) r.v[i] = keep ? x.v[i] : d.v[i];
    return r;
}

ZDEV fr_t fr_add(const fr_t& a, const fr_t& b) {
    fr_t s;
    unsigned c = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) s.v[i] = __builtin_addc(a.v[i], b.v[i], c, &c);
    return fr_reduce_once(s, c);
}

ZDEV fr_t fr_sub(const fr_t& a, const fr_t& b) {
    fr_t d;
    unsigned br = 0, c = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) d.v[i] = __builtin_subc(a.v[i], b.v[i], br, &br);
    // on borrow add r back
    const unsigned mask = 0u - br;
#pragma unroll
    for (int i = 0; i < 8; i++) d.v[i] = __builtin_addc(d.v[i], fr_p(i) & mask, c, &c);
    return d;
}

// 96-bit column accumulation: (lo64, top) += x*y with v_mad_u64_u32's carry-out feeding
// v_addc_co_u32.  A VALU-written SGPR needs one wait state before a VALU reads it as a
// carry, so paired forms interleave two independent chains and single forms use s_nop.
ZDEV void mac1_v(uint64_t& lo, uint32_t& top, uint32_t x, uint32_t y) {
    uint64_t c;
    asm("v_mad_u64_u32 %0, %2, %3, %4, %0\n\ts_nop 0\n\tv_addc_co_u32 %1, %2, 0, %1, %2"
        : "+v"(lo), "+v"(top), "=&s"(c) : "v"(x), "v"(y));
}
ZDEV void mac1_s(uint64_t& lo, uint32_t& top, uint32_t x, uint32_t y) {
    uint64_t c;
    asm("v_mad_u64_u32 %0, %2, %3, %4, %0\n\ts_nop 0\n\tv_addc_co_u32 %1, %2, 0, %1, %2"
        : "+v"(lo), "+v"(top), "=&s"(c) : "v"(x), "s"(y));
}
#define ZKH_MAC2(NAME, C1, C2)                                                                  \
    ZDEV void NAME(uint64_t& lo0, uint32_t& top0, uint32_t x0, uint32_t y0, uint64_t& lo1,       \
                   uint32_t& top1, uint32_t x1, uint32_t y1) {                                  \
        uint64_t c0, c1;                                                                        \
        asm("v_mad_u64_u32 %0, %2, %6, %7, %0\n\t"                                              \
            "v_mad_u64_u32 %3, %5, %8, %9, %3\n\t"                                              \
            "v_addc_co_u32 %1, %2, 0, %1, %2\n\t"                                               \
            "v_addc_co_u32 %4, %5, 0, %4, %5"                                                   \
            : "+v"(lo0), "+v"(top0), "=&s"(c0), "+v"(lo1), "+v"(top1), "=&s"(c1)                \
            : "v"(x0), C1(y0), "v"(x1), C2(y1));                                                \
    }
ZKH_MAC2(mac2_vv, "v", "v")
ZKH_MAC2(mac2_vs, "v", "s")
ZKH_MAC2(mac2_sv, "s", "v")
ZKH_MAC2(mac2_ss, "s", "s")

// Montgomery product a*b*2^-256 mod r, canonical output for canonical inputs
// (the same value as the reference's blstrs__scalar__Scalar_mul, bls12-381.cu:462-531).
#include "mont_mul_ps.inc"

// Montgomery reduction of a wide non-negative integer T (nl <= 16 limbs, T < r*2^256):
// returns T*2^-256 mod r.  Used to fold wide integer accumulators into the field.
template <int NL>
ZDEV fr_t redc_wide(const uint32_t* in) {
    uint32_t t[17];
#pragma unroll
    for (int j = 0; j < 17; j++) t[j] = j < NL ? in[j] : 0u;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        uint32_t m = 0u - t[i];
        uint64_t c = (uint64_t)m * ZKH_P0 + t[i];
#pragma unroll
        for (int j = 1; j < 8; j++) {
            c = (uint64_t)m * fr_p(j) + t[i + j] + (c >> 32);
            t[i + j] = (uint32_t)c;
        }
#pragma unroll
        for (int j = i + 8; j < 17; j++) {
            c = (uint64_t)t[j] + (c >> 32);
            t[j] = (uint32_t)c;
        }
    }
    fr_t r;
#pragma unroll
    for (int j = 0; j < 8; j++) r.v[j] = t[8 + j];
    return fr_reduce_once(r, t[16]);
}

// ---- 64-bit column accumulators for small-integer x field products ----
// acc[j] += w * e[j] with w < 2^20: each product < 2^52, so 2^11 additions stay < 2^63.
ZDEV void cols_mac(uint64_t acc[8], uint32_t w, const fr_t& e) {
#pragma unroll
    for (int j = 0; j < 8; j++) acc[j] += (uint64_t)w * e.v[j];
}
// sum_j acc[j] * 2^(32j) as a 10-limb integer (each acc[j] < 2^63)
ZDEV void cols_normalize(const uint64_t acc[8], uint32_t out[10]) {
    uint64_t c = 0;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        uint64_t s = acc[j] + c;  // < 2^63 + 2^33
        out[j] = (uint32_t)s;
        c = s >> 32;
    }
    out[8] = (uint32_t)c;
    out[9] = (uint32_t)(c >> 32);
}

// ---- loads / stores in the limb-quad layout ----
struct FrPlanes {
    uint4* lo;
    uint4* hi;
};
ZDEV fr_t ld_fr(const uint4* lo, const uint4* hi, uint32_t i) {
    uint4 a = lo[i], b = hi[i];
    fr_t r;
    r.v[0] = a.x; r.v[1] = a.y; r.v[2] = a.z; r.v[3] = a.w;
    r.v[4] = b.x; r.v[5] = b.y; r.v[6] = b.z; r.v[7] = b.w;
    return r;
}
ZDEV void st_fr(uint4* lo, uint4* hi, uint32_t i, const fr_t& x) {
    lo[i] = make_uint4(x.v[0], x.v[1], x.v[2], x.v[3]);
    hi[i] = make_uint4(x.v[4], x.v[5], x.v[6], x.v[7]);
}
// AoS (reference Fr_t layout) loads/stores, used for small vectors
ZDEV fr_t ld_aos(const uint32_t* p, uint32_t i) {
    const uint4* q = reinterpret_cast<const uint4*>(p + 8 * (size_t)i);
    uint4 a = q[0], b = q[1];
    fr_t r;
    r.v[0] = a.x; r.v[1] = a.y; r.v[2] = a.z; r.v[3] = a.w;
    r.v[4] = b.x; r.v[5] = b.y; r.v[6] = b.z; r.v[7] = b.w;
    return r;
}
ZDEV void st_aos(uint32_t* p, uint32_t i, const fr_t& x) {
    uint4* q = reinterpret_cast<uint4*>(p + 8 * (size_t)i);
    q[0] = make_uint4(x.v[0], x.v[1], x.v[2], x.v[3]);
    q[1] = make_uint4(x.v[4], x.v[5], x.v[6], x.v[7]);
}

// int -> field (int_to_scalar / long_to_scalar, fr-tensor.cu:701-717)
ZDEV fr_t fr_from_i64(int64_t v) {
    fr_t r = fr_zero();
    if (v >= 0) {
        r.v[0] = (uint32_t)v;
        r.v[1] = (uint32_t)((uint64_t)v >> 32);
        return r;
    }
    uint64_t mag = (uint64_t)(-(v + 1)) + 1;
    fr_t m = fr_zero();
    m.v[0] = (uint32_t)mag;
    m.v[1] = (uint32_t)(mag >> 32);
    return fr_sub(r, m);
}

// t mod r for a 288-bit t < r 2^32 (t[8] the top limb): the quotient q = floor(t / r) <
// 2^32 estimated from the top 64 bits in double precision (2^224 / r as the constant;
// relative error of the estimate below 2^-50, the ignored low limbs below 2^-31 of a unit)
// and biased down by 1/2, so it is q or q - 1; after removing it times r one conditional
// subtraction remains.
ZDEV fr_t fr_reduce288(const uint32_t* t) {
    const double top = (double)t[8] * 4294967296.0 + (double)t[7];  // the product is exact
    const double qd = top * 0x1.1aa84a76ff6f2p-31 - 0.5;
    const uint32_t q = qd > 0.0 ? (uint32_t)qd : 0u;
    uint64_t c = 0;
    unsigned br = 0;
    fr_t x;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        c = (uint64_t)fr_p(i) * q + (c >> 32);
        x.v[i] = __builtin_subc(t[i], (uint32_t)c, br, &br);
    }
    return fr_reduce_once(x, 0);  // t - q r < 2r < 2^256: nothing is left above limb 7
}
// a m mod r for canonical a and m < 2^32 (plain in, plain out): the 288-bit product from one
// multiply-add chain, then fr_reduce288.  About 50 instructions against 332 for a Montgomery
// product.
ZDEV fr_t fr_mul_u32(const fr_t& a, uint32_t m) {
    uint32_t t[9];
    uint64_t acc = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        acc = (uint64_t)a.v[i] * m + (acc >> 32);
        t[i] = (uint32_t)acc;
    }
    t[8] = (uint32_t)(acc >> 32);
    return fr_reduce288(t);
}
// a 2^32 mod r: the limbs shifted by one, then fr_reduce288
ZDEV fr_t fr_shl32(const fr_t& a) {
    uint32_t t[9];
    t[0] = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) t[i + 1] = a.v[i];
    return fr_reduce288(t);
}
// a m mod r for a 64-bit m: the two halves (the high one shifted by 2^32), one when m < 2^32
ZDEV fr_t fr_mul_u64(const fr_t& a, uint64_t m) {
    const fr_t lo = fr_mul_u32(a, (uint32_t)m);
    const uint32_t hi = (uint32_t)(m >> 32);
    return hi ? fr_add(lo, fr_shl32(fr_mul_u32(a, hi))) : lo;
}
// a s mod r for canonical a and |s| < 2^32
ZDEV fr_t fr_mul_i64s(const fr_t& a, int64_t s) {
    const bool neg = s < 0;
    const fr_t p = fr_mul_u32(a, (uint32_t)(neg ? -s : s));
    return neg ? fr_sub(fr_zero(), p) : p;
}
// a s mod r for canonical a and any int64 s
ZDEV fr_t fr_mul_i64(const fr_t& a, int64_t s) {
    const bool neg = s < 0;
    const fr_t p = fr_mul_u64(a, neg ? 0ull - (uint64_t)s : (uint64_t)s);
    return neg ? fr_sub(fr_zero(), p) : p;
}
// x as an integer in (-2^32, 2^32) when it is one (the field element or its negative)
ZDEV bool fr_int32ish(const fr_t& x, int64_t& out) {
    uint32_t hiw = 0;
#pragma unroll
    for (int i = 1; i < 8; i++) hiw |= x.v[i];
    if (!hiw) {
        out = x.v[0];
        return true;
    }
    const fr_t d = fr_sub(fr_zero(), x);  // r - x
    hiw = 0;
#pragma unroll
    for (int i = 1; i < 8; i++) hiw |= d.v[i];
    if (!hiw) {
        out = -(int64_t)d.v[0];
        return true;
    }
    return false;
}

// ---- wave / block reductions of field elements (DPP/swizzle via shuffles, then LDS) ----
ZDEV fr_t fr_shfl_xor(const fr_t& x, int mask) {
    fr_t r;
#pragma unroll
    for (int i = 0; i < 8; i++) r.v[i] = __shfl_xor(x.v[i], mask, 64);
    return r;
}
ZDEV fr_t fr_wave_sum(fr_t x) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) x = fr_add(x, fr_shfl_xor(x, m));
    return x;
}
