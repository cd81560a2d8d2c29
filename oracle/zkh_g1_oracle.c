/*
 * zkh_g1_oracle.c -- CPU restatement of zk-hillclimb's Pedersen commitment over BLS12-381 G1.
 *
 * TEST INFRASTRUCTURE ONLY (same rules as zkh_oracle.c): the checker for the GPU
 * commitment path and the scalar CPU baseline for it; the product library never links it.
 *
 * Base field Fp: canonical residues mod p in Montgomery form with R = 2^384, the
 * reference's representation of G1 coordinates (bls12-381.cuh:220-229; G1_ONE = R mod p,
 * g1-tensor.cuh:62).  Crossing this interface an Fp element is 12 little-endian uint32
 * limbs and a G1 point is the reference's 144-byte G1Jacobian_t {x, y, z} (g1-tensor.cuh:
 * 63).  Internally the limbs are read as 6 uint64 (same bytes on a little-endian host);
 * the Montgomery product is CIOS over 64-bit words, which yields the same canonical
 * a*b*2^-384 mod p as the reference's 32-bit CIOS (bls12-381.cu:935-967): the value is
 * fixed by the arithmetic, not by the limb size.
 *
 * Every G1 routine keeps the reference's formulas and special cases, because the
 * Jacobian representative (and so the 144 bytes the transcript absorbs) depends on them:
 * doubling dbl-2009-l (bls12-381.cu:1359-1386), addition add-2007-bl with its infinity and
 * equal-point branches (bls12-381.cu:1428-1465), and the commitment schedule of
 * commit_pippenger (commitment.cu:47-103).
 */
#include <stdint.h>
#include <string.h>

#include "zkh_oracle.h"

typedef unsigned __int128 u128;
typedef struct { uint64_t v[6]; } fp;
typedef struct { fp x, y, z; } g1;

/* p (bls12-381.cuh:222) */
static const fp FP_P = {{0xb9feffffffffaaabULL, 0x1eabfffeb153ffffULL, 0x6730d2a0f6b0f624ULL,
                         0x64774b84f38512bfULL, 0x4b1ba7b6434bacd7ULL, 0x1a0111ea397fe69aULL}};
/* R mod p: Montgomery one */
static const fp FP_ONE = {{0x760900000002fffdULL, 0xebf4000bc40c0002ULL, 0x5f48985753c758baULL,
                           0x77ce585370525745ULL, 0x5c071a97a256ec6dULL, 0x15f65ec3fa80e493ULL}};
/* -p^-1 mod 2^64 */
static const uint64_t FP_PINV = 0x89f3fffcfffcfffdULL;

static int fp_is_zero(const fp* a) {
    uint64_t o = 0;
    for (int i = 0; i < 6; i++) o |= a->v[i];
    return o == 0;
}
static int fp_eq(const fp* a, const fp* b) { return memcmp(a, b, sizeof(fp)) == 0; }
static int fp_gte(const fp* a, const fp* b) {
    for (int i = 5; i >= 0; i--) {
        if (a->v[i] > b->v[i]) return 1;
        if (a->v[i] < b->v[i]) return 0;
    }
    return 1;
}
static uint64_t fp_add_raw(fp* r, const fp* a, const fp* b) {
    u128 c = 0;
    for (int i = 0; i < 6; i++) {
        c += (u128)a->v[i] + b->v[i];
        r->v[i] = (uint64_t)c;
        c >>= 64;
    }
    return (uint64_t)c;
}
static uint64_t fp_sub_raw(fp* r, const fp* a, const fp* b) {
    uint64_t br = 0;
    for (int i = 0; i < 6; i++) {
        uint64_t ai = a->v[i], d = ai - b->v[i] - br;
        br = (ai < b->v[i]) || (ai - b->v[i] < br);
        r->v[i] = d;
    }
    return br;
}
/* modular add/sub/double with one correction each (bls12-381.cu:724-736, :984-992) */
static fp fp_add(fp a, fp b) {
    fp r;
    fp_add_raw(&r, &a, &b); /* a + b < 2p < 2^383: no carry out */
    if (fp_gte(&r, &FP_P)) fp_sub_raw(&r, &r, &FP_P);
    return r;
}
static fp fp_sub(fp a, fp b) {
    fp r;
    if (fp_sub_raw(&r, &a, &b)) fp_add_raw(&r, &r, &FP_P);
    return r;
}
static fp fp_dbl(fp a) { return fp_add(a, a); }
/* Montgomery product a*b*2^-384 mod p, canonical (CIOS, 64-bit words) */
static fp fp_mul(fp a, fp b) {
    uint64_t t[8] = {0};
    for (int i = 0; i < 6; i++) {
        u128 c = 0;
        for (int j = 0; j < 6; j++) {
            c = (u128)a.v[j] * b.v[i] + t[j] + (uint64_t)(c >> 64);
            t[j] = (uint64_t)c;
        }
        u128 s = (u128)t[6] + (uint64_t)(c >> 64);
        t[6] = (uint64_t)s;
        t[7] = (uint64_t)(s >> 64);
        uint64_t m = t[0] * FP_PINV;
        c = (u128)m * FP_P.v[0] + t[0];
        for (int j = 1; j < 6; j++) {
            c = (u128)m * FP_P.v[j] + t[j] + (uint64_t)(c >> 64);
            t[j - 1] = (uint64_t)c;
        }
        s = (u128)t[6] + (uint64_t)(c >> 64);
        t[5] = (uint64_t)s;
        t[6] = t[7] + (uint64_t)(s >> 64);
    }
    fp r;
    memcpy(r.v, t, sizeof(r.v));
    if (t[6] || fp_gte(&r, &FP_P)) fp_sub_raw(&r, &r, &FP_P);
    return r;
}
static fp fp_sqr(fp a) { return fp_mul(a, a); }

static g1 g1_zero(void) {
    g1 o;
    memset(&o, 0, sizeof(o));
    o.y = FP_ONE; /* blstrs__g1__G1Affine_ZERO = {0, ONE, 0} (bls12-381.cuh:422) */
    return o;
}

/* dbl-2009-l; a point with Z = 0 is returned unchanged (bls12-381.cu:1360-1386) */
static g1 g1_dbl(g1 p) {
    if (fp_is_zero(&p.z)) return p;
    fp A = fp_sqr(p.x), B = fp_sqr(p.y), C = fp_sqr(B);
    fp D = fp_dbl(fp_sub(fp_sub(fp_sqr(fp_add(p.x, B)), A), C));
    fp E = fp_add(fp_dbl(A), A), F = fp_sqr(E);
    g1 o;
    o.z = fp_dbl(fp_mul(p.y, p.z));
    o.x = fp_sub(fp_sub(F, D), D);
    fp C8 = fp_dbl(fp_dbl(fp_dbl(C)));
    o.y = fp_sub(fp_mul(fp_sub(D, o.x), E), C8);
    return o;
}

/* add-2007-bl with the reference's branches (bls12-381.cu:1429-1465): an operand with
   Z = 0 returns the other one unchanged; U1 = U2 and S1 = S2 doubles the first operand;
   U1 = U2 with S1 != S2 falls through to the general formula, giving Z3 = 0 */
static g1 g1_add(g1 a, g1 b) {
    if (fp_is_zero(&a.z)) return b;
    if (fp_is_zero(&b.z)) return a;
    fp z1z1 = fp_sqr(a.z), z2z2 = fp_sqr(b.z);
    fp u1 = fp_mul(a.x, z2z2), u2 = fp_mul(b.x, z1z1);
    fp s1 = fp_mul(fp_mul(a.y, b.z), z2z2), s2 = fp_mul(fp_mul(b.y, a.z), z1z1);
    if (fp_eq(&u1, &u2) && fp_eq(&s1, &s2)) return g1_dbl(a);
    fp h = fp_sub(u2, u1);
    fp i = fp_sqr(fp_dbl(h));
    fp j = fp_mul(h, i);
    fp r = fp_dbl(fp_sub(s2, s1));
    fp v = fp_mul(u1, i);
    g1 o;
    o.x = fp_sub(fp_sub(fp_sub(fp_sqr(r), j), v), v);
    o.y = fp_sub(fp_mul(fp_sub(v, o.x), r), fp_dbl(fp_mul(s1, j)));
    o.z = fp_mul(fp_sub(fp_sub(fp_sqr(fp_add(a.z, b.z)), z1z1), z2z2), h);
    return o;
}

static g1 g1_load(const uint32_t* p) {
    g1 o;
    memcpy(&o, p, sizeof(o));
    return o;
}
static void g1_store(uint32_t* out, const g1* p) { memcpy(out, p, sizeof(*p)); }

/* ---- exported ---- */
void or_fp_mul(const uint32_t a[12], const uint32_t b[12], uint32_t out[12]) {
    fp x, y, r;
    memcpy(&x, a, 48);
    memcpy(&y, b, 48);
    r = fp_mul(x, y);
    memcpy(out, &r, 48);
}
void or_fp_add(const uint32_t a[12], const uint32_t b[12], uint32_t out[12]) {
    fp x, y, r;
    memcpy(&x, a, 48);
    memcpy(&y, b, 48);
    r = fp_add(x, y);
    memcpy(out, &r, 48);
}
void or_fp_sub(const uint32_t a[12], const uint32_t b[12], uint32_t out[12]) {
    fp x, y, r;
    memcpy(&x, a, 48);
    memcpy(&y, b, 48);
    r = fp_sub(x, y);
    memcpy(out, &r, 48);
}
void or_g1_dbl(const uint32_t p[36], uint32_t out[36]) {
    g1 o = g1_dbl(g1_load(p));
    g1_store(out, &o);
}
void or_g1_add(const uint32_t a[36], const uint32_t b[36], uint32_t out[36]) {
    g1 o = g1_add(g1_load(a), g1_load(b));
    g1_store(out, &o);
}
/* G1Jacobian_mul: double-and-add over the 256 raw bits of the scalar's limbs, low bit
   first (g1-tensor.cu:445-454) */
void or_g1_mul(const uint32_t a[36], const uint32_t s[8], uint32_t out[36]) {
    g1 acc = g1_zero(), p = g1_load(a);
    for (int i = 0; i < 256; i++) {
        if ((s[i / 32] >> (i % 32)) & 1u) acc = g1_add(acc, p);
        p = g1_dbl(p);
    }
    g1_store(out, &acc);
}

/* commit_pippenger (commitment.cu:47-103): out[row] = sum_i scalars[row*n+i] * gens[i] by
   4-bit windows over the scalar's raw limbs (window w = bits 4w..4w+3).  Per (row, w):
   bucket[d] accumulates gens[i] for every i (ascending) whose digit is d != 0, then the
   running sum acc += bucket[b]; run += acc for b = 15..1 gives sum_b b*bucket[b].  Per
   row: Horner from window 63 down, four doublings then one addition per window. */
int or_g1_commit(const uint32_t* gens, uint32_t n, const uint32_t* scalars, uint32_t m,
                 uint32_t* out) {
    if (n == 0) return 1;
    g1 part[64];
    for (uint32_t row = 0; row < m; row++) {
        const uint32_t* srow = scalars + (size_t)row * n * 8;
        for (uint32_t w = 0; w < 64; w++) {
            g1 bucket[16];
            for (int b = 0; b < 16; b++) bucket[b] = g1_zero();
            for (uint32_t i = 0; i < n; i++) {
                uint32_t d = (srow[(size_t)i * 8 + w / 8] >> (4 * (w % 8))) & 15u;
                if (d) bucket[d] = g1_add(bucket[d], g1_load(gens + (size_t)i * 36));
            }
            g1 acc = g1_zero(), run = g1_zero();
            for (int b = 15; b >= 1; b--) {
                acc = g1_add(acc, bucket[b]);
                run = g1_add(run, acc);
            }
            part[w] = run;
        }
        g1 acc = g1_zero();
        for (int w = 63; w >= 0; w--) {
            for (int k = 0; k < 4; k++) acc = g1_dbl(acc);
            acc = g1_add(acc, part[w]);
        }
        g1_store(out + (size_t)row * 36, &acc);
    }
    return 0;
}

/* ---- inner-product argument (ipa_prove, vrf_common.cuh:302-336) ----
 * Fr values cross as plain canonical 8-limb arrays; the Fr arithmetic is zkh_oracle.c's. */
#include <stdlib.h>

static void fr_plain_mul(const uint32_t* a, const uint32_t* b, uint32_t* out) { or_fr_mul(a, b, out); }

/* dev_msm (vrf_common.cuh:166-183): elementwise G1Jacobian_mul, then the pairwise tree
   x[i] = x[i] + x[i + half] down to one point */
static g1 msm_tree(const uint32_t* g, const uint32_t* a, uint32_t n, g1* tmp) {
    for (uint32_t i = 0; i < n; i++) {
        uint32_t p[36];
        or_g1_mul(g + (size_t)i * 36, a + (size_t)i * 8, p);
        tmp[i] = g1_load(p);
    }
    for (uint32_t sz = n; sz > 1; sz /= 2)
        for (uint32_t i = 0; i < sz / 2; i++) tmp[i] = g1_add(tmp[i], tmp[i + sz / 2]);
    return tmp[0];
}
/* dev_ip (vrf_common.cuh:185-203): sum of plain products */
static void inner(const uint32_t* a, const uint32_t* b, uint32_t n, uint32_t out[8]) {
    uint32_t acc[8] = {0}, t[8];
    for (uint32_t i = 0; i < n; i++) {
        fr_plain_mul(a + (size_t)i * 8, b + (size_t)i * 8, t);
        or_fr_add(acc, t, acc);
    }
    memcpy(out, acc, 32);
}

int or_ipa_prove(uint8_t st[32], const uint32_t* a_in, const uint32_t* b_in, const uint32_t* g_in,
                 const uint32_t Q[36], uint32_t n, uint32_t* L_out, uint32_t* R_out, uint32_t a_final[8]) {
    if (!n || (n & (n - 1))) return 1;
    uint32_t* a = malloc((size_t)n * 32);
    uint32_t* b = malloc((size_t)n * 32);
    uint32_t* g = malloc((size_t)n * 144);
    g1* tmp = malloc((size_t)n * sizeof(g1));
    memcpy(a, a_in, (size_t)n * 32);
    memcpy(b, b_in, (size_t)n * 32);
    memcpy(g, g_in, (size_t)n * 144);
    uint32_t r = 0;
    for (uint32_t sz = n; sz > 1; sz /= 2, r++) {
        const uint32_t h = sz / 2;
        uint32_t ip[8], qp[36], Lp[36], Rp[36];
        g1 m = msm_tree(g + (size_t)h * 36, a, h, tmp);
        inner(a, b + (size_t)h * 8, h, ip);
        or_g1_mul(Q, ip, qp);
        g1 t = g1_add(m, g1_load(qp));
        g1_store(Lp, &t);
        m = msm_tree(g, a + (size_t)h * 8, h, tmp);
        inner(a + (size_t)h * 8, b, h, ip);
        or_g1_mul(Q, ip, qp);
        t = g1_add(m, g1_load(qp));
        g1_store(Rp, &t);
        or_tr_absorb(st, "L", 1, Lp, 144);
        or_tr_absorb(st, "R", 1, Rp, 144);
        uint32_t x[8], xi[8];
        or_tr_challenge_fr(st, x);
        or_fr_inv(x, xi);
        /* k_fr_fold2 (vrf_common.cuh:63-69): a' = x a_lo + xi a_hi, b' = xi b_lo + x b_hi;
           k_g1_fold2 (:71-76): g' = xi g_lo + x g_hi, added in that order */
        for (uint32_t i = 0; i < h; i++) {
            uint32_t u[8], v[8];
            fr_plain_mul(x, a + (size_t)i * 8, u);
            fr_plain_mul(xi, a + (size_t)(i + h) * 8, v);
            or_fr_add(u, v, a + (size_t)i * 8);
            fr_plain_mul(xi, b + (size_t)i * 8, u);
            fr_plain_mul(x, b + (size_t)(i + h) * 8, v);
            or_fr_add(u, v, b + (size_t)i * 8);
            uint32_t p1[36], p2[36];
            or_g1_mul(g + (size_t)i * 36, xi, p1);
            or_g1_mul(g + (size_t)(i + h) * 36, x, p2);
            g1 s = g1_add(g1_load(p1), g1_load(p2));
            g1_store(g + (size_t)i * 36, &s);
        }
        memcpy(L_out + (size_t)r * 36, Lp, 144);
        memcpy(R_out + (size_t)r * 36, Rp, 144);
    }
    memcpy(a_final, a, 32);
    free(a);
    free(b);
    free(g);
    free(tmp);
    return 0;
}
