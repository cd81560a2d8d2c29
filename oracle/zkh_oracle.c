/*
 * zkh_oracle.c -- CPU restatement of zk-hillclimb's Fr sumcheck / fold / logUp path.
 *
 * TEST INFRASTRUCTURE ONLY (checker and scalar CPU baseline); the product library
 * never links or calls it.  Written from the published methods and from the
 * reference's source text; each function cites the reference lines it follows.
 *
 * Field: BLS12-381 scalar field r = 0x73eda753...00000001 (bls12-381.cu:3-6).
 * Montgomery multiplication by CIOS (Koc, Acar, Kaliski 1996) on 4x64-bit limbs with
 * unsigned __int128; R = 2^256 as in the reference's 8x32-bit limbs, so the raw
 * Montgomery product a*b*2^-256 is the same value.
 *
 * Loops over table entries run under OpenMP (or_set_threads; 1 thread gives the scalar
 * baseline).  Every parallel loop either writes disjoint entries or adds field elements,
 * and addition mod r is exact, so results do not depend on the thread count.
 */
#include "zkh_oracle.h"

#include <omp.h>
#include <stdlib.h>
#include <string.h>

/* loops shorter than this stay on one thread */
#define PAR_MIN 8192

typedef unsigned __int128 u128;
typedef struct { uint64_t v[4]; } fr;

static const fr P = {{0xffffffff00000001ULL, 0x53bda402fffe5bfeULL,
                      0x3339d80809a1d805ULL, 0x73eda753299d7d48ULL}};
static const fr R2 = {{0xc999e990f3f29c6dULL, 0x2b6cedcb87925c23ULL,
                       0x05d314967254398fULL, 0x0748d9d99f59ff11ULL}};
/* -r^-1 mod 2^64 */
static const uint64_t INV64 = 0xfffffffeffffffffULL;
static const fr ZERO = {{0, 0, 0, 0}};
static const fr ONE = {{1, 0, 0, 0}};
/* (r+1)/2, the reference's TWO_INV / F_INV2 (tlookup.cu:180, vrf_common.cuh:30-31) */
static const fr INV2 = {{0x7fffffff80000001ULL, 0xa9ded2017fff2dffULL,
                         0x199cec0404d0ec02ULL, 0x39f6d3a994cebea4ULL}};

static fr ld(const uint32_t* p) {
    fr x;
    for (int i = 0; i < 4; i++) x.v[i] = (uint64_t)p[2 * i] | ((uint64_t)p[2 * i + 1] << 32);
    return x;
}
static void st(uint32_t* p, fr x) {
    for (int i = 0; i < 4; i++) {
        p[2 * i] = (uint32_t)x.v[i];
        p[2 * i + 1] = (uint32_t)(x.v[i] >> 32);
    }
}
static int geq(fr a, fr b) {
    for (int i = 3; i >= 0; i--) {
        if (a.v[i] > b.v[i]) return 1;
        if (a.v[i] < b.v[i]) return 0;
    }
    return 1;
}
static int feq(fr a, fr b) {
    return a.v[0] == b.v[0] && a.v[1] == b.v[1] && a.v[2] == b.v[2] && a.v[3] == b.v[3];
}
static fr raw_sub(fr a, fr b) {
    fr r;
    uint64_t br = 0;
    for (int i = 0; i < 4; i++) {
        u128 d = (u128)a.v[i] - b.v[i] - br;
        r.v[i] = (uint64_t)d;
        br = (uint64_t)(d >> 64) & 1;
    }
    return r;
}
static fr raw_add(fr a, fr b) {
    fr r;
    uint64_t c = 0;
    for (int i = 0; i < 4; i++) {
        u128 s = (u128)a.v[i] + b.v[i] + c;
        r.v[i] = (uint64_t)s;
        c = (uint64_t)(s >> 64);
    }
    return r;
}
/* bls12-381.cu:289-300: one conditional correction (inputs canonical) */
static fr add(fr a, fr b) {
    fr s = raw_add(a, b);
    if (geq(s, P)) s = raw_sub(s, P);
    return s;
}
static fr sub(fr a, fr b) {
    fr d = raw_sub(a, b);
    if (!geq(a, b)) d = raw_add(d, P);
    return d;
}
/* CIOS Montgomery product a*b*2^-256 mod r (same value as bls12-381.cu:499-531) */
static fr mmul(fr a, fr b) {
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
        uint64_t m = t[0] * INV64;
        c = (u128)m * P.v[0] + t[0];
        for (int j = 1; j < 4; j++) {
            c = (u128)m * P.v[j] + t[j] + (uint64_t)(c >> 64);
            t[j - 1] = (uint64_t)c;
        }
        c = (u128)t[4] + (uint64_t)(c >> 64);
        t[3] = (uint64_t)c;
        t[4] = t[5] + (uint64_t)(c >> 64);
    }
    fr r = {{t[0], t[1], t[2], t[3]}};
    if (t[4] || geq(r, P)) r = raw_sub(r, P);
    return r;
}
static fr mont(fr a) { return mmul(a, R2); }
/* plain product (the reference's mont(mul(a,b)) / host operator*) */
static fr mul(fr a, fr b) { return mont(mmul(a, b)); }
/* Fermat inverse x^(r-2) of a plain value (polynomial.cu:127-131); 0 -> 0 */
static fr inv(fr a) {
    fr am = mont(a);
    fr e = raw_sub(P, (fr){{2, 0, 0, 0}});
    fr res = mont(ONE);
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 64; j++) {
            if ((e.v[i] >> j) & 1) res = mmul(res, am);
            am = mmul(am, am);
        }
    return mmul(res, ONE); /* unmont */
}
static fr from_i64(int64_t v) {
    if (v >= 0) return (fr){{(uint64_t)v, 0, 0, 0}};
    uint64_t mag = (uint64_t)(-(v + 1)) + 1;
    return sub(ZERO, (fr){{mag, 0, 0, 0}});
}
static fr from_u32(uint32_t v) { return (fr){{v, 0, 0, 0}}; }
/* eq(u,v) = 2uv - (u+v) + 1 (polynomial.cu:355-372) */
static fr eq2(fr u, fr v) {
    fr uv = mul(u, v);
    return add(sub(add(uv, uv), add(u, v)), ONE);
}

void or_fr_add(const uint32_t a[8], const uint32_t b[8], uint32_t out[8]) { st(out, add(ld(a), ld(b))); }
void or_fr_sub(const uint32_t a[8], const uint32_t b[8], uint32_t out[8]) { st(out, sub(ld(a), ld(b))); }
void or_fr_montmul(const uint32_t a[8], const uint32_t b[8], uint32_t out[8]) { st(out, mmul(ld(a), ld(b))); }
void or_fr_mul(const uint32_t a[8], const uint32_t b[8], uint32_t out[8]) { st(out, mul(ld(a), ld(b))); }
void or_fr_inv(const uint32_t a[8], uint32_t out[8]) { st(out, inv(ld(a))); }
void or_fr_from_i64(int64_t v, uint32_t out[8]) { st(out, from_i64(v)); }

/* ------------------------------------------------------------------------------ */
/* SHA-256 (FIPS 180-4), framing of fs_transcript.hpp:115-166                      */
/* ------------------------------------------------------------------------------ */
typedef struct {
    uint32_t h[8];
    uint64_t len;
    uint8_t buf[64];
    size_t blen;
} sha_ctx;

static const uint32_t SHA_K[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};

static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

static void sha_compress(uint32_t h[8], const uint8_t* p) {
    uint32_t w[64];
    for (int i = 0; i < 16; i++)
        w[i] = ((uint32_t)p[4 * i] << 24) | ((uint32_t)p[4 * i + 1] << 16) |
               ((uint32_t)p[4 * i + 2] << 8) | (uint32_t)p[4 * i + 3];
    for (int i = 16; i < 64; i++) {
        uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
        uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
        w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for (int i = 0; i < 64; i++) {
        uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) +
                      SHA_K[i] + w[i];
        uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
        hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
}
static void sha_init(sha_ctx* c) {
    static const uint32_t iv[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                   0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    memcpy(c->h, iv, sizeof(iv));
    c->len = 0;
    c->blen = 0;
}
static void sha_update(sha_ctx* c, const void* data, size_t n) {
    const uint8_t* p = (const uint8_t*)data;
    c->len += n;
    while (n) {
        size_t take = 64 - c->blen;
        if (take > n) take = n;
        memcpy(c->buf + c->blen, p, take);
        c->blen += take; p += take; n -= take;
        if (c->blen == 64) { sha_compress(c->h, c->buf); c->blen = 0; }
    }
}
static void sha_final(sha_ctx* c, uint8_t out[32]) {
    uint64_t bits = c->len * 8;
    uint8_t pad = 0x80, z = 0;
    sha_update(c, &pad, 1);
    while (c->blen != 56) sha_update(c, &z, 1);
    uint8_t lb[8];
    for (int i = 0; i < 8; i++) lb[i] = (uint8_t)(bits >> (56 - 8 * i));
    sha_update(c, lb, 8);
    for (int i = 0; i < 8; i++) {
        out[4 * i] = (uint8_t)(c->h[i] >> 24);
        out[4 * i + 1] = (uint8_t)(c->h[i] >> 16);
        out[4 * i + 2] = (uint8_t)(c->h[i] >> 8);
        out[4 * i + 3] = (uint8_t)c->h[i];
    }
}
void or_sha256(const uint8_t* data, size_t n, uint8_t out[32]) {
    sha_ctx c;
    sha_init(&c);
    sha_update(&c, data, n);
    sha_final(&c, out);
}
void or_tr_init(uint8_t s[32], const char* seed, size_t seed_len) {
    or_sha256((const uint8_t*)seed, seed_len, s);
}
/* state = SHA256(state || len32(label) || label || len64(data) || data), little-endian
 * lengths (fs_transcript.hpp:121-134) */
void or_tr_absorb(uint8_t s[32], const char* label, size_t label_len, const void* data,
                  size_t len) {
    sha_ctx c;
    sha_init(&c);
    sha_update(&c, s, 32);
    uint8_t ll[4], dl[8];
    for (int i = 0; i < 4; i++) ll[i] = (uint8_t)((uint32_t)label_len >> (8 * i));
    for (int i = 0; i < 8; i++) dl[i] = (uint8_t)((uint64_t)len >> (8 * i));
    sha_update(&c, ll, 4);
    sha_update(&c, label, label_len);
    sha_update(&c, dl, 8);
    sha_update(&c, data, len);
    sha_final(&c, s);
}
/* out = SHA256(state||"chal"); state = SHA256(state||"rtch") (fs_transcript.hpp:149-165) */
void or_tr_challenge_bytes(uint8_t s[32], uint8_t out[32]) {
    sha_ctx c;
    sha_init(&c);
    sha_update(&c, s, 32);
    sha_update(&c, "chal", 4);
    sha_final(&c, out);
    uint8_t tmp[32];
    sha_init(&c);
    sha_update(&c, s, 32);
    sha_update(&c, "rtch", 4);
    sha_final(&c, tmp);
    memcpy(s, tmp, 32);
}
/* 8 LE u32 limbs, top limb %= 1944954707, redraw on zero (vrf_common.cuh:235-245) */
void or_tr_challenge_fr(uint8_t s[32], uint32_t out[8]) {
    for (;;) {
        uint8_t b[32];
        or_tr_challenge_bytes(s, b);
        for (int i = 0; i < 8; i++)
            out[i] = (uint32_t)b[4 * i] | ((uint32_t)b[4 * i + 1] << 8) |
                     ((uint32_t)b[4 * i + 2] << 16) | ((uint32_t)b[4 * i + 3] << 24);
        out[7] %= 1944954707u;
        for (int i = 0; i < 8; i++)
            if (out[i]) return;
    }
}
static fr challenge(uint8_t s[32]) {
    uint32_t x[8];
    or_tr_challenge_fr(s, x);
    return ld(x);
}
static void absorb_fr(uint8_t s[32], const char* label, fr x) {
    uint32_t b[8];
    st(b, x);
    or_tr_absorb(s, label, strlen(label), b, 32);
}

/* ------------------------------------------------------------------------------ */
/* tensors                                                                          */
/* ------------------------------------------------------------------------------ */
static uint32_t ceil_log2(uint32_t n) { /* fr-tensor.cu:26-41 */
    if (n == 0) return 0;
    n--;
    uint32_t r = 0;
    while (n) { n >>= 1; r++; }
    return r;
}
static fr* falloc(size_t n) { return (fr*)calloc(n ? n : 1, sizeof(fr)); }
static fr* from_aos(const uint32_t* t, size_t n) {
    fr* o = falloc(n);
#pragma omp parallel for if (n >= PAR_MIN)
    for (size_t i = 0; i < n; i++) o[i] = ld(t + 8 * i);
    return o;
}

void or_set_threads(int n) { omp_set_num_threads(n < 1 ? 1 : n); }
int or_get_threads(void) { return omp_get_max_threads(); }

static fr sum_fr(const fr* t, size_t n) {
    fr total = ZERO;
#pragma omp parallel if (n >= PAR_MIN)
    {
        fr s = ZERO;
#pragma omp for nowait
        for (size_t i = 0; i < n; i++) s = add(s, t[i]);
#pragma omp critical
        total = add(total, s);
    }
    return total;
}
void or_sum(const uint32_t* t, uint32_t n, uint32_t out[8]) {
    fr* a = from_aos(t, n);
    st(out, sum_fr(a, n));
    free(a);
}
/* int64 values -> Fr array (int_to_scalar / long_to_scalar per entry, fr-tensor.cu:701-717) */
void or_ints_to_fr(const int64_t* v, size_t n, uint32_t* out) {
#pragma omp parallel for if (n >= PAR_MIN)
    for (size_t i = 0; i < n; i++) st(out + 8 * i, from_i64(v[i]));
}

/* Fr_me: pairs (2i, 2i+1), u[0] binds the LSB; odd tail a0 - x*a0 (fr-tensor.cu:588-609) */
static fr me_fr(const fr* t, uint32_t n, const fr* u, uint32_t k) {
    fr* cur = falloc(n);
    memcpy(cur, t, n * sizeof(fr));
    uint32_t sz = n;
    for (uint32_t r = 0; r < k; r++) {
        uint32_t out = (sz + 1) / 2;
        const fr x = mont(u[r]);
        fr* nxt = falloc(out);
#pragma omp parallel for if (out >= PAR_MIN)
        for (uint32_t i = 0; i < out; i++) {
            uint32_t g0 = 2 * i, g1 = 2 * i + 1;
            if (g1 < sz) nxt[i] = add(cur[g0], mmul(x, sub(cur[g1], cur[g0])));
            else nxt[i] = sub(cur[g0], mmul(x, cur[g0]));
        }
        free(cur);
        cur = nxt;
        sz = out;
    }
    fr res = cur[0];
    free(cur);
    return res;
}
int or_me(const uint32_t* t, uint32_t n, const uint32_t* u, uint32_t k, uint32_t out[8]) {
    /* FrTensor::operator()(u) size check (fr-tensor.cu:437-442) */
    if (k >= 32 || n <= ((1u << k) / 2) || n > (1u << k)) return 1;
    fr* a = from_aos(t, n);
    fr* uu = from_aos(u, k);
    st(out, me_fr(a, n, uu, k));
    free(a);
    free(uu);
    return 0;
}

/* Fr_multi_dim_partial_me_step recursion (fr-tensor.cu:518-552); returns new buffer */
static fr* partial_me_fr(const fr* t, uint32_t n, const fr* u, uint32_t k, uint32_t cur_dim,
                         uint32_t window, uint32_t* out_n) {
    fr* cur = falloc(n);
    memcpy(cur, t, n * sizeof(fr));
    uint32_t sz = n, cd = cur_dim;
    for (uint32_t r = 0; r < k; r++) {
        uint32_t cdo = (cd + 1) / 2;
        uint32_t other = sz / (cd * window);
        uint32_t osz = other * cdo * window;
        fr* nxt = falloc(osz);
        fr x = mont(u[r]);
#pragma omp parallel for if (osz >= PAR_MIN)
        for (uint32_t g = 0; g < osz; g++) {
            uint32_t i0 = g / (cdo * window), i1 = (g / window) % cdo, i2 = g % window;
            uint32_t g0 = i0 * cd * window + (2 * i1) * window + i2;
            if (2 * i1 + 1 < cd) {
                uint32_t g1 = i0 * cd * window + (2 * i1 + 1) * window + i2;
                nxt[g] = add(cur[g0], mmul(x, sub(cur[g1], cur[g0])));
            } else {
                nxt[g] = sub(cur[g0], mmul(x, cur[g0]));
            }
        }
        free(cur);
        cur = nxt;
        sz = osz;
        cd = cdo;
    }
    *out_n = sz;
    return cur;
}
int or_partial_me(const uint32_t* t, uint32_t n, const uint32_t* u, uint32_t k,
                  uint32_t cur_dim, uint32_t window, uint32_t* out, uint32_t* out_n) {
    /* FrTensor::partial_me(u, cur_dim, window) checks (fr-tensor.cu:554-560) */
    if (k >= 32 || cur_dim <= ((1u << k) >> 1) || cur_dim > (1u << k)) return 1;
    if (window == 0 || n % (cur_dim * window) != 0) return 1;
    fr* a = from_aos(t, n);
    fr* uu = from_aos(u, k);
    uint32_t on;
    fr* r = partial_me_fr(a, n, uu, k, cur_dim, window, &on);
    for (uint32_t i = 0; i < on; i++) st(out + 8 * i, r[i]);
    *out_n = on;
    free(a); free(uu); free(r);
    return 0;
}
/* Fr_partial_me_step (window form, fr-tensor.cu:612-641) */
int or_partial_me_window(const uint32_t* t, uint32_t n, const uint32_t* u, uint32_t k,
                         uint32_t window, uint32_t* out, uint32_t* out_n) {
    if (k == 0 || window == 0) return 1;
    if (n <= window * (1u << (k - 1))) return 1; /* fr-tensor.cu:512-516 */
    fr* cur = from_aos(t, n);
    uint32_t sz = n;
    for (uint32_t r = 0; r < k; r++) {
        fr x = mont(ld(u + 8 * r));
        uint32_t nw = (sz + 2 * window - 1) / (2 * window);
        uint32_t osz = window * nw;
        fr* nxt = falloc(osz);
#pragma omp parallel for if (osz >= PAR_MIN)
        for (uint32_t g = 0; g < osz; g++) {
            uint32_t w = g / window, j = g % window;
            uint32_t g0 = 2 * w * window + j, g1 = (2 * w + 1) * window + j;
            if (g1 < sz) nxt[g] = add(cur[g0], mmul(x, sub(cur[g1], cur[g0])));
            else if (g0 < sz) nxt[g] = sub(cur[g0], mmul(x, cur[g0]));
            else nxt[g] = ZERO;
        }
        free(cur);
        cur = nxt;
        sz = osz;
    }
    for (uint32_t i = 0; i < sz; i++) st(out + 8 * i, cur[i]);
    *out_n = sz;
    free(cur);
    return 0;
}
/* multi_dim_me: bind the LAST dimension first (fr-tensor.cu:643-652) */
static int multi_dim_me_fr(const fr* t, uint32_t n, const fr* const* us, const uint32_t* ks,
                           const uint32_t* shape, uint32_t nd, fr* out) {
    if (nd == 0) { *out = t[0]; return 0; }
    if (nd == 1) {
        uint32_t k = ks[0];
        if (k >= 32 || n <= ((1u << k) / 2) || n > (1u << k)) return 1;
        *out = me_fr(t, n, us[0], k);
        return 0;
    }
    uint32_t k = ks[nd - 1], cd = shape[nd - 1];
    if (k >= 32 || cd <= ((1u << k) >> 1) || cd > (1u << k)) return 1;
    if (n % cd != 0) return 1;
    uint32_t on;
    fr* r = partial_me_fr(t, n, us[nd - 1], k, cd, 1, &on);
    int rc = multi_dim_me_fr(r, on, us, ks, shape, nd - 1, out);
    free(r);
    return rc;
}
int or_multi_dim_me(const uint32_t* t, uint32_t n, const uint32_t* us, const uint32_t* ks,
                    const uint32_t* shape, uint32_t ndim, uint32_t out[8]) {
    if (ndim > 16) return 1;
    fr* a = from_aos(t, n);
    fr* ptrs[16];
    size_t off = 0;
    for (uint32_t d = 0; d < ndim; d++) {
        ptrs[d] = from_aos(us + 8 * off, ks[d]);
        off += ks[d];
    }
    fr res;
    int rc = multi_dim_me_fr(a, n, (const fr* const*)ptrs, ks, shape, ndim, &res);
    if (!rc) st(out, res);
    for (uint32_t d = 0; d < ndim; d++) free(ptrs[d]);
    free(a);
    return rc;
}
/* pad: last dimension to pow2 first, then recurse with it merged (fr-tensor.cu:809-828) */
int or_pad_val(const uint32_t* t, const uint32_t* shape, uint32_t ndim, const uint32_t pad[8],
               uint32_t* out, uint32_t* out_n) {
    if (ndim == 0 || ndim > 16) return 1;
    uint64_t total = 1;
    for (uint32_t d = 0; d < ndim; d++) total *= shape[d];
    uint32_t sh[16];
    memcpy(sh, shape, ndim * sizeof(uint32_t));
    uint32_t nd = ndim;
    uint32_t* cur = (uint32_t*)malloc(total * 32 + 32);
    memcpy(cur, t, total * 32);
    uint64_t sz = total;
    for (;;) {
        uint32_t last = sh[nd - 1], lastp = 1u << ceil_log2(last);
        uint64_t osz = (sz / last) * lastp;
        uint32_t* nxt = (uint32_t*)malloc(osz * 32 + 32);
        for (uint64_t g = 0; g < osz; g++) {
            uint64_t g0 = g / lastp, g1 = g % lastp;
            if (g1 >= last) memcpy(nxt + 8 * g, pad, 32); /* FrTensor_pad_kernel pad_val */
            else memcpy(nxt + 8 * g, cur + 8 * (g0 * last + g1), 32);
        }
        free(cur);
        cur = nxt;
        sz = osz;
        if (nd == 1) break;
        nd--;
        sh[nd - 1] *= lastp;
    }
    memcpy(out, cur, sz * 32);
    *out_n = (uint32_t)sz;
    free(cur);
    return 0;
}
int or_pad(const uint32_t* t, const uint32_t* shape, uint32_t ndim, uint32_t* out,
           uint32_t* out_n) {
    static const uint32_t zero[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    return or_pad_val(t, shape, ndim, zero, out, out_n);
}
/* eq table by doubling; bit i becomes the new top bit (zkob_lookup.cuh:202-209) */
static fr* build_eq_fr(const fr* u, uint32_t k) {
    fr* e = falloc((size_t)1 << k);
    e[0] = ONE;
    uint32_t n = 1;
    for (uint32_t i = 0; i < k; i++) {
        fr om = sub(ONE, u[i]);
#pragma omp parallel for if (n >= PAR_MIN)
        for (uint32_t g = 0; g < n; g++) {
            fr v = e[g];
            e[g] = mul(om, v);
            e[g + n] = mul(u[i], v);
        }
        n <<= 1;
    }
    return e;
}
void or_build_eq(const uint32_t* u, uint32_t k, uint32_t* out) {
    fr* uu = from_aos(u, k);
    fr* e = build_eq_fr(uu, k);
    for (size_t i = 0; i < ((size_t)1 << k); i++) st(out + 8 * i, e[i]);
    free(uu);
    free(e);
}

/* ------------------------------------------------------------------------------ */
/* polynomial helpers                                                               */
/* ------------------------------------------------------------------------------ */
/* p(x) from p0,p1,p2 (vrf_common.cuh:130-140) */
static fr lagrange3(fr p0, fr p1, fr p2, fr u) {
    fr two = from_u32(2);
    fr um1 = sub(u, ONE), um2 = sub(u, two);
    fr l0 = mul(mul(um1, um2), INV2);
    fr l1 = mul(u, sub(two, u));
    fr l2 = mul(mul(u, um1), INV2);
    return add(add(mul(p0, l0), mul(p1, l1)), mul(p2, l2));
}
/* p(v) from p(0..3) (zkob_lookup.cuh:62-73) */
static fr lagrange4(const fr p[4], fr v) {
    fr inv6 = inv(from_u32(6));
    fr vm1 = sub(v, ONE), vm2 = sub(v, from_u32(2)), vm3 = sub(v, from_u32(3));
    fr l0 = sub(ZERO, mul(mul(mul(vm1, vm2), vm3), inv6));
    fr l1 = mul(mul(mul(v, vm2), vm3), INV2);
    fr l2 = sub(ZERO, mul(mul(mul(v, vm1), vm3), INV2));
    fr l3 = mul(mul(mul(v, vm1), vm2), inv6);
    fr acc = mul(p[0], l0);
    acc = add(acc, mul(p[1], l1));
    acc = add(acc, mul(p[2], l2));
    return add(acc, mul(p[3], l3));
}
void or_lagrange3(const uint32_t p[24], const uint32_t x[8], uint32_t out[8]) {
    st(out, lagrange3(ld(p), ld(p + 8), ld(p + 16), ld(x)));
}
void or_lagrange4(const uint32_t p[32], const uint32_t x[8], uint32_t out[8]) {
    fr q[4] = {ld(p), ld(p + 8), ld(p + 16), ld(p + 24)};
    st(out, lagrange4(q, ld(x)));
}
/* coefficient-form evaluation (polynomial.cu:296-305) */
static fr poly_eval(const fr* c, int deg, fr x) {
    fr acc = ZERO, pw = ONE;
    for (int i = 0; i <= deg; i++) {
        acc = add(acc, mul(c[i], pw));
        pw = mul(pw, x);
    }
    return acc;
}

/* ------------------------------------------------------------------------------ */
/* matmul sumcheck: zkob_fc.cu:259-440 with zkfc.cu:94-127 kernels                  */
/* ------------------------------------------------------------------------------ */
/* the segment over field tables X (B x IN), W (IN x OUT), Y (B x OUT): the FrTensors that
 * zkob_fc binds (zkob_fc.cu:276-277, :337-338) */
static int mm_prove_core(uint8_t s[32], const fr* Xf, const fr* Wf, const fr* Yf,
                         uint32_t B, uint32_t IN, uint32_t OUT, uint32_t* ev_out,
                         uint32_t* claims_out, uint32_t* u_batch_out, uint32_t* u_output_out,
                         uint32_t* u_input_out) {
    uint32_t lb = ceil_log2(B), lo = ceil_log2(OUT), L = ceil_log2(IN);
    fr* ub = falloc(lb);
    fr* uo = falloc(lo);
    for (uint32_t i = 0; i < lb; i++) ub[i] = challenge(s);
    for (uint32_t i = 0; i < lo; i++) uo[i] = challenge(s);
    int rc = 0;
    fr claim;
    {
        const fr* us[2] = {ub, uo};
        uint32_t ks[2] = {lb, lo}, sh[2] = {B, OUT};
        if (multi_dim_me_fr(Yf, B * OUT, us, ks, sh, 2, &claim)) { rc = 1; goto done0; }
    }
    absorb_fr(s, "claim", claim);
    uint32_t nx, nw;
    fr* a = partial_me_fr(Xf, B * IN, ub, lb, B, IN, &nx);   /* size IN */
    fr* b = partial_me_fr(Wf, IN * OUT, uo, lo, OUT, 1, &nw); /* size IN */
    fr* xs = falloc(L);
    fr cur = claim;
    uint32_t sz = IN;
    for (uint32_t r = 0; r < L; r++) {
        uint32_t no = (1u << ceil_log2(sz)) >> 1;
        fr c0 = ZERO, c1 = ZERO, c2 = ZERO;
#pragma omp parallel if (no >= PAR_MIN)
        {
            fr l0 = ZERO, l1 = ZERO, l2 = ZERO;
#pragma omp for nowait
            for (uint32_t i = 0; i < no; i++) { /* zkip_poly_kernel, zero-fill */
                fr a0 = i < sz ? a[i] : ZERO, b0 = i < sz ? b[i] : ZERO;
                fr a1 = i + no < sz ? a[i + no] : ZERO, b1 = i + no < sz ? b[i + no] : ZERO;
                l0 = add(l0, mul(a0, b0));
                l1 = add(l1, mont(add(mmul(a0, sub(b1, b0)), mmul(b0, sub(a1, a0)))));
                l2 = add(l2, mul(sub(a1, a0), sub(b1, b0)));
            }
#pragma omp critical
            {
                c0 = add(c0, l0);
                c1 = add(c1, l1);
                c2 = add(c2, l2);
            }
        }
        fr p0 = c0, p1 = add(add(c0, c1), c2);
        fr two = from_u32(2);
        fr p2 = add(add(c0, mul(two, c1)), mul(mul(two, two), c2));
        if (!feq(cur, add(p0, p1))) { rc = 2; }
        absorb_fr(s, "p0", p0);
        absorb_fr(s, "p1", p1);
        absorb_fr(s, "p2", p2);
        fr x = challenge(s);
        xs[r] = x;
        st(ev_out + 24 * r, p0);
        st(ev_out + 24 * r + 8, p1);
        st(ev_out + 24 * r + 16, p2);
        cur = lagrange3(p0, p1, p2, x);
        fr xm = mont(x);
#pragma omp parallel for if (no >= PAR_MIN)
        for (uint32_t i = 0; i < no; i++) { /* zkip_reduce_kernel */
            fr a0 = i < sz ? a[i] : ZERO, b0 = i < sz ? b[i] : ZERO;
            fr a1 = i + no < sz ? a[i + no] : ZERO, b1 = i + no < sz ? b[i + no] : ZERO;
            a[i] = add(a0, mmul(xm, sub(a1, a0)));
            b[i] = add(b0, mmul(xm, sub(b1, b0)));
        }
        sz = no;
        if (rc) break;
    }
    if (!rc) {
        fr* ui = falloc(L);
        for (uint32_t i = 0; i < L; i++) ui[i] = xs[L - 1 - i];
        fr cx, cw;
        const fr* usx[2] = {ub, ui};
        uint32_t ksx[2] = {lb, L}, shx[2] = {B, IN};
        const fr* usw[2] = {ui, uo};
        uint32_t ksw[2] = {L, lo}, shw[2] = {IN, OUT};
        if (multi_dim_me_fr(Xf, B * IN, usx, ksx, shx, 2, &cx) ||
            multi_dim_me_fr(Wf, IN * OUT, usw, ksw, shw, 2, &cw)) {
            rc = 1;
        } else {
            /* zkob_fc.cu:344-347 */
            if (!feq(a[0], cx) || !feq(b[0], cw) || !feq(cur, mul(cx, cw))) rc = 2;
            absorb_fr(s, "claim_X", cx);
            absorb_fr(s, "claim_W", cw);
            st(claims_out, claim);
            st(claims_out + 8, cx);
            st(claims_out + 16, cw);
            for (uint32_t i = 0; i < L; i++) st(u_input_out + 8 * i, ui[i]);
        }
        free(ui);
    }
    for (uint32_t i = 0; i < lb; i++) st(u_batch_out + 8 * i, ub[i]);
    for (uint32_t i = 0; i < lo; i++) st(u_output_out + 8 * i, uo[i]);
    free(a); free(b); free(xs);
done0:
    free(ub); free(uo);
    return rc;
}
/* zkob_fc's segment on its int32 input files (load_int_tensor, zkob_fc.cu:178-185) and
 * the int64 product */
int or_mm_prove(uint8_t s[32], const int32_t* X, const int32_t* W, const int64_t* Y,
                uint32_t B, uint32_t IN, uint32_t OUT, uint32_t* ev_out,
                uint32_t* claims_out, uint32_t* u_batch_out, uint32_t* u_output_out,
                uint32_t* u_input_out) {
    if (!B || !IN || !OUT) return 1;
    fr* Xf = falloc((size_t)B * IN);
    fr* Wf = falloc((size_t)IN * OUT);
    fr* Yf = falloc((size_t)B * OUT);
#pragma omp parallel for
    for (size_t i = 0; i < (size_t)B * IN; i++) Xf[i] = from_i64(X[i]);
#pragma omp parallel for
    for (size_t i = 0; i < (size_t)IN * OUT; i++) Wf[i] = from_i64(W[i]);
#pragma omp parallel for
    for (size_t i = 0; i < (size_t)B * OUT; i++) Yf[i] = from_i64(Y[i]);
    int rc = mm_prove_core(s, Xf, Wf, Yf, B, IN, OUT, ev_out, claims_out, u_batch_out, u_output_out,
                           u_input_out);
    free(Xf); free(Wf); free(Yf);
    return rc;
}
/* the same on field-element tables (Fr arrays, canonical) */
int or_mm_prove_fr(uint8_t s[32], const uint32_t* X, const uint32_t* W, const uint32_t* Y,
                   uint32_t B, uint32_t IN, uint32_t OUT, uint32_t* ev_out,
                   uint32_t* claims_out, uint32_t* u_batch_out, uint32_t* u_output_out,
                   uint32_t* u_input_out) {
    if (!B || !IN || !OUT) return 1;
    fr* Xf = from_aos(X, (size_t)B * IN);
    fr* Wf = from_aos(W, (size_t)IN * OUT);
    fr* Yf = from_aos(Y, (size_t)B * OUT);
    int rc = mm_prove_core(s, Xf, Wf, Yf, B, IN, OUT, ev_out, claims_out, u_batch_out, u_output_out,
                           u_input_out);
    free(Xf); free(Wf); free(Yf);
    return rc;
}

/* ------------------------------------------------------------------------------ */
/* logUp (tlookup.cu, zkob_lookup.cuh fs_phase1/fs_phase2)                          */
/* ------------------------------------------------------------------------------ */
void or_range_table(int32_t low, uint32_t len, uint32_t table_size, uint32_t* T) {
    /* tlookuprange_init_kernel (tlookup.cu:372-380) adds in C++ int: a 32-bit add on the
       device, so entries past 2^31 - 1 wrap to negative values */
    for (uint32_t i = 0; i < table_size; i++) {
        int32_t v = (int32_t)((uint32_t)low + (i < len ? i : len - 1));
        st(T + 8 * i, from_i64(v));
    }
}
int or_lu_prep(const uint32_t* S, uint32_t D, int32_t low, uint32_t N, uint32_t* m) {
    uint32_t* cnt = (uint32_t*)calloc(N ? N : 1, sizeof(uint32_t));
    fr lowf = from_i64(low);
    int rc = 0;
    for (uint32_t i = 0; i < D; i++) {
        fr d = sub(ld(S + 8 * i), lowf);
        uint32_t idx = (uint32_t)d.v[0]; /* limb 0 only (tlookup.cu:419) */
        if (idx >= N) { rc = 1; continue; }
        cnt[idx]++;
    }
    for (uint32_t j = 0; j < N; j++) st(m + 8 * j, from_u32(cnt[j]));
    free(cnt);
    return rc;
}
static void inv_table(const fr* in, uint32_t n, fr beta, fr* out) {
#pragma omp parallel for if (n >= 256)
    for (uint32_t i = 0; i < n; i++) out[i] = inv(add(in[i], beta));
}
void or_lu_inverse(const uint32_t* S, uint32_t n, const uint32_t beta[8], uint32_t* A) {
    fr b = ld(beta);
#pragma omp parallel for if (n >= 256)
    for (uint32_t i = 0; i < n; i++) st(A + 8 * i, inv(add(ld(S + 8 * i), b)));
}

/* out = a + c*b (FrTensor operator+ with a scalar multiple, e.g. comb = G + r*S,
 * zkob_glu.cu:155-156) and out = a (.) b (FrTensor operator*, fr-tensor.cu elementwise) */
void or_axpy(const uint32_t* a, const uint32_t c[8], const uint32_t* b, size_t n, uint32_t* out) {
    const fr cm = mont(ld(c));
#pragma omp parallel for if (n >= PAR_MIN)
    for (size_t i = 0; i < n; i++) st(out + 8 * i, add(ld(a + 8 * i), mmul(cm, ld(b + 8 * i))));
}
void or_hadamard(const uint32_t* a, const uint32_t* b, size_t n, uint32_t* out) {
#pragma omp parallel for if (n >= PAR_MIN)
    for (size_t i = 0; i < n; i++) st(out + 8 * i, mul(ld(a + 8 * i), ld(b + 8 * i)));
}
/* entries violating A[i] (S[i] + beta) = 1, with A[i] = 0 required where S[i] + beta = 0
 * (the Fermat convention of tlookup.cu:50-62): the identity that fixes 1/(S + beta) */
size_t or_check_inverse(const uint32_t* S, const uint32_t* A, size_t n, const uint32_t beta[8]) {
    const fr b = ld(beta);
    size_t bad = 0;
#pragma omp parallel for reduction(+ : bad) if (n >= PAR_MIN)
    for (size_t i = 0; i < n; i++) {
        const fr d = add(ld(S + 8 * i), b), a = ld(A + 8 * i);
        const int ok = feq(d, ZERO) ? feq(a, ZERO) : feq(mul(a, d), ONE);
        bad += !ok;
    }
    return bad;
}

/* Polynomial::eq(u) * {q0,q1,q2} -> degree-3 coefficients */
static void eq_times(fr u, const fr q[3], fr out[4]) {
    fr e0 = sub(ONE, u), e1 = sub(add(u, u), ONE);
    out[0] = mul(e0, q[0]);
    out[1] = add(mul(e0, q[1]), mul(e1, q[0]));
    out[2] = add(mul(e0, q[2]), mul(e1, q[1]));
    out[3] = mul(e1, q[2]);
}

int or_lu_prove(uint8_t s[32], const uint32_t* Ain, const uint32_t* Sin, const uint32_t* Tin,
                const uint32_t* min, uint32_t D, uint32_t N, const uint32_t alpha_in[8],
                const uint32_t beta_in[8], const uint32_t* u_in, int strict,
                uint32_t* ev_out, uint32_t* term_out, uint32_t* ws_out) {
    /* tLookup::prove shape rules (tlookup.cu:330-336) */
    if (!D || !N || (D & (D - 1)) || (N & (N - 1)) || D % N) return 1;
    uint32_t logD = ceil_log2(D);
    fr* A = from_aos(Ain, D);
    fr* S = from_aos(Sin, D);
    fr* T = from_aos(Tin, N);
    fr* m = from_aos(min, N);
    fr* Bv = falloc(N);
    fr alpha = ld(alpha_in), beta = ld(beta_in);
    fr* u = from_aos(u_in, logD);
    inv_table(T, N, beta, Bv); /* zkob_rescale.cu:132-135 */
    fr alpha_sq = mul(alpha, alpha);
    fr* bm = falloc(N);
#pragma omp parallel for if (N >= PAR_MIN)
    for (uint32_t i = 0; i < N; i++) bm[i] = mul(Bv[i], m[i]);
    fr Cc = sub(alpha_sq, sum_fr(bm, N));
    free(bm);
    fr claim = add(alpha, alpha_sq);
    fr inv_ratio = mul(from_u32(N), inv(from_u32(D)));
    int rc = 0;
    uint32_t ulen = logD, sz = D, r = 0;
    fr* t0 = falloc(D / 2 + 1);
    fr* t1 = falloc(D / 2 + 1);
    fr* t2 = falloc(D / 2 + 1);
    /* phase 1 (zkob_lookup.cuh:172-198, tlookup.cu:74-104, :184-200) */
    while (sz != N) {
        uint32_t h = sz >> 1;
        fr sA0 = ZERO, sA1 = ZERO;
        const fr am = mont(alpha);
#pragma omp parallel if (h >= PAR_MIN)
        {
            fr l0 = ZERO, l1 = ZERO;
#pragma omp for nowait
            for (uint32_t i = 0; i < h; i++) {
                fr c00 = A[i], c01 = sub(A[i + h], A[i]);
                fr c10 = add(S[i], beta), c11 = sub(S[i + h], S[i]);
                t0[i] = mmul(am, mul(c00, c10));
                t1[i] = mmul(am, mont(add(mmul(c01, c10), mmul(c00, c11))));
                t2[i] = mmul(am, mul(c01, c11));
                l0 = add(l0, c00);
                l1 = add(l1, c01);
            }
#pragma omp critical
            {
                sA0 = add(sA0, l0);
                sA1 = add(sA1, l1);
            }
        }
        fr q[3] = {me_fr(t0, h, u, ulen - 1), me_fr(t1, h, u, ulen - 1),
                   me_fr(t2, h, u, ulen - 1)};
        fr c[4];
        eq_times(u[ulen - 1], q, c);
        c[0] = add(c[0], sA0);
        c[1] = add(c[1], sA1);
        c[0] = add(c[0], mul(Cc, INV2));
        fr e[4];
        for (int t = 0; t < 4; t++) e[t] = poly_eval(c, 3, from_u32((uint32_t)t));
        if (strict && !feq(claim, add(e[0], e[1]))) { rc = 2; break; }
        for (int t = 0; t < 4; t++) st(ev_out + 32 * r + 8 * t, e[t]);
        absorb_fr(s, "p0", e[0]); absorb_fr(s, "p1", e[1]);
        absorb_fr(s, "p2", e[2]); absorb_fr(s, "p3", e[3]);
        fr v = challenge(s);
        st(ws_out + 8 * r, v);
        fr vm = mont(v);
#pragma omp parallel for if (h >= PAR_MIN)
        for (uint32_t i = 0; i < h; i++) {
            A[i] = add(A[i], mmul(vm, sub(A[i + h], A[i])));
            S[i] = add(S[i], mmul(vm, sub(S[i + h], S[i])));
        }
        fr eqv = eq2(u[ulen - 1], v);
        claim = poly_eval(c, 3, v);
        ulen--;
        alpha = mul(alpha, eqv);
        Cc = mul(Cc, INV2);
        sz = h;
        r++;
    }
    /* phase 2 (zkob_lookup.cuh:143-171, tlookup.cu:161-279) */
    fr* t3 = falloc(sz / 2 + 1);
    fr* t4 = falloc(sz / 2 + 1);
    while (!rc && ulen > 0) {
        uint32_t h = sz >> 1;
        fr am = mont(alpha), cm = mont(mul(inv_ratio, alpha_sq));
        fr q[3];
        /* A,S with alpha_ */
#pragma omp parallel for if (h >= PAR_MIN)
        for (uint32_t i = 0; i < h; i++) {
            fr c00 = A[i], c01 = sub(A[i + h], A[i]);
            fr c10 = add(S[i], beta), c11 = sub(S[i + h], S[i]);
            t0[i] = mmul(am, mul(c00, c10));
            t1[i] = mmul(am, mont(add(mmul(c01, c10), mmul(c00, c11))));
            t2[i] = mmul(am, mul(c01, c11));
        }
        for (int j = 0; j < 3; j++)
            q[j] = me_fr(j == 0 ? t0 : j == 1 ? t1 : t2, h, u, ulen - 1);
        /* B,T with inv_ratio*alpha_sq */
#pragma omp parallel for if (h >= PAR_MIN)
        for (uint32_t i = 0; i < h; i++) {
            fr c00 = Bv[i], c01 = sub(Bv[i + h], Bv[i]);
            fr c10 = add(T[i], beta), c11 = sub(T[i + h], T[i]);
            t0[i] = mmul(cm, mul(c00, c10));
            t1[i] = mmul(cm, mont(add(mmul(c01, c10), mmul(c00, c11))));
            t2[i] = mmul(cm, mul(c01, c11));
        }
        for (int j = 0; j < 3; j++)
            q[j] = add(q[j], me_fr(j == 0 ? t0 : j == 1 ? t1 : t2, h, u, ulen - 1));
        fr c[4];
        eq_times(u[ulen - 1], q, c);
        /* + {sum A0, sum A1} (tLookup_phase2_poly_sum_kernel) */
#pragma omp parallel for if (h >= PAR_MIN)
        for (uint32_t i = 0; i < h; i++) { t3[i] = A[i]; t4[i] = sub(A[i + h], A[i]); }
        c[0] = add(c[0], sum_fr(t3, h));
        c[1] = add(c[1], sum_fr(t4, h));
        /* - inv_ratio * {sum m0B0, sum m1B0+m0B1, sum m1B1} (dotprod kernel) */
#pragma omp parallel for if (h >= PAR_MIN)
        for (uint32_t i = 0; i < h; i++) {
            fr a0 = m[i], a1 = sub(m[i + h], m[i]);
            fr b0 = Bv[i], b1 = sub(Bv[i + h], Bv[i]);
            t0[i] = mul(a0, b0);
            t1[i] = mont(add(mmul(a1, b0), mmul(a0, b1)));
            t2[i] = mul(a1, b1);
        }
        c[0] = sub(c[0], mul(sum_fr(t0, h), inv_ratio));
        c[1] = sub(c[1], mul(sum_fr(t1, h), inv_ratio));
        c[2] = sub(c[2], mul(sum_fr(t2, h), inv_ratio));
        fr e[4];
        for (int t = 0; t < 4; t++) e[t] = poly_eval(c, 3, from_u32((uint32_t)t));
        if (strict && !feq(claim, add(e[0], e[1]))) { rc = 2; break; }
        for (int t = 0; t < 4; t++) st(ev_out + 32 * r + 8 * t, e[t]);
        absorb_fr(s, "p0", e[0]); absorb_fr(s, "p1", e[1]);
        absorb_fr(s, "p2", e[2]); absorb_fr(s, "p3", e[3]);
        fr v = challenge(s);
        st(ws_out + 8 * r, v);
        fr vm = mont(v);
#pragma omp parallel for if (h >= PAR_MIN)
        for (uint32_t i = 0; i < h; i++) {
            A[i] = add(A[i], mmul(vm, sub(A[i + h], A[i])));
            S[i] = add(S[i], mmul(vm, sub(S[i + h], S[i])));
            Bv[i] = add(Bv[i], mmul(vm, sub(Bv[i + h], Bv[i])));
            T[i] = add(T[i], mmul(vm, sub(T[i + h], T[i])));
            m[i] = add(m[i], mmul(vm, sub(m[i + h], m[i])));
        }
        fr eqv = eq2(u[ulen - 1], v);
        claim = poly_eval(c, 3, v);
        ulen--;
        alpha = mul(alpha, eqv);
        alpha_sq = mul(alpha_sq, eqv);
        sz = h;
        r++;
    }
    if (!rc) {
        st(term_out, A[0]);
        st(term_out + 8, S[0]);
        st(term_out + 16, Bv[0]);
        st(term_out + 24, T[0]);
        st(term_out + 32, m[0]);
        absorb_fr(s, "A_f", A[0]);
        absorb_fr(s, "S_f", S[0]);
        absorb_fr(s, "m_f", m[0]);
    }
    free(t0); free(t1); free(t2); free(t3); free(t4);
    free(A); free(S); free(T); free(m); free(Bv); free(u);
    return rc;
}

/* ------------------------------------------------------------------------------ */
/* Hadamard sumcheck (zkob_lookup.cuh:212-233 k_hp3_step, :292-315 fs_hadamard)     */
/* ------------------------------------------------------------------------------ */
int or_hp_prove(uint8_t s[32], const uint32_t claim_in[8], const uint32_t* Ein,
                const uint32_t* Sin, const uint32_t* Uin, uint32_t n, int strict,
                uint32_t* ev_out, uint32_t* term_out, uint32_t* ws_out) {
    if (!n || (n & (n - 1))) return 1;
    fr* E = from_aos(Ein, n);
    fr* S = from_aos(Sin, n);
    fr* U = from_aos(Uin, n);
    fr claim = ld(claim_in);
    int rc = 0;
    uint32_t sz = n, r = 0;
    while (sz > 1) {
        uint32_t h = sz >> 1;
        fr e[4] = {ZERO, ZERO, ZERO, ZERO};
#pragma omp parallel if (h >= PAR_MIN)
        {
            fr l[4] = {ZERO, ZERO, ZERO, ZERO};
#pragma omp for nowait
            for (uint32_t i = 0; i < h; i++) {
                fr ee = E[i], de = sub(E[i + h], E[i]);
                fr ss = S[i], ds = sub(S[i + h], S[i]);
                fr uu = U[i], du = sub(U[i + h], U[i]);
                for (int t = 0; t < 4; t++) {
                    fr es = mmul(mont(ee), mont(ss));
                    l[t] = add(l[t], mmul(es, uu));
                    ee = add(ee, de);
                    ss = add(ss, ds);
                    uu = add(uu, du);
                }
            }
#pragma omp critical
            for (int t = 0; t < 4; t++) e[t] = add(e[t], l[t]);
        }
        if (strict && !feq(claim, add(e[0], e[1]))) { rc = 2; break; }
        for (int t = 0; t < 4; t++) st(ev_out + 32 * r + 8 * t, e[t]);
        absorb_fr(s, "hp0", e[0]); absorb_fr(s, "hp1", e[1]);
        absorb_fr(s, "hp2", e[2]); absorb_fr(s, "hp3", e[3]);
        fr w = challenge(s);
        st(ws_out + 8 * r, w);
        fr wm = mont(w);
#pragma omp parallel for if (h >= PAR_MIN)
        for (uint32_t i = 0; i < h; i++) { /* k_fr_fold x3 */
            E[i] = add(E[i], mmul(wm, sub(E[i + h], E[i])));
            S[i] = add(S[i], mmul(wm, sub(S[i + h], S[i])));
            U[i] = add(U[i], mmul(wm, sub(U[i + h], U[i])));
        }
        claim = lagrange4(e, w);
        sz = h;
        r++;
    }
    if (!rc) {
        st(term_out, S[0]);
        st(term_out + 8, U[0]);
        st(term_out + 16, E[0]);
    }
    free(E); free(S); free(U);
    return rc;
}

/* ------------------------------------------------------------------------------ */
/* zkip and zkip_stacked without a transcript: zkfc.cu:94-246, :288-307              */
/* ------------------------------------------------------------------------------ */
/* one round of zkip_stacked_poly_kernel / zkip_poly_kernel over [N, D] (rows n, n+no
 * paired, rows >= N zero) followed by partial_me(u_, no, D).sum() of each output: the
 * reference's two-step schedule (products into three tensors, then MLE reductions) */
static void stk_poly(const fr* a, const fr* b, uint32_t N, uint32_t D, const fr* u_, uint32_t ku,
                     fr p[3]) {
    uint32_t no = (1u << ceil_log2(N)) >> 1;
    size_t so = (size_t)no * D;
    fr* o[3] = {falloc(so), falloc(so), falloc(so)};
    for (size_t g = 0; g < so; g++) {
        fr a0 = a[g], b0 = b[g];
        fr a1 = g + so < (size_t)N * D ? sub(a[g + so], a0) : sub(ZERO, a0);
        fr b1 = g + so < (size_t)N * D ? sub(b[g + so], b0) : sub(ZERO, b0);
        o[0][g] = mul(a0, b0);
        o[1][g] = add(mul(a0, b1), mul(a1, b0));
        o[2][g] = mul(a1, b1);
    }
    for (int k = 0; k < 3; k++) {
        if (ku) {
            uint32_t on;
            fr* r = partial_me_fr(o[k], (uint32_t)so, u_, ku, no, D, &on);
            p[k] = sum_fr(r, on);
            free(r);
        } else {
            p[k] = sum_fr(o[k], so);
        }
        free(o[k]);
    }
}
/* zkip_stacked_reduce_kernel / zkip_reduce_kernel: a[g] = a0 + v (a1 - a0), g < no*D */
static void stk_reduce(fr* a, fr* b, uint32_t N, uint32_t D, fr v) {
    uint32_t no = (1u << ceil_log2(N)) >> 1;
    size_t so = (size_t)no * D;
    fr vm = mont(v);
    for (size_t g = 0; g < so; g++) {
        fr a1 = g + so < (size_t)N * D ? a[g + so] : ZERO;
        fr b1 = g + so < (size_t)N * D ? b[g + so] : ZERO;
        a[g] = add(a[g], mmul(vm, sub(a1, a[g])));
        b[g] = add(b[g], mmul(vm, sub(b1, b[g])));
    }
}
/* zkip (zkfc.cu:139-151): u.back() binds first; claim != p(0)+p(1) -> 2 */
static int zkip_fr(fr* claim, fr* a, fr* b, uint32_t n, const fr* u, uint32_t k, fr* proof) {
    uint32_t sz = n;
    for (uint32_t r = 0; r < k; r++) {
        fr p[3];
        stk_poly(a, b, sz, 1, NULL, 0, p);
        proof[3 * r] = p[0];
        proof[3 * r + 1] = p[1];
        proof[3 * r + 2] = p[2];
        if (!feq(*claim, add(poly_eval(p, 2, ZERO), poly_eval(p, 2, ONE)))) return 2;
        fr x = u[k - 1 - r];
        *claim = poly_eval(p, 2, x);
        stk_reduce(a, b, sz, 1, x);
        sz = (1u << ceil_log2(sz)) >> 1;
    }
    return 0;
}
int or_zkip(const uint32_t claim[8], const uint32_t* a, const uint32_t* b, uint32_t n,
            const uint32_t* u, uint32_t k, uint32_t* proof_out, uint32_t final_out[8]) {
    if (!n || k > ceil_log2(n)) return 1;
    fr* A = from_aos(a, n);
    fr* B = from_aos(b, n);
    fr* U = from_aos(u, k);
    fr* pr = falloc(3 * (size_t)k);
    fr c = ld(claim);
    int rc = zkip_fr(&c, A, B, n, U, k, pr);
    for (uint32_t i = 0; i < 3 * k; i++) st(proof_out + 8 * i, pr[i]);
    if (!rc) st(final_out, c);
    free(A); free(B); free(U); free(pr);
    return rc;
}
/* zkip_stacked (zkfc.cu:230-246): q = eq(uN.back(), X) * p must satisfy claim = q(0)+q(1)
 * (Polynomial::eq: 1 - u + (2u - 1) X, polynomial.cu:342-353); next claim p(vN.back()) */
static int zkip_stacked_fr(fr* claim, fr* a, fr* b, uint32_t N, uint32_t D, const fr* uN,
                           uint32_t kN, const fr* uD, uint32_t kD, const fr* vN, fr* proof) {
    uint32_t n = N;
    for (uint32_t r = 0; r < kN; r++) {
        uint32_t ku = kN - 1 - r;
        fr p[3];
        stk_poly(a, b, n, D, uN, ku, p);
        proof[3 * r] = p[0];
        proof[3 * r + 1] = p[1];
        proof[3 * r + 2] = p[2];
        fr ul = uN[ku];
        fr e[2] = {sub(ONE, ul), sub(add(ul, ul), ONE)};
        fr q0 = mul(poly_eval(e, 1, ZERO), poly_eval(p, 2, ZERO));
        fr q1 = mul(poly_eval(e, 1, ONE), poly_eval(p, 2, ONE));
        if (!feq(*claim, add(q0, q1))) return 2;
        fr v = vN[ku];
        *claim = poly_eval(p, 2, v);
        stk_reduce(a, b, n, D, v);
        n = (1u << ceil_log2(n)) >> 1;
    }
    return zkip_fr(claim, a, b, D, uD, kD, proof + 3 * kN);
}
int or_zkip_stacked(const uint32_t claim[8], const uint32_t* a, const uint32_t* b,
                    const uint32_t* uN, uint32_t kN, const uint32_t* uD, uint32_t kD,
                    const uint32_t* vN, uint32_t N, uint32_t D, uint32_t* proof_out,
                    uint32_t final_out[8]) {
    if (!N || !D || kN != ceil_log2(N) || kD > ceil_log2(D)) return 1;
    size_t n = (size_t)N * D;
    fr* A = from_aos(a, n);
    fr* B = from_aos(b, n);
    fr* UN = from_aos(uN, kN);
    fr* VN = from_aos(vN, kN);
    fr* UD = from_aos(uD, kD);
    fr* pr = falloc(3 * (size_t)(kN + kD));
    fr c = ld(claim);
    int rc = zkip_stacked_fr(&c, A, B, N, D, UN, kN, UD, kD, VN, pr);
    for (uint32_t i = 0; i < 3 * (kN + kD); i++) st(proof_out + 8 * i, pr[i]);
    if (!rc) st(final_out, c);
    free(A); free(B); free(UN); free(VN); free(UD); free(pr);
    return rc;
}
/* zkFCStacked::prove (zkfc.cu:288-307) on field inputs */
int or_fc_stacked_prove(const uint32_t* X, const uint32_t* W, const uint32_t* Y, const uint32_t* bias,
                        uint32_t num, uint32_t B, uint32_t IN, uint32_t OUT, const uint32_t* u_num,
                        const uint32_t* v_num, const uint32_t* u_batch, const uint32_t* u_input,
                        const uint32_t* u_output, uint32_t* proof_out, uint32_t* claims_out) {
    if (!num || !B || !IN || !OUT) return 1;
    uint32_t kn = ceil_log2(num), kb = ceil_log2(B), ki = ceil_log2(IN), ko = ceil_log2(OUT);
    fr* Xf = from_aos(X, (size_t)num * B * IN);
    fr* Wf = from_aos(W, (size_t)num * IN * OUT);
    fr* Yf = from_aos(Y, (size_t)num * B * OUT);
    fr *un = from_aos(u_num, kn), *vn = from_aos(v_num, kn), *ub = from_aos(u_batch, kb);
    fr *ui = from_aos(u_input, ki), *uo = from_aos(u_output, ko);
    int rc = 0;
    fr claim, fin, ox, ow;
    fr *xr = NULL, *wr = NULL, *pr = falloc(3 * (size_t)(kn + ki));
    {
        const fr* us[3] = {un, ub, uo};
        uint32_t ks[3] = {kn, kb, ko}, sh[3] = {num, B, OUT};
        if (multi_dim_me_fr(Yf, num * B * OUT, us, ks, sh, 3, &claim)) { rc = 1; goto done; }
    }
    if (bias) {
        /* broadcasting_ones(u_batch) * b.multi_dim_me({u_num, u_output}, {num, OUT}) */
        fr* ones = falloc(B);
        for (uint32_t i = 0; i < B; i++) ones[i] = ONE;
        fr* bf = from_aos(bias, (size_t)num * OUT);
        const fr* us[2] = {un, uo};
        uint32_t ks[2] = {kn, ko}, sh[2] = {num, OUT};
        fr bb, ob = me_fr(ones, B, ub, kb);
        rc = multi_dim_me_fr(bf, num * OUT, us, ks, sh, 2, &bb);
        free(ones); free(bf);
        if (rc) { rc = 1; goto done; }
        claim = sub(claim, mul(ob, bb));
    }
    {
        uint32_t nx, nw;
        xr = partial_me_fr(Xf, num * B * IN, ub, kb, B, IN, &nx);
        wr = partial_me_fr(Wf, num * IN * OUT, uo, ko, OUT, 1, &nw);
    }
    fin = claim;
    rc = zkip_stacked_fr(&fin, xr, wr, num, IN, un, kn, ui, ki, vn, pr);
    for (uint32_t i = 0; i < 3 * (kn + ki); i++) st(proof_out + 8 * i, pr[i]);
    if (rc) goto done;
    {
        const fr* usx[3] = {vn, ub, ui};
        uint32_t ksx[3] = {kn, kb, ki}, shx[3] = {num, B, IN};
        const fr* usw[3] = {vn, ui, uo};
        uint32_t ksw[3] = {kn, ki, ko}, shw[3] = {num, IN, OUT};
        if (multi_dim_me_fr(Xf, num * B * IN, usx, ksx, shx, 3, &ox) ||
            multi_dim_me_fr(Wf, num * IN * OUT, usw, ksw, shw, 3, &ow)) { rc = 1; goto done; }
    }
    st(claims_out, claim);
    st(claims_out + 8, fin);
    if (!feq(fin, mul(ox, ow))) rc = 2; /* zkfc.cu:306 */
done:
    free(Xf); free(Wf); free(Yf); free(un); free(vn); free(ub); free(ui); free(uo);
    free(xr); free(wr); free(pr);
    return rc;
}

/* ------------------------------------------------------------------------------ */
/* rescaling witness: rescaling.cu:8-21 with scalar_to_long (fr-tensor.cu:935-945)   */
/* ------------------------------------------------------------------------------ */
/* 64-bit limbs here: the reference's limbs 0,1 are v[0]; limbs 2..7 are v[1..3] */
static uint64_t scalar_to_ulong(fr x) {
    if (x.v[1] || x.v[2] || x.v[3]) return 0;
    return x.v[0];
}
int64_t or_scalar_to_long(const uint32_t x[8]) {
    fr v = ld(x);
    if (!v.v[1] && !v.v[2] && !v.v[3] && !(v.v[0] >> 63)) return (int64_t)v.v[0];
    return (int64_t)(0 - scalar_to_ulong(sub(ZERO, v)));
}
static void rescale1(int64_t x, int64_t sf, int64_t* q, int64_t* rem) {
    int64_t hsf = sf >> 1;
    int64_t temp = (int64_t)((uint64_t)x + (uint64_t)hsf) % sf;
    int64_t r = (temp < 0 ? temp + sf : temp) - hsf;
    *q = (int64_t)((uint64_t)x - (uint64_t)r) / sf;
    *rem = r;
}
int or_rescale_i64(const int64_t* x, uint32_t n, uint32_t sf, int64_t* q, int64_t* rem) {
    if (!sf) return 1;
    for (uint32_t i = 0; i < n; i++) rescale1(x[i], sf, q + i, rem + i);
    return 0;
}
int or_rescale_fr(const uint32_t* x, uint32_t n, uint32_t sf, int64_t* q, int64_t* rem) {
    if (!sf) return 1;
    for (uint32_t i = 0; i < n; i++) rescale1(or_scalar_to_long(x + 8 * i), sf, q + i, rem + i);
    return 0;
}

/* ------------------------------------------------------------------------------ */
/* witness GEMM: matrixMultiplyOptimized / FrTensor::matmul (fr-tensor.cu:831-878)   */
/* ------------------------------------------------------------------------------ */
/* C[i][j] = mont(sum_k mmul(A[i][k], B[k][j])) (the reference accumulates Montgomery
 * products and converts once, fr-tensor.cu:862-872), plus bias[j] when given (zkFC adds it
 * per column, zkfc.cu:38-40, :53-56) */
int or_matmul_fr(const uint32_t* A, const uint32_t* B, const uint32_t* bias, uint32_t M, uint32_t N, uint32_t Pc,
                 uint32_t* C) {
    if (!M || !N || !Pc) return 1;
#pragma omp parallel for collapse(2) if ((size_t)M * Pc >= 64)
    for (uint32_t i = 0; i < M; i++)
        for (uint32_t j = 0; j < Pc; j++) {
            fr sum = ZERO;
            for (uint32_t k = 0; k < N; k++) sum = add(sum, mmul(ld(A + 8 * ((size_t)i * N + k)), ld(B + 8 * ((size_t)k * Pc + j))));
            fr c = mont(sum);
            if (bias) c = add(c, ld(bias + 8 * j));
            st(C + 8 * ((size_t)i * Pc + j), c);
        }
    return 0;
}
