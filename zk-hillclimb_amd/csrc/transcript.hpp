// transcript.hpp -- the reference's SHA-256 Fiat-Shamir transcript (fs_transcript.hpp:115-166)
// and Fr challenge derivation (vrf_common.cuh:219-250), host side.
//
//   state_0 = SHA256(seed)
//   absorb(label, data): state = SHA256(state || le32(|label|) || label || le64(|data|) || data)
//   challenge_bytes():   out = SHA256(state || "chal"); state = SHA256(state || "rtch")
//   challenge_fr():      8 LE u32 limbs of out, limb 7 %= 1944954707, redraw while zero
//
// SHA-256 itself follows FIPS 180-4.
#pragma once
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#if defined(__x86_64__) && !defined(__HIP_DEVICE_COMPILE__)
#include <cpuid.h>
#include <immintrin.h>
#endif

#include "fr_host.hpp"

namespace zkh {

struct Sha256 {
    uint32_t h[8];
    uint64_t len;
    uint8_t buf[64];
    uint32_t blen;

    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
    void init() {
        static const uint32_t iv[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                       0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
        memcpy(h, iv, sizeof(iv));
        len = 0;
        blen = 0;
    }
    void block(const uint8_t* p) {
        static const uint32_t K[64] = {
            0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4,
            0xab1c5ed5, 0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe,
            0x9bdc06a7, 0xc19bf174, 0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f,
            0x4a7484aa, 0x5cb0a9dc, 0x76f988da, 0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7,
            0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967, 0x27b70a85, 0x2e1b2138, 0x4d2c6dfc,
            0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85, 0xa2bfe8a1, 0xa81a664b,
            0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070, 0x19a4c116,
            0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
            0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7,
            0xc67178f2};
        uint32_t w[64];
        for (int i = 0; i < 16; i++)
            w[i] = ((uint32_t)p[4 * i] << 24) | ((uint32_t)p[4 * i + 1] << 16) |
                   ((uint32_t)p[4 * i + 2] << 8) | (uint32_t)p[4 * i + 3];
        for (int i = 16; i < 64; i++) {
            uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6],
                 hh = h[7];
        for (int i = 0; i < 64; i++) {
            uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) +
                          K[i] + w[i];
            uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
            hh = g;
            g = f;
            f = e;
            e = d + t1;
            d = c;
            c = b;
            b = a;
            a = t1 + t2;
        }
        h[0] += a; h[1] += b; h[2] += c; h[3] += d;
        h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
    }
    void compress(const uint8_t* p);
    void compress_blocks(const uint8_t* p, size_t nb);  // nb consecutive 64-byte blocks
    void update(const void* data, size_t n) {
        const uint8_t* p = (const uint8_t*)data;
        len += n;
        if (blen) {  // top up the buffered partial block
            const size_t take = n < 64 - blen ? n : 64 - blen;
            memcpy(buf + blen, p, take);
            blen += (uint32_t)take;
            p += take;
            n -= take;
            if (blen < 64) return;
            compress(buf);
            blen = 0;
        }
        if (n >= 64) {  // whole blocks straight from the input
            const size_t nb = n / 64;
            compress_blocks(p, nb);
            p += nb * 64;
            n -= nb * 64;
        }
        memcpy(buf, p, n);
        blen = (uint32_t)n;
    }
    void final(uint8_t out[32]) {
        const uint64_t bits = len * 8;
        buf[blen++] = 0x80;
        if (blen > 56) {  // no room for the length: pad out this block
            memset(buf + blen, 0, 64 - blen);
            compress(buf);
            blen = 0;
        }
        memset(buf + blen, 0, 56 - blen);
        for (int i = 0; i < 8; i++) buf[56 + i] = (uint8_t)(bits >> (56 - 8 * i));
        compress(buf);
        blen = 0;
        for (int i = 0; i < 8; i++) {
            out[4 * i] = (uint8_t)(h[i] >> 24);
            out[4 * i + 1] = (uint8_t)(h[i] >> 16);
            out[4 * i + 2] = (uint8_t)(h[i] >> 8);
            out[4 * i + 3] = (uint8_t)h[i];
        }
    }
};

#if defined(__x86_64__) && !defined(__HIP_DEVICE_COMPILE__)
// SHA-256 compression with the x86 SHA extensions (Intel, "Intel SHA Extensions", 2013):
// sha256rnds2 performs two rounds on the (ABEF, CDGH) state halves; sha256msg1/msg2 form the
// message schedule four words at a time.  Used when CPUID reports SHA; same digest as block().
__attribute__((target("sha,sse4.1,ssse3"))) inline void sha256_blocks_ni(uint32_t h[8], const uint8_t* p, size_t nb) {
    alignas(16) static const uint32_t K[64] = {
        0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
        0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
        0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
        0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
        0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
        0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
        0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
        0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};
    const __m128i bswap = _mm_set_epi64x(0x0c0d0e0f08090a0bULL, 0x0405060700010203ULL);
    __m128i tmp = _mm_loadu_si128((const __m128i*)&h[0]);  // A B C D (low to high)
    __m128i s1 = _mm_loadu_si128((const __m128i*)&h[4]);   // E F G H
    tmp = _mm_shuffle_epi32(tmp, 0xB1);                     // B A D C
    s1 = _mm_shuffle_epi32(s1, 0x1B);                       // H G F E
    __m128i s0 = _mm_alignr_epi8(tmp, s1, 8);               // F E B A = ABEF (high to low)
    s1 = _mm_blend_epi16(s1, tmp, 0xF0);                    // D C G H = CDGH
    // the state stays in the (ABEF, CDGH) form from block to block
    for (; nb; nb--, p += 64) {
        const __m128i abef = s0, cdgh = s1;
        __m128i w[4];
        for (int i = 0; i < 4; i++) w[i] = _mm_shuffle_epi8(_mm_loadu_si128((const __m128i*)(p + 16 * i)), bswap);
#pragma GCC unroll 16
        for (int g = 0; g < 16; g++) {
            __m128i wg;
            if (g < 4) {
                wg = w[g];
            } else {
                // W[t..t+3] from W[t-16..t-13], W[t-12..t-9], W[t-7..t-4] and W[t-4..t-1]
                __m128i x = _mm_sha256msg1_epu32(w[g & 3], w[(g + 1) & 3]);
                x = _mm_add_epi32(x, _mm_alignr_epi8(w[(g + 3) & 3], w[(g + 2) & 3], 4));
                wg = _mm_sha256msg2_epu32(x, w[(g + 3) & 3]);
                w[g & 3] = wg;
            }
            __m128i m = _mm_add_epi32(wg, _mm_load_si128((const __m128i*)&K[4 * g]));
            s1 = _mm_sha256rnds2_epu32(s1, s0, m);
            s0 = _mm_sha256rnds2_epu32(s0, s1, _mm_shuffle_epi32(m, 0x0E));
        }
        s0 = _mm_add_epi32(s0, abef);
        s1 = _mm_add_epi32(s1, cdgh);
    }
    tmp = _mm_shuffle_epi32(s0, 0x1B);
    s1 = _mm_shuffle_epi32(s1, 0xB1);
    s0 = _mm_blend_epi16(tmp, s1, 0xF0);  // A B C D (low to high)
    s1 = _mm_alignr_epi8(s1, tmp, 8);     // E F G H
    _mm_storeu_si128((__m128i*)&h[0], s0);
    _mm_storeu_si128((__m128i*)&h[4], s1);
}
inline bool cpu_has_sha() {
    static const bool has = [] {
        unsigned a, b, c, d;
        if (!__get_cpuid_count(7, 0, &a, &b, &c, &d)) return false;
        return ((b >> 29) & 1) != 0;
    }();
    return has;
}
inline void Sha256::compress(const uint8_t* p) {
    if (cpu_has_sha()) sha256_blocks_ni(h, p, 1);
    else block(p);
}
inline void Sha256::compress_blocks(const uint8_t* p, size_t nb) {
    if (cpu_has_sha()) sha256_blocks_ni(h, p, nb);
    else
        for (; nb; nb--, p += 64) block(p);
}
#else
inline void Sha256::compress(const uint8_t* p) { block(p); }
inline void Sha256::compress_blocks(const uint8_t* p, size_t nb) {
    for (; nb; nb--, p += 64) block(p);
}
#endif

// SHA-256 of a message of at most 119 bytes: the padded message is built in place and
// compressed as one or two blocks
inline void sha256_short(const uint8_t* msg, size_t n, uint8_t out[32]) {
    uint8_t b[128];
    memcpy(b, msg, n);
    b[n] = 0x80;
    const size_t nb = n + 9 <= 64 ? 64 : 128;
    memset(b + n + 1, 0, nb - n - 1);
    const uint64_t bits = (uint64_t)n * 8;
    for (int i = 0; i < 8; i++) b[nb - 8 + i] = (uint8_t)(bits >> (56 - 8 * i));
    Sha256 c;
    c.init();
    c.compress(b);
    if (nb == 128) c.compress(b + 64);
    for (int i = 0; i < 8; i++) {
        out[4 * i] = (uint8_t)(c.h[i] >> 24);
        out[4 * i + 1] = (uint8_t)(c.h[i] >> 16);
        out[4 * i + 2] = (uint8_t)(c.h[i] >> 8);
        out[4 * i + 3] = (uint8_t)c.h[i];
    }
}

inline void tr_init(uint8_t st[32], const char* seed, size_t n) {
    Sha256 c;
    c.init();
    c.update(seed, n);
    c.final(st);
}
// Absorb trace, the reference's P3_ABLOG switch (fs_transcript.hpp:135-148): with
// P3_ABLOG=path set, every absorb appends "label length state[0..8)" (hex) to that file, the
// reference's own line format, so a run of this library and a run of the reference can be
// diffed to find the first diverging absorb.  Debug only; no protocol effect.  Lines of
// transcripts absorbed on several threads interleave as whole lines.
inline void tr_ablog(const uint8_t st[32], const char* label, size_t llen, size_t len) {
    static FILE* f = [] {
        const char* p = getenv("P3_ABLOG");
        return p ? fopen(p, "w") : nullptr;
    }();
    if (!f) return;
    static std::mutex mu;
    std::lock_guard<std::mutex> lk(mu);
    fprintf(f, "%.*s %zu %02x%02x%02x%02x%02x%02x%02x%02x\n", (int)llen, label, len, st[0], st[1], st[2], st[3],
            st[4], st[5], st[6], st[7]);
    fflush(f);
}
inline void tr_absorb_raw(uint8_t st[32], const char* label, size_t llen, const void* data, size_t len);
inline void tr_absorb(uint8_t st[32], const char* label, size_t llen, const void* data,
                      size_t len) {
    tr_absorb_raw(st, label, llen, data, len);
    tr_ablog(st, label, llen, len);
}
inline void tr_absorb_raw(uint8_t st[32], const char* label, size_t llen, const void* data,
                          size_t len) {
    if (32 + 4 + llen + 8 + len <= 119) {  // the per-round absorbs: one short message
        uint8_t m[119];
        size_t o = 0;
        memcpy(m, st, 32);
        o = 32;
        for (int i = 0; i < 4; i++) m[o++] = (uint8_t)((uint32_t)llen >> (8 * i));
        memcpy(m + o, label, llen);
        o += llen;
        for (int i = 0; i < 8; i++) m[o++] = (uint8_t)((uint64_t)len >> (8 * i));
        memcpy(m + o, data, len);
        o += len;
        sha256_short(m, o, st);
        return;
    }
    Sha256 c;
    c.init();
    c.update(st, 32);
    uint8_t ll[4], dl[8];
    for (int i = 0; i < 4; i++) ll[i] = (uint8_t)((uint32_t)llen >> (8 * i));
    for (int i = 0; i < 8; i++) dl[i] = (uint8_t)((uint64_t)len >> (8 * i));
    c.update(ll, 4);
    c.update(label, llen);
    c.update(dl, 8);
    c.update(data, len);
    c.final(st);
}
inline void tr_challenge_bytes(uint8_t st[32], uint8_t out[32]) {
    uint8_t m[36];
    memcpy(m, st, 32);
    memcpy(m + 32, "chal", 4);
    sha256_short(m, 36, out);
    memcpy(m + 32, "rtch", 4);
    sha256_short(m, 36, st);
}
inline void tr_challenge_limbs(uint8_t st[32], uint32_t out[8]) {
    for (;;) {
        uint8_t b[32];
        tr_challenge_bytes(st, b);
        for (int i = 0; i < 8; i++)
            out[i] = (uint32_t)b[4 * i] | ((uint32_t)b[4 * i + 1] << 8) |
                     ((uint32_t)b[4 * i + 2] << 16) | ((uint32_t)b[4 * i + 3] << 24);
        out[7] %= 1944954707u;
        for (int i = 0; i < 8; i++)
            if (out[i]) return;
    }
}
inline Fr tr_challenge(uint8_t st[32]) {
    uint32_t l[8];
    tr_challenge_limbs(st, l);
    return fr_load(l);
}
inline void tr_absorb_fr(uint8_t st[32], const char* label, const Fr& x) {
    uint32_t b[8];
    fr_store(x, b);
    tr_absorb(st, label, strlen(label), b, 32);
}

}  // namespace zkh
