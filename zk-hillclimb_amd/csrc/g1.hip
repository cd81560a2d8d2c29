// g1.hip -- G1 Pedersen commitment kernels (bucket method, commitment.cu:47-103).
#include "fp_dev.hpp"
#include "fr_dev.hpp"
#include "g1.hpp"

// Lane w of the row's wave owns window w (bits 4w..4w+3 of the raw scalar, commitment.cu:
// 50-55): it reads limb w/8 of every element, counts the digits in its LDS row, turns the
// counts into offsets, then lists every element with a nonzero digit under that digit.
// Lists hold at most n entries per (row, window); offs[.][0] is the total, offs[.][d] the
// start of digit d.
__global__ __launch_bounds__(64) void k_pip_sort(const uint32_t* __restrict__ lo,
                                                 const uint32_t* __restrict__ hi, uint32_t n,
                                                 uint16_t* __restrict__ lists, uint32_t* __restrict__ offs) {
    __shared__ uint32_t cnt[64 * 17];
    const uint32_t row = blockIdx.x, w = threadIdx.x;
    const uint32_t limb = w >> 3, sh = 4 * (w & 7);
    const uint32_t* src = (limb < 4 ? lo : hi) + (limb & 3) + 4 * (size_t)row * n;
    uint32_t* my = cnt + 17 * w;
#pragma unroll
    for (int d = 0; d < 16; d++) my[d] = 0;
    for (uint32_t i = 0; i < n; i++) my[(src[4 * (size_t)i] >> sh) & 15u] += 1;
    const size_t rw = (size_t)row * 64 + w;
    uint32_t* o = offs + rw * 16;
    uint32_t run = 0;
    for (int d = 1; d < 16; d++) {
        const uint32_t c = my[d];
        my[d] = run;
        o[d] = run;
        run += c;
    }
    o[0] = run;
    uint16_t* L = lists + rw * n;
    for (uint32_t i = 0; i < n; i++) {
        const uint32_t d = (src[4 * (size_t)i] >> sh) & 15u;
        if (d) {
            const uint32_t pos = my[d];
            my[d] = pos + 1;
            L[pos] = (uint16_t)i;
        }
    }
}

// 64-bit mix of a generator index (the splitmix64 finaliser); a list's fingerprint is the
// sum over its entries, so equal sets give equal fingerprints in any order
__device__ __forceinline__ uint64_t pip_mix(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Identical chains.  A bucket is a fixed sequence of additions over its list, so two
// (window, digit) chains of a row with the same list produce the same bytes.  For small
// signed scalars this is the common case: a negative v is r - |v|, whose digits above
// |v|'s top window are those of r - 2^k for every such element, so the windows above
// the witness width all hold the list of negative entries under one digit each.  One
// wave per row works through the row's chains together (coalesced list reads): it
// fingerprints each nonempty list (count, sum of mixed indices), then, in window order,
// looks for the first earlier chain with an equal fingerprint and confirms the match
// entry by entry.  alias holds the (window * 16 + digit) whose bucket stands in, itself
// when there is none; representatives are always first occurrences.
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__global__ __launch_bounds__(64) void k_pip_alias(const uint16_t* __restrict__ lists,
                                                  const uint32_t* __restrict__ offs, uint32_t n,
                                                  uint16_t* __restrict__ alias) {
    __shared__ uint32_t beg_s[1024], cnt_s[1024];
    __shared__ uint64_t fp_s[1024];
    __shared__ uint16_t tgt_s[1024];
    const uint32_t row = blockIdx.x, lane = threadIdx.x;
    const uint16_t* Lrow = lists + (size_t)row * 64 * n;
    {
        const uint32_t* o = offs + ((size_t)row * 64 + lane) * 16;
        for (int d = 1; d < 16; d++) {
            const uint32_t b = o[d], e = d == 15 ? o[0] : o[d + 1];
            beg_s[lane * 16 + d] = b;
            cnt_s[lane * 16 + d] = e - b;
        }
    }
    __syncthreads();
    for (uint32_t c = 0; c < 1024; c++) {
        if ((c & 15) == 0) continue;
        const uint32_t cnt = cnt_s[c];
        uint64_t h = 0;
        if (cnt) {
            const uint16_t* L = Lrow + (size_t)(c >> 4) * n + beg_s[c];
            for (uint32_t k = lane; k < cnt; k += 64) h += pip_mix(L[k]);
            h = wave_sum_u64(h);
        }
        if (lane == 0) fp_s[c] = h;
    }
    __syncthreads();
    for (uint32_t c = 0; c < 1024; c++) {
        if ((c & 15) == 0) continue;
        const uint32_t cnt = cnt_s[c];
        uint32_t target = c;
        if (cnt && c >= 16) {
            const uint64_t h = fp_s[c];
            const uint16_t* A = Lrow + (size_t)(c >> 4) * n + beg_s[c];
            // candidates in earlier windows, 64 at a time, lowest first
            for (uint32_t base = 0; base < (c & ~15u) && target == c; base += 64) {
                const uint32_t cc = base + lane;
                const bool hit = cc < (c & ~15u) && (cc & 15) && cnt_s[cc] == cnt && fp_s[cc] == h;
                uint64_t hits = __ballot(hit);
                while (hits && target == c) {
                    const uint32_t cand = base + __builtin_ctzll(hits);
                    hits &= hits - 1;
                    const uint16_t* B = Lrow + (size_t)(cand >> 4) * n + beg_s[cand];
                    bool diff = false;
                    for (uint32_t k = lane; k < cnt; k += 64) diff |= A[k] != B[k];
                    if (!__any(diff)) target = cand;
                }
            }
        }
        if (lane == 0) tgt_s[c] = (uint16_t)target;
    }
    __syncthreads();
    uint16_t* out = alias + (size_t)row * 1024;
    for (uint32_t c = lane; c < 1024; c += 64) out[c] = tgt_s[c];
}

// Bucket chains, two ways in one launch.  A long chain (at least long_min additions: with
// small signed scalars, the shared list of negative entries) is latency-bound, so one
// quad (4 lanes) shares each addition (g1_add_quad: 5 multiply rounds instead of 16); a
// short chain runs on one lane (g1_add), which costs fewer instructions in total.  Blocks
// [0, nq) are quad blocks: a wave holds 16 rows of one (window, digit); the rest are lane
// blocks of 64 rows.  In both, block b -> row block b % RB, digit (b / RB) % 15 + 1,
// window b / (15 RB): the row block varies fastest because blocks go round-robin to the 8
// XCDs and nearly all of a window's work sits in one digit, so any other order puts a
// window's long chains on one XCD.  A chain starts from the point at infinity, so its
// first addition returns the generator itself (bls12-381.cu:1432), as the reference's
// bucket does; the next generator is loaded one addition ahead.
template <bool QUAD>
__device__ __forceinline__ void pip_chain(const uint32_t* __restrict__ gens, const uint16_t* __restrict__ L,
                                          uint32_t beg, uint32_t end, int q, uint32_t* out) {
    g1_t acc = g1_load(gens + 36 * (size_t)L[beg]);
    g1_t nxt = acc;
    uint32_t idx = beg + 1 < end ? L[beg + 1] : 0;
    if (beg + 1 < end) nxt = g1_load(gens + 36 * (size_t)idx);
    if (beg + 2 < end) idx = L[beg + 2];
    for (uint32_t k = beg + 1; k < end; k++) {
        const g1_t g = nxt;
        if (k + 1 < end) nxt = g1_load(gens + 36 * (size_t)idx);
        if (k + 2 < end) idx = L[k + 2];
        acc = QUAD ? g1_add_quad(acc, g, q) : g1_add(acc, g);
    }
    if (!QUAD || q == 0) g1_store(out, acc);
}
__global__ __launch_bounds__(64) void k_pip_bucket(const uint32_t* __restrict__ gens,
                                                   const uint16_t* __restrict__ lists,
                                                   const uint32_t* __restrict__ offs,
                                                   const uint16_t* __restrict__ alias, uint32_t m, uint32_t n,
                                                   uint32_t long_min, uint32_t nq,
                                                   uint32_t* __restrict__ buckets) {
    const bool quad = blockIdx.x < nq;
    const uint32_t b = quad ? blockIdx.x : blockIdx.x - nq;
    const uint32_t RB = quad ? (m + 15) / 16 : (m + 63) / 64;
    const uint32_t d = (b / RB) % 15 + 1, w = b / (15 * RB);
    const uint32_t row = (b % RB) * (quad ? 16 : 64) + (quad ? threadIdx.x / 4 : threadIdx.x);
    if (row >= m) return;
    const size_t rw = (size_t)row * 64 + w;
    const uint32_t* o = offs + rw * 16;
    const uint32_t beg = o[d], end = d == 15 ? o[0] : o[d + 1];
    // empty chains are the point at infinity and aliased ones are another chain's bucket:
    // k_pip_window reads neither from here
    if (beg == end || alias[rw * 16 + d] != w * 16 + d || (end - beg >= long_min) != quad) return;
    const uint16_t* L = lists + rw * n;
    uint32_t* out = buckets + (rw * 16 + d) * 36;
    if (quad) {
        // the long chains set the kernel's length: their waves issue first on a shared SIMD
        __builtin_amdgcn_s_setprio(3);
        pip_chain<true>(gens, L, beg, end, threadIdx.x & 3, out);
    }
    else pip_chain<false>(gens, L, beg, end, 0, out);
}

// sum_b b * bucket[b] by the running sum acc += bucket[b]; run += acc, b = 15..1
// (commitment.cu:73-77); one quad per (row, window) shares each addition
__global__ __launch_bounds__(64) void k_pip_window(const uint32_t* __restrict__ buckets,
                                                   const uint32_t* __restrict__ offs,
                                                   const uint16_t* __restrict__ alias, uint32_t m,
                                                   uint32_t* __restrict__ partials) {
    const size_t t = (size_t)blockIdx.x * 16 + threadIdx.x / 4;
    const int q = threadIdx.x & 3;
    if (t >= (size_t)m * 64) return;
    const uint32_t* o = offs + t * 16;
    const size_t row0 = t / 64 * 64;
    g1_t acc = g1_zero(), run = g1_zero();
    for (int b = 15; b >= 1; b--) {
        const uint32_t e = b == 15 ? o[0] : o[b + 1];
        const g1_t bk = e == o[b] ? g1_zero() : g1_load(buckets + ((row0 * 16 + alias[t * 16 + b])) * 36);
        acc = g1_add_quad(acc, bk, q);
        run = g1_add_quad(run, acc, q);
    }
    if (q == 0) g1_store(partials + t * 36, run);
}

// Horner over the windows, most significant first (commitment.cu:81-89); one quad per row
__global__ __launch_bounds__(64) void k_pip_combine(const uint32_t* __restrict__ partials, uint32_t m,
                                                    uint32_t* __restrict__ out) {
    const uint32_t row = blockIdx.x * 16 + threadIdx.x / 4;
    const int q = threadIdx.x & 3;
    if (row >= m) return;
    g1_t acc = g1_zero();
    for (int w = 63; w >= 0; w--) {
        for (int k = 0; k < 4; k++) acc = g1_dbl_quad(acc, q);
        acc = g1_add_quad(acc, g1_load(partials + ((size_t)row * 64 + w) * 36), q);
    }
    if (q == 0) g1_store(out + (size_t)row * 36, acc);
}

// G1Jacobian_mul (g1-tensor.cu:445-454) on a quad: double-and-add over the scalar's raw
// bits, low bit first.  The doublings after the highest set bit do not reach the result
// and are skipped.
__device__ __forceinline__ uint32_t limb8(const uint32_t s[8], uint32_t l) {
    return l == 0 ? s[0] : l == 1 ? s[1] : l == 2 ? s[2] : l == 3 ? s[3]
         : l == 4 ? s[4] : l == 5 ? s[5] : l == 6 ? s[6] : s[7];
}
__device__ __forceinline__ g1_t g1_mul_quad(g1_t a, const uint32_t s[8], int q) {
    int top = -1;
    for (int l = 7; l >= 0 && top < 0; l--)
        if (s[l]) top = 32 * l + 31 - __builtin_clz(s[l]);
    g1_t acc = g1_zero();
    uint32_t w = 0;
    for (int i = 0; i <= top; i++) {
        if ((i & 31) == 0) w = limb8(s, (uint32_t)i >> 5);
        if ((w >> (i & 31)) & 1u) acc = g1_add_quad(acc, a, q);
        if (i < top) a = g1_dbl_quad(a, q);
    }
    return acc;
}

// G1Jacobian_mul as g1_mul_quad, split over the two waves of a 128-thread block: wave 0 runs
// the doubling chain a, 2a, 4a, ... and hands each 2^i a to wave 1 through LDS, G1P_B
// doublings per block barrier; wave 1 adds the ones whose bit is set into acc one barrier
// later.  The additions and doublings are those of g1_mul_quad in the same order (the same
// Jacobian representative); the two chains run side by side instead of one after the
// other.  Both waves call it with the same scalar for lane slot threadIdx.x & 63 and the
// same `active` (wave 1 does not read `a`); the product is in wave 1's lanes.  Every thread
// of the block takes the same 256 / G1P_B + 1 barriers.
#define G1P_B 8
typedef uint32_t g1_pipe_buf[2][G1P_B][16][36];
__device__ __forceinline__ g1_t g1_mul_quad_pipe(g1_t a, const uint32_t s[8], int q, bool active,
                                                 g1_pipe_buf& buf) {
    static_assert(32 % G1P_B == 0, "a chunk's bits lie in one scalar limb");
    const bool dbl_wave = threadIdx.x < 64;
    const uint32_t slot = (threadIdx.x & 63) >> 2;
    int top = -1;
    if (active)
        for (int l = 7; l >= 0 && top < 0; l--)
            if (s[l]) top = 32 * l + 31 - __builtin_clz(s[l]);
    g1_t acc = g1_zero();
    constexpr int NC = 256 / G1P_B;
    for (int k = 0; k <= NC; k++) {
        if (dbl_wave) {
            if (k < NC) {
                for (int j = 0; j < G1P_B; j++) {
                    const int i = k * G1P_B + j;
                    if (i <= top) {
                        if (q == 0) g1_store(buf[k & 1][j][slot], a);
                        if (i < top) a = g1_dbl_quad(a, q);
                    }
                }
            }
        } else if (k > 0) {
            const uint32_t w = limb8(s, (uint32_t)((k - 1) * G1P_B) >> 5);
            for (int j = 0; j < G1P_B; j++) {
                const int i = (k - 1) * G1P_B + j;
                if (i <= top && ((w >> (i & 31)) & 1u)) acc = g1_add_quad(acc, g1_load(buf[(k - 1) & 1][j][slot]), q);
            }
        }
        __syncthreads();
    }
    return acc;
}

// elementwise with a broadcast base (G1_jacobian_elementwise_mul_broadcast,
// g1-tensor.cu:463-468): out[i] = base[i % nb] * s[i], one quad per element
__global__ __launch_bounds__(64) void k_g1_mul(const uint32_t* __restrict__ base, uint32_t nb,
                                               const uint32_t* __restrict__ lo, const uint32_t* __restrict__ hi,
                                               uint32_t n, uint32_t* __restrict__ out) {
    const uint32_t i = blockIdx.x * 16 + threadIdx.x / 4;
    const int q = threadIdx.x & 3;
    if (i >= n) return;
    const uint4 s0 = ((const uint4*)lo)[i], s1 = ((const uint4*)hi)[i];
    const uint32_t sc[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    const g1_t r = g1_mul_quad(g1_load(base + 36 * (size_t)(i % nb)), sc, q);
    if (q == 0) g1_store(out + 36 * (size_t)i, r);
}

// out[i] = b[i] + a[i] * s: one scalar for every row, the sum with b[i] as first operand
// (hb_addmul with mul_first = false, zkob_fastg1.cuh:56-88: k_g1_mul then k_g1_addsub)
__global__ __launch_bounds__(64) void k_g1_addmul(const uint32_t* __restrict__ a, G1Scalar sc,
                                                  const uint32_t* __restrict__ b, uint32_t n,
                                                  uint32_t* __restrict__ out) {
    const uint32_t i = blockIdx.x * 16 + threadIdx.x / 4;
    const int q = threadIdx.x & 3;
    if (i >= n) return;
    const g1_t m = g1_mul_quad(g1_load(a + 36 * (size_t)i), sc.v, q);
    const g1_t r = g1_add_quad(g1_load(b + 36 * (size_t)i), m, q);
    if (q == 0) g1_store(out + 36 * (size_t)i, r);
}

// ---- inner-product argument rounds (ipa_prove, vrf_common.cuh:302-336) ----
// a, b: plain Fr, 8 words per entry; g, P: points.  Round of size 2h:
//   ip = (<a_lo, b_hi>, <a_hi, b_lo>)                       (dev_ip, one block)
//   P[j] = g_hi[j] a_lo[j], P[h + j] = g_lo[j] a_hi[j], P[2h] = Q ip_L, P[2h+1] = Q ip_R
//   pairwise trees over P[0, h) and P[h, 2h)                  (dev_msm's order)
//   L = P[0] + P[2h], R = P[h] + P[2h+1]
//   fold: a' = x a_lo + x^-1 a_hi, b' = x^-1 b_lo + x b_hi, g' = x^-1 g_lo + x g_hi
__global__ __launch_bounds__(256) void k_ipa_ip(IpaBatchDev B, fr_t r2) {
    const IpaJobDev& J = B.j[blockIdx.y];
    const uint32_t h = J.h;
    if (!h) return;  // the job has finished its rounds (whole block)
    const uint32_t *a = J.a, *b = J.b;
    __shared__ fr_t red[2][256];
    fr_t sl = fr_zero(), sr = fr_zero();
    for (uint32_t i = threadIdx.x; i < h; i += 256) {
        sl = fr_add(sl, mont_mul(ld_aos(a, i), ld_aos(b, h + i)));
        sr = fr_add(sr, mont_mul(ld_aos(a, h + i), ld_aos(b, i)));
    }
    red[0][threadIdx.x] = sl;
    red[1][threadIdx.x] = sr;
    __syncthreads();
    for (uint32_t o = 128; o > 0; o >>= 1) {
        if (threadIdx.x < o) {
            red[0][threadIdx.x] = fr_add(red[0][threadIdx.x], red[0][threadIdx.x + o]);
            red[1][threadIdx.x] = fr_add(red[1][threadIdx.x], red[1][threadIdx.x + o]);
        }
        __syncthreads();
    }
    // sums of a b 2^-256; times R^2 2^-256 gives the plain sums
    if (threadIdx.x < 2) st_aos(J.ip, threadIdx.x, mont_mul(red[threadIdx.x][0], r2));
}
// L and R terms (vrf_common.cuh:316-319): P[j] = g[h + j] a[j], P[h + j] = g[j] a[h + j],
// P[2h], P[2h + 1] = Q <a_lo, b_hi>, Q <a_hi, b_lo>; 16 products per 128-thread block, each
// on a quad of both waves (g1_mul_quad_pipe); blockIdx.y is the job
__global__ __launch_bounds__(128) void k_ipa_scale(IpaBatchDev B) {
    const IpaJobDev& J = B.j[blockIdx.y];
    const uint32_t h = J.h;
    if (blockIdx.x * 16 >= 2 * h + 2 || !h) return;  // whole block: past the job's products
    __shared__ g1_pipe_buf buf;
    const uint32_t j = blockIdx.x * 16 + (threadIdx.x & 63) / 4;
    const int q = threadIdx.x & 3;
    const bool active = j < 2 * h + 2;
    uint32_t sc[8] = {};
    g1_t base = g1_zero();
    if (active) {
        const uint32_t* bp = j < h ? J.g + 36 * (size_t)(h + j) : j < 2 * h ? J.g + 36 * (size_t)(j - h) : J.Q;
        const uint32_t* sp = j < 2 * h ? J.a + 8 * (size_t)j : J.ip + 8 * (j - 2 * h);
#pragma unroll
        for (int k = 0; k < 8; k++) sc[k] = sp[k];
        if (threadIdx.x < 64) base = g1_load(bp);
    }
    const g1_t r = g1_mul_quad_pipe(base, sc, q, active, buf);
    if (active && threadIdx.x >= 64 && q == 0) g1_store(J.P + 36 * (size_t)j, r);
}
// one level of the pairwise trees over P[0, h) and P[h, 2h): half = h >> shift per job
__global__ __launch_bounds__(64) void k_ipa_tree(IpaBatchDev B, uint32_t shift) {
    const IpaJobDev& J = B.j[blockIdx.y];
    const uint32_t h = J.h, half = h >> shift;
    const uint32_t i = blockIdx.x * 16 + threadIdx.x / 4;
    const int q = threadIdx.x & 3;
    if (i >= 2 * half) return;
    const size_t k = (size_t)(i / half) * h + i % half;
    const g1_t r = g1_add_quad(g1_load(J.P + 36 * k), g1_load(J.P + 36 * (k + half)), q);
    if (q == 0) g1_store(J.P + 36 * k, r);
}
__global__ __launch_bounds__(64) void k_ipa_lr(IpaBatchDev B) {
    const IpaJobDev& J = B.j[blockIdx.y];
    const uint32_t side = threadIdx.x / 4, h = J.h;
    const int q = threadIdx.x & 3;
    if (side >= 2 || !h) return;
    const g1_t r = g1_add_quad(g1_load(J.P + 36 * (size_t)(side * h)), g1_load(J.P + 36 * (size_t)(2 * h + side)), q);
    if (q == 0) g1_store(J.LR + 36 * side, r);
}
// eight lanes per element: quad 0 computes x^-1 g_lo[i], quad 1 x g_hi[i] (k_g1_fold2's
// two products, vrf_common.cuh:71-76), then quad 0 adds them in that order
__global__ __launch_bounds__(128) void k_ipa_fold(IpaBatchDev B) {
    const IpaJobDev& J = B.j[blockIdx.y];
    const uint32_t h = J.h;
    if (blockIdx.x * 8 >= h) return;  // whole block: past the job's pairs (or a finished job)
    __shared__ g1_pipe_buf buf;
    __shared__ uint32_t hi_pt[8][36];
    const uint32_t e = (threadIdx.x & 63) / 8, i = blockIdx.x * 8 + e;
    const int q = threadIdx.x & 3, half_sel = (threadIdx.x >> 2) & 1;
    const bool active = i < h, add_wave = threadIdx.x >= 64;
    g1_t base = g1_zero();
    if (active && !add_wave) base = g1_load(J.g + 36 * (size_t)(i + half_sel * h));
    g1_t r = g1_mul_quad_pipe(base, half_sel ? J.x : J.xi, q, active, buf);
    if (add_wave && active && half_sel && q == 0) g1_store(hi_pt[e], r);
    __syncthreads();
    if (add_wave && active && !half_sel) {
        r = g1_add_quad(r, g1_load(hi_pt[e]), q);
        if (q == 0) {
            fr_t xm, xim;
#pragma unroll
            for (int k = 0; k < 8; k++) xm.v[k] = J.xm[k], xim.v[k] = J.xim[k];
            g1_store(J.g2 + 36 * (size_t)i, r);
            st_aos(J.a2, i, fr_add(mont_mul(xm, ld_aos(J.a, i)), mont_mul(xim, ld_aos(J.a, i + h))));
            st_aos(J.b2, i, fr_add(mont_mul(xim, ld_aos(J.b, i)), mont_mul(xm, ld_aos(J.b, i + h))));
        }
    }
}
void launch_ipa_ip(hipStream_t s, const IpaBatchDev& B, uint32_t nj, const uint32_t r2[8]) {
    fr_t R2;
    for (int k = 0; k < 8; k++) R2.v[k] = r2[k];
    hipLaunchKernelGGL(k_ipa_ip, dim3(1, nj), dim3(256), 0, s, B, R2);
}
void launch_ipa_scale(hipStream_t s, const IpaBatchDev& B, uint32_t nj, uint32_t hmax) {
    hipLaunchKernelGGL(k_ipa_scale, dim3((2 * hmax + 2 + 15) / 16, nj), dim3(128), 0, s, B);
}
void launch_ipa_tree(hipStream_t s, const IpaBatchDev& B, uint32_t nj, uint32_t hmax, uint32_t shift) {
    hipLaunchKernelGGL(k_ipa_tree, dim3((2 * (hmax >> shift) + 15) / 16, nj), dim3(64), 0, s, B, shift);
}
void launch_ipa_lr(hipStream_t s, const IpaBatchDev& B, uint32_t nj) {
    hipLaunchKernelGGL(k_ipa_lr, dim3(1, nj), dim3(64), 0, s, B);
}
void launch_ipa_fold(hipStream_t s, const IpaBatchDev& B, uint32_t nj, uint32_t hmax) {
    hipLaunchKernelGGL(k_ipa_fold, dim3((hmax + 7) / 8, nj), dim3(128), 0, s, B);
}
// planes -> 8-word entries
__global__ __launch_bounds__(256) void k_planes_to_aos(const uint32_t* __restrict__ lo, const uint32_t* __restrict__ hi,
                                                       uint32_t n, uint32_t* __restrict__ out) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    st_aos(out, i, ld_fr((const uint4*)lo, (const uint4*)hi, i));
}
void launch_planes_to_aos(hipStream_t s, const uint32_t* lo, const uint32_t* hi, uint32_t n, uint32_t* out) {
    hipLaunchKernelGGL(k_planes_to_aos, dim3((n + 255) / 256), dim3(256), 0, s, lo, hi, n, out);
}
void launch_g1_addmul(hipStream_t s, const uint32_t* a, const G1Scalar& sc, const uint32_t* b, uint32_t n,
                      uint32_t* out) {
    hipLaunchKernelGGL(k_g1_addmul, dim3((n + 15) / 16), dim3(64), 0, s, a, sc, b, n, out);
}
void launch_g1_mul(hipStream_t s, const uint32_t* base, uint32_t nb, const uint32_t* lo, const uint32_t* hi,
                   uint32_t n, uint32_t* out) {
    hipLaunchKernelGGL(k_g1_mul, dim3((n + 15) / 16), dim3(64), 0, s, base, nb, lo, hi, n, out);
}
void launch_pip_sort(hipStream_t s, const uint32_t* lo, const uint32_t* hi, uint32_t m, uint32_t n,
                     uint16_t* lists, uint32_t* offs) {
    hipLaunchKernelGGL(k_pip_sort, dim3(m), dim3(64), 0, s, lo, hi, n, lists, offs);
}
void launch_pip_alias(hipStream_t s, const uint16_t* lists, const uint32_t* offs, uint32_t m, uint32_t n,
                      uint16_t* alias) {
    hipLaunchKernelGGL(k_pip_alias, dim3(m), dim3(64), 0, s, lists, offs, n, alias);
}
void launch_pip_bucket(hipStream_t s, const uint32_t* gens, const uint16_t* lists, const uint32_t* offs,
                       const uint16_t* alias, uint32_t m, uint32_t n, uint32_t* buckets) {
    // a chain is long from n/8 additions on: twice the mean of a window whose digits are
    // spread evenly, so evenly spread scalars never take the quad path
    const uint32_t long_min = n / 8 > 32 ? n / 8 : 32;
    const uint32_t nq = (m + 15) / 16 * 960, ns = (m + 63) / 64 * 960;
    hipLaunchKernelGGL(k_pip_bucket, dim3(nq + ns), dim3(64), 0, s, gens, lists, offs, alias, m, n, long_min, nq,
                       buckets);
}
void launch_pip_window(hipStream_t s, const uint32_t* buckets, const uint32_t* offs, const uint16_t* alias,
                       uint32_t m, uint32_t* partials) {
    hipLaunchKernelGGL(k_pip_window, dim3(4 * m), dim3(64), 0, s, buckets, offs, alias, m, partials);
}
void launch_pip_combine(hipStream_t s, const uint32_t* partials, uint32_t m, uint32_t* out) {
    hipLaunchKernelGGL(k_pip_combine, dim3((m + 15) / 16), dim3(64), 0, s, partials, m, out);
}
