// g1.hip -- G1 Pedersen commitment kernels (bucket method, commitment.cu:47-103).
#include "fp_dev.hpp"
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
// the witness width all hold the list of negative entries under one digit each.  Lane w
// fingerprints its 15 lists (count, sum of mixed indices), then looks for the first
// earlier window with an equal fingerprint and confirms the match entry by entry; alias
// holds the (window * 16 + digit) whose bucket stands in, itself when there is none.
__global__ __launch_bounds__(64) void k_pip_alias(const uint16_t* __restrict__ lists,
                                                  const uint32_t* __restrict__ offs, uint32_t n,
                                                  uint16_t* __restrict__ alias) {
    __shared__ uint32_t beg_s[64 * 16], cnt_s[64 * 16];
    __shared__ uint64_t fp_s[64 * 16];
    const uint32_t row = blockIdx.x, w = threadIdx.x;
    const size_t rw = (size_t)row * 64 + w;
    const uint32_t* o = offs + rw * 16;
    const uint16_t* L = lists + rw * n;
    for (int d = 1; d < 16; d++) {
        const uint32_t b = o[d], e = d == 15 ? o[0] : o[d + 1];
        uint64_t h = 0;
        for (uint32_t k = b; k < e; k++) h += pip_mix(L[k]);
        beg_s[w * 16 + d] = b;
        cnt_s[w * 16 + d] = e - b;
        fp_s[w * 16 + d] = h;
    }
    __syncthreads();
    const uint16_t* Lrow = lists + (size_t)row * 64 * n;
    for (int d = 1; d < 16; d++) {
        const uint32_t c = cnt_s[w * 16 + d], b = beg_s[w * 16 + d];
        const uint64_t h = fp_s[w * 16 + d];
        uint32_t target = w * 16 + d;
        for (uint32_t w2 = 0; c && w2 < w && target == w * 16 + d; w2++) {
            for (int d2 = 1; d2 < 16; d2++) {
                if (cnt_s[w2 * 16 + d2] != c || fp_s[w2 * 16 + d2] != h) continue;
                const uint16_t* A = L + b;
                const uint16_t* B = Lrow + (size_t)w2 * n + beg_s[w2 * 16 + d2];
                uint32_t k = 0;
                while (k < c && A[k] == B[k]) k++;
                if (k == c) {
                    target = w2 * 16 + d2;
                    break;
                }
            }
        }
        alias[rw * 16 + d] = (uint16_t)target;
    }
}

// block b -> row block b % RB (rows 64 (b % RB) + lane), digit (b / RB) % 15 + 1, window
// b / (15 RB).  The row block varies fastest: blocks go round-robin to the 8 XCDs, and for
// small-integer scalars nearly all the work of a window sits in one digit (the digit of
// r - |v| for negative v), so any other order puts a window's long chains on one XCD.
// The chain starts from the point at infinity, so its first addition returns the
// generator itself (bls12-381.cu:1432), as the reference's bucket does.
__global__ __launch_bounds__(64) void k_pip_bucket(const uint32_t* __restrict__ gens,
                                                   const uint16_t* __restrict__ lists,
                                                   const uint32_t* __restrict__ offs,
                                                   const uint16_t* __restrict__ alias, uint32_t m, uint32_t n,
                                                   uint32_t* __restrict__ buckets) {
    const uint32_t b = blockIdx.x, RB = (m + 63) / 64;
    const uint32_t d = (b / RB) % 15 + 1, w = b / (15 * RB);
    const uint32_t row = (b % RB) * 64 + threadIdx.x;
    if (row >= m) return;
    const size_t rw = (size_t)row * 64 + w;
    const uint32_t* o = offs + rw * 16;
    const uint32_t beg = o[d], end = d == 15 ? o[0] : o[d + 1];
    // empty chains are the point at infinity and aliased ones are another chain's bucket:
    // k_pip_window reads neither from here
    if (beg == end || alias[rw * 16 + d] != w * 16 + d) return;
    const uint16_t* L = lists + rw * n;
    g1_t acc = g1_zero();
    {
        // the next generator (and the index after it) are loaded one addition ahead
        g1_t nxt = g1_load(gens + 36 * (size_t)L[beg]);
        uint32_t idx = beg + 1 < end ? L[beg + 1] : 0;
        for (uint32_t k = beg; k < end; k++) {
            const g1_t g = nxt;
            if (k + 1 < end) nxt = g1_load(gens + 36 * (size_t)idx);
            if (k + 2 < end) idx = L[k + 2];
            acc = g1_add(acc, g);
        }
    }
    g1_store(buckets + (rw * 16 + d) * 36, acc);
}

// sum_b b * bucket[b] by the running sum acc += bucket[b]; run += acc, b = 15..1
// (commitment.cu:73-77)
__global__ __launch_bounds__(64) void k_pip_window(const uint32_t* __restrict__ buckets,
                                                   const uint32_t* __restrict__ offs,
                                                   const uint16_t* __restrict__ alias, uint32_t m,
                                                   uint32_t* __restrict__ partials) {
    const size_t t = (size_t)blockIdx.x * 64 + threadIdx.x;
    if (t >= (size_t)m * 64) return;
    const uint32_t* o = offs + t * 16;
    const size_t row0 = t / 64 * 64;
    g1_t acc = g1_zero(), run = g1_zero();
    for (int b = 15; b >= 1; b--) {
        const uint32_t e = b == 15 ? o[0] : o[b + 1];
        const g1_t bk = e == o[b] ? g1_zero() : g1_load(buckets + ((row0 * 16 + alias[t * 16 + b])) * 36);
        acc = g1_add(acc, bk);
        run = g1_add(run, acc);
    }
    g1_store(partials + t * 36, run);
}

// Horner over the windows, most significant first (commitment.cu:81-89)
__global__ __launch_bounds__(64) void k_pip_combine(const uint32_t* __restrict__ partials, uint32_t m,
                                                    uint32_t* __restrict__ out) {
    const uint32_t row = blockIdx.x * 64 + threadIdx.x;
    if (row >= m) return;
    g1_t acc = g1_zero();
    for (int w = 63; w >= 0; w--) {
        for (int k = 0; k < 4; k++) acc = g1_dbl(acc);
        acc = g1_add(acc, g1_load(partials + ((size_t)row * 64 + w) * 36));
    }
    g1_store(out + (size_t)row * 36, acc);
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
    const uint32_t rb = (m + 63) / 64;
    hipLaunchKernelGGL(k_pip_bucket, dim3(rb * 960), dim3(64), 0, s, gens, lists, offs, alias, m, n, buckets);
}
void launch_pip_window(hipStream_t s, const uint32_t* buckets, const uint32_t* offs, const uint16_t* alias,
                       uint32_t m, uint32_t* partials) {
    hipLaunchKernelGGL(k_pip_window, dim3(m), dim3(64), 0, s, buckets, offs, alias, m, partials);
}
void launch_pip_combine(hipStream_t s, const uint32_t* partials, uint32_t m, uint32_t* out) {
    hipLaunchKernelGGL(k_pip_combine, dim3((m + 63) / 64), dim3(64), 0, s, partials, m, out);
}
