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

// block b -> row block b % RB (rows 64 (b % RB) + lane), digit (b / RB) % 15 + 1, window
// b / (15 RB).  The row block varies fastest: blocks go round-robin to the 8 XCDs, and for
// small-integer scalars nearly all the work of a window sits in one digit (the digit of
// r - |v| for negative v), so any other order puts a window's long chains on one XCD.
// The chain starts from the point at infinity, so its first addition returns the
// generator itself (bls12-381.cu:1432), as the reference's bucket does.
__global__ __launch_bounds__(64) void k_pip_bucket(const uint32_t* __restrict__ gens,
                                                   const uint16_t* __restrict__ lists,
                                                   const uint32_t* __restrict__ offs, uint32_t m, uint32_t n,
                                                   uint32_t* __restrict__ buckets) {
    const uint32_t b = blockIdx.x, RB = (m + 63) / 64;
    const uint32_t d = (b / RB) % 15 + 1, w = b / (15 * RB);
    const uint32_t row = (b % RB) * 64 + threadIdx.x;
    if (row >= m) return;
    const size_t rw = (size_t)row * 64 + w;
    const uint32_t* o = offs + rw * 16;
    const uint32_t beg = o[d], end = d == 15 ? o[0] : o[d + 1];
    const uint16_t* L = lists + rw * n;
    g1_t acc = g1_zero();
    if (beg < end) {
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
__global__ __launch_bounds__(64) void k_pip_window(const uint32_t* __restrict__ buckets, uint32_t m,
                                                   uint32_t* __restrict__ partials) {
    const size_t t = (size_t)blockIdx.x * 64 + threadIdx.x;
    if (t >= (size_t)m * 64) return;
    g1_t acc = g1_zero(), run = g1_zero();
    for (int b = 15; b >= 1; b--) {
        acc = g1_add(acc, g1_load(buckets + (t * 16 + b) * 36));
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
void launch_pip_bucket(hipStream_t s, const uint32_t* gens, const uint16_t* lists, const uint32_t* offs,
                       uint32_t m, uint32_t n, uint32_t* buckets) {
    const uint32_t rb = (m + 63) / 64;
    hipLaunchKernelGGL(k_pip_bucket, dim3(rb * 960), dim3(64), 0, s, gens, lists, offs, m, n, buckets);
}
void launch_pip_window(hipStream_t s, const uint32_t* buckets, uint32_t m, uint32_t* partials) {
    hipLaunchKernelGGL(k_pip_window, dim3(m), dim3(64), 0, s, buckets, m, partials);
}
void launch_pip_combine(hipStream_t s, const uint32_t* partials, uint32_t m, uint32_t* out) {
    hipLaunchKernelGGL(k_pip_combine, dim3((m + 63) / 64), dim3(64), 0, s, partials, m, out);
}
