// g1.hpp -- host launchers of the G1 commitment kernels (g1.hip).
//
// Pedersen commitment by the bucket method, producing the reference's commit_pippenger
// result byte for byte (commitment.cu:47-103): for every row of a [m][n] scalar table,
// out[row] = sum_i s[row][i] * gens[i] over 4-bit windows of the scalar's raw limbs.
// Points are 144-byte G1Jacobian_t in Montgomery form, array-of-structures.
//
// The reference runs one thread per (row, window) that walks all n generators adding
// each into one of 16 buckets.  Here the work is split where the Jacobian result allows
// it -- each bucket's additions form an independent chain (its generators in ascending
// index order), so one lane runs one (row, window, digit) chain with its bucket in
// registers, after a sort pass has listed each chain's generator indices:
//   pip_sort    one wave per row, lane w = window w: per-digit counts, then the index
//               lists (uint16, generators in ascending order) and their offsets;
//   pip_alias   one wave per row: chains whose index lists are equal (the usual case for
//               small signed scalars, where every window above the witness width holds
//               the list of negative entries) are computed once; lists are matched by a
//               fingerprint and confirmed entry by entry;
//   pip_bucket  each distinct nonempty (row, window, digit) chain once: a long chain on a
//               quad of lanes that share every point addition (latency-bound), a short
//               one on one lane (throughput-bound);
//   pip_window  one quad per (row, window): the running sum over digits 15..1;
//   pip_combine one quad per row: Horner over windows 63..0 (four doublings, one add).
// Quads share each point operation (g1_add_quad, g1_dbl_quad): the window and Horner
// chains are short in total work but sequential, so their latency is what counts.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define ZKH_PIP_MAX_GENS 65536u  // generator indices are stored as uint16

// scalars: FR limb planes (lo: limbs 0-3, hi: limbs 4-7 as uint4 per element), m*n entries
void launch_pip_sort(hipStream_t s, const uint32_t* lo, const uint32_t* hi, uint32_t m, uint32_t n,
                     uint16_t* lists, uint32_t* offs);
void launch_pip_alias(hipStream_t s, const uint16_t* lists, const uint32_t* offs, uint32_t m, uint32_t n,
                      uint16_t* alias);
void launch_pip_bucket(hipStream_t s, const uint32_t* gens, const uint16_t* lists, const uint32_t* offs,
                       const uint16_t* alias, uint32_t m, uint32_t n, uint32_t* buckets);
void launch_pip_window(hipStream_t s, const uint32_t* buckets, const uint32_t* offs, const uint16_t* alias,
                       uint32_t m, uint32_t* partials);
void launch_pip_combine(hipStream_t s, const uint32_t* partials, uint32_t m, uint32_t* out);
// inner-product argument rounds (ipa_prove) of up to ZKH_IPA_MAX_JOBS openings per launch
// (blockIdx.y = job); a, b plain Fr 8 words per entry, g/P points.  A job with h = 0 has
// finished its rounds and is skipped.  x, xi plain; xm, xim in Montgomery form.
#define ZKH_IPA_MAX_JOBS 8
struct IpaJobDev {
    const uint32_t *g, *a, *b, *Q;
    uint32_t *ip, *P, *LR, *g2, *a2, *b2;
    uint32_t h, pad;
    uint32_t x[8], xi[8], xm[8], xim[8];
};
struct IpaBatchDev {
    IpaJobDev j[ZKH_IPA_MAX_JOBS];
};
void launch_ipa_ip(hipStream_t s, const IpaBatchDev& B, uint32_t nj, const uint32_t r2[8]);
void launch_ipa_scale(hipStream_t s, const IpaBatchDev& B, uint32_t nj, uint32_t hmax);
// one tree level: half = h >> shift per job (hmax the largest h)
void launch_ipa_tree(hipStream_t s, const IpaBatchDev& B, uint32_t nj, uint32_t hmax, uint32_t shift);
void launch_ipa_lr(hipStream_t s, const IpaBatchDev& B, uint32_t nj);
void launch_ipa_fold(hipStream_t s, const IpaBatchDev& B, uint32_t nj, uint32_t hmax);
void launch_planes_to_aos(hipStream_t s, const uint32_t* lo, const uint32_t* hi, uint32_t n, uint32_t* out);
// out[i] = base[i % nb] * s[i] (G1Jacobian_mul, raw scalar bits)
// a scalar passed by value to a kernel: 8 plain little-endian words
struct G1Scalar {
    uint32_t v[8];
};
// out[i] = b[i] + a[i] * sc (hb_addmul, mul_first = false)
void launch_g1_addmul(hipStream_t s, const uint32_t* a, const G1Scalar& sc, const uint32_t* b, uint32_t n,
                      uint32_t* out);
void launch_g1_mul(hipStream_t s, const uint32_t* base, uint32_t nb, const uint32_t* lo, const uint32_t* hi,
                   uint32_t n, uint32_t* out);
