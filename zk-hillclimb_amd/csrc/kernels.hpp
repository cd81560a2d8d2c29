// kernels.hpp -- launch wrappers for the gfx950 kernels in kernels.hip.
//
// All wrappers enqueue on the given stream and return immediately.  Device tables of
// full field elements use the limb-quad layout (FrPlanes: lo/hi uint4 planes of `cap`
// entries); small vectors (eq factor tables, partial sums) use the reference's AoS Fr_t
// layout (8 consecutive uint32 per element).
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace zkh {

struct DevPlanes {
    uint32_t* base;  // lo plane at base, hi plane at base + 4*cap uint32
    uint32_t cap;
    uint32_t* lo() const { return base; }
    uint32_t* hi() const { return base + 4 * (size_t)cap; }
};

// Round completion without a host synchronisation: every block of a publishing kernel
// writes its K partial sums to `part` (device) and the first block of each job its layout
// (first block, blocks, K) to `layout`; a one-block kernel queued right behind it
// (launch_publish) adds each job's partials, writes the job's K sums to host_out (coherent
// pinned host memory) and stores `seq` into *host_flag (system-scope release), which the
// host spins on.  The kernel boundary orders the partials before their reads, so the
// round kernel's blocks take no fence and no atomic.
struct Publish {
    uint32_t* part;       // device, [total blocks][K] AoS
    uint32_t* layout;     // device, 3 words per job
    uint32_t* host_out;   // pinned, [njobs][K] AoS
    uint32_t* host_flag;  // pinned
    uint32_t seq, njobs;
};
// the sums of a publishing kernel's jobs to the host (queue right behind that kernel)
void launch_publish(hipStream_t s, const Publish& P);

// A table in a fused fold+evaluate round: read from src; folded entries go to dst (which
// may be src itself).  The first fold of a caller-owned table targets a scratch copy.
struct Tab {
    DevPlanes src;
    DevPlanes dst;
};

// One eq weighting over the first 2^K indices: the device weight of index i is
// Elo[i & 1023] * Ehi[i >> 10], with Elo the eq table of u[0..10) and Ehi that of
// u[10..kmax) (both Montgomery form, built once per proof; missing variables count as
// u_t = 0).  For i < 2^K this is eq(i, u[0..K)) * prod_{t=K}^{kmax-1} (1 - u_t); the host
// multiplies each round's sums by the inverse of that product.
struct EqW {
    const uint32_t* elo;  // AoS, 1024 entries
    const uint32_t* ehi;  // AoS, 2^(kmax-10) entries (one entry when kmax <= 10)
    uint32_t K;           // variables of this round's weighting
};

// ---- conversions / layout ----
void launch_i32_to_planes(hipStream_t s, const int32_t* in, uint32_t n, DevPlanes out);
void launch_i64_to_planes(hipStream_t s, const int64_t* in, uint32_t n, DevPlanes out);
void launch_aos_to_planes(hipStream_t s, const uint32_t* aos, uint32_t n, DevPlanes out);
// *bad (zeroed by the caller) += entries of aos that are not below r
void launch_count_noncanonical(hipStream_t s, const uint32_t* aos, uint32_t n, uint32_t* bad);
void launch_planes_to_aos(hipStream_t s, DevPlanes in, uint32_t n, uint32_t* aos);
// out[0] = max |in[i]|, out[1] |= 1 when some entry is not 1 (both zeroed by the caller)
void launch_absmax_i32(hipStream_t s, const int32_t* in, uint32_t n, uint32_t* out);
void launch_absmax_i64(hipStream_t s, const int64_t* in, uint32_t n, unsigned long long* out);
void launch_transpose_i32(hipStream_t s, const int32_t* in, uint32_t rows, uint32_t cols,
                          int32_t* out);

// ---- eq tables ----
// out[b] = prod_t fac[2t + bit_t(b)] (Montgomery form) for b < n, AoS; K = #factors
void launch_eq_mont(hipStream_t s, const uint32_t* fac, uint32_t K, uint32_t n, uint32_t* out);
// two eq tables in one launch (the small Elo, Ehi a proof builds first)
void launch_eq_mont2(hipStream_t s, const uint32_t* fac0, uint32_t K0, uint32_t n0, uint32_t* out0,
                     const uint32_t* fac1, uint32_t K1, uint32_t n1, uint32_t* out1);

// the same with the factors (1 - u_t, u_t) as launch arguments: table 0 from factors [0, K0),
// table 1 from [K0, K0 + K1) (plain form when plain1); false (nothing launched) when a table
// exceeds the four-lanes form's size or the factors do not fit
#define ZKH_FAC_ARG_VARS 32
struct FacArg {
    uint32_t w[ZKH_FAC_ARG_VARS * 16];
};
bool launch_eq_mont2_ka(hipStream_t s, const FacArg& f, uint32_t K0, uint32_t n0, uint32_t* out0, uint32_t K1,
                        uint32_t n1, uint32_t* out1, bool plain1 = false);

// ---- dot products / sums (block partials, AoS, summed on the host) ----
// partial[b] = sum montmul(a_i, b_i) over the block's range (carries 2^-256)
uint32_t launch_dot_planes(hipStream_t s, DevPlanes a, DevPlanes b, uint32_t n, Publish pub);
// sums of a_t b_t over MSB pairs for t = 0, 1, 2 (three published sums)
uint32_t launch_prod_round(hipStream_t s, DevPlanes a, DevPlanes b, uint32_t h, Publish pub);
uint32_t launch_sum_planes(hipStream_t s, DevPlanes a, uint32_t n, Publish pub);

// ---- generic MLE pieces ----
// out[o*W + w] = sum_{c < C} montmul(E_m[c], t[(o*C + c)*W + w])  (t as FR planes)
void launch_partial_me_planes(hipStream_t s, DevPlanes t, uint32_t O, uint32_t C, uint32_t W,
                              const uint32_t* E, DevPlanes out);
void launch_partial_me_i32(hipStream_t s, const int32_t* t, uint32_t O, uint32_t C, uint32_t W,
                           const uint32_t* E, DevPlanes out);
void launch_partial_me_i64(hipStream_t s, const int64_t* t, uint32_t O, uint32_t C, uint32_t W,
                           const uint32_t* E, DevPlanes out);
// the same over a [O, C, W] view of a tensor with only n stored entries (entries at index
// >= n read as zero); kind 0: FR planes (t, cap), 1: int32, 2: int64
void launch_partial_me_window(hipStream_t s, int kind, const void* t, uint32_t cap, uint32_t n,
                              uint32_t O, uint32_t C, uint32_t W, const uint32_t* E, DevPlanes out);
// padding (FrTensor::pad): dimension d of shape[d] entries padded to 2^lg[d]
struct PadDims {
    uint32_t nd;
    uint32_t shape[8];
    uint32_t lg[8];
};
void launch_pad(hipStream_t s, DevPlanes src, const PadDims& pd, uint32_t total, const uint32_t* pad_host,
                DevPlanes out);
// tLookupRange table of N entries: low + min(i, len - 1)
void launch_range_table(hipStream_t s, int32_t low, uint32_t len, uint32_t N, DevPlanes out);
void launch_range_table_i32(hipStream_t s, int32_t low, uint32_t len, uint32_t N, int32_t* out);
// zkip / zkip_stacked round over a [N, D] layout (rows n, n + Nh paired, rows >= N zero,
// weights E[n] Montgomery AoS of Nh entries, or 1 when E is null): publishes c0, c1, c2
// (x 2^-256) as job 0 of pub; the fold binds the top row bit in place with v (Montgomery)
uint32_t launch_stk_round(hipStream_t s, DevPlanes a, DevPlanes b, uint32_t N, uint32_t D, uint32_t Nh,
                          const uint32_t* E, Publish pub);
void launch_stk_fold(hipStream_t s, DevPlanes a, DevPlanes b, uint32_t N, uint32_t D, uint32_t Nh,
                     const uint32_t* v_m_host);
// rescaling witness: q = (x - rem) / sf, rem = ((x + sf/2) mod sf) - sf/2 for x of the given
// kind (0: FR planes read through scalar_to_long, 1: int32, 2: int64)
void launch_rescale(hipStream_t s, int kind, const void* x, uint32_t cap, uint32_t n, int64_t sf,
                    int64_t* q, int64_t* rem);
// MSB fold dst[i] = src[i] + v*(src[i+h]-src[i]), i < h (v in Montgomery form)
void launch_fold(hipStream_t s, Tab t, uint32_t h, const uint32_t* v_m_host);
// an operand read in place: kind 0 FR planes (p, cap), 1 int32, 2 int64 (field view)
struct Src {
    int kind;
    const void* p;
    uint32_t cap;
};
// out = a + c b (c plain and in Montgomery form; an int32 b takes the 32-bit multiply)
void launch_axpy(hipStream_t s, Src a, const uint32_t* c_host, const uint32_t* c_m_host, Src b, uint32_t n,
                 DevPlanes out);
void launch_hadamard(hipStream_t s, Src a, Src b, uint32_t n, DevPlanes out);
// int32 a (.) b into the exact int64 products
void launch_hadamard_i64(hipStream_t s, const int32_t* a, const int32_t* b, uint32_t n, int64_t* out);

// ---- logUp ----
void launch_lu_count_planes(hipStream_t s, DevPlanes S, uint32_t n, const uint32_t* low_host,
                            uint32_t N, uint32_t* counts, uint32_t* bad);
void launch_lu_count_i32(hipStream_t s, const int32_t* S, uint32_t n, int32_t low, uint32_t N,
                         uint32_t* counts, uint32_t* bad);
void launch_counts_to_planes(hipStream_t s, const uint32_t* counts, uint32_t N, DevPlanes m);
// Multiplicities without global atomics (tlookup.cu:10-48, :414-433 semantics): every
// index idx = limb 0 of (S - low) is bucketed by idx >> ZKH_HIST_BITS (16,384 bins per
// bucket, one 64 KB LDS histogram); the indices are partitioned by bucket (tile counts,
// per-bucket prefixes, a scatter with LDS cursors); each work slot (at most ZKH_HIST_CHUNK
// indices of one bucket, so a skewed bucket such as the zero padding spreads over many
// blocks) counts in LDS and stores its histogram; m[j] is the sum of bin j over its
// bucket's slots, written as field elements.  With one bucket (N <= 16,384) the slots read
// the input directly.  An index >= N sets *bad.  N <= 2^24 (1,024 buckets).
#define ZKH_HIST_BITS 14
#define ZKH_HIST_BINS (1u << ZKH_HIST_BITS)
#define ZKH_HIST_CHUNK 16384u
#define ZKH_HIST_TILE 4096u
#define ZKH_HIST_MAX_BUCKETS 1024u
struct HistArgs {
    Src S;          // int32 or FR planes
    uint32_t n;     // entries of S
    int32_t low;    // table offset (int32 inputs)
    uint32_t low_fr[8];  // the same as a field element (FR inputs)
    uint32_t N;     // table size
    uint32_t nbuckets, ntiles, max_slots;
    uint32_t* tile_cnt;     // [nbuckets][ntiles]: counts, then in-row exclusive prefixes
    uint32_t* bucket_info;  // [nbuckets][4]: start, total, first slot, slots
    uint32_t* work;         // [max_slots][4]: bucket, begin, count, -
    uint32_t* nslots;       // one word
    uint16_t* part;         // n partitioned low index bits
    uint32_t* slot_hist;    // [max_slots][ZKH_HIST_BINS]
    uint32_t* bad;          // set to tag when an index is outside the table
    uint32_t tag;
};
// scratch words needed by launch_hist for these sizes (tile_cnt .. slot_hist, 16-byte aligned parts)
size_t hist_scratch_bytes(uint32_t n, uint32_t N);
// lays HistArgs' buffers out in `scratch` (hist_scratch_bytes bytes) and enqueues the passes
// (m32 set: the counts go to m32 as int32 instead of m's planes)
void launch_hist(hipStream_t s, HistArgs a, void* scratch, DevPlanes m, int32_t* m32);

void launch_lu_map_planes(hipStream_t s, DevPlanes S, uint32_t n, const uint32_t* low_host,
                          DevPlanes mapped, DevPlanes out);
void launch_lu_map_i32(hipStream_t s, const int32_t* S, uint32_t n, int32_t low,
                       Src mapped, uint32_t N, DevPlanes out);
// the same into int32 entries for an int32 mapped table (out[i] = 0 outside the table)
void launch_lu_map_to_i32(hipStream_t s, Src S, uint32_t n, const uint32_t* low_host, const int32_t* mapped,
                          uint32_t N, int32_t* out);
// tuple lookup, j = (G[i] - low).limb0: comb[i] = G[i] + r mapped[j]; A[i] = Binv[j] where
// T[j] == G[i]; flags[0] = tag (j >= N), flags[1] = tag (T[j] != G[i]); r plain and in
// Montgomery form;
// tlen > 0: T is the range table low + min(j, tlen - 1) (not read); seq_s: `mapped` is
// S = mapped[(G - low).limb0] (n entries), read at i; binv_aos (optional): Binv as AoS
// (32 contiguous bytes per entry: one cache line per random read instead of one per plane)
void launch_lu_tuple_gather(hipStream_t s, Src G, uint32_t n, const uint32_t* low_host, Src T, uint32_t tlen,
                            Src mapped, int seq_s, uint32_t N, const uint32_t* r_host, const uint32_t* r_m_host,
                            DevPlanes Binv, const uint32_t* binv_aos, DevPlanes comb, DevPlanes A, uint32_t* flags,
                            uint32_t tag);
// the same for a plain range lookup: A[i] = Binv[j] (j = (S[i] - low).limb0) where T[j] == S[i]
void launch_lu_range_gather(hipStream_t s, Src S, uint32_t n, const uint32_t* low_host, Src T, uint32_t tlen,
                            uint32_t N, DevPlanes Binv, DevPlanes A, uint32_t* flags, uint32_t tag);
// A[i] = 1/(S[i]+beta) (0 -> 0), Montgomery's batched inversion with M(a, b) = a b 2^-256
// products of the plain values: pass 1 writes the running products P_j to A, per-thread
// "other threads" products to `others` (inv_blocks(n)*256 AoS) and block totals to
// blockprod (inv_blocks(n) AoS); k_inv_blocks writes others_blk[b] = the M-product of the
// other blocks' totals and publishes the grand product G (job 0 of pub); the host computes
// the plain inverse 1/G once; pass 2 writes the plain inverses into A given inv_total = 1/G.
uint32_t inv_blocks(uint32_t n);
// zflag: a device word that pass 1 sets to tag when some S[i] + beta is zero (a word no
// earlier call left at this tag); k_inv_blocks publishes (zflag == tag) as word 8 of
// pub.host_out, after G
void launch_inv_pass1(hipStream_t s, DevPlanes S, uint32_t n, const uint32_t* beta_host,
                      DevPlanes A, uint32_t* others, uint32_t* blockprod, uint32_t* zflag, uint32_t tag);
void launch_inv_blocks(hipStream_t s, const uint32_t* blockprod, uint32_t nb, uint32_t* others_blk,
                       Publish pub, const uint32_t* zflag, uint32_t tag);
// 1/G from the host (inv_total_host) or, when invp is given, from device words invp[0..8)
// written by a relay (invp[8] != 0: return at once); aos (optional): the inverses also as
// AoS (n entries)
void launch_inv_pass2(hipStream_t s, DevPlanes S, uint32_t n, const uint32_t* beta_host,
                      DevPlanes A, const uint32_t* others, const uint32_t* others_blk,
                      const uint32_t* inv_total_host, const uint32_t* invp, uint32_t* aos = nullptr);
// Round kernels take the previous round's challenge (Montgomery form) either from the host
// at launch (v_m_host) or, when vmp is given, from device words vmp[0..8) written by a relay
// (launch_relay) that runs between the previous round and this one; vmp[8] != 0 makes the
// kernel return at once (the host abandoned the proof).
// phase-1 round over A, S (size n): sums e*a0*s0, e*a1*s1, e*da*ds (x 2^-256), a0, a1
// inv: A is 1/(S + beta) entry-wise and no fold is owed: sums 0 and 1 become sum_{a != 0} w
// with w = e 2^256 (sum e after one Montgomery reduction), two products per pair fewer
// derive (with fold): the sums at 1 are left out: e*a0*s0, e*da*ds, a0 (see kernels.hip)
uint32_t launch_lu_phase1(hipStream_t s, Tab A, Tab S, uint32_t n, int fold,
                          const uint32_t* v_m_host, const uint32_t* vmp, const uint32_t* beta_host, EqW eq,
                          Publish pub, int inv, int derive);
// the first (unfolded) round of phase 1 (phase2 = 0: A, S only) or phase 2 when A = 1/(S + beta)
// and B = 1/(T + beta) have no zero entry: sum w a (s + beta) and sum w b (t + beta) are
// sum eq = 1 and not formed.  Job 0 (A, S): w da ds (x 2^-256), a0, a1; job 1 (B, T, m):
// w db dt (x 2^-256), m0 b0, m1 b1, dm db (x 1); m read as int32 when m32 is set.
uint32_t launch_lu_first_nz(hipStream_t s, Tab A, Tab S, Tab B, Tab T, Tab m, uint32_t n, int phase2, EqW eq,
                            Publish pub, const int32_t* m32);
// phase-2 round over A, S, B, T, m as two launches publishing jobs 0 (A, S: 5 sums) and
// 1 (B, T, m: 6 sums) of `pub` (made for 2 jobs; see kernels.hip)
// inv_as / inv_btm: A = 1/(S + beta) / B = 1/(T + beta) with that group's fold not owed, as
// inv of launch_lu_phase1 (sums 0, 1 of the group then carry 2^256 instead of 2^-256); with
// inv_btm the m b sums (3..5 of job 1) are exact (x 1)
// derive: the folding groups leave out their sums at 1: job 0 publishes 3 sums (w*a0*s0,
// w*da*ds, a0), job 1 (when it folds) 4 (w*b0*t0, w*db*dt, m0*b0, dm*db)
// m32: m read as int32 entries (not yet folded) instead of m's source planes
uint32_t launch_lu_phase2(hipStream_t s, Tab A, Tab S, Tab B, Tab T, Tab m, uint32_t n,
                          int fold_as, int fold_btm,
                          const uint32_t* v_m_host, const uint32_t* vmp, const uint32_t* beta_host, EqW eq,
                          Publish pub, int inv_as, int inv_btm, int derive,
                          const int32_t* m32);

// ---- Hadamard ----
// With derive (folding rounds only) each Hadamard round kernel leaves out its sum at t = 1,
// which the host takes from the previous round's claim.
// generic: sums_t = sum E_t*S_t*U_t, t = 0..3 (x 2^-512); derive: t = 0, 2, 3
uint32_t launch_hp_round(hipStream_t s, Tab E, Tab S, Tab U, uint32_t n,
                         int fold, const uint32_t* v_m_host, const uint32_t* vmp, Publish pub, int derive);
// generic with U = 1 everywhere: sums e0*s0, e1*s1, de*ds (x 2^-256); U is not touched;
// derive: e0*s0, de*ds; s_int (first round, S of int32 values): the sums exact (x 1);
// s32: S read as int32 entries (not yet folded) instead of its source planes
uint32_t launch_hp_round_ones(hipStream_t s, Tab E, Tab S, uint32_t n, int fold, const uint32_t* v_m_host,
                              const uint32_t* vmp, Publish pub, int derive, int s_int, const int32_t* s32);
// eq-specialised: sums w*s0*u0, w*s1*u1, w*ds*du with w = eq(i,u_) (x 2^-256 when folding,
// x 2^256 in the first round); derive: w*s0*u0, w*ds*du
uint32_t launch_hp_eq_round(hipStream_t s, Tab S, Tab U, uint32_t n, int fold,
                            const uint32_t* v_m_host, const uint32_t* vmp, EqW eq, Publish pub, int derive,
                            const int32_t* s32, const int32_t* u32);
// sum_i eq(i, u[0..K)) * S[i] over integer entries (kind 1 int32, 2 int64), x 2^256
uint32_t launch_eq_sum_int(hipStream_t s, int kind, const void* S, uint32_t n, EqW eq, Publish partial);
// sum_i eq(i, u[0..K)) * S[i] * U[i] over i < n (x 2^-256); U may be null (then S only, x 1)
uint32_t launch_eq_sum(hipStream_t s, DevPlanes S, const DevPlanes* U, uint32_t n, EqW eq,
                       Publish pub);

// setup of the allocation-free MLE evaluation: copies `words` factor words (passed by value)
// to fac_dst and zeroes ncnt words at cnt (its publish layout), all inside caller-provided
// device memory
#define ZKH_STATIC_MAX_VARS 24
struct StaticFacArg {
    uint32_t w[ZKH_STATIC_MAX_VARS * 16];  // (1 - u_t, u_t) per variable, Montgomery form
};
// the Montgomery-multiply rate probe: `blocks` x kFrMulPeakThreads threads, four independent
// chains of `iters` products per thread; out[thread] receives a digest of the chains
constexpr uint32_t kFrMulPeakThreads = 256;
void launch_fr_mul_peak(hipStream_t s, uint32_t blocks, uint32_t iters, uint32_t* out, hipEvent_t t0, hipEvent_t t1);
void launch_static_setup(hipStream_t s, const StaticFacArg& fac, uint32_t words, uint32_t* fac_dst,
                         uint32_t* cnt, uint32_t ncnt);

uint32_t grid_for(uint32_t work_items, uint32_t per_block, uint32_t max_blocks);


// ---- batched (multi-job) launches: descriptors live in device memory; each job's
// blocks are contiguous from blk_begin ----
struct fr_arg {
    uint32_t v[8];
};
struct EqTabDesc {  // eq table over K variables, n entries, AoS out (Montgomery unless plain)
    const uint32_t* fac;
    uint32_t* out;
    uint32_t K, n, blk_begin, plain;
};
// out[b] = tlo_m[b mod 2^klo] * thi_p[b >> klo]: the plain eq table from two small ones
void launch_eq_outer(hipStream_t s, const uint32_t* tlo_m, const uint32_t* thi_p, uint32_t klo,
                     uint32_t n, DevPlanes out);
struct EqDotDesc {  // partial[c*N+i] = sum_{k in rows [c*kchunk, (c+1)*kchunk)} (M[k*N+i] + 2^bits) e_k
    const void* M;
    const uint32_t* E;
    uint32_t* partial;
    uint32_t K, N, kchunk, bits, blk_begin;
    uint32_t variant;  // 0: int32 elements, 1: int64 elements (pieces fixed by the launch)
};
struct SumChunksDesc {
    const uint32_t* partial;
    uint32_t* out_lo;  // planes output (when E == null)
    uint32_t* out_hi;
    const uint32_t* E;  // Montgomery eq table: dot mode (block partials into dot)
    uint32_t* dot;
    uint32_t nch, N, Npad, blk_begin;
    fr_arg corr;
};
struct ZkipDesc {
    uint32_t* a_lo;
    uint32_t* a_hi;
    uint32_t* b_lo;
    uint32_t* b_hi;
    uint32_t* partial;  // 3 Fr per block
    uint32_t n, fold, blk_begin, pad_;
    fr_arg vm;  // challenge of the fold, Montgomery form
};
// t0 / t1: optional events stamped at the start / end of the launch (hipExtLaunchKernel)
void launch_eq_mont_multi(hipStream_t s, const EqTabDesc* d_dev, uint32_t nd, uint32_t nblocks,
                          hipEvent_t t0 = nullptr, hipEvent_t t1 = nullptr);
// eq-weighted integer reductions; wide = 0: int32 with |v| < 2^19 (one 20-bit piece, chunks
// <= 2048 rows) and int64 with |v| < 2^43 (two 22-bit pieces); wide = 1: any int32 (two
// 22-bit pieces) and any int64 (three); chunks <= 512 rows for 22-bit pieces
void launch_eqdot_multi(hipStream_t s, int wide, const EqDotDesc* d_dev, uint32_t nd, uint32_t nblocks,
                        hipEvent_t t0 = nullptr, hipEvent_t t1 = nullptr);
// eq-weighted reductions of full field-element tables (the FrTensor inputs of zkob_fc,
// zkob_fc.cu:276-277): column mode (rowmode = 0) partial[c*N+i] = sum_{k in rows
// [c*kchunk, (c+1)*kchunk) of K} M[k*N+i] e_k, as for the integer reductions; row mode
// (rowmode = 1) partial[i] = sum_{k < K} M[i*K+k] e_k, one wave per output i (row-major W
// reduced over OUT).  M: limb-quad planes (lo, hi); E: Montgomery eq table, AoS; partials
// plain.
struct EqDotFrDesc {
    const uint32_t* lo;
    const uint32_t* hi;
    const uint32_t* E;
    uint32_t* partial;
    uint32_t K, N, kchunk, blk_begin, rowmode, pad_;
};
void launch_eqdot_fr_multi(hipStream_t s, const EqDotFrDesc* d_dev, uint32_t nd, uint32_t nblocks,
                           hipEvent_t t0 = nullptr, hipEvent_t t1 = nullptr);
void launch_sum_chunks_multi(hipStream_t s, const SumChunksDesc* d_dev, uint32_t nd, uint32_t nblocks,
                             hipEvent_t t0 = nullptr, hipEvent_t t1 = nullptr);
#define ZKH_MAX_BATCH 32
struct ZkipBatch {  // passed by value as the kernel argument (<= 2.1 KB)
    ZkipDesc d[ZKH_MAX_BATCH];
    uint32_t nd;
};
void launch_zkip_round_multi(hipStream_t s, const ZkipBatch& b, uint32_t nblocks, Publish pub);
void launch_fold_last_multi(hipStream_t s, const ZkipBatch& b);

// ---- witness GEMM: Y = X W (+ bias) over the integers, exact ----
// X [B][IN] int32, WT [OUT][IN] int32 (W transposed, the registered-weights layout), bias
// [OUT] int64 or null, Y [B][OUT] int64.  f64: fp64 matrix cores, exact while every partial
// sum stays below 2^53 (the caller checks the magnitude bounds); otherwise int64 VALU.
void launch_matmul_i32(hipStream_t s, const int32_t* X, const int32_t* WT, const int64_t* bias, uint32_t B,
                       uint32_t IN, uint32_t OUT, int64_t* Y, int f64);
void launch_widen_i32(hipStream_t s, const int32_t* in, uint32_t n, int64_t* out);
// scalar_to_long of every entry (FrTensor::save_long, fr-tensor.cu:210-218)
void launch_to_long(hipStream_t s, DevPlanes p, uint32_t n, int64_t* out);

// ---- persistent matmul round loop ----
// Each job's tables a, b (n = 2^L entries) are spread cyclically over nb = 2^lgnb blocks
// (block l holds entries l + nb*k in LDS), so the pairs (i, i + m/2) of every round with
// m >= 2*nb stay inside one block.  Messages between host and device are 16-byte quads
// [seq, w, w, w] (zkh_quad_* below), each written with one 16-byte store: a message is
// complete when all its quads show the expected seq.  A block with m >= 4 local entries
// serves two rounds per message: over the halves L = T[0, m/2), H = T[m/2, m), D = H - L
// and the quarter index j < m/4 (j' = j + m/4) it publishes nine sums (each x 2^-256,
// ZKH_MSG_PAIR words): L_j.L_j, H_j.H_j, D_j.D_j, the same three at j', and
// (L_j' - L_j).(L_j' - L_j), (H_j' - H_j).(H_j' - H_j), (D_j' - D_j).(D_j' - D_j), where
// u.v means u_a * u_b over the two tables.  They give this round's sums and, as quadratics
// in its challenge x, the next round's sums over the table folded by x; the host derives
// both challenges and answers with the four weights (1-x)(1-y), x(1-y), (1-x)y, xy
// (Montgomery form, 32 words) of the double fold T[k] <- w00 T[k] + w01 T[k + m/2] +
// w10 T[k + m/4] + w11 T[k + 3m/4].  With m = 2 the block publishes one round's sums
// (a0b0, a1b1, da*db: ZKH_MSG_ONE words) and receives the challenge (8 words); with m = 1
// its folded entries a[0], b[0] (ZKH_MSG_FINAL words), then exits.  Message s carries seq
// s (1, 2, ...) both ways.  A command quad with seq ZKH_QUIT makes the job's blocks exit;
// a block that waits longer than `deadline` ticks of the 100 MHz clock sets *err and
// exits.  Slot words 128..131 hold the block's clock at its last message (publication, and
// receipt of the previous command) and words 132 + 2s, 133 + 2s (s < 14) the same per
// message s (tracing only); words 0..127 carry messages of up to 32 quads.
#define ZKH_QUIT 0xffffffffu
#define ZKH_PSLOT 160  // words per block slot and per job command area
#define ZKH_PSTAMP 128  // first clock-stamp word of a slot
#define ZKH_MSG_PAIR 72
#define ZKH_MSG_ONE 24
#define ZKH_MSG_FINAL 16
// quad messages: data word i lives at 4*(i/3) + 1 + i%3, quad q's seq at 4*q
__host__ __device__ inline uint32_t zkh_quad_word(uint32_t i) { return 4 * (i / 3) + 1 + i % 3; }
__host__ __device__ inline uint32_t zkh_quad_count(uint32_t nwords) { return (nwords + 2) / 3; }
#define ZKH_PLS_MAX 512u  // entries per block and table (32 KiB of LDS for both tables)

// ---- persistent Hadamard rounds (the small rounds of zkh_hp_prove / zkh_hp_prove_eq) ----
// Tables S, U (and E) of n entries (after the fold owed by the last launched round, applied
// while they load into LDS) spread cyclically over nb = 2^lgnb blocks as in the matmul
// loop.  Per local round with m entries per block each block publishes, over its pairs
// (k, k + m/2), sum_k eq_w(g) S_t[k] U_t[k] for t = 0..3 (g = block + nb*k the global pair
// index, eq_w the device eq weight of the per-round kernels; x 2^-256) or, with E,
// sum_k E_t[k] S_t[k] U_t[k] (x 2^-512): 32 words, 11 quads.  It then waits for the
// challenge (Montgomery form, 3 quads) and folds the tables; with m = 1 it publishes S[0],
// U[0] (and E[0]) (16 or 24 words) and exits.  Message s carries seq s.  Slot layout,
// ZKH_QUIT and the deadline as in ZkipPersist.
// With `two` set (eq mode, or an E table with U all ones) a message covers two rounds while
// m >= 4: over its cells c < m/4 (entries c + j m/4, j = 2 y1 + y2, y1 the first round's
// variable) each block publishes sum_c eq_w(g_c) S_c(y) U_c(y) (eq mode, x 2^-256) or
// sum_c E_c(y) S_c(y) (x 2^-256) at the nine points y of {0, 1, inf}^2, point 3 a + b
// (inf: the difference along that axis), ZKH_HP_MSG2 words, and receives the four weights
// of the double fold as ZkipPersist does (32 words).
struct HpPersist {
    const uint32_t* s_lo;
    const uint32_t* s_hi;
    const uint32_t* u_lo;
    const uint32_t* u_hi;
    const uint32_t* e_lo;  // an explicit E table (zkh_hp_prove), or null: the eq weights
    const uint32_t* e_hi;
    const uint32_t* elo;  // eq factor tables (EqW)
    const uint32_t* ehi;
    uint32_t* out;  // pinned host, nb slots
    uint32_t* cmd;  // pinned host, one command area
    uint32_t* err;
    unsigned long long deadline;
    fr_arg vm;        // the owed fold's challenge (Montgomery form) when fold != 0
    const uint32_t* vmp;  // or, when given, device words from a relay (vmp[8] != 0: return at once)
    uint32_t n, lgnb, fold, two;  // fold: entries g and g + n of the sources fold into g
};
#define ZKH_HP_MSG 32
#define ZKH_HP_MSG2 72

// ---- persistent logUp phase-2 rounds (the small rounds of zkh_lu_prove) ----
// Tables A, S, B, T, m of n entries (n <= N: phase 2), each group (A, S) / (B, T, m) after
// the fold it owes, spread cyclically over nb = 2^lgnb blocks as in the matmul loop.  Per
// local round with m entries per block each block publishes its 11 sums over the pairs
// (k, k + m/2), in the order of the per-round kernels' jobs 0 and 1: sum w a0 (s0 + beta),
// w a1 (s1 + beta), w da ds, sum a0, sum a1, sum w b0 (t0 + beta), w b1 (t1 + beta),
// w db dt, m0 b0, m1 b1, dm db (products x 2^-256; w = eq_w(g) of the global pair index;
// 88 words, 30 quads), waits for the challenge (3 quads) and folds all five tables; with
// m = 1 it publishes A[0], S[0], B[0], T[0], m[0] (40 words) and exits.  Slots of
// ZKH_LU_PSLOT words (clock stamps from word ZKH_LU_PSTAMP); ZKH_QUIT and the deadline as in
// ZkipPersist.
// With `two` set a message covers two rounds while m >= 4: over its cells c < m/4 (entries
// c + j m/4, j = 2 y1 + y2, y1 the first round's variable) each block publishes, at the
// nine points y of {0, 1, inf}^2 (point 3 a + b, inf: the difference along that axis),
// sum_c W_c A(y) (S(y) + beta'), sum_c W_c B(y) (T(y) + beta'), sum_c m(y) B(y) (x 2^-256;
// W_c = eq_w(g_c), beta' = beta at the points without inf, 0 at the others), then sum_c A
// at the four corners j (ZKH_LU_MSG2 words), and receives the four weights of the double
// fold as ZkipPersist does (32 words).
struct LuPersist {
    const uint32_t* lo[5];  // A, S, B, T, m: sources (limb-quad planes)
    const uint32_t* hi[5];
    const uint32_t* elo;  // eq factor tables (EqW)
    const uint32_t* ehi;
    uint32_t* out;  // pinned host, nb slots
    uint32_t* cmd;  // pinned host, one command area
    uint32_t* err;
    unsigned long long deadline;
    fr_arg vm;    // the owed folds' challenge (Montgomery form)
    const uint32_t* vmp;  // or, when given, device words from a relay (vmp[8] != 0: return at once)
    fr_arg beta;  // plain
    uint32_t n, lgnb, fold_as, fold_btm;  // fold_*: that group's sources hold 2n entries
    uint32_t two, pad_[3];
};
#define ZKH_LU_MSG 88
#define ZKH_LU_MSG2 248
#define ZKH_LU_PSLOT 384   // words per block slot and command area of the logUp loop
#define ZKH_LU_PSTAMP 352  // first clock-stamp word of its slots
hipError_t launch_lu_persist(hipStream_t s, const LuPersist& p);
// one thread: word[0..nwords) (when word is given) to host_word, then seq to *flag (pinned
// host memory, system scope): the completion flag of everything queued before it on the stream
void launch_fence(hipStream_t s, uint32_t* flag, uint32_t seq, const uint32_t* word, uint32_t nwords,
                  uint32_t* host_word);
// One wave that waits (as a persistent block waits for its command) until the three quads
// at cmd carry seq `want`, then writes their eight data words to vmp[0..8) and 0 to vmp[8];
// on ZKH_QUIT or past `deadline` (100 MHz ticks; then *err = 1) it writes 1 to vmp[8].
void launch_relay(hipStream_t s, const uint32_t* cmd, uint32_t want, uint32_t* err, unsigned long long deadline,
                  uint32_t* vmp);
// at most 16 blocks of ZKH_PLS_MAX entries; returns the HIP status of the launch
hipError_t launch_hp_persist(hipStream_t s, const HpPersist& p);

struct ZkipPJob {
    const uint32_t* a_lo;
    const uint32_t* a_hi;
    const uint32_t* b_lo;
    const uint32_t* b_hi;
    uint32_t* out;  // pinned host, nb slots
    uint32_t* cmd;  // pinned host, one command area
    uint32_t n, lgnb, blk_begin, pad_;
};
struct ZkipPersist {  // passed by value as the kernel argument
    ZkipPJob d[ZKH_MAX_BATCH];
    uint32_t* err;
    unsigned long long deadline;
    uint32_t nd, ls_max;
};
// at most 256 blocks; returns the HIP status of the launch
hipError_t launch_zkip_persist(hipStream_t s, const ZkipPersist& p, uint32_t nblocks);
}  // namespace zkh
