/*
 * zkh.h -- C ABI of the MI355X (gfx950) prover hot path for zk-hillclimb's BLS12-381
 * Fr sumchecks: MLE fold/bind, the matmul (zkip) sumcheck, the logUp (tLookup)
 * lookup sumcheck and the eq-weighted Hadamard sumcheck.
 *
 * Conventions (shared by every entry point):
 *  - A field element crosses the ABI as the reference's Fr_t: 8 little-endian uint32
 *    limbs, canonical residue in [0, r), plain integer view (zkllm-src/fr-tensor.cuh:15,
 *    bls12-381.cuh:116-120).  "Fr array" below means n*8 uint32.
 *  - Return codes: ZKH_OK 0, ZKH_EARG 1 (bad dims/args, as the reference's
 *    std::runtime_error on dimension mismatch), ZKH_EROUND 2 (prover-side round or
 *    terminal inconsistency: "witness bug" in the reference), ZKH_EDEV 3 (HIP error).
 *    zkh_last_error() gives the message of the last failure on that context.
 *  - A context owns one HIP stream (default priority) on one device, its scratch
 *    memory and its pinned host staging.  Calls on one context are serialised by the
 *    caller; independent contexts may be driven from different host threads, which is
 *    how independent sumchecks (e.g. the 7 matmuls of a layer) overlap.
 *  - Transcripts are the reference's SHA-256 Fiat-Shamir transcript
 *    (fs_transcript.hpp:115-166): a 32-byte state owned by the caller.
 */
#ifndef ZKH_H
#define ZKH_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ZKH_OK 0
#define ZKH_EARG 1
#define ZKH_EROUND 2
#define ZKH_EDEV 3

typedef struct zkh_ctx zkh_ctx;
typedef struct zkh_tensor zkh_tensor;
typedef struct zkh_g1 zkh_g1; /* device array of G1 points (G1TensorJacobian) */

/* element kinds held by a tensor */
#define ZKH_KIND_FR 0  /* full field elements (device: two uint4 limb planes) */
#define ZKH_KIND_I32 1 /* small signed integers, int_to_scalar view (fr-tensor.cu:713-717) */
#define ZKH_KIND_I64 2 /* signed 64-bit integers, long_to_scalar view (fr-tensor.cu:701-705) */

/* ---------------- context ---------------- */
int zkh_ctx_create(int device, zkh_ctx** out);
int zkh_ctx_destroy(zkh_ctx* ctx);
const char* zkh_last_error(const zkh_ctx* ctx);
/* wait for all work queued on the context's stream */
int zkh_ctx_sync(zkh_ctx* ctx);

/* kernel timing, a tracing aid (the reference's BoTimer laps, zkob_claims.cuh:68-75):
 * when enabled, each kernel class launched on the context is bracketed by HIP events on
 * its stream; zkh_prof_get returns the summed device time, launch count and algorithmic
 * bytes (bytes the algorithm must move, not measured traffic) for one class name;
 * zkh_prof_names lists the recorded names, comma-separated.  Enabling clears the records. */
int zkh_prof_enable(zkh_ctx* ctx, int on);
int zkh_prof_get(zkh_ctx* ctx, const char* name, double* ms, uint64_t* launches, double* bytes);
int zkh_prof_names(zkh_ctx* ctx, char* buf, size_t len);

/* ---------------- tensors (replace FrTensor ctors/save/load: fr-tensor.cu:158-248,
 * zkob_fc.cu:178-185 load_int_tensor, zkob_lookup.cuh:103-110 load_long_tensor) ------- */
/* host Fr array (AoS, reference byte layout) -> device tensor */
int zkh_tensor_from_fr(zkh_ctx* ctx, const uint32_t* fr_aos, uint32_t n, zkh_tensor** out);
/* host int32 / int64 -> device tensor holding the same field values (v<0 -> r-|v|) */
int zkh_tensor_from_i32(zkh_ctx* ctx, const int32_t* v, uint32_t n, zkh_tensor** out);
int zkh_tensor_from_i64(zkh_ctx* ctx, const int64_t* v, uint32_t n, zkh_tensor** out);
/* the same from device pointers (data already resident in HBM; copied, not adopted) */
int zkh_tensor_from_i32_device(zkh_ctx* ctx, const int32_t* dptr, uint32_t n, zkh_tensor** out);
int zkh_tensor_from_i64_device(zkh_ctx* ctx, const int64_t* dptr, uint32_t n, zkh_tensor** out);
/* matmul weight registration: W is IN x OUT row-major int32 (zkob_fc.cu:178 layout); the
 * device copy is laid out OUT-major so the eq-weighted row reduction streams it
 * coalesced.  The tensor's logical content is still W (to_fr returns W row-major). */
int zkh_tensor_weights_i32(zkh_ctx* ctx, const int32_t* W, uint32_t in_dim, uint32_t out_dim,
                           zkh_tensor** out);
int zkh_tensor_free(zkh_tensor* t);
uint32_t zkh_tensor_size(const zkh_tensor* t);
int zkh_tensor_kind(const zkh_tensor* t);
/* device tensor -> host Fr array (n*8 uint32) */
int zkh_tensor_to_fr(zkh_ctx* ctx, const zkh_tensor* t, uint32_t* fr_aos_out);
/* device tensor -> host int64 by scalar_to_long per entry (FrTensor::save_long,
 * fr-tensor.cu:210-218; scalar_to_long :935-945): exact for integer tensors */
int zkh_tensor_to_i64(zkh_ctx* ctx, const zkh_tensor* t, int64_t* out);

/* ---------------- MLE primitives (fr-tensor.cu) ---------------- */
/* sum of all entries (FrTensor::sum, fr-tensor.cu:407-434) */
int zkh_sum(zkh_ctx* ctx, const zkh_tensor* t, uint32_t out[8]);
/* FrTensor::operator()(u): LSB-first MLE evaluation, u[0] binds bit 0 (fr-tensor.cu:437-442,
 * :588-609); requires 2^(k-1) < n <= 2^k */
int zkh_me(zkh_ctx* ctx, const zkh_tensor* t, const uint32_t* u, uint32_t k, uint32_t out[8]);
/* zkh_me without device allocation.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (tight serving loops, harnesses that forbid hipMalloc,
 * a process between the captures of a HIP graph that must not grow the device heap).  Its
 * device scratch (eq tables, block partials, job layout: 557,312 bytes) is one static array
 * per device, held until the process ends and resolved at zkh_ctx_create; the call
 * allocates nothing.  It is synchronous: it runs on the context's stream and waits for its
 * result there (a host spin with hipStreamQuery), so the call itself cannot be recorded into
 * a graph.  t: a field-element tensor; k <= 24 (ZKH_EARG beyond).  Calls that overlap on one
 * device share that scratch and race. */
int zkh_me_static(zkh_ctx* ctx, const zkh_tensor* t, const uint32_t* u, uint32_t k, uint32_t out[8]);
/* one degree-2 product round over MSB pairs (k_bo_hp2 + bo_dev_sum, zkob_claims.cuh:367-383,
 * :577-592): out[t] = sum_{i < n/2} a_t[i] b_t[i] for t = 0, 1, 2, with
 * X_t[i] = X[i] + t (X[i + n/2] - X[i]); a, b FR tensors of one even size n.  With zkh_fold
 * this runs the batch-evaluation sumcheck of the claims accumulator. */
int zkh_prod_round(zkh_ctx* ctx, const zkh_tensor* a, const zkh_tensor* b, uint32_t out[24]);
/* host scalar arithmetic on canonical Fr, the reference's h_scalar / k_scalar_op
 * (vrf_common.cuh:30-38, :100-104): op 0 a+b, 1 a-b, 2 a*b, 3 a^-1 (0 -> 0); no device */
int zkh_fr_scalar(const uint32_t a[8], const uint32_t b[8], int op, uint32_t out[8]);
/* Calibration, no counterpart in the reference: the device's rate of this build's Montgomery
 * multiply (the one every field kernel uses), from a launch of 2048 blocks x 256 threads,
 * each thread running four independent chains of `iters` products; *mul_per_s receives
 * products per second over the launch's device time.  ZKH_EARG when iters is 0. */
int zkh_calib_fr_mul(zkh_ctx* ctx, uint32_t iters, double* mul_per_s);
/* SHA-256 of a byte string (bo_file_sha256's digest, zkob_claims.cuh:310-318); no device */
int zkh_sha256(const void* data, size_t n, uint8_t out[32]);
/* FrTensor::partial_me(u, cur_dim, window) (fr-tensor.cu:518-560): binds the middle
 * dimension of a row-major [other, cur_dim, window] view; returns a new FR tensor of
 * other*window entries */
int zkh_partial_me(zkh_ctx* ctx, const zkh_tensor* t, const uint32_t* u, uint32_t k,
                   uint32_t cur_dim, uint32_t window, zkh_tensor** out);
/* FrTensor::multi_dim_me(us, shape) (fr-tensor.cu:643-652); us concatenated, ks[i] = |us[i]| */
int zkh_multi_dim_me(zkh_ctx* ctx, const zkh_tensor* t, const uint32_t* us, const uint32_t* ks,
                     const uint32_t* shape, uint32_t ndim, uint32_t out[8]);
/* build_eq_tensor(u) (zkob_lookup.cuh:245-265): E[b] = prod_i (b>>i&1 ? u_i : 1-u_i) */
int zkh_eq_table(zkh_ctx* ctx, const uint32_t* u, uint32_t k, zkh_tensor** out);
/* FrTensor::partial_me(u, window) (fr-tensor.cu:512-516, :612-641): k LSB-first binds of
 * the row index of a [rows, window] view (a partial last row reads as zero-filled);
 * requires size > window * 2^(k-1); returns ceil(rows / 2^k) * window entries */
int zkh_partial_me_window(zkh_ctx* ctx, const zkh_tensor* t, const uint32_t* u, uint32_t k,
                          uint32_t window, zkh_tensor** out);
/* FrTensor::pad(shape, pad_val) (fr-tensor.cu:800-828; fr-tensor.cuh:150): every
 * dimension padded to a power of two, padding entries = pad_val (NULL: zero) */
int zkh_pad(zkh_ctx* ctx, const zkh_tensor* t, const uint32_t* shape, uint32_t ndim,
            const uint32_t pad_val[8], zkh_tensor** out);
/* k_fr_fold (zkob_lookup.cuh:35-41): in-place MSB fold t[i] += v*(t[i+h]-t[i]), n -> n/2 */
int zkh_fold(zkh_ctx* ctx, zkh_tensor* t, const uint32_t v[8]);
/* elementwise: out = a + c*b (FrTensor operator+ / operator* by scalar, e.g. the SwiGLU
 * combiner comb = G + r*S, zkob_glu.cu:155-156) and out = a (.) b (Hadamard product).
 * Both return once the work is queued on the context's stream (later calls are ordered
 * behind it; a device error surfaces at the next call that waits for the device). */
int zkh_axpy(zkh_ctx* ctx, const zkh_tensor* a, const uint32_t c[8], const zkh_tensor* b,
             zkh_tensor** out);
int zkh_hadamard(zkh_ctx* ctx, const zkh_tensor* a, const zkh_tensor* b, zkh_tensor** out);

/* ---------------- Fiat-Shamir transcript (fs_transcript.hpp; vrf_common.cuh:219-250) ----- */
int zkh_transcript_init(uint8_t state[32], const char* seed, size_t seed_len);
int zkh_transcript_absorb(uint8_t state[32], const char* label, size_t label_len,
                          const void* data, size_t len);
int zkh_transcript_challenge_fr(uint8_t state[32], uint32_t out[8]);
/* fs_challenge_vec (vrf_common.cuh:246-250): n challenges drawn in sequence, out: n Fr */
int zkh_transcript_challenge_vec(uint8_t state[32], uint32_t n, uint32_t* out);

/* ---------------- matmul sumcheck: zkob_fc.cu:259-440 ----------------
 * X: B x IN, W: IN x OUT, Y: B x OUT with Y = X*W over Fr, each either a field-element
 * tensor (the FrTensors zkob_fc binds, zkob_fc.cu:276-277, :337-338) or an integer tensor
 * (X, W: I32, W preferably from zkh_tensor_weights_i32; Y: I32 or I64 -- the int32 input
 * files of zkob_fc.cu:178-185 and their product); kinds may be mixed.  The caller has
 * absorbed B, IN, OUT and the commitments; this
 * draws u_batch, u_output, evaluates claim = Y~(u_batch,u_output), absorbs "claim", runs
 * the ceilLog2(IN) rounds (absorbing "p0","p1","p2" each) and absorbs "claim_X","claim_W".
 * ev_out: 3L Fr (p(0),p(1),p(2) per round: the sumcheck.bin evals, zkob_fc.cu:101-123);
 * claims_out: claim, claim_X, claim_W; u_batch_out, u_output_out, u_input_out (any may be
 * NULL). */
int zkh_mm_prove(zkh_ctx* ctx, uint8_t transcript[32], const zkh_tensor* X,
                 const zkh_tensor* W, const zkh_tensor* Y, uint32_t B, uint32_t IN, uint32_t OUT,
                 uint32_t* ev_out, uint32_t* claims_out, uint32_t* u_batch_out,
                 uint32_t* u_output_out, uint32_t* u_input_out);

/* Several independent matmul sumchecks (e.g. the Q,K,V,O,gate,up,down matmuls of a layer,
 * each with its own transcript) proven together: every device step is one launch for
 * all jobs and each round costs one host synchronisation for the whole batch.  Each job
 * has exactly the inputs, transcript effects and outputs of zkh_mm_prove; status holds
 * its own return code, and the call returns the first non-zero one.  No counterpart in
 * the reference, which runs one zkob_fc process per matmul. */
typedef struct zkh_mm_job {
    const zkh_tensor* X;
    const zkh_tensor* W;
    const zkh_tensor* Y;
    uint32_t B, IN, OUT;
    uint8_t* transcript; /* 32-byte state, updated in place */
    uint32_t* ev_out;
    uint32_t* claims_out;
    uint32_t* u_batch_out;
    uint32_t* u_output_out;
    uint32_t* u_input_out;
    int status;
} zkh_mm_job;
int zkh_mm_prove_batch(zkh_ctx* ctx, zkh_mm_job* jobs, uint32_t njobs);

/* ---------------- inner-product sumchecks without a transcript (zkfc.cu) ----------------
 * proof_out receives 3 Fr per round: the coefficients c0, c1, c2 of the round polynomial
 * p(X) = c0 + c1 X + c2 X^2 (the reference's Polynomial, zkfc.cu:94-137); final_out the
 * last claim.  ZKH_EROUND when a round's check fails (the reference's runtime_error). */
/* zkip(claim, a, b, u, proof) (zkfc.cu:139-151): k = |u| <= ceilLog2(n) MSB-first rounds,
 * u[k-1] binding first; tables of n entries, zero-filled to the next power of two */
int zkh_zkip(zkh_ctx* ctx, const uint32_t claim[8], const zkh_tensor* a, const zkh_tensor* b,
             const uint32_t* u, uint32_t k, uint32_t* proof_out, uint32_t final_out[8]);
/* zkip_stacked(claim, A, B, uN, uD, vN, N, D, proof) (zkfc.cu:153-246): A, B are [N, D]
 * row-major; kN = ceilLog2(N) eq(uN)-weighted rounds over the rows (checked against
 * eq(uN.back(), X) * p), binding vN.back() first, then zkip over D with uD (kD entries) */
int zkh_zkip_stacked(zkh_ctx* ctx, const uint32_t claim[8], const zkh_tensor* A, const zkh_tensor* B,
                     const uint32_t* uN, uint32_t kN, const uint32_t* uD, uint32_t kD,
                     const uint32_t* vN, uint32_t N, uint32_t D, uint32_t* proof_out,
                     uint32_t final_out[8]);
/* zkFCStacked::prove(u_num, v_num, u_batch, u_input, u_output, proof) (zkfc.cu:288-307):
 * X num x B x IN, W num x IN x OUT (row-major, not from zkh_tensor_weights_i32), Y num x B x
 * OUT, optional bias num x OUT (NULL: none).  Challenge counts are ceilLog2 of num, num, B,
 * IN, OUT.  proof_out: 3*(ceilLog2 num + ceilLog2 IN) Fr; claims_out: claim, final claim.
 * ZKH_EROUND when the final claim differs from X(v_num,u_batch,u_input)*W(v_num,u_input,u_output). */
int zkh_fc_stacked_prove(zkh_ctx* ctx, const zkh_tensor* X, const zkh_tensor* W, const zkh_tensor* Y,
                         const zkh_tensor* bias, uint32_t num, uint32_t B, uint32_t IN, uint32_t OUT,
                         const uint32_t* u_num, const uint32_t* v_num, const uint32_t* u_batch,
                         const uint32_t* u_input, const uint32_t* u_output, uint32_t* proof_out,
                         uint32_t claims_out[16]);

/* ---------------- rescaling witness (rescaling.cu:8-34, zkob_rescale.cu:83-86) ----------- */
/* x = sf * q + rem with rem = ((x + sf/2) mod sf) - sf/2 (C remainder, made non-negative),
 * q = (x - rem) / sf; x read through scalar_to_long for FR tensors (fr-tensor.cu:941-945).
 * q_out, rem_out: new int64 tensors. */
int zkh_rescale(zkh_ctx* ctx, const zkh_tensor* X, uint32_t sf, zkh_tensor** q_out,
                zkh_tensor** rem_out);

/* ---------------- witness GEMM (zkob_fc.cu:211-214, zkfc.cu:44-58, fr-tensor.cu:831-878) ------ */
/* Y = X W (+ bias) over the integers: X int32 [B][IN], W int32 [IN][OUT] (row-major, or
 * registered with zkh_tensor_weights_i32), bias NULL or an int32/int64 tensor of OUT
 * entries; Y_out: a new int64 tensor [B][OUT], exact.  Replaces zkFC::operator() / Y = fc(X)
 * for integer witnesses: the reference's field product equals this integer product
 * reduced mod r.  ZKH_EARG when the operands' magnitude bounds allow a sum beyond 63 bits. */
int zkh_matmul_i32(zkh_ctx* ctx, const zkh_tensor* X, const zkh_tensor* W, const zkh_tensor* bias,
                   uint32_t B, uint32_t IN, uint32_t OUT, zkh_tensor** Y_out);

/* ---------------- logUp lookup (tlookup.cu, zkob_lookup.cuh, zkob_rescale.cu) ---------- */
/* tLookupRange table (tlookup.cu:372-391): T[i] = low+i (i<len) else low+len-1, size N, as an
 * int32-kind tensor (the sum in 32-bit int arithmetic, wrapping as the reference's int does) */
int zkh_lu_range_table(zkh_ctx* ctx, int32_t low, uint32_t len, uint32_t N, zkh_tensor** out);
/* multiplicities m (tlookup.cu:10-48, :414-433): idx = (S-low).limb0, m[idx] += 1.
 * Fails with ZKH_EARG if an index falls outside [0, N) (out-of-range witness). */
int zkh_lu_prep(zkh_ctx* ctx, const zkh_tensor* S, int32_t low, uint32_t N, zkh_tensor** m_out);
/* tLookupRangeMapping::operator() (tlookup.cu:469-482): S_out[i] = mapped[idx_i] and m */
int zkh_lu_mapping(zkh_ctx* ctx, const zkh_tensor* S_in, int32_t low, const zkh_tensor* mapped,
                   zkh_tensor** S_out, zkh_tensor** m_out);
/* tlookup_inv_kernel (tlookup.cu:50-62): A[i] = 1/(S[i]+beta), inverse(0) = 0; batched
 * (Montgomery's trick) */
int zkh_lu_inverse(zkh_ctx* ctx, const zkh_tensor* S, const uint32_t beta[8], zkh_tensor** A_out);
/* zkh_lu_inverse's A = 1/(S+beta) (inverse(0) = 0) for a range lookup against the table T
 * (N entries): A[i] is read off the table inverse 1/(T+beta) at j = (S[i]-low).limb0 wherever
 * T[j] == S[i] (one table-sized inversion instead of a witness-sized one), with a direct
 * inversion of S if some entry is not; the table inverse stays with the context, and the
 * next zkh_lu_prove on this T and beta uses it instead of inverting T again.  Retention: the
 * context holds that inverse (N field elements, 128 MiB at N = 2^22) until a zkh_lu_prove
 * takes it over or, on another table or beta, frees it; until the next zkh_lu_range_inverse
 * or zkh_lu_tuple_inverse replaces it; or until zkh_ctx_destroy.  No counterpart in the
 * reference, which inverts S (zkob_rescale.cu:121-123) and T separately. */
int zkh_lu_range_inverse(zkh_ctx* ctx, const zkh_tensor* S, int32_t low, const zkh_tensor* T,
                         const uint32_t beta[8], zkh_tensor** A_out);
/* zkob_glu.cu:155-170 in one call, for int32 G (D entries), T and mapped (N entries):
 * comb = G + r*S with S[i] = mapped[(G[i]-low).limb0] (zkh_lu_mapping's S), T_comb = T +
 * r*mapped, A = 1/(comb+beta) (inverse(0) = 0) -- the outputs of zkh_lu_mapping's S with
 * zkh_axpy twice and zkh_lu_inverse.  No counterpart in the reference, which inverts comb
 * (D entries) and T_comb (N entries) separately: here A[i] is read off the table inverse
 * 1/(T_comb+beta) wherever T[j] == G[i] (comb[i] is then T_comb[j]), with a direct inversion
 * of comb if some entry is not; the table inverse stays with the context, and the next
 * zkh_lu_prove on this T_comb and beta uses it instead of inverting T_comb again (retained
 * as zkh_lu_range_inverse's).  ZKH_EARG if an index falls outside [0, N) (as zkh_lu_mapping).
 * S (may be NULL): the S that zkh_lu_mapping returned for this G, low and mapped; comb then
 * reads S[i] in order instead of mapped[j] at random (the same values); ZKH_EARG for any
 * other tensor. */
int zkh_lu_tuple_inverse(zkh_ctx* ctx, const zkh_tensor* G, int32_t low, const zkh_tensor* T,
                         const zkh_tensor* mapped, const zkh_tensor* S, const uint32_t r[8],
                         const uint32_t beta[8], zkh_tensor** comb_out, zkh_tensor** Tcomb_out,
                         zkh_tensor** A_out);
/* FS lookup recursion, zkob_rescale.cu:132-146 with fs_phase1/fs_phase2
 * (zkob_lookup.cuh:143-198): from Bv = 1/(T+beta) through the rounds (absorbing
 * "p0".."p3" each) to absorbing "A_f","S_f","m_f".  A, S: D entries; T, m: N entries;
 * u: logD challenges drawn by the caller.  ev_out: 4*logD Fr (lookup.bin evals);
 * term_out: A_f, S_f, B_f, T_f, m_f; ws_out: logD round challenges (may be NULL). */
int zkh_lu_prove(zkh_ctx* ctx, uint8_t transcript[32], const zkh_tensor* A,
                 const zkh_tensor* S, const zkh_tensor* T, const zkh_tensor* m,
                 const uint32_t alpha[8], const uint32_t beta[8], const uint32_t* u,
                 uint32_t* ev_out, uint32_t* term_out, uint32_t* ws_out);

/* ---------------- eq-weighted Hadamard sumcheck (zkob_lookup.cuh:212-315) -------------- */
/* fs_hadamard over E, S, U (2^k entries each).  The caller absorbs the claim before and
 * S_f2/U_f2 after, as the drivers do (zkob_glu.cu:242-247, zkob_rope.cu:234-240).
 * ev_out: 4k Fr; term_out: S_f2, U_f2, E_f; ws_out: k challenges (may be NULL). */
int zkh_hp_prove(zkh_ctx* ctx, uint8_t transcript[32], const uint32_t claim[8],
                 const zkh_tensor* E, const zkh_tensor* S, const zkh_tensor* U,
                 uint32_t* ev_out, uint32_t* term_out, uint32_t* ws_out);
/* the same with E = build_eq_tensor(u) (zkob_glu.cu:243), never materialised */
int zkh_hp_prove_eq(zkh_ctx* ctx, uint8_t transcript[32], const uint32_t claim[8],
                    const uint32_t* u, uint32_t k, const zkh_tensor* S, const zkh_tensor* U,
                    uint32_t* ev_out, uint32_t* term_out, uint32_t* ws_out);
/* No single counterpart in the reference: zkob_rope.cu:230-238 (and :268-275) in one call --
 * the claim c = (E * S * U).sum(), its absorb under `label`, then fs_hadamard over E, S, U.
 * The claim comes from the first round's sums (q(0) + q(1) = c), so the products E * S * U
 * are never formed; claim_out receives it.  Transcript, ev_out, term_out and ws_out are
 * byte-identical to zkh_sum(zkh_hadamard(zkh_hadamard(S, U), E)) + zkh_transcript_absorb(
 * label, c) + zkh_hp_prove.  With ZKH_XCHECK=1 the claim is also recomputed by that sum. */
int zkh_hp_prove_claim(zkh_ctx* ctx, uint8_t transcript[32], const char* label, const zkh_tensor* E,
                       const zkh_tensor* S, const zkh_tensor* U, uint32_t claim_out[8], uint32_t* ev_out,
                       uint32_t* term_out, uint32_t* ws_out);
/* No single counterpart in the reference: zkob_glu.cu:231-247's claim_H = H(u) of H = S * U
 * (multi_dim_me), its absorb under `label`, then fs_hadamard, in one call.  The claim
 * sum eq(i, u) S[i] U[i] comes from the first round's own sums (q(0) + q(1) of the round
 * polynomial equals the claim), so H and its evaluation are never formed; claim_out receives
 * it.  Transcript, ev_out, term_out and ws_out are byte-identical to zkh_me(zkh_hadamard(S,
 * U), u) + zkh_transcript_absorb(label, claim) + zkh_hp_prove_eq.  The claim equals the
 * committed H's evaluation only when that H is S * U: a caller whose H is sourced separately
 * (e.g. a driver testing a forged H) keeps zkh_me on H and calls zkh_hp_prove_eq.  With
 * ZKH_XCHECK=1 the claim is also recomputed as the eq-weighted sum of S * U and compared. */
int zkh_hp_prove_eq_claim(zkh_ctx* ctx, uint8_t transcript[32], const char* label, const uint32_t* u,
                          uint32_t k, const zkh_tensor* S, const zkh_tensor* U, uint32_t claim_out[8],
                          uint32_t* ev_out, uint32_t* term_out, uint32_t* ws_out);

/* ---------------- Pedersen commitments over BLS12-381 G1 (commitment.cu, g1-tensor.cu) -------
 * A point is the reference's 144-byte G1Jacobian_t (g1-tensor.cuh:63): x, y, z, each 12
 * little-endian uint32 limbs of a canonical Fp residue in Montgomery form (R = 2^384);
 * {0, R mod p, 0} is the point at infinity.  Point arrays have their own handle type, so
 * they cannot reach an Fr entry point. */
/* host points -> device (G1TensorJacobian(filename) / loadbin, g1-tensor.cu:179-183) */
int zkh_g1_from_host(zkh_ctx* ctx, const uint32_t* pts, uint32_t n, zkh_g1** out);
/* device points -> host, n*36 uint32 (G1TensorJacobian::save, g1-tensor.cu:174-177) */
int zkh_g1_to_host(zkh_ctx* ctx, const zkh_g1* g, uint32_t* pts);
int zkh_g1_free(zkh_g1* g);
uint32_t zkh_g1_size(const zkh_g1* g);
/* the reference's G1Jacobian_generator (g1-tensor.cuh:63): 36 uint32 */
void zkh_g1_generator(uint32_t* out);
/* out[i] = base[i % size(base)] * t[i], G1Jacobian_mul (g1-tensor.cu:445-454) elementwise
 * with a broadcast base (G1_jacobian_elementwise_mul_broadcast, :463-468): double-and-add
 * over the scalar's raw bits.  With the generator as base and random scalars this is
 * Commitment::random (commitment.cu:3-8), the public generators of a commitment key. */
int zkh_g1_mul(zkh_ctx* ctx, const zkh_g1* base, const zkh_tensor* t, zkh_g1** out);
/* out[i] = b[i] + a[i] * s for point arrays a, b of one size and one plain scalar s: the
 * reference's hb_addmul with mul_first = false (zkob_fastg1.cuh:56-88; G1Jacobian_mul, then
 * the addition with b[i] as first operand), e.g. the SwiGLU claim mode's com_comb =
 * com_G + r com_S row by row (zkob_glu.cu:207-215), byte-identical */
int zkh_g1_addmul(zkh_ctx* ctx, const zkh_g1* a, const uint32_t s[8], const zkh_g1* b, zkh_g1** out);
/* Commitment::commit (commitment.cu:105-108 -> commit_pippenger :85-103): t holds m rows of
 * n = size(gens) scalars (row-major, any tensor kind); out[row] = sum_i t[row][i] gens[i],
 * byte-identical to the reference's bucket method (4-bit windows over the raw scalar
 * limbs, buckets in generator order, running sum, Horner).  ZKH_EARG when size(t) is not a
 * multiple of n (the reference's "Incompatible dimensions") or n > 65536. */
int zkh_commit(zkh_ctx* ctx, const zkh_g1* gens, const zkh_tensor* t, zkh_g1** out);
/* ipa_prove (vrf_common.cuh:302-336), continuing the caller's transcript: a and b n field
 * elements (b: me_weights(u) in the drivers, i.e. zkh_eq_table), g n generators, Q one point,
 * n a power of two.  Per round it absorbs "L" and "R" (144 raw bytes each, as absorb_g1) and
 * draws x; L_out, R_out receive log2(n) points each (36 uint32) and a_final the folded a --
 * the IpaProof fields write_ipa saves (vrf_common.cuh:280-289), byte-identical. */
int zkh_ipa_prove(zkh_ctx* ctx, uint8_t transcript[32], const zkh_tensor* a, const zkh_tensor* b,
                  const zkh_g1* g, const uint32_t Q[36], uint32_t* L_out, uint32_t* R_out,
                  uint32_t a_final[8]);
/* nj <= 8 independent ipa_prove calls (vrf_common.cuh:302-336) in lockstep, job j exactly as
 * zkh_ipa_prove(ctx, transcripts[j], a[j], b[j], g[j], Q[j], L_out[j], R_out[j], a_final[j]):
 * one launch per kernel per round for every job still folding (jobs of different n drop out
 * as they finish).  A round's length is that of one scalar-multiply chain whatever the
 * number of products, so openings that a driver runs side by side (the matmuls of a layer)
 * cost about one opening's time here instead of sharing the device's hardware queues.
 * No reference counterpart as one call: the reference's drivers call ipa_prove once per
 * opening; each job's transcript and outputs are byte-identical to that call's. */
int zkh_ipa_prove_batch(zkh_ctx* ctx, uint32_t nj, uint8_t* const transcripts[], const zkh_tensor* const a[],
                        const zkh_tensor* const b[], const zkh_g1* const g[], const uint32_t* const Q[],
                        uint32_t* const L_out[], uint32_t* const R_out[], uint32_t* const a_final[]);

#ifdef __cplusplus
}
#endif
#endif
