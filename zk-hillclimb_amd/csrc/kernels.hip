// kernels.hip -- gfx950 kernels for the Fr sumcheck / fold / logUp hot path.
//
// Every kernel is integer VALU work on 255-bit field elements (fr_dev.hpp); nothing here
// uses MFMA.  Reductions go lane -> wave (cross-lane shuffles) -> block (LDS) -> one AoS
// partial per block; the host adds the few hundred block partials.  Round kernels fuse the
// previous round's fold (bind) with the current round's evaluation so each table is read
// once per round and halved in place.
//
// Sum conventions: a sum built from mont_mul(x, y) of plain x, y carries a factor 2^-256
// per Montgomery product; each wrapper's comment states the power, and the host multiplies
// it back out (fr_rpow) once per round instead of once per element.
#include "fr_dev.hpp"
#include "kernels.hpp"

namespace zkh {

__device__ __attribute__((noinline)) fr_t mont_mul_ol(fr_t x, fr_t y) { return mont_mul(x, y); }

#define NT 256  // threads per block for the streaming kernels (4 waves of 64)

ZDEV fr_t mk(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, uint32_t a4, uint32_t a5,
             uint32_t a6, uint32_t a7) {
    fr_t r;
    r.v[0] = a0; r.v[1] = a1; r.v[2] = a2; r.v[3] = a3;
    r.v[4] = a4; r.v[5] = a5; r.v[6] = a6; r.v[7] = a7;
    return r;
}
// 2^256 mod r (Montgomery one)
ZDEV fr_t one_m() {
    return mk(0xfffffffeu, 0x00000001u, 0x00034802u, 0x5884b7fau, 0xecbc4ff5u, 0x998c4fefu,
              0xacc5056fu, 0x1824b159u);
}
// 2^512 mod r
ZDEV fr_t r2_m() {
    return mk(0xf3f29c6du, 0xc999e990u, 0x87925c23u, 0x2b6cedcbu, 0x7254398fu, 0x05d31496u,
              0x9f59ff11u, 0x0748d9d9u);
}
ZDEV fr_t plain_one() { return mk(1, 0, 0, 0, 0, 0, 0, 0); }
// 2^(20p) * 2^256 mod r, p = 1..3: recombine 20-bit integer pieces
ZDEV fr_t piece_scale(int p) {
    if (p == 1)
        return mk(0xffdcaaf7u, 0x00235508u, 0xf7a61909u, 0xaa773d1eu, 0x63db3014u, 0x75236b64u,
                  0x1dfe9e8bu, 0x23b7d0bau);
    if (p == 2)
        return mk(0xaf6b1202u, 0x5094ebc8u, 0xa709a833u, 0x9ae3f86fu, 0x3da414adu, 0xf5c24e47u,
                  0xdc58603fu, 0x64a13769u);
    return mk(0x20121c89u, 0xbc98da28u, 0x4c7228c5u, 0x1d3d8a4cu, 0x55cc49e3u, 0xd198d0c2u,
              0xa9088038u, 0x588d22f7u);
}
ZDEV bool fr_is_zero(const fr_t& x) {
    uint32_t o = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) o |= x.v[i];
    return o == 0;
}
static inline __host__ __device__ fr_t to_fr(const uint32_t* h) {
    fr_t r;
#pragma unroll
    for (int i = 0; i < 8; i++) r.v[i] = h[i];
    return r;
}

#define PL_LO(p) reinterpret_cast<uint4*>((p).lo())
#define PL_HI(p) reinterpret_cast<uint4*>((p).hi())

uint32_t grid_for(uint32_t work_items, uint32_t per_block, uint32_t max_blocks) {
    uint32_t g = (work_items + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > max_blocks) g = max_blocks;
    return g;
}

// K field accumulators per thread -> one AoS partial per block (partial[blockIdx*K + k])
template <int K>
ZDEV void block_reduce_store_at(fr_t* acc, uint32_t* partial, uint32_t slot) {
    __shared__ fr_t red[NT / 64][K];
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    // one accumulator at a time: interleaved wave sums of K accumulators would hold all
    // their shuffle temporaries at once and set the kernel's register budget (occupancy)
#pragma unroll
    for (int k = 0; k < K; k++) {
        __builtin_amdgcn_sched_barrier(0);
        const fr_t w = fr_wave_sum(acc[k]);
        if (lane == 0) red[wid][k] = w;
    }
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    if (threadIdx.x < K) {
        const int k = threadIdx.x;
        fr_t s = red[0][k];
#pragma unroll
        for (int w = 1; w < NT / 64; w++) s = fr_add(s, red[w][k]);
        st_aos(partial, slot * K + k, s);
    }
}
template <int K>
ZDEV void block_reduce_store(fr_t* acc, uint32_t* partial) {
    block_reduce_store_at<K>(acc, partial, blockIdx.x);
}

// A job's layout word triple (see Publish), written by the job's first block
ZDEV void publish_layout(const Publish& P, uint32_t job, uint32_t first, uint32_t nblk, uint32_t K) {
    P.layout[3 * job] = first;
    P.layout[3 * job + 1] = nblk;
    P.layout[3 * job + 2] = K;
}
// Block partials of a publishing kernel (see Publish); every thread of the block calls it.
// first/nblk: the job's block range.
template <int K>
ZDEV void reduce_publish(fr_t* acc, const Publish& P, uint32_t job, uint32_t first, uint32_t nblk,
                         uint32_t local) {
    block_reduce_store_at<K>(acc, P.part, first + local);
    if (local == 0 && threadIdx.x == 0) publish_layout(P, job, first, nblk, K);
}
// The publish kernel: W = 16 / (job sums) waves (at least 1) per sum, each adding every
// W-th run of 64 block partials with four loads in flight per lane, then the W wave sums of
// each sum in LDS (job j's sum k to host_out[j K_j + k]); thread 0 raises the host flag.
#define NTPUB 1024
ZDEV void pub_locate(const Publish& P, uint32_t q, uint32_t& j, uint32_t& k) {
    j = 0;
    k = q;
    while (k >= P.layout[3 * j + 2]) k -= P.layout[3 * j + 2], j++;
}
__global__ __launch_bounds__(NTPUB) void k_publish(Publish P) {
    constexpr uint32_t NW = NTPUB / 64;
    __shared__ fr_t red[NW];
    const uint32_t wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    uint32_t tot = 0;
    for (uint32_t j = 0; j < P.njobs; j++) tot += P.layout[3 * j + 2];
    const uint32_t W = tot >= NW || tot == 0 ? 1 : NW / tot, per = NW / W;  // waves per sum, sums per pass
    for (uint32_t q0 = 0; q0 < tot; q0 += per) {
        const uint32_t q = q0 + wv / W, share = wv % W;
        fr_t t = fr_zero();
        if (wv < per * W && q < tot) {
            uint32_t j, k;
            pub_locate(P, q, j, k);
            const uint32_t first = P.layout[3 * j], nblk = P.layout[3 * j + 1], K = P.layout[3 * j + 2];
            const uint32_t step = 64 * W;
            for (uint32_t b = share * 64 + lane; b < nblk; b += 4 * step) {
                fr_t x[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const uint32_t bb = b + u * step;
                    x[u] = bb < nblk ? ld_aos(P.part, (first + bb) * K + k) : fr_zero();
                }
                t = fr_add(t, fr_add(fr_add(x[0], x[1]), fr_add(x[2], x[3])));
            }
        }
        t = fr_wave_sum(t);
        if (lane == 0) red[wv] = t;
        __syncthreads();
        if (threadIdx.x < per && q0 + threadIdx.x < tot) {
            fr_t sum = red[threadIdx.x * W];
            for (uint32_t w = 1; w < W; w++) sum = fr_add(sum, red[threadIdx.x * W + w]);
            uint32_t j, k;
            pub_locate(P, q0 + threadIdx.x, j, k);
            st_aos(P.host_out, j * P.layout[3 * j + 2] + k, sum);
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        __threadfence_system();
        __hip_atomic_store(P.host_flag, P.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}
void launch_publish(hipStream_t s, const Publish& P) { k_publish<<<1, NTPUB, 0, s>>>(P); }

// ------------------------------------------------------------------------------------
// conversions and layout
// ------------------------------------------------------------------------------------
__global__ void k_i32_to_planes(const int32_t* __restrict__ in, uint32_t n, uint4* lo, uint4* hi) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        st_fr(lo, hi, i, fr_from_i64(in[i]));
}
__global__ void k_i64_to_planes(const int64_t* __restrict__ in, uint32_t n, uint4* lo, uint4* hi) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        st_fr(lo, hi, i, fr_from_i64(in[i]));
}
__global__ void k_aos_to_planes(const uint32_t* __restrict__ aos, uint32_t n, uint4* lo, uint4* hi) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        st_fr(lo, hi, i, ld_aos(aos, i));
}
__global__ void k_planes_to_aos(const uint4* lo, const uint4* hi, uint32_t n, uint32_t* aos) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        st_aos(aos, i, ld_fr(lo, hi, i));
}
// |v| maximum: lane -> wave (shuffles) -> block (LDS) -> one atomic per block
template <typename U>
ZDEV U absmax_block(U m) {
    __shared__ U red[NT / 64];
#pragma unroll
    for (int s = 32; s >= 1; s >>= 1) {
        U o = __shfl_xor(m, s, 64);
        m = o > m ? o : m;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; w++) m = red[w] > m ? red[w] : m;
    return m;
}
__global__ __launch_bounds__(NT) void k_absmax_i32(const int32_t* __restrict__ in, uint32_t n, uint32_t* out) {
    uint32_t m = 0, not_one = 0;
    for (uint32_t i = blockIdx.x * NT + threadIdx.x; i < n; i += gridDim.x * NT) {
        int64_t v = in[i];
        uint32_t a = (uint32_t)(v < 0 ? -v : v);
        m = a > m ? a : m;
        not_one |= v != 1;
    }
    m = absmax_block<uint32_t>(m);
    not_one = absmax_block<uint32_t>(not_one);
    if (threadIdx.x == 0) {
        atomicMax(out, m);
        if (not_one) atomicOr(out + 1, 1u);
    }
}
__global__ __launch_bounds__(NT) void k_absmax_i64(const int64_t* __restrict__ in, uint32_t n,
                                                   unsigned long long* out) {
    unsigned long long m = 0;
    for (uint32_t i = blockIdx.x * NT + threadIdx.x; i < n; i += gridDim.x * NT) {
        int64_t v = in[i];
        unsigned long long a = v < 0 ? (unsigned long long)(-(v + 1)) + 1 : (unsigned long long)v;
        m = a > m ? a : m;
    }
    m = absmax_block<unsigned long long>(m);
    if (threadIdx.x == 0) atomicMax(out, m);
}
// 32x32 LDS tile transpose: out[c*rows + r] = in[r*cols + c]
__global__ void k_transpose_i32(const int32_t* __restrict__ in, uint32_t rows, uint32_t cols,
                                int32_t* __restrict__ out) {
    __shared__ int32_t tile[32][33];
    uint32_t c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    uint32_t tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 256 threads: ty 0..7
    for (uint32_t j = ty; j < 32; j += 8) {
        uint32_t r = r0 + j, c = c0 + tx;
        if (r < rows && c < cols) tile[j][tx] = in[(size_t)r * cols + c];
    }
    __syncthreads();
    for (uint32_t j = ty; j < 32; j += 8) {
        uint32_t c = c0 + j, r = r0 + tx;
        if (r < rows && c < cols) out[(size_t)c * rows + r] = tile[tx][j];
    }
}

void launch_i32_to_planes(hipStream_t s, const int32_t* in, uint32_t n, DevPlanes out) {
    if (!n) return;
    k_i32_to_planes<<<grid_for(n, NT, 8192), NT, 0, s>>>(in, n, PL_LO(out), PL_HI(out));
}
void launch_i64_to_planes(hipStream_t s, const int64_t* in, uint32_t n, DevPlanes out) {
    if (!n) return;
    k_i64_to_planes<<<grid_for(n, NT, 8192), NT, 0, s>>>(in, n, PL_LO(out), PL_HI(out));
}
// *bad += number of 8-word entries >= r (an upload's canonical-form check, on the device so
// that multi-GB witness files are not scanned by one host thread)
__global__ void k_count_noncanonical(const uint32_t* __restrict__ aos, uint32_t n, uint32_t* bad) {
    uint32_t cnt = 0;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const uint4 a = ((const uint4*)aos)[2 * (size_t)i], b = ((const uint4*)aos)[2 * (size_t)i + 1];
        const uint32_t v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint32_t br = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) (void)__builtin_subc(v[k], fr_p(k), br, &br);
        cnt += br ? 0u : 1u;  // no borrow from v - r: v >= r
    }
    if (cnt) atomicAdd(bad, cnt);
}
void launch_count_noncanonical(hipStream_t s, const uint32_t* aos, uint32_t n, uint32_t* bad) {
    if (!n) return;
    k_count_noncanonical<<<grid_for(n, NT, 8192), NT, 0, s>>>(aos, n, bad);
}
void launch_aos_to_planes(hipStream_t s, const uint32_t* aos, uint32_t n, DevPlanes out) {
    if (!n) return;
    k_aos_to_planes<<<grid_for(n, NT, 8192), NT, 0, s>>>(aos, n, PL_LO(out), PL_HI(out));
}
void launch_planes_to_aos(hipStream_t s, DevPlanes in, uint32_t n, uint32_t* aos) {
    if (!n) return;
    k_planes_to_aos<<<grid_for(n, NT, 8192), NT, 0, s>>>(PL_LO(in), PL_HI(in), n, aos);
}
void launch_absmax_i32(hipStream_t s, const int32_t* in, uint32_t n, uint32_t* out) {
    if (!n) return;
    k_absmax_i32<<<grid_for(n, NT * 8, 512), NT, 0, s>>>(in, n, out);
}
void launch_absmax_i64(hipStream_t s, const int64_t* in, uint32_t n, unsigned long long* out) {
    if (!n) return;
    k_absmax_i64<<<grid_for(n, NT * 8, 512), NT, 0, s>>>(in, n, out);
}
void launch_transpose_i32(hipStream_t s, const int32_t* in, uint32_t rows, uint32_t cols,
                          int32_t* out) {
    dim3 g((cols + 31) / 32, (rows + 31) / 32);
    k_transpose_i32<<<g, NT, 0, s>>>(in, rows, cols, out);
}

// ------------------------------------------------------------------------------------
// eq tables
// ------------------------------------------------------------------------------------
ZDEV fr_t eq_prod(const uint32_t* __restrict__ fac, uint32_t K, uint32_t b) {
    fr_t e = one_m();
    for (uint32_t t = 0; t < K; t++) e = mont_mul(e, ld_aos(fac, 2 * t + ((b >> t) & 1)));
    return e;
}
__global__ void k_eq_mont(const uint32_t* __restrict__ fac, uint32_t K, uint32_t n, uint32_t* out) {
    for (uint32_t b = blockIdx.x * blockDim.x + threadIdx.x; b < n; b += gridDim.x * blockDim.x)
        st_aos(out, b, eq_prod(fac, K, b));
}
// The same by four lanes an entry: lane q of an entry's quad multiplies the factors t = q,
// q + 4, ... (a chain of K/4 products), then two shuffle levels combine the quad -- the
// latency of about K/4 + 2 products instead of K, for the small tables a proof builds first
// (Elo, Ehi).  Two tables per launch: blocks [0, g0) build table 0, the rest table 1.
ZDEV fr_t eq_prod_quad(const uint32_t* __restrict__ fac, uint32_t K, uint32_t b, uint32_t q) {
    fr_t e = q < K ? ld_aos(fac, 2 * q + ((b >> q) & 1)) : one_m();
    for (uint32_t t = q + 4; t < K; t += 4) e = mont_mul(e, ld_aos(fac, 2 * t + ((b >> t) & 1)));
    e = mont_mul(e, fr_shfl_xor(e, 1));
    return mont_mul(e, fr_shfl_xor(e, 2));
}
struct EqTab {
    const uint32_t* fac;
    uint32_t K, n;
    uint32_t* out;
};
__global__ __launch_bounds__(NT) void k_eq_mont_quad(EqTab t0, EqTab t1, uint32_t g0) {
    const bool second = blockIdx.x >= g0;
    const EqTab& T = second ? t1 : t0;
    const uint32_t i = (blockIdx.x - (second ? g0 : 0)) * NT + threadIdx.x;
    const uint32_t b = i >> 2, q = i & 3;
    const fr_t e = eq_prod_quad(T.fac, T.K, b < T.n ? b : 0, q);  // every lane of a quad takes part
    if (q == 0 && b < T.n) st_aos(T.out, b, e);
}
// The same with the factors in the launch's arguments (no upload ahead of it): table 0 takes
// factors [0, K0), table 1 factors [K0, K0 + K1), in plain form when plain1 is set.
__global__ __launch_bounds__(NT) void k_eq_mont_quad_ka(FacArg f, uint32_t K0, uint32_t n0, uint32_t* out0,
                                                        uint32_t K1, uint32_t n1, uint32_t* out1, uint32_t g0,
                                                        uint32_t plain1) {
    const bool second = blockIdx.x >= g0;
    const uint32_t K = second ? K1 : K0, n = second ? n1 : n0;
    uint32_t* out = second ? out1 : out0;
    const uint32_t i = (blockIdx.x - (second ? g0 : 0)) * NT + threadIdx.x;
    const uint32_t b = i >> 2, q = i & 3;
    const fr_t e = eq_prod_quad(f.w + (second ? 16 * K0 : 0), K, b < n ? b : 0, q);
    if (q == 0 && b < n) st_aos(out, b, second && plain1 ? mont_mul(e, plain_one()) : e);
}
#define EQ_QUAD_MAX (1u << 14)  // larger tables: one entry per thread (product throughput)
void launch_eq_mont(hipStream_t s, const uint32_t* fac, uint32_t K, uint32_t n, uint32_t* out) {
    if (n <= EQ_QUAD_MAX) {
        const uint32_t g0 = (4 * n + NT - 1) / NT;
        k_eq_mont_quad<<<g0, NT, 0, s>>>(EqTab{fac, K, n, out}, EqTab{fac, K, 0, out}, g0);
        return;
    }
    k_eq_mont<<<grid_for(n, NT, 4096), NT, 0, s>>>(fac, K, n, out);
}
bool launch_eq_mont2_ka(hipStream_t s, const FacArg& f, uint32_t K0, uint32_t n0, uint32_t* out0, uint32_t K1,
                        uint32_t n1, uint32_t* out1, bool plain1) {
    if (n0 > EQ_QUAD_MAX || n1 > EQ_QUAD_MAX || K0 + K1 > ZKH_FAC_ARG_VARS) return false;
    const uint32_t g0 = (4 * n0 + NT - 1) / NT, g1 = (4 * n1 + NT - 1) / NT;
    k_eq_mont_quad_ka<<<g0 + g1, NT, 0, s>>>(f, K0, n0, out0, K1, n1, out1, g0, plain1 ? 1u : 0u);
    return true;
}
void launch_eq_mont2(hipStream_t s, const uint32_t* fac0, uint32_t K0, uint32_t n0, uint32_t* out0,
                     const uint32_t* fac1, uint32_t K1, uint32_t n1, uint32_t* out1) {
    if (n0 > EQ_QUAD_MAX || n1 > EQ_QUAD_MAX) {
        launch_eq_mont(s, fac0, K0, n0, out0);
        launch_eq_mont(s, fac1, K1, n1, out1);
        return;
    }
    const uint32_t g0 = (4 * n0 + NT - 1) / NT, g1 = (4 * n1 + NT - 1) / NT;
    k_eq_mont_quad<<<g0 + g1, NT, 0, s>>>(EqTab{fac0, K0, n0, out0}, EqTab{fac1, K1, n1, out1}, g0);
}

// ------------------------------------------------------------------------------------
// dot products and sums (block partials)
// ------------------------------------------------------------------------------------
__global__ __launch_bounds__(NT) void k_dot_planes(const uint4* alo, const uint4* ahi,
                                                   const uint4* blo, const uint4* bhi, uint32_t n,
                                                   Publish pub) {
    fr_t acc[1] = {fr_zero()};
    for (uint32_t i = blockIdx.x * NT + threadIdx.x; i < n; i += gridDim.x * NT)
        acc[0] = fr_add(acc[0], mont_mul(ld_fr(alo, ahi, i), ld_fr(blo, bhi, i)));
    reduce_publish<1>(acc, pub, 0, 0, gridDim.x, blockIdx.x);
}
__global__ __launch_bounds__(NT) void k_sum_planes(const uint4* alo, const uint4* ahi, uint32_t n,
                                                   Publish pub) {
    fr_t acc[1] = {fr_zero()};
    for (uint32_t i = blockIdx.x * NT + threadIdx.x; i < n; i += gridDim.x * NT)
        acc[0] = fr_add(acc[0], ld_fr(alo, ahi, i));
    reduce_publish<1>(acc, pub, 0, 0, gridDim.x, blockIdx.x);
}
// degree-2 product round over MSB pairs (k_bo_hp2 + bo_dev_sum, zkob_claims.cuh:367-383,
// :577-592): sums of a_t[i] b_t[i] for t = 0, 1, 2, X_t = X[i] + t (X[i+h] - X[i])
__global__ __launch_bounds__(NT) void k_prod_round(const uint4* alo, const uint4* ahi, const uint4* blo,
                                                   const uint4* bhi, uint32_t h, Publish pub) {
    fr_t acc[3] = {fr_zero(), fr_zero(), fr_zero()};
    for (uint32_t i = blockIdx.x * NT + threadIdx.x; i < h; i += gridDim.x * NT) {
        const fr_t a0 = ld_fr(alo, ahi, i), a1 = ld_fr(alo, ahi, i + h);
        const fr_t b0 = ld_fr(blo, bhi, i), b1 = ld_fr(blo, bhi, i + h);
        acc[0] = fr_add(acc[0], mont_mul(a0, b0));
        acc[1] = fr_add(acc[1], mont_mul(a1, b1));
        acc[2] = fr_add(acc[2], mont_mul(fr_sub(fr_add(a1, a1), a0), fr_sub(fr_add(b1, b1), b0)));
    }
    reduce_publish<3>(acc, pub, 0, 0, gridDim.x, blockIdx.x);
}
uint32_t launch_prod_round(hipStream_t s, DevPlanes a, DevPlanes b, uint32_t h, Publish pub) {
    uint32_t g = grid_for(h, NT * 4, 1024);
    k_prod_round<<<g, NT, 0, s>>>(PL_LO(a), PL_HI(a), PL_LO(b), PL_HI(b), h, pub);
    launch_publish(s, pub);
    return g;
}
uint32_t launch_dot_planes(hipStream_t s, DevPlanes a, DevPlanes b, uint32_t n, Publish pub) {
    uint32_t g = grid_for(n, NT * 4, 1024);
    k_dot_planes<<<g, NT, 0, s>>>(PL_LO(a), PL_HI(a), PL_LO(b), PL_HI(b), n, pub);
    launch_publish(s, pub);
    return g;
}
uint32_t launch_sum_planes(hipStream_t s, DevPlanes a, uint32_t n, Publish pub) {
    uint32_t g = grid_for(n, NT * 8, 1024);
    k_sum_planes<<<g, NT, 0, s>>>(PL_LO(a), PL_HI(a), n, pub);
    launch_publish(s, pub);
    return g;
}

// ------------------------------------------------------------------------------------
// generic MLE pieces
// ------------------------------------------------------------------------------------
template <typename Ld>
__global__ void k_partial_me(Ld ld, uint32_t O, uint32_t C, uint32_t W,
                             const uint32_t* __restrict__ E, uint4* olo, uint4* ohi) {
    const uint32_t total = O * W;
    for (uint32_t g = blockIdx.x * blockDim.x + threadIdx.x; g < total; g += gridDim.x * blockDim.x) {
        uint32_t o = g / W, w = g % W;
        fr_t acc = fr_zero();
        for (uint32_t c = 0; c < C; c++)
            acc = fr_add(acc, mont_mul(ld_aos(E, c), ld(((size_t)o * C + c) * W + w)));
        st_fr(olo, ohi, g, acc);
    }
}
struct LdPlanes {
    const uint4* lo;
    const uint4* hi;
    ZDEV fr_t operator()(size_t i) const { return ld_fr(lo, hi, (uint32_t)i); }
};
struct LdI32 {
    const int32_t* p;
    ZDEV fr_t operator()(size_t i) const { return fr_from_i64(p[i]); }
};
struct LdI64 {
    const int64_t* p;
    ZDEV fr_t operator()(size_t i) const { return fr_from_i64(p[i]); }
};
void launch_partial_me_planes(hipStream_t s, DevPlanes t, uint32_t O, uint32_t C, uint32_t W,
                              const uint32_t* E, DevPlanes out) {
    LdPlanes ld{PL_LO(t), PL_HI(t)};
    k_partial_me<<<grid_for(O * W, NT, 8192), NT, 0, s>>>(ld, O, C, W, E, PL_LO(out), PL_HI(out));
}
void launch_partial_me_i32(hipStream_t s, const int32_t* t, uint32_t O, uint32_t C, uint32_t W,
                           const uint32_t* E, DevPlanes out) {
    LdI32 ld{t};
    k_partial_me<<<grid_for(O * W, NT, 8192), NT, 0, s>>>(ld, O, C, W, E, PL_LO(out), PL_HI(out));
}
void launch_partial_me_i64(hipStream_t s, const int64_t* t, uint32_t O, uint32_t C, uint32_t W,
                           const uint32_t* E, DevPlanes out) {
    LdI64 ld{t};
    k_partial_me<<<grid_for(O * W, NT, 8192), NT, 0, s>>>(ld, O, C, W, E, PL_LO(out), PL_HI(out));
}
// the same loaders with entries at index >= n reading as zero (a [rows, W] view whose
// last rows are partial or missing)
template <typename Ld>
struct LdBounded {
    Ld ld;
    size_t n;
    ZDEV fr_t operator()(size_t i) const { return i < n ? ld(i) : fr_zero(); }
};
template <typename Ld>
static void partial_me_bounded(hipStream_t s, Ld ld, size_t n, uint32_t O, uint32_t C, uint32_t W,
                               const uint32_t* E, DevPlanes out) {
    LdBounded<Ld> b{ld, n};
    k_partial_me<<<grid_for(O * W, NT, 8192), NT, 0, s>>>(b, O, C, W, E, PL_LO(out), PL_HI(out));
}
void launch_partial_me_window(hipStream_t s, int kind, const void* t, uint32_t cap, uint32_t n,
                              uint32_t O, uint32_t C, uint32_t W, const uint32_t* E, DevPlanes out) {
    if (kind == 0) {
        DevPlanes p{(uint32_t*)t, cap};
        partial_me_bounded(s, LdPlanes{PL_LO(p), PL_HI(p)}, n, O, C, W, E, out);
    } else if (kind == 1) {
        partial_me_bounded(s, LdI32{(const int32_t*)t}, n, O, C, W, E, out);
    } else {
        partial_me_bounded(s, LdI64{(const int64_t*)t}, n, O, C, W, E, out);
    }
}

// ------------------------------------------------------------------------------------
// padding and table initialisation
// ------------------------------------------------------------------------------------
// out[g] over the padded shape (every dimension 2^lg[d]) = src at the unpadded index, or
// the pad value where any coordinate lies in a dimension's padding
__global__ void k_pad(const uint4* slo, const uint4* shi, PadDims pd, uint32_t total, fr_t pv,
                      uint4* olo, uint4* ohi) {
    for (uint32_t g = blockIdx.x * blockDim.x + threadIdx.x; g < total; g += gridDim.x * blockDim.x) {
        uint32_t rem = g;
        size_t sidx = 0, mul = 1;
        bool in = true;
        for (int d = (int)pd.nd - 1; d >= 0; d--) {
            const uint32_t i = rem & ((1u << pd.lg[d]) - 1);
            rem >>= pd.lg[d];
            in = in && i < pd.shape[d];
            sidx += (size_t)i * mul;
            mul *= pd.shape[d];
        }
        st_fr(olo, ohi, g, in ? ld_fr(slo, shi, (uint32_t)sidx) : pv);
    }
}
void launch_pad(hipStream_t s, DevPlanes src, const PadDims& pd, uint32_t total, const uint32_t* pad_host,
                DevPlanes out) {
    k_pad<<<grid_for(total, NT, 8192), NT, 0, s>>>(PL_LO(src), PL_HI(src), pd, total, to_fr(pad_host),
                                                  PL_LO(out), PL_HI(out));
}
// tLookupRange table: T[i] = low + i for i < len, low + len - 1 beyond (int arithmetic)
__global__ void k_range_table(int32_t low, uint32_t len, uint32_t N, uint4* olo, uint4* ohi) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < N; i += gridDim.x * blockDim.x) {
        const uint32_t off = i < len ? i : len - 1;
        st_fr(olo, ohi, i, fr_from_i64((int32_t)((uint32_t)low + off)));
    }
}
void launch_range_table(hipStream_t s, int32_t low, uint32_t len, uint32_t N, DevPlanes out) {
    k_range_table<<<grid_for(N, NT, 8192), NT, 0, s>>>(low, len, N, PL_LO(out), PL_HI(out));
}
// the same entries as int32 (the table's own 32-bit arithmetic)
__global__ void k_range_table_i32(int32_t low, uint32_t len, uint32_t N, int32_t* out) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < N; i += gridDim.x * blockDim.x)
        out[i] = (int32_t)((uint32_t)low + (i < len ? i : len - 1));
}
void launch_range_table_i32(hipStream_t s, int32_t low, uint32_t len, uint32_t N, int32_t* out) {
    k_range_table_i32<<<grid_for(N, NT, 8192), NT, 0, s>>>(low, len, N, out);
}

// ------------------------------------------------------------------------------------
// plain and stacked inner-product sumcheck rounds over a [N, D] row layout: row n < Nh
// pairs with row n + Nh (Nh = 2^ceil(log2 N) / 2; rows >= N read as zero) and carries the
// weight E[n] (Montgomery form, AoS) or 1 when E is null.  Sums, each x 2^-256:
// c0 = sum w a0 b0, c1 = sum w (a0 db + b0 da), c2 = sum w da db.
// ------------------------------------------------------------------------------------
__global__ __launch_bounds__(NT) void k_stk_round(const uint4* alo, const uint4* ahi, const uint4* blo,
                                                  const uint4* bhi, uint32_t N, uint32_t D, uint32_t Nh,
                                                  const uint32_t* __restrict__ E, Publish pub) {
    fr_t acc[3] = {fr_zero(), fr_zero(), fr_zero()};
    const uint32_t tot = Nh * D, hiD = Nh * D, full = N * D;
    for (uint32_t idx = blockIdx.x * NT + threadIdx.x; idx < tot; idx += gridDim.x * NT) {
        fr_t a0 = ld_fr(alo, ahi, idx), b0 = ld_fr(blo, bhi, idx);
        const bool up = idx + hiD < full;
        fr_t da = fr_sub(up ? ld_fr(alo, ahi, idx + hiD) : fr_zero(), a0);
        fr_t db = fr_sub(up ? ld_fr(blo, bhi, idx + hiD) : fr_zero(), b0);
        if (E) {
            const fr_t wm = ld_aos(E, idx / D);
            a0 = mont_mul(wm, a0);  // w * a0 (plain)
            da = mont_mul(wm, da);
        }
        acc[0] = fr_add(acc[0], mont_mul(a0, b0));
        acc[1] = fr_add(acc[1], fr_add(mont_mul(a0, db), mont_mul(da, b0)));
        acc[2] = fr_add(acc[2], mont_mul(da, db));
    }
    reduce_publish<3>(acc, pub, 0, 0, gridDim.x, blockIdx.x);
}
// in-place bind of the top row bit: t[idx] = t0 + v (t1 - t0) for idx < Nh*D (t1 = 0 past N)
__global__ void k_stk_fold(uint4* alo, uint4* ahi, uint4* blo, uint4* bhi, uint32_t N, uint32_t D,
                           uint32_t Nh, fr_t vm) {
    const uint32_t tot = Nh * D, hiD = Nh * D, full = N * D;
    for (uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x; idx < tot; idx += gridDim.x * blockDim.x) {
        const bool up = idx + hiD < full;
        const fr_t a0 = ld_fr(alo, ahi, idx), b0 = ld_fr(blo, bhi, idx);
        const fr_t a1 = up ? ld_fr(alo, ahi, idx + hiD) : fr_zero();
        const fr_t b1 = up ? ld_fr(blo, bhi, idx + hiD) : fr_zero();
        st_fr(alo, ahi, idx, fr_add(a0, mont_mul(vm, fr_sub(a1, a0))));
        st_fr(blo, bhi, idx, fr_add(b0, mont_mul(vm, fr_sub(b1, b0))));
    }
}
uint32_t launch_stk_round(hipStream_t s, DevPlanes a, DevPlanes b, uint32_t N, uint32_t D, uint32_t Nh,
                          const uint32_t* E, Publish pub) {
    const uint32_t g = grid_for(Nh * D, NT, 1024);
    k_stk_round<<<g, NT, 0, s>>>(PL_LO(a), PL_HI(a), PL_LO(b), PL_HI(b), N, D, Nh, E, pub);
    launch_publish(s, pub);
    return g;
}
void launch_stk_fold(hipStream_t s, DevPlanes a, DevPlanes b, uint32_t N, uint32_t D, uint32_t Nh,
                     const uint32_t* v_m_host) {
    k_stk_fold<<<grid_for(Nh * D, NT, 8192), NT, 0, s>>>(PL_LO(a), PL_HI(a), PL_LO(b), PL_HI(b), N, D, Nh,
                                                        to_fr(v_m_host));
}

// ------------------------------------------------------------------------------------
// rescaling witness (rescaling.cu:8-21): x = sf * q + rem with rem in [-sf/2, sf - sf/2)
// ------------------------------------------------------------------------------------
// scalar_to_long (fr-tensor.cu:935-945): small non-negative values as they are, otherwise
// minus the low 64 bits of r - x (0 when r - x has any limb above the second set)
ZDEV int64_t fr_to_long(const fr_t& x) {
    if (!(x.v[7] | x.v[6] | x.v[5] | x.v[4] | x.v[3] | x.v[2]) && !(x.v[1] >> 31))
        return (int64_t)(((uint64_t)x.v[1] << 32) | x.v[0]);
    const fr_t y = fr_sub(fr_zero(), x);
    const uint64_t u = (y.v[7] | y.v[6] | y.v[5] | y.v[4] | y.v[3] | y.v[2])
                           ? 0
                           : (((uint64_t)y.v[1] << 32) | y.v[0]);
    return (int64_t)(0 - u);
}
template <typename T>
struct LdInt {
    const T* p;
    ZDEV int64_t operator()(uint32_t i) const { return (int64_t)p[i]; }
};
struct LdLong {
    const uint4* lo;
    const uint4* hi;
    ZDEV int64_t operator()(uint32_t i) const { return fr_to_long(ld_fr(lo, hi, i)); }
};
template <typename Ld>
__global__ void k_rescale(Ld ld, uint32_t n, int64_t sf, int64_t* __restrict__ q, int64_t* __restrict__ rem) {
    const int64_t hsf = sf >> 1;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const int64_t x = ld(i);
        const int64_t t = (int64_t)((uint64_t)x + (uint64_t)hsf) % sf;  // C remainder: sign of the dividend
        const int64_t r = (t < 0 ? t + sf : t) - hsf;
        q[i] = (int64_t)((uint64_t)x - (uint64_t)r) / sf;
        rem[i] = r;
    }
}
void launch_rescale(hipStream_t s, int kind, const void* x, uint32_t cap, uint32_t n, int64_t sf,
                    int64_t* q, int64_t* rem) {
    const uint32_t g = grid_for(n, NT, 8192);
    if (kind == 0) {
        DevPlanes p{(uint32_t*)x, cap};
        k_rescale<<<g, NT, 0, s>>>(LdLong{PL_LO(p), PL_HI(p)}, n, sf, q, rem);
    } else if (kind == 1) {
        k_rescale<<<g, NT, 0, s>>>(LdInt<int32_t>{(const int32_t*)x}, n, sf, q, rem);
    } else {
        k_rescale<<<g, NT, 0, s>>>(LdInt<int64_t>{(const int64_t*)x}, n, sf, q, rem);
    }
}

ZDEV fr_t fold_at(const uint4* lo, const uint4* hi, uint32_t j, uint32_t n, const fr_t& vm) {
    fr_t x = ld_fr(lo, hi, j), y = ld_fr(lo, hi, j + n);
    return fr_add(x, mont_mul_ol(vm, fr_sub(y, x)));
}
// A table taking part in a fused round: read from (slo, shi), or from the int32 entries s32
// when set (an integer table not yet folded); when the round folds, the folded entries go
// to (dlo, dhi), which may alias the source (in-place halving).
struct TabDev {
    const uint4* slo;
    const uint4* shi;
    uint4* dlo;
    uint4* dhi;
    const int32_t* s32;
};
ZDEV fr_t tab_ld(const TabDev& t, uint32_t i) { return t.s32 ? fr_from_i64(t.s32[i]) : ld_fr(t.slo, t.shi, i); }
ZDEV fr_t tab_fold_at(const TabDev& t, uint32_t j, uint32_t n, const fr_t& vm) {
    if (!t.s32) return fold_at(t.slo, t.shi, j, n, vm);
    const fr_t x = fr_from_i64(t.s32[j]), y = fr_from_i64(t.s32[j + n]);
    return fr_add(x, mont_mul_ol(vm, fr_sub(y, x)));
}
// The same with the challenge also plain (vp = v, wave-uniform): an int32 table folds as
// x + v (y - x) by the 32-bit multiply (|y - x| < 2^32), about 70 instructions instead of a
// Montgomery product's 332
ZDEV fr_t tab_fold_at(const TabDev& t, uint32_t j, uint32_t n, const fr_t& vm, const fr_t& vp) {
    if (!t.s32) return fold_at(t.slo, t.shi, j, n, vm);
    const int32_t x = t.s32[j], y = t.s32[j + n];
    return fr_add(fr_from_i64(x), fr_mul_i64s(vp, (int64_t)y - x));
}
// the plain challenge of a relayed or passed vm (Montgomery form), in scalar registers
ZDEV fr_t plain_uniform(const fr_t& vm) {
    fr_t one = fr_zero();
    one.v[0] = 1;
    fr_t v = mont_mul_ol(vm, one);
#pragma unroll
    for (int k = 0; k < 8; k++) v.v[k] = __builtin_amdgcn_readfirstlane(v.v[k]);
    return v;
}
static inline TabDev tab_dev(const Tab& t) {
    return TabDev{reinterpret_cast<const uint4*>(t.src.lo()), reinterpret_cast<const uint4*>(t.src.hi()),
                  reinterpret_cast<uint4*>(t.dst.lo()), reinterpret_cast<uint4*>(t.dst.hi()), nullptr};
}
// entries i and i+h of this round's table (folding the previous round's table of size 2n
// when fold is set, and storing the folded pair)
ZDEV void load_pair(const TabDev& t, uint32_t i, uint32_t h, uint32_t n, int fold, const fr_t& vm,
                    fr_t& x0, fr_t& x1) {
    if (fold) {
        x0 = tab_fold_at(t, i, n, vm);
        st_fr(t.dlo, t.dhi, i, x0);
        __builtin_amdgcn_sched_barrier(0);  // one fold's temporaries at a time
        x1 = tab_fold_at(t, i + h, n, vm);
        st_fr(t.dlo, t.dhi, i + h, x1);
    } else {
        x0 = tab_ld(t, i);
        x1 = tab_ld(t, i + h);
    }
}
// the same with the plain challenge for an int32 table's fold (see tab_fold_at)
ZDEV void load_pair(const TabDev& t, uint32_t i, uint32_t h, uint32_t n, int fold, const fr_t& vm, const fr_t& vp,
                    fr_t& x0, fr_t& x1) {
    if (fold) {
        x0 = tab_fold_at(t, i, n, vm, vp);
        st_fr(t.dlo, t.dhi, i, x0);
        __builtin_amdgcn_sched_barrier(0);
        x1 = tab_fold_at(t, i + h, n, vm, vp);
        st_fr(t.dlo, t.dhi, i + h, x1);
    } else {
        x0 = tab_ld(t, i);
        x1 = tab_ld(t, i + h);
    }
}
__global__ void k_fold(TabDev t, uint32_t h, fr_t vm) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < h; i += gridDim.x * blockDim.x)
        st_fr(t.dlo, t.dhi, i, fold_at(t.slo, t.shi, i, h, vm));
}
void launch_fold(hipStream_t s, Tab t, uint32_t h, const uint32_t* v_m_host) {
    k_fold<<<grid_for(h, NT, 8192), NT, 0, s>>>(tab_dev(t), h, to_fr(v_m_host));
}
// calls f with the loader of an in-place operand
template <typename F>
static void with_loader(const Src& x, F&& f) {
    if (x.kind == 0) {
        DevPlanes p{(uint32_t*)x.p, x.cap};
        f(LdPlanes{PL_LO(p), PL_HI(p)});
    } else if (x.kind == 1) {
        f(LdI32{(const int32_t*)x.p});
    } else {
        f(LdI64{(const int64_t*)x.p});
    }
}
// c b for the scalar c (Montgomery form cm, plain c): one Montgomery product, or with an
// int32 b the 32-bit multiply
template <typename LB>
ZDEV fr_t scale_of(const fr_t& cm, const fr_t&, const LB& b, uint32_t i) {
    return mont_mul(cm, b(i));
}
ZDEV fr_t scale_of(const fr_t&, const fr_t& c, const LdI32& b, uint32_t i) { return fr_mul_i64s(c, b.p[i]); }
template <typename LA, typename LB>
__global__ void k_axpy(LA a, fr_t cm, fr_t c, LB b, uint32_t n, uint4* olo, uint4* ohi) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        st_fr(olo, ohi, i, fr_add(a(i), scale_of(cm, c, b, i)));
}
void launch_axpy(hipStream_t s, Src a, const uint32_t* c_host, const uint32_t* c_m_host, Src b, uint32_t n,
                 DevPlanes out) {
    const fr_t cm = to_fr(c_m_host), c = to_fr(c_host);
    with_loader(a, [&](auto la) {
        with_loader(b, [&](auto lb) {
            k_axpy<<<grid_for(n, NT, 8192), NT, 0, s>>>(la, cm, c, lb, n, PL_LO(out), PL_HI(out));
        });
    });
}
// the plain product a b: two Montgomery products (the second by 2^512 mod r), or with an
// int32 operand the 32-bit multiply, or with two int32 operands the exact 64-bit product
template <typename LA, typename LB>
ZDEV fr_t prod_of(const LA& a, const LB& b, uint32_t i) {
    return mont_mul(mont_mul(a(i), b(i)), r2_m());
}
template <typename LA>
ZDEV fr_t prod_of(const LA& a, const LdI32& b, uint32_t i) {
    return fr_mul_i64s(a(i), b.p[i]);
}
template <typename LB>
ZDEV fr_t prod_of(const LdI32& a, const LB& b, uint32_t i) {
    return fr_mul_i64s(b(i), a.p[i]);
}
ZDEV fr_t prod_of(const LdI32& a, const LdI32& b, uint32_t i) { return fr_from_i64((int64_t)a.p[i] * b.p[i]); }
template <typename LA, typename LB>
__global__ void k_hadamard(LA a, LB b, uint32_t n, uint4* olo, uint4* ohi) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        st_fr(olo, ohi, i, prod_of(a, b, i));
}
// int32 x int32 -> the exact int64 product
__global__ void k_hadamard_i64(const int32_t* __restrict__ a, const int32_t* __restrict__ b, uint32_t n, int64_t* out) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        out[i] = (int64_t)a[i] * b[i];
}
void launch_hadamard_i64(hipStream_t s, const int32_t* a, const int32_t* b, uint32_t n, int64_t* out) {
    k_hadamard_i64<<<grid_for(n, NT, 8192), NT, 0, s>>>(a, b, n, out);
}
void launch_hadamard(hipStream_t s, Src a, Src b, uint32_t n, DevPlanes out) {
    with_loader(a, [&](auto la) {
        with_loader(b, [&](auto lb) {
            k_hadamard<<<grid_for(n, NT, 8192), NT, 0, s>>>(la, lb, n, PL_LO(out), PL_HI(out));
        });
    });
}

// ------------------------------------------------------------------------------------
// logUp: multiplicities, mapping, batched inversion
// ------------------------------------------------------------------------------------
// Histogram update with wave aggregation: the lanes holding the same index as the first
// active lane add their count with one atomic (zero padding makes long runs of one index);
// the others add individually.  Indices >= N raise *bad.  All lanes of the wave call it.
ZDEV void hist_add(uint32_t idx, bool valid, uint32_t N, uint32_t* counts, uint32_t* bad) {
    const bool in = valid && idx < N;
    if (valid && idx >= N) atomicOr(bad, 1u);
    const uint64_t act = __ballot(in);
    if (!act) return;
    const int leader = __ffsll((unsigned long long)act) - 1;
    const uint32_t lidx = __shfl(idx, leader, 64);
    const bool same = in && idx == lidx;
    const uint64_t sm = __ballot(same);
    if (same) {
        if ((int)(threadIdx.x & 63) == leader) atomicAdd(&counts[lidx], (uint32_t)__popcll(sm));
    } else if (in) {
        atomicAdd(&counts[idx], 1u);
    }
}
// limb 0 of the field element (v - low) for int32 v, low
ZDEV uint32_t lu_index_i32(int32_t v, int32_t low) {
    int64_t d = (int64_t)v - low;
    return d >= 0 ? (uint32_t)d : (uint32_t)(1u - (uint32_t)(-d));
}
__global__ void k_lu_count_planes(const uint4* lo, const uint4* hi, uint32_t n, fr_t low,
                                  uint32_t N, uint32_t* counts, uint32_t* bad) {
    for (uint32_t base = blockIdx.x * blockDim.x; base < n; base += gridDim.x * blockDim.x) {
        const uint32_t i = base + threadIdx.x;
        uint32_t idx = 0;
        if (i < n) idx = fr_sub(ld_fr(lo, hi, i), low).v[0];  // limb 0 (tlookup.cu:419)
        hist_add(idx, i < n, N, counts, bad);
    }
}
__global__ void k_lu_count_i32(const int32_t* __restrict__ S, uint32_t n, int32_t low, uint32_t N,
                               uint32_t* counts, uint32_t* bad) {
    for (uint32_t base = blockIdx.x * blockDim.x; base < n; base += gridDim.x * blockDim.x) {
        const uint32_t i = base + threadIdx.x;
        const uint32_t idx = i < n ? lu_index_i32(S[i], low) : 0u;
        hist_add(idx, i < n, N, counts, bad);
    }
}
__global__ void k_counts_to_planes(const uint32_t* __restrict__ counts, uint32_t N, uint4* lo,
                                   uint4* hi) {
    for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < N; j += gridDim.x * blockDim.x) {
        fr_t m = fr_zero();
        m.v[0] = counts[j];
        st_fr(lo, hi, j, m);
    }
}
void launch_lu_count_planes(hipStream_t s, DevPlanes S, uint32_t n, const uint32_t* low_host,
                            uint32_t N, uint32_t* counts, uint32_t* bad) {
    k_lu_count_planes<<<grid_for(n, NT, 8192), NT, 0, s>>>(PL_LO(S), PL_HI(S), n, to_fr(low_host),
                                                         N, counts, bad);
}
void launch_lu_count_i32(hipStream_t s, const int32_t* S, uint32_t n, int32_t low, uint32_t N,
                         uint32_t* counts, uint32_t* bad) {
    k_lu_count_i32<<<grid_for(n, NT, 8192), NT, 0, s>>>(S, n, low, N, counts, bad);
}
void launch_counts_to_planes(hipStream_t s, const uint32_t* counts, uint32_t N, DevPlanes m) {
    k_counts_to_planes<<<grid_for(N, NT, 8192), NT, 0, s>>>(counts, N, PL_LO(m), PL_HI(m));
}
// ---- multiplicities by LDS histograms (see HistArgs) ----
// index of entry i (limb 0 of S[i] - low), and whether it lies in the table
ZDEV uint32_t hist_index(const HistArgs& a, uint32_t i) {
    if (a.S.kind == 1) return lu_index_i32(reinterpret_cast<const int32_t*>(a.S.p)[i], a.low);
    const uint4* lo = reinterpret_cast<const uint4*>(a.S.p);
    return fr_sub(ld_fr(lo, lo + a.S.cap, i), to_fr(a.low_fr)).v[0];
}
// pass 1: per tile of ZKH_HIST_TILE entries, the count of each bucket
__global__ __launch_bounds__(NT) void k_hist_tiles(HistArgs a) {
    __shared__ uint32_t cnt[ZKH_HIST_MAX_BUCKETS];
    for (uint32_t b = threadIdx.x; b < a.nbuckets; b += NT) cnt[b] = 0;
    __syncthreads();
    const uint32_t base = blockIdx.x * ZKH_HIST_TILE;
    bool bad = false;
    for (uint32_t k = threadIdx.x; k < ZKH_HIST_TILE; k += NT) {
        const uint32_t i = base + k;
        if (i >= a.n) break;
        const uint32_t idx = hist_index(a, i);
        if (idx >= a.N) bad = true;
        else atomicAdd(&cnt[idx >> ZKH_HIST_BITS], 1u);
    }
    if (bad) *a.bad = a.tag;
    __syncthreads();
    for (uint32_t b = threadIdx.x; b < a.nbuckets; b += NT) a.tile_cnt[(size_t)b * a.ntiles + blockIdx.x] = cnt[b];
}
// pass 2: one block per bucket: exclusive prefix of its tile counts (in place) and its total
__global__ __launch_bounds__(NT) void k_hist_rows(HistArgs a) {
    __shared__ uint32_t part[NT];
    uint32_t* row = a.tile_cnt + (size_t)blockIdx.x * a.ntiles;
    const uint32_t per = (a.ntiles + NT - 1) / NT;
    const uint32_t t0 = threadIdx.x * per, t1 = min(a.ntiles, t0 + per);
    uint32_t loc = 0;
    for (uint32_t t = t0; t < t1; t++) loc += row[t];
    part[threadIdx.x] = loc;
    __syncthreads();
    for (uint32_t off = 1; off < NT; off <<= 1) {  // inclusive scan of the thread sums
        const uint32_t v = threadIdx.x >= off ? part[threadIdx.x - off] : 0u;
        __syncthreads();
        part[threadIdx.x] += v;
        __syncthreads();
    }
    uint32_t run = threadIdx.x ? part[threadIdx.x - 1] : 0u;
    for (uint32_t t = t0; t < t1; t++) {
        const uint32_t c = row[t];
        row[t] = run;
        run += c;
    }
    if (threadIdx.x == NT - 1) a.bucket_info[4 * blockIdx.x + 1] = part[NT - 1];
}
// pass 3 (one block): bucket starts, slots per bucket and the slot work list
__global__ __launch_bounds__(NT) void k_hist_plan(HistArgs a) {
    __shared__ uint32_t st[ZKH_HIST_MAX_BUCKETS], sl[ZKH_HIST_MAX_BUCKETS];
    for (uint32_t b = threadIdx.x; b < a.nbuckets; b += NT) st[b] = a.bucket_info[4 * b + 1];
    __syncthreads();
    if (threadIdx.x == 0) {  // serial scans over at most 1,024 buckets, in LDS
        uint32_t start = 0, slot = 0;
        for (uint32_t b = 0; b < a.nbuckets; b++) {
            const uint32_t tot = st[b];
            st[b] = start;
            sl[b] = slot;
            start += tot;
            slot += (tot + ZKH_HIST_CHUNK - 1) / ZKH_HIST_CHUNK;
        }
        *a.nslots = slot;
    }
    __syncthreads();
    for (uint32_t b = threadIdx.x; b < a.nbuckets; b += NT) {
        const uint32_t tot = a.bucket_info[4 * b + 1], ns = (tot + ZKH_HIST_CHUNK - 1) / ZKH_HIST_CHUNK;
        a.bucket_info[4 * b + 0] = st[b];
        a.bucket_info[4 * b + 2] = sl[b];
        a.bucket_info[4 * b + 3] = ns;
        for (uint32_t s = 0; s < ns; s++) {
            uint32_t* w = a.work + 4 * (size_t)(sl[b] + s);
            w[0] = b;
            w[1] = st[b] + s * ZKH_HIST_CHUNK;
            w[2] = min(ZKH_HIST_CHUNK, tot - s * ZKH_HIST_CHUNK);
        }
    }
}
// pass 4: scatter each tile's low index bits to its bucket's range (LDS cursors)
__global__ __launch_bounds__(NT) void k_hist_scatter(HistArgs a) {
    __shared__ uint32_t cur[ZKH_HIST_MAX_BUCKETS];
    for (uint32_t b = threadIdx.x; b < a.nbuckets; b += NT)
        cur[b] = a.bucket_info[4 * b] + a.tile_cnt[(size_t)b * a.ntiles + blockIdx.x];
    __syncthreads();
    const uint32_t base = blockIdx.x * ZKH_HIST_TILE;
    for (uint32_t k = threadIdx.x; k < ZKH_HIST_TILE; k += NT) {
        const uint32_t i = base + k;
        if (i >= a.n) break;
        const uint32_t idx = hist_index(a, i);
        if (idx >= a.N) continue;
        const uint32_t pos = atomicAdd(&cur[idx >> ZKH_HIST_BITS], 1u);
        a.part[pos] = (uint16_t)(idx & (ZKH_HIST_BINS - 1));
    }
}
// LDS histogram update aggregated over the lanes of a wave holding the leader's bin
ZDEV void lds_hist_add(uint32_t* h, uint32_t bin, bool valid) {
    const uint64_t act = __ballot(valid);
    if (!act) return;
    const int leader = __ffsll((unsigned long long)act) - 1;
    const uint32_t lb = __shfl(bin, leader, 64);
    const bool same = valid && bin == lb;
    const uint64_t sm = __ballot(same);
    if (same) {
        if ((int)(threadIdx.x & 63) == leader) atomicAdd(&h[lb], (uint32_t)__popcll(sm));
    } else if (valid) {
        atomicAdd(&h[bin], 1u);
    }
}
#define NTH 512
// pass 5: one block per work slot: its indices counted in a 64 KB LDS histogram, stored
// (direct: one bucket, slot s reads input entries [s CHUNK, (s + 1) CHUNK) itself)
template <int direct>
__global__ __launch_bounds__(NTH) void k_hist_slots(HistArgs a) {
    __shared__ uint32_t h[ZKH_HIST_BINS];
    const uint32_t slot = blockIdx.x;
    uint32_t begin, count;
    if (direct) {
        begin = slot * ZKH_HIST_CHUNK;
        count = min(ZKH_HIST_CHUNK, a.n - begin);
    } else {
        if (slot >= *a.nslots) return;  // uniform per block
        begin = a.work[4 * slot + 1];
        count = a.work[4 * slot + 2];
    }
    for (uint32_t j = threadIdx.x; j < ZKH_HIST_BINS; j += NTH) h[j] = 0;
    __syncthreads();
    bool bad = false;
    for (uint32_t k0 = 0; k0 < count; k0 += NTH) {  // every lane takes part in the wave votes
        const uint32_t k = k0 + threadIdx.x;
        uint32_t bin = 0;
        bool valid = k < count;
        if (valid) {
            if (direct) {
                const uint32_t idx = hist_index(a, begin + k);
                if (idx >= a.N) {
                    bad = true;
                    valid = false;
                }
                bin = idx;
            } else {
                bin = a.part[begin + k];
            }
        }
        lds_hist_add(h, bin, valid);
    }
    if (bad) *a.bad = a.tag;
    __syncthreads();
    uint4* out = reinterpret_cast<uint4*>(a.slot_hist + (size_t)slot * ZKH_HIST_BINS);
    for (uint32_t j = threadIdx.x; j < ZKH_HIST_BINS / 4; j += NTH)
        out[j] = make_uint4(h[4 * j], h[4 * j + 1], h[4 * j + 2], h[4 * j + 3]);
}
// pass 6: m[j] = sum of bin j over its bucket's slots, as a field element (direct: the
// one bucket's direct_slots slots, possibly none)
__global__ void k_hist_sum(HistArgs a, int direct, uint32_t direct_slots, uint4* lo, uint4* hi, int32_t* out32) {
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= a.N) return;
    uint32_t s0, ns;
    if (direct) {
        s0 = 0;
        ns = direct_slots;
    } else {
        const uint32_t b = j >> ZKH_HIST_BITS;
        s0 = a.bucket_info[4 * b + 2];
        ns = a.bucket_info[4 * b + 3];
    }
    const uint32_t* h = a.slot_hist + (size_t)s0 * ZKH_HIST_BINS + (j & (ZKH_HIST_BINS - 1));
    uint32_t c = 0, s = 0;
    for (; s + 8 <= ns; s += 8) {  // eight loads in flight (a skewed bucket has many slots)
        uint32_t v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = h[(size_t)(s + u) * ZKH_HIST_BINS];
#pragma unroll
        for (int u = 0; u < 8; u++) c += v[u];
    }
    for (; s < ns; s++) c += h[(size_t)s * ZKH_HIST_BINS];
    if (out32) {
        out32[j] = (int32_t)c;
        return;
    }
    fr_t m = fr_zero();
    m.v[0] = c;
    st_fr(lo, hi, j, m);
}
static size_t align16(size_t x) { return (x + 15) & ~(size_t)15; }
size_t hist_scratch_bytes(uint32_t n, uint32_t N) {
    const uint32_t nb = (N + ZKH_HIST_BINS - 1) / ZKH_HIST_BINS, nt = (n + ZKH_HIST_TILE - 1) / ZKH_HIST_TILE;
    const uint32_t ms = nb + (n + ZKH_HIST_CHUNK - 1) / ZKH_HIST_CHUNK;
    return align16((size_t)nb * nt * 4) + align16((size_t)nb * 16) + align16((size_t)ms * 16) + 16 +
           align16((size_t)n * 2) + (size_t)ms * ZKH_HIST_BINS * 4;
}
void launch_hist(hipStream_t s, HistArgs a, void* scratch, DevPlanes m, int32_t* m32) {
    a.nbuckets = (a.N + ZKH_HIST_BINS - 1) / ZKH_HIST_BINS;
    a.ntiles = (a.n + ZKH_HIST_TILE - 1) / ZKH_HIST_TILE;
    a.max_slots = a.nbuckets + (a.n + ZKH_HIST_CHUNK - 1) / ZKH_HIST_CHUNK;
    uint8_t* p = static_cast<uint8_t*>(scratch);
    a.tile_cnt = reinterpret_cast<uint32_t*>(p);
    p += align16((size_t)a.nbuckets * a.ntiles * 4);
    a.bucket_info = reinterpret_cast<uint32_t*>(p);
    p += align16((size_t)a.nbuckets * 16);
    a.work = reinterpret_cast<uint32_t*>(p);
    p += align16((size_t)a.max_slots * 16);
    a.nslots = reinterpret_cast<uint32_t*>(p);
    p += 16;
    a.part = reinterpret_cast<uint16_t*>(p);
    p += align16((size_t)a.n * 2);
    a.slot_hist = reinterpret_cast<uint32_t*>(p);
    const uint32_t gsum = (a.N + NT - 1) / NT;
    if (a.nbuckets == 1) {  // one LDS histogram covers the table: slots read the input
        const uint32_t ns = (a.n + ZKH_HIST_CHUNK - 1) / ZKH_HIST_CHUNK;
        if (ns) k_hist_slots<1><<<ns, NTH, 0, s>>>(a);
        k_hist_sum<<<gsum, NT, 0, s>>>(a, 1, ns, PL_LO(m), PL_HI(m), m32);
        return;
    }
    k_hist_tiles<<<a.ntiles, NT, 0, s>>>(a);
    k_hist_rows<<<a.nbuckets, NT, 0, s>>>(a);
    k_hist_plan<<<1, NT, 0, s>>>(a);
    k_hist_scatter<<<a.ntiles, NT, 0, s>>>(a);
    k_hist_slots<0><<<a.max_slots, NTH, 0, s>>>(a);
    k_hist_sum<<<gsum, NT, 0, s>>>(a, 0, 0, PL_LO(m), PL_HI(m), m32);
}

__global__ void k_lu_map_planes(const uint4* lo, const uint4* hi, uint32_t n, fr_t low,
                                const uint4* mlo, const uint4* mhi, uint32_t N, uint4* olo,
                                uint4* ohi) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        uint32_t idx = fr_sub(ld_fr(lo, hi, i), low).v[0];
        st_fr(olo, ohi, i, idx < N ? ld_fr(mlo, mhi, idx) : fr_zero());
    }
}
template <typename LM>
__global__ void k_lu_map_i32(const int32_t* __restrict__ S, uint32_t n, int32_t low, LM mapped, uint32_t N,
                             uint4* olo, uint4* ohi) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        uint32_t idx = lu_index_i32(S[i], low);
        st_fr(olo, ohi, i, idx < N ? mapped(idx) : fr_zero());
    }
}
void launch_lu_map_planes(hipStream_t s, DevPlanes S, uint32_t n, const uint32_t* low_host,
                          DevPlanes mapped, DevPlanes out) {
    k_lu_map_planes<<<grid_for(n, NT, 8192), NT, 0, s>>>(PL_LO(S), PL_HI(S), n, to_fr(low_host),
                                                       PL_LO(mapped), PL_HI(mapped), mapped.cap,
                                                       PL_LO(out), PL_HI(out));
}
// S_out[i] = mapped[j] as int32, j = (S[i] - low).limb0 (0 outside the table, which the
// multiplicity pass flags): the mapping of an int32 table keeps its 4-byte entries
template <typename LS>
__global__ void k_lu_map_to_i32(LS S, uint32_t n, fr_t low, const int32_t* __restrict__ mapped, uint32_t N,
                                int32_t* out) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const uint32_t j = fr_sub(S(i), low).v[0];
        out[i] = j < N ? mapped[j] : 0;
    }
}
void launch_lu_map_to_i32(hipStream_t s, Src S, uint32_t n, const uint32_t* low_host, const int32_t* mapped,
                          uint32_t N, int32_t* out) {
    const fr_t low = to_fr(low_host);
    with_loader(S, [&](auto ls) { k_lu_map_to_i32<<<grid_for(n, NT, 8192), NT, 0, s>>>(ls, n, low, mapped, N, out); });
}
void launch_lu_map_i32(hipStream_t s, const int32_t* S, uint32_t n, int32_t low, Src mapped, uint32_t N,
                       DevPlanes out) {
    with_loader(mapped, [&](auto lm) {
        k_lu_map_i32<<<grid_for(n, NT, 8192), NT, 0, s>>>(S, n, low, lm, N, PL_LO(out), PL_HI(out));
    });
}
// The tuple lookup's witness side from the table side: with j = (G[i] - low).limb0 (the
// reference's index, tlookup.cu:469-482), comb[i] = G[i] + r mapped[j] (the combiner of
// zkob_glu.cu:155 with S = mapped[j], the product formed as k_axpy forms it) and, where
// T[j] == G[i] (comb[i] is then T_comb[j]), A[i] = Binv[j] = 1/(T_comb[j] + beta).
// *flags |= 1 for j outside [0, N) (nothing written at i), |= 2 for T[j] != G[i] (A[i] left
// for the caller's direct inversion).  tlen > 0: T is the range table low + min(j, tlen - 1),
// so T[j] == G[i] iff G[i] - low is the integer j < tlen, and T is not read.  Without Comb
// (a plain range lookup: A = 1/(G + beta)) neither mapped nor comb is touched.  SeqS: the
// loader `mapped` is the caller's S = mapped[(G - low).limb0] itself, read at i (sequential)
// instead of mapped at j (a random 4-byte read per entry).
template <bool Comb, bool SeqS, typename LG, typename LT, typename LM>
__global__ void k_lu_tuple_gather(LG G, uint32_t n, fr_t low, LT T, uint32_t tlen, LM mapped, uint32_t N, fr_t rm,
                                  fr_t r,
                                  const uint4* __restrict__ blo, const uint4* __restrict__ bhi,
                                  const uint32_t* __restrict__ baos, uint4* clo, uint4* chi, uint4* alo, uint4* ahi,
                                  uint32_t* flags, uint32_t tag) {
    uint32_t f = 0;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        const fr_t g = G(i);
        const fr_t d = fr_sub(g, low);
        const uint32_t j = d.v[0];
        if (j >= N) {
            f |= 1u;
            continue;
        }
        if constexpr (Comb) st_fr(clo, chi, i, fr_add(g, scale_of(rm, r, mapped, SeqS ? i : j)));
        bool same = true;
        if (tlen) {
            same = j < tlen;
            for (int k = 1; k < 8; k++) same = same && d.v[k] == 0;
        } else {
            const fr_t t = T(j);
            for (int k = 0; k < 8; k++) same = same && t.v[k] == g.v[k];
        }
        if (same) {
            if (baos) {  // one 32-byte line
                const uint4* q = reinterpret_cast<const uint4*>(baos + 8 * (size_t)j);
                alo[i] = q[0];
                ahi[i] = q[1];
            } else {
                alo[i] = blo[j];
                ahi[i] = bhi[j];
            }
        } else {
            f |= 2u;
        }
    }
    // one store per wave that saw a flag: flags[0] (a witness outside the table), flags[1]
    // (a witness that is not the table's entry at its index) receive the call's tag
    const uint64_t any1 = __ballot(f & 1u), any2 = __ballot(f & 2u);
    if ((threadIdx.x & 63) == 0) {
        if (any1) flags[0] = tag;
        if (any2) flags[1] = tag;
    }
}
void launch_lu_tuple_gather(hipStream_t s, Src G, uint32_t n, const uint32_t* low_host, Src T, uint32_t tlen,
                            Src mapped, int seq_s, uint32_t N, const uint32_t* r_host, const uint32_t* r_m_host,
                            DevPlanes Binv, const uint32_t* binv_aos, DevPlanes comb, DevPlanes A, uint32_t* flags,
                            uint32_t tag) {
    const fr_t low = to_fr(low_host), r = to_fr(r_host), rm = to_fr(r_m_host);
    const uint32_t g = grid_for(n, NT, 8192);
    with_loader(G, [&](auto lg) {
        with_loader(T, [&](auto lt) {
            with_loader(mapped, [&](auto lm) {
                if (seq_s)
                    k_lu_tuple_gather<true, true><<<g, NT, 0, s>>>(lg, n, low, lt, tlen, lm, N, rm, r, PL_LO(Binv),
                                                                    PL_HI(Binv), binv_aos, PL_LO(comb), PL_HI(comb),
                                                                    PL_LO(A), PL_HI(A), flags, tag);
                else
                    k_lu_tuple_gather<true, false><<<g, NT, 0, s>>>(lg, n, low, lt, tlen, lm, N, rm, r, PL_LO(Binv),
                                                                     PL_HI(Binv), binv_aos, PL_LO(comb), PL_HI(comb),
                                                                     PL_LO(A), PL_HI(A), flags, tag);
            });
        });
    });
}
void launch_lu_range_gather(hipStream_t s, Src S, uint32_t n, const uint32_t* low_host, Src T, uint32_t tlen,
                            uint32_t N, DevPlanes Binv, DevPlanes A, uint32_t* flags, uint32_t tag) {
    const fr_t low = to_fr(low_host);
    with_loader(S, [&](auto ls) {
        with_loader(T, [&](auto lt) {
            k_lu_tuple_gather<false, false><<<grid_for(n, NT, 8192), NT, 0, s>>>(
                ls, n, low, lt, tlen, LdI32{nullptr}, N, fr_t{}, fr_t{}, PL_LO(Binv), PL_HI(Binv), nullptr, nullptr,
                nullptr, PL_LO(A), PL_HI(A), flags, tag);
        });
    });
}

// Batched inversion (Montgomery's trick) in three Montgomery products per entry.  With
// M(a, b) = a b 2^-256, the running products P_0 = 2^256, P_j = M(P_{j-1}, x_j) of the plain
// values x_j need no conversion into the Montgomery domain, and for Y_j = 1/P_j:
//   1/x_j = M(P_{j-1}, Y_j)   and   Y_{j-1} = M(x_j, Y_j)
// (P_j = P_{j-1} x_j / 2^256), so the backward walk yields plain inverses directly.  The
// same identities combine totals: for Q = M(a, b), 1/a = M(b, 1/Q).  Block b covers
// CHK*NT entries (CHK = inv_chunk(n)); thread t owns entries base + j*NT + t.  Pass 1 stores P_j in A, and
// a product tree over the thread totals (others_tree) gives each thread the M-product of
// all OTHER threads' totals; the block total goes to blockprod.  Between the
// passes, k_inv_blocks turns the block totals into "all other blocks" products and
// publishes the grand product G, whose plain inverse the host computes once.  Pass 2 walks
// each thread's entries backwards.  Zero entries (x + beta = 0) take 2^256, M's identity,
// in the products and produce 0, the reference's Fermat convention; pass 1 sets *zflag to
// the call's tag when it meets one (the inverse then has a zero entry).
// entries per thread: 16 for tables that fill the device several times over (the chains'
// products then run at the device's rate), 4 below 2^20 entries, where a 16-long chain of
// dependent products on few blocks sets the pass's time
static inline uint32_t inv_chunk(uint32_t n) { return n >= (1u << 20) ? 16u : 4u; }
// The M-product of all OTHER leaves, for each of NL leaves (NL a power of 2, at most the
// block size; thread t < NL gives leaf t): a product tree up, tr[k] = M(tr[2k], tr[2k + 1])
// with the leaves at tr[NL + t] and the block total at tr[1], then the products outside
// each subtree down, out[1] = 2^256 (the empty product), out[c] = M(out[c / 2], tr[c ^ 1]),
// so out[NL + t] is the product of every leaf but t.  An M-product of a set does not depend
// on its bracketing, so this equals the prefix-times-suffix scan, with 3 NL products
// instead of 2 NL log2(NL) over 2 log2(NL) levels.  Every thread of the block calls it.
template <uint32_t NL>
ZDEV fr_t others_tree(fr_t* tr, fr_t* out, const fr_t& v) {
    const uint32_t t = threadIdx.x;
    if (t < NL) tr[NL + t] = v;
    __syncthreads();
    for (uint32_t w = NL / 2; w >= 1; w >>= 1) {  // nodes [w, 2w)
        if (t < w) tr[w + t] = mont_mul(tr[2 * (w + t)], tr[2 * (w + t) + 1]);
        __syncthreads();
    }
    if (t == 0) out[1] = one_m();
    __syncthreads();
    for (uint32_t w = 1; w < NL; w <<= 1) {  // the children [2w, 4w) of nodes [w, 2w)
        if (t < 2 * w) {
            const uint32_t c = 2 * w + t;
            out[c] = mont_mul(out[c >> 1], tr[c ^ 1]);
        }
        __syncthreads();
    }
    return t < NL ? out[NL + t] : one_m();
}
template <uint32_t CHK>
__global__ __launch_bounds__(NT) void k_inv_pass1(const uint4* slo, const uint4* shi, uint32_t n,
                                                  fr_t beta, uint4* alo, uint4* ahi,
                                                  uint32_t* others, uint32_t* blockprod, uint32_t* zflag,
                                                  uint32_t tag) {
    __shared__ fr_t tr[2 * NT], out[2 * NT];
    const uint32_t t = threadIdx.x;
    const uint32_t base = blockIdx.x * NT * CHK;
    fr_t run = one_m();
    bool zero = false;
    for (uint32_t j = 0; j < CHK; j++) {
        uint32_t idx = base + j * NT + t;
        if (idx < n) {
            const fr_t x = fr_add(ld_fr(slo, shi, idx), beta);
            const bool z = fr_is_zero(x);
            zero = zero || z;
            run = mont_mul(run, z ? one_m() : x);
            st_fr(alo, ahi, idx, run);
        }
    }
    if (__ballot(zero) && (t & 63) == 0) *zflag = tag;  // one store per wave that met a zero
    st_aos(others, blockIdx.x * NT + t, others_tree<NT>(tr, out, run));
    if (t == 0) st_aos(blockprod, blockIdx.x, tr[1]);
}
// One block over the nb block products (Montgomery form): others[b] = product of all the
// other blocks' products, and the grand product P published (pub.host_out[0], then the
// flag) for the host to invert.  Thread t owns products [t*per, (t+1)*per).
#define NTI 256
__global__ __launch_bounds__(NTI) void k_inv_blocks(const uint32_t* __restrict__ bp, uint32_t nb,
                                                    uint32_t* others, Publish pub, const uint32_t* zflag,
                                                    uint32_t tag) {
    __shared__ fr_t tr[2 * NTI], out[2 * NTI];
    const uint32_t t = threadIdx.x;
    const uint32_t per = (nb + NTI - 1) / NTI;
    const uint32_t b0 = t * per, b1 = min(nb, b0 + per);
    fr_t loc = one_m();
    for (uint32_t b = b0; b < b1; b++) {  // local exclusive prefixes into others[]
        st_aos(others, b, loc);
        loc = mont_mul(loc, ld_aos(bp, b));
    }
    fr_t rs = others_tree<NTI>(tr, out, loc);  // the other threads' products
    for (int b = (int)b1 - 1; b >= (int)b0; b--) {  // times the local suffix
        st_aos(others, b, mont_mul(ld_aos(others, b), rs));
        rs = mont_mul(rs, ld_aos(bp, b));
    }
    if (t == 0) {
        st_aos(pub.host_out, 0, tr[1]);
        pub.host_out[8] = *zflag == tag ? 1u : 0u;  // pass 1 met a zero entry
        __threadfence_system();
        __hip_atomic_store(pub.host_flag, pub.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}
void launch_inv_blocks(hipStream_t s, const uint32_t* blockprod, uint32_t nb, uint32_t* others_blk,
                       Publish pub, const uint32_t* zflag, uint32_t tag) {
    k_inv_blocks<<<1, NTI, 0, s>>>(blockprod, nb, others_blk, pub, zflag, tag);
}
// 1/blockprod[b] = M(others_blk[b], 1/G), 1/(thread total) = M(others[t], 1/blockprod[b]);
// then each thread walks its entries backwards
template <uint32_t CHK>
__global__ __launch_bounds__(NT) void k_inv_pass2(const uint4* slo, const uint4* shi, uint32_t n,
                                                  fr_t beta, uint4* alo, uint4* ahi,
                                                  const uint32_t* __restrict__ others,
                                                  const uint32_t* __restrict__ others_blk, fr_t inv_total,
                                                  const uint32_t* invp, uint32_t* aos) {
    const uint32_t t = threadIdx.x;
    const uint32_t base = blockIdx.x * NT * CHK;
    if (invp) {  // 1/G from a relay: invp[0..8), invp[8] != 0 when the host abandoned the call
        if (invp[8]) return;
        inv_total = ld_aos(invp, 0);
    }
    const fr_t binv = mont_mul(inv_total, ld_aos(others_blk, blockIdx.x));
    fr_t y = mont_mul(binv, ld_aos(others, blockIdx.x * NT + t));
    for (int j = CHK - 1; j >= 0; j--) {
        uint32_t idx = base + (uint32_t)j * NT + t;
        if (idx >= n) continue;
        const fr_t x = fr_add(ld_fr(slo, shi, idx), beta);
        const bool z = fr_is_zero(x);
        const fr_t prev = j > 0 ? ld_fr(alo, ahi, idx - NT) : one_m();
        const fr_t inv = mont_mul(prev, y);
        y = mont_mul(z ? one_m() : x, y);
        st_fr(alo, ahi, idx, z ? fr_zero() : inv);
        if (aos) st_aos(aos, idx, z ? fr_zero() : inv);
    }
}
uint32_t inv_blocks(uint32_t n) {
    const uint32_t c = inv_chunk(n);
    return (n + NT * c - 1) / (NT * c);
}
void launch_inv_pass1(hipStream_t s, DevPlanes S, uint32_t n, const uint32_t* beta_host,
                      DevPlanes A, uint32_t* others, uint32_t* blockprod, uint32_t* zflag, uint32_t tag) {
    auto k = inv_chunk(n) == 16 ? k_inv_pass1<16> : k_inv_pass1<4>;
    k<<<inv_blocks(n), NT, 0, s>>>(PL_LO(S), PL_HI(S), n, to_fr(beta_host), PL_LO(A),
                                             PL_HI(A), others, blockprod, zflag, tag);
}
void launch_inv_pass2(hipStream_t s, DevPlanes S, uint32_t n, const uint32_t* beta_host,
                      DevPlanes A, const uint32_t* others, const uint32_t* others_blk,
                      const uint32_t* inv_total_host, const uint32_t* invp, uint32_t* aos) {
    auto k = inv_chunk(n) == 16 ? k_inv_pass2<16> : k_inv_pass2<4>;
    k<<<inv_blocks(n), NT, 0, s>>>(PL_LO(S), PL_HI(S), n, to_fr(beta_host), PL_LO(A), PL_HI(A), others,
                                             others_blk, inv_total_host ? to_fr(inv_total_host) : fr_t{}, invp,
                                             aos);
}

// ------------------------------------------------------------------------------------
// eq weighting for pair sums: eq(i, u[0..K)) = elo[i & 1023] * ehi(i >> 10)
// ------------------------------------------------------------------------------------
struct EqDev {
    const uint32_t* elo;
    const uint32_t* ehi;
    uint32_t K;
};
// device weight of index i (see EqW)
ZDEV fr_t eq_w(const EqDev& eq, uint32_t i) { return mont_mul_ol(ld_aos(eq.elo, i & 1023), ld_aos(eq.ehi, i >> 10)); }
// A thread whose pairs i = i0 + k s have a stride s that is a multiple of 1024 keeps one Elo
// factor, Elo[i0 & 1023], for all of them: its weighted products can take Ehi[i >> 10] alone
// (one product per pair less) and its weighted sums the Elo factor once at the end
// (elo_scale).  Worth it from two pairs per thread on.
ZDEV bool elo_factored(uint32_t h, uint32_t stride) { return (stride & 1023) == 0 && h >= 2 * stride; }
ZDEV fr_t pair_w(const EqDev& eq, uint32_t i, bool ef) { return ef ? ld_aos(eq.ehi, i >> 10) : eq_w(eq, i); }

#define SB() __builtin_amdgcn_sched_barrier(0)
// the product x y as a field element (x 1): a Montgomery product lifted by 2^512
ZDEV fr_t exact_mul(const fr_t& x, const fr_t& y) { return mont_mul_ol(mont_mul_ol(x, y), r2_m()); }
// blocks of a logUp phase-2 round (both groups; 256 CUs hold 768 of them at once)
#ifndef LU2_GRID
#define LU2_GRID 1536
#endif
// blocks of the derived (folding) logUp phase-2 round, the first phase-2 round with no zero
// inverse, and the folding eq-form Hadamard round
#ifndef ZKH_LU2D_GRID
#define ZKH_LU2D_GRID 1280
#endif
#ifndef ZKH_NZ_GRID
#define ZKH_NZ_GRID 1280
#endif
#ifndef ZKH_HPE_GRID
#define ZKH_HPE_GRID 1280
#endif
// Per-thread field accumulators kept in LDS (limb-quad planes, 16-byte lanes): registers
// then hold only the current stage's operands, which lifts the round kernels' occupancy.
template <int K>
struct LdsAcc {
    uint4* lo;  // [K][NT]
    uint4* hi;
    ZDEV void zero() {
#pragma unroll
        for (int k = 0; k < K; k++) st_fr(lo + k * NT, hi + k * NT, threadIdx.x, fr_zero());
    }
    ZDEV void add(int k, const fr_t& x) {
        const fr_t c = ld_fr(lo + k * NT, hi + k * NT, threadIdx.x);
        st_fr(lo + k * NT, hi + k * NT, threadIdx.x, fr_add(c, x));
    }
    ZDEV void get(fr_t* out) const {
#pragma unroll
        for (int k = 0; k < K; k++) out[k] = ld_fr(lo + k * NT, hi + k * NT, threadIdx.x);
    }
    // slots [0, nk) times the thread's Elo factor (see elo_factored)
    ZDEV void elo_scale(const EqDev& eq, uint32_t i0, int nk) {
        const fr_t e = ld_aos(eq.elo, i0 & 1023);
        for (int k = 0; k < nk; k++)
            st_fr(lo + k * NT, hi + k * NT, threadIdx.x, mont_mul_ol(ld_fr(lo + k * NT, hi + k * NT, threadIdx.x), e));
    }
};
// Tree over the block's LDS accumulators: level s adds entry t + s into entry t (t < s) of
// every plane, all threads sharing the K*s additions; afterwards entry 0 of plane k holds
// the block's sum k.  Cheaper than K 64-lane shuffle trees (one after the other) when the
// block's work is small.
template <int K>
ZDEV void lds_tree(const LdsAcc<K>& acc) {
    for (uint32_t s = NT / 2; s >= 1; s >>= 1) {
        __syncthreads();
        for (uint32_t q = threadIdx.x; q < K * s; q += NT) {
            const uint32_t k = q / s, t = q - k * s;
            uint4* lo = acc.lo + k * NT;
            uint4* hi = acc.hi + k * NT;
            st_fr(lo, hi, t, fr_add(ld_fr(lo, hi, t), ld_fr(lo, hi, t + s)));
        }
    }
    __syncthreads();
}
// reduce_publish over LDS accumulators: the block's sums by an LDS tree (entry 0 of each
// plane), then the partials and layout as reduce_publish.
template <int K>
ZDEV void reduce_publish_lds(const LdsAcc<K>& acc, const Publish& P, uint32_t job, uint32_t first, uint32_t nblk,
                             uint32_t local) {
    lds_tree<K>(acc);
    if (threadIdx.x < K) st_aos(P.part, (first + local) * K + threadIdx.x, ld_fr(acc.lo + threadIdx.x * NT, acc.hi + threadIdx.x * NT, 0));
    if (local == 0 && threadIdx.x == 0) publish_layout(P, job, first, nblk, K);
}
// the challenge of a relayed launch: false when the relay says the proof was abandoned
ZDEV bool relayed_vm(const uint32_t* vmp, fr_t& vm) {
    if (!vmp) return true;
    if (vmp[8]) return false;
#pragma unroll
    for (int i = 0; i < 8; i++) vm.v[i] = vmp[i];
    return true;
}
// First-round sums of a table X known to be 1/(Y + beta) entry-wise (inverse(0) = 0), with
// no fold owed: x (y + beta) is 1 for x != 0 and 0 for x = 0, so the two weighted products
// reduce to sums of the weight w = e 2^256 over the nonzero entries (the host takes them
// as sum e, removing the 2^256, where the general path's sums carry 2^-256); the third,
// w (x1 - x0)(y1 - y0), keeps its two products.  Accumulator slots 0, 1, 2 as the general
// path's.
ZDEV bool fr_nonzero(const fr_t& x) {
    uint32_t o = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) o |= x.v[i];
    return o != 0;
}
template <int K>
ZDEV void inverse_pair_sums(const fr_t& x0, const fr_t& x1, const fr_t& y0, const fr_t& y1, const fr_t& w,
                            LdsAcc<K>& acc) {
    acc.add(0, fr_nonzero(x0) ? w : fr_zero());
    acc.add(1, fr_nonzero(x1) ? w : fr_zero());
    const fr_t wdx = mont_mul_ol(w, fr_sub(x1, x0));
    SB();
    acc.add(2, mont_mul_ol(wdx, fr_sub(y1, y0)));
}
// the (A, S) group's first round with A = 1/(S + beta): sums 0..2 as above, 3, 4 sum a0, a1
ZDEV void lu_as_inverse(const TabDev& A, const TabDev& S, uint32_t i, uint32_t h, const EqDev& eq, LdsAcc<5>& acc) {
    const fr_t a0 = ld_fr(A.slo, A.shi, i), a1 = ld_fr(A.slo, A.shi, i + h);
    acc.add(3, a0);
    acc.add(4, a1);
    const fr_t w = eq_w(eq, i);
    SB();
    const fr_t s0 = ld_fr(S.slo, S.shi, i), s1 = ld_fr(S.slo, S.shi, i + h);
    inverse_pair_sums<5>(a0, a1, s0, s1, w, acc);
    SB();
}
// First round of a group whose table X is 1/(Y + beta) with no zero entry: x (y + beta) = 1
// for every pair entry, so the two weighted sums of those products are sum_i eq(i, u) = 1
// (the host takes them as such) and only w dx dy is formed.  A/S slots: 0 w da ds
// (x 2^-256), 1 a0, 2 a1.  B/T/m slots: 0 w db dt (x 2^-256), 1..3 m0 b0, m1 b1, dm db
// (exact, x 1).
ZDEV void lu_as_first_nz(const TabDev& A, const TabDev& S, uint32_t n, const EqDev& eq, uint32_t lb, uint32_t g,
                         const Publish& pub, uint4* accl, uint4* acch) {
    const uint32_t h = n >> 1;
    LdsAcc<3> acc{accl, acch};
    acc.zero();
    const bool ef = elo_factored(h, g * NT);
    for (uint32_t i = lb * NT + threadIdx.x; i < h; i += g * NT) {
        // every load of the iteration first: one wait for memory per pair
        const fr_t a0 = ld_fr(A.slo, A.shi, i), a1 = ld_fr(A.slo, A.shi, i + h);
        const fr_t s0 = ld_fr(S.slo, S.shi, i), s1 = ld_fr(S.slo, S.shi, i + h);
        const fr_t w = pair_w(eq, i, ef);
        SB();
        acc.add(1, a0);
        acc.add(2, a1);
        const fr_t ds = fr_sub(s1, s0);
        const fr_t wda = mont_mul_ol(w, fr_sub(a1, a0));
        SB();
        acc.add(0, mont_mul_ol(wda, ds));
        SB();
    }
    if (ef) acc.elo_scale(eq, lb * NT + threadIdx.x, 1);
    reduce_publish_lds<3>(acc, pub, 0, 0, g, lb);
}
// M32: m is an int32 table (m.s32), its entries taken as integers directly; otherwise field
// planes, whose small-integer entries take the same 32-bit multiply
template <bool M32>
ZDEV void lu_btm_first_nz(const TabDev& B, const TabDev& T, const TabDev& m, uint32_t n, const EqDev& eq, uint32_t lb,
                          uint32_t g, uint32_t ga, const Publish& pub, uint4* accl, uint4* acch) {
    const uint32_t h = n >> 1;
    LdsAcc<4> acc{accl, acch};
    acc.zero();
    const bool ef = elo_factored(h, g * NT);
    for (uint32_t i = lb * NT + threadIdx.x; i < h; i += g * NT) {
        // every load of the iteration first: one wait for memory per pair
        const fr_t b0 = ld_fr(B.slo, B.shi, i), b1 = ld_fr(B.slo, B.shi, i + h);
        const fr_t t0 = ld_fr(T.slo, T.shi, i), t1 = ld_fr(T.slo, T.shi, i + h);
        const fr_t dt = fr_sub(t1, t0);
        if constexpr (M32) {  // multiplicities are small integers: exact (x 1) by the 32-bit multiply
            const int64_t i0 = m.s32[i], i1 = m.s32[i + h];
            SB();
            acc.add(1, fr_mul_i64s(b0, i0));
            acc.add(2, fr_mul_i64s(b1, i1));
            acc.add(3, fr_mul_i64(fr_sub(b1, b0), i1 - i0));
        } else {
            const fr_t m0 = ld_fr(m.slo, m.shi, i), m1 = ld_fr(m.slo, m.shi, i + h);
            SB();
            int64_t i0, i1;
            if (fr_int32ish(m0, i0) && fr_int32ish(m1, i1)) {
                acc.add(1, fr_mul_i64s(b0, i0));
                acc.add(2, fr_mul_i64s(b1, i1));
                acc.add(3, fr_mul_i64(fr_sub(b1, b0), i1 - i0));
            } else {
                acc.add(1, exact_mul(m0, b0));
                SB();
                acc.add(2, exact_mul(m1, b1));
                SB();
                acc.add(3, exact_mul(fr_sub(m1, m0), fr_sub(b1, b0)));
            }
        }
        SB();
        const fr_t w = pair_w(eq, i, ef);
        SB();
        const fr_t wdb = mont_mul_ol(w, fr_sub(b1, b0));
        SB();
        acc.add(0, mont_mul_ol(wdb, dt));
        SB();
    }
    if (ef) acc.elo_scale(eq, lb * NT + threadIdx.x, 1);
    reduce_publish_lds<4>(acc, pub, 1, ga, g, lb);
}
// phase 2 (tlookup.cu:161-279 eval/sum/dotprod + reduce kernels, fused), one launch whose
// blocks [0, ga) take the (A, S) group and blocks [ga, ga + gb) the (B, T, m) group,
// publishing as jobs 0 and 1 of one round (each group keeps its fold, weights and sums in
// registers at a fraction of a single fused body's pressure; one launch instead of two
// halves the fixed cost of a small round).  The groups' block counts follow their work per
// pair (6 / 9 Montgomery products, 10 / 15 with the folds):
// job 0 (A, S): sum w*a0*s0, w*a1*s1, w*da*ds (x 2^-256), sum a0, sum a1  (s + beta)
// job 1 (B, T, m): sum w*b0*t0, w*b1*t1, w*db*dt, m0*b0, m1*b1, dm*db (x 2^-256)  (t + beta)
// derive (folding groups only): the sums at 1 are left out, the host taking them from the
// previous round's claims of each piece (q(0)(1 - u) + q(1) u = claim for the eq-weighted
// pieces, q(0) + q(1) = claim for the plain ones):
// job 0: sum w*a0*s0, w*da*ds, a0;  job 1: sum w*b0*t0, w*db*dt, m0*b0, dm*db
template <int fold, int derive>
ZDEV void lu_phase2_as(const TabDev& A, const TabDev& S, uint32_t n, const fr_t& vm, const fr_t& beta,
                       const EqDev& eq, const Publish& pub, uint32_t lb, uint32_t g, uint4* accl, uint4* acch,
                       int inv) {
    const uint32_t h = n >> 1;
    if constexpr (derive) {
        LdsAcc<3> acc{accl, acch};
        acc.zero();
        const bool ef = elo_factored(h, g * NT);
        for (uint32_t i = lb * NT + threadIdx.x; i < h; i += g * NT) {
            fr_t wa0, wda;
            {
                fr_t a0, a1;
                load_pair(A, i, h, n, 1, vm, a0, a1);
                SB();
                acc.add(2, a0);
                SB();
                const fr_t w = pair_w(eq, i, ef);
                SB();
                wa0 = mont_mul_ol(w, a0);
                SB();
                wda = mont_mul_ol(w, fr_sub(a1, a0));
            }
            SB();
            fr_t s0, s1;
            load_pair(S, i, h, n, 1, vm, s0, s1);
            SB();
            acc.add(0, mont_mul_ol(wa0, fr_add(s0, beta)));
            SB();
            acc.add(1, mont_mul_ol(wda, fr_sub(s1, s0)));
            SB();
        }
        if (ef) acc.elo_scale(eq, lb * NT + threadIdx.x, 2);
        reduce_publish_lds<3>(acc, pub, 0, 0, g, lb);
        return;
    }
    LdsAcc<5> acc{accl, acch};
    acc.zero();
    if (!fold && inv) {
        for (uint32_t i = lb * NT + threadIdx.x; i < h; i += g * NT) lu_as_inverse(A, S, i, h, eq, acc);
        reduce_publish_lds<5>(acc, pub, 0, 0, g, lb);
        return;
    }
    for (uint32_t i = lb * NT + threadIdx.x; i < h; i += g * NT) {
        fr_t wa0, wda;
        {
            fr_t a0, a1;
            load_pair(A, i, h, n, fold, vm, a0, a1);
            SB();
            acc.add(3, a0);
            acc.add(4, a1);
            SB();
            const fr_t w = eq_w(eq, i);
            SB();
            wa0 = mont_mul_ol(w, a0);
            SB();
            wda = mont_mul_ol(w, fr_sub(a1, a0));
        }
        SB();
        fr_t s0, s1;
        load_pair(S, i, h, n, fold, vm, s0, s1);
        SB();
        acc.add(0, mont_mul_ol(wa0, fr_add(s0, beta)));
        SB();
        acc.add(1, mont_mul_ol(fr_add(wa0, wda), fr_add(s1, beta)));
        SB();
        acc.add(2, mont_mul_ol(wda, fr_sub(s1, s0)));
        SB();
    }
    reduce_publish_lds<5>(acc, pub, 0, 0, g, lb);
}
template <int fold, int derive>
ZDEV void lu_phase2_btm(const TabDev& B, const TabDev& T, const TabDev& m, uint32_t n, const fr_t& vm,
                        const fr_t& beta, const EqDev& eq, const Publish& pub, uint32_t lb, uint32_t g, uint32_t ga,
                        uint4* accl, uint4* acch, int inv) {
    const uint32_t h = n >> 1;
    // partials after the (A, S) group's ga entries of K_as <= K sums: indices (ga + lb) * K + k
    if constexpr (derive) {
        LdsAcc<4> acc{accl, acch};
        acc.zero();
        const bool ef = elo_factored(h, g * NT);
        const fr_t vp = m.s32 ? plain_uniform(vm) : fr_zero();  // m's first fold
        for (uint32_t i = lb * NT + threadIdx.x; i < h; i += g * NT) {
            fr_t b0, b1;
            load_pair(B, i, h, n, 1, vm, b0, b1);
            SB();
            {
                fr_t m0, m1;
                load_pair(m, i, h, n, 1, vm, vp, m0, m1);
                SB();
                acc.add(2, mont_mul_ol(m0, b0));
                SB();
                acc.add(3, mont_mul_ol(fr_sub(m1, m0), fr_sub(b1, b0)));
            }
            SB();
            fr_t wb0, wdb;
            {
                const fr_t w = pair_w(eq, i, ef);
                SB();
                wb0 = mont_mul_ol(w, b0);
                SB();
                wdb = mont_mul_ol(w, fr_sub(b1, b0));
            }
            SB();
            fr_t t0, t1;
            load_pair(T, i, h, n, 1, vm, t0, t1);
            SB();
            acc.add(0, mont_mul_ol(wb0, fr_add(t0, beta)));
            SB();
            acc.add(1, mont_mul_ol(wdb, fr_sub(t1, t0)));
            SB();
        }
        if (ef) acc.elo_scale(eq, lb * NT + threadIdx.x, 2);
        reduce_publish_lds<4>(acc, pub, 1, ga, g, lb);
        return;
    }
    LdsAcc<6> acc{accl, acch};
    acc.zero();
    if (!fold && inv) {  // B = 1/(T + beta) unfolded (see inverse_pair_sums); 3..5 as below
        for (uint32_t i = lb * NT + threadIdx.x; i < h; i += g * NT) {
            const fr_t b0 = ld_fr(B.slo, B.shi, i), b1 = ld_fr(B.slo, B.shi, i + h);
            {  // multiplicities are small integers: sums 3..5 exact (x 1) by the 32-bit multiply
                const fr_t m0 = tab_ld(m, i), m1 = tab_ld(m, i + h);
                SB();
                int64_t i0, i1;
                if (fr_int32ish(m0, i0) && fr_int32ish(m1, i1)) {
                    acc.add(3, fr_mul_i64s(b0, i0));
                    acc.add(4, fr_mul_i64s(b1, i1));
                    acc.add(5, fr_mul_i64(fr_sub(b1, b0), i1 - i0));
                } else {
                    acc.add(3, exact_mul(m0, b0));
                    SB();
                    acc.add(4, exact_mul(m1, b1));
                    SB();
                    acc.add(5, exact_mul(fr_sub(m1, m0), fr_sub(b1, b0)));
                }
            }
            SB();
            const fr_t w = eq_w(eq, i);
            SB();
            const fr_t t0 = ld_fr(T.slo, T.shi, i), t1 = ld_fr(T.slo, T.shi, i + h);
            inverse_pair_sums<6>(b0, b1, t0, t1, w, acc);
            SB();
        }
        reduce_publish_lds<6>(acc, pub, 1, ga, g, lb);
        return;
    }
    for (uint32_t i = lb * NT + threadIdx.x; i < h; i += g * NT) {
        fr_t b0, b1;
        load_pair(B, i, h, n, fold, vm, b0, b1);
        SB();
        {
            fr_t m0, m1;
            load_pair(m, i, h, n, fold, vm, m0, m1);
            SB();
            acc.add(3, mont_mul_ol(m0, b0));
            SB();
            acc.add(4, mont_mul_ol(m1, b1));
            SB();
            acc.add(5, mont_mul_ol(fr_sub(m1, m0), fr_sub(b1, b0)));
        }
        SB();
        fr_t wb0, wdb;
        {
            const fr_t w = eq_w(eq, i);
            SB();
            wb0 = mont_mul_ol(w, b0);
            SB();
            wdb = mont_mul_ol(w, fr_sub(b1, b0));
        }
        SB();
        fr_t t0, t1;
        load_pair(T, i, h, n, fold, vm, t0, t1);
        SB();
        acc.add(0, mont_mul_ol(wb0, fr_add(t0, beta)));
        SB();
        acc.add(1, mont_mul_ol(fr_add(wb0, wdb), fr_add(t1, beta)));
        SB();
        acc.add(2, mont_mul_ol(wdb, fr_sub(t1, t0)));
        SB();
    }
    reduce_publish_lds<6>(acc, pub, 1, ga, g, lb);
}
// phase 1 (tlookup.cu:74-104 poly + reduce kernels, fused): the (A, S) group of phase 2 over
// the whole grid, same sums (derive as there)
template <int fold, int derive>
__global__ __launch_bounds__(NT) void k_lu_phase1(TabDev A, TabDev S, uint32_t n, fr_t vm, const uint32_t* vmp,
                                                  fr_t beta, EqDev eq, Publish pub, int inv) {
    if (!relayed_vm(vmp, vm)) return;
    constexpr int K = derive ? 3 : 5;
    __shared__ uint4 accl[K * NT], acch[K * NT];
    lu_phase2_as<fold, derive>(A, S, n, vm, beta, eq, pub, blockIdx.x, gridDim.x, accl, acch, inv);
}
// the first round of phase 1 when A = 1/(S + beta) has no zero entry (lu_as_first_nz): 24 KiB
// of accumulators, 6 blocks per CU
__global__ __launch_bounds__(NT) void k_lu_phase1_first_nz(TabDev A, TabDev S, uint32_t n, EqDev eq, Publish pub) {
    __shared__ uint4 accl[3 * NT], acch[3 * NT];
    lu_as_first_nz(A, S, n, eq, blockIdx.x, gridDim.x, pub, accl, acch);
}
// the first round of phase 2 when A and B have no zero entry: 32 KiB, 5 blocks per CU
template <bool M32>
__global__ __launch_bounds__(NT, 5) void k_lu_phase2_first_nz(TabDev A, TabDev S, TabDev B, TabDev T, TabDev m,
                                                           uint32_t n, EqDev eq, Publish pub, uint32_t ga,
                                                           uint32_t gb) {
    __shared__ uint4 accl[4 * NT], acch[4 * NT];
    if (blockIdx.x < ga) lu_as_first_nz(A, S, n, eq, blockIdx.x, ga, pub, accl, acch);
    else lu_btm_first_nz<M32>(B, T, m, n, eq, blockIdx.x - ga, gb, ga, pub, accl, acch);
}
uint32_t launch_lu_first_nz(hipStream_t s, Tab A, Tab S, Tab B, Tab T, Tab m, uint32_t n, int phase2, EqW eq,
                            Publish partial, const int32_t* m32) {
    const EqDev e{eq.elo, eq.ehi, eq.K};
    if (!phase2) {
        const uint32_t g = grid_for(n >> 1, NT, 1536);
        k_lu_phase1_first_nz<<<g, NT, 0, s>>>(tab_dev(A), tab_dev(S), n, e, partial);
        launch_publish(s, partial);
        return g;
    }
    const uint32_t ga = grid_for(n >> 1, NT, ZKH_NZ_GRID * 2 / 5), gb = grid_for(n >> 1, NT, ZKH_NZ_GRID * 3 / 5);
    TabDev md = tab_dev(m);
    md.s32 = m32;
    if (m32) k_lu_phase2_first_nz<true><<<ga + gb, NT, 0, s>>>(tab_dev(A), tab_dev(S), tab_dev(B), tab_dev(T), md, n, e, partial, ga, gb);
    else k_lu_phase2_first_nz<false><<<ga + gb, NT, 0, s>>>(tab_dev(A), tab_dev(S), tab_dev(B), tab_dev(T), md, n, e, partial, ga, gb);
    launch_publish(s, partial);
    return ga + gb;
}
uint32_t launch_lu_phase1(hipStream_t s, Tab A, Tab S, uint32_t n, int fold,
                          const uint32_t* v_m_host, const uint32_t* vmp, const uint32_t* beta_host, EqW eq,
                          Publish partial, int inv, int derive) {
    const uint32_t g = grid_for(n >> 1, NT, 1024);
    fr_t vm = fold && !vmp ? to_fr(v_m_host) : fr_t{};
    EqDev e{eq.elo, eq.ehi, eq.K};
    const fr_t beta = to_fr(beta_host);
    if (fold && derive) k_lu_phase1<1, 1><<<g, NT, 0, s>>>(tab_dev(A), tab_dev(S), n, vm, vmp, beta, e, partial, inv);
    else if (fold) k_lu_phase1<1, 0><<<g, NT, 0, s>>>(tab_dev(A), tab_dev(S), n, vm, vmp, beta, e, partial, inv);
    else k_lu_phase1<0, 0><<<g, NT, 0, s>>>(tab_dev(A), tab_dev(S), n, vm, vmp, beta, e, partial, inv);
    launch_publish(s, partial);
    return g;
}
// ------------------------------------------------------------------------------------
// Small folding rounds, one pair's products spread over the block's lanes
// ------------------------------------------------------------------------------------
// Below about 2^17 pairs a folding round is bound by the chain of dependent Montgomery
// products each thread runs for its pair (13 in the (B, T, m) group of logUp phase 2, 9 in
// the eq-form Hadamard), not by the device's product rate.  These kernels give each block
// a run of P pairs and split the round into levels of independent products that every lane
// of the block shares: (1) the folds of the tables' pair entries and the eq weight, (2) the
// weighted differences, (3) the products that are summed.  Each level's results go to LDS
// rows; one wave per sum adds its row.  The products, their operands and their order are
// those of k_lu_phase2<1, 1, 1> / k_hp_eq_round<1> / k_hp_round_ones<1> (derive form), so
// the sums, the folded tables and the Publish layout are the same; the critical path is
// three or two products instead of a pair's whole chain.
#define NTW 512  // threads of a wide round block (8 waves)
// rows of P field elements in LDS, limb-quad planes
template <uint32_t P>
struct Rows {
    uint4* lo;
    uint4* hi;
    ZDEV fr_t ld(uint32_t r, uint32_t p) const { return ld_fr(lo + r * P, hi + r * P, p); }
    ZDEV void st(uint32_t r, uint32_t p, const fr_t& x) const { st_fr(lo + r * P, hi + r * P, p, x); }
};
// The block's sums (wave w < nsum holds sum w of the block in lane 0, after fr_wave_sum)
// go to the partials of their jobs (see Publish).  Sum w belongs to job jw(w) as its entry
// kw(w) of K(jw) (K = {k0, k1}, k1 = 0 for one job); job j's block b partial is
// part[(j g + b) K_j + k], as reduce_publish_lds lays out two jobs of g blocks each.
ZDEV void wide_publish(const fr_t& bsum, uint32_t nsum, uint32_t k0, const Publish& P) {
    const uint32_t wv = threadIdx.x >> 6, lane = threadIdx.x & 63, g = gridDim.x, b = blockIdx.x;
    const uint32_t k1 = nsum - k0;
    if (wv < nsum && lane == 0)
        st_aos(P.part, wv < k0 ? b * k0 + wv : (g + b) * k1 + (wv - k0), bsum);
    if (b == 0 && threadIdx.x == 0) {
        publish_layout(P, 0, 0, g, k0);
        if (k1) publish_layout(P, 1, g, g, k1);
    }
}
// sum of row r over the block's np entries, by wave (lane-strided, then the wave's tree)
template <uint32_t P>
ZDEV fr_t wide_row_sum(const Rows<P>& R, uint32_t r, uint32_t np) {
    fr_t acc = fr_zero();
    for (uint32_t p = threadIdx.x & 63; p < np; p += 64) acc = fr_add(acc, R.ld(r, p));
    return fr_wave_sum(acc);
}
#ifndef LUW_P
#define LUW_P 64
#endif
// logUp phase 2, both groups folding, derived sums (lu_phase2_as / lu_phase2_btm derive):
// rows 0..9 the folded a0 a1 s0 s1 b0 b1 t0 t1 m0 m1, 10 W, 11..14 W a0, W da, W b0, W db,
// 15 m0 b0, 16 dm db, 17..20 W a0 (s0 + beta), W da ds, W b0 (t0 + beta), W db dt.
// Job 0 sums: rows 17, 18, 0; job 1: rows 19, 20, 15, 16.
__global__ __launch_bounds__(NTW) void k_lu_phase2_wide(TabDev A, TabDev S, TabDev B, TabDev T, TabDev m, uint32_t n,
                                                       fr_t vm, const uint32_t* vmp, fr_t beta, EqDev eq,
                                                       Publish pub) {
    if (!relayed_vm(vmp, vm)) return;
    constexpr uint32_t P = LUW_P;
    __shared__ uint4 rlo[21 * P], rhi[21 * P];
    const Rows<P> R{rlo, rhi};
    const uint32_t h = n >> 1, np = h < P ? h : P, base = blockIdx.x * P;
    for (uint32_t q = threadIdx.x; q < 11 * np; q += NTW) {  // level 1
        const uint32_t k = q / np, p = q - k * np, i = base + p;
        if (k == 10) {
            R.st(10, p, eq_w(eq, i));
            continue;
        }
        const uint32_t tt = k >> 1, e = i + (k & 1) * h;
        const TabDev t = tt == 0 ? A : tt == 1 ? S : tt == 2 ? B : tt == 3 ? T : m;
        const fr_t v = tab_fold_at(t, e, n, vm);
        st_fr(t.dlo, t.dhi, e, v);
        R.st(k, p, v);
    }
    __syncthreads();
    for (uint32_t q = threadIdx.x; q < 6 * np; q += NTW) {  // level 2
        const uint32_t k = q / np, p = q - k * np;
        fr_t x, y;
        if (k < 4) {
            x = R.ld(10, p);
            const uint32_t r0 = k < 2 ? 0 : 4;  // a or b
            y = (k & 1) ? fr_sub(R.ld(r0 + 1, p), R.ld(r0, p)) : R.ld(r0, p);
        } else if (k == 4) {
            x = R.ld(8, p);
            y = R.ld(4, p);
        } else {
            x = fr_sub(R.ld(9, p), R.ld(8, p));
            y = fr_sub(R.ld(5, p), R.ld(4, p));
        }
        R.st(11 + k, p, mont_mul_ol(x, y));
    }
    __syncthreads();
    for (uint32_t q = threadIdx.x; q < 4 * np; q += NTW) {  // level 3
        const uint32_t k = q / np, p = q - k * np;
        const uint32_t r0 = k < 2 ? 2 : 6;  // s or t
        const fr_t x = R.ld(11 + k, p);
        const fr_t y = (k & 1) ? fr_sub(R.ld(r0 + 1, p), R.ld(r0, p)) : fr_add(R.ld(r0, p), beta);
        R.st(17 + k, p, mont_mul_ol(x, y));
    }
    __syncthreads();
    const uint32_t wv = threadIdx.x >> 6;
    fr_t bs = fr_zero();
    if (wv < 7) {
        const uint32_t row = wv == 0 ? 17 : wv == 1 ? 18 : wv == 2 ? 0 : wv == 3 ? 19 : wv == 4 ? 20 : wv == 5 ? 15 : 16;
        bs = wide_row_sum<P>(R, row, np);
    }
    wide_publish(bs, 7, 3, pub);
}
#ifndef HPW_P
#define HPW_P 128
#endif
// eq-form Hadamard, folding, derived sums (k_hp_eq_round<1>): rows 0..3 the folded s0 s1 u0
// u1, 4 W, 5 W s0, 6 W ds, 7 W s0 u0, 8 W ds du; sums rows 7, 8
__global__ __launch_bounds__(NTW) void k_hp_eq_round_wide(TabDev S, TabDev U, uint32_t n, fr_t vm, const uint32_t* vmp,
                                                         EqDev eq, Publish pub) {
    if (!relayed_vm(vmp, vm)) return;
    constexpr uint32_t P = HPW_P;
    __shared__ uint4 rlo[9 * P], rhi[9 * P];
    const Rows<P> R{rlo, rhi};
    const uint32_t h = n >> 1, np = h < P ? h : P, base = blockIdx.x * P;
    for (uint32_t q = threadIdx.x; q < 5 * np; q += NTW) {
        const uint32_t k = q / np, p = q - k * np, i = base + p;
        if (k == 4) {
            R.st(4, p, eq_w(eq, i));
            continue;
        }
        const TabDev t = k < 2 ? S : U;
        const uint32_t e = i + (k & 1) * h;
        const fr_t v = tab_fold_at(t, e, n, vm);
        st_fr(t.dlo, t.dhi, e, v);
        R.st(k, p, v);
    }
    __syncthreads();
    for (uint32_t q = threadIdx.x; q < 2 * np; q += NTW) {
        const uint32_t k = q / np, p = q - k * np;
        const fr_t y = k ? fr_sub(R.ld(1, p), R.ld(0, p)) : R.ld(0, p);
        R.st(5 + k, p, mont_mul_ol(R.ld(4, p), y));
    }
    __syncthreads();
    for (uint32_t q = threadIdx.x; q < 2 * np; q += NTW) {
        const uint32_t k = q / np, p = q - k * np;
        const fr_t y = k ? fr_sub(R.ld(3, p), R.ld(2, p)) : R.ld(2, p);
        R.st(7 + k, p, mont_mul_ol(R.ld(5 + k, p), y));
    }
    __syncthreads();
    const uint32_t wv = threadIdx.x >> 6;
    fr_t bs = fr_zero();
    if (wv < 2) bs = wide_row_sum<P>(R, 7 + wv, np);
    wide_publish(bs, 2, 2, pub);
}
// Hadamard with U = 1, folding, derived sums (k_hp_round_ones<1>): rows 0..3 the folded e0
// e1 s0 s1, 4 e0 s0, 5 de ds; sums rows 4, 5
__global__ __launch_bounds__(NTW) void k_hp_ones_wide(TabDev E, TabDev S, uint32_t n, fr_t vm, const uint32_t* vmp,
                                                     Publish pub) {
    if (!relayed_vm(vmp, vm)) return;
    constexpr uint32_t P = HPW_P;
    __shared__ uint4 rlo[6 * P], rhi[6 * P];
    const Rows<P> R{rlo, rhi};
    const uint32_t h = n >> 1, np = h < P ? h : P, base = blockIdx.x * P;
    for (uint32_t q = threadIdx.x; q < 4 * np; q += NTW) {
        const uint32_t k = q / np, p = q - k * np, i = base + p;
        const TabDev t = k < 2 ? E : S;
        const uint32_t e = i + (k & 1) * h;
        const fr_t v = tab_fold_at(t, e, n, vm);
        st_fr(t.dlo, t.dhi, e, v);
        R.st(k, p, v);
    }
    __syncthreads();
    for (uint32_t q = threadIdx.x; q < 2 * np; q += NTW) {
        const uint32_t k = q / np, p = q - k * np;
        const fr_t x = k ? fr_sub(R.ld(1, p), R.ld(0, p)) : R.ld(0, p);
        const fr_t y = k ? fr_sub(R.ld(3, p), R.ld(2, p)) : R.ld(2, p);
        R.st(4 + k, p, mont_mul_ol(x, y));
    }
    __syncthreads();
    const uint32_t wv = threadIdx.x >> 6;
    fr_t bs = fr_zero();
    if (wv < 2) bs = wide_row_sum<P>(R, 4 + wv, np);
    wide_publish(bs, 2, 2, pub);
}
// the wide kernels take rounds of at most 2^ZKH_WIDE_LG pairs
#ifndef ZKH_WIDE_LG
#define ZKH_WIDE_LG 15
#endif
static bool wide_round(uint32_t n) { return (n >> 1) <= (1u << ZKH_WIDE_LG); }

// per-thread accumulator slots of a phase-2 launch: the larger group's
template <int fold_as, int fold_btm, int derive>
constexpr int lu2_slots() {
    return (derive && fold_btm) ? 4 : 6;
}
template <int fold_as, int fold_btm, int derive>
__global__ __launch_bounds__(NT) void k_lu_phase2(TabDev A, TabDev S, TabDev B, TabDev T, TabDev m, uint32_t n,
                                                  fr_t vm, const uint32_t* vmp, fr_t beta, EqDev eq, Publish pub,
                                                  uint32_t ga, uint32_t gb, int inv_as, int inv_btm) {
    if (!relayed_vm(vmp, vm)) return;
    constexpr int K = lu2_slots<fold_as, fold_btm, derive>();
    __shared__ uint4 accl[K * NT], acch[K * NT];
    if (blockIdx.x < ga) lu_phase2_as<fold_as, derive && fold_as>(A, S, n, vm, beta, eq, pub, blockIdx.x, ga, accl, acch, inv_as);
    else lu_phase2_btm<fold_btm, derive && fold_btm>(B, T, m, n, vm, beta, eq, pub, blockIdx.x - ga, gb, ga, accl, acch, inv_btm);
}
uint32_t launch_lu_phase2(hipStream_t s, Tab A, Tab S, Tab B, Tab T, Tab m, uint32_t n, int fold_as,
                          int fold_btm, const uint32_t* v_m_host, const uint32_t* vmp, const uint32_t* beta_host,
                          EqW eq, Publish partial, int inv_as, int inv_btm, int derive, const int32_t* m32) {
    // the derived variant holds 5 blocks per CU (32 KiB of accumulators): one resident wave
    const uint32_t G = derive && fold_as && fold_btm ? ZKH_LU2D_GRID : LU2_GRID;
    const uint32_t ga = grid_for(n >> 1, NT, G * 2 / 5), gb = grid_for(n >> 1, NT, G * 3 / 5);
    const fr_t vm = (fold_as || fold_btm) && !vmp ? to_fr(v_m_host) : fr_t{};
    EqDev e{eq.elo, eq.ehi, eq.K};
    const fr_t beta = to_fr(beta_host);
    const TabDev a = tab_dev(A), sd = tab_dev(S), b = tab_dev(B), t = tab_dev(T);
    TabDev md = tab_dev(m);
    md.s32 = m32;
    if (fold_as && fold_btm && derive && wide_round(n)) {
        const uint32_t gw = ((n >> 1) + LUW_P - 1) / LUW_P;
        k_lu_phase2_wide<<<gw, NTW, 0, s>>>(a, sd, b, t, md, n, vm, vmp, beta, e, partial);
        launch_publish(s, partial);
        return gw;
    }
    const uint32_t g = ga + gb;
#define LU2(FA, FB, DV) k_lu_phase2<FA, FB, DV><<<g, NT, 0, s>>>(a, sd, b, t, md, n, vm, vmp, beta, e, partial, ga, gb, inv_as, inv_btm)
    if (fold_as && fold_btm) {
        if (derive) LU2(1, 1, 1);
        else LU2(1, 1, 0);
    } else if (fold_as) {
        if (derive) LU2(1, 0, 1);
        else LU2(1, 0, 0);
    } else if (fold_btm) LU2(0, 1, 0);
    else LU2(0, 0, 0);
#undef LU2
    launch_publish(s, partial);
    return g;
}

// ------------------------------------------------------------------------------------
// Hadamard sumcheck rounds (zkob_lookup.cuh:212-233 k_hp3_step + k_fr_fold, fused)
// ------------------------------------------------------------------------------------
// derive (folding rounds): the sum at t = 1 is left out (the host takes it as claim - sum_0)
template <int derive>
__global__ __launch_bounds__(NT) void k_hp_round(TabDev E, TabDev S, TabDev U, uint32_t n, int fold,
                                                 fr_t vm, const uint32_t* vmp, Publish pub) {
    if (!relayed_vm(vmp, vm)) return;
    const uint32_t h = n >> 1;
    constexpr int K = derive ? 3 : 4;
    __shared__ uint4 accl[K * NT], acch[K * NT];
    LdsAcc<K> acc{accl, acch};
    acc.zero();
    for (uint32_t i = blockIdx.x * NT + threadIdx.x; i < h; i += gridDim.x * NT) {
        fr_t e0, e1, s0, s1;
        load_pair(E, i, h, n, fold, vm, e0, e1);
        SB();
        load_pair(S, i, h, n, fold, vm, s0, s1);
        SB();
        const fr_t de = fr_sub(e1, e0), ds = fr_sub(s1, s0);
        // es_t = E_t * S_t (x 2^-256) for t = 0..3 (t = 1 skipped under derive)
        fr_t es[4];
#pragma unroll
        for (int t = 0; t < 4; t++) {
            if (!derive || t != 1) es[t] = mont_mul_ol(e0, s0);
            SB();
            if (t < 3) {
                e0 = fr_add(e0, de);
                s0 = fr_add(s0, ds);
            }
        }
        fr_t u0, u1;
        load_pair(U, i, h, n, fold, vm, u0, u1);
        SB();
        const fr_t du = fr_sub(u1, u0);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            if (!derive || t != 1) acc.add(derive && t > 1 ? t - 1 : t, mont_mul_ol(es[t], u0));
            SB();
            if (t < 3) u0 = fr_add(u0, du);
        }
    }
    reduce_publish_lds<K>(acc, pub, 0, 0, gridDim.x, blockIdx.x);
}
uint32_t launch_hp_round(hipStream_t s, Tab E, Tab S, Tab U, uint32_t n, int fold,
                         const uint32_t* v_m_host, const uint32_t* vmp, Publish partial, int derive) {
    uint32_t g = grid_for(n >> 1, NT * 2, 1024);
    fr_t vm = fold && !vmp ? to_fr(v_m_host) : fr_t{};
    if (fold && derive) k_hp_round<1><<<g, NT, 0, s>>>(tab_dev(E), tab_dev(S), tab_dev(U), n, fold, vm, vmp, partial);
    else k_hp_round<0><<<g, NT, 0, s>>>(tab_dev(E), tab_dev(S), tab_dev(U), n, fold, vm, vmp, partial);
    launch_publish(s, partial);
    return g;
}
// U = 1 everywhere (the RoPE obligations' Hadamard): E_t S_t U_t = E_t S_t, a quadratic in t
// from three products per pair: sums e0 s0, e1 s1, (e1 - e0)(s1 - s0) (x 2^-256).  U is
// neither read nor folded (every fold of an all-ones table is all ones).
// derive (folding rounds): sum e1 s1 is left out (the host takes it as claim - sum e0 s0)
// s_int (first round only): S holds int32 values, and the three sums are formed exactly
// (x 1) with the 32-bit multiply (a pair outside that range takes two Montgomery products)
template <int derive>
__global__ __launch_bounds__(NT) void k_hp_round_ones(TabDev E, TabDev S, uint32_t n, int fold, fr_t vm,
                                                      const uint32_t* vmp, Publish pub, int s_int) {
    if (!relayed_vm(vmp, vm)) return;
    const uint32_t h = n >> 1;
    constexpr int K = derive ? 2 : 3;
    __shared__ uint4 accl[K * NT], acch[K * NT];
    LdsAcc<K> acc{accl, acch};
    acc.zero();
    const fr_t vp = fold && S.s32 ? plain_uniform(vm) : fr_zero();  // an int32 S's first fold
    for (uint32_t i = blockIdx.x * NT + threadIdx.x; i < h; i += gridDim.x * NT) {
        fr_t e0, e1, s0, s1;
        load_pair(E, i, h, n, fold, vm, e0, e1);
        SB();
        load_pair(S, i, h, n, fold, vm, vp, s0, s1);
        SB();
        if constexpr (!derive) {
            int64_t a0, a1;
            if (!fold && s_int && fr_int32ish(s0, a0) && fr_int32ish(s1, a1)) {
                acc.add(0, fr_mul_i64s(e0, a0));
                acc.add(1, fr_mul_i64s(e1, a1));
                acc.add(2, fr_mul_i64(fr_sub(e1, e0), a1 - a0));
                continue;
            }
            if (!fold && s_int) {
                acc.add(0, exact_mul(e0, s0));
                acc.add(1, exact_mul(e1, s1));
                acc.add(2, exact_mul(fr_sub(e1, e0), fr_sub(s1, s0)));
                continue;
            }
        }
        acc.add(0, mont_mul_ol(e0, s0));
        SB();
        if constexpr (!derive) {
            acc.add(1, mont_mul_ol(e1, s1));
            SB();
        }
        acc.add(K - 1, mont_mul_ol(fr_sub(e1, e0), fr_sub(s1, s0)));
        SB();
    }
    reduce_publish_lds<K>(acc, pub, 0, 0, gridDim.x, blockIdx.x);
}
uint32_t launch_hp_round_ones(hipStream_t s, Tab E, Tab S, uint32_t n, int fold, const uint32_t* v_m_host,
                              const uint32_t* vmp, Publish partial, int derive, int s_int, const int32_t* s32) {
    uint32_t g = grid_for(n >> 1, NT, 1024);
    fr_t vm = fold && !vmp ? to_fr(v_m_host) : fr_t{};
    TabDev sd = tab_dev(S);
    sd.s32 = s32;
    if (fold && derive && wide_round(n) && !s32) {
        const uint32_t gw = ((n >> 1) + HPW_P - 1) / HPW_P;
        k_hp_ones_wide<<<gw, NTW, 0, s>>>(tab_dev(E), sd, n, vm, vmp, partial);
        launch_publish(s, partial);
        return gw;
    }
    if (fold && derive) k_hp_round_ones<1><<<g, NT, 0, s>>>(tab_dev(E), sd, n, fold, vm, vmp, partial, 0);
    else k_hp_round_ones<0><<<g, NT, 0, s>>>(tab_dev(E), sd, n, fold, vm, vmp, partial, s_int);
    launch_publish(s, partial);
    return g;
}
// x as an integer in (-2^30, 2^30) when it is one (a field element or its negative)
ZDEV bool small_int(const fr_t& x, int32_t& out) {
    uint32_t hiw = 0;
#pragma unroll
    for (int i = 1; i < 8; i++) hiw |= x.v[i];
    if (!hiw && x.v[0] < (1u << 30)) {
        out = (int32_t)x.v[0];
        return true;
    }
    const fr_t d = fr_sub(fr_zero(), x);  // r - x
    hiw = 0;
#pragma unroll
    for (int i = 1; i < 8; i++) hiw |= d.v[i];
    if (!hiw && d.v[0] < (1u << 30)) {
        out = -(int32_t)d.v[0];
        return true;
    }
    return false;
}
// eq-specialised: with w = eq(i, u[0..K)) of the pair, S_t U_t = (s0 + t ds)(u0 + t du) is a
// quadratic in t, so three sums give the round: sum w s0 u0, sum w s1 u1, sum w ds du.  In a
// round that folds, w s0 and w ds are formed first and the sums carry 2^-256.  In the first
// round (no fold) the tables still hold the witness' small integers: the three products are
// formed exactly as 64-bit integers and the Montgomery-form weight multiplies them with the
// 64-bit multiply (sums x 2^256; a pair whose values are not all in (-2^30, 2^30) forms them
// as exact field products weighted to the same factor).
// derive (folding rounds): sum w s1 u1 is left out (the host takes it from the previous
// round's claim, q(0)(1 - u) + q(1) u)
// the folding form holds 5 waves per SIMD (16 KiB of accumulators, <= 96 VGPRs), the first
// round 4 (its 64-bit products take more registers)
// Sums of w p over a thread's pairs for weights w < 2^256 (canonical) and 63-bit p, as an
// 11-limb integer (up to 2^33 terms): two multiply-add rows of 8 limbs per term, no reduction
// until wide_mod, once per thread.  Reduction is linear, so the residue of the sum equals the
// sum of the per-term fr_mul_u64 residues.
ZDEV void wide_mac(uint32_t (&a)[11], const fr_t& w, uint64_t p) {
    // the two 288-bit rows w p0 and w p1 (as fr_mul_u32 forms them), then two 32-bit carry
    // chains into the accumulator: its limbs stay 32-bit values across the pair loop
    const uint32_t p0 = (uint32_t)p, p1 = (uint32_t)(p >> 32);
    uint32_t r[9];
    uint64_t c = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        c = (uint64_t)w.v[i] * p0 + (c >> 32);
        r[i] = (uint32_t)c;
    }
    r[8] = (uint32_t)(c >> 32);
    unsigned k = 0;
#pragma unroll
    for (int i = 0; i < 9; i++) a[i] = __builtin_addc(a[i], r[i], k, &k);
    a[9] = __builtin_addc(a[9], 0u, k, &k);
    a[10] += k;
    c = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        c = (uint64_t)w.v[i] * p1 + (c >> 32);
        r[i] = (uint32_t)c;
    }
    r[8] = (uint32_t)(c >> 32);
    k = 0;
#pragma unroll
    for (int i = 0; i < 9; i++) a[i + 1] = __builtin_addc(a[i + 1], r[i], k, &k);
    a[10] += k;
}
// a mod r: the low 256 bits by fr_reduce288 (below r 2^32), limbs 8..10 times 2^256, 2^288,
// 2^320 mod r by fr_mul_u32
ZDEV fr_t wide_mod(const uint32_t (&a)[11]) {
    const fr_t c256 = one_m();
    const fr_t c288 = {{0xcaaf6b13u, 0x355094eau, 0x69a568efu, 0xf6b10cb3u, 0x40cc3869u, 0xe2c926a6u, 0xed269aadu,
                        0x736a6d3bu}};
    const fr_t c320 = {{0x0121c884u, 0xc98da28eu, 0xc7363c67u, 0xe6f4f4a0u, 0xe92e7df1u, 0xb2d6ebc4u, 0x9d26242au,
                        0x19ae5794u}};
    uint32_t t[9];
#pragma unroll
    for (int i = 0; i < 8; i++) t[i] = a[i];
    t[8] = 0;
    fr_t x = fr_reduce288(t);
    x = fr_add(x, fr_mul_u32(c256, a[8]));
    x = fr_add(x, fr_mul_u32(c288, a[9]));
    return fr_add(x, fr_mul_u32(c320, a[10]));
}
template <int derive>
__global__ __attribute__((amdgpu_flat_work_group_size(1, NT), amdgpu_waves_per_eu(derive ? 5 : 4))) void k_hp_eq_round(TabDev S, TabDev U, uint32_t n, int fold, fr_t vm,
                                                    const uint32_t* vmp, EqDev eq, Publish pub) {
    if (!relayed_vm(vmp, vm)) return;
    const uint32_t h = n >> 1;
    constexpr int K = derive ? 2 : 3;
    __shared__ uint4 accl[K * NT], acch[K * NT];
    LdsAcc<K> acc{accl, acch};
    acc.zero();
    const bool ef = elo_factored(h, gridDim.x * NT);
    const fr_t vp = fold && (S.s32 || U.s32) ? plain_uniform(vm) : fr_zero();  // int32 tables' first fold
    for (uint32_t i = blockIdx.x * NT + threadIdx.x; i < h; i += gridDim.x * NT) {
        fr_t s0, s1, u0, u1, w;
        if (fold) {
            s0 = tab_fold_at(S, i, n, vm, vp);
            s1 = tab_fold_at(S, i + h, n, vm, vp);
            st_fr(S.dlo, S.dhi, i, s0);
            st_fr(S.dlo, S.dhi, i + h, s1);
            SB();
            u0 = tab_fold_at(U, i, n, vm, vp);
            w = pair_w(eq, i, ef);
            st_fr(U.dlo, U.dhi, i, u0);
            SB();
            u1 = tab_fold_at(U, i + h, n, vm, vp);
            st_fr(U.dlo, U.dhi, i + h, u1);
            SB();
            const fr_t ws = mont_mul_ol(w, s0);
            SB();
            const fr_t wds = mont_mul_ol(w, fr_sub(s1, s0));
            acc.add(0, mont_mul_ol(ws, u0));
            SB();
            if constexpr (!derive) {
                acc.add(1, mont_mul_ol(fr_add(ws, wds), u1));
                SB();
            }
            acc.add(K - 1, mont_mul_ol(wds, fr_sub(u1, u0)));
            SB();
            continue;
        }
        if constexpr (!derive) {
            int32_t a0, a1, b0, b1;
            if (S.s32 && U.s32) {  // int32 tables: the exact 64-bit products directly
                a0 = S.s32[i];
                a1 = S.s32[i + h];
                b0 = U.s32[i];
                b1 = U.s32[i + h];
                // small_int's range (-2^30, 2^30): differences and their product stay exact
                auto in30 = [](int32_t v) { return v > -(1 << 30) && v < (1 << 30); };
                if (in30(a0) && in30(a1) && in30(b0) && in30(b1)) {
                    w = pair_w(eq, i, ef);
                    acc.add(0, fr_mul_i64(w, (int64_t)a0 * b0));
                    acc.add(1, fr_mul_i64(w, (int64_t)a1 * b1));
                    acc.add(2, fr_mul_i64(w, (int64_t)(a1 - a0) * (b1 - b0)));
                    SB();
                    continue;
                }
            }
            s0 = tab_ld(S, i);
            s1 = tab_ld(S, i + h);
            u0 = tab_ld(U, i);
            u1 = tab_ld(U, i + h);
            w = pair_w(eq, i, ef);
            SB();
            if (small_int(s0, a0) && small_int(s1, a1) && small_int(u0, b0) && small_int(u1, b1)) {
                // the weight (e 2^256) times the exact 64-bit products: sums e s u 2^256
                acc.add(0, fr_mul_i64(w, (int64_t)a0 * b0));
                acc.add(1, fr_mul_i64(w, (int64_t)a1 * b1));
                acc.add(2, fr_mul_i64(w, (int64_t)(a1 - a0) * (b1 - b0)));
            } else {  // exact field products, weighted to the same e s u 2^256
                const fr_t w2 = mont_mul_ol(w, r2_m());
                acc.add(0, mont_mul_ol(w2, exact_mul(s0, u0)));
                SB();
                acc.add(1, mont_mul_ol(w2, exact_mul(s1, u1)));
                SB();
                acc.add(2, mont_mul_ol(w2, exact_mul(fr_sub(s1, s0), fr_sub(u1, u0))));
            }
            SB();
        }
    }
    if (ef) acc.elo_scale(eq, blockIdx.x * NT + threadIdx.x, K);
    reduce_publish_lds<K>(acc, pub, 0, 0, gridDim.x, blockIdx.x);
}
// The first round over int32 S and U (no fold): sum w (p_k + 2^62) for the exact products
// p_0 = s0 u0, p_1 = s1 u1, p_2 = (s1 - s0)(u1 - u0) (|p_k| < 2^62 when every entry lies in
// (-2^30, 2^30)) and sum w as wide integers, so that one reduction per thread gives
// sum w p_k: two rows of 8 multiply-adds per term instead of a field x int64 multiply and a
// field add.  A pair outside that range takes the field x int64 multiplies into the LDS
// accumulators.  Same sums as k_hp_eq_round<0>.
__global__ __launch_bounds__(NT, 4) void k_hp_eq_first_i32(TabDev S, TabDev U, uint32_t n, EqDev eq, Publish pub) {
    const uint32_t h = n >> 1;
    __shared__ uint4 accl[3 * NT], acch[3 * NT];
    LdsAcc<3> acc{accl, acch};
    acc.zero();
    const bool ef = elo_factored(h, gridDim.x * NT);
    uint32_t wp[3][11] = {}, wsum[9] = {};
    auto in30 = [](int32_t v) { return v > -(1 << 30) && v < (1 << 30); };
    for (uint32_t i = blockIdx.x * NT + threadIdx.x; i < h; i += gridDim.x * NT) {
        const int32_t a0 = S.s32[i], a1 = S.s32[i + h], b0 = U.s32[i], b1 = U.s32[i + h];
        const fr_t w = pair_w(eq, i, ef);
        if (in30(a0) && in30(a1) && in30(b0) && in30(b1)) {
            constexpr int64_t off = (int64_t)1 << 62;
            wide_mac(wp[0], w, (uint64_t)((int64_t)a0 * b0 + off));
            SB();
            wide_mac(wp[1], w, (uint64_t)((int64_t)a1 * b1 + off));
            SB();
            wide_mac(wp[2], w, (uint64_t)((int64_t)(a1 - a0) * (b1 - b0) + off));
            SB();
            unsigned k = 0;
#pragma unroll
            for (int t = 0; t < 8; t++) wsum[t] = __builtin_addc(wsum[t], w.v[t], k, &k);
            wsum[8] += k;
        } else {  // int32 products exact in int64; the differences' product by two multiplies
            acc.add(0, fr_mul_i64(w, (int64_t)a0 * b0));
            acc.add(1, fr_mul_i64(w, (int64_t)a1 * b1));
            acc.add(2, fr_mul_i64(fr_mul_i64(w, (int64_t)a1 - a0), (int64_t)b1 - b0));
        }
        SB();
    }
    // sum w p_k = sum w (p_k + 2^62) - 2^62 sum w
    uint32_t ws11[11] = {wsum[0], wsum[1], wsum[2], wsum[3], wsum[4], wsum[5], wsum[6], wsum[7], wsum[8], 0u, 0u};
    const fr_t off = fr_mul_u64(wide_mod(ws11), (uint64_t)1 << 62);
#pragma unroll
    for (int k = 0; k < 3; k++) acc.add(k, fr_sub(wide_mod(wp[k]), off));
    if (ef) acc.elo_scale(eq, blockIdx.x * NT + threadIdx.x, 3);
    reduce_publish_lds<3>(acc, pub, 0, 0, gridDim.x, blockIdx.x);
}
uint32_t launch_hp_eq_round(hipStream_t s, Tab S, Tab U, uint32_t n, int fold,
                            const uint32_t* v_m_host, const uint32_t* vmp, EqW eq, Publish partial, int derive,
                            const int32_t* s32, const int32_t* u32) {
    const uint32_t g = grid_for(n >> 1, NT, fold && derive ? ZKH_HPE_GRID : 1024);
    fr_t vm = fold && !vmp ? to_fr(v_m_host) : fr_t{};
    EqDev e{eq.elo, eq.ehi, eq.K};
    TabDev sd = tab_dev(S), ud = tab_dev(U);
    sd.s32 = s32;
    ud.s32 = u32;
    if (fold && derive && wide_round(n)) {
        const uint32_t gw = ((n >> 1) + HPW_P - 1) / HPW_P;
        k_hp_eq_round_wide<<<gw, NTW, 0, s>>>(sd, ud, n, vm, vmp, e, partial);
        launch_publish(s, partial);
        return gw;
    }
    if (fold && derive) k_hp_eq_round<1><<<g, NT, 0, s>>>(sd, ud, n, fold, vm, vmp, e, partial);
    else if (!fold && s32 && u32 && !vmp) k_hp_eq_first_i32<<<g, NT, 0, s>>>(sd, ud, n, e, partial);
    else k_hp_eq_round<0><<<g, NT, 0, s>>>(sd, ud, n, fold, vm, vmp, e, partial);
    launch_publish(s, partial);
    return g;
}
// sum_i eq(i, u[0..K)) S[i] (U[i]) over i < n, by chunks of 1024 indices sharing their
// Ehi factor: sum_c Ehi[c] * sum_{j < 1024} Elo[j] S[1024c + j] (U[...]), one product per
// entry for the Elo weight and one per chunk and thread for Ehi
__global__ __launch_bounds__(NT) void k_eq_sum(const uint4* slo, const uint4* shi, const uint4* ulo,
                                               const uint4* uhi, int has_u, uint32_t n, EqDev eq,
                                               Publish pub) {
    fr_t acc[1] = {fr_zero()};
    const uint32_t nchunk = (n + 1023) >> 10;
    for (uint32_t c = blockIdx.x; c < nchunk; c += gridDim.x) {
        fr_t part = fr_zero();
#pragma unroll
        for (uint32_t k = 0; k < 1024 / NT; k++) {
            const uint32_t j = k * NT + threadIdx.x, i = (c << 10) + j;
            if (i < n) {
                fr_t ws = mont_mul_ol(ld_aos(eq.elo, j), ld_fr(slo, shi, i));
                if (has_u) ws = mont_mul_ol(ws, ld_fr(ulo, uhi, i));
                part = fr_add(part, ws);
            }
        }
        acc[0] = fr_add(acc[0], mont_mul_ol(part, ld_aos(eq.ehi, c)));
    }
    reduce_publish<1>(acc, pub, 0, 0, gridDim.x, blockIdx.x);
}
// the same over integer entries: the Elo weight times the entry by the field x int64
// multiply (its sums carry 2^256 for the host to remove), no field planes read
template <typename T>
__global__ __launch_bounds__(NT) void k_eq_sum_int(const T* __restrict__ S, uint32_t n, EqDev eq, Publish pub) {
    fr_t acc[1] = {fr_zero()};
    const uint32_t nchunk = (n + 1023) >> 10;
    for (uint32_t c = blockIdx.x; c < nchunk; c += gridDim.x) {
        fr_t part = fr_zero();
#pragma unroll
        for (uint32_t k = 0; k < 1024 / NT; k++) {
            const uint32_t j = k * NT + threadIdx.x, i = (c << 10) + j;
            if (i < n) part = fr_add(part, fr_mul_i64(ld_aos(eq.elo, j), (int64_t)S[i]));
        }
        acc[0] = fr_add(acc[0], mont_mul_ol(part, ld_aos(eq.ehi, c)));
    }
    reduce_publish<1>(acc, pub, 0, 0, gridDim.x, blockIdx.x);
}
uint32_t launch_eq_sum_int(hipStream_t s, int kind, const void* S, uint32_t n, EqW eq, Publish partial) {
    const uint32_t g = grid_for((n + 1023) >> 10, 1, 1024);
    EqDev e{eq.elo, eq.ehi, eq.K};
    if (kind == 1) k_eq_sum_int<<<g, NT, 0, s>>>((const int32_t*)S, n, e, partial);
    else k_eq_sum_int<<<g, NT, 0, s>>>((const int64_t*)S, n, e, partial);
    launch_publish(s, partial);
    return g;
}
uint32_t launch_eq_sum(hipStream_t s, DevPlanes S, const DevPlanes* U, uint32_t n, EqW eq,
                       Publish partial) {
    const uint32_t g = grid_for((n + 1023) >> 10, 1, 1024);
    EqDev e{eq.elo, eq.ehi, eq.K};
    k_eq_sum<<<g, NT, 0, s>>>(PL_LO(S), PL_HI(S), U ? PL_LO(*U) : nullptr, U ? PL_HI(*U) : nullptr,
                              U ? 1 : 0, n, e, partial);
    launch_publish(s, partial);
    return g;
}


__global__ void k_static_setup(StaticFacArg fac, uint32_t words, uint32_t* fac_dst, uint32_t* cnt, uint32_t ncnt) {
    for (uint32_t i = threadIdx.x; i < words; i += blockDim.x) fac_dst[i] = fac.w[i];
    for (uint32_t i = threadIdx.x; i < ncnt; i += blockDim.x) cnt[i] = 0;
}
static_assert(NT == kFrMulPeakThreads, "k_fr_mul_peak runs NT threads per block");
__global__ __launch_bounds__(NT) void k_fr_mul_peak(uint32_t iters, uint32_t* out) {
    const uint32_t t = blockIdx.x * NT + threadIdx.x;
    fr_t x[4], y[4];
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
        for (int i = 0; i < 8; i++) {  // canonical: the top limb stays below r's
            x[c].v[i] = (i == 7 ? 0x0fffffffu : 0xffffffffu) & (t * 0x9e3779b9u + (uint32_t)(c * 8 + i) * 0x85ebca6bu);
            y[c].v[i] = (i == 7 ? 0x0fffffffu : 0xffffffffu) & ((uint32_t)(c * 8 + i + 1) * 0xc2b2ae35u);
        }
    for (uint32_t k = 0; k < iters; k++)
#pragma unroll
        for (int c = 0; c < 4; c++) x[c] = mont_mul(x[c], y[c]);
    uint32_t d = 0;
#pragma unroll
    for (int c = 0; c < 4; c++)
#pragma unroll
        for (int i = 0; i < 8; i++) d ^= x[c].v[i];
    out[t] = d;
}
void launch_fr_mul_peak(hipStream_t s, uint32_t blocks, uint32_t iters, uint32_t* out, hipEvent_t t0, hipEvent_t t1) {
    hipExtLaunchKernelGGL(k_fr_mul_peak, dim3(blocks), dim3(NT), 0, s, t0, t1, 0, iters, out);
}
void launch_static_setup(hipStream_t s, const StaticFacArg& fac, uint32_t words, uint32_t* fac_dst,
                         uint32_t* cnt, uint32_t ncnt) {
    k_static_setup<<<1, NT, 0, s>>>(fac, words, fac_dst, cnt, ncnt);
}

// ------------------------------------------------------------------------------------
// Batched (multi-job) kernels: one launch serves every independent sumcheck of a batch
// (e.g. the 7 matmuls of a layer).  Blocks are assigned to jobs contiguously; each job's
// descriptor holds its first block index.  Thread 0 locates the descriptor.
// ------------------------------------------------------------------------------------
template <typename D>
ZDEV void find_desc(const D* __restrict__ d, uint32_t nd, D& out) {
    __shared__ uint32_t sj;
    if (threadIdx.x == 0) {
        uint32_t j = 0;
        while (j + 1 < nd && d[j + 1].blk_begin <= blockIdx.x) j++;
        sj = j;
    }
    __syncthreads();
    out = d[sj];
}

// eq tables in Montgomery form: E[b] = Tlo[b mod 2^klo] * Thi[b >> klo], the two small
// factor-product tables built in LDS by separate threads (latency of ~8 products).
// prod_{i < k} fs[2 (i0 + i) + bit i of t] (Montgomery form), k <= 7, as a balanced tree of
// six products (three levels): the independent products of a level overlap, where a chain of
// k products waits on each in turn
ZDEV fr_t eq_lds_tree(const fr_t* fs, uint32_t i0, uint32_t k, uint32_t t) {
    fr_t p[7];
#pragma unroll
    for (uint32_t i = 0; i < 7; i++) p[i] = i < k ? fs[2 * (i0 + i) + ((t >> i) & 1)] : one_m();
    const fr_t a = mont_mul(p[0], p[1]), b = mont_mul(p[2], p[3]), c = mont_mul(p[4], p[5]);
    const fr_t ab = mont_mul(a, b), cd = mont_mul(c, p[6]);
    return mont_mul(ab, cd);
}
__global__ __launch_bounds__(NT) void k_eq_mont_multi(const EqTabDesc* __restrict__ d, uint32_t nd) {
    EqTabDesc q;
    find_desc(d, nd, q);
    __shared__ fr_t tlo[128], thi[128], fs[28];
    const uint32_t K = q.K;
    const uint32_t klo = K < 7 ? K : 7, khi = K - klo;
    const uint32_t t = threadIdx.x;
    if (khi <= 7) {
        // the 2K factors into LDS with one load per thread, so that the product chains
        // below wait on LDS instead of on a dependent global load per factor
        if (t < 2 * K) fs[t] = ld_aos(q.fac, t);
        __syncthreads();
        if (t < (1u << klo)) tlo[t] = eq_lds_tree(fs, 0, klo, t);
        else if (t >= 128 && t - 128 < (1u << khi)) thi[t - 128] = eq_lds_tree(fs, klo, khi, t - 128);
    }
    __syncthreads();
    const uint32_t b = (blockIdx.x - q.blk_begin) * NT + t;
    if (b >= q.n) return;
    fr_t e;
    if (khi <= 7) {
        e = khi ? mont_mul(tlo[b & ((1u << klo) - 1)], thi[b >> klo]) : tlo[b];
    } else {
        e = eq_prod(q.fac, K, b);
    }
    if (q.plain) e = mont_mul(e, plain_one());
    st_aos(q.out, b, e);
}
// out[b] = Tlo_m[b mod 2^klo] * Thi_p[b >> klo] (plain result), into planes
__global__ void k_eq_outer(const uint32_t* __restrict__ tlo, const uint32_t* __restrict__ thi,
                           uint32_t klo, uint32_t n, uint4* olo, uint4* ohi) {
    for (uint32_t b = blockIdx.x * blockDim.x + threadIdx.x; b < n; b += gridDim.x * blockDim.x)
        st_fr(olo, ohi, b, mont_mul(ld_aos(tlo, b & ((1u << klo) - 1)), ld_aos(thi, b >> klo)));
}
void launch_eq_outer(hipStream_t s, const uint32_t* tlo_m, const uint32_t* thi_p, uint32_t klo,
                     uint32_t n, DevPlanes out) {
    k_eq_outer<<<grid_for(n, NT, 8192), NT, 0, s>>>(tlo_m, thi_p, klo, n, PL_LO(out), PL_HI(out));
}
void launch_eq_mont_multi(hipStream_t s, const EqTabDesc* d_dev, uint32_t nd, uint32_t nblocks, hipEvent_t t0,
                          hipEvent_t t1) {
    hipExtLaunchKernelGGL(k_eq_mont_multi, dim3(nblocks), dim3(NT), 0, s, t0, t1, 0, d_dev, nd);
}

// ------------------------------------------------------------------------------------
// eq-weighted reductions of small-integer matrices.
// Lane i owns output column i and walks rows k of its chunk; the eq weight e_k is the same
// for every lane (uniform load).  Each integer (offset by 2^bits so it is non-negative) is
// cut into 20-bit pieces; piece x limb products (< 2^52) accumulate in 64-bit columns
// without carries for up to 2^11 rows, then one wide Montgomery reduction per piece folds
// the column sums into the field.  E is in Montgomery form, so the reduction leaves the
// plain sum.
// ------------------------------------------------------------------------------------
// uniform descriptor search: the last d[j] with d[j].blk_begin <= blockIdx.x (binary search
// over scalar loads, so every field of the result stays in scalar registers)
template <typename D>
ZDEV uint32_t find_desc_uniform(const D* __restrict__ d, uint32_t nd) {
    uint32_t lo = 0, hi = nd;  // d[lo].blk_begin <= blockIdx.x < d[hi].blk_begin
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (d[mid].blk_begin <= blockIdx.x) lo = mid;
        else hi = mid;
    }
    return lo;
}
typedef __attribute__((address_space(4))) const uint32_t* const_u32p;
// wave-uniform AoS load through the scalar cache (the table is read-only in the kernel)
ZDEV fr_t ld_aos_uniform(const uint32_t* p, uint32_t i) {
    const_u32p c = (const_u32p)(p + 8 * (size_t)i);
    fr_t r;
#pragma unroll
    for (int j = 0; j < 8; j++) r.v[j] = c[j];
    return r;
}
// streaming (read-once) global load
template <typename T>
ZDEV T ld_stream(const T* p) {
    return __builtin_nontemporal_load((__attribute__((address_space(1))) const T*)p);
}

// 2^(22p) * 2^256 mod r, p = 1..2: recombine 22-bit integer pieces
ZDEV fr_t piece_scale22(int p) {
    if (p == 1)
        return mk(0xff72abdbu, 0x008d5424u, 0xde9a0825u, 0x561f5078u, 0x85cae84du, 0xa153d589u,
                  0x4e5cfce5u, 0x1af19b95u);
    return mk(0xf6b12013u, 0x094ebc97u, 0x70afd742u, 0x6d9e32d3u, 0x5d095294u, 0xc234ec0bu,
              0xa886a754u, 0x6701f764u);
}
// Reduction variants: element type, pieces per element, piece width (bits).  A piece
// times a 32-bit eq limb is < 2^(32+PB), so a 64-bit column sum takes 2^(31-PB) rows
// without overflow (2048 rows at PB = 20, 512 at PB = 22); the host sizes chunks to that.
template <typename T_, int NP_, int PB_>
struct EqdotV {
    typedef T_ T;
    static constexpr int NP = NP_, PB = PB_;
};
typedef EqdotV<int32_t, 1, 20> EqdotI32x1;
typedef EqdotV<int32_t, 2, 22> EqdotI32x2;
typedef EqdotV<int64_t, 2, 22> EqdotI64x2;
typedef EqdotV<int64_t, 3, 22> EqdotI64x3;

// partial[c*N+i] = sum_{k in chunk c} (M[k*N+i] + 2^bits) e_k: one column per thread, rows
// in groups of EQDOT_GROUP with the next group's loads issued before the current group's
// products (2 * EQDOT_GROUP rows of the column in flight per wave); e_k comes through
// scalar loads.
#ifndef EQDOT_GROUP
#define EQDOT_GROUP 8
#endif
template <typename V>
ZDEV void eqdot_body(const EqDotDesc& q, uint32_t local) {
    typedef typename V::T T;
    constexpr int NP = V::NP, PB = V::PB;
    constexpr uint32_t PMASK = (1u << PB) - 1;
    const uint32_t N = q.N;
    const uint32_t ncb = (N + NT - 1) / NT;
    const uint32_t i = (local % ncb) * NT + threadIdx.x;
    const uint32_t c = local / ncb;
    const uint32_t k0 = c * q.kchunk;
    const uint32_t k1 = min(q.K, k0 + q.kchunk);
    const uint32_t* E = q.E;
    uint64_t acc[NP][8];
#pragma unroll
    for (int p = 0; p < NP; p++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[p][j] = 0;
    const uint64_t off = (uint64_t)1 << q.bits;
    const T* M = reinterpret_cast<const T*>(q.M);
    const uint32_t off32 = (uint32_t)off;
    auto mac = [&](T x, uint32_t k) {
        const fr_t e = ld_aos_uniform(E, k);
        if (sizeof(T) == 4 && NP == 1) {  // |x| < 2^19: x + 2^bits < 2^20 in one 32-bit add
            cols_mac(acc[0], (uint32_t)x + off32, e);
        } else {
            const uint64_t w = (uint64_t)(int64_t)x + off;
#pragma unroll
            for (int p = 0; p < NP; p++) cols_mac(acc[p], (uint32_t)(w >> (PB * p)) & PMASK, e);
        }
    };
    if (i < N) {
        const T* col = M + i;
        uint32_t k = k0;
        constexpr uint32_t G = EQDOT_GROUP;
        if (k + G <= k1) {
            T v[G];
#pragma unroll
            for (uint32_t u = 0; u < G; u++) v[u] = ld_stream(col + (size_t)(k + u) * N);
            for (; k + 2 * G <= k1; k += G) {
                T nx[G];
#pragma unroll
                for (uint32_t u = 0; u < G; u++) nx[u] = ld_stream(col + (size_t)(k + G + u) * N);
#pragma unroll
                for (uint32_t u = 0; u < G; u++) mac(v[u], k + u);
#pragma unroll
                for (uint32_t u = 0; u < G; u++) v[u] = nx[u];
            }
#pragma unroll
            for (uint32_t u = 0; u < G; u++) mac(v[u], k + u);
            k += G;
        }
        for (; k < k1; k++) mac(ld_stream(col + (size_t)k * N), k);
    }
    fr_t r = fr_zero();
#pragma unroll
    for (int p = 0; p < NP; p++) {
        uint32_t tt[10];
        cols_normalize(acc[p], tt);
        fr_t f = redc_wide<10>(tt);
        if (p > 0) f = mont_mul(f, PB == 20 ? piece_scale(p) : piece_scale22(p));
        r = fr_add(r, f);
    }
    if (i < N) st_aos(q.partial, (size_t)c * N + i, r);
}
// one launch for two variants: each descriptor's `variant` selects V0 or V1 (uniform per
// block), so the int32 (X, W) and int64 (Y) reductions of a batch share one grid
template <typename V0, typename V1>
__global__ __launch_bounds__(NT) void k_eqdot_multi(const EqDotDesc* __restrict__ d, uint32_t nd) {
    const EqDotDesc& q = d[find_desc_uniform(d, nd)];
    const uint32_t local = blockIdx.x - q.blk_begin;
    if (q.variant) eqdot_body<V1>(q, local);
    else eqdot_body<V0>(q, local);
}
void launch_eqdot_multi(hipStream_t s, int wide, const EqDotDesc* d_dev, uint32_t nd, uint32_t nblocks,
                        hipEvent_t t0, hipEvent_t t1) {
    if (!wide)
        hipExtLaunchKernelGGL(k_eqdot_multi<EqdotI32x1, EqdotI64x2>, dim3(nblocks), dim3(NT), 0, s, t0, t1, 0, d_dev, nd);
    else
        hipExtLaunchKernelGGL(k_eqdot_multi<EqdotI32x2, EqdotI64x3>, dim3(nblocks), dim3(NT), 0, s, t0, t1, 0, d_dev, nd);
}

// ------------------------------------------------------------------------------------
// eq-weighted reductions of full field-element tables.  A product x e of two 8-limb
// values is accumulated without reduction: its 64 limb products x_i e_j go into 15 column
// sums of 96 bits (one v_mad_u64_u32 whose carry-out feeds one v_addc_co_u32 per
// product), and a (column, chunk) cell is reduced once: two Montgomery reductions take the
// 527-bit column total T to T 2^-512 mod r, and one multiplication by 2^512 mod r leaves
// sum x (e 2^256) 2^-256 = sum x e for the Montgomery-form weights e.  Per element that is
// 128 VALU instructions against ~330 for a reduced Montgomery product and a field add.
// ------------------------------------------------------------------------------------
struct Cols15 {
    uint64_t lo[15];
    uint32_t top[15];
};
ZDEV void cols15_zero(Cols15& a) {
#pragma unroll
    for (int p = 0; p < 15; p++) {
        a.lo[p] = 0;
        a.top[p] = 0;
    }
}
// a += x e with the weight e in scalar registers (wave-uniform)
ZDEV void cols15_mac_s(Cols15& a, const fr_t& x, const fr_t& e) {
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 8; j += 2)
            mac2_ss(a.lo[i + j], a.top[i + j], x.v[i], e.v[j], a.lo[i + j + 1], a.top[i + j + 1], x.v[i], e.v[j + 1]);
}
// a += x e with a per-lane weight
ZDEV void cols15_mac_v(Cols15& a, const fr_t& x, const fr_t& e) {
#pragma unroll
    for (int i = 0; i < 8; i++)
#pragma unroll
        for (int j = 0; j < 8; j += 2)
            mac2_vv(a.lo[i + j], a.top[i + j], x.v[i], e.v[j], a.lo[i + j + 1], a.top[i + j + 1], x.v[i], e.v[j + 1]);
}
// sum_p (lo_p + top_p 2^64) 2^(32p) mod r, for a total below 2^544
ZDEV fr_t cols15_reduce(const Cols15& a) {
    uint32_t t[18];
    uint64_t c = 0;
#pragma unroll
    for (int k = 0; k < 18; k++) {
        uint64_t s = c;
        if (k < 15) s += (uint32_t)a.lo[k];
        if (k >= 1 && k <= 15) s += a.lo[k - 1] >> 32;
        if (k >= 2 && k <= 16) s += a.top[k - 2];
        t[k] = (uint32_t)s;
        c = s >> 32;
    }
    // first reduction: t[8..17] = (T + m r) / 2^256 < 2^288 + r
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t m = 0u - t[i];
        uint64_t cc = (uint64_t)m * ZKH_P0 + t[i];
#pragma unroll
        for (int j = 1; j < 8; j++) {
            cc = (uint64_t)m * fr_p(j) + t[i + j] + (cc >> 32);
            t[i + j] = (uint32_t)cc;
        }
#pragma unroll
        for (int j = i + 8; j < 18; j++) {
            cc = (uint64_t)t[j] + (cc >> 32);
            t[j] = (uint32_t)cc;
        }
    }
    // second reduction (its input is below r 2^256), then undo the remaining 2^-256
    return mont_mul(redc_wide<10>(t + 8), r2_m());
}
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
ZDEV fr_t ld_fr_stream(const uint4* lo, const uint4* hi, size_t i) {
    const u32x4 a = ld_stream(reinterpret_cast<const u32x4*>(lo) + i);
    const u32x4 b = ld_stream(reinterpret_cast<const u32x4*>(hi) + i);
    fr_t r;
    r.v[0] = a.x; r.v[1] = a.y; r.v[2] = a.z; r.v[3] = a.w;
    r.v[4] = b.x; r.v[5] = b.y; r.v[6] = b.z; r.v[7] = b.w;
    return r;
}
// column mode: lane = output column i, rows of chunk c in groups of 4 with the next group's
// loads issued before the current group's products
ZDEV void eqdot_fr_cols(const EqDotFrDesc& q, uint32_t local) {
    const uint32_t N = q.N;
    const uint32_t ncb = (N + NT - 1) / NT;
    const uint32_t i = (local % ncb) * NT + threadIdx.x;
    const uint32_t c = local / ncb;
    const uint32_t k0 = c * q.kchunk;
    const uint32_t k1 = min(q.K, k0 + q.kchunk);
    Cols15 a;
    cols15_zero(a);
    if (i < N) {
        const uint4* lo = reinterpret_cast<const uint4*>(q.lo) + i;
        const uint4* hi = reinterpret_cast<const uint4*>(q.hi) + i;
        constexpr uint32_t G = 4;
        uint32_t k = k0;
        if (k + G <= k1) {
            fr_t v[G];
#pragma unroll
            for (uint32_t u = 0; u < G; u++) v[u] = ld_fr_stream(lo, hi, (size_t)(k + u) * N);
            for (; k + 2 * G <= k1; k += G) {
                fr_t nx[G];
#pragma unroll
                for (uint32_t u = 0; u < G; u++) nx[u] = ld_fr_stream(lo, hi, (size_t)(k + G + u) * N);
#pragma unroll
                for (uint32_t u = 0; u < G; u++) cols15_mac_s(a, v[u], ld_aos_uniform(q.E, k + u));
#pragma unroll
                for (uint32_t u = 0; u < G; u++) v[u] = nx[u];
            }
#pragma unroll
            for (uint32_t u = 0; u < G; u++) cols15_mac_s(a, v[u], ld_aos_uniform(q.E, k + u));
            k += G;
        }
        for (; k < k1; k++) cols15_mac_s(a, ld_fr_stream(lo, hi, (size_t)k * N), ld_aos_uniform(q.E, k));
    }
    const fr_t r = cols15_reduce(a);
    if (i < N) st_aos(q.partial, (size_t)c * N + i, r);
}
// row mode: wave w of the block reduces row i = local * 4 + w over its K entries (lane l
// takes k = l, l + 64, ...), then a wave sum
ZDEV void eqdot_fr_rows(const EqDotFrDesc& q, uint32_t local) {
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t row = local * (NT / 64) + (threadIdx.x >> 6);
    Cols15 a;
    cols15_zero(a);
    if (row < q.N) {
        const size_t base = (size_t)row * q.K;
        const uint4* lo = reinterpret_cast<const uint4*>(q.lo) + base;
        const uint4* hi = reinterpret_cast<const uint4*>(q.hi) + base;
        uint32_t k = lane;
        for (; k + 64 < q.K; k += 128) {  // two entries in flight per lane
            const fr_t x0 = ld_fr_stream(lo, hi, k), x1 = ld_fr_stream(lo, hi, k + 64);
            const fr_t e0 = ld_aos(q.E, k), e1 = ld_aos(q.E, k + 64);
            cols15_mac_v(a, x0, e0);
            cols15_mac_v(a, x1, e1);
        }
        if (k < q.K) cols15_mac_v(a, ld_fr_stream(lo, hi, k), ld_aos(q.E, k));
    }
    const fr_t r = fr_wave_sum(cols15_reduce(a));
    if (row < q.N && lane == 0) st_aos(q.partial, row, r);
}
__global__ __launch_bounds__(NT) void k_eqdot_fr_multi(const EqDotFrDesc* __restrict__ d, uint32_t nd) {
    const EqDotFrDesc& q = d[find_desc_uniform(d, nd)];
    const uint32_t local = blockIdx.x - q.blk_begin;
    if (q.rowmode) eqdot_fr_rows(q, local);
    else eqdot_fr_cols(q, local);
}
void launch_eqdot_fr_multi(hipStream_t s, const EqDotFrDesc* d_dev, uint32_t nd, uint32_t nblocks, hipEvent_t t0,
                           hipEvent_t t1) {
    hipExtLaunchKernelGGL(k_eqdot_fr_multi, dim3(nblocks), dim3(NT), 0, s, t0, t1, 0, d_dev, nd);
}

// out[i] = sum_c partial[c*N+i] - corr (i < N; zero up to Npad), or, when E is set, the
// block partial of sum_i E_m[i] * (sum_c partial[c*N+i] - corr) into dot[slot].  A block
// covers 64 columns; wave w adds the chunks c = w (mod 4) with four loads in flight, and
// the four wave sums meet in LDS.
__global__ __launch_bounds__(NT) void k_sum_chunks_multi(const SumChunksDesc* __restrict__ d, uint32_t nd) {
    const SumChunksDesc& q = d[find_desc_uniform(d, nd)];
    const uint32_t local = blockIdx.x - q.blk_begin;
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const uint32_t i = local * 64 + lane;
    __shared__ fr_t part[NT / 64][64];
    fr_t s = fr_zero();
    if (i < q.N) {
        uint32_t c = w;
        for (; c + 12 < q.nch; c += 16) {
            fr_t v[4];
#pragma unroll
            for (int u = 0; u < 4; u++) v[u] = ld_aos(q.partial, (size_t)(c + 4 * u) * q.N + i);
#pragma unroll
            for (int u = 0; u < 4; u++) s = fr_add(s, v[u]);
        }
        for (; c < q.nch; c += 4) s = fr_add(s, ld_aos(q.partial, (size_t)c * q.N + i));
    }
    part[w][lane] = s;
    __syncthreads();
    if (w) return;
#pragma unroll
    for (int u = 1; u < NT / 64; u++) s = fr_add(s, part[u][lane]);
    s = i < q.N ? fr_sub(s, to_fr(q.corr.v)) : fr_zero();
    if (q.E) {
        fr_t t = i < q.N ? mont_mul(ld_aos(q.E, i), s) : fr_zero();
        t = fr_wave_sum(t);
        if (lane == 0) st_aos(q.dot, local, t);
    } else if (i < q.Npad) {
        st_fr(reinterpret_cast<uint4*>(q.out_lo), reinterpret_cast<uint4*>(q.out_hi), i, s);
    }
}
void launch_sum_chunks_multi(hipStream_t s, const SumChunksDesc* d_dev, uint32_t nd, uint32_t nblocks,
                             hipEvent_t t0, hipEvent_t t1) {
    hipExtLaunchKernelGGL(k_sum_chunks_multi, dim3(nblocks), dim3(NT), 0, s, t0, t1, 0, d_dev, nd);
}

// zkip rounds of several jobs in one launch: one pair per thread; fold of the previous
// round fused in (in place); per job: sum a0b0, a1b1, da*db (x 2^-256) published.
__global__ __launch_bounds__(NT) void k_zkip_round_multi(ZkipBatch bt, Publish pub) {
    __shared__ uint32_t sj;
    if (threadIdx.x == 0) {
        uint32_t j = 0;
        while (j + 1 < bt.nd && bt.d[j + 1].blk_begin <= blockIdx.x) j++;
        sj = j;
    }
    __syncthreads();
    const uint32_t job = sj;
    const ZkipDesc& q = bt.d[job];
    const uint32_t local = blockIdx.x - q.blk_begin;
    const uint32_t h = q.n >> 1;
    const uint32_t nblk = (h + NT - 1) / NT;
    const uint32_t i = local * NT + threadIdx.x;
    fr_t acc[3] = {fr_zero(), fr_zero(), fr_zero()};
    if (i < h) {
        const TabDev a{reinterpret_cast<const uint4*>(q.a_lo), reinterpret_cast<const uint4*>(q.a_hi),
                       reinterpret_cast<uint4*>(q.a_lo), reinterpret_cast<uint4*>(q.a_hi)};
        const TabDev b{reinterpret_cast<const uint4*>(q.b_lo), reinterpret_cast<const uint4*>(q.b_hi),
                       reinterpret_cast<uint4*>(q.b_lo), reinterpret_cast<uint4*>(q.b_hi)};
        fr_t a0, a1, b0, b1;
        const fr_t vm = to_fr(q.vm.v);
        load_pair(a, i, h, q.n, q.fold, vm, a0, a1);
        load_pair(b, i, h, q.n, q.fold, vm, b0, b1);
        acc[0] = mont_mul(a0, b0);
        acc[1] = mont_mul(a1, b1);
        acc[2] = mont_mul(fr_sub(a1, a0), fr_sub(b1, b0));
    }
    reduce_publish<3>(acc, pub, job, q.blk_begin, nblk, local);
}
void launch_zkip_round_multi(hipStream_t s, const ZkipBatch& b, uint32_t nblocks, Publish pub) {
    k_zkip_round_multi<<<nblocks, NT, 0, s>>>(b, pub);
    launch_publish(s, pub);
}
// final binds of several 2-entry tables (t[0] += v*(t[1]-t[0]) when fold is set) and the
// terminal values a[0], b[0] written to partial[0..1] (AoS)
__global__ void k_fold_last_multi(ZkipBatch bt) {
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= 2 * bt.nd) return;
    const ZkipDesc& q = bt.d[j >> 1];
    uint4* lo = reinterpret_cast<uint4*>((j & 1) ? q.b_lo : q.a_lo);
    uint4* hi = reinterpret_cast<uint4*>((j & 1) ? q.b_hi : q.a_hi);
    const fr_t x = q.fold ? fold_at(lo, hi, 0, 1, to_fr(q.vm.v)) : ld_fr(lo, hi, 0);
    st_fr(lo, hi, 0, x);
    st_aos(q.partial, j & 1, x);
}
void launch_fold_last_multi(hipStream_t s, const ZkipBatch& b) {
    k_fold_last_multi<<<1, 64, 0, s>>>(b);
}


// ------------------------------------------------------------------------------------
// witness GEMM (zkfc.cu:44-58, fr-tensor.cu:831-878 for integer operands): Y = X W exactly
// ------------------------------------------------------------------------------------
typedef double zkh_d4 __attribute__((ext_vector_type(4)));
typedef int32_t zkh_i4 __attribute__((ext_vector_type(4)));
// four consecutive int32 of a row from column k (zero past the row's end or for a row
// outside the matrix)
ZDEV zkh_i4 ld_row4(const int32_t* row, uint32_t k, uint32_t len, bool ok, bool vec) {
    if (ok && vec && k + 3 < len) return *reinterpret_cast<const zkh_i4*>(row + k);
    zkh_i4 v = {0, 0, 0, 0};
    if (ok)
        for (int i = 0; i < 4; i++)
            if (k + i < len) v[i] = row[k + i];
    return v;
}
// fp64 matrix cores (v_mfma_f64_16x16x4f64: lane l holds A[l%16][l/16], B[l/16][l%16]; result
// register r of lane l is D[l/16 + 4r][l%16]).  A wave computes a 32 x 32 tile of Y as 2 x 2
// fragments; a block of 4 waves a 64 x 64 tile.  Per 16 values of k a lane loads four
// consecutive k of one X row and of one WT row per fragment and feeds them to four
// products; A and B use the same order of k, so each product sums a permutation of k.
// Integers below 2^53 are exact doubles and every partial sum stays below 2^53 (checked by
// the caller from the operands' magnitude bounds), so the result is exact.
__global__ __launch_bounds__(256) void k_matmul_f64(const int32_t* __restrict__ X, const int32_t* __restrict__ WT,
                                                    const int64_t* __restrict__ bias, uint32_t B, uint32_t IN,
                                                    uint32_t OUT, int64_t* __restrict__ Y) {
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t row0 = blockIdx.y * 64 + (wv >> 1) * 32, col0 = blockIdx.x * 64 + (wv & 1) * 32;
    const uint32_t li = lane & 15, lk = lane >> 4;
    const bool vec = (IN & 3) == 0;
    zkh_d4 acc[2][2];
#pragma unroll
    for (int f = 0; f < 2; f++)
#pragma unroll
        for (int g = 0; g < 2; g++) acc[f][g] = zkh_d4{0.0, 0.0, 0.0, 0.0};
    const uint32_t r0 = row0 + li, r1 = row0 + 16 + li, c0 = col0 + li, c1 = col0 + 16 + li;
    const int32_t* xr0 = X + (size_t)(r0 < B ? r0 : 0) * IN;
    const int32_t* xr1 = X + (size_t)(r1 < B ? r1 : 0) * IN;
    const int32_t* wr0 = WT + (size_t)(c0 < OUT ? c0 : 0) * IN;
    const int32_t* wr1 = WT + (size_t)(c1 < OUT ? c1 : 0) * IN;
    // the next 16 values of k load while this step's products issue
    zkh_i4 nx0 = ld_row4(xr0, 4 * lk, IN, r0 < B, vec), nx1 = ld_row4(xr1, 4 * lk, IN, r1 < B, vec);
    zkh_i4 nw0 = ld_row4(wr0, 4 * lk, IN, c0 < OUT, vec), nw1 = ld_row4(wr1, 4 * lk, IN, c1 < OUT, vec);
    for (uint32_t k0 = 0; k0 < IN; k0 += 16) {
        const zkh_i4 xa0 = nx0, xa1 = nx1, wb0 = nw0, wb1 = nw1;
        if (k0 + 16 < IN) {
            const uint32_t k = k0 + 16 + 4 * lk;
            nx0 = ld_row4(xr0, k, IN, r0 < B, vec);
            nx1 = ld_row4(xr1, k, IN, r1 < B, vec);
            nw0 = ld_row4(wr0, k, IN, c0 < OUT, vec);
            nw1 = ld_row4(wr1, k, IN, c1 < OUT, vec);
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const double a0 = (double)xa0[t], a1 = (double)xa1[t], b0 = (double)wb0[t], b1 = (double)wb1[t];
            acc[0][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a1, b1, acc[1][1], 0, 0, 0);
        }
    }
#pragma unroll
    for (int f = 0; f < 2; f++)
#pragma unroll
        for (int g = 0; g < 2; g++) {
            const uint32_t col = col0 + 16 * g + li;
            if (col >= OUT) continue;
            const int64_t bv = bias ? bias[col] : 0;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const uint32_t row = row0 + 16 * f + lk + 4 * r;
                if (row < B) Y[(size_t)row * OUT + col] = (int64_t)acc[f][g][r] + bv;
            }
        }
}
// int64 VALU (operands whose partial sums may exceed 2^53): 16 x 16 output tile per block,
// 16-wide k tiles of X and WT through LDS
__global__ __launch_bounds__(256) void k_matmul_i64(const int32_t* __restrict__ X, const int32_t* __restrict__ WT,
                                                    const int64_t* __restrict__ bias, uint32_t B, uint32_t IN,
                                                    uint32_t OUT, int64_t* __restrict__ Y) {
    __shared__ int32_t xs[16][17], ws[16][17];
    const uint32_t tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    const uint32_t row = blockIdx.y * 16 + ty, col = blockIdx.x * 16 + tx;
    const uint32_t wrow = blockIdx.x * 16 + ty;  // WT row loaded by this thread
    int64_t acc = 0;
    for (uint32_t k0 = 0; k0 < IN; k0 += 16) {
        xs[ty][tx] = (row < B && k0 + tx < IN) ? X[(size_t)row * IN + k0 + tx] : 0;
        ws[ty][tx] = (wrow < OUT && k0 + tx < IN) ? WT[(size_t)wrow * IN + k0 + tx] : 0;
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 16; k++) acc += (int64_t)xs[ty][k] * (int64_t)ws[tx][k];
        __syncthreads();
    }
    if (row < B && col < OUT) Y[(size_t)row * OUT + col] = acc + (bias ? bias[col] : 0);
}
void launch_matmul_i32(hipStream_t s, const int32_t* X, const int32_t* WT, const int64_t* bias, uint32_t B,
                       uint32_t IN, uint32_t OUT, int64_t* Y, int f64) {
    if (f64)
        k_matmul_f64<<<dim3((OUT + 63) / 64, (B + 63) / 64), 256, 0, s>>>(X, WT, bias, B, IN, OUT, Y);
    else
        k_matmul_i64<<<dim3((OUT + 15) / 16, (B + 15) / 16), 256, 0, s>>>(X, WT, bias, B, IN, OUT, Y);
}
__global__ void k_widen_i32(const int32_t* __restrict__ in, uint32_t n, int64_t* __restrict__ out) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) out[i] = in[i];
}
__global__ void k_to_long(const uint4* __restrict__ lo, const uint4* __restrict__ hi, uint32_t n,
                          int64_t* __restrict__ out) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        out[i] = fr_to_long(ld_fr(lo, hi, i));
}
void launch_to_long(hipStream_t s, DevPlanes p, uint32_t n, int64_t* out) {
    k_to_long<<<grid_for(n, NT, 1024), NT, 0, s>>>((const uint4*)p.lo(), (const uint4*)p.hi(), n, out);
}
void launch_widen_i32(hipStream_t s, const int32_t* in, uint32_t n, int64_t* out) {
    k_widen_i32<<<grid_for(n, NT, 1024), NT, 0, s>>>(in, n, out);
}

// ------------------------------------------------------------------------------------
// persistent matmul round loop (see ZkipPersist): tables in LDS, one host round trip per
// round, no device-side reduction or barrier across blocks
// ------------------------------------------------------------------------------------
// Host <-> device words travel as 16-byte quads [seq, w0, w1, w2], each written and read
// with one 16-byte access (system coherent); a reader takes the data words of a message
// only when every quad of it shows the expected seq, so no fence orders data and flag and
// the challenge arrives with the poll itself.
typedef uint32_t zkh_v4u __attribute__((ext_vector_type(4)));
ZDEV uint4 ld_quad_sys(const uint32_t* p) {
    zkh_v4u r;
    asm volatile("global_load_dwordx4 %0, %1, off sc0 sc1\n\ts_waitcnt vmcnt(0)" : "=v"(r) : "v"((uint64_t)p) : "memory");
    return make_uint4(r.x, r.y, r.z, r.w);
}
ZDEV void st_quad_sys(uint32_t* p, uint4 v) {
    const zkh_v4u x = {v.x, v.y, v.z, v.w};
    asm volatile("global_store_dwordx4 %0, %1, off sc0 sc1" : : "v"((uint64_t)p), "v"(x) : "memory");
}
// wave 0: wait until the first nq (<= 11) command quads show want; lane i < nq then holds
// command words 3i .. 3i+2 in (y, z, w).  False on ZKH_QUIT or when the deadline passes
// (then *err is set).  Every lane of wave 0 calls it and gets the same result.
ZDEV bool persist_wait(const uint32_t* cmd, uint32_t nq, uint32_t want, uint32_t* err, uint64_t deadline,
                       uint4& quad) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t t0 = wall_clock64();
    for (;;) {
        const uint4 qd = lane < nq ? ld_quad_sys(cmd + 4 * lane) : make_uint4(want, 0, 0, 0);
        if (__ballot(qd.x == ZKH_QUIT)) return false;
        if (!__ballot(qd.x != want)) {
            quad = qd;
            return true;
        }
        if (wall_clock64() - t0 > deadline) {
            if (lane == 0) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}
// wave 0: words[0 .. nw) of pub (LDS) as quads with seq into slot (lanes < ceil(nw/3))
ZDEV void persist_publish(uint32_t* slot, const uint32_t* pub, uint32_t nw, uint32_t seq) {
    for (uint32_t qd = threadIdx.x & 63; qd * 3 < nw; qd += 64) {
        const uint32_t b = 3 * qd;
        st_quad_sys(slot + 4 * qd, make_uint4(seq, pub[b], b + 1 < nw ? pub[b + 1] : 0u, b + 2 < nw ? pub[b + 2] : 0u));
    }
}
// completion flag of a stream (the host's settle): the value of *word (when given) to
// host_word, then seq to the host flag
__global__ void k_fence(uint32_t* flag, uint32_t seq, const uint32_t* word, uint32_t nwords, uint32_t* host_word) {
    for (uint32_t i = 0; word && i < nwords; i++)
        __hip_atomic_store(host_word + i, word[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(flag, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}
void launch_fence(hipStream_t s, uint32_t* flag, uint32_t seq, const uint32_t* word, uint32_t nwords,
                  uint32_t* host_word) {
    k_fence<<<1, 1, 0, s>>>(flag, seq, word, nwords, host_word);
}
// the relay between two round launches (launch_relay)
__global__ __launch_bounds__(64) void k_relay(const uint32_t* cmd, uint32_t want, uint32_t* err,
                                              unsigned long long deadline, uint32_t* vmp) {
    uint4 qd;
    const bool ok = persist_wait(cmd, 3, want, err, deadline, qd);
    __shared__ uint32_t w[9];
    const uint32_t lane = threadIdx.x;
    if (lane < 3) {
        w[3 * lane] = qd.y;
        w[3 * lane + 1] = qd.z;
        w[3 * lane + 2] = qd.w;
    }
    __builtin_amdgcn_wave_barrier();
    if (lane < 8) vmp[lane] = ok ? w[lane] : 0u;
    if (lane == 8) vmp[8] = ok ? 0u : 1u;
}
void launch_relay(hipStream_t s, const uint32_t* cmd, uint32_t want, uint32_t* err, unsigned long long deadline,
                  uint32_t* vmp) {
    k_relay<<<1, 64, 0, s>>>(cmd, want, err, deadline, vmp);
}
#define NTP 1024  // threads of a persistent round block (16 waves)
static_assert(2 * ZKH_PLS_MAX <= NTP, "the double fold takes one product per thread");

// block clock -> slot words ZKH_PSTAMP + 0..3 (publication time, receipt of the previous
// command), and the low words of both per message s < 14 into words ZKH_PSTAMP + 4 + 2s
// (publication of message s) and ZKH_PSTAMP + 5 + 2(s - 1) (receipt of command s - 1); the
// host reads the per-message words after the kernel has ended
ZDEV void persist_stamp(uint32_t* slot, uint32_t s, uint64_t t_cmd, uint32_t stamp = ZKH_PSTAMP) {
    const uint64_t now = wall_clock64();
    uint32_t* st = slot + stamp;
    st[0] = (uint32_t)now;
    st[1] = (uint32_t)(now >> 32);
    st[2] = (uint32_t)t_cmd;
    st[3] = (uint32_t)(t_cmd >> 32);
    if (s < 14) st[4 + 2 * s] = (uint32_t)now;
    if (s >= 1 && s <= 14) st[5 + 2 * (s - 1)] = (uint32_t)t_cmd;
}
// operand sel of a table at position p of the halves (L = T[p], H = T[p + h], D = H - L)
ZDEV fr_t half_opnd(const uint4* lo, const uint4* hi, uint32_t sel, uint32_t p, uint32_t h) {
    if (sel == 0) return ld_fr(lo, hi, p);
    if (sel == 1) return ld_fr(lo, hi, p + h);
    return fr_sub(ld_fr(lo, hi, p + h), ld_fr(lo, hi, p));
}
// Two-round products by operand class, so that the lanes of a wave run the same code:
// class X (types 0, 3, 1, 4): T[p]; class D (types 2, 5, 6, 7): T[p + d] - T[p]; class E
// (type 8): (T[j'+h] - T[j']) - (T[j+h] - T[j]).  kPairType lists the types in wave order.
__constant__ uint32_t kPairType[9] = {0, 3, 1, 4, 2, 5, 6, 7, 8};
// offsets of type t's operand at quarter index j (j' = j + q4): p and, for class D, d
ZDEV void pair_pos(uint32_t t, uint32_t j, uint32_t q4, uint32_t h, uint32_t& p, uint32_t& d) {
    const uint32_t jq = j + q4;
    switch (t) {
        case 0: p = j; d = 0; break;
        case 1: p = j + h; d = 0; break;
        case 3: p = jq; d = 0; break;
        case 4: p = jq + h; d = 0; break;
        case 2: p = j; d = h; break;
        case 5: p = jq; d = h; break;
        case 6: p = j; d = q4; break;
        default: p = j + h; d = q4; break;  // 7
    }
}
ZDEV fr_t pair_opnd_e(const uint4* lo, const uint4* hi, uint32_t j, uint32_t q4, uint32_t h) {
    return fr_sub(fr_sub(ld_fr(lo, hi, j + q4 + h), ld_fr(lo, hi, j + q4)),
                  fr_sub(ld_fr(lo, hi, j + h), ld_fr(lo, hi, j)));
}
// Round loop of one block over its LDS slice (see ZkipPersist).  A two-round message: a
// group of min(m/4, 64) lanes accumulates product type t over j < m/4; the double fold
// computes the four products of an output entry on a quad of lanes and adds them with two
// lane swaps.  A one-round message (m = 2): lanes 0..2 of wave 0 form a0b0, a1b1,
// (a1-a0)(b1-b0).
__global__ __launch_bounds__(NTP) void k_zkip_persist(ZkipPersist P) {
    extern __shared__ uint4 zl[];  // a.lo | a.hi | b.lo | b.hi, ls entries each
    __shared__ uint32_t sj, sok, pubw[ZKH_MSG_PAIR], sxw[33];
    __shared__ fr_t red[9];
    if (threadIdx.x == 0) {
        uint32_t j = 0;
        while (j + 1 < P.nd && P.d[j + 1].blk_begin <= blockIdx.x) j++;
        sj = j;
    }
    __syncthreads();
    const ZkipPJob& q = P.d[sj];
    const uint32_t lb = blockIdx.x - q.blk_begin;
    const uint32_t ls = q.n >> q.lgnb;
    uint4* alo = zl;
    uint4* ahi = zl + ls;
    uint4* blo = zl + 2 * ls;
    uint4* bhi = zl + 3 * ls;
    {
        const uint4* ga_lo = reinterpret_cast<const uint4*>(q.a_lo);
        const uint4* ga_hi = reinterpret_cast<const uint4*>(q.a_hi);
        const uint4* gb_lo = reinterpret_cast<const uint4*>(q.b_lo);
        const uint4* gb_hi = reinterpret_cast<const uint4*>(q.b_hi);
        for (uint32_t k = threadIdx.x; k < ls; k += NTP) {
            const uint32_t g = lb + (k << q.lgnb);
            alo[k] = ga_lo[g];
            ahi[k] = ga_hi[g];
            blo[k] = gb_lo[g];
            bhi[k] = gb_hi[g];
        }
    }
    __syncthreads();
    uint32_t* slot = q.out + (size_t)lb * ZKH_PSLOT;
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    uint32_t m = ls;
    uint64_t t_cmd = 0;
    for (uint32_t seq = 1;; seq++) {
        uint32_t nw;
        if (m >= 4) {
            const uint32_t q4 = m >> 2, h = m >> 1;
            // S = min(q4, 64) lanes per type and k = min(4, 64 / S) types per wave, the
            // waves of a class (X: 4 types, D: 4, E: 1) next to each other: 8/k + 1 waves
            // (3 for q4 <= 16), each running one class's code, so a wave's SIMD does one
            // multiply per lane per 64 / (k S) products (a wave's Montgomery products
            // nearly fill its SIMD: fewer waves per SIMD finish sooner)
            const uint32_t S = q4 < 64 ? q4 : 64;
            const uint32_t k = S <= 16 ? 4 : 64 / S;
            const uint32_t nwx = 4 / k;  // waves per class X and D
            if (wv < 2 * nwx + 1) {
                const uint32_t cls = wv < nwx ? 0 : wv < 2 * nwx ? 1 : 2;
                const uint32_t slot = lane / S, sub = lane % S;
                const bool live = cls < 2 ? slot < k : slot == 0;
                const uint32_t t = cls == 2 ? 8 : kPairType[(wv - cls * nwx) * k + (live ? slot : 0) + 4 * cls];
                fr_t acc = fr_zero();
                if (live) {
                    for (uint32_t j = sub; j < q4; j += S) {
                        fr_t x, y;
                        if (cls == 2) {
                            x = pair_opnd_e(alo, ahi, j, q4, h);
                            y = pair_opnd_e(blo, bhi, j, q4, h);
                        } else {
                            uint32_t pp, d;
                            pair_pos(t, j, q4, h, pp, d);
                            x = ld_fr(alo, ahi, pp + d);
                            y = ld_fr(blo, bhi, pp + d);
                            if (cls == 1) {
                                x = fr_sub(x, ld_fr(alo, ahi, pp));
                                y = fr_sub(y, ld_fr(blo, bhi, pp));
                            }
                        }
                        acc = fr_add(acc, mont_mul_ol(x, y));
                    }
                }
                for (uint32_t z = S >> 1; z >= 1; z >>= 1) acc = fr_add(acc, fr_shfl_xor(acc, z));
                if (live && sub == 0) red[t] = acc;
            }
            __syncthreads();
            nw = ZKH_MSG_PAIR;
            if (wv == 0 && lane < 9) {
#pragma unroll
                for (int i = 0; i < 8; i++) pubw[8 * lane + i] = red[lane].v[i];
            }
        } else if (m == 2) {
            nw = ZKH_MSG_ONE;
            if (wv == 0 && lane < 3) {
                const fr_t x = half_opnd(alo, ahi, lane, 0, 1), y = half_opnd(blo, bhi, lane, 0, 1);
                const fr_t t = mont_mul_ol(x, y);
#pragma unroll
                for (int i = 0; i < 8; i++) pubw[8 * lane + i] = t.v[i];
            }
        } else {  // the block's folded entries a[0], b[0]
            nw = ZKH_MSG_FINAL;
            if (wv == 0 && lane < 2) {
                const fr_t t = lane ? ld_fr(blo, bhi, 0) : ld_fr(alo, ahi, 0);
#pragma unroll
                for (int i = 0; i < 8; i++) pubw[8 * lane + i] = t.v[i];
            }
        }
        if (wv == 0) {
            __builtin_amdgcn_wave_barrier();
            if (lane == 0) persist_stamp(slot, seq, t_cmd);
            persist_publish(slot, pubw, nw, seq);
        }
        if (m == 1) return;
        if (wv == 0) {
            uint4 qd;
            const uint32_t nq = zkh_quad_count(m >= 4 ? 32 : 8);
            const bool ok = persist_wait(q.cmd, nq, seq, P.err, P.deadline, qd);
            if (lane < nq) {
                sxw[3 * lane] = qd.y;
                sxw[3 * lane + 1] = qd.z;
                sxw[3 * lane + 2] = qd.w;
            }
            if (lane == 0) sok = ok;
            t_cmd = wall_clock64();
        }
        __syncthreads();
        if (!sok) return;
        if (m >= 4) {  // double fold: m -> m/4; the four products of an output on four lanes
            const uint32_t q4 = m >> 2, h = m >> 1;
            const uint32_t t = threadIdx.x;  // 8*q4 <= 8*ZKH_PLS_MAX/4 = NTP products, one per thread
            if (t < 8 * q4) {                // whole lane quads (8*q4 is a multiple of 8)
                const uint32_t o = t >> 2, term = t & 3;  // output o (a for o < q4, b after), term
                const bool tb = o >= q4;
                const uint32_t k = tb ? o - q4 : o;
                uint4* lo = tb ? blo : alo;
                uint4* hi = tb ? bhi : ahi;
                fr_t w;
#pragma unroll
                for (int i = 0; i < 8; i++) w.v[i] = sxw[8 * term + i];
                fr_t r = mont_mul_ol(w, ld_fr(lo, hi, k + (term & 1 ? h : 0) + (term & 2 ? q4 : 0)));
                r = fr_add(r, fr_shfl_xor(r, 1));
                r = fr_add(r, fr_shfl_xor(r, 2));
                if (term == 0) st_fr(lo, hi, k, r);  // T[k] is read only by this quad
            }
            m = q4;
        } else {  // m == 2: T[0] <- T[0] + x (T[1] - T[0])
            fr_t x;
#pragma unroll
            for (int i = 0; i < 8; i++) x.v[i] = sxw[i];
            if (threadIdx.x < 2) {
                uint4* lo = threadIdx.x ? blo : alo;
                uint4* hi = threadIdx.x ? bhi : ahi;
                const fr_t v0 = ld_fr(lo, hi, 0), v1 = ld_fr(lo, hi, 1);
                st_fr(lo, hi, 0, fr_add(v0, mont_mul(x, fr_sub(v1, v0))));
            }
            m = 1;
        }
        __syncthreads();
    }
}
// Value at point pt = 3 a + b of {0, 1, inf}^2 of the bilinear function of a cell whose
// corners are X[c + (2 y1 + y2) q] (inf: the difference along that axis)
ZDEV fr_t pt_val(const uint4* lo, const uint4* hi, uint32_t c, uint32_t q, uint32_t pt) {
    const uint32_t a = pt / 3, b = pt - 3 * a;
    auto along2 = [&](uint32_t y1) {
        const uint32_t o = c + 2 * y1 * q;
        if (b == 0) return ld_fr(lo, hi, o);
        if (b == 1) return ld_fr(lo, hi, o + q);
        return fr_sub(ld_fr(lo, hi, o + q), ld_fr(lo, hi, o));
    };
    if (a < 2) return along2(a);
    return fr_sub(along2(1), along2(0));
}
// Persistent Hadamard rounds (see HpPersist).  Eq mode: the eq weight of a local pair k is
// the same in every round (g = block + nb*k; only the host's correction changes), so
// W[k] = eq_w(g) is formed once while the tables load.  Per round, with h = m/2 pairs, two
// levels of one Montgomery product per thread, each spread over as many waves as it has
// products:
//   eq mode   level 1: WS[k] = W[k] s0[k], WD[k] = W[k] (s1[k] - s0[k]);
//             level 2: P[t][k] = (WS[k] + t WD[k]) (u0[k] + t du[k]), t < 4;
//   E mode    level 1: Q[t][k] = E_t[k] S_t[k];  level 2: P[t][k] = Q[t][k] U_t[k];
// then wave t < 4 adds row t.  After the challenge one thread per entry folds the tables.
// LDS: the tables (ls entries each, lo plane then hi plane) and 8 rows of ls/2 entries
// (eq mode: W, WS, WD, -, P[0..3]; E mode: Q[0..3], P[0..3]).
__global__ __launch_bounds__(NTP) void k_hp_persist(HpPersist P) {
    extern __shared__ uint4 zl[];
    __shared__ uint32_t sok, pubw[ZKH_HP_MSG2], sxw[33];
    const uint32_t lb = blockIdx.x;
    const uint32_t ls = P.n >> P.lgnb, hs = ls >> 1;
    const bool em = P.e_lo != nullptr;
    const uint32_t ntab = em ? 3 : 2;  // S, U (, E)
    uint4* tlo[3];
    uint4* thi[3];
    for (uint32_t i = 0; i < 3; i++) {
        tlo[i] = zl + 2 * i * ls;
        thi[i] = tlo[i] + ls;
    }
    uint4* rlo = zl + 2 * ntab * ls;  // 8 rows of hs: lo planes, then hi planes
    uint4* rhi = rlo + 8 * hs;
    const EqDev eq{P.elo, P.ehi, 0};
    if (P.vmp && P.vmp[8]) return;  // the host abandoned the proof before the relay
    {
        const uint4* glo_[3] = {reinterpret_cast<const uint4*>(P.s_lo), reinterpret_cast<const uint4*>(P.u_lo),
                                reinterpret_cast<const uint4*>(P.e_lo)};
        const uint4* ghi_[3] = {reinterpret_cast<const uint4*>(P.s_hi), reinterpret_cast<const uint4*>(P.u_hi),
                                reinterpret_cast<const uint4*>(P.e_hi)};
        const fr_t vm = P.vmp ? ld_aos(P.vmp, 0) : to_fr(P.vm.v);
        const uint32_t nload = ntab * ls + (em ? 0 : hs);
        for (uint32_t t = threadIdx.x; t < nload; t += NTP) {  // tables, then (eq mode) W
            if (t < ntab * ls) {
                const uint32_t i = t / ls, k = t - i * ls;
                const uint32_t g = lb + (k << P.lgnb);
                const fr_t v = P.fold ? fold_at(glo_[i], ghi_[i], g, P.n, vm) : ld_fr(glo_[i], ghi_[i], g);
                st_fr(tlo[i], thi[i], k, v);
            } else {
                const uint32_t k = t - ntab * ls;
                st_fr(rlo, rhi, k, eq_w(eq, lb + (k << P.lgnb)));
            }
        }
    }
    __syncthreads();
    uint32_t* slot = P.out + (size_t)lb * ZKH_PSLOT;
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    uint32_t m = ls;
    uint64_t t_cmd = 0;
    for (uint32_t seq = 1;; seq++) {
        uint32_t nw;
        const bool dbl = P.two && m >= 4;
        if (dbl) {  // two rounds: the nine point sums over the cells c < q
            const uint32_t q = m >> 2;
            uint4* xlo = rlo + (em ? 0 : hs);  // 9 rows of q after the W row (eq mode)
            uint4* xhi = rhi + (em ? 0 : hs);
            for (uint32_t t = threadIdx.x; t < 9 * q; t += NTP) {  // W S(y) or E(y) S(y)
                const uint32_t pt = t / q, cc = t - pt * q;
                const fr_t x = em ? pt_val(tlo[2], thi[2], cc, q, pt) : ld_fr(rlo, rhi, cc);
                st_fr(xlo, xhi, t, mont_mul_ol(x, pt_val(tlo[0], thi[0], cc, q, pt)));
            }
            __syncthreads();
            if (wv < 9) {  // wave pt: sum over the cells of W S(y) U(y), or of E(y) S(y)
                fr_t acc = fr_zero();
                for (uint32_t cc = lane; cc < q; cc += 64) {
                    const fr_t x = ld_fr(xlo, xhi, wv * q + cc);
                    acc = fr_add(acc, em ? x : mont_mul_ol(x, pt_val(tlo[1], thi[1], cc, q, wv)));
                }
                acc = fr_wave_sum(acc);
                if (lane == 0)
#pragma unroll
                    for (int i = 0; i < 8; i++) pubw[8 * wv + i] = acc.v[i];
            }
            nw = ZKH_HP_MSG2;
        } else if (m >= 2) {
            const uint32_t h = m >> 1;
            if (!em) {
                for (uint32_t t = threadIdx.x; t < 2 * h; t += NTP) {  // level 1
                    const bool d = t >= h;
                    const uint32_t k = d ? t - h : t;
                    const fr_t s0 = ld_fr(tlo[0], thi[0], k);
                    const fr_t x = d ? fr_sub(ld_fr(tlo[0], thi[0], k + h), s0) : s0;
                    st_fr(rlo + (1 + d) * hs, rhi + (1 + d) * hs, k, mont_mul_ol(ld_fr(rlo, rhi, k), x));
                }
            } else {
                for (uint32_t q = threadIdx.x; q < 4 * h; q += NTP) {  // level 1: q = t * h + k
                    const uint32_t t = q / h, k = q - t * h;
                    fr_t e = ld_fr(tlo[2], thi[2], k), sv = ld_fr(tlo[0], thi[0], k);
                    const fr_t de = fr_sub(ld_fr(tlo[2], thi[2], k + h), e), ds = fr_sub(ld_fr(tlo[0], thi[0], k + h), sv);
                    for (uint32_t i = 0; i < t; i++) {
                        e = fr_add(e, de);
                        sv = fr_add(sv, ds);
                    }
                    st_fr(rlo + t * hs, rhi + t * hs, k, mont_mul_ol(e, sv));
                }
            }
            __syncthreads();
            for (uint32_t q = threadIdx.x; q < 4 * h; q += NTP) {  // level 2: q = t * h + k
                const uint32_t t = q / h, k = q - t * h;
                const fr_t u0 = ld_fr(tlo[1], thi[1], k), du = fr_sub(ld_fr(tlo[1], thi[1], k + h), u0);
                fr_t a, c = u0;
                if (!em) {
                    a = ld_fr(rlo + hs, rhi + hs, k);
                    const fr_t wd = ld_fr(rlo + 2 * hs, rhi + 2 * hs, k);
                    for (uint32_t i = 0; i < t; i++) a = fr_add(a, wd);
                } else {
                    a = ld_fr(rlo + t * hs, rhi + t * hs, k);
                }
                for (uint32_t i = 0; i < t; i++) c = fr_add(c, du);
                st_fr(rlo + (4 + t) * hs, rhi + (4 + t) * hs, k, mont_mul_ol(a, c));
            }
            __syncthreads();
            if (wv < 4) {  // wave t adds row 4 + t
                fr_t acc = fr_zero();
                for (uint32_t k = lane; k < h; k += 64)
                    acc = fr_add(acc, ld_fr(rlo + (4 + wv) * hs, rhi + (4 + wv) * hs, k));
                acc = fr_wave_sum(acc);
                if (lane == 0)
#pragma unroll
                    for (int i = 0; i < 8; i++) pubw[8 * wv + i] = acc.v[i];
            }
            nw = ZKH_HP_MSG;
        } else {  // the block's folded entries S[0], U[0] (, E[0])
            nw = 8 * ntab;
            if (wv == 0 && lane < ntab) {
                const fr_t t = ld_fr(tlo[lane], thi[lane], 0);
#pragma unroll
                for (int i = 0; i < 8; i++) pubw[8 * lane + i] = t.v[i];
            }
        }
        __syncthreads();
        if (wv == 0) {
            if (lane == 0) persist_stamp(slot, seq, t_cmd);
            persist_publish(slot, pubw, nw, seq);
        }
        if (m == 1) return;
        if (wv == 0) {
            uint4 qd;
            const uint32_t nq = dbl ? zkh_quad_count(32) : 3;
            const bool ok = persist_wait(P.cmd, nq, seq, P.err, P.deadline, qd);
            if (lane < nq) {
                sxw[3 * lane] = qd.y;
                sxw[3 * lane + 1] = qd.z;
                sxw[3 * lane + 2] = qd.w;
            }
            if (lane == 0) sok = ok;
            t_cmd = wall_clock64();
        }
        __syncthreads();
        if (!sok) return;
        if (dbl) {  // double fold m -> m/4: the four products of an output on four lanes
            const uint32_t q = m >> 2;
            for (uint32_t t = threadIdx.x; t < ntab * q * 4; t += NTP) {  // whole lane quads
                const uint32_t o = t >> 2, term = t & 3, i = o / q, cc = o - i * q;
                fr_t w;
#pragma unroll
                for (int j = 0; j < 8; j++) w.v[j] = sxw[8 * term + j];
                fr_t r = mont_mul_ol(w, ld_fr(tlo[i], thi[i], cc + term * q));
                r = fr_add(r, fr_shfl_xor(r, 1));
                r = fr_add(r, fr_shfl_xor(r, 2));
                if (term == 0) st_fr(tlo[i], thi[i], cc, r);  // T[cc] is read only by this quad
            }
            m >>= 2;
            __syncthreads();
            continue;
        }
        {  // fold the tables: T[k] <- T[k] + x (T[k + m/2] - T[k])
            fr_t x;
#pragma unroll
            for (int i = 0; i < 8; i++) x.v[i] = sxw[i];
            const uint32_t h = m >> 1;
            for (uint32_t t = threadIdx.x; t < ntab * h; t += NTP) {
                const uint32_t i = t / h, k = t - i * h;
                const fr_t v0 = ld_fr(tlo[i], thi[i], k), v1 = ld_fr(tlo[i], thi[i], k + h);
                st_fr(tlo[i], thi[i], k, fr_add(v0, mont_mul_ol(x, fr_sub(v1, v0))));
            }
        }
        m >>= 1;
        __syncthreads();
    }
}
hipError_t launch_hp_persist(hipStream_t s, const HpPersist& p) {
    const uint32_t ls = p.n >> p.lgnb;  // LDS: 2 or 3 tables of ls + 8 rows of ls/2 entries, 32 B each
    const size_t lds = (size_t)ls * 32 * (p.e_lo ? 3 : 2) + (size_t)(ls >> 1) * 8 * 32;
    k_hp_persist<<<1u << p.lgnb, NTP, lds, s>>>(p);
    return hipGetLastError();
}
// Persistent logUp phase-2 rounds (see LuPersist).  W[k] = eq_w(g) is formed once while the
// tables load.  Per round, with h = m/2 pairs: level 1, one product per thread, rows
// WA0 = W a0, WDA = W (a1 - a0), WB0 = W b0, WDB = W (b1 - b0); level 2, wave j < 11
// accumulates sum type kLuType[j] over the pairs (one product per pair, none for sum a0 /
// sum a1) and adds its lanes.  The type order puts 3, 2, 2, 2 product waves on the four
// SIMDs.  After the challenge one thread per entry folds the five tables.
// LDS: 5 tables (ls entries each, lo plane then hi plane) and 5 rows of ls/2 (W, WA0, WDA,
// WB0, WDB).
__constant__ uint32_t kLuType[11] = {0, 1, 2, 5, 6, 3, 4, 7, 8, 9, 10};
__global__ __launch_bounds__(NTP) void k_lu_persist(LuPersist P) {
    extern __shared__ uint4 zl[];
    __shared__ uint32_t sok, pubw[ZKH_LU_MSG2], sxw[33];
    const uint32_t lb = blockIdx.x;
    const uint32_t ls = P.n >> P.lgnb, hs = ls >> 1;
    uint4* tlo[5];
    uint4* thi[5];
    for (uint32_t i = 0; i < 5; i++) {
        tlo[i] = zl + 2 * i * ls;
        thi[i] = tlo[i] + ls;
    }
    uint4* rlo = zl + 10 * ls;  // 5 rows of hs: lo planes, then hi planes
    uint4* rhi = rlo + 5 * hs;
    const EqDev eq{P.elo, P.ehi, 0};
    const fr_t beta = to_fr(P.beta.v);
    if (P.vmp && P.vmp[8]) return;  // the host abandoned the proof before the relay
    {
        const fr_t vm = P.vmp ? ld_aos(P.vmp, 0) : to_fr(P.vm.v);
        for (uint32_t t = threadIdx.x; t < 5 * ls + hs; t += NTP) {  // tables, then W
            if (t < 5 * ls) {
                const uint32_t i = t / ls, k = t - i * ls;
                const uint32_t g = lb + (k << P.lgnb);
                const uint4* glo = reinterpret_cast<const uint4*>(P.lo[i]);
                const uint4* ghi = reinterpret_cast<const uint4*>(P.hi[i]);
                const bool f = i < 2 ? P.fold_as : P.fold_btm;
                st_fr(tlo[i], thi[i], k, f ? fold_at(glo, ghi, g, P.n, vm) : ld_fr(glo, ghi, g));
            } else {
                const uint32_t k = t - 5 * ls;
                st_fr(rlo, rhi, k, eq_w(eq, lb + (k << P.lgnb)));
            }
        }
    }
    __syncthreads();
    uint32_t* slot = P.out + (size_t)lb * ZKH_LU_PSLOT;
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    uint32_t m = ls;
    uint64_t t_cmd = 0;
    for (uint32_t seq = 1;; seq++) {
        uint32_t nw;
        const bool dbl = P.two && m >= 4;
        if (dbl) {  // two rounds: the point sums over the cells c < q
            const uint32_t q = m >> 2;
            uint4* wlo = rlo + hs;  // W A, then W B, at the corners (2 rows of m after the W row)
            uint4* whi = rhi + hs;
            for (uint32_t t = threadIdx.x; t < 2 * m; t += NTP) {
                const uint32_t g2 = t >= m, r = t - g2 * m;  // A or B; table entry r = cc + j q
                st_fr(wlo, whi, t, mont_mul_ol(ld_fr(rlo, rhi, r & (q - 1)), ld_fr(tlo[2 * g2], thi[2 * g2], r)));
            }
            __syncthreads();
            // wave wv: sum types wv, wv + 16: 0..8 W A(y) (S(y) + beta'), 9..17 W B(y) (T(y) +
            // beta'), 18..26 m(y) B(y), 27..30 A at corner j
            for (uint32_t ty = wv; ty < 31; ty += NTP / 64) {
                fr_t acc = fr_zero();
                const uint32_t grp = ty / 9, pt = ty - 9 * grp;
                for (uint32_t cc = lane; cc < q; cc += 64) {
                    if (ty >= 27) {
                        acc = fr_add(acc, ld_fr(tlo[0], thi[0], cc + (ty - 27) * q));
                        continue;
                    }
                    fr_t x, y;
                    if (grp < 2) {
                        x = pt_val(wlo + grp * m, whi + grp * m, cc, q, pt);
                        y = pt_val(tlo[1 + 2 * grp], thi[1 + 2 * grp], cc, q, pt);
                        if (pt / 3 < 2 && pt % 3 < 2) y = fr_add(y, beta);
                    } else {
                        x = pt_val(tlo[4], thi[4], cc, q, pt);
                        y = pt_val(tlo[2], thi[2], cc, q, pt);
                    }
                    acc = fr_add(acc, mont_mul_ol(x, y));
                }
                acc = fr_wave_sum(acc);
                if (lane == 0)
#pragma unroll
                    for (int i = 0; i < 8; i++) pubw[8 * ty + i] = acc.v[i];
            }
            nw = ZKH_LU_MSG2;
        } else if (m >= 2) {
            const uint32_t h = m >> 1;
            for (uint32_t q = threadIdx.x; q < 4 * h; q += NTP) {  // level 1: row 1 + j, j = q / h
                const uint32_t j = q / h, k = q - j * h;
                const uint32_t ti = j < 2 ? 0 : 2;  // A or B
                const fr_t x0 = ld_fr(tlo[ti], thi[ti], k);
                const fr_t x = (j & 1) ? fr_sub(ld_fr(tlo[ti], thi[ti], k + h), x0) : x0;
                st_fr(rlo + (1 + j) * hs, rhi + (1 + j) * hs, k, mont_mul_ol(ld_fr(rlo, rhi, k), x));
            }
            __syncthreads();
            if (wv < 11) {  // level 2: wave wv, sum type ty
                const uint32_t ty = kLuType[wv];
                fr_t acc = fr_zero();
                for (uint32_t k = lane; k < h; k += 64) {
                    if (ty == 3 || ty == 4) {  // sum a0 / sum a1
                        acc = fr_add(acc, ld_fr(tlo[0], thi[0], ty == 3 ? k : k + h));
                        continue;
                    }
                    fr_t x, y;
                    if (ty < 8) {  // (A, S) or (B, T) with the level-1 rows
                        const uint32_t g0 = ty < 3 ? 0 : 1;   // group
                        const uint32_t r0 = 1 + 2 * g0;       // WA0 / WB0 row
                        const uint32_t tt = g0 ? 3 : 1;       // S or T
                        const uint32_t sel = ty < 3 ? ty : ty - 5;
                        const fr_t w0 = ld_fr(rlo + r0 * hs, rhi + r0 * hs, k);
                        const fr_t wd = ld_fr(rlo + (r0 + 1) * hs, rhi + (r0 + 1) * hs, k);
                        const fr_t v0 = ld_fr(tlo[tt], thi[tt], k), v1 = ld_fr(tlo[tt], thi[tt], k + h);
                        x = sel == 0 ? w0 : sel == 1 ? fr_add(w0, wd) : wd;
                        y = sel == 0 ? fr_add(v0, beta) : sel == 1 ? fr_add(v1, beta) : fr_sub(v1, v0);
                    } else {  // m . b
                        const fr_t m0 = ld_fr(tlo[4], thi[4], k), b0 = ld_fr(tlo[2], thi[2], k);
                        if (ty == 8) {
                            x = m0;
                            y = b0;
                        } else {
                            const fr_t m1 = ld_fr(tlo[4], thi[4], k + h), b1 = ld_fr(tlo[2], thi[2], k + h);
                            x = ty == 9 ? m1 : fr_sub(m1, m0);
                            y = ty == 9 ? b1 : fr_sub(b1, b0);
                        }
                    }
                    acc = fr_add(acc, mont_mul_ol(x, y));
                }
                acc = fr_wave_sum(acc);
                if (lane == 0)
#pragma unroll
                    for (int i = 0; i < 8; i++) pubw[8 * ty + i] = acc.v[i];
            }
            nw = ZKH_LU_MSG;
        } else {  // the block's folded entries A[0], S[0], B[0], T[0], m[0]
            nw = 40;
            if (wv == 0 && lane < 5) {
                const fr_t t = ld_fr(tlo[lane], thi[lane], 0);
#pragma unroll
                for (int i = 0; i < 8; i++) pubw[8 * lane + i] = t.v[i];
            }
        }
        __syncthreads();
        if (wv == 0) {
            if (lane == 0) persist_stamp(slot, seq, t_cmd, ZKH_LU_PSTAMP);
            persist_publish(slot, pubw, nw, seq);
        }
        if (m == 1) return;
        if (wv == 0) {
            uint4 qd;
            const uint32_t nq = dbl ? zkh_quad_count(32) : 3;
            const bool ok = persist_wait(P.cmd, nq, seq, P.err, P.deadline, qd);
            if (lane < nq) {
                sxw[3 * lane] = qd.y;
                sxw[3 * lane + 1] = qd.z;
                sxw[3 * lane + 2] = qd.w;
            }
            if (lane == 0) sok = ok;
            t_cmd = wall_clock64();
        }
        __syncthreads();
        if (!sok) return;
        if (dbl) {  // double fold m -> m/4 of the five tables: four products per output
            const uint32_t q = m >> 2;
            for (uint32_t t = threadIdx.x; t < 5 * q * 4; t += NTP) {  // whole lane quads
                const uint32_t o = t >> 2, term = t & 3, i = o / q, cc = o - i * q;
                fr_t w;
#pragma unroll
                for (int j = 0; j < 8; j++) w.v[j] = sxw[8 * term + j];
                fr_t r = mont_mul_ol(w, ld_fr(tlo[i], thi[i], cc + term * q));
                r = fr_add(r, fr_shfl_xor(r, 1));
                r = fr_add(r, fr_shfl_xor(r, 2));
                if (term == 0) st_fr(tlo[i], thi[i], cc, r);  // T[cc] is read only by this quad
            }
            m >>= 2;
            __syncthreads();
            continue;
        }
        {  // fold the five tables: T[k] <- T[k] + x (T[k + m/2] - T[k])
            fr_t x;
#pragma unroll
            for (int i = 0; i < 8; i++) x.v[i] = sxw[i];
            const uint32_t h = m >> 1;
            for (uint32_t t = threadIdx.x; t < 5 * h; t += NTP) {
                const uint32_t i = t / h, k = t - i * h;
                const fr_t v0 = ld_fr(tlo[i], thi[i], k), v1 = ld_fr(tlo[i], thi[i], k + h);
                st_fr(tlo[i], thi[i], k, fr_add(v0, mont_mul_ol(x, fr_sub(v1, v0))));
            }
        }
        m >>= 1;
        __syncthreads();
    }
}
hipError_t launch_lu_persist(hipStream_t s, const LuPersist& p) {
    const uint32_t ls = p.n >> p.lgnb;  // LDS: 5 tables of ls + 5 rows of ls/2 entries, 32 B each
    k_lu_persist<<<1u << p.lgnb, NTP, (size_t)ls * 32 * 5 + (size_t)(ls >> 1) * 5 * 32, s>>>(p);
    return hipGetLastError();
}
// An ordinary launch on the stream: the blocks never wait for each other, only for the
// host, and a launch has at most 256 blocks (one per CU at most 32 KiB LDS and 16 waves),
// so all of them are resident once earlier kernels drain.
hipError_t launch_zkip_persist(hipStream_t s, const ZkipPersist& p, uint32_t nblocks) {
    k_zkip_persist<<<nblocks, NTP, (size_t)p.ls_max * 64, s>>>(p);
    return hipGetLastError();
}

}  // namespace zkh
