// zkh.hip -- host side of the C ABI (include/zkh.h): device tensors, the SHA-256
// Fiat-Shamir round loops of the matmul, logUp and Hadamard sumchecks, and the MLE
// primitives, all driving the gfx950 kernels of kernels.hip on one HIP stream per context.
//
// Per round the host receives a few hundred block partials (AoS Fr), adds them, turns the
// sums into the round polynomial, absorbs it, draws the challenge and launches the next
// fused fold+evaluate kernel.  Only 32-byte scalars cross PCIe per round.
#include <hip/hip_runtime.h>

#include <assert.h>
#include <pthread.h>
#include <sched.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/zkh.h"
#include "fr_host.hpp"
#include "g1.hpp"
#include "kernels.hpp"
#include "transcript.hpp"

using namespace zkh;

// One step of a host spin-wait; step k = 0 mod 256 gives the CPU to any other runnable
// thread on the same CPU.  The host threads of a batch all spin, and the scheduler may put
// a woken thread on the CPU of the thread that woke it: two spinning threads on one CPU
// would take turns at the scheduler's time-slice granularity (a two-job batch lost ~4 ms
// in about one step of 40 so, with no CPU time stolen by the host).
static inline void spin_pause(uint64_t k) {
    if ((k & 255) == 0) sched_yield();
    else __builtin_ia32_pause();
}

// Worker `id` of a pool goes on a CPU of its own: the id-th CPU of the process's allowed
// set after the creating thread's current one (ZKH_PIN_WORKERS=0 leaves placement to the
// scheduler, which left a worker sharing the caller's CPU for the first ~40 ms of a
// TinyLlama layer's matmul steps: 0.208 against 0.18 ms per step until it moved).
static void pin_worker(std::thread& t, int id) {
    static const bool on = !(getenv("ZKH_PIN_WORKERS") && atoi(getenv("ZKH_PIN_WORKERS")) == 0);
    if (!on) return;
    cpu_set_t allowed;
    if (sched_getaffinity(0, sizeof(allowed), &allowed) != 0 || CPU_COUNT(&allowed) < 2) return;
    const int here = sched_getcpu();
    std::vector<int> cpus;
    for (int k = 1; k < CPU_SETSIZE; k++) {
        const int cpu = (here + k) % CPU_SETSIZE;
        if (CPU_ISSET(cpu, &allowed)) cpus.push_back(cpu);
    }
    if (cpus.empty()) return;
    cpu_set_t one;
    CPU_ZERO(&one);
    CPU_SET(cpus[(size_t)(id - 1) % cpus.size()], &one);
    (void)pthread_setaffinity_np(t.native_handle(), sizeof(one), &one);
}

// Host worker threads for the per-job work of a batch (every job has its own transcript,
// so jobs advance independently).  run(n, f) calls f(0) on the calling thread, offers
// f(1) .. f(n-1) to the workers and returns when f(0) returns, without waiting for them:
// a worker that the scheduler leaves off its CPU for a time slice (milliseconds) would
// otherwise stall a caller whose task is already done.  A worker may therefore call f(t)
// late, after run() has returned, or not at all.  A task is written so that the calling thread alone completes it, it touches the
// caller's frame only while holding a claim that the caller waits for, and otherwise
// only state that it holds by value.  After a task a worker polls for the next one for
// about a millisecond, then sleeps on a condition variable.
struct HostPool {
    struct Worker {  // one worker thread and its task slot
        std::mutex mu;
        std::condition_variable cv;
        std::function<void(int)> task;
        std::atomic<uint64_t> gen{0};  // tasks posted to this worker
        bool stop = false;
        std::thread th;
    };
    std::vector<std::unique_ptr<Worker>> w;
    void ensure(int n) {
        while ((int)w.size() < n) {
            w.push_back(std::make_unique<Worker>());
            Worker* W = w.back().get();
            const int id = (int)w.size();
            W->th = std::thread([W, id] {
                uint64_t seen = 0;
                for (;;) {
                    const auto t0 = std::chrono::steady_clock::now();
                    for (uint32_t k = 1; W->gen.load(std::memory_order_acquire) == seen; k++) {
                        spin_pause(k);
                        if ((k & 1023) == 0 &&
                            std::chrono::steady_clock::now() - t0 > std::chrono::microseconds(1000))
                            break;
                    }
                    std::function<void(int)> f;
                    {
                        std::unique_lock<std::mutex> lk(W->mu);
                        W->cv.wait(lk, [&] { return W->stop || W->gen.load(std::memory_order_acquire) != seen; });
                        if (W->stop) return;
                        seen = W->gen.load(std::memory_order_acquire);  // a late worker takes the latest task
                        f = W->task;
                    }
                    f(id);
                }
            });
            pin_worker(W->th, id);
        }
    }
    // wakes workers 1 .. n-1 only: the others stay asleep
    void run(int n, const std::function<void(int)>& f) {
        if (n > 1) ensure(n - 1);
        for (int i = 0; i + 1 < n; i++) {
            Worker& W = *w[i];
            {
                std::lock_guard<std::mutex> lk(W.mu);
                W.task = f;
                W.gen.fetch_add(1, std::memory_order_acq_rel);
            }
            W.cv.notify_one();
        }
        f(0);
    }
    // stop and join the workers (each finishes the task it is in: a task ends by itself
    // once the caller's share has ended)
    void shutdown() {
        for (auto& W : w) {
            {
                std::lock_guard<std::mutex> lk(W->mu);
                W->stop = true;
            }
            W->cv.notify_one();
        }
        for (auto& W : w)
            if (W->th.joinable()) W->th.join();
        w.clear();
    }
    ~HostPool() { shutdown(); }
};
// body(0) .. body(n - 1) on up to T threads, each item taken by claiming; returns when
// every item has completed.  A worker that starts late finds every item claimed and
// touches only the claim counters, which it holds by value.
static void pool_for(HostPool& pool, int T, uint32_t n, const std::function<void(uint32_t)>& body) {
    struct Claims {
        std::atomic<uint32_t> next{0}, done{0};
    };
    auto cl = std::make_shared<Claims>();
    const std::function<void(uint32_t)>* bp = &body;  // called only for a claimed item
    pool.run(T, [cl, bp, n](int) {
        for (uint32_t i; (i = cl->next.fetch_add(1, std::memory_order_acq_rel)) < n;) {
            (*bp)(i);
            cl->done.fetch_add(1, std::memory_order_acq_rel);
        }
    });
    for (uint64_t k = 1; cl->done.load(std::memory_order_acquire) < n; k++) spin_pause(k);
}
// host threads for the per-job work of a batch, the caller included (ZKH_HOST_THREADS,
// default 4: with one thread the jobs of a TinyLlama layer wait on each other's transcript
// work at every round trip, 0.21 against 0.18 ms per matmul step with 4).  The persistent
// round loops hand each ready message to whichever thread is free, so a thread that the OS
// deschedules delays only the message it is serving.
static int host_threads() {
    static const int n = [] {
        const char* e = getenv("ZKH_HOST_THREADS");
        int v = e ? atoi(e) : 4;
        return v < 1 ? 1 : v > 16 ? 16 : v;
    }();
    return n;
}

// Device buffers of a context's tensors.  A freed tensor's buffer goes back to the pool
// and serves later allocations of the same size class: hipFree synchronises the device
// and costs ~0.2 ms for a 128 MiB buffer, hipMalloc ~0.06 ms.  Every entry point returns
// only after its device work has completed, so a buffer is idle when its tensor is freed.
// The pool is shared with the tensors: one freed after its context releases its buffer.
struct MemPool {
    std::mutex mu;
    std::multimap<size_t, void*> idle;  // size class -> buffer
    size_t held = 0;                    // bytes in `idle`
    bool alive = true;
    static constexpr size_t kMaxHeld = (size_t)16 << 30;
    static size_t size_class(size_t bytes) {
        if (bytes <= 4096) return 4096;
        if (bytes < ((size_t)64 << 20)) {
            size_t c = 4096;
            while (c < bytes) c <<= 1;
            return c;
        }
        const size_t g = (size_t)64 << 20;
        return (bytes + g - 1) / g * g;
    }
    void* get(size_t cls) {
        std::lock_guard<std::mutex> lk(mu);
        auto it = idle.find(cls);
        if (it == idle.end()) return nullptr;
        void* p = it->second;
        idle.erase(it);
        held -= cls;
        return p;
    }
    void put(void* p, size_t cls) {
        {
            std::lock_guard<std::mutex> lk(mu);
            if (alive && held + cls <= kMaxHeld) {
                idle.emplace(cls, p);
                held += cls;
                return;
            }
        }
        (void)hipFree(p);
    }
    void release_all() {
        std::lock_guard<std::mutex> lk(mu);
        for (auto& kv : idle) (void)hipFree(kv.second);
        idle.clear();
        held = 0;
        alive = false;
    }
};

struct zkh_ctx {
    int device = 0;
    std::shared_ptr<MemPool> mem = std::make_shared<MemPool>();
    hipStream_t stream = nullptr;
    std::string err;
    uint32_t* pinned = nullptr;  // host staging for partials and small vectors
    size_t pinned_bytes = 0;
    struct Slot {
        void* p = nullptr;
        size_t bytes = 0;
    };
    std::vector<Slot> slots;
    // round completion (Publish): coherent pinned job sums + flag, device partials/job layouts
    uint32_t* pub_host = nullptr;  // [ZKH_MAX_BATCH][11] Fr sums, then the flag word
    // condition words that kernels set to a call's tag (zeroed once, written with tags only)
    uint32_t* flag_d = nullptr;
    uint32_t flag_tag = 0;
    uint32_t* pub_part = nullptr;  // device partial sums (pub_part_cap Fr)
    size_t pub_part_cap = (size_t)4096 * 11;
    uint32_t* pub_lay = nullptr;   // device [ZKH_MAX_BATCH][3] job layouts (see Publish)
    uint32_t pub_seq = 0;
    // relayed round launches: coherent pinned command (three quads; word 16: a relay's
    // timeout flag) and the device words the relay fills (challenge, abandon flag)
    uint32_t* relay_host = nullptr;
    uint32_t* relay_vm = nullptr;
    uint32_t relay_seq = 0;
    // persistent round loops: coherent pinned block slots / command areas, clock rate
    uint32_t* ps_host = nullptr;
    size_t ps_words = 0;
    uint64_t clock_khz = 100000;
    HostPool workers;
    // the table inverse 1/(T_comb + beta) of the last zkh_lu_tuple_inverse, for the
    // zkh_lu_prove on that T_comb (generation lu_tinv_of) and beta, which takes it over
    zkh_tensor* lu_tinv = nullptr;
    uint64_t lu_tinv_of = 0;
    uint32_t lu_tinv_beta[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    std::mutex err_mu;  // error reporting from worker threads
    // pinned ring for small host->device uploads: a region is reused only after a later
    // stream synchronisation, which every API call performs before returning
    uint8_t* ring = nullptr;
    size_t ring_bytes = 0, ring_off = 0;
    // per-kernel-class timing (zkh_prof_*): events around launches on this stream
    bool prof = false;
    struct ProfRec {
        std::string name;
        double ms = 0, bytes = 0;
        uint64_t launches = 0;
    };
    struct Pending {
        int rec;
        hipEvent_t a, b;
        double bytes;
    };
    std::vector<ProfRec> recs;
    std::vector<Pending> pending;
    std::vector<hipEvent_t> pool;
};

// Times the launches issued during its lifetime under `name` when profiling is on.  With
// kernel_events the scope records no markers of its own: the caller hands start() to the
// first launch and stop() to the last (hipExtLaunchKernel stamps them at the dispatch's own
// start and end), so the time is the kernels' execution without marker-packet overhead.
struct ProfScope {
    zkh_ctx* c;
    int rec = -1;
    hipEvent_t a = nullptr, b = nullptr;
    double bytes;
    bool kev;
    hipEvent_t start() const { return rec >= 0 && a && b ? a : nullptr; }
    hipEvent_t stop() const { return rec >= 0 && a && b ? b : nullptr; }
    ProfScope(zkh_ctx* c_, const char* name, double bytes_, bool kernel_events = false)
        : c(c_), bytes(bytes_), kev(kernel_events) {
        if (!c->prof) return;
        for (size_t i = 0; i < c->recs.size(); i++)
            if (c->recs[i].name == name) rec = (int)i;
        if (rec < 0) {
            c->recs.push_back(zkh_ctx::ProfRec{name});
            rec = (int)c->recs.size() - 1;
        }
        for (hipEvent_t* e : {&a, &b}) {
            if (!c->pool.empty()) {
                *e = c->pool.back();
                c->pool.pop_back();
            } else if (hipEventCreate(e) != hipSuccess) {
                *e = nullptr;
            }
        }
        if (a && !kev) (void)hipEventRecord(a, c->stream);
    }
    ~ProfScope() {
        if (rec < 0 || !a || !b) return;
        if (!kev) (void)hipEventRecord(b, c->stream);
        c->pending.push_back(zkh_ctx::Pending{rec, a, b, bytes});
    }
};
// fold finished event pairs into the records, leaving unfinished ones pending
static void prof_resolve_ready(zkh_ctx* c) {
    size_t keep = 0;
    for (size_t i = 0; i < c->pending.size(); i++) {
        auto& p = c->pending[i];
        float ms = 0;
        if (hipEventQuery(p.b) == hipSuccess && hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
            c->recs[p.rec].ms += ms;
            c->recs[p.rec].bytes += p.bytes;
            c->recs[p.rec].launches++;
            c->pool.push_back(p.a);
            c->pool.push_back(p.b);
        } else {
            c->pending[keep++] = p;
        }
    }
    c->pending.resize(keep);
}
// fold finished event pairs into the records (call after a stream synchronisation)
static void prof_resolve(zkh_ctx* c) {
    for (auto& p : c->pending) {
        float ms = 0;
        if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) {
            c->recs[p.rec].ms += ms;
            c->recs[p.rec].bytes += p.bytes;
            c->recs[p.rec].launches++;
        }
        c->pool.push_back(p.a);
        c->pool.push_back(p.b);
    }
    c->pending.clear();
}

struct zkh_tensor {
    zkh_ctx* ctx = nullptr;
    int kind = ZKH_KIND_FR;
    uint32_t n = 0;
    void* d = nullptr;  // FR: planes (cap entries each); I32/I64: n ints
    uint32_t cap = 0;
    uint32_t bits = 0;  // integer kinds: |v| < 2^bits
    int weights = 0;    // I32 matmul weights stored OUT-major (transposed)
    uint32_t w_in = 0, w_out = 0;
    std::shared_ptr<MemPool> pool;  // owner of d (size class cls)
    size_t cls = 0;
    bool ones = false;  // an I32 tensor whose entries are all 1 (measured at ingest)
    // identity of the contents: a fresh number at creation and after every in-place change
    uint64_t gen = 0;
    // set by zkh_lu_inverse: this tensor is 1/(S + beta) entry-wise (inverse(0) = 0) for
    // the tensor S of generation inv_of (0: no such knowledge)
    uint64_t inv_of = 0;
    uint32_t inv_beta[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    // an inverse (as inv_of) known to have no zero entry (no S[i] + beta was zero)
    bool inv_nz = false;
    // set by zkh_lu_mapping on its S: S[i] = mapped[(G[i] - low).limb0] for the tensors G and
    // mapped of generations map_G, map_mapped (0: no such knowledge)
    uint64_t map_G = 0, map_mapped = 0;
    int32_t map_low = 0;
    // set by zkh_lu_range_table: entry j is range_low + min(j, range_len - 1) while gen is
    // range_gen (0: no such knowledge)
    uint64_t range_gen = 0;
    int32_t range_low = 0;
    uint32_t range_len = 0;
    DevPlanes planes() const { return DevPlanes{(uint32_t*)d, cap}; }
};
static uint64_t next_gen() {
    static std::atomic<uint64_t> g{0};
    return ++g;
}

// ---------------------------------------------------------------------------------------
// errors and scratch
// ---------------------------------------------------------------------------------------
static int fail(zkh_ctx* c, int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (c) c->err = buf;
    return code;
}
#define HIPCHK(ctx, x)                                                                  \
    do {                                                                                \
        hipError_t e_ = (x);                                                            \
        if (e_ != hipSuccess)                                                           \
            return fail((ctx), ZKH_EDEV, "%s failed: %s", #x, hipGetErrorString(e_)); \
    } while (0)

// named scratch slots, grown on demand (freed with the context)
enum {
    SL_PARTIAL = 0,
    SL_SMALL,
    SL_FAC,
    SL_ELO,
    SL_EHI,
    SL_EB,
    SL_EO,
    SL_TMP0,
    SL_TMP1,
    SL_TMP2,
    SL_TMP3,
    SL_TMP4,
    SL_TMP5,
    SL_TMP6,
    SL_DESC,
    SL_COUNT
};
static void* scratch_slot(zkh_ctx* c, int slot, size_t bytes, int* rc) {
    if ((int)c->slots.size() < SL_COUNT) c->slots.resize(SL_COUNT);
    zkh_ctx::Slot& s = c->slots[slot];
    if (s.bytes >= bytes && s.p) return s.p;
    if (s.p) {
        (void)hipStreamSynchronize(c->stream);
        (void)hipFree(s.p);
        s.p = nullptr;
        s.bytes = 0;
    }
    size_t want = bytes < 4096 ? 4096 : bytes;
    if (hipMalloc(&s.p, want) != hipSuccess) {
        *rc = fail(c, ZKH_EDEV, "hipMalloc(%zu) failed", want);
        return nullptr;
    }
    s.bytes = want;
    return s.p;
}
// Device scratch of the allocation-free entry point zkh_me_static: its eq factor table, the
// two eq tables (up to ZKH_STATIC_MAX_VARS variables), the block partials and job layout of
// its one reduction.  Every device holds its own copy, at its own address, for
// the life of the process; host code uses only the address that hipGetSymbolAddress gives
// for the current device (kept per device at context creation), never the array's name.
// Calls that overlap on one device share the copy and race.
static constexpr size_t kStFac = 0;                                  // <= 24 x 2 Fr
static constexpr size_t kStElo = 4096;                               // 1024 Fr
static constexpr size_t kStEhi = kStElo + 1024 * 32;                 // 2^(24-10) Fr
static constexpr size_t kStPart = kStEhi + ((size_t)32 << (ZKH_STATIC_MAX_VARS - 10));  // 1024 Fr
static constexpr size_t kStLay = kStPart + 1024 * 32;               // 3 words (+ padding)
static constexpr size_t kStBytes = kStLay + 256;                     // 557,312 bytes
static __device__ __align__(256) uint8_t scratch[kStBytes];
#define ZKH_MAX_DEVICES 64
static uint8_t* g_static_scratch[ZKH_MAX_DEVICES];
static std::mutex g_static_mu;
// resolve this device's copy once (the device must be current)
static int static_scratch_init(int device) {
    if (device < 0 || device >= ZKH_MAX_DEVICES) return ZKH_EARG;
    std::lock_guard<std::mutex> lk(g_static_mu);
    if (g_static_scratch[device]) return ZKH_OK;
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return ZKH_EDEV;
    g_static_scratch[device] = (uint8_t*)p;
    return ZKH_OK;
}
static uint8_t* static_scratch(int device) {
    std::lock_guard<std::mutex> lk(g_static_mu);
    return device >= 0 && device < ZKH_MAX_DEVICES ? g_static_scratch[device] : nullptr;
}

static DevPlanes scratch_planes(zkh_ctx* c, int slot, uint32_t n, int* rc) {
    uint32_t cap = n ? n : 1;
    void* p = scratch_slot(c, slot, (size_t)cap * 32, rc);
    return DevPlanes{(uint32_t*)p, cap};
}
static int ensure_pinned(zkh_ctx* c, size_t bytes) {
    if (c->pinned_bytes >= bytes) return 0;
    if (c->pinned) (void)hipHostFree(c->pinned);
    c->pinned = nullptr;
    size_t want = std::max(bytes, (size_t)1 << 20);
    if (hipHostMalloc((void**)&c->pinned, want, hipHostMallocDefault) != hipSuccess)
        return fail(c, ZKH_EDEV, "hipHostMalloc(%zu) failed", want);
    c->pinned_bytes = want;
    return 0;
}
// coherent pinned words for the persistent loops' block slots and command areas; the
// stream is drained before a regrow so no running kernel still points at the old area
static int ensure_ps(zkh_ctx* c, size_t words) {
    if (c->ps_words >= words) return 0;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    if (c->ps_host) (void)hipHostFree(c->ps_host);
    c->ps_host = nullptr;
    c->ps_words = 0;
    const size_t want = std::max(words, (size_t)1 << 16);
    if (hipHostMalloc((void**)&c->ps_host, want * 4, hipHostMallocCoherent) != hipSuccess)
        return fail(c, ZKH_EDEV, "hipHostMalloc(coherent, %zu) failed", want * 4);
    memset(c->ps_host, 0, want * 4);
    c->ps_words = want;
    return 0;
}
// ---- convention cross-checks (ZKH_XCHECK=1): the reference's "fold terminals ==
// multi_dim_me" guards (zkob_fc.cu:337-345, zkob_glu.cu:186-192, :254-260,
// zkob_rescale.cu:151-165): after a proof, each folded terminal is recomputed as the MLE of
// its input table at the opening point, and a mismatch fails the call (ZKH_EROUND).  The
// logUp and Hadamard round kernels then also compute every round's sums at 1 instead of
// deriving them from the pieces' claims, so p(0) + p(1) = claim is checked per round on
// device sums (zkob_lookup.cuh:155, :183, :303).  Off by default: the sumcheck algebra
// already implies the equalities, the re-evaluations cost extra passes over the inputs. ----
static bool xcheck_on() {
    static const bool on = getenv("ZKH_XCHECK") && atoi(getenv("ZKH_XCHECK")) > 0;
    return on;
}
// ---- host-side round trace (ZKH_TRACE=1): per-round launch / wait / host times ----
static bool trace_on() {
    static const bool on = getenv("ZKH_TRACE") && atoi(getenv("ZKH_TRACE")) > 0;
    return on;
}
static double now_us() {
    return std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

// ---- round completion without stream synchronisation ----
static uint32_t* pub_flag(zkh_ctx* c) { return c->pub_host + ZKH_MAX_BATCH * 11 * 8; }
static Publish make_pub(zkh_ctx* c, uint32_t njobs) {
    Publish p;
    p.part = c->pub_part;
    p.layout = c->pub_lay;
    p.host_out = c->pub_host;
    p.host_flag = pub_flag(c);
    p.seq = ++c->pub_seq;
    p.njobs = njobs;
    return p;
}
// spin until the launch carrying `seq` has published (the kernel never waits on the host,
// so this cannot hang the GPU; a stream error or a finished stream without the flag fails)
static int wait_pub(zkh_ctx* c, uint32_t seq) {
    uint32_t* f = pub_flag(c);
    for (uint64_t spins = 1;; spins++) {
        if (__atomic_load_n(f, __ATOMIC_ACQUIRE) == seq) break;
        if ((spins & 0x3FFF) == 0) {
            hipError_t e = hipStreamQuery(c->stream);
            if (e == hipSuccess) {
                if (__atomic_load_n(f, __ATOMIC_ACQUIRE) == seq) break;
                return fail(c, ZKH_EDEV, "round kernel finished without publishing its sums");
            }
            if (e != hipErrorNotReady) return fail(c, ZKH_EDEV, "round kernel: %s", hipGetErrorString(e));
        }
        spin_pause(spins);
    }
    c->ring_off = 0;  // everything queued before the publishing kernel has completed
    if (c->prof) prof_resolve_ready(c);
    return 0;
}
// the K published sums of job j
static void pub_read(zkh_ctx* c, uint32_t j, int K, Fr* out) {
    for (int k = 0; k < K; k++) out[k] = fr_load(c->pub_host + ((size_t)j * K + k) * 8);
}
// completion of everything queued on the stream so far: a one-thread kernel stores a flag
// to pinned memory and the host spins on it (wakes sooner than hipStreamSynchronize); when
// word (device) is given, its value reaches *out on the way.  Only for device-side work:
// a copy into pageable host memory still needs hipStreamSynchronize.
static int settle(zkh_ctx* c, const uint32_t* word = nullptr, uint32_t* out = nullptr, uint32_t nwords = 1) {
    const uint32_t seq = ++c->pub_seq;
    uint32_t* hw = pub_flag(c) + 1;
    launch_fence(c->stream, pub_flag(c), seq, word, nwords, hw);
    const int rc = wait_pub(c, seq);
    for (uint32_t i = 0; !rc && out && i < nwords; i++) out[i] = __atomic_load_n(hw + i, __ATOMIC_ACQUIRE);
    return rc;
}
// A condition word of the device (c->flag_d + word) that kernels set to `tag` (plain stores,
// no prior clearing): its words start at 0 and only ever receive tags, so a word left by an
// earlier call never equals a new call's tag.  tag 0 (the global-atomics multiplicity
// path): a word the caller zeroed, nonzero when set.
struct DevFlag {
    uint32_t* d;
    uint32_t tag;
    bool hit(uint32_t w) const { return tag ? w == tag : w != 0; }
};
enum { kFlagHist = 0, kFlagInvZero = 1, kFlagGather = 2 /* 2 words */ };
static DevFlag dev_flag(zkh_ctx* c, uint32_t word) {
    if (++c->flag_tag == 0) {  // tags wrapped: clear the words once, then start again at 1
        (void)hipMemsetAsync(c->flag_d, 0, 64 * 4, c->stream);
        c->flag_tag = 1;
    }
    return DevFlag{c->flag_d + word, c->flag_tag};
}

// ---- relayed round launches.  A round kernel can be queued before the host has the
// previous round's challenge: a relay (one wave, launch_relay) ahead of it on the stream
// waits for the challenge in the pinned command and copies it to device words that the
// kernel reads, so the kernel's launch overlaps the previous round and the host's
// transcript work.  At most one relay is outstanding per context. ----
static uint32_t relay_enqueue(zkh_ctx* c) {
    uint32_t seq = ++c->relay_seq;
    if (seq == 0 || seq == ZKH_QUIT) seq = c->relay_seq = 1;
    launch_relay(c->stream, c->relay_host, seq, c->relay_host + 16, c->clock_khz * 1000 * 20, c->relay_vm);
    return seq;
}
// hand the challenge (Montgomery form) to the relay waiting for seq
static void relay_send(zkh_ctx* c, uint32_t seq, const uint32_t vm[8]) {
    uint32_t* cmd = c->relay_host;
    for (uint32_t i = 0; i < 8; i++) __atomic_store_n(cmd + zkh_quad_word(i), vm[i], __ATOMIC_RELAXED);
    for (uint32_t q = 0; q < 3; q++) __atomic_store_n(cmd + 4 * q, seq, __ATOMIC_RELEASE);
}
// release a waiting relay without a challenge: it flags its kernel to return at once; the
// stream drains before the command is cleared for the next relay
static void relay_quit(zkh_ctx* c) {
    uint32_t* cmd = c->relay_host;
    for (uint32_t q = 0; q < 3; q++) __atomic_store_n(cmd + 4 * q, ZKH_QUIT, __ATOMIC_RELEASE);
    (void)hipStreamSynchronize(c->stream);
    for (uint32_t q = 0; q < 3; q++) __atomic_store_n(cmd + 4 * q, 0u, __ATOMIC_RELEASE);
}
// releases the outstanding relay of a round loop that returns early
struct RelayGuard {
    zkh_ctx* c;
    uint32_t pending = 0;
    ~RelayGuard() {
        if (pending) relay_quit(c);
    }
};

// small host -> device upload through the pinned ring (asynchronous; ordered on the stream)
static int upload(zkh_ctx* c, void* dst, const void* src, size_t bytes) {
    size_t need = (bytes + 255) & ~(size_t)255;
    if (need > c->ring_bytes) {
        HIPCHK(c, hipStreamSynchronize(c->stream));
        if (c->ring) (void)hipHostFree(c->ring);
        c->ring = nullptr;
        c->ring_bytes = std::max(need, (size_t)1 << 20);
        if (hipHostMalloc((void**)&c->ring, c->ring_bytes, hipHostMallocDefault) != hipSuccess) {
            c->ring_bytes = 0;
            return fail(c, ZKH_EDEV, "hipHostMalloc(ring) failed");
        }
        c->ring_off = 0;
    }
    if (c->ring_off + need > c->ring_bytes) {  // wrap: earlier regions must have been consumed
        HIPCHK(c, hipStreamSynchronize(c->stream));
        c->ring_off = 0;
    }
    uint8_t* h = c->ring + c->ring_off;
    c->ring_off += need;
    memcpy(h, src, bytes);
    HIPCHK(c, hipMemcpyAsync(dst, h, bytes, hipMemcpyHostToDevice, c->stream));
    return 0;
}
static uint32_t ceil_log2(uint32_t n) {
    uint32_t r = 0;
    if (n <= 1) return 0;
    n--;
    while (n) {
        n >>= 1;
        r++;
    }
    return r;
}
static uint32_t bits_for(uint64_t absmax) {
    uint32_t b = 0;
    while (b < 63 && ((uint64_t)1 << b) <= absmax) b++;
    return b;  // absmax < 2^b
}
static Fr fix1(const Fr& x) { return fr_mont_mul(x, kR2); }  // undo one 2^-256
// The round logic's products take one Montgomery product each when one operand is prepared:
// mulm(a, to_m(b)) = a b (plain), and mulm(x, to_mm(c)) = fix1(x) c for a device sum x that
// carries one 2^-256.
static inline Fr mulm(const Fr& a, const Fr& bm) { return fr_mont_mul(a, bm); }
static inline Fr to_m(const Fr& b) { return fr_to_mont(b); }
static inline Fr to_mm(const Fr& c) { return fr_to_mont(fr_to_mont(c)); }
// e(1), e(2), e(3) of the cubic c0 + c1 t + c2 t^2 + c3 t^3 (Horner by additions)
static void cubic_at123(const Fr c[4], Fr e[4]) {
    e[0] = c[0];
    e[1] = fr_add(fr_add(c[0], c[1]), fr_add(c[2], c[3]));
    Fr a2 = c[3], a3 = c[3];
    for (int i = 2; i >= 0; i--) {
        a2 = fr_add(fr_add(a2, a2), c[i]);
        a3 = fr_add(fr_add(fr_add(a3, a3), a3), c[i]);
    }
    e[2] = a2;
    e[3] = a3;
}
// c(v) of the cubic by Horner, vm = to_m(v)
static Fr cubic_at(const Fr c[4], const Fr& vm) {
    Fr acc = c[3];
    for (int i = 2; i >= 0; i--) acc = fr_add(mulm(acc, vm), c[i]);
    return acc;
}
static Fr fix2(const Fr& x) {
    static const Fr r3 = fr_rpow(3);
    return fr_mont_mul(x, r3);
}

// Montgomery factor table of u: fac[2t] = mont(1-u_t), fac[2t+1] = mont(u_t), for
// t < nvars; positions t >= len(u) (up to pad) are (mont(1), 0)
static void make_fac(const std::vector<Fr>& u, uint32_t pad, std::vector<uint32_t>& out) {
    uint32_t nv = std::max<uint32_t>((uint32_t)u.size(), pad);
    out.assign((size_t)nv * 16, 0);
    for (uint32_t t = 0; t < nv; t++) {
        Fr a, b;
        if (t < u.size()) {
            a = fr_to_mont(fr_sub(kOne, u[t]));
            b = fr_to_mont(u[t]);
        } else {
            a = fr_to_mont(kOne);
            b = kZero;
        }
        fr_store(a, &out[(size_t)t * 16]);
        fr_store(b, &out[(size_t)t * 16 + 8]);
    }
}
// sum_{b < K} eq(b, u) for K <= 2^|u|
static Fr eq_prefix_sum(const std::vector<Fr>& u, uint64_t K) {
    uint32_t k = (uint32_t)u.size();
    if (K >= ((uint64_t)1 << k)) return kOne;
    Fr sum = kZero, prod = kOne;
    for (int j = (int)k - 1; j >= 0; j--) {
        Fr om = fr_sub(kOne, u[j]);
        if ((K >> j) & 1) {
            sum = fr_add(sum, fr_mul(prod, om));
            prod = fr_mul(prod, u[j]);
        } else {
            prod = fr_mul(prod, om);
        }
    }
    return sum;
}

// eq weighting state for the Elo/Ehi kernels (EqW): Elo over u[0..10), Ehi over
// u[10..kmax), kmax = max(|u|, 10); corr[K] = 1/prod_{t=K}^{kmax-1}(1 - u_t) turns the
// device weights of the first 2^K indices into eq(i, u[0..K)).
struct EqState {
    uint32_t* elo_d = nullptr;
    uint32_t* ehi_d = nullptr;
    std::vector<Fr> corr;     // corr[K] for K = 0..kmax
    std::vector<Fr> inv1mu;   // 1 / (1 - u_t) for t < kmax (empty for a degenerate point)
    uint32_t nvars = 0;
    bool host_done = false;   // corr and inv1mu formed (eq_setup_host)
};
// all_rounds: the caller will weight shorter prefixes K < |u| (sumcheck rounds), which
// needs every 1 - u_t invertible; a single full-length weighting (K = |u|) needs no
// correction and accepts any point, e.g. a Boolean one.
// The host part (corr, inv1mu: one inversion) can be left to eq_setup_host, so that a prover
// queues its first round before that work (host_now = false).
static int eq_setup_host(zkh_ctx* c, const std::vector<Fr>& u, EqState& st, bool all_rounds = true);
static int eq_setup(zkh_ctx* c, const std::vector<Fr>& u, EqState& st, bool all_rounds = true,
                    bool host_now = true) {
    int rc = 0;
    std::vector<uint32_t> fac;
    make_fac(u, 10, fac);
    st.nvars = (uint32_t)u.size();
    const uint32_t kmax = std::max<uint32_t>(st.nvars, 10), khi = kmax - 10;
    st.elo_d = (uint32_t*)scratch_slot(c, SL_ELO, 1024 * 32, &rc);
    if (rc) return rc;
    st.ehi_d = (uint32_t*)scratch_slot(c, SL_EHI, ((size_t)32 << khi), &rc);
    if (rc) return rc;
    // the factors as launch arguments where they fit (no upload ahead of the tables' launch)
    bool launched = false;
    if (fac.size() <= sizeof(FacArg) / 4) {
        FacArg fa;
        memcpy(fa.w, fac.data(), fac.size() * 4);
        launched = launch_eq_mont2_ka(c->stream, fa, 10, 1024, st.elo_d, khi, 1u << khi, st.ehi_d);
    }
    if (!launched) {
        uint32_t* fac_d = (uint32_t*)scratch_slot(c, SL_FAC, fac.size() * 4, &rc);
        if (rc) return rc;
        if ((rc = upload(c, fac_d, fac.data(), fac.size() * 4))) return rc;
        launch_eq_mont2(c->stream, fac_d, 10, 1024, st.elo_d, fac_d + 2 * 10 * 8, khi, 1u << khi, st.ehi_d);
    }
    return host_now ? eq_setup_host(c, u, st, all_rounds) : 0;
}
static int eq_setup_host(zkh_ctx* c, const std::vector<Fr>& u, EqState& st, bool all_rounds) {
    if (st.host_done) return 0;
    st.host_done = true;
    const uint32_t kmax = std::max<uint32_t>(st.nvars, 10);
    // prefix[K] = prod_{t<K} (1 - u_t); corr[K] = prefix[K] / prefix[kmax]
    std::vector<Fr> prefix(kmax + 1);
    prefix[0] = kOne;
    for (uint32_t t = 0; t < kmax; t++)
        prefix[t + 1] = fr_mul(prefix[t], t < st.nvars ? fr_sub(kOne, u[t]) : kOne);
    if (fr_eq(prefix[kmax], kZero)) {
        if (all_rounds) return fail(c, ZKH_EARG, "degenerate eq challenge (u_t = 1)");
        st.corr.assign(kmax + 1, kZero);
        st.corr[st.nvars] = kOne;  // the factors of positions >= |u| are 1 - 0
        return 0;
    }
    const Fr inv = fr_inv(prefix[kmax]);
    st.corr.resize(kmax + 1);
    for (uint32_t K = 0; K <= kmax; K++) st.corr[K] = fr_mul(prefix[K], inv);
    // 1 / (1 - u_t) = prefix[t] / prefix[t + 1], with 1 / prefix[t] = (1 - u_t) / prefix[t + 1]
    st.inv1mu.resize(kmax);
    Fr ip = inv;  // 1 / prefix[t + 1]
    for (uint32_t t = kmax; t-- > 0;) {
        st.inv1mu[t] = fr_mul(prefix[t], ip);
        ip = fr_mul(ip, t < st.nvars ? fr_sub(kOne, u[t]) : kOne);
    }
    return 0;
}
static Fr eq_corr(const EqState& st, uint32_t K) {
    assert(st.host_done);
    return st.corr[K];
}

static std::vector<Fr> load_frs(const uint32_t* p, uint32_t n) {
    std::vector<Fr> v(n);
    for (uint32_t i = 0; i < n; i++) v[i] = fr_load(p + 8 * (size_t)i);
    return v;
}
static bool all_canonical(const uint32_t* p, uint32_t n) {
    for (uint32_t i = 0; i < n; i++)
        if (!fr_is_canonical(p + 8 * (size_t)i)) return false;
    return true;
}

// ---------------------------------------------------------------------------------------
// context
// ---------------------------------------------------------------------------------------
extern "C" int zkh_ctx_create(int device, zkh_ctx** out) {
    if (!out) return ZKH_EARG;
    *out = nullptr;
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev <= 0) return ZKH_EDEV;
    if (device < 0 || device >= ndev) return ZKH_EARG;
    zkh_ctx* c = new zkh_ctx();
    c->device = device;
    if (hipSetDevice(device) != hipSuccess || static_scratch_init(device) != ZKH_OK ||
        hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return ZKH_EDEV;
    }
    c->slots.resize(SL_COUNT);
    if (hipHostMalloc((void**)&c->pub_host, (ZKH_MAX_BATCH * 11 * 8 + 64) * 4, hipHostMallocCoherent) != hipSuccess ||
        hipMalloc((void**)&c->pub_part, (size_t)4096 * 11 * 32) != hipSuccess ||
        hipMalloc((void**)&c->pub_lay, ZKH_MAX_BATCH * 3 * 4) != hipSuccess ||
        hipMemset(c->pub_lay, 0, ZKH_MAX_BATCH * 3 * 4) != hipSuccess ||
        hipHostMalloc((void**)&c->relay_host, 64 * 4, hipHostMallocCoherent) != hipSuccess ||
        hipMalloc((void**)&c->relay_vm, 16 * 4) != hipSuccess || hipMalloc((void**)&c->flag_d, 64 * 4) != hipSuccess ||
        hipMemset(c->flag_d, 0, 64 * 4) != hipSuccess) {
        (void)hipStreamDestroy(c->stream);
        delete c;
        return ZKH_EDEV;
    }
    memset(c->pub_host, 0, (ZKH_MAX_BATCH * 11 * 8 + 64) * 4);
    memset(c->relay_host, 0, 64 * 4);
    int khz = 0;
    if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device) == hipSuccess && khz > 0)
        c->clock_khz = (uint64_t)khz;
    if (ensure_pinned(c, (size_t)1 << 20)) {
        (void)hipStreamDestroy(c->stream);
        delete c;
        return ZKH_EDEV;
    }
    *out = c;
    return ZKH_OK;
}
extern "C" int zkh_ctx_destroy(zkh_ctx* c) {
    if (!c) return ZKH_EARG;
    c->workers.shutdown();  // a worker still in a finished task may poll the stream and pinned areas
    (void)hipSetDevice(c->device);
    (void)hipStreamSynchronize(c->stream);
    if (c->lu_tinv) zkh_tensor_free(c->lu_tinv);
    c->mem->release_all();
    for (auto& s : c->slots)
        if (s.p) (void)hipFree(s.p);
    if (c->pinned) (void)hipHostFree(c->pinned);
    if (c->ring) (void)hipHostFree(c->ring);
    if (c->pub_host) (void)hipHostFree(c->pub_host);
    if (c->ps_host) (void)hipHostFree(c->ps_host);
    if (c->pub_part) (void)hipFree(c->pub_part);
    if (c->pub_lay) (void)hipFree(c->pub_lay);
    if (c->relay_host) (void)hipHostFree(c->relay_host);
    if (c->relay_vm) (void)hipFree(c->relay_vm);
    if (c->flag_d) (void)hipFree(c->flag_d);
    for (auto& p : c->pending) {
        c->pool.push_back(p.a);
        c->pool.push_back(p.b);
    }
    for (hipEvent_t e : c->pool) (void)hipEventDestroy(e);
    (void)hipStreamDestroy(c->stream);
    delete c;
    return ZKH_OK;
}

// ---------------------------------------------------------------------------------------
// kernel timing (tracing aid; the reference's BoTimer laps, zkob_claims.cuh:68-75)
// ---------------------------------------------------------------------------------------
extern "C" int zkh_prof_enable(zkh_ctx* c, int on) {
    if (!c) return ZKH_EARG;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    prof_resolve(c);
    c->recs.clear();
    c->prof = on != 0;
    return ZKH_OK;
}
extern "C" int zkh_prof_get(zkh_ctx* c, const char* name, double* ms, uint64_t* launches,
                            double* bytes) {
    if (!c || !name) return ZKH_EARG;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    prof_resolve(c);
    for (auto& r : c->recs)
        if (r.name == name) {
            if (ms) *ms = r.ms;
            if (launches) *launches = r.launches;
            if (bytes) *bytes = r.bytes;
            return ZKH_OK;
        }
    if (ms) *ms = 0;
    if (launches) *launches = 0;
    if (bytes) *bytes = 0;
    return ZKH_OK;
}
extern "C" int zkh_prof_names(zkh_ctx* c, char* buf, size_t len) {
    if (!c || !buf || !len) return ZKH_EARG;
    std::string all;
    for (auto& r : c->recs) {
        if (!all.empty()) all += ",";
        all += r.name;
    }
    snprintf(buf, len, "%s", all.c_str());
    return ZKH_OK;
}
extern "C" const char* zkh_last_error(const zkh_ctx* c) { return c ? c->err.c_str() : "null context"; }
extern "C" int zkh_ctx_sync(zkh_ctx* c) {
    if (!c) return ZKH_EARG;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return ZKH_OK;
}

// ---------------------------------------------------------------------------------------
// tensors
// ---------------------------------------------------------------------------------------
static int tensor_alloc(zkh_ctx* c, int kind, uint32_t n, zkh_tensor** out) {
    zkh_tensor* t = new zkh_tensor();
    t->ctx = c;
    t->kind = kind;
    t->n = n;
    t->gen = next_gen();
    size_t bytes;
    if (kind == ZKH_KIND_FR) {
        t->cap = n ? n : 1;
        bytes = (size_t)t->cap * 32;
    } else {
        bytes = (size_t)(n ? n : 1) * (kind == ZKH_KIND_I32 ? 4 : 8);
    }
    t->pool = c->mem;
    t->cls = MemPool::size_class(bytes);
    t->d = c->mem->get(t->cls);
    if (!t->d && hipMalloc(&t->d, t->cls) != hipSuccess) {
        delete t;
        return fail(c, ZKH_EDEV, "hipMalloc(%zu) failed", t->cls);
    }
    *out = t;
    return ZKH_OK;
}
static int int_bits_i32(zkh_ctx* c, const int32_t* d, uint32_t n, uint32_t* bits, bool* ones) {
    int rc = 0;
    uint32_t* m = (uint32_t*)scratch_slot(c, SL_SMALL, 64, &rc);
    if (rc) return rc;
    HIPCHK(c, hipMemsetAsync(m, 0, 8, c->stream));
    launch_absmax_i32(c->stream, d, n, m);
    uint32_t h[2] = {0, 0};
    HIPCHK(c, hipMemcpyAsync(h, m, 8, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    *bits = bits_for(h[0]);
    *ones = n > 0 && h[1] == 0;
    return 0;
}
static int int_bits_i64(zkh_ctx* c, const int64_t* d, uint32_t n, uint32_t* bits) {
    int rc = 0;
    unsigned long long* m = (unsigned long long*)scratch_slot(c, SL_SMALL, 64, &rc);
    if (rc) return rc;
    HIPCHK(c, hipMemsetAsync(m, 0, 8, c->stream));
    launch_absmax_i64(c->stream, d, n, m);
    unsigned long long h = 0;
    HIPCHK(c, hipMemcpyAsync(&h, m, 8, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    *bits = bits_for(h);
    return 0;
}
static int make_int_tensor(zkh_ctx* c, const void* src, uint32_t n, int kind, hipMemcpyKind dir,
                           zkh_tensor** out) {
    if (!c || !out || (!src && n)) return fail(c, ZKH_EARG, "null argument");
    *out = nullptr;
    HIPCHK(c, hipSetDevice(c->device));
    zkh_tensor* t;
    int rc = tensor_alloc(c, kind, n, &t);
    if (rc) return rc;
    size_t es = kind == ZKH_KIND_I32 ? 4 : 8;
    if (n) {
        hipError_t e = hipMemcpyAsync(t->d, src, (size_t)n * es, dir, c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) {
            zkh_tensor_free(t);
            return fail(c, ZKH_EDEV, "tensor upload failed: %s", hipGetErrorString(e));
        }
        rc = kind == ZKH_KIND_I32 ? int_bits_i32(c, (const int32_t*)t->d, n, &t->bits, &t->ones)
                                  : int_bits_i64(c, (const int64_t*)t->d, n, &t->bits);
        if (rc) {
            zkh_tensor_free(t);
            return rc;
        }
    }
    *out = t;
    return ZKH_OK;
}
extern "C" int zkh_tensor_from_i32(zkh_ctx* c, const int32_t* v, uint32_t n, zkh_tensor** out) {
    return make_int_tensor(c, v, n, ZKH_KIND_I32, hipMemcpyHostToDevice, out);
}
extern "C" int zkh_tensor_from_i64(zkh_ctx* c, const int64_t* v, uint32_t n, zkh_tensor** out) {
    return make_int_tensor(c, v, n, ZKH_KIND_I64, hipMemcpyHostToDevice, out);
}
extern "C" int zkh_tensor_from_i32_device(zkh_ctx* c, const int32_t* d, uint32_t n, zkh_tensor** out) {
    return make_int_tensor(c, d, n, ZKH_KIND_I32, hipMemcpyDeviceToDevice, out);
}
extern "C" int zkh_tensor_from_i64_device(zkh_ctx* c, const int64_t* d, uint32_t n, zkh_tensor** out) {
    return make_int_tensor(c, d, n, ZKH_KIND_I64, hipMemcpyDeviceToDevice, out);
}
extern "C" int zkh_tensor_weights_i32(zkh_ctx* c, const int32_t* W, uint32_t in_dim,
                                      uint32_t out_dim, zkh_tensor** out) {
    if (!c || !out || !W || !in_dim || !out_dim) return fail(c, ZKH_EARG, "bad weights arguments");
    uint64_t n64 = (uint64_t)in_dim * out_dim;
    if (n64 >= (1ull << 32)) return fail(c, ZKH_EARG, "weights too large");
    zkh_tensor* rm;
    int rc = zkh_tensor_from_i32(c, W, (uint32_t)n64, &rm);
    if (rc) return rc;
    zkh_tensor* t;
    rc = tensor_alloc(c, ZKH_KIND_I32, (uint32_t)n64, &t);
    if (rc) {
        zkh_tensor_free(rm);
        return rc;
    }
    launch_transpose_i32(c->stream, (const int32_t*)rm->d, in_dim, out_dim, (int32_t*)t->d);
    hipError_t e = hipStreamSynchronize(c->stream);
    t->bits = rm->bits;
    t->weights = 1;
    t->w_in = in_dim;
    t->w_out = out_dim;
    zkh_tensor_free(rm);
    if (e != hipSuccess) {
        zkh_tensor_free(t);
        return fail(c, ZKH_EDEV, "transpose failed: %s", hipGetErrorString(e));
    }
    *out = t;
    return ZKH_OK;
}
extern "C" int zkh_tensor_from_fr(zkh_ctx* c, const uint32_t* aos, uint32_t n, zkh_tensor** out) {
    if (!c || !out || (!aos && n)) return fail(c, ZKH_EARG, "null argument");
    *out = nullptr;
    HIPCHK(c, hipSetDevice(c->device));
    zkh_tensor* t;
    int rc = tensor_alloc(c, ZKH_KIND_FR, n, &t);
    if (rc) return rc;
    if (n) {
        // the entries, then one word counting non-canonical entries (checked on the device)
        uint32_t* stage = (uint32_t*)scratch_slot(c, SL_TMP6, (size_t)n * 32 + 256, &rc);
        uint32_t* bad = stage + 8 * (size_t)n;
        uint32_t nbad = 0;
        hipError_t e = hipSuccess;
        if (!rc) e = hipMemcpyAsync(stage, aos, (size_t)n * 32, hipMemcpyHostToDevice, c->stream);
        if (!rc && e == hipSuccess) e = hipMemsetAsync(bad, 0, 4, c->stream);
        if (!rc && e == hipSuccess) {
            launch_count_noncanonical(c->stream, stage, n, bad);
            launch_aos_to_planes(c->stream, stage, n, t->planes());
            e = hipMemcpyAsync(&nbad, bad, 4, hipMemcpyDeviceToHost, c->stream);
        }
        if (!rc && e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (rc || e != hipSuccess) {
            zkh_tensor_free(t);
            return rc ? rc : fail(c, ZKH_EDEV, "upload failed: %s", hipGetErrorString(e));
        }
        if (nbad) {
            zkh_tensor_free(t);
            return fail(c, ZKH_EARG, "non-canonical field element");
        }
    }
    *out = t;
    return ZKH_OK;
}
extern "C" int zkh_tensor_free(zkh_tensor* t) {
    if (!t) return ZKH_EARG;
    if (t->d) {
        if (t->pool) t->pool->put(t->d, t->cls);
        else (void)hipFree(t->d);
    }
    delete t;
    return ZKH_OK;
}
extern "C" uint32_t zkh_tensor_size(const zkh_tensor* t) { return t ? t->n : 0; }
extern "C" int zkh_tensor_kind(const zkh_tensor* t) { return t ? t->kind : -1; }

// FR planes view of any tensor (integer tensors are converted into the given scratch slot)
static int as_planes(zkh_ctx* c, const zkh_tensor* t, int slot, DevPlanes* out) {
    int rc = 0;
    if (t->kind == ZKH_KIND_FR) {
        *out = t->planes();
        return 0;
    }
    DevPlanes p = scratch_planes(c, slot, t->n, &rc);
    if (rc) return rc;
    if (t->kind == ZKH_KIND_I32) {
        if (t->weights) {
            // logical W (IN x OUT) from the OUT-major copy
            int32_t* rm = (int32_t*)scratch_slot(c, SL_TMP5, (size_t)t->n * 4, &rc);
            if (rc) return rc;
            launch_transpose_i32(c->stream, (const int32_t*)t->d, t->w_out, t->w_in, rm);
            launch_i32_to_planes(c->stream, rm, t->n, p);
        } else {
            launch_i32_to_planes(c->stream, (const int32_t*)t->d, t->n, p);
        }
    } else {
        launch_i64_to_planes(c->stream, (const int64_t*)t->d, t->n, p);
    }
    *out = p;
    return 0;
}
extern "C" int zkh_tensor_to_i64(zkh_ctx* c, const zkh_tensor* t, int64_t* out) {
    if (!c || !t || (!out && t->n)) return fail(c, ZKH_EARG, "null argument");
    if (!t->n) return ZKH_OK;
    HIPCHK(c, hipSetDevice(c->device));
    int rc;
    DevPlanes p;
    if ((rc = as_planes(c, t, SL_TMP4, &p))) return rc;
    int64_t* d = (int64_t*)scratch_slot(c, SL_TMP6, (size_t)t->n * 8, &rc);
    if (rc) return rc;
    launch_to_long(c->stream, p, t->n, d);
    HIPCHK(c, hipMemcpyAsync(out, d, (size_t)t->n * 8, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return ZKH_OK;
}
extern "C" int zkh_tensor_to_fr(zkh_ctx* c, const zkh_tensor* t, uint32_t* aos) {
    if (!c || !t || (!aos && t->n)) return fail(c, ZKH_EARG, "null argument");
    if (!t->n) return ZKH_OK;
    HIPCHK(c, hipSetDevice(c->device));
    int rc = 0;
    DevPlanes p;
    if ((rc = as_planes(c, t, SL_TMP4, &p))) return rc;
    uint32_t* stage = (uint32_t*)scratch_slot(c, SL_TMP6, (size_t)t->n * 32, &rc);
    if (rc) return rc;
    launch_planes_to_aos(c->stream, p, t->n, stage);
    HIPCHK(c, hipMemcpyAsync(aos, stage, (size_t)t->n * 32, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return ZKH_OK;
}

// ---------------------------------------------------------------------------------------
// transcript
// ---------------------------------------------------------------------------------------
extern "C" int zkh_transcript_init(uint8_t st[32], const char* seed, size_t n) {
    if (!st || (!seed && n)) return ZKH_EARG;
    tr_init(st, seed, n);
    return ZKH_OK;
}
extern "C" int zkh_transcript_absorb(uint8_t st[32], const char* label, size_t llen,
                                     const void* data, size_t len) {
    if (!st || (!label && llen) || (!data && len)) return ZKH_EARG;
    tr_absorb(st, label, llen, data, len);
    return ZKH_OK;
}
extern "C" int zkh_transcript_challenge_fr(uint8_t st[32], uint32_t out[8]) {
    if (!st || !out) return ZKH_EARG;
    tr_challenge_limbs(st, out);
    return ZKH_OK;
}
extern "C" int zkh_transcript_challenge_vec(uint8_t st[32], uint32_t n, uint32_t* out) {
    if (!st || (!out && n)) return ZKH_EARG;
    for (uint32_t i = 0; i < n; i++) tr_challenge_limbs(st, out + 8 * (size_t)i);
    return ZKH_OK;
}

// ---------------------------------------------------------------------------------------
// MLE primitives
// ---------------------------------------------------------------------------------------
// sum_i eq(i,u) * S[i] (* U[i]) over i < n, with n <= 2^|u|
static int eq_weighted_sum(zkh_ctx* c, DevPlanes S, const DevPlanes* U, uint32_t n,
                           const std::vector<Fr>& u, Fr* out) {
    int rc = 0;
    EqState st;
    if ((rc = eq_setup(c, u, st, false))) return rc;
    uint32_t K = (uint32_t)u.size();
    uint32_t nb;
    {
        ProfScope ps(c, "eq_sum", (double)n * (U ? 64 : 32));
        Publish pb = make_pub(c, 1);
        nb = launch_eq_sum(c->stream, S, U, n, EqW{st.elo_d, st.ehi_d, K}, pb);
        (void)nb;
        if ((rc = wait_pub(c, pb.seq))) return rc;
    }
    Fr s;
    pub_read(c, 0, 1, &s);
    s = fr_mul(s, eq_corr(st, K));
    if (U) s = fix1(s);
    *out = s;
    return 0;
}
// the same over an integer tensor's own entries (no conversion to planes)
static int eq_weighted_sum_int(zkh_ctx* c, const zkh_tensor* t, const std::vector<Fr>& u, Fr* out) {
    int rc = 0;
    EqState st;
    if ((rc = eq_setup(c, u, st, false))) return rc;
    const uint32_t K = (uint32_t)u.size();
    {
        ProfScope ps(c, "eq_sum", (double)t->n * (t->kind == ZKH_KIND_I32 ? 4 : 8));
        Publish pb = make_pub(c, 1);
        launch_eq_sum_int(c->stream, t->kind, t->d, t->n, EqW{st.elo_d, st.ehi_d, K}, pb);
        if ((rc = wait_pub(c, pb.seq))) return rc;
    }
    Fr s;
    pub_read(c, 0, 1, &s);
    *out = fr_from_mont(fr_mul(s, eq_corr(st, K)));  // the int64 multiply's 2^256 removed
    return 0;
}
extern "C" int zkh_sum(zkh_ctx* c, const zkh_tensor* t, uint32_t out[8]) {
    if (!c || !t || !out) return fail(c, ZKH_EARG, "null argument");
    HIPCHK(c, hipSetDevice(c->device));
    int rc = 0;
    DevPlanes p;
    if ((rc = as_planes(c, t, SL_TMP0, &p))) return rc;
    Fr s = kZero;
    if (t->n) {
        Publish pb = make_pub(c, 1);
        launch_sum_planes(c->stream, p, t->n, pb);
        if ((rc = wait_pub(c, pb.seq))) return rc;
        pub_read(c, 0, 1, &s);
    }
    fr_store(s, out);
    return ZKH_OK;
}
extern "C" int zkh_prod_round(zkh_ctx* c, const zkh_tensor* a, const zkh_tensor* b, uint32_t out[24]) {
    if (!c || !a || !b || !out) return fail(c, ZKH_EARG, "null argument");
    if (a->kind != ZKH_KIND_FR || b->kind != ZKH_KIND_FR || a->n != b->n || a->n < 2 || (a->n & 1))
        return fail(c, ZKH_EARG, "prod_round needs two FR tensors of one even size");
    HIPCHK(c, hipSetDevice(c->device));
    Publish pb = make_pub(c, 1);
    launch_prod_round(c->stream, a->planes(), b->planes(), a->n / 2, pb);
    int rc;
    if ((rc = wait_pub(c, pb.seq))) return rc;
    Fr s[3];
    pub_read(c, 0, 3, s);
    // each sum carries 2^-256 (Montgomery products of plain values)
    for (int t = 0; t < 3; t++) fr_store(fr_mont_mul(s[t], kR2), out + 8 * t);
    return ZKH_OK;
}
extern "C" int zkh_calib_fr_mul(zkh_ctx* c, uint32_t iters, double* mul_per_s) {
    if (!c || !mul_per_s || !iters) return fail(c, ZKH_EARG, "calib_fr_mul: null argument or zero iterations");
    HIPCHK(c, hipSetDevice(c->device));
    const uint32_t blocks = 2048;
    int rc = 0;
    uint32_t* out = (uint32_t*)scratch_slot(c, SL_TMP6, (size_t)blocks * kFrMulPeakThreads * 4, &rc);
    if (rc) return rc;
    hipEvent_t a, b;
    HIPCHK(c, hipEventCreate(&a));
    if (hipEventCreate(&b) != hipSuccess) {
        (void)hipEventDestroy(a);
        return fail(c, ZKH_EDEV, "hipEventCreate failed");
    }
    launch_fr_mul_peak(c->stream, blocks, iters, out, a, b);
    hipError_t e = hipStreamSynchronize(c->stream);
    float ms = 0;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, a, b);
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    if (e != hipSuccess) return fail(c, ZKH_EDEV, "calib_fr_mul: %s", hipGetErrorString(e));
    *mul_per_s = (double)blocks * kFrMulPeakThreads * 4.0 * iters / (ms * 1e-3);
    return ZKH_OK;
}
extern "C" int zkh_fr_scalar(const uint32_t a[8], const uint32_t b[8], int op, uint32_t out[8]) {
    if (!a || !out || (op != 3 && !b) || op < 0 || op > 3) return ZKH_EARG;
    if (!fr_is_canonical(a) || (op != 3 && !fr_is_canonical(b))) return ZKH_EARG;
    const Fr x = fr_load(a);
    Fr r;
    switch (op) {
        case 0: r = fr_add(x, fr_load(b)); break;
        case 1: r = fr_sub(x, fr_load(b)); break;
        case 2: r = fr_mul(x, fr_load(b)); break;
        default: r = fr_inv(x); break;
    }
    fr_store(r, out);
    return ZKH_OK;
}
extern "C" int zkh_sha256(const void* data, size_t n, uint8_t out[32]) {
    if ((!data && n) || !out) return ZKH_EARG;
    Sha256 h;
    h.init();
    h.update(data, n);
    h.final(out);
    return ZKH_OK;
}
extern "C" int zkh_me(zkh_ctx* c, const zkh_tensor* t, const uint32_t* u, uint32_t k,
                      uint32_t out[8]) {
    if (!c || !t || !out || (!u && k)) return fail(c, ZKH_EARG, "null argument");
    // FrTensor::operator()(u) (fr-tensor.cu:437-442)
    if (k >= 32 || t->n <= ((1u << k) / 2) || t->n > (1u << k))
        return fail(c, ZKH_EARG, "Incompatible dimensions");
    if (!all_canonical(u, k)) return fail(c, ZKH_EARG, "non-canonical challenge");
    HIPCHK(c, hipSetDevice(c->device));
    int rc = 0;
    Fr s;
    if (t->kind != ZKH_KIND_FR && !t->weights) {  // integer entries read as such
        if ((rc = eq_weighted_sum_int(c, t, load_frs(u, k), &s))) return rc;
        fr_store(s, out);
        return ZKH_OK;
    }
    DevPlanes p;
    if ((rc = as_planes(c, t, SL_TMP0, &p))) return rc;
    if ((rc = eq_weighted_sum(c, p, nullptr, t->n, load_frs(u, k), &s))) return rc;
    fr_store(s, out);
    return ZKH_OK;
}
// zkh_me without device allocation: the same eq-weighted sum (eq tables Elo, Ehi from the
// factors of u, one reduction kernel publishing through the context's pinned words), with
// every device buffer in the static scratch.  Field-element tensors of up to 2^24 entries.
extern "C" int zkh_me_static(zkh_ctx* c, const zkh_tensor* t, const uint32_t* u, uint32_t k, uint32_t out[8]) {
    if (!c || !t || !out || (!u && k)) return fail(c, ZKH_EARG, "null argument");
    if (k >= 32 || t->n <= ((1u << k) / 2) || t->n > (1u << k))
        return fail(c, ZKH_EARG, "Incompatible dimensions");
    if (k > ZKH_STATIC_MAX_VARS)
        return fail(c, ZKH_EARG, "zkh_me_static: %u variables exceed its static scratch (at most %u)", k,
                    (unsigned)ZKH_STATIC_MAX_VARS);
    if (t->kind != ZKH_KIND_FR) return fail(c, ZKH_EARG, "zkh_me_static takes a field-element tensor");
    if (!all_canonical(u, k)) return fail(c, ZKH_EARG, "non-canonical challenge");
    HIPCHK(c, hipSetDevice(c->device));
    uint8_t* base = static_scratch(c->device);
    if (!base) return fail(c, ZKH_EDEV, "static scratch of device %d not resolved", c->device);
    // factors (1 - u_t, u_t) in Montgomery form for t < max(k, 10); positions >= k are (1, 0)
    const uint32_t kmax = std::max<uint32_t>(k, 10), khi = kmax - 10;
    StaticFacArg fac;
    for (uint32_t t2 = 0; t2 < kmax; t2++) {
        Fr a = fr_to_mont(kOne), b = kZero;
        if (t2 < k) {
            const Fr ut = fr_load(u + 8 * (size_t)t2);
            a = fr_to_mont(fr_sub(kOne, ut));
            b = fr_to_mont(ut);
        }
        fr_store(a, fac.w + 16 * t2);
        fr_store(b, fac.w + 16 * t2 + 8);
    }
    uint32_t* fac_d = (uint32_t*)(base + kStFac);
    uint32_t* elo = (uint32_t*)(base + kStElo);
    uint32_t* ehi = (uint32_t*)(base + kStEhi);
    uint32_t* lay = (uint32_t*)(base + kStLay);
    launch_static_setup(c->stream, fac, kmax * 16, fac_d, lay, 3);
    launch_eq_mont2(c->stream, fac_d, 10, 1024, elo, fac_d + 2 * 10 * 8, khi, 1u << khi, ehi);
    Publish pb = make_pub(c, 1);
    pb.part = (uint32_t*)(base + kStPart);  // launch_eq_sum uses at most 1024 blocks
    pb.layout = lay;
    launch_eq_sum(c->stream, t->planes(), nullptr, t->n, EqW{elo, ehi, k}, pb);
    int rc;
    if ((rc = wait_pub(c, pb.seq))) return rc;
    Fr s;
    pub_read(c, 0, 1, &s);  // the full-length weighting needs no correction
    fr_store(s, out);
    return ZKH_OK;
}
// eq table (Montgomery AoS) of u over n entries into a scratch slot
static int eq_table_mont(zkh_ctx* c, const std::vector<Fr>& u, uint32_t n, int slot, uint32_t** out) {
    int rc = 0;
    std::vector<uint32_t> fac;
    make_fac(u, 0, fac);
    uint32_t* fac_d = (uint32_t*)scratch_slot(c, SL_FAC, std::max<size_t>(fac.size() * 4, 32), &rc);
    if (rc) return rc;
    if (!fac.empty() && (rc = upload(c, fac_d, fac.data(), fac.size() * 4))) return rc;
    uint32_t* e = (uint32_t*)scratch_slot(c, slot, (size_t)std::max<uint32_t>(n, 1) * 32, &rc);
    if (rc) return rc;
    launch_eq_mont(c->stream, fac_d, (uint32_t)u.size(), n, e);
    *out = e;
    return 0;
}
static int partial_me_impl(zkh_ctx* c, const zkh_tensor* t, const std::vector<Fr>& u,
                           uint32_t cur_dim, uint32_t window, zkh_tensor** out) {
    uint32_t k = (uint32_t)u.size();
    // FrTensor::partial_me(u, cur_dim, window) checks (fr-tensor.cu:554-560)
    if (k >= 32 || cur_dim <= ((1u << k) >> 1) || cur_dim > (1u << k))
        return fail(c, ZKH_EARG, "partial_me: incompatible dimensions");
    if (!window || t->n % ((uint64_t)cur_dim * window) != 0)
        return fail(c, ZKH_EARG, "t.size %% (cur_dim * window) != 0");
    uint32_t O = t->n / (cur_dim * window);
    int rc = 0;
    uint32_t* E;
    if ((rc = eq_table_mont(c, u, cur_dim, SL_EB, &E))) return rc;
    zkh_tensor* o;
    if ((rc = tensor_alloc(c, ZKH_KIND_FR, O * window, &o))) return rc;
    if (t->kind == ZKH_KIND_FR) launch_partial_me_planes(c->stream, t->planes(), O, cur_dim, window, E, o->planes());
    else if (t->kind == ZKH_KIND_I64)
        launch_partial_me_i64(c->stream, (const int64_t*)t->d, O, cur_dim, window, E, o->planes());
    else {
        DevPlanes p;
        if (t->weights) {
            if ((rc = as_planes(c, t, SL_TMP0, &p))) {
                zkh_tensor_free(o);
                return rc;
            }
            launch_partial_me_planes(c->stream, p, O, cur_dim, window, E, o->planes());
        } else {
            launch_partial_me_i32(c->stream, (const int32_t*)t->d, O, cur_dim, window, E, o->planes());
        }
    }
    hipError_t e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        zkh_tensor_free(o);
        return fail(c, ZKH_EDEV, "partial_me: %s", hipGetErrorString(e));
    }
    *out = o;
    return 0;
}
extern "C" int zkh_partial_me(zkh_ctx* c, const zkh_tensor* t, const uint32_t* u, uint32_t k,
                              uint32_t cur_dim, uint32_t window, zkh_tensor** out) {
    if (!c || !t || !out || (!u && k)) return fail(c, ZKH_EARG, "null argument");
    if (!all_canonical(u, k)) return fail(c, ZKH_EARG, "non-canonical challenge");
    HIPCHK(c, hipSetDevice(c->device));
    return partial_me_impl(c, t, load_frs(u, k), cur_dim, window, out);
}
extern "C" int zkh_multi_dim_me(zkh_ctx* c, const zkh_tensor* t, const uint32_t* us,
                                const uint32_t* ks, const uint32_t* shape, uint32_t ndim,
                                uint32_t out[8]) {
    if (!c || !t || !out || (ndim && (!ks || !shape))) return fail(c, ZKH_EARG, "null argument");
    HIPCHK(c, hipSetDevice(c->device));
    if (ndim == 0) {  // (*this)(0) in the reference is element 0
        if (!t->n) return fail(c, ZKH_EARG, "empty tensor");
        return zkh_me(c, t, nullptr, 0, out);
    }
    size_t off = 0;
    std::vector<std::vector<Fr>> uv(ndim);
    for (uint32_t d = 0; d < ndim; d++) {
        if (ks[d] && !us) return fail(c, ZKH_EARG, "null challenges");
        if (ks[d] && !all_canonical(us + 8 * off, ks[d])) return fail(c, ZKH_EARG, "non-canonical challenge");
        uv[d] = load_frs(us + 8 * off, ks[d]);
        off += ks[d];
    }
    // bind the last dimension first (fr-tensor.cu:643-652)
    const zkh_tensor* cur = t;
    zkh_tensor* owned = nullptr;
    int rc = 0;
    for (uint32_t d = ndim - 1; d >= 1; d--) {
        zkh_tensor* nxt;
        rc = partial_me_impl(c, cur, uv[d], shape[d], 1, &nxt);
        if (owned) zkh_tensor_free(owned);
        if (rc) return rc;
        owned = nxt;
        cur = nxt;
    }
    uint32_t k0 = ks[0];
    std::vector<uint32_t> u0(8 * (size_t)k0);
    for (uint32_t i = 0; i < k0; i++) fr_store(uv[0][i], &u0[8 * (size_t)i]);
    rc = zkh_me(c, cur, u0.data(), k0, out);
    if (owned) zkh_tensor_free(owned);
    return rc;
}
extern "C" int zkh_eq_table(zkh_ctx* c, const uint32_t* u, uint32_t k, zkh_tensor** out) {
    if (!c || !out || (!u && k) || k > 30) return fail(c, ZKH_EARG, "bad arguments");
    if (!all_canonical(u, k)) return fail(c, ZKH_EARG, "non-canonical challenge");
    HIPCHK(c, hipSetDevice(c->device));
    int rc = 0;
    std::vector<uint32_t> fac;
    make_fac(load_frs(u, k), 0, fac);
    // E = Tlo (first min(k,10) variables, Montgomery) (x) Thi (the rest, plain)
    const uint32_t klo = k < 10 ? k : 10, khi = k - klo;
    uint32_t* tlo = (uint32_t*)scratch_slot(c, SL_EB, ((size_t)1 << klo) * 32, &rc);
    if (rc) return rc;
    uint32_t* thi = (uint32_t*)scratch_slot(c, SL_EO, ((size_t)1 << khi) * 32, &rc);
    if (rc) return rc;
    zkh_tensor* t;
    // the factors as launch arguments where they fit (no uploads ahead of the launches)
    if (k && fac.size() <= sizeof(FacArg) / 4) {
        FacArg fa;
        memcpy(fa.w, fac.data(), fac.size() * 4);
        if ((rc = tensor_alloc(c, ZKH_KIND_FR, 1u << k, &t))) return rc;
        if (launch_eq_mont2_ka(c->stream, fa, klo, 1u << klo, tlo, khi, 1u << khi, thi, true)) {
            launch_eq_outer(c->stream, tlo, thi, klo, 1u << k, t->planes());
            *out = t;
            return ZKH_OK;
        }
        zkh_tensor_free(t);
    }
    uint32_t* fac_d = (uint32_t*)scratch_slot(c, SL_FAC, std::max<size_t>(fac.size() * 4, 32), &rc);
    if (rc) return rc;
    if (k && (rc = upload(c, fac_d, fac.data(), fac.size() * 4))) return rc;
    EqTabDesc d[2] = {};
    d[0].fac = fac_d;
    d[0].out = tlo;
    d[0].K = klo;
    d[0].n = 1u << klo;
    d[0].blk_begin = 0;
    d[1].fac = fac_d + 16 * (size_t)klo;
    d[1].out = thi;
    d[1].K = khi;
    d[1].n = 1u << khi;
    d[1].blk_begin = (d[0].n + 255) / 256;
    d[1].plain = 1;
    EqTabDesc* d_dev = (EqTabDesc*)scratch_slot(c, SL_DESC, sizeof(d), &rc);
    if (rc) return rc;
    if ((rc = upload(c, d_dev, d, sizeof(d)))) return rc;
    if ((rc = tensor_alloc(c, ZKH_KIND_FR, 1u << k, &t))) return rc;
    launch_eq_mont_multi(c->stream, d_dev, 2, d[1].blk_begin + (d[1].n + 255) / 256);
    launch_eq_outer(c->stream, tlo, thi, klo, 1u << k, t->planes());
    HIPCHK(c, hipStreamSynchronize(c->stream));
    *out = t;
    return ZKH_OK;
}
extern "C" int zkh_fold(zkh_ctx* c, zkh_tensor* t, const uint32_t v[8]) {
    if (!c || !t || !v) return fail(c, ZKH_EARG, "null argument");
    if (t->kind != ZKH_KIND_FR || t->n < 2 || (t->n & 1)) return fail(c, ZKH_EARG, "fold needs an even FR tensor");
    if (!fr_is_canonical(v)) return fail(c, ZKH_EARG, "non-canonical challenge");
    HIPCHK(c, hipSetDevice(c->device));
    uint32_t vm[8];
    fr_store(fr_to_mont(fr_load(v)), vm);
    launch_fold(c->stream, Tab{t->planes(), t->planes()}, t->n / 2, vm);
    t->n /= 2;
    t->gen = next_gen();
    t->inv_of = 0;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return ZKH_OK;
}
// in-place operand view for the kernels that read int32 / int64 / FR sources directly
// (transposed matmul weights are converted to their logical layout first)
static int src_of(zkh_ctx* c, const zkh_tensor* t, int slot, Src* out) {
    if (t->kind == ZKH_KIND_FR) {
        *out = Src{0, t->d, t->cap};
        return 0;
    }
    if (t->weights) {
        DevPlanes p;
        int rc = as_planes(c, t, slot, &p);
        if (rc) return rc;
        *out = Src{0, p.base, p.cap};
        return 0;
    }
    *out = Src{t->kind == ZKH_KIND_I32 ? 1 : 2, t->d, 0};
    return 0;
}
extern "C" int zkh_axpy(zkh_ctx* c, const zkh_tensor* a, const uint32_t cc[8], const zkh_tensor* b,
                        zkh_tensor** out) {
    if (!c || !a || !b || !cc || !out) return fail(c, ZKH_EARG, "null argument");
    if (a->n != b->n) return fail(c, ZKH_EARG, "size mismatch");
    if (!fr_is_canonical(cc)) return fail(c, ZKH_EARG, "non-canonical scalar");
    HIPCHK(c, hipSetDevice(c->device));
    int rc = 0;
    Src sa, sb;
    if ((rc = src_of(c, a, SL_TMP0, &sa)) || (rc = src_of(c, b, SL_TMP1, &sb))) return rc;
    zkh_tensor* o;
    if ((rc = tensor_alloc(c, ZKH_KIND_FR, a->n, &o))) return rc;
    uint32_t cm[8];
    fr_store(fr_to_mont(fr_load(cc)), cm);
    if (a->n) launch_axpy(c->stream, sa, cc, cm, sb, a->n, o->planes());
    // queued only: later work on the context's stream is ordered behind it (a device error
    // surfaces at the next call that waits)
    if (const hipError_t e = hipGetLastError(); e != hipSuccess) {
        zkh_tensor_free(o);
        return fail(c, ZKH_EDEV, "axpy launch: %s", hipGetErrorString(e));
    }
    *out = o;
    return ZKH_OK;
}
extern "C" int zkh_hadamard(zkh_ctx* c, const zkh_tensor* a, const zkh_tensor* b, zkh_tensor** out) {
    if (!c || !a || !b || !out) return fail(c, ZKH_EARG, "null argument");
    if (a->n != b->n) return fail(c, ZKH_EARG, "size mismatch");
    HIPCHK(c, hipSetDevice(c->device));
    int rc = 0;
    zkh_tensor* o;
    if (a->kind == ZKH_KIND_I32 && b->kind == ZKH_KIND_I32 && !a->weights && !b->weights) {
        // two int32 tensors: the exact int64 products (8 bytes an entry where planes take 32)
        if ((rc = tensor_alloc(c, ZKH_KIND_I64, a->n, &o))) return rc;
        o->bits = std::min<uint32_t>(a->bits + b->bits, 63);  // |a b| < 2^(bits_a + bits_b), <= 2^62
        if (a->n) launch_hadamard_i64(c->stream, (const int32_t*)a->d, (const int32_t*)b->d, a->n, (int64_t*)o->d);
    } else {
        Src sa, sb;
        if ((rc = src_of(c, a, SL_TMP0, &sa)) || (rc = src_of(c, b, SL_TMP1, &sb))) return rc;
        if ((rc = tensor_alloc(c, ZKH_KIND_FR, a->n, &o))) return rc;
        if (a->n) launch_hadamard(c->stream, sa, sb, a->n, o->planes());
    }
    if (const hipError_t e = hipGetLastError(); e != hipSuccess) {  // queued only, as zkh_axpy
        zkh_tensor_free(o);
        return fail(c, ZKH_EDEV, "hadamard launch: %s", hipGetErrorString(e));
    }
    *out = o;
    return ZKH_OK;
}
extern "C" int zkh_pad(zkh_ctx* c, const zkh_tensor* t, const uint32_t* shape, uint32_t ndim,
                       const uint32_t pad_val[8], zkh_tensor** out) {
    if (!c || !t || !shape || !out || ndim == 0 || ndim > 8) return fail(c, ZKH_EARG, "bad arguments");
    if (pad_val && !fr_is_canonical(pad_val)) return fail(c, ZKH_EARG, "non-canonical pad value");
    uint64_t total = 1;
    uint32_t lgsum = 0;
    PadDims pd{};
    pd.nd = ndim;
    for (uint32_t d = 0; d < ndim; d++) {
        total = std::min<uint64_t>(total * shape[d], 1ull << 33);
        pd.shape[d] = shape[d];
        pd.lg[d] = ceil_log2(shape[d]);
        lgsum += pd.lg[d];
    }
    // FrTensor::pad checks (fr-tensor.cu:809-813)
    if (total != t->n) return fail(c, ZKH_EARG, "pad: cum_shape != size");
    if (lgsum >= 32) return fail(c, ZKH_EARG, "pad: too large");
    const uint64_t ptotal = 1ull << lgsum;
    HIPCHK(c, hipSetDevice(c->device));
    int rc = 0;
    DevPlanes p;
    if ((rc = as_planes(c, t, SL_TMP0, &p))) return rc;
    zkh_tensor* o;
    if ((rc = tensor_alloc(c, ZKH_KIND_FR, (uint32_t)ptotal, &o))) return rc;
    static const uint32_t zero[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    launch_pad(c->stream, p, pd, (uint32_t)ptotal, pad_val ? pad_val : zero, o->planes());
    hipError_t e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        zkh_tensor_free(o);
        return fail(c, ZKH_EDEV, "pad: %s", hipGetErrorString(e));
    }
    *out = o;
    return ZKH_OK;
}

// ---------------------------------------------------------------------------------------
// matmul sumcheck (zkob_fc.cu:259-440)
// ---------------------------------------------------------------------------------------
// Batched matmul sumchecks: all jobs share each launch (eq tables, eq-weighted
// reductions, every round) and one host synchronisation per round; transcripts stay
// independent, one per job.

static int mm_batch(zkh_ctx* c, zkh_mm_job* jobs, uint32_t nj);
extern "C" int zkh_mm_prove_batch(zkh_ctx* c, zkh_mm_job* jobs, uint32_t nj) {
    if (!c || (!jobs && nj)) return fail(c, ZKH_EARG, "null argument");
    int rc = 0;
    for (uint32_t at = 0; at < nj; at += ZKH_MAX_BATCH) {
        int r = mm_batch(c, jobs + at, std::min<uint32_t>(ZKH_MAX_BATCH, nj - at));
        if (r && !rc) rc = r;
    }
    return rc;
}
static int mm_batch(zkh_ctx* c, zkh_mm_job* jobs, uint32_t nj) {
    int first_rc = 0;
    const double t_in = now_us();
    auto stamp = [&](const char* what) {
        if (trace_on()) fprintf(stderr, "[zkh] mm %-28s %8.1f us\n", what, now_us() - t_in);
    };
    for (uint32_t j = 0; j < nj; j++) {
        zkh_mm_job& J = jobs[j];
        J.status = ZKH_OK;
        const zkh_tensor *X = J.X, *W = J.W, *Y = J.Y;
        const char* why = nullptr;
        if (!J.transcript || !X || !W || !Y) why = "null argument";
        else if (!J.B || !J.IN || !J.OUT) why = "zero dimension";
        else if ((X->kind != ZKH_KIND_I32 && X->kind != ZKH_KIND_FR) ||
                 (W->kind != ZKH_KIND_I32 && W->kind != ZKH_KIND_FR))
            why = "mm_prove takes int32 or field-element X and W";
        else if ((uint64_t)X->n != (uint64_t)J.B * J.IN || (uint64_t)W->n != (uint64_t)J.IN * J.OUT ||
                 (uint64_t)Y->n != (uint64_t)J.B * J.OUT)
            why = "input dims";
        else if (W->weights && (W->w_in != J.IN || W->w_out != J.OUT)) why = "weights dims";
        else if ((Y->kind != ZKH_KIND_FR && Y->bits > 62) || J.IN > (1u << 24) || J.B > (1u << 24) ||
                 J.OUT > (1u << 24))
            why = "integer range / size";
        if (why) {
            J.status = ZKH_EARG;
            if (!first_rc) first_rc = fail(c, ZKH_EARG, "job %u: %s", j, why);
        }
    }
    if (first_rc || !nj) return first_rc;
    HIPCHK(c, hipSetDevice(c->device));
    int rc = 0;
    struct Job {
        uint32_t lb, lo, L, INp;
        std::vector<Fr> ub, uo, xs;
        Fr claim, cur, xm;  // xm: the last challenge in Montgomery form
        Fr cx, cw;          // the folded terminals (kept for the convention cross-check)
        Fr SEb, SEo;        // sum of the eq table entries over the first B / OUT indices
        size_t eb_off, eo_off, fac_b, fac_o;  // element offsets
        size_t red_off;                       // planes offset (entries) of a; b follows
        uint32_t dot_blocks, dot_slot;        // claim partials in pinned memory
        bool live;
    };
    std::vector<Job> J(nj);
    size_t eq_total = 0, fac_total = 0, red_total = 0, wt_total = 0;
    for (uint32_t j = 0; j < nj; j++) {
        Job& q = J[j];
        const zkh_mm_job& in = jobs[j];
        q.lb = ceil_log2(in.B);
        q.lo = ceil_log2(in.OUT);
        q.L = ceil_log2(in.IN);
        q.INp = 1u << q.L;
        q.ub.resize(q.lb);
        q.uo.resize(q.lo);
        q.fac_b = fac_total;
        fac_total += 2 * (size_t)q.lb;
        q.fac_o = fac_total;
        fac_total += 2 * (size_t)q.lo;
        q.eb_off = eq_total;
        eq_total += in.B;
        q.eo_off = eq_total;
        eq_total += in.OUT;
        q.red_off = red_total;
        red_total += 2 * (size_t)q.INp;
        if (in.W->kind == ZKH_KIND_I32 && !in.W->weights) wt_total += in.W->n;
        q.live = true;
    }
    // device areas
    // u_batch, u_output draws (zkob_fc.cu:259-262), eq factors and eq prefix sums, per job
    // on the host workers
    std::vector<uint32_t> fac(std::max<size_t>(fac_total, 1) * 8, 0);
    pool_for(c->workers, (int)std::min<uint32_t>(nj, (uint32_t)host_threads()), nj, [&](uint32_t j) {
        Job& q = J[j];
        for (auto& x : q.ub) x = tr_challenge(jobs[j].transcript);
        for (auto& x : q.uo) x = tr_challenge(jobs[j].transcript);
        std::vector<uint32_t> fb, fo;
        make_fac(q.ub, 0, fb);
        make_fac(q.uo, 0, fo);
        std::copy(fb.begin(), fb.end(), fac.begin() + q.fac_b * 8);
        std::copy(fo.begin(), fo.end(), fac.begin() + q.fac_o * 8);
        q.SEb = eq_prefix_sum(q.ub, jobs[j].B);
        q.SEo = eq_prefix_sum(q.uo, jobs[j].OUT);
    });
    // one device area and one upload for the eq factors and every stage's descriptors: the
    // factors first, the descriptors (at most 2 eq tables and 3 reductions per job) after
    const size_t fac_bytes = (fac.size() * 4 + 255) & ~(size_t)255;
    const size_t desc_cap = (size_t)nj * (2 * sizeof(EqTabDesc) + 3 * (sizeof(EqDotDesc) + sizeof(SumChunksDesc) +
                                                                      sizeof(EqDotFrDesc))) + 256;
    uint8_t* area_d = (uint8_t*)scratch_slot(c, SL_DESC, fac_bytes + desc_cap, &rc);
    if (rc) return rc;
    uint32_t* fac_d = (uint32_t*)area_d;
    uint32_t* eq_d = (uint32_t*)scratch_slot(c, SL_EB, eq_total * 32, &rc);
    if (rc) return rc;
    DevPlanes red = scratch_planes(c, SL_TMP0, (uint32_t)red_total, &rc);
    if (rc) return rc;
    int32_t* wt_d = wt_total ? (int32_t*)scratch_slot(c, SL_TMP5, wt_total * 4, &rc) : nullptr;
    if (rc) return rc;

    stamp("challenges");
    // 1) eq tables (Montgomery AoS)
    std::vector<EqTabDesc> eqd;
    uint32_t eq_blocks = 0;
    for (uint32_t j = 0; j < nj; j++) {
        const Job& q = J[j];
        for (int t = 0; t < 2; t++) {
            EqTabDesc d{};
            d.fac = fac_d + 8 * (t ? q.fac_o : q.fac_b);
            d.out = eq_d + 8 * (t ? q.eo_off : q.eb_off);
            d.K = t ? q.lo : q.lb;
            d.n = t ? jobs[j].OUT : jobs[j].B;
            d.blk_begin = eq_blocks;
            eq_blocks += (d.n + 255) / 256;
            eqd.push_back(d);
        }
    }
    // 2) eq-weighted reductions: Y by eb (then dotted with eo -> claim), X by eb, W^T by eo
    struct Red {
        EqDotDesc d;   // integer operands (d.partial, d.N also describe field operands)
        EqDotFrDesc f;  // field-element operands
        int is64, wide, fr;
        uint32_t nch, Npad, job, what;  // what: 0 Y, 1 X, 2 W
        Fr corr;
    };
    std::vector<Red> reds;
    size_t part_total = 0;
    size_t wt_off = 0;
    for (uint32_t j = 0; j < nj; j++) {
        const zkh_mm_job& in = jobs[j];
        const Job& q = J[j];
        const Fr SEb = q.SEb, SEo = q.SEo;
        const int32_t* WT = (const int32_t*)in.W->d;
        if (in.W->kind == ZKH_KIND_I32 && !in.W->weights) {
            launch_transpose_i32(c->stream, (const int32_t*)in.W->d, in.IN, in.OUT, wt_d + wt_off);
            WT = wt_d + wt_off;
            wt_off += in.W->n;
        }
        for (uint32_t what = 0; what < 3; what++) {
            Red r{};
            const zkh_tensor* T = what == 0 ? in.Y : what == 1 ? in.X : in.W;
            if (T->kind == ZKH_KIND_FR) {
                // X (B x IN) and Y (B x OUT) reduce over their rows by eq(u_batch); W (IN x
                // OUT, row-major) over its columns by eq(u_output), one wave per row
                r.fr = 1;
                r.f.lo = T->planes().lo();
                r.f.hi = T->planes().hi();
                r.f.E = eq_d + 8 * (what == 2 ? q.eo_off : q.eb_off);
                r.f.rowmode = what == 2;
                r.f.K = what == 2 ? in.OUT : in.B;
                r.f.N = what == 0 ? in.OUT : in.IN;
                uint32_t nch = 1;
                if (!r.f.rowmode) {
                    // about 2^16 (column, chunk) cells, 32..512 rows each: enough blocks for
                    // the chip while a cell's reduction stays small next to its rows
                    const uint32_t ncell = std::max<uint32_t>(1, 65536 / r.f.N);
                    r.f.kchunk = std::min<uint32_t>(std::max<uint32_t>((r.f.K + ncell - 1) / ncell, 32), 512);
                    nch = (r.f.K + r.f.kchunk - 1) / r.f.kchunk;
                }
                r.d.N = r.f.N;
                r.d.K = r.f.K;
                r.nch = nch;
                r.Npad = what == 0 ? r.f.N : q.INp;
                r.job = j;
                r.what = what;
                r.corr = kZero;
                r.d.partial = (uint32_t*)(uintptr_t)(part_total * 32);  // offset, fixed below
                part_total += (size_t)nch * r.f.N;
                reds.push_back(r);
                continue;
            }
            const void* M = what == 0 ? in.Y->d : what == 1 ? in.X->d : (const void*)WT;
            uint32_t K = what == 2 ? in.OUT : in.B;
            uint32_t N = what == 0 ? in.OUT : in.IN;
            uint32_t bits = what == 0 ? in.Y->bits : what == 1 ? in.X->bits : in.W->bits;
            r.is64 = what == 0 && in.Y->kind == ZKH_KIND_I64;
            // piece layout (see launch_eqdot_multi): narrow = one 20-bit piece for int32 /
            // two 22-bit pieces for int64; chunks hold at most 2048 / 512 rows accordingly
            r.wide = r.is64 ? bits + 1 > 44 : bits + 1 > 20;
            const uint32_t maxrows = (!r.is64 && !r.wide) ? 2048 : 512;
            // row chunks: up to 2^17 (column, chunk) cells per reduction spread it over the
            // CUs; at least 128 rows (64 for 8-byte elements) per chunk keep the per-cell
            // field reduction and the partials' traffic small next to the streamed rows
            const uint32_t ncell = std::max<uint32_t>(1, (131072 + N - 1) / N);
            const uint32_t minrows = r.is64 ? 64 : 128;
            const uint32_t kchunk = std::min<uint32_t>(std::max<uint32_t>((K + ncell - 1) / ncell, minrows), maxrows);
            const uint32_t nch = (K + kchunk - 1) / kchunk;
            r.d.M = M;
            r.d.E = eq_d + 8 * (what == 2 ? q.eo_off : q.eb_off);
            r.d.K = K;
            r.d.N = N;
            r.d.kchunk = kchunk;
            r.d.bits = bits;
            r.d.variant = r.is64 ? 1 : 0;
            r.nch = nch;
            r.Npad = what == 0 ? N : q.INp;
            r.job = j;
            r.what = what;
            Fr two_b = kOne;
            for (uint32_t b = 0; b < bits; b++) two_b = fr_add(two_b, two_b);
            r.corr = fr_mul(two_b, what == 2 ? SEo : SEb);
            r.d.partial = (uint32_t*)(uintptr_t)(part_total * 32);  // offset, fixed below
            part_total += (size_t)nch * N;
            reds.push_back(r);
        }
    }
    uint32_t* part_d = (uint32_t*)scratch_slot(c, SL_TMP6, part_total * 32, &rc);
    if (rc) return rc;
    for (auto& r : reds) {
        r.d.partial = part_d + (uintptr_t)r.d.partial / 4;
        r.f.partial = r.d.partial;
    }
    // field-element reductions: one launch for all of them
    std::vector<EqDotFrDesc> frds;
    uint32_t fr_blocks = 0;
    for (auto& r : reds) {
        if (!r.fr) continue;
        EqDotFrDesc d = r.f;
        d.blk_begin = fr_blocks;
        // 256-thread blocks: four rows per block in row mode, 256 columns per block otherwise
        fr_blocks += r.f.rowmode ? (r.f.N + 3) / 4 : ((r.f.N + 255) / 256) * r.nch;
        frds.push_back(d);
    }
    // group the integer reductions by piece layout -> one launch per group (normally one)
    std::vector<EqDotDesc> dots;
    struct Grp {
        int wide;
        uint32_t first, count, blocks;
    };
    std::vector<Grp> groups;
    for (int wide = 0; wide < 2; wide++) {
        Grp g{wide, (uint32_t)dots.size(), 0, 0};
        for (auto& r : reds) {
            if (r.fr || r.wide != wide) continue;
            EqDotDesc d = r.d;
            d.blk_begin = g.blocks;
            g.blocks += ((r.d.N + 255) / 256) * r.nch;
            dots.push_back(d);
            g.count++;
        }
        if (g.count) groups.push_back(g);
    }
    // 3) chunk sums (X, W -> planes; Y -> dot with eo into pinned claim partials)
    std::vector<SumChunksDesc> sums;
    uint32_t sum_blocks = 0, claim_slots = 0;
    for (auto& r : reds) {
        SumChunksDesc d{};
        const Job& q = J[r.job];
        d.partial = r.d.partial;
        d.nch = r.nch;
        d.N = r.d.N;
        d.Npad = r.Npad;
        d.blk_begin = sum_blocks;
        fr_store(r.corr, d.corr.v);
        uint32_t nb = (r.Npad + 63) / 64;  // k_sum_chunks_multi: 64 columns per block
        if (r.what == 0) {
            d.E = eq_d + 8 * q.eo_off;
            d.dot = (uint32_t*)(uintptr_t)claim_slots;  // slot index, fixed below
            J[r.job].dot_slot = claim_slots;
            J[r.job].dot_blocks = nb;
            claim_slots += nb;
        } else {
            size_t off = q.red_off + (r.what == 1 ? 0 : q.INp);
            d.out_lo = red.lo() + 4 * off;
            d.out_hi = red.hi() + 4 * off;
        }
        sum_blocks += nb;
        sums.push_back(d);
    }
    // pinned host layout: claim partials | round partials (per job, max blocks) | terminals
    uint32_t max_rb = 0;
    for (auto& q : J) max_rb = std::max(max_rb, (q.INp / 2 + 255) / 256);
    size_t pin_claim = 0, pin_round = (size_t)claim_slots * 8,
           pin_term = pin_round + (size_t)nj * std::max<uint32_t>(max_rb, 1) * 24;
    if ((rc = ensure_pinned(c, (pin_term + (size_t)nj * 16) * 4))) return rc;
    uint32_t* pin = c->pinned;
    for (auto& d : sums)
        if (d.E) d.dot = pin + pin_claim + 8 * (uintptr_t)d.dot;
    // eq factors and descriptors -> device in one upload
    uint8_t* desc_d = area_d + fac_bytes;
    size_t o_eq = 0, o_dot = o_eq + eqd.size() * sizeof(EqTabDesc);
    size_t o_sum = o_dot + dots.size() * sizeof(EqDotDesc);
    size_t o_fr = o_sum + sums.size() * sizeof(SumChunksDesc);
    size_t o_end = o_fr + frds.size() * sizeof(EqDotFrDesc);
    if (o_end > desc_cap) return fail(c, ZKH_EDEV, "descriptor area overflow (%zu > %zu)", o_end, desc_cap);
    std::vector<uint8_t> blob(fac_bytes + o_end, 0);
    memcpy(blob.data(), fac.data(), fac.size() * 4);
    memcpy(blob.data() + fac_bytes + o_eq, eqd.data(), eqd.size() * sizeof(EqTabDesc));
    memcpy(blob.data() + fac_bytes + o_dot, dots.data(), dots.size() * sizeof(EqDotDesc));
    memcpy(blob.data() + fac_bytes + o_sum, sums.data(), sums.size() * sizeof(SumChunksDesc));
    memcpy(blob.data() + fac_bytes + o_fr, frds.data(), frds.size() * sizeof(EqDotFrDesc));
    if ((rc = upload(c, area_d, blob.data(), blob.size()))) return rc;
    stamp("factors + descriptors uploaded");
    {
        ProfScope ps(c, "eq_tables", (double)eq_total * 32, true);
        launch_eq_mont_multi(c->stream, (const EqTabDesc*)(desc_d + o_eq), (uint32_t)eqd.size(), eq_blocks,
                             ps.start(), ps.stop());
    }
    double red_bytes = 0, fr_bytes = 0;  // algorithmic: every stored entry of X, W and Y read once
    for (auto& r : reds) {
        if (r.fr) fr_bytes += (double)r.d.K * r.d.N * 32;
        else red_bytes += (double)r.d.K * r.d.N * (r.is64 ? 8 : 4);
    }
    if (!frds.empty()) {
        ProfScope ps(c, "eqdot_fr", fr_bytes, true);
        launch_eqdot_fr_multi(c->stream, (const EqDotFrDesc*)(desc_d + o_fr), (uint32_t)frds.size(), fr_blocks,
                              ps.start(), ps.stop());
    }
    if (!groups.empty()) {
        ProfScope ps(c, "eqdot", red_bytes, true);
        for (size_t gi = 0; gi < groups.size(); gi++) {
            const Grp& g = groups[gi];
            launch_eqdot_multi(c->stream, g.wide, (const EqDotDesc*)(desc_d + o_dot) + g.first, g.count, g.blocks,
                               gi == 0 ? ps.start() : nullptr, gi + 1 == groups.size() ? ps.stop() : nullptr);
        }
    }
    {
        double b = 0;
        for (auto& r : reds) b += (double)r.nch * r.d.N * 32 + (double)r.Npad * 32;
        ProfScope ps(c, "sum_chunks", b, true);
        launch_sum_chunks_multi(c->stream, (const SumChunksDesc*)(desc_d + o_sum), (uint32_t)sums.size(),
                                sum_blocks, ps.start(), ps.stop());
    }
    for (auto& q : J) q.xs.resize(q.L);
    // claim = <Y(u_batch, .), eq(u_output, .)> from the pinned block partials
    auto absorb_claim = [&](uint32_t j) {
        Job& q = J[j];
        Fr s = kZero;
        for (uint32_t b = 0; b < q.dot_blocks; b++)
            s = fr_add(s, fr_load(pin + pin_claim + 8 * (size_t)(q.dot_slot + b)));
        q.claim = q.cur = s;
        tr_absorb_fr(jobs[j].transcript, "claim", s);
    };
    // one round from its three sums c0 = sum a0b0, q1 = sum a1b1, c2 = sum da*db
    // (zkob_fc.cu:294-332): p(0) = c0, p(1) = q1, p(2) = c0 + 2c1 + 4c2
    // The running claim becomes p(x) = c0 + x(c1 + x c2), with x in Montgomery form so each
    // product is one Montgomery multiplication; q.xm keeps it for the device folds.
    auto round_step = [&](uint32_t j, uint32_t r, const Fr& c0, const Fr& q1, const Fr& c2) -> bool {
        Job& q = J[j];
        const Fr c1 = fr_sub(fr_sub(q1, c0), c2);
        const Fr c1x2 = fr_add(c1, c1), c2x2 = fr_add(c2, c2);
        Fr p[3] = {c0, q1, fr_add(fr_add(c0, c1x2), fr_add(c2x2, c2x2))};
        if (!fr_eq(q.cur, fr_add(p[0], p[1]))) {
            q.live = false;
            jobs[j].status = ZKH_EROUND;
            std::lock_guard<std::mutex> lk(c->err_mu);
            if (!first_rc)
                first_rc = fail(c, ZKH_EROUND, "job %u: prover sumcheck round inconsistency (witness bug) at round %u",
                                j, r);
            return false;
        }
        uint8_t* tr = jobs[j].transcript;
        tr_absorb_fr(tr, "p0", p[0]);
        tr_absorb_fr(tr, "p1", p[1]);
        tr_absorb_fr(tr, "p2", p[2]);
        const Fr x = tr_challenge(tr);
        q.xs[r] = x;
        q.xm = fr_to_mont(x);
        if (jobs[j].ev_out)
            for (int k = 0; k < 3; k++) fr_store(p[k], jobs[j].ev_out + 8 * (3 * r + k));
        q.cur = fr_add(c0, fr_mont_mul(q.xm, fr_add(c1, fr_mont_mul(q.xm, c2))));
        return true;
    };
    // terminal check claim == X(u_batch, u_input) * W(u_input, u_output), outputs
    auto finish = [&](uint32_t j, const Fr& cx, const Fr& cw) {
        Job& q = J[j];
        zkh_mm_job& in = jobs[j];
        q.cx = cx;
        q.cw = cw;
        if (!fr_eq(q.cur, fr_mul(cx, cw))) {
            q.live = false;
            in.status = ZKH_EROUND;
            std::lock_guard<std::mutex> lk(c->err_mu);
            if (!first_rc) first_rc = fail(c, ZKH_EROUND, "job %u: terminal product mismatch (witness bug)", j);
            return;
        }
        tr_absorb_fr(in.transcript, "claim_X", cx);
        tr_absorb_fr(in.transcript, "claim_W", cw);
        if (in.claims_out) {
            fr_store(q.claim, in.claims_out);
            fr_store(cx, in.claims_out + 8);
            fr_store(cw, in.claims_out + 16);
        }
        if (in.u_batch_out)
            for (uint32_t i = 0; i < q.lb; i++) fr_store(q.ub[i], in.u_batch_out + 8 * i);
        if (in.u_output_out)
            for (uint32_t i = 0; i < q.lo; i++) fr_store(q.uo[i], in.u_output_out + 8 * i);
        if (in.u_input_out)
            for (uint32_t i = 0; i < q.L; i++) fr_store(q.xs[q.L - 1 - i], in.u_input_out + 8 * i);
    };

    // zkob_fc.cu:337-345 with ZKH_XCHECK: claim_X = X(u_batch, u_input), claim_W =
    // W(u_input, u_output) by multi_dim_me against the folded terminals, after every round
    // (the persistent loop no longer holds the stream)
    auto xcheck = [&]() -> int {
        if (!xcheck_on()) return first_rc;
        for (uint32_t j = 0; j < nj; j++) {
            Job& q = J[j];
            if (jobs[j].status != ZKH_OK) continue;
            std::vector<uint32_t> ux, uw;
            auto put = [](std::vector<uint32_t>& v, const std::vector<Fr>& a) {
                for (const Fr& x : a) {
                    uint32_t w[8];
                    fr_store(x, w);
                    v.insert(v.end(), w, w + 8);
                }
            };
            std::vector<Fr> ui(q.xs.rbegin(), q.xs.rend());
            put(ux, q.ub);
            put(ux, ui);
            put(uw, ui);
            put(uw, q.uo);
            const uint32_t kx[2] = {q.lb, q.L}, kw[2] = {q.L, q.lo};
            const uint32_t sx[2] = {jobs[j].B, jobs[j].IN}, sw[2] = {jobs[j].IN, jobs[j].OUT};
            uint32_t ex[8], ew[8];
            int r2 = zkh_multi_dim_me(c, jobs[j].X, ux.data(), kx, sx, 2, ex);
            if (!r2) r2 = zkh_multi_dim_me(c, jobs[j].W, uw.data(), kw, sw, 2, ew);
            if (!r2 && (!fr_eq(fr_load(ex), q.cx) || !fr_eq(fr_load(ew), q.cw)))
                r2 = fail(c, ZKH_EROUND, "job %u: folded terminals != multi_dim_me claims (convention bug)", j);
            if (r2) {
                jobs[j].status = r2;
                if (!first_rc) first_rc = r2;
            }
        }
        return first_rc;
    };

    // 4) rounds.  Tables of up to ZKH_PLS_MAX * 128 entries: one persistent launch per group
    // of jobs (<= 256 blocks), tables in LDS, one host round trip per round and job.
    uint32_t max_inp = 0;
    for (auto& q : J) max_inp = std::max(max_inp, q.INp);
    if (max_inp <= ZKH_PLS_MAX * 128 && !getenv("ZKH_NO_PERSIST")) {
        std::vector<uint32_t> lgnb(nj), slot_off(nj), cmd_off(nj), grp_of(nj);
        std::vector<ZkipPersist> groups_p;
        std::vector<uint32_t> grp_blocks;
        size_t words = ZKH_PSLOT;  // word 0: error flag
        for (uint32_t j = 0; j < nj; j++) {
            const uint32_t INp = J[j].INp;
            // ZKH_PLS_MAX entries per block (up to 128 blocks)
            lgnb[j] = INp > ZKH_PLS_MAX ? ceil_log2(INp / ZKH_PLS_MAX) : 0;
            const uint32_t nb = 1u << lgnb[j];
            slot_off[j] = (uint32_t)words;
            words += (size_t)nb * ZKH_PSLOT;
            cmd_off[j] = (uint32_t)words;
            words += ZKH_PSLOT;
            if (groups_p.empty() || grp_blocks.back() + nb > 256 || groups_p.back().nd == ZKH_MAX_BATCH) {
                groups_p.emplace_back();
                memset(&groups_p.back(), 0, sizeof(ZkipPersist));
                grp_blocks.push_back(0);
            }
            grp_of[j] = (uint32_t)groups_p.size() - 1;
        }
        if ((rc = ensure_ps(c, words))) return rc;
        uint32_t* ps = c->ps_host;
        for (uint32_t j = 0; j < nj; j++) {
            const uint32_t nb = 1u << lgnb[j];
            for (uint32_t b = 0; b < nb; b++) memset(ps + slot_off[j] + b * ZKH_PSLOT, 0, ZKH_PSLOT * 4);
            memset(ps + cmd_off[j], 0, ZKH_PSLOT * 4);
        }
        ps[0] = 0;
        const uint64_t deadline_ticks = c->clock_khz * 1000 * 20;  // 20 s without a command
        for (uint32_t j = 0; j < nj; j++) {
            ZkipPersist& P = groups_p[grp_of[j]];
            ZkipPJob& d = P.d[P.nd++];
            d.a_lo = red.lo() + 4 * J[j].red_off;
            d.a_hi = red.hi() + 4 * J[j].red_off;
            d.b_lo = red.lo() + 4 * (J[j].red_off + J[j].INp);
            d.b_hi = red.hi() + 4 * (J[j].red_off + J[j].INp);
            d.out = ps + slot_off[j];
            d.cmd = ps + cmd_off[j];
            d.n = J[j].INp;
            d.lgnb = lgnb[j];
            d.blk_begin = grp_blocks[grp_of[j]];
            grp_blocks[grp_of[j]] += 1u << lgnb[j];
            P.err = ps;
            P.deadline = deadline_ticks;
            P.ls_max = std::max(P.ls_max, J[j].INp >> lgnb[j]);
        }
        // a job's command: nw data words (the challenge or the four fold weights, Montgomery
        // form), then the seqs of its quads; without data, seq (ZKH_QUIT) goes to every quad
        // a block may poll
        auto send_cmd = [&](uint32_t j, uint32_t seq, const uint32_t* w, uint32_t nw) {
            uint32_t* cmd = ps + cmd_off[j];
            for (uint32_t i = 0; i < nw; i++) __atomic_store_n(cmd + zkh_quad_word(i), w[i], __ATOMIC_RELAXED);
            const uint32_t nq = zkh_quad_count(w ? nw : 32);
            for (uint32_t qd = 0; qd < nq; qd++) __atomic_store_n(cmd + 4 * qd, seq, __ATOMIC_RELEASE);
        };
        auto quit_all = [&]() {
            for (uint32_t j = 0; j < nj; j++) send_cmd(j, ZKH_QUIT, nullptr, 0);
            (void)hipStreamSynchronize(c->stream);
        };
        double pbytes = 0;
        for (auto& q : J) pbytes += 2.0 * q.INp * 32;
        {
            ProfScope psc(c, "zkip_rounds", pbytes);
            for (size_t g = 0; g < groups_p.size(); g++) {
                hipError_t e = launch_zkip_persist(c->stream, groups_p[g], grp_blocks[g]);
                if (e != hipSuccess) {
                    quit_all();
                    return fail(c, ZKH_EDEV, "persistent round launch: %s", hipGetErrorString(e));
                }
            }
        }
        stamp("all launched");
        // host side: each worker thread advances its jobs (j = t mod T) whenever all of a
        // job's blocks have published
        std::vector<uint32_t> R(nj);
        for (uint32_t j = 0; j < nj; j++) R[j] = J[j].L - lgnb[j];
        const double t_start = now_us();
        // words of the message that follows `done` local rounds: two rounds' sums, one
        // round's sums, or the folded entries after the last local round
        auto msg_words = [&](uint32_t j, uint32_t done) {
            const uint32_t rem = R[j] - done;
            return rem >= 2 ? (uint32_t)ZKH_MSG_PAIR : rem == 1 ? (uint32_t)ZKH_MSG_ONE : (uint32_t)ZKH_MSG_FINAL;
        };
        // all blocks of job j have published message seq of nw words
        auto ready = [&](uint32_t j, uint32_t seq, uint32_t nw) {
            const uint32_t nb = 1u << lgnb[j];
            const uint32_t nq = zkh_quad_count(nw);
            for (uint32_t b = 0; b < nb; b++)
                for (uint32_t qd = 0; qd < nq; qd++)
                    if (__atomic_load_n(ps + slot_off[j] + b * ZKH_PSLOT + 4 * qd, __ATOMIC_ACQUIRE) != seq)
                        return false;
            return true;
        };
        auto slot_fr = [&](const uint32_t* sl, uint32_t k) {  // Fr k of a block's message
            uint32_t v[8];
            for (uint32_t i = 0; i < 8; i++) v[i] = sl[zkh_quad_word(8 * k + i)];
            return fr_load(v);
        };
        const int T = (int)std::min<uint32_t>(nj, (uint32_t)host_threads());
        const bool tracing = trace_on();
        std::vector<std::vector<uint64_t>> tr_gpu(tracing ? nj : 0);
        std::vector<std::vector<double>> tr_host(tracing ? nj : 0);
        // Any worker serves any job whose message is complete: a job is taken with a
        // try-lock, so a worker that the OS preempts holds up at most the message it is
        // serving, and the others keep every other job moving.
        std::vector<uint32_t> rnd(nj, 0), msg(nj, 0);  // local rounds done, messages answered
        // What a worker touches outside a job's lock lives on the heap, held by each worker
        // by value: a worker that the OS deschedules may return after this frame has ended.
        // A worker touches this frame only inside serve() and the stall check, holding
        // busy[j] for an unfinished job; this frame ends only after every job is finished
        // or abandoned and it has taken every job's lock.
        struct Loop {
            std::unique_ptr<std::atomic<uint8_t>[]> busy;
            std::vector<uint8_t> fin;  // written and read under busy[j]
            std::atomic<uint32_t> open_jobs;
            std::atomic<int> abort_why{0};  // 1 device error, 2 kernel ended early, 3 no progress, 4 stream idle
            std::atomic<int> dev_err{0};
            std::atomic<bool> closed{false};
            std::vector<double> tr_thr;  // each thread's entry / exit / longest stream query (tracing)
            Loop(uint32_t nj, int T, bool tracing)
                : busy(new std::atomic<uint8_t>[nj]), fin(nj, 0), open_jobs(nj), tr_thr(tracing ? 3 * T : 0) {
                for (uint32_t j = 0; j < nj; j++) busy[j].store(0, std::memory_order_relaxed);
            }
        };
        const auto lp = std::make_shared<Loop>(nj, T, tracing);
        // serve job j's pending message if complete (caller holds busy[j]); false if not ready
        auto serve = [&](uint32_t j, std::vector<Fr>& ta, std::vector<Fr>& tb) -> bool {
            const uint32_t nb = 1u << lgnb[j];
            const uint32_t* sl = ps + slot_off[j];
            const uint32_t nw = msg_words(j, rnd[j]);
            if (!ready(j, msg[j] + 1, nw)) return false;
            if (tracing) tr_host[j].push_back(now_us());
            // a block has run, so every earlier launch (the claim partials) has completed
            if (msg[j] == 0) absorb_claim(j);
            const uint32_t r = rnd[j];
            auto stop_job = [&]() {
                send_cmd(j, ZKH_QUIT, nullptr, 0);
                lp->fin[j] = 1;
                lp->open_jobs.fetch_sub(1, std::memory_order_acq_rel);
            };
            if (nw == ZKH_MSG_PAIR) {  // rounds r and r + 1
                Fr sm[9];
                for (int k = 0; k < 9; k++) sm[k] = kZero;
                for (uint32_t b = 0; b < nb; b++)
                    for (int k = 0; k < 9; k++) sm[k] = fr_add(sm[k], slot_fr(sl + b * ZKH_PSLOT, k));
                // (the sums carry 2^-256; fix1 removes it from the combinations)
                bool ok = round_step(j, r, fix1(fr_add(sm[0], sm[3])), fix1(fr_add(sm[1], sm[4])),
                                     fix1(fr_add(sm[2], sm[5])));
                const Fr x0m = J[j].xm;
                if (ok) {
                    // round r + 1's sum k at x: A + x (B + x C) with A = sm[3k],
                    // C = sm[3k + 2] and B = sm[3k + 1] - A - C
                    Fr nx[3];
                    for (int k = 0; k < 3; k++) {
                        const Fr A = sm[3 * k], C = sm[3 * k + 2];
                        const Fr Bc = fr_sub(fr_sub(sm[3 * k + 1], A), C);
                        nx[k] = fix1(fr_add(A, fr_mont_mul(x0m, fr_add(Bc, fr_mont_mul(x0m, C)))));
                    }
                    ok = round_step(j, r + 1, nx[0], nx[1], nx[2]);
                }
                if (!ok) {
                    stop_job();
                    return true;
                }
                // fold weights in Montgomery form from x0 R, x1 R: (1 - x) R = R - x R
                const Fr x1m = J[j].xm;
                const Fr u0m = fr_sub(fr_one_m(), x0m), u1m = fr_sub(fr_one_m(), x1m);
                const Fr w[4] = {fr_mont_mul(u0m, u1m), fr_mont_mul(x0m, u1m), fr_mont_mul(u0m, x1m),
                                 fr_mont_mul(x0m, x1m)};
                uint32_t cw[32];
                for (int k = 0; k < 4; k++) fr_store(w[k], cw + 8 * k);
                rnd[j] += 2;
                msg[j]++;
                send_cmd(j, msg[j], cw, 32);
                if (tracing) tr_host[j].push_back(now_us());
                return true;
            }
            if (nw == ZKH_MSG_ONE) {
                Fr s3[3] = {kZero, kZero, kZero};
                for (uint32_t b = 0; b < nb; b++)
                    for (int k = 0; k < 3; k++) s3[k] = fr_add(s3[k], slot_fr(sl + b * ZKH_PSLOT, k));
                if (!round_step(j, r, fix1(s3[0]), fix1(s3[1]), fix1(s3[2]))) {
                    stop_job();
                    return true;
                }
                uint32_t xm[8];
                fr_store(J[j].xm, xm);
                rnd[j]++;
                msg[j]++;
                send_cmd(j, msg[j], xm, 8);
                if (tracing) tr_host[j].push_back(now_us());
                return true;
            }
            if (tracing) {  // block 0's per-message clock stamps are complete once it has exited
                for (uint32_t m2 = 1; m2 <= msg[j] + 1 && m2 < 14; m2++) {
                    const uint32_t* st = sl + ZKH_PSTAMP;
                    tr_gpu[j].push_back(st[4 + 2 * m2] - st[3 + 2 * m2]);
                    tr_gpu[j].push_back(m2 <= msg[j] ? st[5 + 2 * m2] - st[4 + 2 * m2] : 0);
                }
            }
            // the blocks' folded entries: the remaining lgnb rounds on the host
            ta.resize(nb);
            tb.resize(nb);
            for (uint32_t b = 0; b < nb; b++) {
                ta[b] = slot_fr(sl + b * ZKH_PSLOT, 0);
                tb[b] = slot_fr(sl + b * ZKH_PSLOT, 1);
            }
            bool ok = true;
            for (uint32_t rr = R[j], m = nb; m > 1 && ok; rr++, m >>= 1) {
                const uint32_t h = m >> 1;
                Fr c0 = kZero, q1 = kZero, c2 = kZero;  // each x 2^-256
                for (uint32_t i = 0; i < h; i++) {
                    c0 = fr_add(c0, fr_mont_mul(ta[i], tb[i]));
                    q1 = fr_add(q1, fr_mont_mul(ta[i + h], tb[i + h]));
                    c2 = fr_add(c2, fr_mont_mul(fr_sub(ta[i + h], ta[i]), fr_sub(tb[i + h], tb[i])));
                }
                ok = round_step(j, rr, fix1(c0), fix1(q1), fix1(c2));
                const Fr xm = J[j].xm;
                for (uint32_t i = 0; ok && i < h; i++) {
                    ta[i] = fr_add(ta[i], fr_mont_mul(xm, fr_sub(ta[i + h], ta[i])));
                    tb[i] = fr_add(tb[i], fr_mont_mul(xm, fr_sub(tb[i + h], tb[i])));
                }
            }
            if (ok) finish(j, ta[0], tb[0]);
            lp->fin[j] = 1;
            lp->open_jobs.fetch_sub(1, std::memory_order_acq_rel);
            return true;
        };
        // captures by value but for what is used under a job's lock
        auto worker = [lp, c, ps, nj, tracing, &serve, &ready, &msg_words, &msg, &rnd](int t) {
            Loop& L = *lp;
            struct Stamp {
                double* at;
                ~Stamp() {
                    if (at) *at = now_us();
                }
            } on_exit{tracing ? &L.tr_thr[3 * t + 1] : nullptr};
            if (tracing) L.tr_thr[3 * t] = now_us();
            std::vector<Fr> ta, tb;
            double t_prog = now_us();
            for (uint64_t spins = 1;
                 !L.closed.load(std::memory_order_acquire) && L.open_jobs.load(std::memory_order_acquire); spins++) {
                bool prog = false;
                for (uint32_t k = 0; k < nj; k++) {
                    const uint32_t j = (k + (uint32_t)t) % nj;  // each worker starts at its own job
                    if (L.busy[j].load(std::memory_order_relaxed) || L.busy[j].exchange(1, std::memory_order_acquire))
                        continue;
                    if (!L.fin[j] && serve(j, ta, tb)) prog = true;
                    L.busy[j].store(0, std::memory_order_release);
                }
                if (prog) {
                    t_prog = now_us();
                    continue;
                }
                spin_pause(spins);
                if ((spins & 0x3FFF) == 0) {
                    if (L.abort_why.load(std::memory_order_relaxed) || L.closed.load(std::memory_order_acquire)) return;
                    const double q0 = tracing ? now_us() : 0.0;
                    hipError_t e = hipStreamQuery(c->stream);
                    if (tracing) L.tr_thr[3 * t + 2] = std::max(L.tr_thr[3 * t + 2], now_us() - q0);
                    int why = 0;
                    if (e != hipSuccess && e != hipErrorNotReady) {
                        L.dev_err.store((int)e);
                        why = 1;
                    } else if (__atomic_load_n(ps, __ATOMIC_ACQUIRE)) {
                        why = 2;
                    } else if (e == hipSuccess) {  // the kernel has ended: whatever is missing never comes
                        bool all = true;
                        for (uint32_t j = 0; j < nj; j++) {
                            if (L.busy[j].exchange(1, std::memory_order_acquire)) continue;  // being served
                            all = all && (L.fin[j] || ready(j, msg[j] + 1, msg_words(j, rnd[j])));
                            L.busy[j].store(0, std::memory_order_release);
                        }
                        if (!all) why = 4;
                    } else if (now_us() - t_prog > 30e6) {
                        why = 3;
                    }
                    if (why) {
                        int z = 0;
                        L.abort_why.compare_exchange_strong(z, why);
                        return;
                    }
                }
            }
        };
        c->workers.run(T, worker);
        // the calling thread's share has ended: every job is finished, or the loop is
        // abandoned; close it and wait out any worker still inside a job's work
        lp->closed.store(true, std::memory_order_release);
        for (uint32_t j = 0; j < nj; j++)
            for (uint64_t k = 1; lp->busy[j].exchange(1, std::memory_order_acquire); k++) spin_pause(k);
        if (int why = lp->abort_why.load()) {
            quit_all();
            if (why == 1)
                return fail(c, ZKH_EDEV, "persistent round loop: %s", hipGetErrorString((hipError_t)lp->dev_err.load()));
            return fail(c, ZKH_EDEV, "persistent round loop stopped (%s; clock %llu kHz)",
                        why == 2 ? "a block timed out" : why == 4 ? "stream idle before the last round" : "no progress",
                        (unsigned long long)c->clock_khz);
        }
        c->ring_off = 0;  // every launch before the round loop has completed
        stamp("round loops done");
        if (tracing) {
            fprintf(stderr, "[zkh] mm persistent rounds: %.1f us (%d host threads; entry/exit us", now_us() - t_start, T);
            for (int t = 0; t < T; t++) {  // a worker still running (or not started) shows 0
                const double* th = &lp->tr_thr[3 * t];
                fprintf(stderr, " %.1f/%.1f (longest stream query %.1f)", th[0] ? th[0] - t_start : 0.0,
                        th[1] ? th[1] - t_start : 0.0, th[2]);
            }
            fprintf(stderr, ")\n");
            const double tick_us = 1000.0 / (double)c->clock_khz;
            // per message: block 0's compute (device clock: previous command received -> sums
            // published) and round trip (sums published -> command received), and the host's
            // work (sums seen -> command sent)
            for (uint32_t j = 0; j < nj; j++) {
                const auto& g = tr_gpu[j];
                const auto& h = tr_host[j];
                fprintf(stderr, "[zkh]   job %u (n=%u, %u blocks, %u local rounds): compute/trip/host us", j, J[j].INp,
                        1u << lgnb[j], R[j]);
                for (size_t m2 = 0; 2 * m2 + 1 < g.size(); m2++)
                    fprintf(stderr, " %.1f/%.1f/%.1f", m2 ? (double)(uint32_t)g[2 * m2] * tick_us : 0.0,
                            (double)(uint32_t)g[2 * m2 + 1] * tick_us, 2 * m2 + 1 < h.size() ? h[2 * m2 + 1] - h[2 * m2] : 0.0);
                fprintf(stderr, "\n");
            }
        }
        if (c->prof) prof_resolve_ready(c);
        return xcheck();
    }

    // tables beyond the LDS loop: one launch and one synchronisation per round for all jobs
    HIPCHK(c, hipStreamSynchronize(c->stream));
    c->ring_off = 0;
    if (c->prof) prof_resolve(c);
    for (uint32_t j = 0; j < nj; j++) absorb_claim(j);
    uint32_t maxL = 0;
    for (auto& q : J) maxL = std::max(maxL, q.L);
    std::vector<ZkipDesc> zk(nj);
    for (uint32_t j = 0; j < nj; j++) {
        zk[j] = ZkipDesc{};
        zk[j].a_lo = red.lo() + 4 * J[j].red_off;
        zk[j].a_hi = red.hi() + 4 * J[j].red_off;
        zk[j].b_lo = red.lo() + 4 * (J[j].red_off + J[j].INp);
        zk[j].b_hi = red.hi() + 4 * (J[j].red_off + J[j].INp);
    }
    for (uint32_t r = 0; r < maxL; r++) {
        std::vector<ZkipDesc> act;
        std::vector<uint32_t> who;
        uint32_t blocks = 0;
        double bytes = 0;
        for (uint32_t j = 0; j < nj; j++) {
            Job& q = J[j];
            if (!q.live || r >= q.L) continue;
            ZkipDesc d = zk[j];
            d.n = q.INp >> r;
            d.fold = r > 0;
            d.blk_begin = blocks;
            blocks += (d.n / 2 + 255) / 256;
            bytes += (r > 0 ? 3.0 * d.n : (double)d.n) * 64;
            act.push_back(d);
            who.push_back(j);
        }
        if (act.empty()) break;
        if ((size_t)blocks * 3 > c->pub_part_cap) {
            HIPCHK(c, hipStreamSynchronize(c->stream));
            (void)hipFree(c->pub_part);
            c->pub_part = nullptr;
            HIPCHK(c, hipMalloc((void**)&c->pub_part, (size_t)blocks * 3 * 32));
            c->pub_part_cap = (size_t)blocks * 3;
        }
        ZkipBatch bt;
        memset(&bt, 0, sizeof(bt));
        for (size_t a = 0; a < act.size(); a++) bt.d[a] = act[a];
        bt.nd = (uint32_t)act.size();
        Publish pb = make_pub(c, bt.nd);
        {
            ProfScope ps(c, "zkip_round", bytes);
            launch_zkip_round_multi(c->stream, bt, blocks, pb);
        }
        if ((rc = wait_pub(c, pb.seq))) return rc;
        for (size_t a = 0; a < act.size(); a++) {
            uint32_t j = who[a];
            Fr s3[3];
            pub_read(c, (uint32_t)a, 3, s3);
            if (round_step(j, r, fix1(s3[0]), fix1(s3[1]), fix1(s3[2]))) fr_store(J[j].xm, zk[j].vm.v);
        }
    }
    // 5) final binds and terminals (written to pinned memory by the kernel)
    std::vector<ZkipDesc> fin;
    std::vector<uint32_t> fwho;
    for (uint32_t j = 0; j < nj; j++) {
        if (!J[j].live) continue;
        ZkipDesc d = zk[j];
        d.fold = J[j].L > 0;
        d.partial = pin + pin_term + (size_t)j * 16;
        fin.push_back(d);
        fwho.push_back(j);
    }
    if (!fin.empty()) {
        ZkipBatch bt;
        memset(&bt, 0, sizeof(bt));
        for (size_t a = 0; a < fin.size(); a++) bt.d[a] = fin[a];
        bt.nd = (uint32_t)fin.size();
        launch_fold_last_multi(c->stream, bt);
        HIPCHK(c, hipStreamSynchronize(c->stream));
        c->ring_off = 0;
        if (c->prof) prof_resolve(c);
    }
    for (uint32_t j : fwho)
        finish(j, fr_load(pin + pin_term + (size_t)j * 16), fr_load(pin + pin_term + (size_t)j * 16 + 8));
    return xcheck();
}

extern "C" int zkh_mm_prove(zkh_ctx* c, uint8_t tr[32], const zkh_tensor* X, const zkh_tensor* W,
                            const zkh_tensor* Y, uint32_t B, uint32_t IN, uint32_t OUT,
                            uint32_t* ev_out, uint32_t* claims_out, uint32_t* ub_out,
                            uint32_t* uo_out, uint32_t* ui_out) {
    zkh_mm_job j{X, W, Y, B, IN, OUT, tr, ev_out, claims_out, ub_out, uo_out, ui_out, 0};
    return zkh_mm_prove_batch(c, &j, 1);
}

// ---------------------------------------------------------------------------------------
// logUp
// ---------------------------------------------------------------------------------------
extern "C" int zkh_lu_range_table(zkh_ctx* c, int32_t low, uint32_t len, uint32_t N, zkh_tensor** out) {
    if (!c || !out || !len || N < len) return fail(c, ZKH_EARG, "bad range table arguments");
    HIPCHK(c, hipSetDevice(c->device));
    // int32 entries (4 bytes where field planes take 32): the table's values are 32-bit
    zkh_tensor* t;
    int rc = tensor_alloc(c, ZKH_KIND_I32, N, &t);
    if (rc) return rc;
    {
        const int64_t last = (int64_t)low + (int64_t)len - 1;
        const uint64_t lo_abs = low < 0 ? (uint64_t)(-(int64_t)low) : (uint64_t)low;
        t->bits = last > INT32_MAX ? 32 : bits_for(std::max<uint64_t>(lo_abs, last < 0 ? (uint64_t)-last : (uint64_t)last));
    }
    launch_range_table_i32(c->stream, low, len, N, (int32_t*)t->d);
    hipError_t e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        zkh_tensor_free(t);
        return fail(c, ZKH_EDEV, "range table: %s", hipGetErrorString(e));
    }
    t->range_gen = t->gen;
    t->range_low = low;
    t->range_len = len;
    *out = t;
    return ZKH_OK;
}
static int lu_counts(zkh_ctx* c, const zkh_tensor* S, int32_t low, uint32_t N, uint32_t** counts_out,
                     DevFlag* bad_out) {
    int rc = 0;
    uint32_t* counts = (uint32_t*)scratch_slot(c, SL_TMP5, (size_t)(N + 1) * 4, &rc);
    if (rc) return rc;
    uint32_t* bad = counts + N;
    HIPCHK(c, hipMemsetAsync(counts, 0, (size_t)(N + 1) * 4, c->stream));
    if (S->kind == ZKH_KIND_I32) {
        launch_lu_count_i32(c->stream, (const int32_t*)S->d, S->n, low, N, counts, bad);
    } else {
        DevPlanes p;
        if ((rc = as_planes(c, S, SL_TMP0, &p))) return rc;
        uint32_t lowl[8];
        fr_store(fr_from_i64(low), lowl);
        launch_lu_count_planes(c->stream, p, S->n, lowl, N, counts, bad);
    }
    *counts_out = counts;
    *bad_out = DevFlag{bad, 0};
    return 0;
}
// the tensor for the multiplicities of S against N entries: int32 counts (a 4-byte entry
// where field planes take 32) when the LDS histogram counts them and no count can reach
// 2^31, field elements otherwise
static int mult_alloc(zkh_ctx* c, const zkh_tensor* S, uint32_t N, zkh_tensor** m) {
    const bool i32 = N <= ZKH_HIST_MAX_BUCKETS * ZKH_HIST_BINS && S->n < (1u << 31);
    int rc = tensor_alloc(c, i32 ? ZKH_KIND_I32 : ZKH_KIND_FR, N, m);
    if (!rc && i32) (*m)->bits = bits_for(S->n);  // every count is at most |S|
    return rc;
}
// multiplicities m (N entries, from mult_alloc) of the witness S against a table of N entries
// at low: LDS histograms for N <= 2^24 (launch_hist), global atomics beyond.  Queues the work
// only; *bad_out (a device condition) is set when a witness lies outside the table (check_bad).
static int lu_multiplicities(zkh_ctx* c, const zkh_tensor* S, int32_t low, uint32_t N, zkh_tensor* mt,
                             DevFlag* bad_out) {
    int rc = 0;
    const DevPlanes m = mt->kind == ZKH_KIND_FR ? mt->planes() : DevPlanes{};
    int32_t* m32 = mt->kind == ZKH_KIND_I32 ? (int32_t*)mt->d : nullptr;
    if (N > ZKH_HIST_MAX_BUCKETS * ZKH_HIST_BINS) {
        if (m32) return fail(c, ZKH_EARG, "int32 multiplicities beyond the histogram's table size");
        uint32_t* counts;
        if ((rc = lu_counts(c, S, low, N, &counts, bad_out))) return rc;
        launch_counts_to_planes(c->stream, counts, N, m);
        return 0;
    }
    HistArgs a{};
    if (S->kind == ZKH_KIND_I32) {
        a.S = Src{1, S->d, 0};
    } else {
        DevPlanes p;
        if ((rc = as_planes(c, S, SL_TMP0, &p))) return rc;
        a.S = Src{0, p.base, p.cap};
    }
    a.n = S->n;
    a.low = low;
    fr_store(fr_from_i64(low), a.low_fr);
    a.N = N;
    const DevFlag bad = dev_flag(c, kFlagHist);
    void* hs = scratch_slot(c, SL_TMP5, hist_scratch_bytes(S->n, N), &rc);
    if (rc) return rc;
    a.bad = bad.d;
    a.tag = bad.tag;
    {
        ProfScope ps(c, "lu_hist", (double)S->n * (S->kind == ZKH_KIND_I32 ? 4 : 32) + (double)N * 32);
        launch_hist(c->stream, a, hs, m, m32);
    }
    *bad_out = bad;
    return 0;
}
// waits for the queued work and fails when the multiplicity pass flagged a witness outside
// the table
static int check_bad(zkh_ctx* c, const DevFlag& bad) {
    uint32_t hb = 0;
    int rc = settle(c, bad.d, &hb);
    if (rc) return rc;
    if (bad.hit(hb)) return fail(c, ZKH_EARG, "lookup witness outside the table");
    return 0;
}
extern "C" int zkh_lu_prep(zkh_ctx* c, const zkh_tensor* S, int32_t low, uint32_t N, zkh_tensor** m_out) {
    if (!c || !S || !m_out || !N) return fail(c, ZKH_EARG, "bad arguments");
    HIPCHK(c, hipSetDevice(c->device));
    zkh_tensor* m;
    int rc;
    if ((rc = mult_alloc(c, S, N, &m))) return rc;
    DevFlag bad{};
    if ((rc = lu_multiplicities(c, S, low, N, m, &bad)) || (rc = check_bad(c, bad))) {
        zkh_tensor_free(m);
        return rc;
    }
    *m_out = m;
    return ZKH_OK;
}
extern "C" int zkh_lu_mapping(zkh_ctx* c, const zkh_tensor* S_in, int32_t low, const zkh_tensor* mapped,
                              zkh_tensor** S_out, zkh_tensor** m_out) {
    if (!c || !S_in || !mapped || !S_out || !m_out || !mapped->n)
        return fail(c, ZKH_EARG, "bad arguments");
    HIPCHK(c, hipSetDevice(c->device));
    uint32_t N = mapped->n;
    zkh_tensor *m, *so;
    int rc;
    if ((rc = mult_alloc(c, S_in, N, &m))) return rc;
    // the mapping is queued behind the multiplicities (its kernels bound-check the index) and
    // one completion wait then checks the witness range
    DevFlag bad{};
    if ((rc = lu_multiplicities(c, S_in, low, N, m, &bad))) {
        zkh_tensor_free(m);
        return rc;
    }
    // an int32 mapped table maps into int32 entries (4 bytes where field planes take 32)
    const bool out_i32 = mapped->kind == ZKH_KIND_I32 && !mapped->weights;
    if ((rc = tensor_alloc(c, out_i32 ? ZKH_KIND_I32 : ZKH_KIND_FR, S_in->n, &so))) {
        zkh_tensor_free(m);
        return rc;
    }
    if (out_i32) {
        so->bits = mapped->bits;  // the entries are mapped's
        Src ss;
        rc = src_of(c, S_in, SL_TMP0, &ss);
        uint32_t lowl[8];
        fr_store(fr_from_i64(low), lowl);
        if (!rc)
            launch_lu_map_to_i32(c->stream, ss, S_in->n, lowl, (const int32_t*)mapped->d, N, (int32_t*)so->d);
    } else if (S_in->kind == ZKH_KIND_I32) {
        Src ms;
        rc = src_of(c, mapped, SL_TMP1, &ms);
        if (!rc) launch_lu_map_i32(c->stream, (const int32_t*)S_in->d, S_in->n, low, ms, N, so->planes());
    } else {
        DevPlanes p, mp;
        rc = as_planes(c, mapped, SL_TMP1, &mp);
        if (!rc) rc = as_planes(c, S_in, SL_TMP0, &p);
        uint32_t lowl[8];
        fr_store(fr_from_i64(low), lowl);
        if (!rc) launch_lu_map_planes(c->stream, p, S_in->n, lowl, mp, so->planes());
    }
    if (!rc) rc = check_bad(c, bad);
    if (rc) {
        zkh_tensor_free(m);
        zkh_tensor_free(so);
        return rc;
    }
    so->map_G = S_in->gen;
    so->map_mapped = mapped->gen;
    so->map_low = low;
    *S_out = so;
    *m_out = m;
    return ZKH_OK;
}
// waits for the queued work; *hf = 1 (a witness outside the table) | 2 (a witness that is not
// the table's entry at its index) from the gather's two condition words
static int gather_flags(zkh_ctx* c, const DevFlag& f, uint32_t* hf) {
    uint32_t w[2] = {0, 0};
    const int rc = settle(c, f.d, w, 2);
    *hf = (f.hit(w[0]) ? 1u : 0u) | (f.hit(w[1]) ? 2u : 0u);
    return rc;
}
// A = 1/(S + beta) into planes A (n entries)
// any_zero (when given): whether some S[i] + beta was zero (its inverse entry is 0)
static int batch_inverse(zkh_ctx* c, DevPlanes S, uint32_t n, const Fr& beta, DevPlanes A,
                         bool* any_zero = nullptr, uint32_t* aos = nullptr) {
    int rc = 0;
    uint32_t nb = inv_blocks(n);
    uint32_t* others = (uint32_t*)scratch_slot(c, SL_TMP4, (size_t)nb * 256 * 32, &rc);
    if (rc) return rc;
    uint32_t* bp = (uint32_t*)scratch_slot(c, SL_SMALL, (size_t)nb * 64 + 64, &rc);
    if (rc) return rc;
    uint32_t* others_blk = bp + 8 * (size_t)nb;
    uint32_t bl[8];
    fr_store(beta, bl);
    const DevFlag zf = dev_flag(c, kFlagInvZero);
    Publish pb = make_pub(c, 1);
    {
        ProfScope ps(c, "inv_pass1", (double)n * 64 + (double)nb * 256 * 32);
        launch_inv_pass1(c->stream, S, n, bl, A, others, bp, zf.d, zf.tag);
        launch_inv_blocks(c->stream, bp, nb, others_blk, pb, zf.d, zf.tag);
    }
    // pass 2 is queued now behind a relay that hands it 1/G, so that its launch overlaps the
    // block pass and the host's inversion
    RelayGuard relay{c};
    relay.pending = relay_enqueue(c);
    {
        ProfScope ps(c, "inv_pass2", (double)n * (aos ? 128 : 96) + (double)nb * 256 * 32);
        launch_inv_pass2(c->stream, S, n, bl, A, others, others_blk, nullptr, c->relay_vm, aos);
    }
    if ((rc = wait_pub(c, pb.seq))) return rc;
    // the grand product G (never zero) -> its plain inverse, once, on the host
    Fr G;
    pub_read(c, 0, 1, &G);
    if (any_zero) *any_zero = __atomic_load_n(c->pub_host + 8, __ATOMIC_ACQUIRE) != 0;
    uint32_t inv_g[8];
    fr_store(fr_inv(G), inv_g);
    relay_send(c, relay.pending, inv_g);
    relay.pending = 0;
    return 0;
}
extern "C" int zkh_lu_inverse(zkh_ctx* c, const zkh_tensor* S, const uint32_t beta[8], zkh_tensor** A_out) {
    if (!c || !S || !beta || !A_out) return fail(c, ZKH_EARG, "null argument");
    if (!fr_is_canonical(beta)) return fail(c, ZKH_EARG, "non-canonical beta");
    HIPCHK(c, hipSetDevice(c->device));
    int rc = 0;
    DevPlanes p;
    if ((rc = as_planes(c, S, SL_TMP0, &p))) return rc;
    zkh_tensor* A;
    if ((rc = tensor_alloc(c, ZKH_KIND_FR, S->n, &A))) return rc;
    bool zero = false;
    if ((S->n && (rc = batch_inverse(c, p, S->n, fr_load(beta), A->planes(), &zero))) || (rc = settle(c))) {
        zkh_tensor_free(A);
        return rc;
    }
    A->inv_of = S->gen;
    memcpy(A->inv_beta, beta, 32);
    A->inv_nz = !zero;
    *A_out = A;
    return ZKH_OK;
}
// Entries j < the returned length of the range table T are the true integers low + j, so
// T[j] == G iff G - low is the integer j below it (the gathers then read G alone).  The
// table's entries are int32 sums that wrap past 2^31 - 1 (tlookup.cu:376), so the length
// stops at the last entry that does not wrap; 0 when T is not a known range table at low.
static uint32_t range_shortcut_len(const zkh_tensor* T, int32_t low) {
    if (T->range_gen != T->gen || T->range_low != low) return 0;
    const int64_t fit = (int64_t)INT32_MAX - (int64_t)low + 1;  // entries low .. INT32_MAX
    return (uint32_t)std::min<int64_t>((int64_t)T->range_len, fit);
}
extern "C" int zkh_lu_range_inverse(zkh_ctx* c, const zkh_tensor* S, int32_t low, const zkh_tensor* T,
                                    const uint32_t beta[8], zkh_tensor** A_out) {
    if (!c || !S || !T || !beta || !A_out) return fail(c, ZKH_EARG, "null argument");
    const uint32_t D = S->n, N = T->n;
    if (!N) return fail(c, ZKH_EARG, "empty table");
    if (!fr_is_canonical(beta)) return fail(c, ZKH_EARG, "non-canonical beta");
    HIPCHK(c, hipSetDevice(c->device));
    int rc = 0;
    Src ss, st;
    DevPlanes Tp;
    if ((rc = src_of(c, S, SL_TMP0, &ss)) || (rc = src_of(c, T, SL_TMP1, &st)) || (rc = as_planes(c, T, SL_TMP2, &Tp)))
        return rc;
    zkh_tensor *A = nullptr, *Binv = nullptr;
    auto drop = [&](int code) {
        for (zkh_tensor* t : {A, Binv})
            if (t) zkh_tensor_free(t);
        return code;
    };
    if ((rc = tensor_alloc(c, ZKH_KIND_FR, D, &A)) || (rc = tensor_alloc(c, ZKH_KIND_FR, N, &Binv))) return drop(rc);
    // the table's inverse (tlookup.cu:50-62 over T, as zkh_lu_prove takes it), then A read off it
    bool tzero = false, szero = false;
    if ((rc = batch_inverse(c, Tp, N, fr_load(beta), Binv->planes(), &tzero))) return drop(rc);
    const DevFlag flags = dev_flag(c, kFlagGather);
    uint32_t hf = 0;
    if (D) {
        ProfScope ps(c, "lu_range_gather", (double)D * (32 + 32 + 32));
        uint32_t lowl[8];
        fr_store(fr_from_i64(low), lowl);
        const uint32_t tlen = range_shortcut_len(T, low);
        launch_lu_range_gather(c->stream, ss, D, lowl, st, tlen, N, Binv->planes(), A->planes(), flags.d, flags.tag);
    }
    if ((rc = gather_flags(c, flags, &hf))) return drop(rc);
    // a witness outside the table or not the table's entry at its index: the direct batched
    // inversion of S (zkob_rescale.cu:121-123), as zkh_lu_inverse
    if (hf) {
        DevPlanes Sp;
        if ((rc = as_planes(c, S, SL_TMP0, &Sp)) ||
            (rc = batch_inverse(c, Sp, D, fr_load(beta), A->planes(), &szero)) || (rc = settle(c)))
            return drop(rc);
    }
    A->inv_of = S->gen;
    memcpy(A->inv_beta, beta, 32);
    // A is the table inverse's entries (no zero there: none in A) or S's own inverse
    A->inv_nz = hf ? !szero : !tzero;
    Binv->inv_nz = !tzero;
    if (c->lu_tinv) zkh_tensor_free(c->lu_tinv);
    c->lu_tinv = Binv;
    c->lu_tinv_of = T->gen;
    memcpy(c->lu_tinv_beta, beta, 32);
    *A_out = A;
    return ZKH_OK;
}
extern "C" int zkh_lu_tuple_inverse(zkh_ctx* c, const zkh_tensor* G, int32_t low, const zkh_tensor* T,
                                    const zkh_tensor* mapped, const zkh_tensor* S, const uint32_t r[8],
                                    const uint32_t beta[8], zkh_tensor** comb_out, zkh_tensor** Tcomb_out,
                                    zkh_tensor** A_out) {
    if (!c || !G || !T || !mapped || !r || !beta || !comb_out || !Tcomb_out || !A_out)
        return fail(c, ZKH_EARG, "null argument");
    const uint32_t D = G->n, N = T->n;
    if (!N || mapped->n != N) return fail(c, ZKH_EARG, "T and mapped differ in size or are empty");
    if (S && (S->n != D || S->map_G != G->gen || S->map_mapped != mapped->gen || S->map_low != low))
        return fail(c, ZKH_EARG, "S is not zkh_lu_mapping's output for this G, low and mapped");
    if (!fr_is_canonical(r) || !fr_is_canonical(beta)) return fail(c, ZKH_EARG, "non-canonical r or beta");
    HIPCHK(c, hipSetDevice(c->device));
    int rc = 0;
    Src sg, st, sm, ss{};
    if ((rc = src_of(c, G, SL_TMP0, &sg)) || (rc = src_of(c, T, SL_TMP1, &st)) || (rc = src_of(c, mapped, SL_TMP2, &sm)) ||
        (S && (rc = src_of(c, S, SL_TMP3, &ss))))
        return rc;
    zkh_tensor *comb = nullptr, *Tcomb = nullptr, *A = nullptr, *Binv = nullptr;
    auto drop = [&](int code) {
        for (zkh_tensor* t : {comb, Tcomb, A, Binv})
            if (t) zkh_tensor_free(t);
        return code;
    };
    if ((rc = tensor_alloc(c, ZKH_KIND_FR, D, &comb)) || (rc = tensor_alloc(c, ZKH_KIND_FR, N, &Tcomb)) ||
        (rc = tensor_alloc(c, ZKH_KIND_FR, D, &A)) || (rc = tensor_alloc(c, ZKH_KIND_FR, N, &Binv)))
        return drop(rc);
    uint32_t rm[8];
    fr_store(fr_to_mont(fr_load(r)), rm);
    // T_comb = T + r mapped (zkob_glu.cu:156) and its inverse (zkob_glu.cu:168-170)
    launch_axpy(c->stream, st, r, rm, sm, N, Tcomb->planes());
    bool tzero = false, czero = false;
    // the table inverse also as AoS for the gather's random reads (a table larger than the
    // caches: one line per read instead of one per plane)
    uint32_t* binv_aos = D ? (uint32_t*)scratch_slot(c, SL_TMP6, (size_t)N * 32, &rc) : nullptr;
    if (rc) return drop(rc);
    if ((rc = batch_inverse(c, Tcomb->planes(), N, fr_load(beta), Binv->planes(), &tzero, binv_aos)))
        return drop(rc);
    const DevFlag flags = dev_flag(c, kFlagGather);
    uint32_t hf = 0;
    if (D) {
        ProfScope ps(c, "lu_tuple_gather", (double)D * (4 + 4 + 4 + 32 + 32 + 32));
        // comb from the mapping's S when the caller has it (read in order), else mapped[j]
        uint32_t lowl[8];
        fr_store(fr_from_i64(low), lowl);
        // a range table at this low: T[j] == G[i] iff G[i] - low is j < len, read from G alone
        const uint32_t tlen = range_shortcut_len(T, low);
        launch_lu_tuple_gather(c->stream, sg, D, lowl, st, tlen, S ? ss : sm, S != nullptr, N, r, rm, Binv->planes(),
                               binv_aos, comb->planes(), A->planes(), flags.d, flags.tag);
    }
    if ((rc = gather_flags(c, flags, &hf))) return drop(rc);
    if (hf & 1u) return drop(fail(c, ZKH_EARG, "lookup witness outside the table"));
    // an entry whose G is not the table's at its index (comb is then no table entry): A by
    // the direct batched inversion of comb (zkob_glu.cu:158-160)
    if ((hf & 2u) && ((rc = batch_inverse(c, comb->planes(), D, fr_load(beta), A->planes(), &czero)) ||
                      (rc = settle(c))))
        return drop(rc);
    A->inv_of = comb->gen;
    memcpy(A->inv_beta, beta, 32);
    A->inv_nz = (hf & 2u) ? !czero : !tzero;
    Binv->inv_nz = !tzero;
    if (c->lu_tinv) zkh_tensor_free(c->lu_tinv);
    c->lu_tinv = Binv;
    c->lu_tinv_of = Tcomb->gen;
    memcpy(c->lu_tinv_beta, beta, 32);
    *comb_out = comb;
    *Tcomb_out = Tcomb;
    *A_out = A;
    return ZKH_OK;
}

// The logUp round polynomial is a sum of pieces, each itself a sumcheck over the remaining
// variables: Ia = sum eq A (S + beta), Sa = sum A, Ib = sum eq B (T + beta), Mb = sum m B
// (eq over the variables after the round's own, the round's eq factor kept outside).  A
// round's piece q satisfies (1 - u) q(0) + u q(1) = I (eq-weighted) or q(0) + q(1) = I
// (plain) and binds to I' = q(v), so a round that folds can leave its sums at 1 to the
// host.  At the end I equals the piece of the terminals.
struct LuPieces {
    Fr Ia = kZero, Sa = kZero, Ib = kZero, Mb = kZero;
    bool b = false;  // Ib, Mb hold (a phase-2 round has run)
};
// q(v) of a quadratic piece from q(0), q(1) and its t^2 coefficient c2
// (vm = to_m(v))
static Fr quad_at_m(const Fr& q0, const Fr& q1, const Fr& c2, const Fr& vm) {
    return fr_add(q0, mulm(fr_add(fr_sub(fr_sub(q1, q0), c2), mulm(c2, vm)), vm));
}
// logUp phase-2 state carried across rounds (zkob_lookup.cuh:143-198): the running claim,
// alpha and alpha^2 eq accumulators, N/D, the eq point u and its device tables
struct LuState {
    Fr claim, alpha, alpha_sq, inv_ratio;
    const std::vector<Fr>* u;
    const EqState* eq;
    uint32_t logD;
    LuPieces* pc;
    Fr inv_ratio_m;  // to_m(inv_ratio)
    // a round's state update left for after its challenge is sent (lu_phase2_round's defer)
    struct Pending {
        bool on = false;
        Fr coef[4], q[9], s3, s4, ul, v, v_m;
    } pend;
};
// applies the update of the round whose challenge is v (the claim c(v), alpha and alpha^2
// times eq(ul, v), the pieces at v)
static void lu_apply(LuState& L) {
    LuState::Pending& p = L.pend;
    if (!p.on) return;
    p.on = false;
    L.claim = cubic_at(p.coef, p.v_m);
    const Fr uv = mulm(p.ul, p.v_m);
    const Fr eqv_m = to_m(fr_add(fr_sub(fr_add(uv, uv), fr_add(p.ul, p.v)), kOne));  // eq(ul, v)
    L.alpha = mulm(L.alpha, eqv_m);
    L.alpha_sq = mulm(L.alpha_sq, eqv_m);
    L.pc->Ia = quad_at_m(p.q[0], p.q[1], p.q[2], p.v_m);
    L.pc->Sa = fr_add(p.s3, mulm(fr_sub(p.s4, p.s3), p.v_m));
    L.pc->Ib = quad_at_m(p.q[3], p.q[4], p.q[5], p.v_m);
    L.pc->Mb = quad_at_m(p.q[6], p.q[7], p.q[8], p.v_m);
    L.pc->b = true;
}
// One phase-2 round from its 11 sums (device order: w a s sums 0..2, sum a0, sum a1, w b t
// sums 0..2, m b sums 0..2).  dev: sums from the device (products x 2^-256, eq weights with
// the padded factors that corr(K) removes); otherwise exact host sums.  Absorbs "p0".."p3",
// draws the challenge v, updates the state; false on a round inconsistency.
static bool lu_phase2_round(uint8_t tr[32], LuState& L, uint32_t r, const Fr sm[11], bool dev, Fr& v,
                            uint32_t* ev_out, uint32_t* ws_out, bool defer = false) {
    lu_apply(L);
    const uint32_t k = L.logD - r, K = k - 1;
    const Fr ul = (*L.u)[k - 1];
    const Fr corr_mm = dev ? to_mm(eq_corr(*L.eq, K)) : kZero;
    auto pr = [&](const Fr& x) { return dev ? mulm(x, corr_mm) : x; };  // w-weighted product sums
    auto mb = [&](const Fr& x) { return dev ? fix1(x) : x; };          // m b product sums
    LuState::Pending& p = L.pend;
    const Fr qa0 = pr(sm[0]), qa1 = pr(sm[1]), qa2 = pr(sm[2]);
    const Fr qb0 = pr(sm[5]), qb1 = pr(sm[6]), qb2 = pr(sm[7]);
    const Fr alpha_m = to_m(L.alpha), coefBT_m = to_m(mulm(L.alpha_sq, L.inv_ratio_m));
    const Fr Q0 = fr_add(mulm(qa0, alpha_m), mulm(qb0, coefBT_m));
    const Fr Q1 = fr_add(mulm(fr_sub(fr_sub(qa1, qa0), qa2), alpha_m), mulm(fr_sub(fr_sub(qb1, qb0), qb2), coefBT_m));
    const Fr Q2 = fr_add(mulm(qa2, alpha_m), mulm(qb2, coefBT_m));
    const Fr M0 = mb(sm[8]), M1 = mb(sm[9]), M2 = mb(sm[10]);
    const Fr Mc1 = fr_sub(fr_sub(M1, M0), M2);
    const Fr e0_m = to_m(fr_sub(kOne, ul)), e1_m = to_m(fr_sub(fr_add(ul, ul), kOne));
    const Fr& ir_m = L.inv_ratio_m;
    Fr* coef = p.coef;
    coef[0] = fr_sub(fr_add(mulm(Q0, e0_m), sm[3]), mulm(M0, ir_m));
    coef[1] = fr_sub(fr_add(fr_add(mulm(Q1, e0_m), mulm(Q0, e1_m)), fr_sub(sm[4], sm[3])), mulm(Mc1, ir_m));
    coef[2] = fr_sub(fr_add(mulm(Q2, e0_m), mulm(Q1, e1_m)), mulm(M2, ir_m));
    coef[3] = mulm(Q2, e1_m);
    Fr e[4];
    cubic_at123(coef, e);
    if (!fr_eq(L.claim, fr_add(e[0], e[1]))) return false;
    static const char* lab[4] = {"p0", "p1", "p2", "p3"};
    for (int t = 0; t < 4; t++) {
        tr_absorb_fr(tr, lab[t], e[t]);
        if (ev_out) fr_store(e[t], ev_out + 8 * (4 * r + t));
    }
    v = tr_challenge(tr);
    if (ws_out) fr_store(v, ws_out + 8 * r);
    const Fr q[9] = {qa0, qa1, qa2, qb0, qb1, qb2, M0, M1, M2};
    for (int i = 0; i < 9; i++) p.q[i] = q[i];
    p.s3 = sm[3];
    p.s4 = sm[4];
    p.ul = ul;
    p.v = v;
    p.v_m = to_m(v);
    p.on = true;
    if (!defer) lu_apply(L);
    return true;
}
// Phase-2 rounds r0 .. logD-1 in one persistent launch (see LuPersist) once the tables have
// n <= ZKH_LU_PERSIST_MAX entries; the block-count rounds at the end run on the host with
// the exact eq weights.  fin receives the terminals A_f, S_f, B_f, T_f, m_f.
#define ZKH_LU_PERSIST_MAX 8192u
// entries per block and table of the logUp and Hadamard persistent loops
#ifndef ZKH_LH_PLS
#define ZKH_LH_PLS ZKH_PLS_MAX
#endif
// Per message of a persistent loop (ZKH_TRACE): block 0's compute (command received -> sums
// published, device clock; the first message's load and round are not bracketed), round
// trip (sums published -> command received) and the host's work (sums seen -> command
// sent).  slot0: block 0's slot after the kernel has exited; host: the sums-seen and
// command-sent times of each message.
static void trace_persist(zkh_ctx* c, const char* what, const uint32_t* slot0, uint32_t nmsg,
                          const std::vector<double>& host, uint32_t stamp = ZKH_PSTAMP) {
    const double tick_us = 1000.0 / (double)c->clock_khz;
    const uint32_t* st = slot0 + stamp;
    fprintf(stderr, "[zkh]   %s messages (compute/trip/host us):", what);
    for (uint32_t m = 1; m <= nmsg && m < 14; m++) {
        const double comp = m > 1 ? (double)(uint32_t)(st[4 + 2 * m] - st[3 + 2 * m]) * tick_us : 0.0;
        const double trip = m < nmsg ? (double)(uint32_t)(st[5 + 2 * m] - st[4 + 2 * m]) * tick_us : 0.0;
        const size_t i = 2 * (size_t)(m - 1);
        const double hw = i + 1 < host.size() ? host[i + 1] - host[i] : 0.0;
        fprintf(stderr, " %.1f/%.1f/%.1f", comp, trip, hw);
    }
    fprintf(stderr, "\n");
}
// eq(i, u[0..K)) for i < h (h a power of two, log2 h <= K): the factor (1 - u_j) of every bit
// j >= log2 h that i leaves 0, times the table of the low bits built one bit at a time
// (K - log2 h + 2h - 2 products instead of h K)
static void eq_low_weights(const std::vector<Fr>& u, uint32_t K, uint32_t h, std::vector<Fr>& w) {
    uint32_t lg = 0;
    while ((1u << lg) < h) lg++;
    Fr base = kOne;
    for (uint32_t j = lg; j < K; j++) base = fr_mul(base, fr_sub(kOne, u[j]));
    w.assign(h, kZero);
    w[0] = base;
    for (uint32_t j = 0; j < lg; j++) {
        const uint32_t half = 1u << j;
        const Fr one_m = fr_sub(kOne, u[j]);
        for (uint32_t i = 0; i < half; i++) {
            w[i + half] = fr_mul(w[i], u[j]);
            w[i] = fr_mul(w[i], one_m);
        }
    }
}
// mode: 0 launch and serve; 1 launch only, behind a relay queued here (held by *rg) that
// hands the kernel the owed challenge; 2 serve the loop mode 1 launched.  (The relay goes in
// after the slot memory is in place: its first allocation waits for the stream.)
static int lu_persist_rounds(zkh_ctx* c, uint8_t tr[32], LuState& L, uint32_t r0, uint32_t n, const DevPlanes src[5],
                             bool fold_as, bool fold_btm, const uint32_t vm[8], RelayGuard* rg,
                             const uint32_t beta_l[8], uint32_t* ev_out, uint32_t* ws_out, Fr fin[5], int mode) {
    const uint32_t lgnb = n > ZKH_LH_PLS ? ceil_log2(n / ZKH_LH_PLS) : 0, nb = 1u << lgnb;
    const uint32_t R = ceil_log2(n) - lgnb;  // local rounds
    int rc;
    if ((rc = ensure_ps(c, (size_t)ZKH_LU_PSLOT * (nb + 2)))) return rc;
    uint32_t* ps = c->ps_host;
    uint32_t* slots = ps + ZKH_LU_PSLOT;
    uint32_t* cmd = ps + (size_t)ZKH_LU_PSLOT * (nb + 1);
    if (mode != 2) memset(ps, 0, (size_t)ZKH_LU_PSLOT * (nb + 2) * 4);
    LuPersist P{};
    for (int i = 0; i < 5; i++) {
        P.lo[i] = src[i].lo();
        P.hi[i] = src[i].hi();
    }
    P.elo = L.eq->elo_d;
    P.ehi = L.eq->ehi_d;
    P.out = slots;
    P.cmd = cmd;
    P.err = ps;
    P.deadline = c->clock_khz * 1000 * 20;  // 20 s without a command
    if (vm) memcpy(P.vm.v, vm, 32);
    if (mode == 1) {
        rg->pending = relay_enqueue(c);
        P.vmp = c->relay_vm;
    }
    memcpy(P.beta.v, beta_l, 32);
    P.n = n;
    P.lgnb = lgnb;
    P.fold_as = fold_as;
    P.fold_btm = fold_btm;
    P.two = getenv("ZKH_PERSIST_ONE") ? 0 : 1;  // two rounds per message while a block holds >= 4 entries
    auto send = [&](uint32_t seq, const uint32_t* xm, uint32_t nw) {
        for (uint32_t i = 0; i < nw && xm; i++) __atomic_store_n(cmd + zkh_quad_word(i), xm[i], __ATOMIC_RELAXED);
        for (uint32_t qd = 0; qd < zkh_quad_count(nw); qd++) __atomic_store_n(cmd + 4 * qd, seq, __ATOMIC_RELEASE);
    };
    auto quit = [&]() {
        send(ZKH_QUIT, nullptr, 32);
        (void)hipStreamSynchronize(c->stream);
    };
    if (mode != 2) {
        ProfScope ps_(c, "lu_persist", (double)n * 5 * 32 * 2);
        hipError_t e = launch_lu_persist(c->stream, P);
        if (e != hipSuccess) {
            quit();
            return fail(c, ZKH_EDEV, "persistent logUp launch: %s", hipGetErrorString(e));
        }
        if (mode == 1) return 0;
    }
    const double t_launch = now_us();
    auto slot_fr = [&](uint32_t b, uint32_t i) {
        uint32_t v[8];
        for (uint32_t j = 0; j < 8; j++) v[j] = slots[(size_t)b * ZKH_LU_PSLOT + zkh_quad_word(8 * i + j)];
        return fr_load(v);
    };
    auto wait_msg = [&](uint32_t seq, uint32_t nw) -> int {
        const uint32_t nq = zkh_quad_count(nw);
        const double t0 = now_us();
        for (uint64_t spins = 1;; spins++) {
            bool all = true;
            for (uint32_t b = 0; b < nb && all; b++)
                for (uint32_t qd = 0; qd < nq; qd++)
                    if (__atomic_load_n(slots + (size_t)b * ZKH_LU_PSLOT + 4 * qd, __ATOMIC_ACQUIRE) != seq) {
                        all = false;
                        break;
                    }
            if (all) return 0;
            spin_pause(spins);
            if ((spins & 0x3FFF) == 0) {
                hipError_t e = hipStreamQuery(c->stream);
                if (e != hipSuccess && e != hipErrorNotReady) {
                    quit();
                    return fail(c, ZKH_EDEV, "persistent logUp rounds: %s", hipGetErrorString(e));
                }
                if (__atomic_load_n(ps, __ATOMIC_ACQUIRE) || e == hipSuccess || now_us() - t0 > 30e6) {
                    quit();
                    return fail(c, ZKH_EDEV, "persistent logUp rounds stopped (%s)",
                                ps[0] ? "a block timed out" : e == hipSuccess ? "kernel ended early" : "no progress");
                }
            }
        }
    };
    const bool tracing = trace_on();
    std::vector<double> tr_h;  // per message: sums seen, command sent
    uint32_t seq = 1;
    for (uint32_t lr = 0; lr < R; seq++) {
        const uint32_t r1 = r0 + lr;
        if (!P.two || R - lr < 2) {  // one round
            if ((rc = wait_msg(seq, ZKH_LU_MSG))) return rc;
            if (tracing) tr_h.push_back(now_us());
            Fr sm[11];
            for (int t = 0; t < 11; t++) sm[t] = kZero;
            for (uint32_t b = 0; b < nb; b++)
                for (int t = 0; t < 11; t++) sm[t] = fr_add(sm[t], slot_fr(b, t));
            Fr v;
            if (!lu_phase2_round(tr, L, r1, sm, true, v, ev_out, ws_out, true)) {
                quit();
                return fail(c, ZKH_EROUND, "phase2 round inconsistency (witness bug) at round %u", r1);
            }
            uint32_t xm[8];
            fr_store(L.pend.v_m, xm);
            send(seq, xm, 8);
            lu_apply(L);  // the state update after the command
            if (tracing) tr_h.push_back(now_us());
            lr++;
            continue;
        }
        // two rounds from the point sums (index 3 a + b; a: the first variable y1, b: the
        // second y2; 0, 1, inf): AS = G[0..9), BT = G[9..18), MB = G[18..27), A at corner
        // 2 y1 + y2 = G[27 + j].  Round r1's sums over the pairs (c + y2 q, c + y2 q + 2q):
        // the eq-weighted pieces as X(t, 0) + rho X(t, 1) (rho = u/(1 - u) of y2 relative to
        // the cell weight), the others X(t, 0) + X(t, 1); round r1 + 1's: X(v1, t)
        if ((rc = wait_msg(seq, ZKH_LU_MSG2))) return rc;
        if (tracing) tr_h.push_back(now_us());
        Fr G[31];
        for (int p = 0; p < 31; p++) G[p] = kZero;
        for (uint32_t b = 0; b < nb; b++)
            for (int p = 0; p < 31; p++) G[p] = fr_add(G[p], slot_fr(b, p));
        const uint32_t K2 = L.logD - r1 - 2;  // eq coordinate of y2
        const Fr rho_m = mulm(to_m((*L.u)[K2]), to_m(L.eq->inv1mu[K2]));
        Fr sm[11], v1, v2;
        for (int a = 0; a < 3; a++) {
            sm[a] = fr_add(G[3 * a], mulm(G[3 * a + 1], rho_m));
            sm[5 + a] = fr_add(G[9 + 3 * a], mulm(G[9 + 3 * a + 1], rho_m));
            sm[8 + a] = fr_add(G[18 + 3 * a], G[18 + 3 * a + 1]);
        }
        sm[3] = fr_add(G[27], G[28]);
        sm[4] = fr_add(G[29], G[30]);
        if (!lu_phase2_round(tr, L, r1, sm, true, v1, ev_out, ws_out, true)) {
            quit();
            return fail(c, ZKH_EROUND, "phase2 round inconsistency (witness bug) at round %u", r1);
        }
        const Fr v1_m = L.pend.v_m;
        for (int b = 0; b < 3; b++) {
            sm[b] = quad_at_m(G[b], G[3 + b], G[6 + b], v1_m);
            sm[5 + b] = quad_at_m(G[9 + b], G[12 + b], G[15 + b], v1_m);
            sm[8 + b] = quad_at_m(G[18 + b], G[21 + b], G[24 + b], v1_m);
        }
        sm[3] = fr_add(G[27], mulm(fr_sub(G[29], G[27]), v1_m));
        sm[4] = fr_add(G[28], mulm(fr_sub(G[30], G[28]), v1_m));
        if (!lu_phase2_round(tr, L, r1 + 1, sm, true, v2, ev_out, ws_out, true)) {
            quit();
            return fail(c, ZKH_EROUND, "phase2 round inconsistency (witness bug) at round %u", r1 + 1);
        }
        // double fold weights of T[c + (2 y1 + y2) q], in Montgomery form: (1 - v)_m = 1_m - v_m
        const Fr v2_m = L.pend.v_m, a1_m = fr_sub(fr_one_m(), v1_m), a2_m = fr_sub(fr_one_m(), v2_m);
        const Fr Lw_m[4] = {mulm(a1_m, a2_m), mulm(a1_m, v2_m), mulm(v1_m, a2_m), mulm(v1_m, v2_m)};
        uint32_t xm[32];
        for (int j = 0; j < 4; j++) fr_store(Lw_m[j], xm + 8 * j);
        send(seq, xm, 32);
        lu_apply(L);  // the state update after the command
        if (tracing) tr_h.push_back(now_us());
        lr += 2;
    }
    if ((rc = wait_msg(seq, 40))) return rc;
    std::vector<Fr> t[5];
    for (int i = 0; i < 5; i++) {
        t[i].resize(nb);
        for (uint32_t b = 0; b < nb; b++) t[i][b] = slot_fr(b, i);
    }
    // (no wait for the blocks to exit: none touches the slots after its last message, and
    // later work on the stream is ordered behind the kernel; tracing reads the clock stamps)
    if (tracing) HIPCHK(c, hipStreamSynchronize(c->stream));
    const Fr beta = fr_load(beta_l);
    // the last lgnb rounds over the blocks' entries (entry b is global index b)
    for (uint32_t r = r0 + R, m = nb; m > 1; r++, m >>= 1) {
        const uint32_t h = m >> 1, K = L.logD - r - 1;
        Fr sm[11];
        for (int q = 0; q < 11; q++) sm[q] = kZero;
        const std::vector<Fr>& A = t[0], &S = t[1], &B = t[2], &T = t[3], &M = t[4];
        std::vector<Fr> wl;
        eq_low_weights(*L.u, K, h, wl);
        for (uint32_t i = 0; i < h; i++) {
            // w A, w dA, w B, w dB in Montgomery form (w_mm = w 2^512): each product below is one
            const Fr w_mm = to_mm(wl[i]);
            const Fr wa0 = mulm(A[i], w_mm), wda = mulm(fr_sub(A[i + h], A[i]), w_mm);
            const Fr wb0 = mulm(B[i], w_mm), wdb = mulm(fr_sub(B[i + h], B[i]), w_mm);
            const Fr b0_m = to_m(B[i]), b1_m = to_m(B[i + h]);
            const Fr add[11] = {mulm(fr_add(S[i], beta), wa0), mulm(fr_add(S[i + h], beta), fr_add(wa0, wda)),
                                mulm(fr_sub(S[i + h], S[i]), wda), A[i], A[i + h],
                                mulm(fr_add(T[i], beta), wb0), mulm(fr_add(T[i + h], beta), fr_add(wb0, wdb)),
                                mulm(fr_sub(T[i + h], T[i]), wdb), mulm(M[i], b0_m), mulm(M[i + h], b1_m),
                                mulm(fr_sub(M[i + h], M[i]), fr_sub(b1_m, b0_m))};
            for (int q = 0; q < 11; q++) sm[q] = fr_add(sm[q], add[q]);
        }
        Fr v;
        if (!lu_phase2_round(tr, L, r, sm, false, v, ev_out, ws_out))
            return fail(c, ZKH_EROUND, "phase2 round inconsistency (witness bug) at round %u", r);
        const Fr v_m = to_m(v);
        for (int q = 0; q < 5; q++)
            for (uint32_t i = 0; i < h; i++) t[q][i] = fr_add(t[q][i], mulm(fr_sub(t[q][i + h], t[q][i]), v_m));
    }
    lu_apply(L);
    for (int i = 0; i < 5; i++) fin[i] = t[i][0];
    if (tracing) {
        fprintf(stderr, "[zkh] lu persistent loop: n=%u, %u blocks, %u device + %u host rounds in %.1f us\n", n, nb, R,
                lgnb, now_us() - t_launch);
        trace_persist(c, "lu", slots, seq, tr_h, ZKH_LU_PSTAMP);
    }
    return 0;
}
static int lu_prove_impl(zkh_ctx* c, uint8_t tr[32], const zkh_tensor* A, const zkh_tensor* S,
                         const zkh_tensor* T, const zkh_tensor* m, const uint32_t alpha_l[8],
                         const uint32_t beta_l[8], const uint32_t* u_l, uint32_t* ev_out,
                         uint32_t* term_out, uint32_t* ws_out) {
    if (!c || !tr || !A || !S || !T || !m || !alpha_l || !beta_l) return fail(c, ZKH_EARG, "null argument");
    const uint32_t D = A->n, N = T->n;
    // tLookup::prove shape rules (tlookup.cu:330-336)
    if (S->n != D || m->n != N || !D || !N || (D & (D - 1)) || (N & (N - 1)) || D % N)
        return fail(c, ZKH_EARG, "D or N is not power of 2, or D is not divisible by N");
    const uint32_t logD = ceil_log2(D);
    if (logD && !u_l) return fail(c, ZKH_EARG, "null u");
    if (!fr_is_canonical(alpha_l) || !fr_is_canonical(beta_l) || !all_canonical(u_l, logD))
        return fail(c, ZKH_EARG, "non-canonical challenge");
    HIPCHK(c, hipSetDevice(c->device));
    int rc = 0;
    Fr alpha = fr_load(alpha_l), beta = fr_load(beta_l);
    std::vector<Fr> u = load_frs(u_l, logD);

    // working tables: caller tensors are read in place until their first fold.  An int32 m
    // (the counts of zkh_lu_prep / zkh_lu_mapping) is read as int32 by the round kernels up to
    // its first fold when D == N and the first two rounds (m's first read and first fold) are
    // round kernels, not the persistent loop; otherwise as planes
    const bool m_i32 = m->kind == ZKH_KIND_I32 && !m->weights && D == N && N / 2 > ZKH_LU_PERSIST_MAX;
    DevPlanes Ac, Sc, Tc, mc{};
    if ((rc = as_planes(c, A, SL_TMP0, &Ac)) || (rc = as_planes(c, S, SL_TMP1, &Sc)) ||
        (rc = as_planes(c, T, SL_TMP2, &Tc)) || (!m_i32 && (rc = as_planes(c, m, SL_TMP3, &mc))))
        return rc;
    const int32_t* m_src32 = m_i32 ? (const int32_t*)m->d : nullptr;  // m's source while unfolded
    DevPlanes Aw = A->kind == ZKH_KIND_FR ? scratch_planes(c, SL_TMP0, D / 2, &rc) : Ac;
    if (rc) return rc;
    DevPlanes Sw = S->kind == ZKH_KIND_FR ? scratch_planes(c, SL_TMP1, D / 2, &rc) : Sc;
    if (rc) return rc;
    DevPlanes Tw = T->kind == ZKH_KIND_FR ? scratch_planes(c, SL_TMP2, N / 2, &rc) : Tc;
    if (rc) return rc;
    DevPlanes mw = m->kind == ZKH_KIND_FR || m_i32 ? scratch_planes(c, SL_TMP3, N / 2, &rc) : mc;
    if (rc) return rc;
    // Bv = 1/(T+beta), owned: zkh_lu_tuple_inverse's table inverse when T is its T_comb and
    // beta its beta (taken over: the rounds fold it in place), else inverted here
    struct TakenInverse {
        zkh_ctx* c;
        zkh_tensor* t = nullptr;
        ~TakenInverse() {
            if (!t) return;
            (void)hipStreamSynchronize(c->stream);
            zkh_tensor_free(t);
        }
    } taken{c};
    if (c->lu_tinv && c->lu_tinv_of == T->gen && !memcmp(c->lu_tinv_beta, beta_l, 32) && c->lu_tinv->n == N) {
        taken.t = c->lu_tinv;
        c->lu_tinv = nullptr;
        c->lu_tinv_of = 0;
    } else if (c->lu_tinv) {  // kept for another table or beta: this proof ends its use
        zkh_tensor_free(c->lu_tinv);
        c->lu_tinv = nullptr;
        c->lu_tinv_of = 0;
    }
    DevPlanes Bw = taken.t ? taken.t->planes() : scratch_planes(c, SL_EO, N, &rc);
    if (rc) return rc;
    bool b_zero = taken.t && !taken.t->inv_nz;  // B has a zero entry (or may have)
    if (!taken.t && (rc = batch_inverse(c, Tc, N, beta, Bw, &b_zero))) return rc;

    // C = alpha^2 - sum Bv*m (zkob_rescale.cu:136); only the phase-1 rounds (D > N) use it
    Fr bm = kZero;
    if (D > N) {
        Publish pb = make_pub(c, 1);
        launch_dot_planes(c->stream, Bw, mc, N, pb);
        if ((rc = wait_pub(c, pb.seq))) return rc;
        pub_read(c, 0, 1, &bm);
        bm = fix1(bm);
    }
    Fr alpha_sq = fr_mul(alpha, alpha);
    Fr Cc = fr_sub(alpha_sq, bm);
    Fr claim = fr_add(alpha, alpha_sq);
    // N / D with D / N a power of two: halve 1 log2(D / N) times
    Fr inv_ratio = kOne;
    for (uint32_t t = N; t < D; t <<= 1) inv_ratio = fr_half(inv_ratio);
    const Fr inv_ratio_m = to_m(inv_ratio);

    EqState eq;  // tables now, the host part once the first round is queued
    if ((rc = eq_setup(c, u, eq, true, false))) return rc;

    // table handles: source = current data, dst = working buffer
    DevPlanes a_src = Ac, s_src = Sc, b_src = Bw, t_src = Tc, m_src = mc;
    bool as_pending = false, btm_pending = false;  // a fold with vm is owed
    uint32_t vm[8] = {0};
    const bool tracing = trace_on();
    std::vector<double> tr_t;  // per round: launch, sums seen, challenge done (host clock)
    bool persisted = false;    // the last rounds ran in lu_persist_rounds
    bool persist_queued = false;  // ... launched behind the previous round's relay
    Fr fin[5];
    const bool no_persist = getenv("ZKH_NO_PERSIST") != nullptr;
    auto persists = [&](uint32_t r) {  // phase 2 small enough for the persistent loop
        const uint32_t n = D >> r;
        return n <= N && n <= ZKH_LU_PERSIST_MAX && !no_persist;
    };
    // A from zkh_lu_inverse(S, beta) is 1/(S + beta) entry-wise, and so is the internal B of
    // T: a group's first (unfolded) round then needs two products per pair fewer, its sums
    // 0 and 1 coming as sum e over the nonzero entries (cf: no 2^-256 to undo)
    const bool a_is_inv = A->kind == ZKH_KIND_FR && A->inv_of && A->inv_of == S->gen && !memcmp(A->inv_beta, beta_l, 32);
    // ... and with no zero entry in A (B) every a (s + beta) (b (t + beta)) is 1: the first
    // round's weighted sums of those products are sum eq = 1, not formed on the device
    const bool a_nz = a_is_inv && A->inv_nz, b_nz = !b_zero;
    // a folding round leaves its sums at 1 to the pieces (LuPieces) unless its eq coordinate
    // is 0; inv_u holds 1/u_j, computed while the first round runs
    LuPieces pc;
    std::vector<Fr> inv_u;
    // (ZKH_XCHECK=1: no round derives, so every round's p(0) + p(1) = claim is checked on
    // sums the device computed, and a device error fails at its own round as in the
    // reference, zkob_lookup.cuh:155, :183)
    const bool per_round_check = xcheck_on();
    auto derives = [&](uint32_t r) { return !per_round_check && !fr_eq(u[logD - r - 1], kZero); };
    struct Launched {
        Publish pb;
        bool cf_a, cf_b;
        bool dv_a, dv_b;  // the group's sums at 1 are left out
        bool nz;          // first round with no zero in A (and B in phase 2): reduced sums
    };
    // launches round r (reading the previous challenge from vm, or from the relay when vmp
    // is given) and moves the table handles to the folded copies the launch writes
    auto launch = [&](uint32_t r, const uint32_t* vmp) {
        const uint32_t n = D >> r, K = logD - r - 1;
        Launched l{};
        Publish& pb = l.pb;
        if (n > N) {  // phase 1
            pb = make_pub(c, 1);
            l.cf_a = a_is_inv && !as_pending;
            l.dv_a = as_pending && derives(r);
            l.nz = l.cf_a && a_nz && !vmp;
            if (l.nz) {
                ProfScope ps(c, "lu_phase1", (double)n * 2 * 32);
                launch_lu_first_nz(c->stream, Tab{a_src, Aw}, Tab{s_src, Sw}, Tab{}, Tab{}, Tab{}, n, 0,
                                   EqW{eq.elo_d, eq.ehi_d, K}, pb, nullptr);
            } else {
                ProfScope ps(c, "lu_phase1", (as_pending ? 3.0 * n : (double)n) * 2 * 32);
                launch_lu_phase1(c->stream, Tab{a_src, Aw}, Tab{s_src, Sw}, n, as_pending, vm, vmp, beta_l,
                                 EqW{eq.elo_d, eq.ehi_d, K}, pb, l.cf_a, l.dv_a);
            }
            if (as_pending) {
                a_src = Aw;
                s_src = Sw;
            }
            as_pending = true;
        } else {  // phase 2
            pb = make_pub(c, 2);
            l.cf_a = a_is_inv && !as_pending;
            l.cf_b = !btm_pending;
            const bool dv = as_pending && derives(r);
            l.dv_a = dv;
            l.dv_b = dv && btm_pending;
            l.nz = l.cf_a && l.cf_b && a_nz && b_nz && !vmp;
            {
                // bytes each table moves: read n entries, or fold 2n read into n written; m
                // is read as int32 counts (4 bytes) until its first fold writes its planes
                const double per = as_pending ? 3.0 * n : (double)n, pbt = btm_pending ? 3.0 * n : (double)n;
                const double m_bytes = !m_src32 ? pbt * 32 : btm_pending ? 2.0 * n * 4 + (double)n * 32 : (double)n * 4;
                ProfScope ps(c, "lu_phase2", per * 2 * 32 + pbt * 2 * 32 + m_bytes);
                if (l.nz)
                    launch_lu_first_nz(c->stream, Tab{a_src, Aw}, Tab{s_src, Sw}, Tab{b_src, Bw}, Tab{t_src, Tw},
                                       Tab{m_src, mw}, n, 1, EqW{eq.elo_d, eq.ehi_d, K}, pb, m_src32);
                else
                    launch_lu_phase2(c->stream, Tab{a_src, Aw}, Tab{s_src, Sw}, Tab{b_src, Bw}, Tab{t_src, Tw},
                                     Tab{m_src, mw}, n, as_pending, btm_pending, vm, vmp, beta_l,
                                     EqW{eq.elo_d, eq.ehi_d, K}, pb, l.cf_a, l.cf_b, dv, m_src32);
            }
            if (as_pending) {
                a_src = Aw;
                s_src = Sw;
            }
            if (btm_pending) {
                b_src = Bw;
                t_src = Tw;
                m_src = mw;
                m_src32 = nullptr;
            }
            as_pending = true;
            btm_pending = true;
        }
        return l;
    };
    // a published weighted-product sum as the round polynomial takes it
    auto q_of = [](const Fr& s, bool cf) { return cf ? fr_from_mont(s) : fix1(s); };
    RelayGuard relay{c};
    Launched cur{};
    bool launched = false;  // round r is already queued
    for (uint32_t r = 0; r < logD; r++) {
        const uint32_t n = D >> r;
        if (persists(r)) {  // phase 2: the rest in one launch
            if ((rc = eq_setup_host(c, u, eq))) return rc;
            LuState L{claim, alpha, alpha_sq, inv_ratio, &u, &eq, logD, &pc, inv_ratio_m, {}};
            if (m_src32) return fail(c, ZKH_EDEV, "internal: unfolded int32 m at the persistent loop");
            const DevPlanes src[5] = {a_src, s_src, b_src, t_src, m_src};
            if ((rc = lu_persist_rounds(c, tr, L, r, n, src, as_pending, btm_pending, vm, nullptr, beta_l, ev_out,
                                        ws_out, fin, persist_queued ? 2 : 0)))
                return rc;
            persisted = true;
            break;
        }
        if (tracing) tr_t.push_back(now_us());
        if (!launched) cur = launch(r, nullptr);
        // round r + 1 (or the persistent loop) goes behind a relay now, so that its launch
        // overlaps this round
        const bool relay_next = r + 1 < logD && !persists(r + 1);
        const bool persist_next = r + 1 < logD && persists(r + 1) && !m_src32;
        Launched next{};
        if (relay_next) {
            relay.pending = relay_enqueue(c);
            next = launch(r + 1, c->relay_vm);
        } else if (persist_next) {
            LuState L0{claim, alpha, alpha_sq, inv_ratio, &u, &eq, logD, &pc, inv_ratio_m, {}};
            const DevPlanes src[5] = {a_src, s_src, b_src, t_src, m_src};
            if ((rc = lu_persist_rounds(c, tr, L0, r + 1, D >> (r + 1), src, as_pending, btm_pending, nullptr, &relay,
                                        beta_l, nullptr, nullptr, fin, 1)))
                return rc;
            persist_queued = true;
        }
        if ((rc = eq_setup_host(c, u, eq))) return rc;  // once, behind the first launches
        const uint32_t k = logD - r;  // remaining variables
        const uint32_t K = k - 1;     // eq variables of the pairs
        const Fr ul = u[k - 1];
        const Fr corr = eq_corr(eq, K);
        Fr coef[4];
        if (r == 0 && logD > 1) {  // 1/u_j for the rounds that derive (batch inverse, host)
            inv_u.assign(logD, kZero);
            std::vector<Fr> pre(logD + 1, kOne);
            for (uint32_t j = 0; j < logD; j++) pre[j + 1] = fr_eq(u[j], kZero) ? pre[j] : fr_mul(pre[j], u[j]);
            Fr t = fr_inv(pre[logD]);
            for (uint32_t j = logD; j-- > 0;)
                if (!fr_eq(u[j], kZero)) {
                    inv_u[j] = fr_mul(t, pre[j]);
                    t = fr_mul(t, u[j]);
                }
        }
        // the round's multipliers prepared while the kernel runs (one product per use below)
        const Fr e0 = fr_sub(kOne, ul), e1 = fr_sub(fr_add(ul, ul), kOne);
        const Fr corr_mm = to_mm(corr), e0_m = to_m(e0), e1_m = to_m(e1), alpha_m = to_m(alpha);
        const Fr iu_m = inv_u.empty() ? kZero : to_m(inv_u[k - 1]);
        // a weighted-product sum as the round polynomial takes it: x 2^256 corr, or (cf: the
        // sum carries 2^256 already) x 2^-256 corr
        auto wq = [&](const Fr& x, bool cf) { return mulm(x, cf ? corr : corr_mm); };
        // q(1) of an eq-weighted piece with claim I: (I - (1 - ul) q(0)) / ul
        auto q1_of = [&](const Fr& I, const Fr& q0) { return mulm(fr_sub(I, mulm(q0, e0_m)), iu_m); };
        if ((rc = wait_pub(c, cur.pb.seq))) return rc;
        if (tracing) tr_t.push_back(now_us());
        // the pieces' values at 0 and 1 and their t^2 coefficients (true sums)
        Fr qa[3], sa[2], qb[3] = {kZero, kZero, kZero}, M[3] = {kZero, kZero, kZero};
        {
            Fr s[5];
            if (cur.dv_a) {  // w a0 s0, w da ds, a0
                pub_read(c, 0, 3, s);
                qa[0] = wq(s[0], false);
                qa[2] = wq(s[1], false);
                qa[1] = q1_of(pc.Ia, qa[0]);
                sa[0] = s[2];
                sa[1] = fr_sub(pc.Sa, s[2]);
            } else if (cur.nz) {  // w da ds, a0, a1; sum eq a (s + beta) = sum eq = 1 (no zero in A)
                pub_read(c, 0, 3, s);
                qa[0] = qa[1] = kOne;
                qa[2] = wq(s[0], false);
                sa[0] = s[1];
                sa[1] = s[2];
            } else {
                pub_read(c, 0, 5, s);
                qa[0] = wq(s[0], cur.cf_a);
                qa[1] = wq(s[1], cur.cf_a);
                qa[2] = wq(s[2], false);
                sa[0] = s[3];
                sa[1] = s[4];
            }
        }
        if (n <= N) {
            Fr s[6];
            if (cur.dv_b) {  // w b0 t0, w db dt, m0 b0, dm db
                pub_read(c, 1, 4, s);
                qb[0] = wq(s[0], false);
                qb[2] = wq(s[1], false);
                qb[1] = q1_of(pc.Ib, qb[0]);
                M[0] = fix1(s[2]);
                M[2] = fix1(s[3]);
                M[1] = fr_sub(pc.Mb, M[0]);
            } else if (cur.nz) {  // w db dt, m0 b0, m1 b1, dm db (exact); sum eq b (t + beta) = 1
                pub_read(c, 1, 4, s);
                qb[0] = qb[1] = kOne;
                qb[2] = wq(s[0], false);
                for (int t = 0; t < 3; t++) M[t] = s[1 + t];
            } else {
                pub_read(c, 1, 6, s);
                qb[0] = wq(s[0], cur.cf_b);
                qb[1] = wq(s[1], cur.cf_b);
                qb[2] = wq(s[2], false);
                for (int t = 0; t < 3; t++) M[t] = cur.cf_b ? s[3 + t] : fix1(s[3 + t]);  // exact when cf_b
            }
        }
        if (n > N) {  // phase 1
            const Fr qc1 = fr_sub(fr_sub(qa[1], qa[0]), qa[2]);
            const Fr aq0 = mulm(qa[0], alpha_m), aq1 = mulm(qc1, alpha_m), aq2 = mulm(qa[2], alpha_m);
            coef[0] = fr_add(fr_add(mulm(aq0, e0_m), sa[0]), fr_half(Cc));
            coef[1] = fr_add(fr_add(mulm(aq1, e0_m), mulm(aq0, e1_m)), fr_sub(sa[1], sa[0]));
            coef[2] = fr_add(mulm(aq2, e0_m), mulm(aq1, e1_m));
            coef[3] = mulm(aq2, e1_m);
        } else {  // phase 2
            const Fr coefBT_m = to_m(mulm(alpha_sq, inv_ratio_m));
            const Fr Q0 = fr_add(mulm(qa[0], alpha_m), mulm(qb[0], coefBT_m));
            const Fr Q1 = fr_add(mulm(fr_sub(fr_sub(qa[1], qa[0]), qa[2]), alpha_m),
                                 mulm(fr_sub(fr_sub(qb[1], qb[0]), qb[2]), coefBT_m));
            const Fr Q2 = fr_add(mulm(qa[2], alpha_m), mulm(qb[2], coefBT_m));
            const Fr Mc1 = fr_sub(fr_sub(M[1], M[0]), M[2]);
            coef[0] = fr_sub(fr_add(mulm(Q0, e0_m), sa[0]), mulm(M[0], inv_ratio_m));
            coef[1] = fr_sub(fr_add(fr_add(mulm(Q1, e0_m), mulm(Q0, e1_m)), fr_sub(sa[1], sa[0])),
                             mulm(Mc1, inv_ratio_m));
            coef[2] = fr_sub(fr_add(mulm(Q2, e0_m), mulm(Q1, e1_m)), mulm(M[2], inv_ratio_m));
            coef[3] = mulm(Q2, e1_m);
        }
        Fr e[4];
        cubic_at123(coef, e);
        if (!fr_eq(claim, fr_add(e[0], e[1])))
            return fail(c, ZKH_EROUND, "phase%d round inconsistency (witness bug) at round %u",
                        n > N ? 1 : 2, r);
        static const char* lab[4] = {"p0", "p1", "p2", "p3"};
        for (int t = 0; t < 4; t++) {
            tr_absorb_fr(tr, lab[t], e[t]);
            if (ev_out) fr_store(e[t], ev_out + 8 * (4 * r + t));
        }
        Fr v = tr_challenge(tr);
        if (ws_out) fr_store(v, ws_out + 8 * r);
        const Fr v_m = to_m(v);
        fr_store(v_m, vm);
        if (relay_next || persist_next) {  // the queued launch starts now; the state updates overlap it
            relay_send(c, relay.pending, vm);
            relay.pending = 0;
        }
        claim = cubic_at(coef, v_m);
        const Fr uv = mulm(ul, v_m);
        const Fr eqv_m = to_m(fr_add(fr_sub(fr_add(uv, uv), fr_add(ul, v)), kOne));  // eq(ul, v)
        alpha = mulm(alpha, eqv_m);
        if (n > N) Cc = fr_half(Cc);
        else alpha_sq = mulm(alpha_sq, eqv_m);
        pc.Ia = quad_at_m(qa[0], qa[1], qa[2], v_m);
        pc.Sa = fr_add(sa[0], mulm(fr_sub(sa[1], sa[0]), v_m));
        if (n <= N) {
            pc.Ib = quad_at_m(qb[0], qb[1], qb[2], v_m);
            pc.Mb = quad_at_m(M[0], M[1], M[2], v_m);
            pc.b = true;
        }
        if (relay_next) cur = next;
        launched = relay_next;
        if (tracing) tr_t.push_back(now_us());
    }
    if (tracing) {  // per round: table size, launch -> sums seen, host work (us)
        fprintf(stderr, "[zkh] lu rounds (n: device/host us)%s:", persisted ? ", then the persistent loop" : "");
        for (uint32_t r = 0; r < tr_t.size() / 3; r++)
            fprintf(stderr, " %u:%.1f/%.1f", D >> r, tr_t[3 * r + 1] - tr_t[3 * r], tr_t[3 * r + 2] - tr_t[3 * r + 1]);
        fprintf(stderr, "\n");
    }
    uint32_t tv[5][8];
    if (persisted) {
        for (int i = 0; i < 5; i++) fr_store(fin[i], tv[i]);
    } else {
        // owed folds produce the terminals (size 2 -> 1)
        if (as_pending) {
            launch_fold(c->stream, Tab{a_src, Aw}, 1, vm);
            launch_fold(c->stream, Tab{s_src, Sw}, 1, vm);
            a_src = Aw;
            s_src = Sw;
        }
        if (btm_pending) {
            launch_fold(c->stream, Tab{b_src, Bw}, 1, vm);
            launch_fold(c->stream, Tab{t_src, Tw}, 1, vm);
            if (m_src32) return fail(c, ZKH_EDEV, "internal: unfolded int32 m at the last fold");
            launch_fold(c->stream, Tab{m_src, mw}, 1, vm);
            b_src = Bw;
            t_src = Tw;
            m_src = mw;
        }
        const DevPlanes dfin[5] = {a_src, s_src, b_src, t_src, m_src};
        for (int i = 0; i < 5; i++) {
            HIPCHK(c, hipMemcpyAsync(tv[i], dfin[i].lo(), 16, hipMemcpyDeviceToHost, c->stream));
            HIPCHK(c, hipMemcpyAsync(tv[i] + 4, dfin[i].hi(), 16, hipMemcpyDeviceToHost, c->stream));
        }
        HIPCHK(c, hipStreamSynchronize(c->stream));
    }
    if (logD > 0) {  // every piece's claim is its terminal form (checks the rounds whose sums at 1 were derived)
        const Fr Af = fr_load(tv[0]), Sf = fr_load(tv[1]), Bf = fr_load(tv[2]), Tf = fr_load(tv[3]), mf = fr_load(tv[4]);
        bool ok = fr_eq(pc.Ia, fr_mul(Af, fr_add(Sf, beta))) && fr_eq(pc.Sa, Af);
        if (pc.b) ok = ok && fr_eq(pc.Ib, fr_mul(Bf, fr_add(Tf, beta))) && fr_eq(pc.Mb, fr_mul(mf, Bf));
        if (!ok) return fail(c, ZKH_EROUND, "logUp terminal mismatch (witness bug)");
    }
    if (term_out)
        for (int i = 0; i < 5; i++) memcpy(term_out + 8 * i, tv[i], 32);
    tr_absorb_fr(tr, "A_f", fr_load(tv[0]));
    tr_absorb_fr(tr, "S_f", fr_load(tv[1]));
    tr_absorb_fr(tr, "m_f", fr_load(tv[4]));
    return ZKH_OK;
}
// the opening point of a sumcheck's tables: its round challenges reversed (zkob_fc.cu:334-336,
// zkob_rescale.cu:148-149), as Fr words
static std::vector<uint32_t> reversed_point(const uint32_t* ws, uint32_t k) {
    std::vector<uint32_t> pt(8 * (size_t)std::max<uint32_t>(k, 1));
    for (uint32_t i = 0; i < k; i++) memcpy(&pt[8 * (size_t)i], ws + 8 * (size_t)(k - 1 - i), 32);
    return pt;
}
// t(pt[0..k)) against a terminal (ZKH_EROUND with the reference's message on mismatch)
static int xcheck_me(zkh_ctx* c, const zkh_tensor* t, const uint32_t* pt, uint32_t k, const uint32_t* term,
                     const char* what) {
    uint32_t e[8];
    int rc = zkh_me(c, t, pt, k, e);
    if (rc) return rc;
    if (memcmp(e, term, 32)) return fail(c, ZKH_EROUND, "%s terminal != multi_dim_me (convention bug)", what);
    return ZKH_OK;
}
extern "C" int zkh_lu_prove(zkh_ctx* c, uint8_t tr[32], const zkh_tensor* A, const zkh_tensor* S,
                            const zkh_tensor* T, const zkh_tensor* m, const uint32_t alpha_l[8],
                            const uint32_t beta_l[8], const uint32_t* u_l, uint32_t* ev_out,
                            uint32_t* term_out, uint32_t* ws_out) {
    if (!xcheck_on() || !A || !T) return lu_prove_impl(c, tr, A, S, T, m, alpha_l, beta_l, u_l, ev_out, term_out, ws_out);
    const uint32_t logD = ceil_log2(A->n), logN = ceil_log2(T->n);
    std::vector<uint32_t> wsb(8 * (size_t)std::max<uint32_t>(logD, 1)), tb(40);
    uint32_t* ws = ws_out ? ws_out : wsb.data();
    uint32_t* term = term_out ? term_out : tb.data();
    int rc = lu_prove_impl(c, tr, A, S, T, m, alpha_l, beta_l, u_l, ev_out, term, ws);
    if (rc) return rc;
    // zkob_rescale.cu:151-165, zkob_glu.cu:186-192: A_f, S_f at the point; m_f (and the
    // public T_f) at its first logN coordinates
    const std::vector<uint32_t> pt = reversed_point(ws, logD);
    if ((rc = xcheck_me(c, A, pt.data(), logD, term, "lookup A")) ||
        (rc = xcheck_me(c, S, pt.data(), logD, term + 8, "lookup S")) ||
        (rc = xcheck_me(c, T, pt.data(), logN, term + 24, "lookup T")) ||
        (rc = xcheck_me(c, m, pt.data(), logN, term + 32, "m")))
        return rc;
    return ZKH_OK;
}

// ---------------------------------------------------------------------------------------
// witness GEMM: Y = X W (+ bias) over the integers (zkob_fc.cu:212 Y = fc(X); zkFC::operator()
// zkfc.cu:44-58; FrTensor::matmul fr-tensor.cu:831-878).  The reference multiplies in the
// field; for integer operands its result is the integer product reduced mod r, which is
// what an exact int64 product represents (zkh_tensor_from_i64 semantics), and what its
// driver writes with save_long (zkob_fc.cu:214).
// ---------------------------------------------------------------------------------------
extern "C" int zkh_matmul_i32(zkh_ctx* c, const zkh_tensor* X, const zkh_tensor* W, const zkh_tensor* bias,
                              uint32_t B, uint32_t IN, uint32_t OUT, zkh_tensor** Y_out) {
    if (!c || !X || !W || !Y_out) return fail(c, ZKH_EARG, "null argument");
    *Y_out = nullptr;
    if (!B || !IN || !OUT) return fail(c, ZKH_EARG, "matmul dimensions must be positive");
    if (X->kind != ZKH_KIND_I32 || W->kind != ZKH_KIND_I32)
        return fail(c, ZKH_EARG, "matmul operands must be int32 tensors");
    if ((uint64_t)X->n != (uint64_t)B * IN || (uint64_t)W->n != (uint64_t)IN * OUT)
        return fail(c, ZKH_EARG, "matmul: incompatible dimensions");  // fr-tensor.cu:873
    if (W->weights && (W->w_in != IN || W->w_out != OUT)) return fail(c, ZKH_EARG, "weights registered as another shape");
    if ((uint64_t)B * OUT >= (1ull << 32)) return fail(c, ZKH_EARG, "output too large");
    if (bias && ((bias->kind != ZKH_KIND_I32 && bias->kind != ZKH_KIND_I64) || bias->n != OUT))
        return fail(c, ZKH_EARG, "bias must be an integer tensor of OUT entries");
    // |partial sums| < 2^(bits X + bits W + ceil log2 IN); the bias adds at most one bit
    const uint32_t span = X->bits + W->bits + ceil_log2(IN);
    const uint32_t bb = bias ? bias->bits : 0;
    if (std::max(span, bb) + 1 > 63) return fail(c, ZKH_EARG, "matmul result may exceed 63 bits");
    const int f64 = span <= 53;
    HIPCHK(c, hipSetDevice(c->device));
    int rc = 0;
    const int32_t* WT = (const int32_t*)W->d;
    if (!W->weights) {  // row-major IN x OUT: transpose once into scratch
        int32_t* wt = (int32_t*)scratch_slot(c, SL_TMP5, (size_t)W->n * 4, &rc);
        if (rc) return rc;
        launch_transpose_i32(c->stream, (const int32_t*)W->d, IN, OUT, wt);
        WT = wt;
    }
    const int64_t* bd = nullptr;
    if (bias) {
        if (bias->kind == ZKH_KIND_I32) {
            int64_t* b64 = (int64_t*)scratch_slot(c, SL_TMP4, (size_t)OUT * 8, &rc);
            if (rc) return rc;
            launch_widen_i32(c->stream, (const int32_t*)bias->d, OUT, b64);
            bd = b64;
        } else {
            bd = (const int64_t*)bias->d;
        }
    }
    zkh_tensor* Y;
    if ((rc = tensor_alloc(c, ZKH_KIND_I64, B * OUT, &Y))) return rc;
    {
        ProfScope ps(c, f64 ? "matmul_f64" : "matmul_i64", (double)B * IN * 4 + (double)IN * OUT * 4 + (double)B * OUT * 8);
        launch_matmul_i32(c->stream, (const int32_t*)X->d, WT, bd, B, IN, OUT, (int64_t*)Y->d, f64);
    }
    hipError_t e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        zkh_tensor_free(Y);
        return fail(c, ZKH_EDEV, "matmul: %s", hipGetErrorString(e));
    }
    if ((rc = int_bits_i64(c, (const int64_t*)Y->d, Y->n, &Y->bits))) {
        zkh_tensor_free(Y);
        return rc;
    }
    *Y_out = Y;
    return ZKH_OK;
}

// ---------------------------------------------------------------------------------------
// Pedersen commitments (commitment.cu:85-108).  Points are 144-byte G1Jacobian_t, AoS.
// ---------------------------------------------------------------------------------------
struct zkh_g1 {
    zkh_ctx* ctx = nullptr;
    uint32_t n = 0;
    void* d = nullptr;
    std::shared_ptr<MemPool> pool;
    size_t cls = 0;
};
static int g1_alloc(zkh_ctx* c, uint32_t n, zkh_g1** out) {
    zkh_g1* g = new zkh_g1();
    g->ctx = c;
    g->n = n;
    g->pool = c->mem;
    g->cls = MemPool::size_class((size_t)(n ? n : 1) * 144);
    g->d = c->mem->get(g->cls);
    if (!g->d && hipMalloc(&g->d, g->cls) != hipSuccess) {
        delete g;
        return fail(c, ZKH_EDEV, "hipMalloc(%zu) failed", (size_t)(n ? n : 1) * 144);
    }
    *out = g;
    return ZKH_OK;
}
extern "C" int zkh_g1_free(zkh_g1* g) {
    if (!g) return ZKH_EARG;
    if (g->d) g->pool->put(g->d, g->cls);
    delete g;
    return ZKH_OK;
}
extern "C" uint32_t zkh_g1_size(const zkh_g1* g) { return g ? g->n : 0; }
extern "C" int zkh_g1_from_host(zkh_ctx* c, const uint32_t* pts, uint32_t n, zkh_g1** out) {
    if (!c || !out || (!pts && n)) return fail(c, ZKH_EARG, "null argument");
    *out = nullptr;
    HIPCHK(c, hipSetDevice(c->device));
    zkh_g1* g;
    int rc = g1_alloc(c, n, &g);
    if (rc) return rc;
    if (n) {
        hipError_t e = hipMemcpyAsync(g->d, pts, (size_t)n * 144, hipMemcpyHostToDevice, c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) {
            zkh_g1_free(g);
            return fail(c, ZKH_EDEV, "point upload failed: %s", hipGetErrorString(e));
        }
    }
    *out = g;
    return ZKH_OK;
}
extern "C" int zkh_g1_to_host(zkh_ctx* c, const zkh_g1* g, uint32_t* pts) {
    if (!c || !g || (!pts && g->n)) return fail(c, ZKH_EARG, "null argument");
    if (!g->n) return ZKH_OK;
    HIPCHK(c, hipMemcpyAsync(pts, g->d, (size_t)g->n * 144, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return ZKH_OK;
}
// the reference's G1Jacobian_generator {G1_generator_x_mont, G1_generator_y_mont, G1_ONE}
// (g1-tensor.cuh:26-63): the standard BLS12-381 G1 generator in Montgomery form, Z = R mod p
extern "C" void zkh_g1_generator(uint32_t* out) {
    static const uint32_t g[36] = {
        4250078230u, 1555269520u, 2574712821u, 2014837863u, 339452353u, 357537223u, 4090554183u,
        4037962445u, 568063040u, 3989728972u, 2651585397u, 302085953u,
        216474225u, 3131872213u, 2031680910u, 2351063834u, 1460086222u, 3713621779u, 1346392468u,
        1370249257u, 2902481344u, 236751935u, 1342743146u, 196886268u,
        196605u, 1980301312u, 3289120770u, 3958636555u, 1405573306u, 1598593111u, 1884444485u,
        2010011731u, 2723605613u, 1543969431u, 4202751123u, 368467651u};
    if (out) memcpy(out, g, sizeof(g));
}
extern "C" int zkh_g1_mul(zkh_ctx* c, const zkh_g1* base, const zkh_tensor* t, zkh_g1** out) {
    if (!c || !base || !t || !out) return fail(c, ZKH_EARG, "null argument");
    *out = nullptr;
    if (!base->n) return fail(c, ZKH_EARG, "g1_mul: empty base");
    HIPCHK(c, hipSetDevice(c->device));
    int rc;
    zkh_g1* o;
    if ((rc = g1_alloc(c, t->n, &o))) return rc;
    if (t->n) {
        DevPlanes p;
        if ((rc = as_planes(c, t, SL_TMP0, &p))) {
            zkh_g1_free(o);
            return rc;
        }
        launch_g1_mul(c->stream, (const uint32_t*)base->d, base->n, p.lo(), p.hi(), t->n, (uint32_t*)o->d);
        hipError_t e = hipGetLastError();
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) {
            zkh_g1_free(o);
            return fail(c, ZKH_EDEV, "g1_mul: %s", hipGetErrorString(e));
        }
    }
    *out = o;
    return ZKH_OK;
}
extern "C" int zkh_g1_addmul(zkh_ctx* c, const zkh_g1* a, const uint32_t sc[8], const zkh_g1* b, zkh_g1** out) {
    if (!c || !a || !sc || !b || !out) return fail(c, ZKH_EARG, "null argument");
    *out = nullptr;
    if (a->n != b->n) return fail(c, ZKH_EARG, "g1_addmul: %u and %u points", a->n, b->n);
    HIPCHK(c, hipSetDevice(c->device));
    int rc;
    zkh_g1* o;
    if ((rc = g1_alloc(c, a->n, &o))) return rc;
    if (a->n) {
        G1Scalar s;
        memcpy(s.v, sc, 32);
        launch_g1_addmul(c->stream, (const uint32_t*)a->d, s, (const uint32_t*)b->d, a->n, (uint32_t*)o->d);
        hipError_t e = hipGetLastError();
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) {
            zkh_g1_free(o);
            return fail(c, ZKH_EDEV, "g1_addmul: %s", hipGetErrorString(e));
        }
    }
    *out = o;
    return ZKH_OK;
}
extern "C" int zkh_commit(zkh_ctx* c, const zkh_g1* gens, const zkh_tensor* t, zkh_g1** out) {
    if (!c || !gens || !t || !out) return fail(c, ZKH_EARG, "null argument");
    *out = nullptr;
    const uint32_t n = gens->n;
    if (!n || t->n % n) return fail(c, ZKH_EARG, "commit: incompatible dimensions");  // commitment.cu:87
    if (n > ZKH_PIP_MAX_GENS) return fail(c, ZKH_EARG, "commit: more than %u generators", ZKH_PIP_MAX_GENS);
    const uint32_t m = t->n / n;
    HIPCHK(c, hipSetDevice(c->device));
    int rc = 0;
    zkh_g1* o;
    if ((rc = g1_alloc(c, m, &o))) return rc;
    if (m) {
        DevPlanes p;
        uint16_t* lists = nullptr;
        uint32_t *offs = nullptr, *buckets = nullptr, *partials = nullptr;
        if (!(rc = as_planes(c, t, SL_TMP0, &p))) lists = (uint16_t*)scratch_slot(c, SL_TMP1, (size_t)m * 64 * n * 2, &rc);
        if (!rc) offs = (uint32_t*)scratch_slot(c, SL_TMP2, (size_t)m * 64 * 16 * 4, &rc);
        if (!rc) buckets = (uint32_t*)scratch_slot(c, SL_TMP3, (size_t)m * 64 * 16 * 144, &rc);
        if (!rc) partials = (uint32_t*)scratch_slot(c, SL_TMP6, (size_t)m * 64 * 144, &rc);
        uint16_t* alias = nullptr;
        if (!rc) alias = (uint16_t*)scratch_slot(c, SL_TMP4, (size_t)m * 64 * 16 * 2, &rc);
        if (rc) {
            zkh_g1_free(o);
            return rc;
        }
        {
            ProfScope ps(c, "pip_sort", (double)m * n * 32);
            launch_pip_sort(c->stream, p.lo(), p.hi(), m, n, lists, offs);
        }
        {
            ProfScope ps(c, "pip_alias", (double)m * 64 * 64);
            launch_pip_alias(c->stream, lists, offs, m, n, alias);
        }
        {
            ProfScope ps(c, "pip_bucket", (double)m * n * 32 + (double)n * 144);
            launch_pip_bucket(c->stream, (const uint32_t*)gens->d, lists, offs, alias, m, n, buckets);
        }
        {
            ProfScope ps(c, "pip_window", (double)m * 64 * 144);
            launch_pip_window(c->stream, buckets, offs, alias, m, partials);
        }
        {
            ProfScope ps(c, "pip_combine", (double)m * 144);
            launch_pip_combine(c->stream, partials, m, (uint32_t*)o->d);
        }
        hipError_t e = hipGetLastError();
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) {
            zkh_g1_free(o);
            return fail(c, ZKH_EDEV, "commit: %s", hipGetErrorString(e));
        }
    }
    *out = o;
    return ZKH_OK;
}

// ---------------------------------------------------------------------------------------
// inner-product argument (ipa_prove, vrf_common.cuh:302-336), continuing the caller's
// transcript; the round points are byte-identical to the reference's (they are absorbed)
// ---------------------------------------------------------------------------------------
extern "C" int zkh_ipa_prove_batch(zkh_ctx* c, uint32_t nj, uint8_t* const* transcripts, const zkh_tensor* const* a,
                                   const zkh_tensor* const* b, const zkh_g1* const* g, const uint32_t* const* Q,
                                   uint32_t* const* L_out, uint32_t* const* R_out, uint32_t* const* a_final) {
    if (!c || !transcripts || !a || !b || !g || !Q || !a_final || !L_out || !R_out) return fail(c, ZKH_EARG, "null argument");
    if (!nj || nj > ZKH_IPA_MAX_JOBS) return fail(c, ZKH_EARG, "ipa_prove_batch: 1 to %d jobs", ZKH_IPA_MAX_JOBS);
    size_t fr_words = 0, g_words = 0, p_words = 0;
    uint32_t nmax = 0;
    for (uint32_t j = 0; j < nj; j++) {
        if (!transcripts[j] || !a[j] || !b[j] || !g[j] || !Q[j] || !a_final[j]) return fail(c, ZKH_EARG, "null argument");
        const uint32_t n = g[j]->n;
        if (!n || (n & (n - 1))) return fail(c, ZKH_EARG, "ipa_prove: n not a power of two");  // vrf_common.cuh:305
        if (a[j]->n != n || b[j]->n != n) return fail(c, ZKH_EARG, "ipa_prove: a, b and g sizes differ");
        if (n > 1 && (!L_out[j] || !R_out[j])) return fail(c, ZKH_EARG, "null argument");
        fr_words += (size_t)n * 32;
        g_words += (size_t)n * 72;
        p_words += (size_t)(n + 2) * 36 + 256;
        nmax = std::max(nmax, n);
    }
    HIPCHK(c, hipSetDevice(c->device));
    int rc = 0;
    // per job: a, b, g working copies (two of each, the fold writes the other), round
    // products P, inner products, Q; one L, R area for all jobs (one copy to the host per round)
    uint32_t* fr_w = (uint32_t*)scratch_slot(c, SL_TMP1, fr_words * 4, &rc);
    uint32_t* g_w = rc ? nullptr : (uint32_t*)scratch_slot(c, SL_TMP2, g_words * 4, &rc);
    uint32_t* p_w = rc ? nullptr : (uint32_t*)scratch_slot(c, SL_TMP3, (p_words + 72 * (size_t)nj) * 4, &rc);
    if (rc) return rc;
    uint32_t* LR = p_w + p_words;
    IpaBatchDev B{};
    uint32_t sz[ZKH_IPA_MAX_JOBS];
    uint32_t *A0[ZKH_IPA_MAX_JOBS], *B0[ZKH_IPA_MAX_JOBS], *G0[ZKH_IPA_MAX_JOBS];
    uint32_t *A1[ZKH_IPA_MAX_JOBS], *B1[ZKH_IPA_MAX_JOBS], *G1[ZKH_IPA_MAX_JOBS];
    size_t of = 0, og = 0, op = 0;
    for (uint32_t j = 0; j < nj; j++) {
        const uint32_t n = g[j]->n;
        IpaJobDev& J = B.j[j];
        uint32_t* a0 = fr_w + of;
        uint32_t* b0 = a0 + 16 * (size_t)n;
        A1[j] = a0 + 8 * (size_t)n;
        B1[j] = b0 + 8 * (size_t)n;
        of += 32 * (size_t)n;
        uint32_t* g0 = g_w + og;
        G1[j] = g0 + 36 * (size_t)n;
        og += 72 * (size_t)n;
        J.P = p_w + op;
        J.ip = J.P + 36 * (size_t)(n + 2);
        uint32_t* Qd = J.ip + 16;
        op += (size_t)(n + 2) * 36 + 256;
        J.LR = LR + 72 * (size_t)j;
        DevPlanes pa, pb;
        if ((rc = as_planes(c, a[j], SL_TMP0, &pa))) return rc;
        launch_planes_to_aos(c->stream, pa.lo(), pa.hi(), n, a0);
        if ((rc = as_planes(c, b[j], SL_TMP0, &pb))) return rc;
        launch_planes_to_aos(c->stream, pb.lo(), pb.hi(), n, b0);
        HIPCHK(c, hipMemcpyAsync(g0, g[j]->d, (size_t)n * 144, hipMemcpyDeviceToDevice, c->stream));
        HIPCHK(c, hipMemcpyAsync(Qd, Q[j], 144, hipMemcpyHostToDevice, c->stream));
        J.a = A0[j] = a0;
        J.b = B0[j] = b0;
        J.g = G0[j] = g0;
        J.Q = Qd;
        sz[j] = n;
    }
    uint32_t r2[8];
    fr_store(kR2, r2);
    std::vector<uint32_t> lr(72 * (size_t)nj);
    for (uint32_t round = 0; (nmax >> round) > 1; round++) {
        uint32_t hmax = 0;
        for (uint32_t j = 0; j < nj; j++) {
            B.j[j].h = sz[j] > 1 ? sz[j] / 2 : 0;
            hmax = std::max(hmax, B.j[j].h);
        }
        {
            ProfScope ps(c, "ipa_msm", 0);
            launch_ipa_ip(c->stream, B, nj, r2);
            launch_ipa_scale(c->stream, B, nj, hmax);
            for (uint32_t shift = 1; (hmax >> shift) >= 1; shift++) launch_ipa_tree(c->stream, B, nj, hmax, shift);
            launch_ipa_lr(c->stream, B, nj);
        }
        HIPCHK(c, hipMemcpyAsync(lr.data(), LR, lr.size() * 4, hipMemcpyDeviceToHost, c->stream));
        HIPCHK(c, hipStreamSynchronize(c->stream));
        for (uint32_t j = 0; j < nj; j++) {
            IpaJobDev& J = B.j[j];
            if (!J.h) continue;
            const uint32_t* l = lr.data() + 72 * (size_t)j;
            tr_absorb(transcripts[j], "L", 1, l, 144);
            tr_absorb(transcripts[j], "R", 1, l + 36, 144);
            const Fr x = tr_challenge(transcripts[j]), xi = fr_inv(x);
            fr_store(x, J.x);
            fr_store(xi, J.xi);
            fr_store(fr_to_mont(x), J.xm);
            fr_store(fr_to_mont(xi), J.xim);
            J.g2 = G1[j];
            J.a2 = A1[j];
            J.b2 = B1[j];
            memcpy(L_out[j] + 36 * (size_t)round, l, 144);
            memcpy(R_out[j] + 36 * (size_t)round, l + 36, 144);
        }
        {
            ProfScope ps(c, "ipa_fold", 0);
            launch_ipa_fold(c->stream, B, nj, hmax);
        }
        for (uint32_t j = 0; j < nj; j++) {
            IpaJobDev& J = B.j[j];
            if (!J.h) continue;
            std::swap(G0[j], G1[j]);  // the next round's fold writes the buffers just read
            std::swap(A0[j], A1[j]);
            std::swap(B0[j], B1[j]);
            J.g = G0[j];
            J.a = A0[j];
            J.b = B0[j];
            sz[j] /= 2;
        }
    }
    for (uint32_t j = 0; j < nj; j++) HIPCHK(c, hipMemcpyAsync(a_final[j], B.j[j].a, 32, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    HIPCHK(c, hipGetLastError());
    return ZKH_OK;
}
extern "C" int zkh_ipa_prove(zkh_ctx* c, uint8_t* transcript, const zkh_tensor* a, const zkh_tensor* b,
                             const zkh_g1* g, const uint32_t* Q, uint32_t* L_out, uint32_t* R_out,
                             uint32_t* a_final) {
    if (!c || !transcript || !a || !b || !g || !Q || !a_final) return fail(c, ZKH_EARG, "null argument");
    uint32_t lr_unused[1];
    uint32_t* L = L_out ? L_out : lr_unused;
    uint32_t* R = R_out ? R_out : lr_unused;
    if (g->n > 1 && (!L_out || !R_out)) return fail(c, ZKH_EARG, "null argument");
    return zkh_ipa_prove_batch(c, 1, &transcript, &a, &b, &g, &Q, &L, &R, &a_final);
}

// ---------------------------------------------------------------------------------------
// Hadamard sumcheck (zkob_lookup.cuh:267-315)
// ---------------------------------------------------------------------------------------
// p(v) of the cubic through (t, e[t]), t = 0..3, for vm = to_m(v): Newton differences,
// p(v) = e0 + v (d1 + (v - 1) (dd1 / 2 + (v - 2) ddd / 6))
static Fr lagrange4_m(const Fr e[4], const Fr& vm) {
    static const Fr inv6_m = to_m(fr_inv(fr_u64(6))), one_m = fr_one_m(), two_m = to_m(fr_u64(2));
    const Fr d1 = fr_sub(e[1], e[0]), d2 = fr_sub(e[2], e[1]), d3 = fr_sub(e[3], e[2]);
    const Fr dd1 = fr_sub(d2, d1), ddd = fr_sub(fr_sub(d3, d2), dd1);
    Fr t = fr_add(fr_half(dd1), mulm(mulm(ddd, inv6_m), fr_sub(vm, two_m)));
    t = fr_add(d1, mulm(t, fr_sub(vm, one_m)));
    return fr_add(e[0], mulm(t, vm));
}
// Rounds r0 .. k-1 of a Hadamard sumcheck in one persistent launch (see HpPersist) once the
// tables have sz <= ZKH_HP_PERSIST_MAX entries: one host round trip per round instead of a
// launch; the block-count rounds at the end run on the host.  The per-round host logic is
// hp_common's: e[t] = sums_t * cE * corr(K) * eq(u_last, t) with the eq weights (u given),
// e[t] = sums_t with an explicit E table (e_src given, u null); then the claim check, the
// absorbs "hp0".."hp3" and the challenge.
#define ZKH_HP_PERSIST_MAX 8192u
// mode as in lu_persist_rounds (1: launch only, behind a relay queued here and held by *rg)
static int hp_persist_rounds(zkh_ctx* c, uint8_t tr[32], const std::vector<Fr>* u, const EqState& eq, uint32_t k,
                             uint32_t r0, uint32_t sz, int fold, DevPlanes e_src, DevPlanes s_src, DevPlanes u_src,
                             bool u_ones, const uint32_t vm[8], RelayGuard* rg, Fr& claim, Fr& cE,
                             uint32_t* ev_out, uint32_t* ws_out, Fr& e_fin, Fr& s_fin, Fr& u_fin, int mode) {
    const bool em = u == nullptr;  // explicit E table
    static const char* lab[4] = {"hp0", "hp1", "hp2", "hp3"};
    const uint32_t lgnb = sz > ZKH_LH_PLS ? ceil_log2(sz / ZKH_LH_PLS) : 0, nb = 1u << lgnb;
    const uint32_t R = ceil_log2(sz) - lgnb;  // local rounds
    int rc;
    if ((rc = ensure_ps(c, (size_t)ZKH_PSLOT * (nb + 2)))) return rc;
    uint32_t* ps = c->ps_host;
    uint32_t* slots = ps + ZKH_PSLOT;
    uint32_t* cmd = ps + (size_t)ZKH_PSLOT * (nb + 1);
    if (mode != 2) memset(ps, 0, (size_t)ZKH_PSLOT * (nb + 2) * 4);
    HpPersist P{};
    P.s_lo = s_src.lo();
    P.s_hi = s_src.hi();
    P.u_lo = u_src.lo();
    P.u_hi = u_src.hi();
    P.e_lo = em ? e_src.lo() : nullptr;
    P.e_hi = em ? e_src.hi() : nullptr;
    P.elo = eq.elo_d;
    P.ehi = eq.ehi_d;
    P.out = slots;
    P.cmd = cmd;
    P.err = ps;
    P.deadline = c->clock_khz * 1000 * 20;  // 20 s without a command
    if (vm) memcpy(P.vm.v, vm, 32);
    if (mode == 1) {
        rg->pending = relay_enqueue(c);
        P.vmp = c->relay_vm;
    }
    P.n = sz;
    P.lgnb = lgnb;
    P.fold = fold ? 1 : 0;
    // two rounds per message while a block holds >= 4 entries: the product is then of degree
    // 2 in each variable (eq mode, or an E table with U all ones)
    P.two = (!em || u_ones) && !getenv("ZKH_PERSIST_ONE") ? 1 : 0;
    auto send = [&](uint32_t seq, const uint32_t* xm, uint32_t nw) {
        for (uint32_t i = 0; i < nw && xm; i++) __atomic_store_n(cmd + zkh_quad_word(i), xm[i], __ATOMIC_RELAXED);
        for (uint32_t qd = 0; qd < zkh_quad_count(nw); qd++) __atomic_store_n(cmd + 4 * qd, seq, __ATOMIC_RELEASE);
    };
    auto quit = [&]() {
        send(ZKH_QUIT, nullptr, 32);
        (void)hipStreamSynchronize(c->stream);
    };
    if (mode != 2) {
        ProfScope ps_(c, "hp_persist", (double)sz * (em ? 3 : 2) * 32 * (fold ? 3 : 1));
        hipError_t e = launch_hp_persist(c->stream, P);
        if (e != hipSuccess) {
            quit();
            return fail(c, ZKH_EDEV, "persistent hadamard launch: %s", hipGetErrorString(e));
        }
        if (mode == 1) return 0;
    }
    const double t_launch = now_us();
    auto slot_fr = [&](uint32_t b, uint32_t i) {
        uint32_t v[8];
        for (uint32_t j = 0; j < 8; j++) v[j] = slots[(size_t)b * ZKH_PSLOT + zkh_quad_word(8 * i + j)];
        return fr_load(v);
    };
    // every block has published message seq (nw words); device errors, a block's
    // deadline and an ended kernel stop the wait
    auto wait_msg = [&](uint32_t seq, uint32_t nw) -> int {
        const uint32_t nq = zkh_quad_count(nw);
        const double t0 = now_us();
        for (uint64_t spins = 1;; spins++) {
            bool all = true;
            for (uint32_t b = 0; b < nb && all; b++)
                for (uint32_t qd = 0; qd < nq; qd++)
                    if (__atomic_load_n(slots + (size_t)b * ZKH_PSLOT + 4 * qd, __ATOMIC_ACQUIRE) != seq) {
                        all = false;
                        break;
                    }
            if (all) return 0;
            spin_pause(spins);
            if ((spins & 0x3FFF) == 0) {
                hipError_t e = hipStreamQuery(c->stream);
                if (e != hipSuccess && e != hipErrorNotReady) {
                    quit();
                    return fail(c, ZKH_EDEV, "persistent hadamard rounds: %s", hipGetErrorString(e));
                }
                if (__atomic_load_n(ps, __ATOMIC_ACQUIRE) || e == hipSuccess || now_us() - t0 > 30e6) {
                    quit();
                    return fail(c, ZKH_EDEV, "persistent hadamard rounds stopped (%s)",
                                ps[0] ? "a block timed out" : e == hipSuccess ? "kernel ended early" : "no progress");
                }
            }
        }
    };
    // one round from its sums at t = 0..3; w_m receives to_m(w)
    auto host_round = [&](uint32_t r, const Fr sums[4], bool device, Fr& w, Fr& w_m) -> bool {
        const uint32_t K = k - r - 1;
        const Fr ul = em ? kZero : (*u)[k - r - 1];
        Fr e[4];
        if (em) {
            for (int t = 0; t < 4; t++) e[t] = device ? fix2(sums[t]) : sums[t];
        } else {
            // e[t] = sums_t (x 2^256 from the device) f eq(ul, t), f = cE corr(K), eq(ul, t) =
            // (1 - ul) + t (2 ul - 1): the factors f (1 - ul) and f (2 ul - 1) prepared once
            // f 2^512 for device sums (they carry 2^-256), else f 2^256
            const Fr f_m = device ? mulm(to_mm(cE), to_m(eq_corr(eq, K))) : to_m(cE);
            const Fr f0 = mulm(f_m, to_m(fr_sub(kOne, ul))), fd = mulm(f_m, to_m(fr_sub(fr_add(ul, ul), kOne)));
            Fr ft = f0;
            for (int t = 0; t < 4; t++) {
                e[t] = mulm(sums[t], ft);
                ft = fr_add(ft, fd);
            }
        }
        if (!fr_eq(claim, fr_add(e[0], e[1]))) return false;
        for (int t = 0; t < 4; t++) {
            tr_absorb_fr(tr, lab[t], e[t]);
            if (ev_out) fr_store(e[t], ev_out + 8 * (4 * r + t));
        }
        w = tr_challenge(tr);
        if (ws_out) fr_store(w, ws_out + 8 * r);
        w_m = to_m(w);
        claim = lagrange4_m(e, w_m);
        if (!em) {
            const Fr uw = mulm(ul, w_m);
            cE = mulm(cE, to_m(fr_add(fr_sub(fr_add(uw, uw), fr_add(ul, w)), kOne)));  // cE eq(ul, w)
        }
        return true;
    };
    const bool tracing = trace_on();
    std::vector<double> tr_h;  // per message: sums seen, command sent
    uint32_t seq = 1;
    for (uint32_t lr = 0; lr < R; seq++) {
        const uint32_t r1 = r0 + lr;
        if (!P.two || R - lr < 2) {  // one round
            if ((rc = wait_msg(seq, ZKH_HP_MSG))) return rc;
            if (tracing) tr_h.push_back(now_us());
            Fr sums[4] = {kZero, kZero, kZero, kZero};
            for (uint32_t b = 0; b < nb; b++)
                for (int t = 0; t < 4; t++) sums[t] = fr_add(sums[t], slot_fr(b, t));
            Fr w, w_m;
            if (!host_round(r1, sums, true, w, w_m)) {
                quit();
                return fail(c, ZKH_EROUND, "hadamard round inconsistency (witness bug) at round %u", r1);
            }
            uint32_t xm[8];
            fr_store(w_m, xm);
            send(seq, xm, 8);
            if (tracing) tr_h.push_back(now_us());
            lr++;
            continue;
        }
        // two rounds from the nine point sums G[3 a + b] (a: the first variable y1, b: the
        // second y2; 0, 1, inf): round r1's sums at t, over the pairs (c + y2 q, c + y2 q +
        // 2q) of its table, are G(t, 0) + rho G(t, 1), rho = u/(1 - u) of y2 relative to the
        // cell weight (eq mode; 1 with E); round r1 + 1's are G(w1, t)
        if ((rc = wait_msg(seq, ZKH_HP_MSG2))) return rc;
        if (tracing) tr_h.push_back(now_us());
        Fr G[9];
        for (int p = 0; p < 9; p++) G[p] = kZero;
        for (uint32_t b = 0; b < nb; b++)
            for (int p = 0; p < 9; p++) G[p] = fr_add(G[p], slot_fr(b, p));
        Fr rho_m = fr_one_m();
        if (!em) {
            const uint32_t K2 = k - r1 - 2;  // eq coordinate of y2
            rho_m = mulm(to_m((*u)[K2]), to_m(eq.inv1mu[K2]));
        }
        // E mode: the device sums carry one 2^-256 (E S, U = 1), so they go in as exact values
        auto val = [&](const Fr& x) { return em ? fix1(x) : x; };
        // a quadratic piece (q(0), q(1), t^2 coefficient) at t = 0..3, by additions
        auto at0123 = [](const Fr& q0, const Fr& q1, const Fr& c2, Fr out[4]) {
            const Fr cq[4] = {q0, fr_sub(fr_sub(q1, q0), c2), c2, kZero};
            cubic_at123(cq, out);
        };
        Fr sums[4], w1, w2, w1_m, w2_m, X[4], Y[4];
        at0123(G[0], G[3], G[6], X);
        at0123(G[1], G[4], G[7], Y);
        for (int t = 0; t < 4; t++) sums[t] = val(fr_add(X[t], mulm(Y[t], rho_m)));
        if (!host_round(r1, sums, !em, w1, w1_m)) {
            quit();
            return fail(c, ZKH_EROUND, "hadamard round inconsistency (witness bug) at round %u", r1);
        }
        Fr H[3];
        for (int b = 0; b < 3; b++) H[b] = quad_at_m(G[b], G[3 + b], G[6 + b], w1_m);
        at0123(H[0], H[1], H[2], X);
        for (int t = 0; t < 4; t++) sums[t] = val(X[t]);
        if (!host_round(r1 + 1, sums, !em, w2, w2_m)) {
            quit();
            return fail(c, ZKH_EROUND, "hadamard round inconsistency (witness bug) at round %u", r1 + 1);
        }
        // double fold weights of T[c + (2 y1 + y2) q], in Montgomery form: (1 - w)_m = 1_m - w_m
        const Fr a1_m = fr_sub(fr_one_m(), w1_m), a2_m = fr_sub(fr_one_m(), w2_m);
        const Fr Lw_m[4] = {mulm(a1_m, a2_m), mulm(a1_m, w2_m), mulm(w1_m, a2_m), mulm(w1_m, w2_m)};
        uint32_t xm[32];
        for (int j = 0; j < 4; j++) fr_store(Lw_m[j], xm + 8 * j);
        send(seq, xm, 32);
        if (tracing) tr_h.push_back(now_us());
        lr += 2;
    }
    if ((rc = wait_msg(seq, em ? 24 : 16))) return rc;
    std::vector<Fr> ta(nb), tb(nb), te(em ? nb : 0);
    for (uint32_t b = 0; b < nb; b++) {
        ta[b] = slot_fr(b, 0);
        tb[b] = slot_fr(b, 1);
        if (em) te[b] = slot_fr(b, 2);
    }
    // (no wait for the blocks to exit: none touches the slots after its last message, and
    // later work on the stream is ordered behind the kernel; tracing reads the clock stamps)
    if (tracing) HIPCHK(c, hipStreamSynchronize(c->stream));
    // the last lgnb rounds over the blocks' entries (entry b is global index b)
    for (uint32_t r = r0 + R, m = nb; m > 1; r++, m >>= 1) {
        const uint32_t h = m >> 1, K = k - r - 1;
        Fr sums[4] = {kZero, kZero, kZero, kZero};
        std::vector<Fr> wl;
        if (!em) eq_low_weights(*u, K, h, wl);
        for (uint32_t i = 0; i < h; i++) {
            // w_t S_t U_t with w_t and U_t in Montgomery form (both linear in t: to_m is linear)
            Fr w_m = em ? to_m(te[i]) : to_m(wl[i]), ut_m = to_m(tb[i]);
            const Fr dw_m = em ? to_m(fr_sub(te[i + h], te[i])) : kZero, du_m = to_m(fr_sub(tb[i + h], tb[i]));
            const Fr ds = fr_sub(ta[i + h], ta[i]);
            Fr st = ta[i];
            for (int t = 0; t < 4; t++) {
                sums[t] = fr_add(sums[t], mulm(mulm(st, w_m), ut_m));
                st = fr_add(st, ds);
                ut_m = fr_add(ut_m, du_m);
                w_m = fr_add(w_m, dw_m);
            }
        }
        Fr w, w_m;
        if (!host_round(r, sums, false, w, w_m))
            return fail(c, ZKH_EROUND, "hadamard round inconsistency (witness bug) at round %u", r);
        for (uint32_t i = 0; i < h; i++) {
            ta[i] = fr_add(ta[i], mulm(fr_sub(ta[i + h], ta[i]), w_m));
            tb[i] = fr_add(tb[i], mulm(fr_sub(tb[i + h], tb[i]), w_m));
            if (em) te[i] = fr_add(te[i], mulm(fr_sub(te[i + h], te[i]), w_m));
        }
    }
    s_fin = ta[0];
    u_fin = tb[0];
    e_fin = em ? te[0] : cE;
    if (tracing) {
        fprintf(stderr, "[zkh] hp persistent loop: n=%u, %u blocks, %u device + %u host rounds in %.1f us\n", sz, nb, R,
                lgnb, now_us() - t_launch);
        trace_persist(c, "hp", slots, seq, tr_h);
    }
    return 0;
}
// sum_i E[i] S[i] U[i] by the elementwise products and a sum (zkob_rope.cu:232)
static int explicit_claim(zkh_ctx* c, const zkh_tensor* E, const zkh_tensor* S, const zkh_tensor* U, Fr* out) {
    zkh_tensor *su = nullptr, *esu = nullptr;
    uint32_t o[8];
    int rc = zkh_hadamard(c, S, U, &su);
    if (!rc) rc = zkh_hadamard(c, E, su, &esu);
    if (!rc) rc = zkh_sum(c, esu, o);
    if (su) zkh_tensor_free(su);
    if (esu) zkh_tensor_free(esu);
    if (!rc) *out = fr_load(o);
    return rc;
}
// claim_label: the claim is not given but is sum E[i] S[i] U[i] (E = eq(i, u) in the eq
// form), taken from the first round's sums (q(0) + q(1) of the round's polynomial in t, which
// the check below compares with the claim) and absorbed under that label before the first
// round's evaluations; claim_out receives it
static int hp_common(zkh_ctx* c, uint8_t tr[32], const uint32_t claim_l[8], const zkh_tensor* E,
                     const std::vector<Fr>* ueq, const zkh_tensor* S, const zkh_tensor* U,
                     uint32_t* ev_out, uint32_t* term_out, uint32_t* ws_out, const char* claim_label = nullptr,
                     uint32_t* claim_out = nullptr) {
    const uint32_t n = S->n;
    if (!n || (n & (n - 1)) || U->n != n || (E && E->n != n))
        return fail(c, ZKH_EARG, "hadamard tables must share a power-of-two size");
    if (ueq && ((uint64_t)1 << ueq->size()) != n) return fail(c, ZKH_EARG, "eq size mismatch");
    if (claim_label && !claim_out) return fail(c, ZKH_EARG, "null argument");
    if (!claim_label && !fr_is_canonical(claim_l)) return fail(c, ZKH_EARG, "non-canonical claim");
    HIPCHK(c, hipSetDevice(c->device));
    const uint32_t k = ceil_log2(n);
    int rc = 0;
    // int32 S and U of the eq form (SwiGLU's mapped S and int16-range U) are read as int32 by
    // the round kernels up to their first fold when the first two rounds are round kernels,
    // not the persistent loop; otherwise as planes
    const bool big = (n >> 1) > ZKH_HP_PERSIST_MAX;
    // U all ones (an I32 tensor measured so at ingest: the RoPE obligations' U = 1) with an
    // explicit E: the per-round kernels skip U, whose folds stay all ones in its source
    const bool u_ones = !ueq && U->kind == ZKH_KIND_I32 && U->ones;
    // with U all ones and an int32 S, the first round's sums are exact (x 1): 32-bit multiplies
    const bool s_int = u_ones && S->kind == ZKH_KIND_I32;
    const bool s_i32 = (ueq || u_ones) && big && S->kind == ZKH_KIND_I32 && !S->weights;
    const bool u_i32 = ueq && big && U->kind == ZKH_KIND_I32 && !U->weights;
    DevPlanes Ec{}, Sc{}, Uc{};
    if (E && (rc = as_planes(c, E, SL_TMP0, &Ec))) return rc;
    if (!s_i32 && (rc = as_planes(c, S, SL_TMP1, &Sc))) return rc;
    if (u_ones) {
        // only the persistent loop and the last fold read U (as ones, whatever its folds):
        // entries below 2 ZKH_HP_PERSIST_MAX suffice
        Uc = scratch_planes(c, SL_TMP2, n, &rc);
        if (rc) return rc;
        launch_i32_to_planes(c->stream, (const int32_t*)U->d, std::min<uint32_t>(n, 2 * ZKH_HP_PERSIST_MAX), Uc);
    } else if (!u_i32 && (rc = as_planes(c, U, SL_TMP2, &Uc))) {
        return rc;
    }
    const int32_t* s32 = s_i32 ? (const int32_t*)S->d : nullptr;  // the sources while unfolded
    const int32_t* u32 = u_i32 ? (const int32_t*)U->d : nullptr;
    DevPlanes Ew{}, Sw, Uw;
    if (E) {
        Ew = E->kind == ZKH_KIND_FR ? scratch_planes(c, SL_TMP0, n / 2 + 1, &rc) : Ec;
        if (rc) return rc;
    }
    Sw = S->kind == ZKH_KIND_FR || s_i32 ? scratch_planes(c, SL_TMP1, n / 2 + 1, &rc) : Sc;
    if (rc) return rc;
    Uw = U->kind == ZKH_KIND_FR || u_i32 ? scratch_planes(c, SL_TMP2, n / 2 + 1, &rc) : Uc;
    if (rc) return rc;
    EqState eq;  // tables now, the host part once the first round is queued
    if (ueq && (rc = eq_setup(c, *ueq, eq, true, false))) return rc;
    Fr claim = claim_label ? kZero : fr_load(claim_l), cE = kOne;
    DevPlanes e_src = Ec, s_src = Sc, u_src = Uc;
    uint32_t vm[8] = {0};
    static const char* lab[4] = {"hp0", "hp1", "hp2", "hp3"};
    const bool tracing = trace_on();
    std::vector<double> tr_t;  // per round: launch, sums seen, challenge done (host clock)
    bool persisted = false;    // the last rounds ran in hp_persist_rounds
    bool persist_queued = false;  // ... launched behind the previous round's relay
    Fr e_fin = kZero, s_fin = kZero, u_fin = kZero;
    const bool no_persist = getenv("ZKH_NO_PERSIST") != nullptr;
    auto persists = [&](uint32_t r) { return (n >> r) <= ZKH_HP_PERSIST_MAX && !no_persist; };
    // from the first round kernel's sums (a one-entry table has no round: the sum first)
    const bool derive_claim = claim_label && k > 0 && !persists(0);
    if (claim_label && !derive_claim) {  // all rounds in the persistent loop: the sum first
        // (a table this small is never read as int32, so Sc and Uc hold its planes)
        if ((rc = ueq ? eq_weighted_sum(c, Sc, &Uc, n, *ueq, &claim) : explicit_claim(c, E, S, U, &claim)))
            return rc;
        tr_absorb_fr(tr, claim_label, claim);
    }
    if (claim_label) fr_store(claim, claim_out);
    // A folding round leaves its sum at 1 to the host: claim - p(0) for an explicit E; with
    // the eq form, from the inner claim I = sum eq S U over the remaining variables (the
    // running claim without the eq factor cE) as (I - (1 - u) q(0)) / u, unless u is 0.
    Fr I = claim;
    std::vector<Fr> inv_u;  // 1/u_j, computed while the first round runs
    struct Launched {
        Publish pb;
        bool dv;
    };
    // launches round r (previous challenge from vm, or from the relay when vmp is given) and
    // moves the table handles to the folded copies the launch writes
    auto launch = [&](uint32_t r, const uint32_t* vmp) {
        const uint32_t sz = n >> r;
        const int fold = r > 0;
        // a folding round derives its sum at 1 unless its eq coordinate is 0, or ZKH_XCHECK=1
        // asks for every round's p(0) + p(1) = claim on device sums (zkob_lookup.cuh:303)
        Launched l{make_pub(c, 1), fold && !xcheck_on() && (!ueq || !fr_eq((*ueq)[k - r - 1], kZero))};
        if (u_ones) {
            ProfScope ps(c, "hp_round", (fold ? 3.0 * sz : (double)sz) * 2 * 32);
            launch_hp_round_ones(c->stream, Tab{e_src, Ew}, Tab{s_src, Sw}, sz, fold, vm, vmp, l.pb, l.dv, s_int,
                                 s32);
        } else if (!ueq) {
            ProfScope ps(c, "hp_round", (fold ? 3.0 * sz : (double)sz) * 3 * 32);
            launch_hp_round(c->stream, Tab{e_src, Ew}, Tab{s_src, Sw}, Tab{u_src, Uw}, sz, fold, vm, vmp, l.pb, l.dv);
        } else {
            // S and U read as int32 (4 bytes) until their first fold writes their planes
            auto tab_bytes = [&](bool i32) {
                return !i32 ? (fold ? 3.0 * sz : (double)sz) * 32 : fold ? 2.0 * sz * 4 + (double)sz * 32 : (double)sz * 4;
            };
            ProfScope ps(c, "hp_eq_round", tab_bytes(s32 != nullptr) + tab_bytes(u32 != nullptr));
            launch_hp_eq_round(c->stream, Tab{s_src, Sw}, Tab{u_src, Uw}, sz, fold, vm, vmp,
                               EqW{eq.elo_d, eq.ehi_d, k - r - 1}, l.pb, l.dv, s32, u32);
        }
        if (fold) {
            e_src = Ew;
            s_src = Sw;
            if (!u_ones) u_src = Uw;
            s32 = u32 = nullptr;
        }
        return l;
    };
    RelayGuard relay{c};
    Launched cur{};
    bool launched = false;  // round r is already queued
    for (uint32_t r = 0; r < k; r++) {
        const uint32_t sz = n >> r;
        const int fold = r > 0;
        if (persists(r)) {  // the rest in one launch
            if (s32 || u32) return fail(c, ZKH_EDEV, "internal: unfolded int32 table at the persistent loop");
            if (ueq && (rc = eq_setup_host(c, *ueq, eq))) return rc;
            if ((rc = hp_persist_rounds(c, tr, ueq, eq, k, r, sz, fold, e_src, s_src, u_src, u_ones, vm, nullptr, claim,
                                        cE, ev_out, ws_out, e_fin, s_fin, u_fin, persist_queued ? 2 : 0)))
                return rc;
            persisted = true;
            break;
        }
        if (tracing) tr_t.push_back(now_us());
        if (!launched) cur = launch(r, nullptr);
        // round r + 1 (or the persistent loop) goes behind a relay now, so that its launch
        // overlaps this round
        const bool relay_next = r + 1 < k && !persists(r + 1);
        const bool persist_next = r + 1 < k && persists(r + 1) && !s32 && !u32;
        Launched next{};
        if (relay_next) {
            relay.pending = relay_enqueue(c);
            next = launch(r + 1, c->relay_vm);
        } else if (persist_next) {
            Fr claim0 = claim, cE0 = cE, ef, sf, uf;  // (launch only: not read)
            if ((rc = hp_persist_rounds(c, tr, ueq, eq, k, r + 1, n >> (r + 1), 1, e_src, s_src, u_src, u_ones, nullptr,
                                        &relay, claim0, cE0, nullptr, nullptr, ef, sf, uf, 1)))
                return rc;
            persist_queued = true;
        }
        if (ueq && (rc = eq_setup_host(c, *ueq, eq))) return rc;  // once, behind the first launches
        if (r == 0 && ueq && k > 1) {  // 1/u_j for the rounds that derive (batch inverse, host)
            inv_u.assign(k, kZero);
            std::vector<Fr> pre(k + 1, kOne);
            for (uint32_t j = 0; j < k; j++) pre[j + 1] = fr_eq((*ueq)[j], kZero) ? pre[j] : fr_mul(pre[j], (*ueq)[j]);
            Fr t = fr_inv(pre[k]);
            for (uint32_t j = k; j-- > 0;)
                if (!fr_eq((*ueq)[j], kZero)) {
                    inv_u[j] = fr_mul(t, pre[j]);
                    t = fr_mul(t, (*ueq)[j]);
                }
        }
        Fr e[4], sums[4];
        if ((rc = wait_pub(c, cur.pb.seq))) return rc;
        if (tracing) tr_t.push_back(now_us());
        Fr st_true[3];  // eq form: the inner sum's q(0), q(1) and t^2 coefficient
        if (u_ones) {  // E_t S_t = c0 + c1 t + c2 t^2 from sum e0s0, e1s1, de*ds
            Fr c0, c2, q1;
            if (cur.dv) {
                pub_read(c, 0, 2, sums);
                c0 = fix1(sums[0]);
                c2 = fix1(sums[1]);
                q1 = fr_sub(claim, c0);
            } else {
                pub_read(c, 0, 3, sums);
                auto unfix = [&](const Fr& x) { return !fold && s_int ? x : fix1(x); };
                c0 = unfix(sums[0]);
                c2 = unfix(sums[2]);
                q1 = unfix(sums[1]);
            }
            const Fr cq[4] = {c0, fr_sub(fr_sub(q1, c0), c2), c2, kZero};
            cubic_at123(cq, e);
        } else if (!ueq) {
            if (cur.dv) {
                pub_read(c, 0, 3, sums);
                e[0] = fix2(sums[0]);
                e[1] = fr_sub(claim, e[0]);
                e[2] = fix2(sums[1]);
                e[3] = fix2(sums[2]);
            } else {
                pub_read(c, 0, 4, sums);
                for (int t = 0; t < 4; t++) e[t] = fix2(sums[t]);
            }
        } else {  // sum_t = c0 + c1 t + c2 t^2 from sum w s0u0, w s1u1, w ds du (x 2^256 in round 0)
            const uint32_t K = k - r - 1;
            const Fr ul = (*ueq)[k - r - 1];
            const Fr corr = eq_corr(eq, K);
            const Fr cm = fold ? to_mm(corr) : corr;  // fix1 (or from_mont) and corr in one product
            auto unfix = [&](const Fr& x) { return mulm(x, cm); };
            const Fr e0_m = to_m(fr_sub(kOne, ul)), e1_m = to_m(fr_sub(fr_add(ul, ul), kOne));
            if (cur.dv) {
                pub_read(c, 0, 2, sums);
                st_true[0] = unfix(sums[0]);
                st_true[2] = unfix(sums[1]);
                // q(1) = (I - (1 - ul) q(0)) / ul
                st_true[1] = mulm(fr_sub(I, mulm(st_true[0], e0_m)), to_m(inv_u[k - r - 1]));
            } else {
                pub_read(c, 0, 3, sums);
                st_true[0] = unfix(sums[0]);
                st_true[1] = unfix(sums[1]);
                st_true[2] = unfix(sums[2]);
            }
            const Fr cq[4] = {st_true[0], fr_sub(fr_sub(st_true[1], st_true[0]), st_true[2]), st_true[2], kZero};
            Fr st[4];
            cubic_at123(cq, st);
            // e[t] = st_t cE eq(ul, t), eq(ul, t) = (1 - ul) + t (2 ul - 1): the factors cE (1 - ul)
            // and cE (2 ul - 1) in Montgomery form, then one product per t
            const Fr cE_m = to_m(cE), f0 = mulm(cE_m, e0_m), fd = mulm(cE_m, e1_m);
            Fr ft = f0;
            for (int t = 0; t < 4; t++) {
                e[t] = mulm(st[t], ft);
                ft = fr_add(ft, fd);
            }
        }
        if (r == 0 && derive_claim) {
            claim = I = fr_add(e[0], e[1]);
            tr_absorb_fr(tr, claim_label, claim);
            fr_store(claim, claim_out);
        }
        if (!fr_eq(claim, fr_add(e[0], e[1])))
            return fail(c, ZKH_EROUND, "hadamard round inconsistency (witness bug) at round %u", r);
        for (int t = 0; t < 4; t++) {
            tr_absorb_fr(tr, lab[t], e[t]);
            if (ev_out) fr_store(e[t], ev_out + 8 * (4 * r + t));
        }
        Fr w = tr_challenge(tr);
        if (ws_out) fr_store(w, ws_out + 8 * r);
        const Fr w_m = to_m(w);
        fr_store(w_m, vm);
        if (relay_next || persist_next) {  // the queued launch starts now; the state updates overlap it
            relay_send(c, relay.pending, vm);
            relay.pending = 0;
            if (relay_next) cur = next;
        }
        claim = lagrange4_m(e, w_m);
        if (ueq) {
            const Fr ul = (*ueq)[k - r - 1], uw = mulm(ul, w_m);
            cE = mulm(cE, to_m(fr_add(fr_sub(fr_add(uw, uw), fr_add(ul, w)), kOne)));  // cE eq(ul, w)
            I = quad_at_m(st_true[0], st_true[1], st_true[2], w_m);
        }
        launched = relay_next;
        if (tracing) tr_t.push_back(now_us());
    }
    if (tracing) {  // per round: table size, launch -> sums seen, host work (us)
        fprintf(stderr, "[zkh] hp rounds (n: device/host us)%s:", persisted ? ", then the persistent loop" : "");
        for (uint32_t r = 0; r < tr_t.size() / 3; r++)
            fprintf(stderr, " %u:%.1f/%.1f", n >> r, tr_t[3 * r + 1] - tr_t[3 * r], tr_t[3 * r + 2] - tr_t[3 * r + 1]);
        fprintf(stderr, "\n");
    }
    uint32_t tv[3][8];
    if (persisted) {
        fr_store(s_fin, tv[0]);
        fr_store(u_fin, tv[1]);
        fr_store(e_fin, tv[2]);
    } else {
        if (s32 || u32) return fail(c, ZKH_EDEV, "internal: unfolded int32 table at the last fold");
        if (k > 0) {
            if (!ueq) launch_fold(c->stream, Tab{e_src, Ew}, 1, vm);
            launch_fold(c->stream, Tab{s_src, Sw}, 1, vm);
            launch_fold(c->stream, Tab{u_src, Uw}, 1, vm);
            e_src = Ew;
            s_src = Sw;
            u_src = Uw;
        }
        HIPCHK(c, hipMemcpyAsync(tv[0], s_src.lo(), 16, hipMemcpyDeviceToHost, c->stream));
        HIPCHK(c, hipMemcpyAsync(tv[0] + 4, s_src.hi(), 16, hipMemcpyDeviceToHost, c->stream));
        HIPCHK(c, hipMemcpyAsync(tv[1], u_src.lo(), 16, hipMemcpyDeviceToHost, c->stream));
        HIPCHK(c, hipMemcpyAsync(tv[1] + 4, u_src.hi(), 16, hipMemcpyDeviceToHost, c->stream));
        if (!ueq) {
            HIPCHK(c, hipMemcpyAsync(tv[2], e_src.lo(), 16, hipMemcpyDeviceToHost, c->stream));
            HIPCHK(c, hipMemcpyAsync(tv[2] + 4, e_src.hi(), 16, hipMemcpyDeviceToHost, c->stream));
        } else {
            fr_store(cE, tv[2]);
        }
        HIPCHK(c, hipStreamSynchronize(c->stream));
    }
    // terminal: cur = E_f * S_f2 * U_f2 (zkob_rope.cu:29)
    if (!fr_eq(claim, fr_mul(fr_mul(fr_load(tv[2]), fr_load(tv[0])), fr_load(tv[1]))))
        return fail(c, ZKH_EROUND, "hadamard terminal mismatch (witness bug)");
    if (term_out) memcpy(term_out, tv, sizeof(tv));
    return ZKH_OK;
}
// hp_common with the ZKH_XCHECK guards of zkob_glu.cu:254-260 / zkob_rope.cu:240-246: S_f2
// and U_f2 (and E_f) against the MLEs of S, U (and E, or the eq polynomial) at the point
static int hp_checked(zkh_ctx* c, uint8_t tr[32], const uint32_t claim[8], const zkh_tensor* E,
                      const std::vector<Fr>* ueq, const zkh_tensor* S, const zkh_tensor* U, uint32_t* ev_out,
                      uint32_t* term_out, uint32_t* ws_out, const char* claim_label = nullptr,
                      uint32_t* claim_out = nullptr) {
    if (!xcheck_on() || !S)
        return hp_common(c, tr, claim, E, ueq, S, U, ev_out, term_out, ws_out, claim_label, claim_out);
    const uint32_t k = ceil_log2(S->n);
    std::vector<uint32_t> wsb(8 * (size_t)std::max<uint32_t>(k, 1)), tb(24);
    uint32_t* ws = ws_out ? ws_out : wsb.data();
    uint32_t* term = term_out ? term_out : tb.data();
    int rc = hp_common(c, tr, claim, E, ueq, S, U, ev_out, term, ws, claim_label, claim_out);
    if (rc) return rc;
    const std::vector<uint32_t> pt = reversed_point(ws, k);
    if ((rc = xcheck_me(c, S, pt.data(), k, term, "hadamard S")) ||
        (rc = xcheck_me(c, U, pt.data(), k, term + 8, "hadamard U")))
        return rc;
    if (E) return xcheck_me(c, E, pt.data(), k, term + 16, "hadamard E");
    Fr e = kOne;  // eq(u, pt) = prod_i eq2(u_i, pt_i)
    for (uint32_t i = 0; i < k; i++) e = fr_mul(e, fr_eq2((*ueq)[i], fr_load(&pt[8 * (size_t)i])));
    if (!fr_eq(e, fr_load(term + 16))) return fail(c, ZKH_EROUND, "hadamard E terminal != eq(u, point) (convention bug)");
    if (claim_label) {  // the claim taken from the first round against sum E[i] S[i] U[i]
        Fr direct;
        if (ueq) {
            DevPlanes Sp, Up;
            if ((rc = as_planes(c, S, SL_TMP1, &Sp)) || (rc = as_planes(c, U, SL_TMP2, &Up)) ||
                (rc = eq_weighted_sum(c, Sp, &Up, S->n, *ueq, &direct)))
                return rc;
        } else if ((rc = explicit_claim(c, E, S, U, &direct))) {
            return rc;
        }
        if (!fr_eq(direct, fr_load(claim_out))) return fail(c, ZKH_EROUND, "hadamard claim != sum E S U");
    }
    return ZKH_OK;
}
extern "C" int zkh_hp_prove(zkh_ctx* c, uint8_t tr[32], const uint32_t claim[8], const zkh_tensor* E,
                            const zkh_tensor* S, const zkh_tensor* U, uint32_t* ev_out,
                            uint32_t* term_out, uint32_t* ws_out) {
    if (!c || !tr || !claim || !E || !S || !U) return fail(c, ZKH_EARG, "null argument");
    return hp_checked(c, tr, claim, E, nullptr, S, U, ev_out, term_out, ws_out);
}
extern "C" int zkh_hp_prove_eq(zkh_ctx* c, uint8_t tr[32], const uint32_t claim[8], const uint32_t* u,
                               uint32_t k, const zkh_tensor* S, const zkh_tensor* U, uint32_t* ev_out,
                               uint32_t* term_out, uint32_t* ws_out) {
    if (!c || !tr || !claim || !S || !U || (!u && k)) return fail(c, ZKH_EARG, "null argument");
    if (!all_canonical(u, k)) return fail(c, ZKH_EARG, "non-canonical challenge");
    std::vector<Fr> uv = load_frs(u, k);
    return hp_checked(c, tr, claim, nullptr, &uv, S, U, ev_out, term_out, ws_out);
}
extern "C" int zkh_hp_prove_claim(zkh_ctx* c, uint8_t tr[32], const char* label, const zkh_tensor* E,
                                  const zkh_tensor* S, const zkh_tensor* U, uint32_t claim_out[8], uint32_t* ev_out,
                                  uint32_t* term_out, uint32_t* ws_out) {
    if (!c || !tr || !label || !claim_out || !E || !S || !U) return fail(c, ZKH_EARG, "null argument");
    return hp_checked(c, tr, nullptr, E, nullptr, S, U, ev_out, term_out, ws_out, label, claim_out);
}
extern "C" int zkh_hp_prove_eq_claim(zkh_ctx* c, uint8_t tr[32], const char* label, const uint32_t* u, uint32_t k,
                                     const zkh_tensor* S, const zkh_tensor* U, uint32_t claim_out[8],
                                     uint32_t* ev_out, uint32_t* term_out, uint32_t* ws_out) {
    if (!c || !tr || !label || !claim_out || !S || !U || (!u && k)) return fail(c, ZKH_EARG, "null argument");
    if (!all_canonical(u, k)) return fail(c, ZKH_EARG, "non-canonical challenge");
    std::vector<Fr> uv = load_frs(u, k);
    return hp_checked(c, tr, nullptr, nullptr, &uv, S, U, ev_out, term_out, ws_out, label, claim_out);
}

// ---------------------------------------------------------------------------------------
// window partial_me (fr-tensor.cu:512-516, :612-641)
// ---------------------------------------------------------------------------------------
// k LSB-first binds of the row index of a [rows, window] view (the last row may be
// partial; missing entries are zero): out[w*window + j] = sum_{b < 2^k} eq(b, u) *
// t[(w*2^k + b)*window + j], w < ceil(rows / 2^k) -- the k halving steps of the reference
// in one pass
extern "C" int zkh_partial_me_window(zkh_ctx* c, const zkh_tensor* t, const uint32_t* u, uint32_t k,
                                     uint32_t window, zkh_tensor** out) {
    if (!c || !t || !out || !u || !k || !window) return fail(c, ZKH_EARG, "bad arguments");
    if (k >= 32 || (uint64_t)t->n <= (uint64_t)window * (1ull << (k - 1)))
        return fail(c, ZKH_EARG, "partial_me: Incompatible dimensions");
    if (!all_canonical(u, k)) return fail(c, ZKH_EARG, "non-canonical challenge");
    HIPCHK(c, hipSetDevice(c->device));
    const uint64_t rows = ((uint64_t)t->n + window - 1) / window;
    uint64_t orows = rows;
    for (uint32_t r = 0; r < k; r++) orows = (orows + 1) / 2;  // ceil per step, as the reference
    const uint64_t C = 1ull << k;
    if (orows * window >= (1ull << 32) || orows * C * window > (1ull << 40))
        return fail(c, ZKH_EARG, "partial_me: too large");
    int rc = 0;
    uint32_t* E;
    if ((rc = eq_table_mont(c, load_frs(u, k), (uint32_t)C, SL_EB, &E))) return rc;
    zkh_tensor* o;
    if ((rc = tensor_alloc(c, ZKH_KIND_FR, (uint32_t)(orows * window), &o))) return rc;
    const void* src = t->d;
    int kind = t->kind == ZKH_KIND_FR ? 0 : t->kind == ZKH_KIND_I32 ? 1 : 2;
    DevPlanes p{(uint32_t*)t->d, t->cap};
    if (t->weights) {  // logical (row-major) W from the OUT-major copy
        if ((rc = as_planes(c, t, SL_TMP0, &p))) {
            zkh_tensor_free(o);
            return rc;
        }
        src = p.base;
        kind = 0;
    }
    launch_partial_me_window(c->stream, kind, src, p.cap, t->n, (uint32_t)orows, (uint32_t)C, window, E,
                             o->planes());
    hipError_t e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        zkh_tensor_free(o);
        return fail(c, ZKH_EDEV, "partial_me: %s", hipGetErrorString(e));
    }
    *out = o;
    return ZKH_OK;
}

// ---------------------------------------------------------------------------------------
// zkip and zkip_stacked (zkfc.cu:94-246) and zkFCStacked::prove (zkfc.cu:288-307)
// ---------------------------------------------------------------------------------------
// one round over the [N, D] working tables: p = (c0, c1, c2) with the weights of E
static int stk_round(zkh_ctx* c, DevPlanes a, DevPlanes b, uint32_t N, uint32_t D, uint32_t Nh,
                     const uint32_t* E, Fr p[3]) {
    Publish pb = make_pub(c, 1);
    {
        ProfScope ps(c, "stk_round", (double)N * D * 64);
        launch_stk_round(c->stream, a, b, N, D, Nh, E, pb);
    }
    int rc = wait_pub(c, pb.seq);
    if (rc) return rc;
    pub_read(c, 0, 3, p);
    for (int i = 0; i < 3; i++) p[i] = fix1(p[i]);
    return 0;
}
// working copies of two tensors of n entries (read by the rounds, folded in place)
static int stk_copies(zkh_ctx* c, const zkh_tensor* A, const zkh_tensor* B, DevPlanes* a, DevPlanes* b) {
    int rc = 0;
    DevPlanes sa, sb;
    if ((rc = as_planes(c, A, SL_TMP0, &sa)) || (rc = as_planes(c, B, SL_TMP1, &sb))) return rc;
    *a = scratch_planes(c, SL_TMP2, A->n, &rc);
    if (rc) return rc;
    *b = scratch_planes(c, SL_TMP3, B->n, &rc);
    if (rc) return rc;
    const size_t q = (size_t)A->n * 16;
    HIPCHK(c, hipMemcpyAsync(a->lo(), sa.lo(), q, hipMemcpyDeviceToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(a->hi(), sa.hi(), q, hipMemcpyDeviceToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(b->lo(), sb.lo(), q, hipMemcpyDeviceToDevice, c->stream));
    HIPCHK(c, hipMemcpyAsync(b->hi(), sb.hi(), q, hipMemcpyDeviceToDevice, c->stream));
    return 0;
}
// zkip (zkfc.cu:129-151) over the working tables of n entries: |u| rounds, u.back() first
static int zkip_rounds(zkh_ctx* c, Fr& claim, DevPlanes a, DevPlanes b, uint32_t n,
                       const std::vector<Fr>& u, std::vector<Fr>& proof) {
    uint32_t N = n;
    for (size_t r = 0; r < u.size(); r++) {
        const uint32_t Nh = (1u << ceil_log2(N)) >> 1;
        Fr p[3];
        int rc = stk_round(c, a, b, N, 1, Nh, nullptr, p);
        if (rc) return rc;
        proof.insert(proof.end(), p, p + 3);
        // claim != p(0) + p(1) (zkfc.cu:145)
        if (!fr_eq(claim, fr_add(p[0], fr_add(p[0], fr_add(p[1], p[2])))))
            return fail(c, ZKH_EROUND, "zkip: claim != p(0) + p(1) at round %zu", r);
        const Fr x = u[u.size() - 1 - r];
        claim = fr_poly_eval(p, 2, x);
        uint32_t xm[8];
        fr_store(fr_to_mont(x), xm);
        launch_stk_fold(c->stream, a, b, N, 1, Nh, xm);
        N = Nh;
    }
    return 0;
}
// zkip_stacked (zkfc.cu:230-246): |uN| rounds over the N rows of [N, D] tables, each
// weighted by eq(u_, row) of the remaining uN prefix, then zkip over D with uD
static int zkip_stacked_rounds(zkh_ctx* c, Fr& claim, DevPlanes a, DevPlanes b, uint32_t N, uint32_t D,
                               const std::vector<Fr>& uN, const std::vector<Fr>& uD,
                               const std::vector<Fr>& vN, std::vector<Fr>& proof) {
    int rc = 0;
    std::vector<Fr> u_ = uN;
    for (size_t r = 0; r < uN.size(); r++) {
        const uint32_t Nh = (1u << ceil_log2(N)) >> 1;
        const Fr ul = u_.back();
        u_.pop_back();
        uint32_t* E = nullptr;
        if (!u_.empty() && (rc = eq_table_mont(c, u_, Nh, SL_EB, &E))) return rc;
        Fr p[3];
        if ((rc = stk_round(c, a, b, N, D, Nh, E, p))) return rc;
        proof.insert(proof.end(), p, p + 3);
        // q = eq(u_last, X) * p: claim != q(0) + q(1) (zkfc.cu:236-237)
        const Fr p1 = fr_add(p[0], fr_add(p[1], p[2]));
        if (!fr_eq(claim, fr_add(fr_mul(fr_sub(kOne, ul), p[0]), fr_mul(ul, p1))))
            return fail(c, ZKH_EROUND, "zkip_stacked: claim != q(0) + q(1) at round %zu", r);
        const Fr v = vN[vN.size() - 1 - r];
        claim = fr_poly_eval(p, 2, v);
        uint32_t vm[8];
        fr_store(fr_to_mont(v), vm);
        launch_stk_fold(c->stream, a, b, N, D, Nh, vm);
        N = Nh;
    }
    return zkip_rounds(c, claim, a, b, D, uD, proof);
}
extern "C" int zkh_zkip(zkh_ctx* c, const uint32_t claim_l[8], const zkh_tensor* A, const zkh_tensor* B,
                        const uint32_t* u, uint32_t k, uint32_t* proof_out, uint32_t final_out[8]) {
    if (!c || !claim_l || !A || !B || !final_out || (!u && k)) return fail(c, ZKH_EARG, "null argument");
    if (A->n != B->n) return fail(c, ZKH_EARG, "a.size != b.size");
    if (!A->n || k > ceil_log2(A->n)) return fail(c, ZKH_EARG, "zkip: more challenges than variables");
    if (!fr_is_canonical(claim_l) || !all_canonical(u, k)) return fail(c, ZKH_EARG, "non-canonical input");
    HIPCHK(c, hipSetDevice(c->device));
    DevPlanes a, b;
    int rc = stk_copies(c, A, B, &a, &b);
    if (rc) return rc;
    Fr claim = fr_load(claim_l);
    std::vector<Fr> proof;
    rc = zkip_rounds(c, claim, a, b, A->n, load_frs(u, k), proof);
    if (proof_out)
        for (size_t i = 0; i < proof.size(); i++) fr_store(proof[i], proof_out + 8 * i);
    if (rc) return rc;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    fr_store(claim, final_out);
    return ZKH_OK;
}
static int stacked_args(zkh_ctx* c, const zkh_tensor* A, const zkh_tensor* B, uint32_t N, uint32_t D,
                        uint32_t kN, uint32_t kD) {
    if ((uint64_t)A->n != (uint64_t)N * D || (uint64_t)B->n != (uint64_t)N * D)
        return fail(c, ZKH_EARG, "a.size != N * D");
    if (!N || !D || kN != ceil_log2(N) || kD > ceil_log2(D))
        return fail(c, ZKH_EARG, "zkip_stacked: challenge counts do not match N, D");
    return 0;
}
extern "C" int zkh_zkip_stacked(zkh_ctx* c, const uint32_t claim_l[8], const zkh_tensor* A,
                                const zkh_tensor* B, const uint32_t* uN, uint32_t kN, const uint32_t* uD,
                                uint32_t kD, const uint32_t* vN, uint32_t N, uint32_t D,
                                uint32_t* proof_out, uint32_t final_out[8]) {
    if (!c || !claim_l || !A || !B || !final_out || (kN && (!uN || !vN)) || (kD && !uD))
        return fail(c, ZKH_EARG, "null argument");
    int rc = stacked_args(c, A, B, N, D, kN, kD);
    if (rc) return rc;
    if (!fr_is_canonical(claim_l) || !all_canonical(uN, kN) || !all_canonical(vN, kN) || !all_canonical(uD, kD))
        return fail(c, ZKH_EARG, "non-canonical input");
    HIPCHK(c, hipSetDevice(c->device));
    DevPlanes a, b;
    if ((rc = stk_copies(c, A, B, &a, &b))) return rc;
    Fr claim = fr_load(claim_l);
    std::vector<Fr> proof;
    rc = zkip_stacked_rounds(c, claim, a, b, N, D, load_frs(uN, kN), load_frs(uD, kD), load_frs(vN, kN), proof);
    if (proof_out)
        for (size_t i = 0; i < proof.size(); i++) fr_store(proof[i], proof_out + 8 * i);
    if (rc) return rc;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    fr_store(claim, final_out);
    return ZKH_OK;
}
static int mdm(zkh_ctx* c, const zkh_tensor* t, std::initializer_list<const std::vector<Fr>*> us,
               std::initializer_list<uint32_t> shape, Fr* out) {
    std::vector<uint32_t> cat, ks;
    for (auto* u : us) {
        ks.push_back((uint32_t)u->size());
        for (const Fr& x : *u) {
            uint32_t l[8];
            fr_store(x, l);
            cat.insert(cat.end(), l, l + 8);
        }
    }
    cat.resize(cat.size() + 8);
    std::vector<uint32_t> shp(shape);
    uint32_t o[8];
    int rc = zkh_multi_dim_me(c, t, cat.data(), ks.data(), shp.data(), (uint32_t)shp.size(), o);
    if (!rc) *out = fr_load(o);
    return rc;
}
extern "C" int zkh_fc_stacked_prove(zkh_ctx* c, const zkh_tensor* X, const zkh_tensor* W,
                                    const zkh_tensor* Y, const zkh_tensor* bias, uint32_t num,
                                    uint32_t B, uint32_t IN, uint32_t OUT, const uint32_t* u_num,
                                    const uint32_t* v_num, const uint32_t* u_batch, const uint32_t* u_input,
                                    const uint32_t* u_output, uint32_t* proof_out, uint32_t claims_out[16]) {
    if (!c || !X || !W || !Y || !claims_out) return fail(c, ZKH_EARG, "null argument");
    if (!num || !B || !IN || !OUT) return fail(c, ZKH_EARG, "zero dimension");
    // zkFCStacked constructor checks (zkfc.cu:266-269)
    if ((uint64_t)X->n != (uint64_t)num * B * IN) return fail(c, ZKH_EARG, "X size does not match");
    if ((uint64_t)Y->n != (uint64_t)num * B * OUT) return fail(c, ZKH_EARG, "Y size does not match");
    if ((uint64_t)W->n != (uint64_t)num * IN * OUT || W->weights)
        return fail(c, ZKH_EARG, "W size does not match");
    if (bias && (uint64_t)bias->n != (uint64_t)num * OUT) return fail(c, ZKH_EARG, "b size does not match");
    const uint32_t kn = ceil_log2(num), kb = ceil_log2(B), ki = ceil_log2(IN), ko = ceil_log2(OUT);
    if ((kn && (!u_num || !v_num)) || (kb && !u_batch) || (ki && !u_input) || (ko && !u_output))
        return fail(c, ZKH_EARG, "null challenges");
    if (!all_canonical(u_num, kn) || !all_canonical(v_num, kn) || !all_canonical(u_batch, kb) ||
        !all_canonical(u_input, ki) || !all_canonical(u_output, ko))
        return fail(c, ZKH_EARG, "non-canonical challenge");
    HIPCHK(c, hipSetDevice(c->device));
    const std::vector<Fr> un = load_frs(u_num, kn), vn = load_frs(v_num, kn), ub = load_frs(u_batch, kb),
                          ui = load_frs(u_input, ki), uo = load_frs(u_output, ko);
    int rc = 0;
    // claim = Y(u_num, u_batch, u_output) - ones_B(u_batch) * b(u_num, u_output) (zkfc.cu:292-302)
    Fr claim;
    if ((rc = mdm(c, Y, {&un, &ub, &uo}, {num, B, OUT}, &claim))) return rc;
    if (bias) {
        Fr bb;
        if ((rc = mdm(c, bias, {&un, &uo}, {num, OUT}, &bb))) return rc;
        claim = fr_sub(claim, fr_mul(eq_prefix_sum(ub, B), bb));
    }
    // X_reduced = X.partial_me(u_batch, B, IN), W_reduced = W.partial_me(u_output, OUT, 1)
    zkh_tensor *Xr = nullptr, *Wr = nullptr;
    if ((rc = partial_me_impl(c, X, ub, B, IN, &Xr))) return rc;
    if ((rc = partial_me_impl(c, W, uo, OUT, 1, &Wr))) {
        zkh_tensor_free(Xr);
        return rc;
    }
    DevPlanes a, b;
    Fr cur = claim;
    std::vector<Fr> proof;
    rc = stacked_args(c, Xr, Wr, num, IN, kn, ki);
    if (!rc) rc = stk_copies(c, Xr, Wr, &a, &b);
    if (!rc) rc = zkip_stacked_rounds(c, cur, a, b, num, IN, un, ui, vn, proof);
    if (!rc) rc = hipStreamSynchronize(c->stream) == hipSuccess ? 0 : fail(c, ZKH_EDEV, "zkip_stacked sync");
    zkh_tensor_free(Xr);
    zkh_tensor_free(Wr);
    if (proof_out)
        for (size_t i = 0; i < proof.size(); i++) fr_store(proof[i], proof_out + 8 * i);
    if (rc) return rc;
    // opening = X(v_num, u_batch, u_input) * W(v_num, u_input, u_output) (zkfc.cu:305-306)
    Fr ox, ow;
    if ((rc = mdm(c, X, {&vn, &ub, &ui}, {num, B, IN}, &ox))) return rc;
    if ((rc = mdm(c, W, {&vn, &ui, &uo}, {num, IN, OUT}, &ow))) return rc;
    fr_store(claim, claims_out);
    fr_store(cur, claims_out + 8);
    if (!fr_eq(cur, fr_mul(ox, ow))) return fail(c, ZKH_EROUND, "final claim != opening");
    return ZKH_OK;
}

// ---------------------------------------------------------------------------------------
// rescaling witness (rescaling.cu:8-34; zkob_rescale.cu:83-86)
// ---------------------------------------------------------------------------------------
extern "C" int zkh_rescale(zkh_ctx* c, const zkh_tensor* X, uint32_t sf, zkh_tensor** q_out,
                           zkh_tensor** rem_out) {
    if (!c || !X || !q_out || !rem_out || !sf) return fail(c, ZKH_EARG, "bad arguments");
    HIPCHK(c, hipSetDevice(c->device));
    int rc = 0;
    zkh_tensor *q, *r;
    if ((rc = tensor_alloc(c, ZKH_KIND_I64, X->n, &q))) return rc;
    if ((rc = tensor_alloc(c, ZKH_KIND_I64, X->n, &r))) {
        zkh_tensor_free(q);
        return rc;
    }
    const void* src = X->d;
    int kind = X->kind == ZKH_KIND_FR ? 0 : X->kind == ZKH_KIND_I32 ? 1 : 2;
    uint32_t cap = X->cap;
    if (X->weights) {
        DevPlanes p;
        if ((rc = as_planes(c, X, SL_TMP0, &p))) {
            zkh_tensor_free(q);
            zkh_tensor_free(r);
            return rc;
        }
        src = p.base;
        cap = p.cap;
        kind = 0;
    }
    if (X->n) launch_rescale(c->stream, kind, src, cap, X->n, (int64_t)sf, (int64_t*)q->d, (int64_t*)r->d);
    if (X->n && !rc) rc = int_bits_i64(c, (const int64_t*)q->d, X->n, &q->bits);
    if (X->n && !rc) rc = int_bits_i64(c, (const int64_t*)r->d, X->n, &r->bits);
    if (rc) {
        zkh_tensor_free(q);
        zkh_tensor_free(r);
        return rc;
    }
    *q_out = q;
    *rem_out = r;
    return ZKH_OK;
}
