// zkh_batchopen -- a zkob_batchopen-compatible driver over libzkh (zkob_batchopen.cu:695-755,
// batch_prove zkob_claims.cuh:832-1066).
//
//   zkh_batchopen prove <accdir> <run_seed> <q.bin> <G>=<gen.bin> ...
//   zkh_batchopen serve
//
// `prove` opens every claim the drivers emitted into <accdir> (claims.bin, witrefs.txt,
// drvstates.bin) with ONE batch-evaluation sumcheck and one IPA per generator domain:
//   G0  transcript "<run_seed>:opening_batch" absorbs the claim count, every claim blob,
//       every distinct commitment file (path, SHA-256 of its bytes), every driver state;
//       rho; M_j = sum over tensor j's claims of rho^i eq(point_i), P_j = its witness;
//   G2  m_max rounds, round t binding variable m_max-1-t: sum_j c2_j (sum M_j P_j at
//       0, 1, 2) (a tensor with fewer variables contributes c2_j S_j (1-T)^2); "bp0".."bp2";
//   G3  terminals vfin_j = P_j(r), absorbed, checked against sum_j M_j(r) kappa_j vfin_j;
//   G4  rho'; per domain G ascending, a = sum_j rho'^j kappa_j (w_j folded over its rows by
//       r[logG..vars_j)), b = me_weights(r[0..logG)), an IPA over the domain's generators.
// Files, byte-identical to the reference's: batch_sumcheck.bin ("ZKBS", n_claims, m_max,
// count-prefixed evals), batch_vfin.bin ("ZKBV", count-prefixed terminals),
// ipa_batch_<G>.bin.  With ZKOB_PROF set it prints the reference's lap lines
// ("PROF batch_prove.{setup,rounds,terminal,ipa} <s> s").  `verify`, `genq` and `selftest`
// answer exit status 2.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <chrono>
#include <map>
#include <set>

#include "common.hpp"

using namespace zkhcli;

namespace {

struct TensorInfo {
    std::string comref;
    uint32_t domain = 0, n_rows = 0, vars = 0, logG = 0;
    std::vector<uint32_t> idx;
};

// derive_tensors (zkob_claims.cuh:280-308): distinct comrefs in first-appearance order
std::vector<TensorInfo> derive_tensors(const std::vector<Claim>& cs) {
    std::vector<TensorInfo> out;
    std::map<std::string, uint32_t> key;
    for (uint32_t i = 0; i < cs.size(); i++) {
        const Claim& c = cs[i];
        if (c.domain < 2 || (c.domain & (c.domain - 1)))
            throw Err(1, "claim " + c.id + ": domain not a power of two >= 2");
        const uint32_t logG = ceil_log2(c.domain), vars = c.nvars();
        if (vars < logG) throw Err(1, "claim " + c.id + ": point shorter than logG");
        if (vars - logG >= 32 || c.n_rows != (1u << (vars - logG)))
            throw Err(1, "claim " + c.id + ": n_rows != 2^{vars-logG}");
        auto it = key.find(c.comref);
        if (it == key.end()) {
            TensorInfo t;
            t.comref = c.comref;
            t.domain = c.domain;
            t.n_rows = c.n_rows;
            t.vars = vars;
            t.logG = logG;
            t.idx.push_back(i);
            key[c.comref] = (uint32_t)out.size();
            out.push_back(t);
        } else {
            TensorInfo& t = out[it->second];
            if (t.domain != c.domain || t.n_rows != c.n_rows || t.vars != vars)
                throw Err(1, "claim " + c.id + ": shape disagrees with earlier claim on same tensor");
            t.idx.push_back(i);
        }
    }
    return out;
}

// witnesses kept on the device between the rounds and G5 up to this many bytes in total
constexpr uint64_t kResidentMax = 32ull << 30;

// BoTimer (zkob_claims.cuh:62-75): with ZKOB_PROF set, "PROF batch_prove.<lap> <s> s" per lap,
// after the device has finished the lap's work
struct Laps {
    const bool on = getenv("ZKOB_PROF") != nullptr;
    std::chrono::steady_clock::time_point t0 = std::chrono::steady_clock::now();
    void lap(const char* what) {
        if (on) {
            zkh_ctx_sync(g_ctx);
            printf("PROF batch_prove.%s %.4f s\n", what,
                   std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count());
        }
        t0 = std::chrono::steady_clock::now();
    }
};

std::map<std::string, std::string> witrefs_load(const std::string& accdir) {
    std::map<std::string, std::string> m;
    std::vector<uint8_t> b = read_all(accdir + "/witrefs.txt");
    std::string all((const char*)b.data(), b.size());
    size_t pos = 0;
    while (pos < all.size()) {
        size_t nl = all.find('\n', pos);
        if (nl == std::string::npos) nl = all.size();
        const std::string line = all.substr(pos, nl - pos);
        pos = nl + 1;
        const size_t tab = line.find('\t');
        if (tab != std::string::npos) m[line.substr(0, tab)] = line.substr(tab + 1);
    }
    return m;
}

Fr8 eq1(const Fr8& u, const Fr8& v) {  // bo_eq1: 2uv - (u + v) + 1
    const Fr8 uv = fmul(u, v);
    return fadd(fsub(fadd(uv, uv), fadd(u, v)), fr_u32(1));
}
Fr8 kappa(uint32_t vars, const std::vector<Fr8>& r) {  // prod_{v >= vars} (1 - r[v])
    Fr8 k = fr_u32(1);
    for (uint32_t v = vars; v < r.size(); v++) k = fmul(k, fsub(fr_u32(1), r[v]));
    return k;
}

// FrTensor(witpath) (fr-tensor.cu:190-197): the raw 32-byte entries, mapped rather than copied
void load_witness(const std::string& path, uint64_t n, Tensor& t) {
    const int fd = open(path.c_str(), O_RDONLY);
    if (fd < 0) throw Err(1, "cannot open " + path);
    struct stat sb;
    if (fstat(fd, &sb) != 0 || (uint64_t)sb.st_size != n * 32 || n == 0) {
        close(fd);
        throw Err(1, "batch_prove: witness size mismatch for " + path);
    }
    void* p = mmap(nullptr, n * 32, PROT_READ, MAP_PRIVATE | MAP_POPULATE, fd, 0);
    close(fd);
    if (p == MAP_FAILED) throw Err(1, "cannot map " + path);
    const int rc = zkh_tensor_from_fr(g_ctx, (const uint32_t*)p, (uint32_t)n, &t.t);
    munmap(p, n * 32);
    chk(rc, "witness");
}
void absorb_fr(uint8_t st[32], const char* label, const Fr8& x) { absorb(st, label, x.v, 32); }
Fr8 draw(uint8_t st[32]) {
    Fr8 x;
    zkh_transcript_challenge_fr(st, x.v);
    return x;
}

int do_prove(const std::vector<std::string>& a) {
    Laps T;
    const std::string accdir = a[0], run_seed = a[1];
    std::vector<uint32_t> q = load_points(a[2]);
    if (q.empty()) throw Err(1, "q.bin holds no point");
    std::map<uint32_t, std::string> genpaths;  // parse_genspecs: <G>=<path>
    for (size_t i = 3; i < a.size(); i++) {
        const size_t eq = a[i].find('=');
        if (eq == std::string::npos) throw Err(1, "bad generator spec " + a[i]);
        genpaths[(uint32_t)strtoul(a[i].substr(0, eq).c_str(), nullptr, 10)] = a[i].substr(eq + 1);
    }
    const std::vector<Claim> cs = claims_load(accdir + "/claims.bin");
    if (cs.empty()) throw Err(1, "batch_prove: zero claims");
    const std::vector<TensorInfo> ts = derive_tensors(cs);
    std::vector<DrvState> dss;
    if (file_exists(accdir + "/drvstates.bin")) dss = drvstates_load(accdir + "/drvstates.bin");
    const std::map<std::string, std::string> wits = witrefs_load(accdir);
    uint32_t m_max = 0;
    for (const auto& t : ts) m_max = std::max(m_max, t.vars);
    if (m_max < 1) throw Err(1, "batch_prove: m_max < 1");
    const uint32_t nT = (uint32_t)ts.size();
    std::vector<std::string> witpath(nT);
    for (uint32_t j = 0; j < nT; j++) {
        auto it = wits.find(ts[j].comref);
        if (it == wits.end()) throw Err(1, "batch_prove: no witref for " + ts[j].comref);
        witpath[j] = it->second;
    }

    // G0 (batch_absorb_g0, zkob_claims.cuh:320-346) and rho
    uint8_t st[32];
    const std::string seed = run_seed + ":opening_batch";
    zkh_transcript_init(st, seed.data(), seed.size());
    const uint32_t ncl = (uint32_t)cs.size();
    absorb(st, "n_claims", &ncl, 4);
    for (const auto& c : cs) {
        const std::vector<uint8_t> b = claim_blob(c);
        absorb(st, "claim", b.data(), b.size());
    }
    for (const auto& t : ts) {
        std::vector<uint8_t> b;
        put_u32(b, (uint32_t)t.comref.size());
        put_bytes(b, t.comref.data(), t.comref.size());
        const std::vector<uint8_t> f = read_all(t.comref);
        uint8_t h[32];
        zkh_sha256(f.data(), f.size(), h);
        put_bytes(b, h, 32);
        absorb(st, "comref", b.data(), b.size());
    }
    for (const auto& d : dss) {
        std::vector<uint8_t> b;
        put_u32(b, (uint32_t)d.id.size());
        put_bytes(b, d.id.data(), d.id.size());
        put_bytes(b, d.state, 32);
        absorb(st, "drvstate", b.data(), b.size());
    }
    const Fr8 rho = draw(st);
    std::vector<Fr8> rho_pows(ncl);
    rho_pows[0] = fr_u32(1);
    for (uint32_t i = 1; i < ncl; i++) rho_pows[i] = fmul(rho_pows[i - 1], rho);

    // per tensor: M_j = sum_i rho^i eq(point_i), P_j = witness, S_j = <M_j, P_j> if short
    uint64_t wit_bytes = 0;
    for (const auto& t : ts) wit_bytes += 32ull << t.vars;
    const bool resident = wit_bytes <= kResidentMax;
    std::vector<Tensor> M(nT), Pt(nT), Wt(nT);
    std::vector<Fr8> c2(nT, fr_u32(1)), S(nT);
    for (uint32_t j = 0; j < nT; j++) {
        const uint64_t n = 1ull << ts[j].vars;
        // the witness stays on the device for G5 when the layer's witnesses fit the budget
        // (the reference reloads it there); P_j is a copy that the rounds fold in place
        Tensor w;
        load_witness(witpath[j], n, w);
        chk(zkh_axpy(g_ctx, w.t, fr_u32(0).v, w.t, &Pt[j].t), "P");
        if (resident) std::swap(Wt[j].t, w.t);
        for (uint32_t k = 0; k < ts[j].idx.size(); k++) {
            const Claim& c = cs[ts[j].idx[k]];
            Tensor e, acc;
            chk(zkh_eq_table(g_ctx, c.point.data(), c.nvars(), &e.t), "eq(point)");
            if (k == 0) {  // rho^i eq = eq + (rho^i - 1) eq
                chk(zkh_axpy(g_ctx, e.t, fsub(rho_pows[ts[j].idx[k]], fr_u32(1)).v, e.t, &acc.t), "M");
            } else {
                chk(zkh_axpy(g_ctx, M[j].t, rho_pows[ts[j].idx[k]].v, e.t, &acc.t), "M");
            }
            std::swap(M[j].t, acc.t);
        }
        if (zkh_tensor_size(M[j].t) != n) throw Err(1, "batch_prove: table size");
        if (ts[j].vars < m_max) {
            Tensor h;
            chk(zkh_hadamard(g_ctx, M[j].t, Pt[j].t, &h.t), "M P");
            chk(zkh_sum(g_ctx, h.t, S[j].v), "S_j");
        }
    }
    T.lap("setup");
    Fr8 cur;
    for (uint32_t i = 0; i < ncl; i++) cur = fadd(cur, fmul(rho_pows[i], fr_of(cs[i].eval)));

    // G2 rounds
    std::vector<Fr8> r(m_max);
    std::vector<uint32_t> ev;
    for (uint32_t t = 0; t < m_max; t++) {
        const uint32_t v = m_max - 1 - t;
        Fr8 p[3];
        for (uint32_t j = 0; j < nT; j++) {
            if (ts[j].vars <= v) {
                const Fr8 term = fmul(c2[j], S[j]);
                p[0] = fadd(p[0], term);
                p[2] = fadd(p[2], term);
            } else {
                uint32_t qv[24];
                chk(zkh_prod_round(g_ctx, M[j].t, Pt[j].t, qv), "round sums");
                for (int k = 0; k < 3; k++) p[k] = fadd(p[k], fmul(c2[j], fr_of(qv + 8 * k)));
            }
        }
        if (!feq(cur, fadd(p[0], p[1])))
            throw Err(1, "batch_prove: round " + std::to_string(t) + " inconsistency (witness/claims bug)");
        absorb_fr(st, "bp0", p[0]);
        absorb_fr(st, "bp1", p[1]);
        absorb_fr(st, "bp2", p[2]);
        const Fr8 x = draw(st);
        r[v] = x;
        for (int k = 0; k < 3; k++) ev.insert(ev.end(), p[k].v, p[k].v + 8);
        cur = lagrange3(p[0], p[1], p[2], x);
        const Fr8 omx = fsub(fr_u32(1), x), omx2 = fmul(omx, omx);
        for (uint32_t j = 0; j < nT; j++) {
            if (ts[j].vars <= v) {
                c2[j] = fmul(c2[j], omx2);
            } else {
                chk(zkh_fold(g_ctx, M[j].t, x.v), "fold M");
                chk(zkh_fold(g_ctx, Pt[j].t, x.v), "fold P");
            }
        }
    }
    {
        std::vector<uint8_t> b;
        put_bytes(b, "ZKBS", 4);
        put_u32(b, ncl);
        put_u32(b, m_max);
        put_pod(b, ev.data(), 3 * m_max, 8);
        write_all(accdir + "/batch_sumcheck.bin", b.data(), b.size());
    }
    T.lap("rounds");

    // G3 terminals
    std::vector<Fr8> vfin(nT);
    for (uint32_t j = 0; j < nT; j++) {
        chk(zkh_tensor_to_fr(g_ctx, Pt[j].t, vfin[j].v), "vfin");
        absorb_fr(st, "vfin", vfin[j]);
    }
    {
        std::vector<uint32_t> vv;
        for (const auto& x : vfin) vv.insert(vv.end(), x.v, x.v + 8);
        std::vector<uint8_t> b;
        put_bytes(b, "ZKBV", 4);
        put_pod(b, vv.data(), nT, 8);
        write_all(accdir + "/batch_vfin.bin", b.data(), b.size());
    }
    {  // sum_j M_j(r) kappa_j vfin_j == cur (bo_Mj_at_r, bo_kappa)
        Fr8 chkv;
        for (uint32_t j = 0; j < nT; j++) {
            const Fr8 kap = kappa(ts[j].vars, r);
            Fr8 mj;
            for (uint32_t i : ts[j].idx) {
                Fr8 term = rho_pows[i];
                for (uint32_t v = 0; v < ts[j].vars; v++) term = fmul(term, eq1(fr_of(cs[i].point.data() + 8 * v), r[v]));
                mj = fadd(mj, fmul(term, kap));
            }
            chkv = fadd(chkv, fmul(fmul(mj, kap), vfin[j]));
        }
        if (!feq(chkv, cur)) throw Err(1, "batch_prove: G3 terminal self-check failed");
    }
    for (auto& t : M) {
        zkh_tensor_free(t.t);
        t.t = nullptr;
    }
    for (auto& t : Pt) {
        zkh_tensor_free(t.t);
        t.t = nullptr;
    }

    T.lap("terminal");

    // G4 + G5: one IPA per generator domain, ascending
    const Fr8 rhop = draw(st);
    std::vector<Fr8> rhop_pows(nT);
    rhop_pows[0] = fr_u32(1);
    for (uint32_t j = 1; j < nT; j++) rhop_pows[j] = fmul(rhop_pows[j - 1], rhop);
    std::set<uint32_t> domains;
    for (const auto& t : ts) domains.insert(t.domain);
    for (uint32_t G : domains) {
        const uint32_t logG = ceil_log2(G);
        Tensor acc;
        for (uint32_t j = 0; j < nT; j++) {
            if (ts[j].domain != G) continue;
            const Fr8 coef = fmul(rhop_pows[j], kappa(ts[j].vars, r));
            Tensor w, rf, nxt;
            if (resident) {
                std::swap(w.t, Wt[j].t);
            } else {
                load_witness(witpath[j], (uint64_t)ts[j].n_rows * G, w);
            }
            const zkh_tensor* row = w.t;
            if (ts[j].vars > logG) {
                std::vector<uint32_t> urow;
                for (uint32_t v = logG; v < ts[j].vars; v++) urow.insert(urow.end(), r[v].v, r[v].v + 8);
                chk(zkh_partial_me_window(g_ctx, w.t, urow.data(), ts[j].vars - logG, G, &rf.t), "row fold");
                row = rf.t;
            }
            if (!acc.t) {
                chk(zkh_axpy(g_ctx, row, fsub(coef, fr_u32(1)).v, row, &nxt.t), "group RLC");
            } else {
                chk(zkh_axpy(g_ctx, acc.t, coef.v, row, &nxt.t), "group RLC");
            }
            std::swap(acc.t, nxt.t);
        }
        auto git = genpaths.find(G);
        if (git == genpaths.end()) throw Err(1, "batch_prove: no generator file for domain " + std::to_string(G));
        std::vector<uint32_t> gen = load_points(git->second);
        if (gen.size() / 36 != G) throw Err(1, "batch_prove: generator size mismatch for domain " + std::to_string(G));
        Points g;
        Tensor b;
        chk(zkh_g1_from_host(g_ctx, gen.data(), G, &g.g), "gen");
        std::vector<uint32_t> ucol;
        for (uint32_t v = 0; v < logG; v++) ucol.insert(ucol.end(), r[v].v, r[v].v + 8);
        chk(zkh_eq_table(g_ctx, ucol.data(), logG, &b.t), "me_weights");
        ipa_file(accdir + "/ipa_batch_" + std::to_string(G) + ".bin", st, acc.t, b.t, g.g, q.data());
    }
    T.lap("ipa");
    printf("PROVED opening_batch (%u claims, %u tensors, %zu domains) -> %s\n", ncl, nT, domains.size(),
           accdir.c_str());
    return 0;
}

int run1(const std::vector<std::string>& args) {
    const std::string mode = args.empty() ? "" : args[0];
    std::vector<std::string> rest(args.begin() + (args.empty() ? 0 : 1), args.end());
    reject_flags(rest, "zkh_batchopen");
    if (mode == "prove" && rest.size() >= 3) {
        need_ctx();
        return do_prove(rest);
    }
    fprintf(stderr, "usage: zkh_batchopen prove <accdir> <run_seed> <q.bin> <G>=<gen.bin> ... | serve\n");
    return 2;
}

}  // namespace

int main(int argc, char** argv) { return driver_main(argc, argv, run1); }
