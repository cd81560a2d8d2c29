// zkh_batchopen -- a zkob_batchopen-compatible driver over libzkh (zkob_batchopen.cu:695-755;
// the proof it writes is batch_prove's, zkob_claims.cuh:832-1066).
//
//   zkh_batchopen prove <accdir> <run_seed> <q.bin> <G>=<gen.bin> ...
//   zkh_batchopen serve
//
// `prove` opens every claim the drivers emitted into <accdir> (claims.bin, witrefs.txt,
// drvstates.bin) with one batch-evaluation sumcheck and one IPA per generator domain.
// Protocol (kept byte for byte; the code below is organised differently):
//   header   transcript "<run_seed>:opening_batch" absorbs "n_claims", each claim blob
//            ("claim"), each committed tensor's (path, SHA-256 of its file) ("comref", in
//            the order the tensors first appear among the claims) and each driver state
//            ("drvstate"); rho is drawn; claim i carries weight rho^i.
//   rounds   one round per variable of the largest tensor, from the top variable down:
//            the round polynomial at 0, 1, 2 is absorbed as "bp0".."bp2" and the challenge
//            drawn.  A tensor with fewer variables than the round's index contributes
//            lift * <M_j, P_j> (1 - X)^2, lift being the product of (1 - r)^2 over the
//            rounds already bound; from its first own round on it is an ordinary product
//            sumcheck of M_j = sum_i rho^i eq(point_i, .) and its witness P_j, scaled by
//            the lift at that moment (= kappa_j^2, kappa_j = prod over the variables above
//            it of (1 - r_v)).
//   terms    the folded witnesses P_j(r) are absorbed ("vfin") and checked against the
//            final claim: sum_j kappa_j^2 M_j(r) P_j(r).
//   ipa      rho' is drawn; per domain G, ascending, a = sum_j rho'^j kappa_j (witness j
//            with its rows bound by r[logG..vars_j)) and b = eq(r[0..logG), .), proved by
//            one IPA over the domain's generators.
// Files, byte-identical to the reference's: batch_sumcheck.bin ("ZKBS", n_claims, m_max,
// count-prefixed evaluations), batch_vfin.bin ("ZKBV", count-prefixed terminals),
// ipa_batch_<G>.bin.  ZKOB_PROF prints the reference's lap lines ("PROF
// batch_prove.{setup,rounds,terminal,ipa} <s> s").  ZKOB_BATCH_SELFCHECK also checks, per
// domain, that <gen, a> equals the same combination of the tensors' row commitments
// (the commitment-side identity of zkob_claims.cuh:1038-1052).  `verify`, `genq` and
// `selftest` answer exit status 2.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <map>
#include <unordered_map>

#include "common.hpp"

using namespace zkhcli;

namespace {

// witnesses stay on the device from the setup to the openings up to this many bytes in total
constexpr uint64_t kResidentMax = 32ull << 30;

// one committed tensor and the claims made on it
struct Opened {
    std::string comref, witness;
    uint32_t domain = 0, logG = 0, nv = 0;  // nv: variables of the padded witness
    std::vector<uint32_t> claims;           // indices into the claim list
    Tensor M, P, W;                         // weight table, folded witness, resident witness
    Fr8 inner;                              // <M, P> before the rounds reach the tensor
    Fr8 kappa = fr_u32(1);                  // prod of (1 - r_v) over v >= nv
    Fr8 term;                               // P(r) after the rounds
};

// lap timer with the reference's ZKOB_PROF lines; each lap waits for the device
struct Stopwatch {
    bool on = getenv("ZKOB_PROF") != nullptr;
    std::chrono::steady_clock::time_point since = std::chrono::steady_clock::now();
    void lap(const char* name) {
        if (on) {
            zkh_ctx_sync(g_ctx);
            const double s = std::chrono::duration<double>(std::chrono::steady_clock::now() - since).count();
            printf("PROF batch_prove.%s %.4f s\n", name, s);
        }
        since = std::chrono::steady_clock::now();
    }
};

bool is_pow2_at_least_2(uint64_t x) { return x >= 2 && (x & (x - 1)) == 0; }

// The claims grouped by committed tensor, tensors in order of first appearance.  Every claim
// on a tensor must describe the same geometry: a power-of-two domain of G >= 2 columns, a
// point of logG column coordinates then row coordinates, and 2^(rows coordinates) rows.
std::vector<Opened> group_claims(const std::vector<Claim>& cs) {
    std::vector<Opened> ts;
    std::unordered_map<std::string, size_t> slot;
    for (uint32_t i = 0; i < cs.size(); i++) {
        const Claim& c = cs[i];
        const std::string who = "claim '" + c.id + "' on " + c.comref;
        if (!is_pow2_at_least_2(c.domain))
            throw Err(1, who + ": generator domain " + std::to_string(c.domain) + " is not a power of two >= 2");
        const uint32_t logG = ceil_log2(c.domain), nv = c.nvars();
        if (nv < logG)
            throw Err(1, who + ": point has " + std::to_string(nv) + " coordinates, fewer than log2(domain)");
        if (nv - logG >= 32 || c.n_rows != (1u << (nv - logG)))
            throw Err(1, who + ": " + std::to_string(c.n_rows) + " rows do not match a point of " +
                             std::to_string(nv - logG) + " row coordinates");
        auto [it, fresh] = slot.emplace(c.comref, ts.size());
        if (fresh) {
            ts.emplace_back();
            ts.back().comref = c.comref;
            ts.back().domain = c.domain;
            ts.back().logG = logG;
            ts.back().nv = nv;
        }
        Opened& t = ts[it->second];
        if (t.domain != c.domain || t.nv != nv)
            throw Err(1, who + ": geometry differs from an earlier claim on the same tensor");
        t.claims.push_back(i);
    }
    return ts;
}

// "<G>=<path>" arguments: G a decimal power of two >= 2, each domain named once
std::map<uint32_t, std::string> parse_generators(const std::vector<std::string>& specs) {
    std::map<uint32_t, std::string> out;
    for (const std::string& s : specs) {
        const size_t eq = s.find('=');
        const std::string g = s.substr(0, eq == std::string::npos ? 0 : eq);
        const bool digits = !g.empty() && g.size() <= 10 &&
                            std::all_of(g.begin(), g.end(), [](char ch) { return ch >= '0' && ch <= '9'; });
        const uint64_t G = digits ? std::stoull(g) : 0;
        if (eq == std::string::npos || eq + 1 == s.size() || !digits || !is_pow2_at_least_2(G) || G > (1u << 31))
            throw Err(1, "generator spec '" + s + "': expected <G>=<file> with G a power of two >= 2");
        if (!out.emplace((uint32_t)G, s.substr(eq + 1)).second)
            throw Err(1, "generator spec '" + s + "': domain " + g + " given twice");
    }
    return out;
}

// witrefs.txt: "<comref>\t<witness path>" lines
std::unordered_map<std::string, std::string> read_witrefs(const std::string& accdir) {
    const std::vector<uint8_t> raw = read_all(accdir + "/witrefs.txt");
    std::unordered_map<std::string, std::string> m;
    size_t at = 0;
    while (at < raw.size()) {
        size_t end = at;
        while (end < raw.size() && raw[end] != '\n') end++;
        const std::string line((const char*)raw.data() + at, end - at);
        const size_t tab = line.find('\t');
        if (tab != std::string::npos) m[line.substr(0, tab)] = line.substr(tab + 1);
        at = end + 1;
    }
    return m;
}

// the n 32-byte entries of a witness file (FrTensor(path), fr-tensor.cu:190-197), mapped and
// uploaded without a host copy
void upload_witness(const std::string& path, uint64_t n, Tensor& t) {
    const int fd = open(path.c_str(), O_RDONLY);
    if (fd < 0) throw Err(1, "cannot open witness " + path);
    struct stat sb;
    const bool ok = fstat(fd, &sb) == 0 && n > 0 && (uint64_t)sb.st_size == n * 32;
    void* p = ok ? mmap(nullptr, n * 32, PROT_READ, MAP_PRIVATE | MAP_POPULATE, fd, 0) : MAP_FAILED;
    close(fd);
    if (!ok) throw Err(1, "witness " + path + " does not hold " + std::to_string(n) + " field elements");
    if (p == MAP_FAILED) throw Err(1, "cannot map witness " + path);
    const int rc = zkh_tensor_from_fr(g_ctx, (const uint32_t*)p, (uint32_t)n, &t.t);
    munmap(p, n * 32);
    chk(rc, "witness upload");
}

Fr8 draw(uint8_t st[32]) {
    Fr8 x;
    zkh_transcript_challenge_fr(st, x.v);
    return x;
}
void absorb_fr(uint8_t st[32], const char* label, const Fr8& x) { absorb(st, label, x.v, 32); }
std::vector<Fr8> powers(const Fr8& x, size_t n) {
    std::vector<Fr8> p(n, fr_u32(1));
    for (size_t i = 1; i < n; i++) p[i] = fmul(p[i - 1], x);
    return p;
}
std::vector<uint32_t> words(const std::vector<Fr8>& r, uint32_t from, uint32_t to) {
    std::vector<uint32_t> w;
    for (uint32_t v = from; v < to; v++) w.insert(w.end(), r[v].v, r[v].v + 8);
    return w;
}

// the batch header: claim count, claims, committed tensors (path + file digest), driver states
void absorb_header(uint8_t st[32], const std::vector<Claim>& cs, const std::vector<Opened>& ts,
                   const std::vector<DrvState>& dss) {
    const uint32_t n = (uint32_t)cs.size();
    absorb(st, "n_claims", &n, 4);
    for (const Claim& c : cs) {
        const std::vector<uint8_t> blob = claim_blob(c);
        absorb(st, "claim", blob.data(), blob.size());
    }
    auto named = [](const std::string& s, const uint8_t* tail, size_t tn) {
        std::vector<uint8_t> b;
        put_u32(b, (uint32_t)s.size());
        put_bytes(b, s.data(), s.size());
        put_bytes(b, tail, tn);
        return b;
    };
    for (const Opened& t : ts) {
        const std::vector<uint8_t> file = read_all(t.comref);
        uint8_t digest[32];
        zkh_sha256(file.data(), file.size(), digest);
        const std::vector<uint8_t> b = named(t.comref, digest, 32);
        absorb(st, "comref", b.data(), b.size());
    }
    for (const DrvState& d : dss) {
        const std::vector<uint8_t> b = named(d.id, d.state, 32);
        absorb(st, "drvstate", b.data(), b.size());
    }
}

// M = sum over the tensor's claims of rho^i eq(point_i, .); P = a copy of the witness, which
// the rounds fold in place; the witness itself is kept for the openings when `keep`
void build_tables(Opened& t, const std::vector<Claim>& cs, const std::vector<Fr8>& weight, bool keep) {
    Tensor w;
    upload_witness(t.witness, 1ull << t.nv, w);
    chk(zkh_axpy(g_ctx, w.t, fr_u32(0).v, w.t, &t.P.t), "witness copy");
    if (keep) std::swap(t.W.t, w.t);
    for (uint32_t i : t.claims) {
        Tensor e, next;
        chk(zkh_eq_table(g_ctx, cs[i].point.data(), cs[i].nvars(), &e.t), "eq table");
        if (!t.M.t)  // the first claim: eq + (rho^i - 1) eq
            chk(zkh_axpy(g_ctx, e.t, fsub(weight[i], fr_u32(1)).v, e.t, &next.t), "weights");
        else
            chk(zkh_axpy(g_ctx, t.M.t, weight[i].v, e.t, &next.t), "weights");
        std::swap(t.M.t, next.t);
    }
}

// sum_i rho^i eq(point_i, r) over the tensor's own variables
Fr8 weight_at(const Opened& t, const std::vector<Claim>& cs, const std::vector<Fr8>& weight,
              const std::vector<Fr8>& r) {
    Fr8 s;
    for (uint32_t i : t.claims) {
        Fr8 e = weight[i];
        for (uint32_t v = 0; v < t.nv; v++) {
            const Fr8 a = fr_of(cs[i].point.data() + 8 * v), ar = fmul(a, r[v]);
            e = fmul(e, fadd(fsub(fadd(ar, ar), fadd(a, r[v])), fr_u32(1)));  // eq(a, r_v)
        }
        s = fadd(s, e);
    }
    return s;
}

// ZKOB_BATCH_SELFCHECK: <gen, a> - sum_j coef_j (row commitments of j bound by its row
// challenges) must be the point at infinity (z = 0)
void selfcheck_domain(const Points& gen, const zkh_tensor* a, const std::vector<const Opened*>& group,
                      const std::vector<Fr8>& coef, const std::vector<Fr8>& r) {
    Points acc;
    chk(zkh_commit(g_ctx, gen.g, a, &acc.g), "selfcheck <gen, a>");
    for (size_t k = 0; k < group.size(); k++) {
        const Opened& t = *group[k];
        const std::vector<uint32_t> rows = load_points(t.comref);
        Points com, bound, next;
        chk(zkh_g1_from_host(g_ctx, rows.data(), (uint32_t)(rows.size() / 36), &com.g), "selfcheck com");
        const zkh_g1* c = com.g;
        if (t.nv > t.logG) {
            const std::vector<uint32_t> ur = words(r, t.logG, t.nv);
            Tensor e;
            chk(zkh_eq_table(g_ctx, ur.data(), t.nv - t.logG, &e.t), "selfcheck row weights");
            chk(zkh_commit(g_ctx, com.g, e.t, &bound.g), "selfcheck row fold");
            c = bound.g;
        }
        chk(zkh_g1_addmul(g_ctx, c, fsub(Fr8(), coef[k]).v, acc.g, &next.g), "selfcheck combine");
        std::swap(acc.g, next.g);
    }
    const std::vector<uint32_t> p = to_host(acc.g);
    for (int i = 24; i < 36; i++)
        if (p[i]) throw Err(1, "batch_prove: commitment-side self-check failed for domain " + std::to_string(group[0]->domain));
}

int prove(const std::vector<std::string>& a) {
    Stopwatch sw;
    const std::string accdir = a[0], run_seed = a[1];
    const std::map<uint32_t, std::string> gens = parse_generators({a.begin() + 3, a.end()});
    const std::vector<uint32_t> Q = load_points(a[2]);
    if (Q.empty()) throw Err(1, "q.bin holds no point");

    const std::vector<Claim> cs = claims_load(accdir + "/claims.bin");
    if (cs.empty()) throw Err(1, "batch_prove: claims.bin holds no claim");
    std::vector<Opened> ts = group_claims(cs);
    const std::vector<DrvState> dss =
        file_exists(accdir + "/drvstates.bin") ? drvstates_load(accdir + "/drvstates.bin") : std::vector<DrvState>();
    const auto refs = read_witrefs(accdir);
    uint32_t nvars = 0;
    uint64_t witness_bytes = 0;
    for (Opened& t : ts) {
        auto it = refs.find(t.comref);
        if (it == refs.end()) throw Err(1, "batch_prove: no witref for " + t.comref);
        t.witness = it->second;
        nvars = std::max(nvars, t.nv);
        witness_bytes += 32ull << t.nv;
    }
    if (nvars == 0) throw Err(1, "batch_prove: every claim is on a single entry");

    uint8_t st[32];
    const std::string label = run_seed + ":opening_batch";
    zkh_transcript_init(st, label.data(), label.size());
    absorb_header(st, cs, ts, dss);
    const std::vector<Fr8> weight = powers(draw(st), cs.size());

    need_ctx();
    const bool keep = witness_bytes <= kResidentMax;
    for (Opened& t : ts) {
        build_tables(t, cs, weight, keep);
        if (zkh_tensor_size(t.M.t) != (1u << t.nv)) throw Err(1, "batch_prove: weight table size");
        if (t.nv < nvars) {  // needed by the rounds above the tensor's variables
            Tensor h;
            chk(zkh_hadamard(g_ctx, t.M.t, t.P.t, &h.t), "M P");
            chk(zkh_sum(g_ctx, h.t, t.inner.v), "<M, P>");
        }
    }
    sw.lap("setup");

    Fr8 claim;
    for (uint32_t i = 0; i < cs.size(); i++) claim = fadd(claim, fmul(weight[i], fr_of(cs[i].eval)));

    // rounds, top variable first.  `lin` = prod (1 - r) over the bound variables; a tensor
    // whose variables are all below the bound ones has kappa = lin and weight lin^2.
    std::vector<Fr8> r(nvars);
    std::vector<uint32_t> evals;
    Fr8 lin = fr_u32(1);
    for (uint32_t v = nvars; v-- > 0;) {
        Fr8 p[3], idle;
        for (Opened& t : ts) {
            if (t.nv <= v) {
                idle = fadd(idle, t.inner);
                continue;
            }
            if (t.nv == v + 1) t.kappa = lin;  // the tensor's first own round
            uint32_t q[24];
            chk(zkh_prod_round(g_ctx, t.M.t, t.P.t, q), "round sums");
            const Fr8 c = fmul(t.kappa, t.kappa);
            for (int k = 0; k < 3; k++) p[k] = fadd(p[k], fmul(c, fr_of(q + 8 * k)));
        }
        const Fr8 lifted = fmul(fmul(lin, lin), idle);
        p[0] = fadd(p[0], lifted);
        p[2] = fadd(p[2], lifted);
        if (!feq(fadd(p[0], p[1]), claim))
            throw Err(1, "batch_prove: round " + std::to_string(nvars - 1 - v) +
                             " inconsistency: p(0) + p(1) differs from the claim (witness or claims wrong)");
        absorb_fr(st, "bp0", p[0]);
        absorb_fr(st, "bp1", p[1]);
        absorb_fr(st, "bp2", p[2]);
        for (const Fr8& x : p) evals.insert(evals.end(), x.v, x.v + 8);
        r[v] = draw(st);
        claim = lagrange3(p[0], p[1], p[2], r[v]);
        lin = fmul(lin, fsub(fr_u32(1), r[v]));
        for (Opened& t : ts) {
            if (t.nv <= v) continue;
            chk(zkh_fold(g_ctx, t.M.t, r[v].v), "fold M");
            chk(zkh_fold(g_ctx, t.P.t, r[v].v), "fold P");
        }
    }
    {
        std::vector<uint8_t> b;
        put_bytes(b, "ZKBS", 4);
        put_u32(b, (uint32_t)cs.size());
        put_u32(b, nvars);
        put_pod(b, evals.data(), 3 * nvars, 8);
        write_all(accdir + "/batch_sumcheck.bin", b.data(), b.size());
    }
    sw.lap("rounds");

    // terminals
    std::vector<uint32_t> vfin;
    Fr8 expect;
    for (Opened& t : ts) {
        chk(zkh_tensor_to_fr(g_ctx, t.P.t, t.term.v), "terminal");
        absorb_fr(st, "vfin", t.term);
        vfin.insert(vfin.end(), t.term.v, t.term.v + 8);
        const Fr8 k2 = fmul(t.kappa, t.kappa);
        expect = fadd(expect, fmul(fmul(k2, weight_at(t, cs, weight, r)), t.term));
        zkh_tensor_free(t.M.t);
        zkh_tensor_free(t.P.t);
        t.M.t = t.P.t = nullptr;
    }
    {
        std::vector<uint8_t> b;
        put_bytes(b, "ZKBV", 4);
        put_pod(b, vfin.data(), (uint32_t)ts.size(), 8);
        write_all(accdir + "/batch_vfin.bin", b.data(), b.size());
    }
    if (!feq(expect, claim)) throw Err(1, "batch_prove: terminals do not reproduce the final claim");
    sw.lap("terminal");

    // openings, one per generator domain in ascending order
    const std::vector<Fr8> mix = powers(draw(st), ts.size());
    std::map<uint32_t, std::vector<size_t>> by_domain;
    for (size_t j = 0; j < ts.size(); j++) by_domain[ts[j].domain].push_back(j);
    const bool selfcheck = getenv("ZKOB_BATCH_SELFCHECK") != nullptr;
    for (const auto& [G, members] : by_domain) {
        const uint32_t logG = ceil_log2(G);
        Tensor acc;
        std::vector<const Opened*> group;
        std::vector<Fr8> coefs;
        for (size_t j : members) {
            Opened& t = ts[j];
            const Fr8 coef = fmul(mix[j], t.kappa);
            Tensor w, bound, next;
            if (keep)
                std::swap(w.t, t.W.t);
            else
                upload_witness(t.witness, 1ull << t.nv, w);
            const zkh_tensor* row = w.t;
            if (t.nv > logG) {  // bind the rows by r[logG..nv)
                const std::vector<uint32_t> ur = words(r, logG, t.nv);
                chk(zkh_partial_me_window(g_ctx, w.t, ur.data(), t.nv - logG, G, &bound.t), "row binding");
                row = bound.t;
            }
            if (acc.t)
                chk(zkh_axpy(g_ctx, acc.t, coef.v, row, &next.t), "combination");
            else
                chk(zkh_axpy(g_ctx, row, fsub(coef, fr_u32(1)).v, row, &next.t), "combination");
            std::swap(acc.t, next.t);
            group.push_back(&t);
            coefs.push_back(coef);
        }
        auto g = gens.find(G);
        if (g == gens.end()) throw Err(1, "batch_prove: no generator file for domain " + std::to_string(G));
        const std::vector<uint32_t> pts = load_points(g->second);
        if (pts.size() != (size_t)G * 36)
            throw Err(1, "batch_prove: " + g->second + " does not hold " + std::to_string(G) + " generators");
        Points gen;
        chk(zkh_g1_from_host(g_ctx, pts.data(), G, &gen.g), "generators");
        if (selfcheck) selfcheck_domain(gen, acc.t, group, coefs, r);
        Tensor b;
        const std::vector<uint32_t> uc = words(r, 0, logG);
        chk(zkh_eq_table(g_ctx, uc.data(), logG, &b.t), "column weights");
        ipa_file(accdir + "/ipa_batch_" + std::to_string(G) + ".bin", st, acc.t, b.t, gen.g, Q.data());
    }
    sw.lap("ipa");
    printf("PROVED opening_batch (%zu claims, %zu tensors, %zu domains) -> %s\n", cs.size(), ts.size(),
           by_domain.size(), accdir.c_str());
    return 0;
}

int run1(const std::vector<std::string>& args) {
    const std::string mode = args.empty() ? "" : args[0];
    std::vector<std::string> rest(args.begin() + (args.empty() ? 0 : 1), args.end());
    reject_flags(rest, "zkh_batchopen");
    if (mode == "prove" && rest.size() >= 3) return prove(rest);
    fprintf(stderr, "usage: zkh_batchopen prove <accdir> <run_seed> <q.bin> <G>=<gen.bin> ... | serve\n");
    return 2;
}

}  // namespace

int main(int argc, char** argv) { return driver_main(argc, argv, run1); }
