// common.hpp -- shared host code of the zkob_*-compatible drivers (zkh_fc, zkh_rescale):
// input/output files in the reference's formats, the transcript glue, IPA openings and the
// serve loop (zkob_serve.cuh).  Host C++ over the C ABI in include/zkh.h.
#pragma once
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <iostream>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/zkh.h"

namespace zkhcli {


inline zkh_ctx* g_ctx = nullptr;

struct Err : std::runtime_error {
    int rc;
    Err(int code, const std::string& m) : std::runtime_error(m), rc(code) {}
};

inline void chk(int rc, const char* what) {
    if (rc) throw Err(1, std::string(what) + ": " + zkh_last_error(g_ctx));
}

inline std::vector<uint8_t> read_all(const std::string& path) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) throw Err(1, "cannot open " + path);
    std::vector<uint8_t> b;
    uint8_t buf[1 << 16];
    size_t k;
    while ((k = fread(buf, 1, sizeof(buf), f)) > 0) b.insert(b.end(), buf, buf + k);
    fclose(f);
    return b;
}
inline void write_all(const std::string& path, const void* p, size_t n) {
    FILE* f = fopen(path.c_str(), "wb");
    if (!f) throw Err(1, "cannot open " + path);
    if (n && fwrite(p, 1, n, f) != n) {
        fclose(f);
        throw Err(1, "short write " + path);
    }
    fclose(f);
}
// load_int_tensor: exactly `expect` int32 values must be readable
inline std::vector<int32_t> load_int(const std::string& path, uint64_t expect) {
    std::vector<uint8_t> b = read_all(path);
    if (b.size() < expect * 4) throw Err(1, "short read / wrong dims: " + path);
    std::vector<int32_t> v(expect);
    memcpy(v.data(), b.data(), expect * 4);
    return v;
}
inline std::vector<uint32_t> load_points(const std::string& path) {
    std::vector<uint8_t> b = read_all(path);
    std::vector<uint32_t> v(b.size() / 144 * 36);
    memcpy(v.data(), b.data(), v.size() * 4);
    return v;
}
inline uint32_t ceil_log2(uint64_t n) {
    uint32_t k = 0;
    while ((1ull << k) < n) k++;
    return k;
}
inline uint32_t parse_u32(const char* s) {
    char* end = nullptr;
    unsigned long v = strtoul(s, &end, 10);
    if (!*s || *end || v == 0 || v > 0xffffffffUL) throw Err(1, std::string("bad dimension: ") + s);
    return (uint32_t)v;
}

struct Tensor {
    zkh_tensor* t = nullptr;
    ~Tensor() {
        if (t) zkh_tensor_free(t);
    }
};
struct Points {
    zkh_g1* g = nullptr;
    ~Points() {
        if (g) zkh_g1_free(g);
    }
};

inline void absorb(uint8_t st[32], const char* label, const void* p, size_t n) {
    zkh_transcript_absorb(st, label, strlen(label), p, n);
}
inline std::vector<uint32_t> to_host(const zkh_g1* g) {
    std::vector<uint32_t> v((size_t)zkh_g1_size(g) * 36);
    chk(zkh_g1_to_host(g_ctx, g, v.data()), "g1_to_host");
    return v;
}
// write_pod_vec: uint32 count, then the items
inline void put_pod(std::vector<uint8_t>& out, const uint32_t* items, uint32_t count, size_t item_words) {
    const uint8_t* c = (const uint8_t*)&count;
    out.insert(out.end(), c, c + 4);
    const uint8_t* p = (const uint8_t*)items;
    out.insert(out.end(), p, p + (size_t)count * item_words * 4);
}

inline void ipa_file(const std::string& path, uint8_t st[32], const zkh_tensor* a, const zkh_tensor* b,
              const zkh_g1* g, const uint32_t* Q) {
    const uint32_t n = zkh_g1_size(g), rounds = ceil_log2(n);
    std::vector<uint32_t> L((size_t)(rounds ? rounds : 1) * 36), R(L.size());
    uint32_t af[8];
    chk(zkh_ipa_prove(g_ctx, st, a, b, g, Q, L.data(), R.data(), af), "ipa_prove");
    std::vector<uint8_t> out;
    put_pod(out, L.data(), rounds, 36);
    put_pod(out, R.data(), rounds, 36);
    out.insert(out.end(), (uint8_t*)af, (uint8_t*)af + 32);
    write_all(path, out.data(), out.size());
}

// load_long_tensor (zkob_lookup.cuh:103-110): exactly `expect` int64 values
inline std::vector<int64_t> load_long(const std::string& path, uint64_t expect) {
    std::vector<uint8_t> b = read_all(path);
    if (b.size() < expect * 8) throw Err(1, "short read / wrong dims: " + path);
    std::vector<int64_t> v(expect);
    memcpy(v.data(), b.data(), expect * 8);
    return v;
}
inline std::vector<uint32_t> challenge(uint8_t st[32]) {
    std::vector<uint32_t> x(8);
    zkh_transcript_challenge_fr(st, x.data());
    return x;
}
// open_prove (zkob_lookup.cuh:116-127): the point's first log2(G) coordinates are the column
// point (b = me_weights of them), the rest fold the rows of `padded` (partial_me); an IPA of
// size G over gen, written as write_ipa does
inline void open_prove(const zkh_tensor* padded, uint32_t G, const zkh_g1* gen, const uint32_t* Q,
                       const std::vector<uint32_t>& u_pt, const std::string& path, uint8_t st[32]) {
    const uint32_t logG = ceil_log2(G), k = (uint32_t)(u_pt.size() / 8);
    if (k < logG) throw Err(1, "open_prove: point shorter than the column domain");
    Tensor a, b;
    const zkh_tensor* av = padded;
    if (k > logG) {
        chk(zkh_partial_me_window(g_ctx, padded, u_pt.data() + 8 * logG, k - logG, G, &a.t), "partial_me");
        av = a.t;
    }
    chk(zkh_eq_table(g_ctx, u_pt.data(), logG, &b.t), "me_weights");
    ipa_file(path, st, av, b.t, gen, Q);
}
// the zkob_serve.cuh loop around a driver's run1, or one request from argv
inline int driver_main(int argc, char** argv, int (*run1)(const std::vector<std::string>&)) {
    if (argc > 1 && std::string(argv[1]) == "serve") {
        printf("ZKW-READY\n");
        fflush(stdout);
        std::string line;  // one request per line, of any length
        while (std::getline(std::cin, line)) {
            std::vector<std::string> toks;
            std::istringstream words(line);
            for (std::string t; words >> t;) toks.push_back(t);
            if (toks.empty()) continue;
            int rc;
            try {
                rc = run1(toks);
            } catch (const std::exception& e) {
                printf("serve: request threw: %s\n", e.what());
                rc = 3;
            }
            printf("ZKW-RC %d\n", rc);
            fflush(stdout);
        }
        if (g_ctx) zkh_ctx_destroy(g_ctx);
        return 0;
    }
    int rc;
    try {
        rc = run1(std::vector<std::string>(argv + 1, argv + argc));
    } catch (const Err& e) {
        fprintf(stderr, "%s: %s\n", argv[0], e.what());
        rc = e.rc;
    } catch (const std::exception& e) {
        fprintf(stderr, "%s: %s\n", argv[0], e.what());
        rc = 1;
    }
    if (g_ctx) zkh_ctx_destroy(g_ctx);
    return rc;
}
inline void need_ctx() {
    if (!g_ctx && zkh_ctx_create(0, &g_ctx) != ZKH_OK) throw Err(1, "no GPU context");
}
// removes "--claims" and the nargs arguments after it from rest; returns them (empty: absent)
inline std::vector<std::string> take_claims(std::vector<std::string>& rest, size_t nargs) {
    for (size_t i = 0; i < rest.size(); i++) {
        if (rest[i] != "--claims") continue;
        if (i + 1 + nargs > rest.size()) throw Err(1, "--claims needs " + std::to_string(nargs) + " arguments");
        std::vector<std::string> out(rest.begin() + i + 1, rest.begin() + i + 1 + nargs);
        rest.erase(rest.begin() + i, rest.begin() + i + 1 + nargs);
        return out;
    }
    return {};
}
inline void reject_flags(const std::vector<std::string>& rest, const char* drv) {
    for (const auto& s : rest)
        if (s.rfind("--", 0) == 0) throw Err(2, std::string(drv) + ": " + s + " (claim and privacy modes) is not provided");
}

// ---- field scalars on the host (h_scalar) ----
struct Fr8 {
    uint32_t v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
};
inline Fr8 fr_u32(uint32_t x) {
    Fr8 r;
    r.v[0] = x;
    return r;
}
inline Fr8 fr_of(const uint32_t* p) {
    Fr8 r;
    memcpy(r.v, p, 32);
    return r;
}
inline Fr8 fop(const Fr8& a, const Fr8& b, int op) {
    Fr8 r;
    if (zkh_fr_scalar(a.v, b.v, op, r.v)) throw Err(1, "non-canonical field element");
    return r;
}
inline Fr8 fadd(const Fr8& a, const Fr8& b) { return fop(a, b, 0); }
inline Fr8 fsub(const Fr8& a, const Fr8& b) { return fop(a, b, 1); }
inline Fr8 fmul(const Fr8& a, const Fr8& b) { return fop(a, b, 2); }
inline Fr8 finv(const Fr8& a) { return fop(a, a, 3); }
inline bool feq(const Fr8& a, const Fr8& b) { return memcmp(a.v, b.v, 32) == 0; }
// lagrange3 (vrf_common.cuh:130-140): p(u) through p(0), p(1), p(2)
inline Fr8 lagrange3(const Fr8& p0, const Fr8& p1, const Fr8& p2, const Fr8& u) {
    const Fr8 one = fr_u32(1), two = fr_u32(2), inv2 = finv(two);
    const Fr8 um1 = fsub(u, one), um2 = fsub(u, two);
    const Fr8 l0 = fmul(fmul(um1, um2), inv2), l1 = fmul(u, fsub(two, u)), l2 = fmul(fmul(u, um1), inv2);
    return fadd(fadd(fmul(p0, l0), fmul(p1, l1)), fmul(p2, l2));
}

// ---- claims accumulator files (zkob_claims.cuh:82-270) ----
inline void put_u32(std::vector<uint8_t>& b, uint32_t v) {
    for (int i = 0; i < 4; i++) b.push_back(uint8_t(v >> (8 * i)));
}
inline void put_bytes(std::vector<uint8_t>& b, const void* p, size_t n) {
    const uint8_t* q = (const uint8_t*)p;
    b.insert(b.end(), q, q + n);
}
struct Claim {
    std::string id, comref;
    uint32_t domain = 0, n_rows = 0;
    std::vector<uint32_t> point;  // 8 words per coordinate: u_col ++ u_row
    uint8_t tag = 0;              // 0: plain evaluation
    uint32_t eval[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    uint32_t nvars() const { return (uint32_t)(point.size() / 8); }
};
// claim_blob (zkob_claims.cuh:104-116): length-prefixed id, comref and point, tag, eval
inline std::vector<uint8_t> claim_blob(const Claim& c) {
    std::vector<uint8_t> b;
    put_u32(b, (uint32_t)c.id.size());
    put_bytes(b, c.id.data(), c.id.size());
    put_u32(b, (uint32_t)c.comref.size());
    put_bytes(b, c.comref.data(), c.comref.size());
    put_u32(b, c.domain);
    put_u32(b, c.n_rows);
    put_u32(b, c.nvars());
    put_bytes(b, c.point.data(), c.point.size() * 4);
    b.push_back(c.tag);
    put_bytes(b, c.eval, 32);
    return b;
}
struct Reader {
    const std::vector<uint8_t>& b;
    size_t off = 0;
    explicit Reader(const std::vector<uint8_t>& bytes) : b(bytes) {}
    void bytes(void* p, size_t n) {
        if (off + n > b.size()) throw Err(1, "truncated file");
        memcpy(p, b.data() + off, n);
        off += n;
    }
    uint32_t u32() {
        uint32_t v;
        bytes(&v, 4);
        return v;
    }
    std::string str(uint32_t n) {
        std::string s(n, '\0');
        bytes(&s[0], n);
        return s;
    }
};
inline bool file_exists(const std::string& path) {
    FILE* f = fopen(path.c_str(), "rb");
    if (f) fclose(f);
    return f != nullptr;
}
// claims_parse (zkob_claims.cuh:171-194); committed (tag 1) claims are not provided
inline std::vector<Claim> claims_load(const std::string& path) {
    std::vector<uint8_t> bytes = read_all(path);
    Reader r(bytes);
    char magic[4];
    r.bytes(magic, 4);
    if (memcmp(magic, "ZKCL", 4)) throw Err(1, "claims: bad magic");
    if (r.u32() != 1) throw Err(1, "claims: bad version");
    std::vector<Claim> cs(r.u32());
    for (auto& c : cs) {
        c.id = r.str(r.u32());
        c.comref = r.str(r.u32());
        c.domain = r.u32();
        c.n_rows = r.u32();
        const uint32_t np = r.u32();
        if (np > 64) throw Err(1, "claims: point too long");
        c.point.resize((size_t)np * 8);
        r.bytes(c.point.data(), (size_t)np * 32);
        r.bytes(&c.tag, 1);
        if (c.tag == 1) throw Err(2, "claims: committed evaluations are not provided");
        if (c.tag != 0) throw Err(1, "claims: unknown EvalVar tag");
        r.bytes(c.eval, 32);
    }
    if (r.off != bytes.size()) throw Err(1, "claims: trailing bytes");
    return cs;
}
inline void claims_save(const std::string& path, const std::vector<Claim>& cs) {
    std::vector<uint8_t> b;
    put_bytes(b, "ZKCL", 4);
    put_u32(b, 1);
    put_u32(b, (uint32_t)cs.size());
    for (const auto& c : cs) {
        std::vector<uint8_t> cb = claim_blob(c);
        put_bytes(b, cb.data(), cb.size());
    }
    write_all(path, b.data(), b.size());
}
// claim_emit (zkob_claims.cuh:225-231): append to <accdir>/claims.bin
inline void claim_emit(const std::string& accdir, const Claim& c) {
    const std::string path = accdir + "/claims.bin";
    std::vector<Claim> cs;
    if (file_exists(path)) cs = claims_load(path);
    cs.push_back(c);
    claims_save(path, cs);
}
// witref_emit (zkob_claims.cuh:233-244): one "comref\twitpath" line per distinct tensor
inline void witref_emit(const std::string& accdir, const std::string& comref, const std::string& witpath) {
    const std::string path = accdir + "/witrefs.txt";
    if (file_exists(path)) {
        std::vector<uint8_t> b = read_all(path);
        if (std::string((const char*)b.data(), b.size()).find(comref + "\t") != std::string::npos) return;
    }
    FILE* f = fopen(path.c_str(), "ab");
    if (!f) throw Err(1, "cannot open " + path);
    fprintf(f, "%s\t%s\n", comref.c_str(), witpath.c_str());
    fclose(f);
}
struct DrvState {
    std::string id;
    uint8_t state[32];
};
inline std::vector<DrvState> drvstates_load(const std::string& path) {
    std::vector<uint8_t> bytes = read_all(path);
    Reader r(bytes);
    char magic[4];
    r.bytes(magic, 4);
    if (memcmp(magic, "ZKDS", 4)) throw Err(1, "drvstates: bad magic");
    if (r.u32() != 1) throw Err(1, "drvstates: bad version");
    std::vector<DrvState> ds(r.u32());
    for (auto& d : ds) {
        d.id = r.str(r.u32());
        r.bytes(d.state, 32);
    }
    return ds;
}
// drvstate_emit (zkob_claims.cuh:259-270): append (id, transcript state) to drvstates.bin
inline void drvstate_emit(const std::string& accdir, const std::string& id, const uint8_t st[32]) {
    const std::string path = accdir + "/drvstates.bin";
    std::vector<DrvState> ds;
    if (file_exists(path)) ds = drvstates_load(path);
    DrvState d;
    d.id = id;
    memcpy(d.state, st, 32);
    ds.push_back(d);
    std::vector<uint8_t> b;
    put_bytes(b, "ZKDS", 4);
    put_u32(b, 1);
    put_u32(b, (uint32_t)ds.size());
    for (const auto& e : ds) {
        put_u32(b, (uint32_t)e.id.size());
        put_bytes(b, e.id.data(), e.id.size());
        put_bytes(b, e.state, 32);
    }
    write_all(path, b.data(), b.size());
}
// FrTensor::save of a device tensor: raw 8-word entries
inline void save_fr(const std::string& path, const zkh_tensor* t) {
    std::vector<uint32_t> v((size_t)zkh_tensor_size(t) * 8);
    chk(zkh_tensor_to_fr(g_ctx, t, v.data()), "to_fr");
    write_all(path, v.data(), v.size() * 4);
}

}  // namespace zkhcli
