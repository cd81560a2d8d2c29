// common.hpp -- shared host code of the zkob_*-compatible drivers (zkh_fc, zkh_rescale):
// input/output files in the reference's formats, the transcript glue, IPA openings and the
// serve loop (zkob_serve.cuh).  Host C++ over the C ABI in include/zkh.h.
#pragma once
#include <stdint.h>
#include <stdio.h>
#include <string.h>

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
        char line[1 << 16];
        while (fgets(line, sizeof(line), stdin)) {
            std::vector<std::string> toks;
            for (char* t = strtok(line, " \t\r\n"); t; t = strtok(nullptr, " \t\r\n")) toks.push_back(t);
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
inline void reject_flags(const std::vector<std::string>& rest, const char* drv) {
    for (const auto& s : rest)
        if (s.rfind("--", 0) == 0) throw Err(2, std::string(drv) + ": " + s + " (claim and privacy modes) is not provided");
}

}  // namespace zkhcli
