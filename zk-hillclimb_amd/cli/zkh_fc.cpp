// zkh_fc -- a zkob_fc-compatible driver over libzkh (zkob_fc.cu:1207-1330, zkob_serve.cuh).
//
//   zkh_fc prove  <obdir> <seed> <X-int32> <W-int32> <B> <IN> <OUT> <gen_in> <gen_out> <q> [Y-int64-out]
//   zkh_fc commit <W-int32> <IN> <OUT> <gen_out> <com_out>
//   zkh_fc serve                      (one request per stdin line; "ZKW-READY", "ZKW-RC <rc>")
//
// `prove` is the reference's plain mode (zkob_fc.cu:186-486 without --claims/--wpriv/--apriv):
// Y = X W, the three Pedersen commitments of the padded tensors, the transcript absorbs, the
// matmul sumcheck and the three IPA openings, writing the same obligation files byte for
// byte: com_X.bin, com_Y.bin (raw points, G1TensorJacobian::save), dims.bin (B, IN, OUT as
// uint32), sumcheck.bin (count-prefixed evals, then claim, claim_X, claim_W: write_sumcheck,
// zkob_fc.cu:105-112), ipa_W.bin, ipa_X.bin, ipa_Y.bin (count-prefixed L and R, then
// a_final: write_ipa, vrf_common.cuh:284-289), and the optional int64 Y (save_long).
// Input files: int32 arrays (load_int_tensor, zkob_fc.cu:178-185) and raw point arrays
// (Commitment(filename), g1-tensor.cu:179-183); Q is the first point of q.bin.
// The claim, weight-privacy and activation-privacy modes, `verify` and `selftest` are not
// provided: such a request fails with exit status 2 and a message.
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/zkh.h"

namespace {

zkh_ctx* g_ctx = nullptr;

struct Err : std::runtime_error {
    int rc;
    Err(int code, const std::string& m) : std::runtime_error(m), rc(code) {}
};

void chk(int rc, const char* what) {
    if (rc) throw Err(1, std::string(what) + ": " + zkh_last_error(g_ctx));
}

std::vector<uint8_t> read_all(const std::string& path) {
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) throw Err(1, "cannot open " + path);
    std::vector<uint8_t> b;
    uint8_t buf[1 << 16];
    size_t k;
    while ((k = fread(buf, 1, sizeof(buf), f)) > 0) b.insert(b.end(), buf, buf + k);
    fclose(f);
    return b;
}
void write_all(const std::string& path, const void* p, size_t n) {
    FILE* f = fopen(path.c_str(), "wb");
    if (!f) throw Err(1, "cannot open " + path);
    if (n && fwrite(p, 1, n, f) != n) {
        fclose(f);
        throw Err(1, "short write " + path);
    }
    fclose(f);
}
// load_int_tensor: exactly `expect` int32 values must be readable
std::vector<int32_t> load_int(const std::string& path, uint64_t expect) {
    std::vector<uint8_t> b = read_all(path);
    if (b.size() < expect * 4) throw Err(1, "short read / wrong dims: " + path);
    std::vector<int32_t> v(expect);
    memcpy(v.data(), b.data(), expect * 4);
    return v;
}
std::vector<uint32_t> load_points(const std::string& path) {
    std::vector<uint8_t> b = read_all(path);
    std::vector<uint32_t> v(b.size() / 144 * 36);
    memcpy(v.data(), b.data(), v.size() * 4);
    return v;
}
uint32_t ceil_log2(uint64_t n) {
    uint32_t k = 0;
    while ((1ull << k) < n) k++;
    return k;
}
uint32_t parse_u32(const char* s) {
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

void absorb(uint8_t st[32], const char* label, const void* p, size_t n) {
    zkh_transcript_absorb(st, label, strlen(label), p, n);
}
std::vector<uint32_t> to_host(const zkh_g1* g) {
    std::vector<uint32_t> v((size_t)zkh_g1_size(g) * 36);
    chk(zkh_g1_to_host(g_ctx, g, v.data()), "g1_to_host");
    return v;
}
// write_pod_vec: uint32 count, then the items
void put_pod(std::vector<uint8_t>& out, const uint32_t* items, uint32_t count, size_t item_words) {
    const uint8_t* c = (const uint8_t*)&count;
    out.insert(out.end(), c, c + 4);
    const uint8_t* p = (const uint8_t*)items;
    out.insert(out.end(), p, p + (size_t)count * item_words * 4);
}

void ipa_file(const std::string& path, uint8_t st[32], const zkh_tensor* a, const zkh_tensor* b,
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

int do_prove(const std::vector<std::string>& a) {
    const std::string obdir = a[0], seed = a[1];
    const uint32_t B = parse_u32(a[4].c_str()), IN = parse_u32(a[5].c_str()), OUT = parse_u32(a[6].c_str());
    const uint32_t INp = 1u << ceil_log2(IN), OUTp = 1u << ceil_log2(OUT);
    std::vector<int32_t> X = load_int(a[2], (uint64_t)B * IN), W = load_int(a[3], (uint64_t)IN * OUT);
    std::vector<uint32_t> gin = load_points(a[7]), gout = load_points(a[8]), q = load_points(a[9]);
    if (q.empty()) throw Err(1, "q.bin holds no point");
    if (gin.size() / 36 != INp || gout.size() / 36 != OUTp)
        throw Err(1, "generator sizes don't match padded dims");  // zkob_fc.cu:208-209
    Tensor tX, tW, tY, Xp, Wp, Yp;
    Points g_in, g_out, cX, cW, cY;
    chk(zkh_tensor_from_i32(g_ctx, X.data(), B * IN, &tX.t), "X");
    chk(zkh_tensor_weights_i32(g_ctx, W.data(), IN, OUT, &tW.t), "W");
    chk(zkh_matmul_i32(g_ctx, tX.t, tW.t, nullptr, B, IN, OUT, &tY.t), "Y = fc(X)");
    if (a.size() > 10) {  // Y.save_long (zkob_fc.cu:213-214)
        std::vector<int64_t> y((size_t)B * OUT);
        chk(zkh_tensor_to_i64(g_ctx, tY.t, y.data()), "save_long");
        write_all(a[10], y.data(), y.size() * 8);
    }
    const uint32_t sX[2] = {B, IN}, sW[2] = {IN, OUT}, sY[2] = {B, OUT};
    chk(zkh_pad(g_ctx, tX.t, sX, 2, nullptr, &Xp.t), "pad X");
    chk(zkh_pad(g_ctx, tW.t, sW, 2, nullptr, &Wp.t), "pad W");
    chk(zkh_pad(g_ctx, tY.t, sY, 2, nullptr, &Yp.t), "pad Y");
    chk(zkh_g1_from_host(g_ctx, gin.data(), INp, &g_in.g), "gen_in");
    chk(zkh_g1_from_host(g_ctx, gout.data(), OUTp, &g_out.g), "gen_out");
    chk(zkh_commit(g_ctx, g_in.g, Xp.t, &cX.g), "commit X");
    chk(zkh_commit(g_ctx, g_out.g, Wp.t, &cW.g), "commit W");
    chk(zkh_commit(g_ctx, g_out.g, Yp.t, &cY.g), "commit Y");
    const std::vector<uint32_t> hX = to_host(cX.g), hW = to_host(cW.g), hY = to_host(cY.g);
    write_all(obdir + "/com_X.bin", hX.data(), hX.size() * 4);
    write_all(obdir + "/com_Y.bin", hY.data(), hY.size() * 4);
    const uint32_t dims[3] = {B, IN, OUT};
    write_all(obdir + "/dims.bin", dims, sizeof(dims));

    // transcript (zkob_fc.cu:254-258), then the sumcheck segment (:259-440)
    uint8_t st[32];
    zkh_transcript_init(st, seed.data(), seed.size());
    absorb(st, "B", &B, 4);
    absorb(st, "IN", &IN, 4);
    absorb(st, "OUT", &OUT, 4);
    absorb(st, "com_X", hX.data(), hX.size() * 4);
    absorb(st, "com_W", hW.data(), hW.size() * 4);
    absorb(st, "com_Y", hY.data(), hY.size() * 4);
    const uint32_t L = ceil_log2(IN), lb = ceil_log2(B), lo = ceil_log2(OUT);
    std::vector<uint32_t> ev((size_t)3 * L * 8 + 8), claims(24), ub((size_t)lb * 8 + 8), uo((size_t)lo * 8 + 8),
        ui((size_t)L * 8 + 8);
    int rc = zkh_mm_prove(g_ctx, st, tX.t, tW.t, tY.t, B, IN, OUT, ev.data(), claims.data(), ub.data(), uo.data(),
                          ui.data());
    if (rc == 2) throw Err(1, "prover sumcheck round inconsistency (witness bug)");
    chk(rc, "matmul sumcheck");
    std::vector<uint8_t> sc;
    put_pod(sc, ev.data(), 3 * L, 8);
    sc.insert(sc.end(), (uint8_t*)claims.data(), (uint8_t*)claims.data() + 96);
    write_all(obdir + "/sumcheck.bin", sc.data(), sc.size());

    // IPA openings, order W, X, Y (zkob_fc.cu:473-483)
    Tensor aW, bW, aX, bX, aY;
    chk(zkh_partial_me_window(g_ctx, Wp.t, ui.data(), L, OUTp, &aW.t), "W.partial_me");
    chk(zkh_eq_table(g_ctx, uo.data(), lo, &bW.t), "me_weights(u_output)");
    ipa_file(obdir + "/ipa_W.bin", st, aW.t, bW.t, g_out.g, q.data());
    chk(zkh_partial_me_window(g_ctx, Xp.t, ub.data(), lb, INp, &aX.t), "X.partial_me");
    chk(zkh_eq_table(g_ctx, ui.data(), L, &bX.t), "me_weights(u_input)");
    ipa_file(obdir + "/ipa_X.bin", st, aX.t, bX.t, g_in.g, q.data());
    chk(zkh_partial_me_window(g_ctx, Yp.t, ub.data(), lb, OUTp, &aY.t), "Y.partial_me");
    ipa_file(obdir + "/ipa_Y.bin", st, aY.t, bW.t, g_out.g, q.data());
    printf("PROVED matmul obligation -> %s\n", obdir.c_str());
    return 0;
}

int do_commit(const std::vector<std::string>& a) {
    const uint32_t IN = parse_u32(a[1].c_str()), OUT = parse_u32(a[2].c_str());
    std::vector<int32_t> W = load_int(a[0], (uint64_t)IN * OUT);
    std::vector<uint32_t> gout = load_points(a[3]);
    if (gout.size() / 36 != (1u << ceil_log2(OUT))) throw Err(1, "generator size doesn't match OUT_pad");
    Tensor tW, Wp;
    Points g, c;
    chk(zkh_tensor_from_i32(g_ctx, W.data(), IN * OUT, &tW.t), "W");
    const uint32_t s[2] = {IN, OUT};
    chk(zkh_pad(g_ctx, tW.t, s, 2, nullptr, &Wp.t), "pad W");
    chk(zkh_g1_from_host(g_ctx, gout.data(), (uint32_t)(gout.size() / 36), &g.g), "gen_out");
    chk(zkh_commit(g_ctx, g.g, Wp.t, &c.g), "commit W");
    const std::vector<uint32_t> h = to_host(c.g);
    write_all(a[4], h.data(), h.size() * 4);
    printf("registered commitment -> %s\n", a[4].c_str());
    return 0;
}

int run1(const std::vector<std::string>& args) {
    const std::string mode = args.empty() ? "" : args[0];
    std::vector<std::string> rest(args.begin() + (args.empty() ? 0 : 1), args.end());
    for (const auto& s : rest)
        if (s.rfind("--", 0) == 0) throw Err(2, "zkh_fc: " + s + " (claim and privacy modes) is not provided");
    const bool prove = mode == "prove" && (rest.size() == 10 || rest.size() == 11);
    const bool commit = mode == "commit" && rest.size() == 5;
    if (prove || commit) {
        if (!g_ctx && zkh_ctx_create(0, &g_ctx) != ZKH_OK) throw Err(1, "no GPU context");
        return prove ? do_prove(rest) : do_commit(rest);
    }
    fprintf(stderr,
            "usage: zkh_fc prove <obdir> <seed> <X> <W> <B> <IN> <OUT> <gen_in> <gen_out> <q> [Y-out] | "
            "commit <W> <IN> <OUT> <gen_out> <com_out> | serve\n");
    return 2;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc > 1 && std::string(argv[1]) == "serve") {
        // zkob_serve.cuh: one request per line, its exit status reported as "ZKW-RC <rc>"
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
        fprintf(stderr, "zkh_fc: %s\n", e.what());
        rc = e.rc;
    } catch (const std::exception& e) {
        fprintf(stderr, "zkh_fc: %s\n", e.what());
        rc = 1;
    }
    if (g_ctx) zkh_ctx_destroy(g_ctx);
    return rc;
}
