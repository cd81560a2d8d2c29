// zkh_rope -- a zkob_rope-compatible driver over libzkh (zkob_rope.cu:72-114, prove, CLI).
//
//   zkh_rope prove <obdir> <seed> <T-int32> <B> <C> <HD> <cos-int32> <sin-int32> <gen> <q> [Y64-int64-out]
//   zkh_rope serve
//
// `prove` is the reference's plain mode for the integer RoPE relation
//   Y64[t,e] = T[t,e] W1[t,e] + T[t, e ^ HD/2] W2[t,e],  W1 = cos, W2 = +-sin (sign by bit HD/2)
// on the B x C_pad grid: commitments of T and Y64, the challenge point u, ev = Y64~(u),
// two eq-weighted Hadamard sumchecks (c1 over eq(u).W1 and T, c2 over eq(u).W2 and the
// column-flipped T, U = 1 in both), the openings of T at both terminal points (the second
// with coordinate log2(HD)-1 replaced by its complement) and of Y64 at u.  Files,
// byte-identical to the reference's: dims.bin (B, C, HD, 16), com_T.bin, com_Y64.bin,
// ev.bin, hp1.bin, hp2.bin, ipa_T1.bin, ipa_T2.bin, ipa_Y.bin and the optional unpadded
// int64 Y64.  With `--claims <accdir> <obid>` (claim mode, zkob_rope.cu:250-304) the openings
// become claims <obid>:T1, :T2 (both on com_T.bin) and :Y in <accdir>/claims.bin, with the
// witness files, witrefs.txt lines and the transcript state, for zkh_batchopen.  `verify` and
// `selftest` answer exit status 2.
#include <stdlib.h>

#include "common.hpp"

using namespace zkhcli;

namespace {

const uint32_t SCALE_R = 16;  // table scale 2^16 (zkob_rope.cu:72)
const uint32_t kR[8] = {0x00000001u, 0xffffffffu, 0xfffe5bfeu, 0x53bda402u,
                        0x09a1d805u, 0x3339d808u, 0x299d7d48u, 0x73eda753u};

// 1 - x mod r for a canonical x (h_scalar(F_ONE, x, 1) at zkob_rope.cu pt2p)
void one_minus(const uint32_t* x, uint32_t* out) {
    uint32_t s[8], d[8];
    uint64_t c = 1;  // s = r + 1
    for (int i = 0; i < 8; i++) {
        const uint64_t v = (uint64_t)kR[i] + c;
        s[i] = (uint32_t)v;
        c = v >> 32;
    }
    uint64_t br = 0;  // d = s - x (x < r < s: no borrow out)
    for (int i = 0; i < 8; i++) {
        const uint64_t v = (uint64_t)s[i] - x[i] - br;
        d[i] = (uint32_t)v;
        br = (v >> 63) & 1;
    }
    bool ge = true;  // d >= r ?
    for (int i = 7; i >= 0; i--)
        if (d[i] != kR[i]) {
            ge = d[i] > kR[i];
            break;
        }
    if (ge) {
        br = 0;
        for (int i = 0; i < 8; i++) {
            const uint64_t v = (uint64_t)d[i] - kR[i] - br;
            d[i] = (uint32_t)v;
            br = (v >> 63) & 1;
        }
    }
    memcpy(out, d, 32);
}

std::vector<int32_t> load_table(const std::string& path, uint32_t B, uint32_t HD) {
    std::vector<uint8_t> b = read_all(path);
    if (b.size() != (size_t)B * HD * 4) throw Err(1, "table file size != B*HD int32: " + path);  // :86-97
    std::vector<int32_t> v((size_t)B * HD);
    memcpy(v.data(), b.data(), b.size());
    return v;
}

void hp_file(const std::string& path, const uint32_t claim[8], const std::vector<uint32_t>& ev, uint32_t rounds,
             const uint32_t* term) {
    std::vector<uint8_t> out((uint8_t*)claim, (uint8_t*)claim + 32);
    put_pod(out, ev.data(), 4 * rounds, 8);
    out.insert(out.end(), (const uint8_t*)term, (const uint8_t*)term + 64);
    write_all(path, out.data(), out.size());
}

// claim_args: empty, or {accdir, obid} of the claim mode
int do_prove(const std::vector<std::string>& a, const std::vector<std::string>& claim_args) {
    const std::string obdir = a[0], seed = a[1];
    const uint32_t B = parse_u32(a[3].c_str()), C = parse_u32(a[4].c_str()), HD = parse_u32(a[5].c_str());
    const uint32_t Cp = 1u << ceil_log2(C);
    // layout guards (zkob_rope.cu:75-83)
    if (B != (1u << ceil_log2(B))) throw Err(1, "B not a power of two");
    if (HD < 2 || HD != (1u << ceil_log2(HD))) throw Err(1, "HD must be a power of two >= 2");
    if (C % HD) throw Err(1, "HD must divide C");
    if (Cp % HD) throw Err(1, "HD must divide C_pad");
    if (C / HD < 2) throw Err(1, "NH = C/HD must be >= 2");
    const uint64_t D64 = (uint64_t)B * Cp;
    if (D64 >= (1ull << 31)) throw Err(1, "tensor too large");
    const uint32_t D = (uint32_t)D64, logCp = ceil_log2(Cp), logD = ceil_log2(B) + logCp;
    const uint32_t flipv = HD / 2, fb = ceil_log2(HD) - 1;
    std::vector<int32_t> Th = load_int(a[2], (uint64_t)B * C);
    std::vector<int32_t> cosT = load_table(a[6], B, HD), sinT = load_table(a[7], B, HD);
    std::vector<uint32_t> gen = load_points(a[8]), q = load_points(a[9]);
    if (q.empty()) throw Err(1, "q.bin holds no point");
    if (gen.size() / 36 != Cp) throw Err(1, "generator size != C_pad");

    // weights, padded T, its column flip and Y64 (build_weights, zkob_rope.cu:102-114)
    std::vector<int32_t> W1(D, 0), W2(D, 0), Tg(D, 0), Txg(D), ones(D, 1);
    std::vector<int64_t> Yg(D, 0);
    for (uint32_t t = 0; t < B; t++)
        for (uint32_t e = 0; e < C; e++) {
            const size_t g = (size_t)t * Cp + e;
            W1[g] = cosT[(size_t)t * HD + e % HD];
            W2[g] = ((e & flipv) ? 1 : -1) * sinT[(size_t)t * HD + e % HD];
            Tg[g] = Th[(size_t)t * C + e];
        }
    for (uint32_t t = 0; t < B; t++)
        for (uint32_t e = 0; e < Cp; e++) Txg[(size_t)t * Cp + e] = Tg[(size_t)t * Cp + (e ^ flipv)];
    for (size_t g = 0; g < D; g++) {
        Yg[g] = (int64_t)Tg[g] * W1[g] + (int64_t)Txg[g] * W2[g];
        if (llabs(Yg[g]) >= (1LL << 47)) throw Err(1, "|Y64| >= 2^47 (int32 chain format after rescale at risk)");
    }
    if (a.size() > 10) {  // chain file: unpadded B x C int64
        std::vector<int64_t> yo((size_t)B * C);
        for (uint32_t t = 0; t < B; t++)
            for (uint32_t e = 0; e < C; e++) yo[(size_t)t * C + e] = Yg[(size_t)t * Cp + e];
        write_all(a[10], yo.data(), yo.size() * 8);
    }
    Tensor tT, tTx, tW1, tW2, tY, tU, Eu, E1, E2;
    Points g, cT, cY;
    chk(zkh_tensor_from_i32(g_ctx, Tg.data(), D, &tT.t), "T");
    chk(zkh_tensor_from_i32(g_ctx, Txg.data(), D, &tTx.t), "Tx");
    chk(zkh_tensor_from_i32(g_ctx, W1.data(), D, &tW1.t), "W1");
    chk(zkh_tensor_from_i32(g_ctx, W2.data(), D, &tW2.t), "W2");
    chk(zkh_tensor_from_i64(g_ctx, Yg.data(), D, &tY.t), "Y64");
    chk(zkh_tensor_from_i32(g_ctx, ones.data(), D, &tU.t), "U");
    chk(zkh_g1_from_host(g_ctx, gen.data(), Cp, &g.g), "gen");
    chk(zkh_commit(g_ctx, g.g, tT.t, &cT.g), "commit T");
    chk(zkh_commit(g_ctx, g.g, tY.t, &cY.g), "commit Y64");
    const std::vector<uint32_t> hT = to_host(cT.g), hY = to_host(cY.g);
    write_all(obdir + "/com_T.bin", hT.data(), hT.size() * 4);
    write_all(obdir + "/com_Y64.bin", hY.data(), hY.size() * 4);
    const uint32_t dims[4] = {B, C, HD, SCALE_R};
    write_all(obdir + "/dims.bin", dims, sizeof(dims));

    uint8_t st[32];
    zkh_transcript_init(st, seed.data(), seed.size());
    absorb(st, "B", &B, 4);
    absorb(st, "C", &C, 4);
    absorb(st, "HD", &HD, 4);
    absorb(st, "SCALE_R", &SCALE_R, 4);
    absorb(st, "com_T", hT.data(), hT.size() * 4);
    absorb(st, "com_Y64", hY.data(), hY.size() * 4);
    std::vector<uint32_t> u((size_t)logD * 8);
    for (uint32_t i = 0; i < logD; i++) zkh_transcript_challenge_fr(st, u.data() + 8 * i);
    uint32_t ev[8];
    chk(zkh_me(g_ctx, tY.t, u.data(), logD, ev), "ev = Y64~(u)");  // columns on the low bits
    absorb(st, "ev", ev, 32);
    write_all(obdir + "/ev.bin", ev, 32);
    chk(zkh_eq_table(g_ctx, u.data(), logD, &Eu.t), "eq(u)");

    // hadamard 1: E = eq(u).W1, S = T, U = 1; c1 = sum E S U absorbed, then the sumcheck
    // (zkob_rope.cu:230-238), the claim taken from the first round's sums
    uint32_t c1[8], c2[8];
    chk(zkh_hadamard(g_ctx, Eu.t, tW1.t, &E1.t), "E1");
    std::vector<uint32_t> hev((size_t)4 * logD * 8 + 8), hterm(24), hws((size_t)logD * 8 + 8);
    int rc = zkh_hp_prove_claim(g_ctx, st, "c1", E1.t, tT.t, tU.t, c1, hev.data(), hterm.data(), hws.data());
    if (rc == 2) throw Err(1, "hadamard 1 round inconsistency");
    chk(rc, "hadamard 1");
    absorb(st, "S_f2", hterm.data(), 32);
    absorb(st, "U_f2", hterm.data() + 8, 32);
    hp_file(obdir + "/hp1.bin", c1, hev, logD, hterm.data());
    std::vector<uint32_t> pt((size_t)logD * 8);
    for (uint32_t i = 0; i < logD; i++) memcpy(pt.data() + 8 * i, hws.data() + 8 * (logD - 1 - i), 32);
    // claim mode (zkob_rope.cu:250-268, :296-304): claims T1 (here), T2 and Y replace the IPAs
    const bool claim_mode = !claim_args.empty();
    auto mk_claim = [&](const char* tensor, const char* com, const std::vector<uint32_t>& point,
                        const uint32_t* eval) {
        Claim c;
        c.id = claim_args[1] + ":" + tensor;
        c.comref = obdir + "/" + com;
        c.domain = Cp;
        c.n_rows = B;
        c.point = point;
        memcpy(c.eval, eval, 32);
        claim_emit(claim_args[0], c);
    };
    if (claim_mode) {
        const std::string witT = claim_args[0] + "/wit_" + claim_args[1] + "_T.fr";
        save_fr(witT, tT.t);
        mk_claim("T1", "com_T.bin", pt, hterm.data());
        witref_emit(claim_args[0], obdir + "/com_T.bin", witT);
    } else {
        open_prove(tT.t, Cp, g.g, q.data(), pt, obdir + "/ipa_T1.bin", st);
    }

    // hadamard 2: E = eq(u).W2, S = column-flipped T, U = 1
    chk(zkh_hadamard(g_ctx, Eu.t, tW2.t, &E2.t), "E2");
    rc = zkh_hp_prove_claim(g_ctx, st, "c2", E2.t, tTx.t, tU.t, c2, hev.data(), hterm.data(), hws.data());
    if (rc == 2) throw Err(1, "hadamard 2 round inconsistency");
    chk(rc, "hadamard 2");
    absorb(st, "S_f2", hterm.data(), 32);
    absorb(st, "U_f2", hterm.data() + 8, 32);
    hp_file(obdir + "/hp2.bin", c2, hev, logD, hterm.data());
    for (uint32_t i = 0; i < logD; i++) memcpy(pt.data() + 8 * i, hws.data() + 8 * (logD - 1 - i), 32);
    one_minus(pt.data() + 8 * fb, pt.data() + 8 * fb);  // rotate_half: T~(pt2') = Tx~(pt2)
    if (claim_mode) {
        mk_claim("T2", "com_T.bin", pt, hterm.data());
        const std::string witY = claim_args[0] + "/wit_" + claim_args[1] + "_Y.fr";
        save_fr(witY, tY.t);
        mk_claim("Y", "com_Y64.bin", u, ev);
        witref_emit(claim_args[0], obdir + "/com_Y64.bin", witY);
        drvstate_emit(claim_args[0], claim_args[1], st);
        printf("PROVED rope obligation (claim mode, 3 claims emitted) -> %s\n", obdir.c_str());
        return 0;
    }
    open_prove(tT.t, Cp, g.g, q.data(), pt, obdir + "/ipa_T2.bin", st);
    open_prove(tY.t, Cp, g.g, q.data(), u, obdir + "/ipa_Y.bin", st);
    printf("PROVED rope obligation -> %s\n", obdir.c_str());
    return 0;
}

int run1(const std::vector<std::string>& args) {
    const std::string mode = args.empty() ? "" : args[0];
    std::vector<std::string> rest(args.begin() + (args.empty() ? 0 : 1), args.end());
    const std::vector<std::string> claim_args = take_claims(rest, 2);  // --claims <accdir> <obid>
    reject_flags(rest, "zkh_rope");
    if (mode == "prove" && (rest.size() == 10 || rest.size() == 11)) {
        need_ctx();
        return do_prove(rest, claim_args);
    }
    fprintf(stderr,
            "usage: zkh_rope prove <obdir> <seed> <T> <B> <C> <HD> <cos> <sin> <gen> <q> [Y64-out] "
            "[--claims <accdir> <obid>] | serve\n");
    return 2;
}

}  // namespace

int main(int argc, char** argv) { return driver_main(argc, argv, run1); }
