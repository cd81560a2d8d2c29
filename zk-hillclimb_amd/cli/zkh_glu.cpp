// zkh_glu -- a zkob_glu-compatible driver over libzkh (zkob_glu.cu:67-247, :700-760).
//
//   zkh_glu prove <obdir> <seed> <G-int32> <U-int32> <B> <C> <low> <len> <mapped-int32> <gen> <q> [H-int64-out]
//   zkh_glu serve
//
// `prove` is the reference's plain mode: the mapping lookup S = mapped[G - low] with its
// multiplicities, H = S (.) U, the commitments of G, S, U, H and m, the pair combiner r and
// beta, comb = G + r S against T_comb = T + r mapped, the inverses A and their commitment,
// the logUp proof and the openings of A, comb and m; then u_h, claim_H = H~(u_h), the
// eq-weighted Hadamard sumcheck and the openings of H (at u_h), S and U (at the reversed
// Hadamard challenges).  Files, byte-identical to the reference's: dims.bin (B, C, low, len
// as int32), com_G/S/U/H/m/A.bin, lookup.bin, hp.bin (claim_H, count-prefixed evals,
// S_f2, U_f2: write_hp, zkob_lookup.cuh:272-279), ipa_A/comb/m/H/S/U.bin and the optional
// int64 H (save_long, padding rows and columns stripped).  With `--claims <accdir> <obid>`
// (claim mode, zkob_glu.cu:204-275) it also writes com_comb.bin (com_G + r com_S row by row)
// and the six openings become claims <obid>:A, :comb, :m, :H, :S, :U in <accdir>/claims.bin,
// with their witness files, witrefs.txt lines and the transcript state, for zkh_batchopen.
// `verify` and `selftest` answer exit status 2.
#include "common.hpp"

using namespace zkhcli;

namespace {

// claim_args: empty, or {accdir, obid} of the claim mode
int do_prove(const std::vector<std::string>& a, const std::vector<std::string>& claim_args) {
    const std::string obdir = a[0], seed = a[1];
    const uint32_t B = parse_u32(a[4].c_str()), C = parse_u32(a[5].c_str());
    const int32_t low = (int32_t)strtol(a[6].c_str(), nullptr, 10);
    const uint32_t len = parse_u32(a[7].c_str());
    const uint32_t Bp = 1u << ceil_log2(B), Cp = 1u << ceil_log2(C);
    const uint64_t D64 = (uint64_t)Bp * Cp;
    if (D64 >= (1ull << 32)) throw Err(1, "tensor too large");
    const uint32_t D = (uint32_t)D64, N = len, logD = ceil_log2(D), n1 = ceil_log2(D / N);
    std::vector<int32_t> G = load_int(a[2], (uint64_t)B * C), U = load_int(a[3], (uint64_t)B * C);
    // load_mapped (zkob_glu.cu:67-77)
    std::vector<int32_t> mapped = load_int(a[8], len);
    if (len != (1u << ceil_log2(len))) throw Err(1, "table len must be pow2");
    if (low > 0 || (int64_t)low + (int64_t)len <= 0) throw Err(1, "table must contain x=0");
    if (mapped[-low] != 0) throw Err(1, "layout needs mapped(0) == 0");
    std::vector<uint32_t> gen = load_points(a[9]), q = load_points(a[10]);
    if (q.empty()) throw Err(1, "q.bin holds no point");
    if (gen.size() / 36 != Cp) throw Err(1, "generator size != C_pad");
    if (Cp > N || N > D || D % N) throw Err(1, "layout needs C_pad <= N <= D, N | D");

    Tensor tG, tU, Gp, Up, Sp, m, Hp, tmap, T, comb, Tcomb, A;
    Points g, cG, cS, cU, cH, cm, cA;
    const uint32_t shape[2] = {B, C};
    chk(zkh_tensor_from_i32(g_ctx, G.data(), B * C, &tG.t), "G");
    chk(zkh_tensor_from_i32(g_ctx, U.data(), B * C, &tU.t), "U");
    chk(zkh_tensor_from_i32(g_ctx, mapped.data(), len, &tmap.t), "mapped");
    chk(zkh_pad(g_ctx, tG.t, shape, 2, nullptr, &Gp.t), "pad G");
    chk(zkh_pad(g_ctx, tU.t, shape, 2, nullptr, &Up.t), "pad U");
    chk(zkh_lu_mapping(g_ctx, Gp.t, low, tmap.t, &Sp.t, &m.t), "mapping lookup");
    chk(zkh_hadamard(g_ctx, Sp.t, Up.t, &Hp.t), "H = S . U");
    if (a.size() > 11) {  // H_pad.save_long, padding stripped (zkob_glu.cu:107-121)
        std::vector<int64_t> h(D), out((size_t)B * C);
        chk(zkh_tensor_to_i64(g_ctx, Hp.t, h.data()), "save_long");
        for (uint32_t b = 0; b < B; b++) memcpy(out.data() + (size_t)b * C, h.data() + (size_t)b * Cp, (size_t)C * 8);
        write_all(a[11], out.data(), out.size() * 8);
    }
    chk(zkh_g1_from_host(g_ctx, gen.data(), Cp, &g.g), "gen");
    chk(zkh_commit(g_ctx, g.g, Gp.t, &cG.g), "commit G");
    chk(zkh_commit(g_ctx, g.g, Sp.t, &cS.g), "commit S");
    chk(zkh_commit(g_ctx, g.g, Up.t, &cU.g), "commit U");
    chk(zkh_commit(g_ctx, g.g, Hp.t, &cH.g), "commit H");
    chk(zkh_commit(g_ctx, g.g, m.t, &cm.g), "commit m");
    const std::vector<uint32_t> hG = to_host(cG.g), hS = to_host(cS.g), hU = to_host(cU.g), hH = to_host(cH.g),
                                hm = to_host(cm.g);
    write_all(obdir + "/com_G.bin", hG.data(), hG.size() * 4);
    write_all(obdir + "/com_S.bin", hS.data(), hS.size() * 4);
    write_all(obdir + "/com_U.bin", hU.data(), hU.size() * 4);
    write_all(obdir + "/com_H.bin", hH.data(), hH.size() * 4);
    write_all(obdir + "/com_m.bin", hm.data(), hm.size() * 4);
    const int32_t dims[4] = {(int32_t)B, (int32_t)C, low, (int32_t)len};
    write_all(obdir + "/dims.bin", dims, sizeof(dims));

    // transcript (zkob_glu.cu:140-170)
    uint8_t st[32];
    zkh_transcript_init(st, seed.data(), seed.size());
    const uint32_t lowu = (uint32_t)low;
    absorb(st, "B", &B, 4);
    absorb(st, "C", &C, 4);
    absorb(st, "LOW", &lowu, 4);
    absorb(st, "LEN", &len, 4);
    absorb(st, "com_G", hG.data(), hG.size() * 4);
    absorb(st, "com_S", hS.data(), hS.size() * 4);
    absorb(st, "com_U", hU.data(), hU.size() * 4);
    absorb(st, "com_H", hH.data(), hH.size() * 4);
    absorb(st, "com_m", hm.data(), hm.size() * 4);
    const std::vector<uint32_t> r = challenge(st), beta = challenge(st);
    // comb = G + r S, T_comb = T + r mapped and A = 1/(comb + beta) (zkob_glu.cu:155-160),
    // A through the table inverse, which zkh_lu_prove then takes over (zkob_glu.cu:168-170)
    chk(zkh_lu_range_table(g_ctx, low, len, N, &T.t), "table");
    chk(zkh_lu_tuple_inverse(g_ctx, Gp.t, low, T.t, tmap.t, Sp.t, r.data(), beta.data(), &comb.t, &Tcomb.t, &A.t),
        "comb, T_comb and inverses");
    chk(zkh_commit(g_ctx, g.g, A.t, &cA.g), "commit A");
    const std::vector<uint32_t> hA = to_host(cA.g);
    write_all(obdir + "/com_A.bin", hA.data(), hA.size() * 4);
    absorb(st, "com_A", hA.data(), hA.size() * 4);
    const std::vector<uint32_t> alpha = challenge(st);
    std::vector<uint32_t> u((size_t)logD * 8 + 8);
    for (uint32_t i = 0; i < logD; i++) zkh_transcript_challenge_fr(st, u.data() + 8 * i);
    std::vector<uint32_t> ev((size_t)4 * logD * 8 + 8), term(40), ws((size_t)logD * 8 + 8);
    int rc = zkh_lu_prove(g_ctx, st, A.t, comb.t, Tcomb.t, m.t, alpha.data(), beta.data(), u.data(), ev.data(),
                          term.data(), ws.data());
    if (rc == 2) throw Err(1, "lookup round inconsistency (witness outside the table)");
    chk(rc, "lookup");
    std::vector<uint8_t> lk;
    put_pod(lk, ev.data(), 4 * logD, 8);
    for (int t : {0, 1, 4}) lk.insert(lk.end(), (uint8_t*)(term.data() + 8 * t), (uint8_t*)(term.data() + 8 * t + 8));
    write_all(obdir + "/lookup.bin", lk.data(), lk.size());
    std::vector<uint32_t> u_pt((size_t)logD * 8);
    for (uint32_t i = 0; i < logD; i++) memcpy(u_pt.data() + 8 * i, ws.data() + 8 * (logD - 1 - i), 32);
    std::vector<uint32_t> u_m(u_pt.begin(), u_pt.begin() + 8 * (size_t)(logD - n1));
    const bool claim_mode = !claim_args.empty();
    auto mk_claim = [&](const char* tensor, uint32_t n_rows, const std::vector<uint32_t>& point,
                        const uint32_t* eval) {
        const std::string &accdir = claim_args[0], &obid = claim_args[1];
        const std::string witp = accdir + "/wit_" + obid + "_" + tensor + ".fr";
        Claim c;
        c.id = obid + ":" + tensor;
        c.comref = obdir + "/com_" + tensor + ".bin";
        c.domain = Cp;
        c.n_rows = n_rows;
        c.point = point;
        memcpy(c.eval, eval, 32);
        claim_emit(accdir, c);
        witref_emit(accdir, c.comref, witp);
    };
    if (claim_mode) {  // claims A, comb, m in place of the three IPAs (zkob_glu.cu:204-227)
        Points cC;  // com_comb = com_G + r com_S row by row (hb_addmul, mul_first = false)
        chk(zkh_g1_addmul(g_ctx, cS.g, r.data(), cG.g, &cC.g), "com_comb");
        const std::vector<uint32_t> hC = to_host(cC.g);
        write_all(obdir + "/com_comb.bin", hC.data(), hC.size() * 4);
        const std::string &accdir = claim_args[0], &obid = claim_args[1];
        save_fr(accdir + "/wit_" + obid + "_A.fr", A.t);
        save_fr(accdir + "/wit_" + obid + "_comb.fr", comb.t);
        save_fr(accdir + "/wit_" + obid + "_m.fr", m.t);
        mk_claim("A", Bp, u_pt, term.data());
        mk_claim("comb", Bp, u_pt, term.data() + 8);
        mk_claim("m", N / Cp, u_m, term.data() + 32);
    } else {
        open_prove(A.t, Cp, g.g, q.data(), u_pt, obdir + "/ipa_A.bin", st);
        open_prove(comb.t, Cp, g.g, q.data(), u_pt, obdir + "/ipa_comb.bin", st);
        open_prove(m.t, Cp, g.g, q.data(), u_m, obdir + "/ipa_m.bin", st);
    }

    // Hadamard part (zkob_glu.cu:242-247): u_h, claim_H = H~(u_h) (columns on the low bits)
    std::vector<uint32_t> uh((size_t)logD * 8 + 8);
    for (uint32_t i = 0; i < logD; i++) zkh_transcript_challenge_fr(st, uh.data() + 8 * i);
    uint32_t claimH[8];
    chk(zkh_me(g_ctx, Hp.t, uh.data(), logD, claimH), "claim_H");
    absorb(st, "claim_H", claimH, 32);
    std::vector<uint32_t> hev((size_t)4 * logD * 8 + 8), hterm(24), hws((size_t)logD * 8 + 8);
    rc = zkh_hp_prove_eq(g_ctx, st, claimH, uh.data(), logD, Sp.t, Up.t, hev.data(), hterm.data(), hws.data());
    if (rc == 2) throw Err(1, "hadamard round inconsistency");
    chk(rc, "hadamard");
    absorb(st, "S_f2", hterm.data(), 32);
    absorb(st, "U_f2", hterm.data() + 8, 32);
    std::vector<uint8_t> hp((uint8_t*)claimH, (uint8_t*)claimH + 32);
    put_pod(hp, hev.data(), 4 * logD, 8);
    hp.insert(hp.end(), (uint8_t*)hterm.data(), (uint8_t*)hterm.data() + 64);
    write_all(obdir + "/hp.bin", hp.data(), hp.size());
    std::vector<uint32_t> u_pt2((size_t)logD * 8);
    for (uint32_t i = 0; i < logD; i++) memcpy(u_pt2.data() + 8 * i, hws.data() + 8 * (logD - 1 - i), 32);
    std::vector<uint32_t> uhv(uh.begin(), uh.begin() + 8 * (size_t)logD);
    if (claim_mode) {  // claims H, S, U in place of the three IPAs (zkob_glu.cu:259-275)
        const std::string &accdir = claim_args[0], &obid = claim_args[1];
        save_fr(accdir + "/wit_" + obid + "_H.fr", Hp.t);
        save_fr(accdir + "/wit_" + obid + "_S.fr", Sp.t);
        save_fr(accdir + "/wit_" + obid + "_U.fr", Up.t);
        mk_claim("H", Bp, uhv, claimH);
        mk_claim("S", Bp, u_pt2, hterm.data());
        mk_claim("U", Bp, u_pt2, hterm.data() + 8);
        drvstate_emit(accdir, obid, st);
        printf("PROVED swiglu obligation (claim mode, 6 claims emitted) -> %s\n", obdir.c_str());
        return 0;
    }
    open_prove(Hp.t, Cp, g.g, q.data(), uhv, obdir + "/ipa_H.bin", st);
    open_prove(Sp.t, Cp, g.g, q.data(), u_pt2, obdir + "/ipa_S.bin", st);
    open_prove(Up.t, Cp, g.g, q.data(), u_pt2, obdir + "/ipa_U.bin", st);
    printf("PROVED swiglu obligation -> %s\n", obdir.c_str());
    return 0;
}

int run1(const std::vector<std::string>& args) {
    const std::string mode = args.empty() ? "" : args[0];
    std::vector<std::string> rest(args.begin() + (args.empty() ? 0 : 1), args.end());
    const std::vector<std::string> claim_args = take_claims(rest, 2);  // --claims <accdir> <obid>
    reject_flags(rest, "zkh_glu");
    if (mode == "prove" && (rest.size() == 11 || rest.size() == 12)) {
        need_ctx();
        return do_prove(rest, claim_args);
    }
    fprintf(stderr,
            "usage: zkh_glu prove <obdir> <seed> <G> <U> <B> <C> <low> <len> <mapped> <gen> <q> [H-out] "
            "[--claims <accdir> <obid>] | serve\n");
    return 2;
}

}  // namespace

int main(int argc, char** argv) { return driver_main(argc, argv, run1); }
