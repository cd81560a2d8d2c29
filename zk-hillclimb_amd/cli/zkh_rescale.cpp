// zkh_rescale -- a zkob_rescale-compatible driver over libzkh (zkob_rescale.cu:70-197, :521-580).
//
//   zkh_rescale prove <obdir> <seed> <X-int64> <B> <C> <LOG_SF> <gen> <q> [Xr-int32-out]
//   zkh_rescale serve
//
// `prove` is the reference's plain mode: the rescaling witness X = sf Xr + rem, the
// multiplicities of rem against the range table [-sf/2, sf/2), the commitments of the padded
// X, Xr, rem and of m, beta, the inverses A = 1/(rem + beta) and their commitment, alpha and
// u, the logUp proof, and the openings of A, rem (at the reversed round challenges) and m (at
// their first log N), writing dims.bin (B, C, LOG_SF), com_X.bin, com_Xr.bin, com_rem.bin,
// com_m.bin, com_A.bin, lookup.bin (count-prefixed evals, then A_f, S_f, m_f: write_lookup,
// zkob_lookup.cuh:80-87), ipa_A.bin, ipa_rem.bin, ipa_m.bin and the optional int32 Xr
// (save_int), byte-identical to the reference's.  With `--claims <accdir> <obid>` (claim
// mode, zkob_rescale.cu:165-190) the three openings become claims <obid>:A, :rem, :m in
// <accdir>/claims.bin, with their witness files, witrefs.txt lines and the transcript state
// in drvstates.bin, for zkh_batchopen.  `verify` and `selftest` answer exit status 2.
#include "common.hpp"

using namespace zkhcli;

namespace {

// claim_args: empty, or {accdir, obid} of the claim mode
int do_prove(const std::vector<std::string>& a, const std::vector<std::string>& claim_args) {
    const std::string obdir = a[0], seed = a[1];
    const uint32_t B = parse_u32(a[3].c_str()), C = parse_u32(a[4].c_str());
    const uint32_t log_sf = (uint32_t)strtoul(a[5].c_str(), nullptr, 10);
    if (log_sf < 1 || log_sf > 30) throw Err(1, "bad LOG_SF: " + a[5]);
    const uint32_t sf = 1u << log_sf, Bp = 1u << ceil_log2(B), Cp = 1u << ceil_log2(C);
    const uint64_t D64 = (uint64_t)Bp * Cp;
    if (D64 >= (1ull << 32)) throw Err(1, "tensor too large");
    const uint32_t D = (uint32_t)D64, N = sf, logD = ceil_log2(D), n1 = ceil_log2(D / N);
    std::vector<int64_t> X = load_long(a[2], (uint64_t)B * C);
    std::vector<uint32_t> gen = load_points(a[6]), q = load_points(a[7]);
    if (q.empty()) throw Err(1, "q.bin holds no point");
    if (gen.size() / 36 != Cp) throw Err(1, "generator size != C_pad");  // zkob_rescale.cu:79
    if (Cp > N || N > D || D % N) throw Err(1, "layout needs C_pad <= N <= D, N | D");
    const int32_t low = -(int32_t)(sf >> 1);

    Tensor tX, Xr, rem, T, Xp, Xrp, remp, m, A;
    Points g, cX, cXr, crem, cm, cA;
    chk(zkh_tensor_from_i64(g_ctx, X.data(), B * C, &tX.t), "X");
    chk(zkh_rescale(g_ctx, tX.t, sf, &Xr.t, &rem.t), "rescaling");
    if (a.size() > 8) {  // Xr.save_int
        std::vector<int64_t> v((size_t)B * C);
        chk(zkh_tensor_to_i64(g_ctx, Xr.t, v.data()), "save_int");
        std::vector<int32_t> w(v.begin(), v.end());
        write_all(a[8], w.data(), w.size() * 4);
    }
    const uint32_t shape[2] = {B, C};
    chk(zkh_pad(g_ctx, tX.t, shape, 2, nullptr, &Xp.t), "pad X");
    chk(zkh_pad(g_ctx, Xr.t, shape, 2, nullptr, &Xrp.t), "pad Xr");
    chk(zkh_pad(g_ctx, rem.t, shape, 2, nullptr, &remp.t), "pad rem");
    chk(zkh_lu_range_table(g_ctx, low, sf, N, &T.t), "range table");
    chk(zkh_lu_prep(g_ctx, remp.t, low, N, &m.t), "multiplicities");
    chk(zkh_g1_from_host(g_ctx, gen.data(), Cp, &g.g), "gen");
    chk(zkh_commit(g_ctx, g.g, Xp.t, &cX.g), "commit X");
    chk(zkh_commit(g_ctx, g.g, Xrp.t, &cXr.g), "commit Xr");
    chk(zkh_commit(g_ctx, g.g, remp.t, &crem.g), "commit rem");
    chk(zkh_commit(g_ctx, g.g, m.t, &cm.g), "commit m");
    const std::vector<uint32_t> hX = to_host(cX.g), hXr = to_host(cXr.g), hrem = to_host(crem.g), hm = to_host(cm.g);
    write_all(obdir + "/com_X.bin", hX.data(), hX.size() * 4);
    write_all(obdir + "/com_Xr.bin", hXr.data(), hXr.size() * 4);
    write_all(obdir + "/com_rem.bin", hrem.data(), hrem.size() * 4);
    write_all(obdir + "/com_m.bin", hm.data(), hm.size() * 4);
    const uint32_t dims[3] = {B, C, log_sf};
    write_all(obdir + "/dims.bin", dims, sizeof(dims));

    // transcript (zkob_rescale.cu:113-129)
    uint8_t st[32];
    zkh_transcript_init(st, seed.data(), seed.size());
    absorb(st, "B", &B, 4);
    absorb(st, "C", &C, 4);
    absorb(st, "LOG_SF", &log_sf, 4);
    absorb(st, "com_X", hX.data(), hX.size() * 4);
    absorb(st, "com_Xr", hXr.data(), hXr.size() * 4);
    absorb(st, "com_rem", hrem.data(), hrem.size() * 4);
    absorb(st, "com_m", hm.data(), hm.size() * 4);
    const std::vector<uint32_t> beta = challenge(st);
    // A = 1/(rem + beta) (zkob_rescale.cu:121-123) through the table inverse, which
    // zkh_lu_prove then takes over
    chk(zkh_lu_range_inverse(g_ctx, remp.t, low, T.t, beta.data(), &A.t), "inverses");
    chk(zkh_commit(g_ctx, g.g, A.t, &cA.g), "commit A");
    const std::vector<uint32_t> hA = to_host(cA.g);
    write_all(obdir + "/com_A.bin", hA.data(), hA.size() * 4);
    absorb(st, "com_A", hA.data(), hA.size() * 4);
    const std::vector<uint32_t> alpha = challenge(st);
    std::vector<uint32_t> u((size_t)logD * 8 + 8);
    for (uint32_t i = 0; i < logD; i++) zkh_transcript_challenge_fr(st, u.data() + 8 * i);
    std::vector<uint32_t> ev((size_t)4 * logD * 8 + 8), term(40), ws((size_t)logD * 8 + 8);
    int rc = zkh_lu_prove(g_ctx, st, A.t, remp.t, T.t, m.t, alpha.data(), beta.data(), u.data(), ev.data(),
                          term.data(), ws.data());
    if (rc == 2) throw Err(1, "lookup round inconsistency (witness outside the table)");
    chk(rc, "lookup");
    std::vector<uint8_t> lk;
    put_pod(lk, ev.data(), 4 * logD, 8);
    for (int t : {0, 1, 4}) lk.insert(lk.end(), (uint8_t*)(term.data() + 8 * t), (uint8_t*)(term.data() + 8 * t + 8));
    write_all(obdir + "/lookup.bin", lk.data(), lk.size());

    // opening points: the reversed round challenges, and for m their first log N
    std::vector<uint32_t> u_pt((size_t)logD * 8);
    for (uint32_t i = 0; i < logD; i++) memcpy(u_pt.data() + 8 * i, ws.data() + 8 * (logD - 1 - i), 32);
    std::vector<uint32_t> u_m(u_pt.begin(), u_pt.begin() + 8 * (size_t)(logD - n1));
    if (!claim_args.empty()) {  // claim emission in place of the IPAs, order A, rem, m (zkob_rescale.cu:165-190)
        const std::string &accdir = claim_args[0], &obid = claim_args[1];
        const std::string witA = accdir + "/wit_" + obid + "_A.fr", witR = accdir + "/wit_" + obid + "_rem.fr",
                          witM = accdir + "/wit_" + obid + "_m.fr";
        save_fr(witA, A.t);
        save_fr(witR, remp.t);
        save_fr(witM, m.t);
        auto mk = [&](const char* tensor, uint32_t n_rows, const std::vector<uint32_t>& pt, const uint32_t* eval) {
            Claim c;
            c.id = obid + ":" + tensor;
            c.comref = obdir + "/com_" + tensor + ".bin";
            c.domain = Cp;
            c.n_rows = n_rows;
            c.point = pt;
            memcpy(c.eval, eval, 32);
            claim_emit(accdir, c);
        };
        mk("A", Bp, u_pt, term.data());
        witref_emit(accdir, obdir + "/com_A.bin", witA);
        mk("rem", Bp, u_pt, term.data() + 8);
        witref_emit(accdir, obdir + "/com_rem.bin", witR);
        mk("m", N / Cp, u_m, term.data() + 32);
        witref_emit(accdir, obdir + "/com_m.bin", witM);
        drvstate_emit(accdir, obid, st);
        printf("PROVED rescaling obligation (claim mode, 3 claims emitted) -> %s\n", obdir.c_str());
        return 0;
    }
    open_prove(A.t, Cp, g.g, q.data(), u_pt, obdir + "/ipa_A.bin", st);
    open_prove(remp.t, Cp, g.g, q.data(), u_pt, obdir + "/ipa_rem.bin", st);
    open_prove(m.t, Cp, g.g, q.data(), u_m, obdir + "/ipa_m.bin", st);
    printf("PROVED rescaling obligation -> %s\n", obdir.c_str());
    return 0;
}

int run1(const std::vector<std::string>& args) {
    const std::string mode = args.empty() ? "" : args[0];
    std::vector<std::string> rest(args.begin() + (args.empty() ? 0 : 1), args.end());
    const std::vector<std::string> cm = take_claims(rest, 2);  // --claims <accdir> <obid> (zkob_rescale.cu:528-532)
    reject_flags(rest, "zkh_rescale");
    if (mode == "prove" && (rest.size() == 8 || rest.size() == 9)) {
        need_ctx();
        return do_prove(rest, cm);
    }
    fprintf(stderr,
            "usage: zkh_rescale prove <obdir> <seed> <X-int64> <B> <C> <LOG_SF> <gen> <q> [Xr-out] "
            "[--claims <accdir> <obid>] | serve\n");
    return 2;
}

}  // namespace

int main(int argc, char** argv) { return driver_main(argc, argv, run1); }
