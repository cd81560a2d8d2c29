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
// `--claims <accdir> <obid> <com_W>` is the claim mode (zkob_fc.cu:449-470): the IPAs are
// replaced by three claims appended to <accdir>/claims.bin (ids <obid>:W, :X, :Y; comrefs
// <com_W>, <obdir>/com_X.bin, <obdir>/com_Y.bin), the padded witnesses saved as
// <accdir>/wit_<obid>_{W,X,Y}.fr with their witrefs.txt lines, and the transcript state in
// drvstates.bin; zkh_batchopen later opens them all in one batch.  The weight-privacy and
// activation-privacy modes, `verify` and `selftest` are not provided: such a request fails
// with exit status 2 and a message.
#include "common.hpp"

using namespace zkhcli;

namespace {

// --claims <accdir> <obid> <registered-com_W-path> (zkob_fc.cu:1224-1228)
struct ClaimMode {
    std::string accdir, obid, comW;
    bool on() const { return !accdir.empty(); }
};

int do_prove(const std::vector<std::string>& a, const ClaimMode& cm) {
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

    if (cm.on()) {  // claim emission in place of the IPAs, order W, X, Y (zkob_fc.cu:449-470)
        const std::string witW = cm.accdir + "/wit_" + cm.obid + "_W.fr", witX = cm.accdir + "/wit_" + cm.obid + "_X.fr",
                          witY = cm.accdir + "/wit_" + cm.obid + "_Y.fr";
        save_fr(witW, Wp.t);
        save_fr(witX, Xp.t);
        save_fr(witY, Yp.t);
        auto mk = [&](const char* tensor, const std::string& comref, uint32_t domain, uint32_t n_rows,
                      const std::vector<uint32_t>& ucol, uint32_t ncol, const std::vector<uint32_t>& urow,
                      uint32_t nrow, const uint32_t* eval) {
            Claim c;
            c.id = cm.obid + ":" + tensor;
            c.comref = comref;
            c.domain = domain;
            c.n_rows = n_rows;
            c.point.assign(ucol.begin(), ucol.begin() + 8 * (size_t)ncol);
            c.point.insert(c.point.end(), urow.begin(), urow.begin() + 8 * (size_t)nrow);
            memcpy(c.eval, eval, 32);
            claim_emit(cm.accdir, c);
        };
        const uint32_t Bp = 1u << lb;
        mk("W", cm.comW, OUTp, INp, uo, lo, ui, L, claims.data() + 16);
        witref_emit(cm.accdir, cm.comW, witW);
        mk("X", obdir + "/com_X.bin", INp, Bp, ui, L, ub, lb, claims.data() + 8);
        witref_emit(cm.accdir, obdir + "/com_X.bin", witX);
        mk("Y", obdir + "/com_Y.bin", OUTp, Bp, uo, lo, ub, lb, claims.data());
        witref_emit(cm.accdir, obdir + "/com_Y.bin", witY);
        drvstate_emit(cm.accdir, cm.obid, st);
        printf("PROVED matmul obligation (claim mode, 3 claims emitted) -> %s\n", obdir.c_str());
        return 0;
    }

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
    ClaimMode cm;
    for (size_t i = 0; i < rest.size(); i++) {
        if (rest[i] != "--claims") continue;
        if (i + 4 > rest.size()) throw Err(1, "--claims needs <accdir> <obid> <com_W>");
        cm.accdir = rest[i + 1];
        cm.obid = rest[i + 2];
        cm.comW = rest[i + 3];
        rest.erase(rest.begin() + i, rest.begin() + i + 4);
        break;
    }
    if (cm.on() && mode != "prove") throw Err(1, "--claims applies to prove only");
    reject_flags(rest, "zkh_fc");
    const bool prove = mode == "prove" && (rest.size() == 10 || rest.size() == 11);
    const bool commit = mode == "commit" && rest.size() == 5;
    if (prove || commit) {
        need_ctx();
        return prove ? do_prove(rest, cm) : do_commit(rest);
    }
    fprintf(stderr,
            "usage: zkh_fc prove <obdir> <seed> <X> <W> <B> <IN> <OUT> <gen_in> <gen_out> <q> [Y-out] "
            "[--claims <accdir> <obid> <com_W>] | "
            "commit <W> <IN> <OUT> <gen_out> <com_out> | serve\n");
    return 2;
}

}  // namespace

int main(int argc, char** argv) { return driver_main(argc, argv, run1); }
