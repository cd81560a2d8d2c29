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
#include "common.hpp"

using namespace zkhcli;

namespace {

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
    reject_flags(rest, "zkh_fc");
    const bool prove = mode == "prove" && (rest.size() == 10 || rest.size() == 11);
    const bool commit = mode == "commit" && rest.size() == 5;
    if (prove || commit) {
        need_ctx();
        return prove ? do_prove(rest) : do_commit(rest);
    }
    fprintf(stderr,
            "usage: zkh_fc prove <obdir> <seed> <X> <W> <B> <IN> <OUT> <gen_in> <gen_out> <q> [Y-out] | "
            "commit <W> <IN> <OUT> <gen_out> <com_out> | serve\n");
    return 2;
}

}  // namespace

int main(int argc, char** argv) { return driver_main(argc, argv, run1); }
