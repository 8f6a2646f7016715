// gdn_dropin_decode.cpp -- drives libgdn_amd.so through the call sequence of
// the reference's CPU decode driver (c_impl/gdn_eval.cpp:202-529,
// :612-690), written against include/gdn_amd.h only, so a GPU test can show
// that a caller of gdn_model.h runs unchanged:
//   gdn_model_load -> gdn_run_state_init(max_seq_len) ->
//   gdn_validate_weight_shards(run_state.weight_shards) ->
//   .gdnstate: recurrent section read INTO run_state.recurrent_state, then
//   gdn_scatter_recurrent_state(weight_shards[28..31] +
//   gdn_weight_shard_beats()), conv section through
//   gdn_pack_conv_tails_bf16(head_buffer) ->
//   gdn_set_native_debug_buffers + gdn_reset_mixed_mul_stats ->
//   per step: gdn_decode_step_host, gdn_compute_logits on the debug hidden
//   vector, a host argmax scan, the token line of workspace X_NORM ->
//   gdn_get_mixed_mul_stats, a GDNSDMP1-style dump of the state stripes and
//   the head buffer (after gdn_sync_host_state).
// Usage: gdn_dropin_decode <weights.gdnw> <state.gdnstate> <steps> <out.json> <dump.bin>
// Exit status 0 when every step's token line equals the host scan of the
// debug logits and the logits agree with the scalar LM head to
// 1e-3 + 1e-4 |ref| (the reference driver's tolerance).
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "gdn_amd.h"

static int fail(const char *what) {
    std::fprintf(stderr, "gdn_dropin_decode: %s\n", what);
    return 1;
}

int main(int argc, char **argv) {
    if (argc != 6) return fail("usage: <weights.gdnw> <state.gdnstate> <steps> <out.json> <dump.bin>");
    const unsigned steps = (unsigned)std::strtoul(argv[3], nullptr, 10);
    GDNModel model;
    if (gdn_model_load(&model, argv[1]) != 0) return fail("model load");
    GDNRunState rs;
    if (gdn_run_state_init(&rs, &model, model.config.max_seq_len) != 0) return fail("run state init");
    if (gdn_validate_weight_shards(model.weight_data, &model.config, rs.weight_shards) != 0)
        return fail("weight validation");
    const GDNWeightHeader &c = model.config;

    // the state file: header, prompt ids (skipped), recurrent and conv sections
    FILE *f = std::fopen(argv[2], "rb");
    if (!f) return fail("open state");
    char magic[8];
    uint32_t hv[9];
    if (std::fread(magic, 1, 8, f) != 8 || std::fread(hv, 4, 9, f) != 9) return fail("state header");
    const int32_t seed = (int32_t)hv[8];
    std::fseek(f, 4L * (long)hv[7], SEEK_CUR);
    const size_t rec = (size_t)hv[1] * hv[2] * hv[3] * hv[4];
    if (std::fread(rs.recurrent_state, 4, rec, f) != rec) return fail("recurrent section");
    Beat512 *stripes[GDN_RECURRENT_STATE_PORTS];
    for (int p = 0; p < GDN_RECURRENT_STATE_PORTS; ++p)
        stripes[p] = rs.weight_shards[GDN_RECURRENT_STATE_FIRST_PORT + p] + gdn_weight_shard_beats(&c);
    if (gdn_scatter_recurrent_state(stripes, rs.recurrent_state, rec) != 0) return fail("state scatter");
    const size_t conv = (size_t)hv[1] * 3u * (hv[6] - 1u) * hv[5];
    std::vector<float> tails(conv);
    if (std::fread(tails.data(), 4, conv, f) != conv) return fail("conv section");
    std::fclose(f);
    if (gdn_pack_conv_tails_bf16(reinterpret_cast<Beat512 *>(rs.head_buffer), tails.data(), conv) != 0)
        return fail("conv pack");

    std::vector<float> hidden(c.hidden_size), logits(c.vocab_size), ref(c.vocab_size);
    gdn_set_native_debug_buffers(hidden.data(), logits.data());
    gdn_reset_mixed_mul_stats();
    std::vector<int32_t> traj(steps + 1);
    traj[0] = seed;
    double max_abs = 0.0;
    unsigned tol_fail = 0, argmax_mismatch = 0;
    for (unsigned s = 1; s <= steps; ++s) {
        int32_t prev = traj[s - 1];
        if (gdn_decode_step_host(&model, &rs, &prev) != 0) return fail("decode step");
        gdn_compute_logits(&model, hidden.data(), ref.data());
        uint32_t best = 0, ref_best = 0;
        for (uint32_t v = 0; v < c.vocab_size; ++v) {
            const double err = std::fabs((double)logits[v] - (double)ref[v]);
            if (err > max_abs) max_abs = err;
            if (std::memcmp(&logits[v], &ref[v], 4) != 0 &&
                (!std::isfinite(logits[v]) || !std::isfinite(ref[v]) || err > 1e-3 + 1e-4 * std::fabs(ref[v])))
                ++tol_fail;
            if (v && logits[v] > logits[best]) best = v;
            if (v && ref[v] > ref[ref_best]) ref_best = v;
        }
        const float line = reinterpret_cast<const float *>(rs.workspace)[GDN_WS_OFF_X_NORM];
        if ((uint32_t)line != best) return fail("token line differs from the host scan of the logits");
        if (std::memcmp(rs.x, model.embeddings + (size_t)prev * c.hidden_size, 4 * c.hidden_size) != 0)
            return fail("workspace X is not the token's embedding row");
        argmax_mismatch += best != ref_best;
        traj[s] = (int32_t)best;
    }
    gdn_set_native_debug_buffers(nullptr, nullptr);
    const GDNMixedMulStats st = gdn_get_mixed_mul_stats();
    gdn_stop_mixed_mul_stats();

    // state dump: the four BF16 stripes, then the packed head buffer
    if (gdn_sync_host_state(&rs) != 0) return fail("host state sync");
    FILE *d = std::fopen(argv[5], "wb");
    if (!d) return fail("open dump");
    const char dmagic[8] = {'G', 'D', 'N', 'S', 'D', 'M', 'P', '1'};
    const uint32_t dh[4] = {GDN_RECURRENT_STATE_STRIPE_BF16_BEATS, GDN_RECURRENT_STATE_PORTS, GDN_WSF_HEADBUF / 16u, 0};
    std::fwrite(dmagic, 1, 8, d);
    std::fwrite(dh, 4, 4, d);
    for (int p = 0; p < GDN_RECURRENT_STATE_PORTS; ++p)
        std::fwrite(stripes[p], sizeof(Beat512), GDN_RECURRENT_STATE_STRIPE_BF16_BEATS, d);
    std::fwrite(rs.head_buffer, sizeof(Beat512), GDN_WSF_HEADBUF / 16u, d);
    std::fclose(d);

    FILE *o = std::fopen(argv[4], "w");
    if (!o) return fail("open output");
    std::fprintf(o, "{\"traj\": [");
    for (unsigned s = 0; s <= steps; ++s) std::fprintf(o, "%s%d", s ? ", " : "", traj[s]);
    std::fprintf(o,
                 "], \"max_abs_error\": %.9g, \"tolerance_failures\": %u, \"argmax_mismatches\": %u, "
                 "\"stats\": {\"calls\": %llu, \"special_inputs\": %llu, \"flushed_inputs\": %llu, "
                 "\"flushed_outputs\": %llu, \"overflows\": %llu}}\n",
                 max_abs, tol_fail, argmax_mismatch, (unsigned long long)st.calls,
                 (unsigned long long)st.special_inputs, (unsigned long long)st.flushed_inputs,
                 (unsigned long long)st.flushed_outputs, (unsigned long long)st.overflows);
    std::fclose(o);
    gdn_run_state_free(&rs);
    gdn_model_free(&model);
    return (tol_fail == 0) ? 0 : 2;
}
