// gdn_eval_amd.cpp -- command-line driver over libgdn_amd.so.
//
// It offers the decode-only interface of the reference's c_impl/gdn_eval
// (gdn_eval.cpp:269-529, :556-640), plus the steady-state token-stream
// benchmark (host.cpp:2116-2256) and the rolling teacher-forced scoring
// (host.cpp:1940-2030) of c_impl/host.cpp, on the MI355X engine:
//
//   gdn_eval_amd <weights.gdnw> [fixture.gdnreq] [output.json]
//       --decode-from-state <state.gdnstate> [--decode-len N]
//       [--logits-dump F] [--logits-reference F] [--hidden-dump F]
//       [--dump-state F] [--save-gdnstate F] [--interstep-delay-ms N]
//       [--no-host-check]
//   gdn_eval_amd <weights.gdnw> [output.json] --decode-from-state <state>
//       --benchmark-tokens <tokens.txt> [--benchmark-idle-seconds N]
//       [--benchmark-warmup-seconds N] [--benchmark-interval-seconds N]
//       [--benchmark-intervals N]   (the reference's timed protocol, its
//       defaults 60 / 30 / 60 / 3), or a fixed count: [--benchmark-steps N]
//       [--benchmark-warmup N]
//   gdn_eval_amd <weights.gdnw> <rolling.gdnreq> [output.json] --score
//       [--score-doc-limit N]
//   gdn_eval_amd <weights.gdnw> [output.json] --prefill <prompt.txt|ll.gdnreq>
//       [--example N] --dump-state <out.gdnstate> [--round-bf16] [--prefill-chunked]
//
// --prefill is the GPU prompt pass that produces a .gdnstate
// (export_gdn_state.py:157-201, :290-366): the prompt (a whitespace token
// file, or the context of example N of an LL fixture) runs through the
// multi-stream engine's prefill; the state, conv tails, prompt and the argmax
// of the last position (the seed token) are written as a .gdnstate.  The
// state is the BF16W_FP32S arm's (FP32); --round-bf16 rounds it and the
// tails to BF16 (RNE) once at the end, so the REF contract can load it.
// --prefill-chunked runs the recurrence in the chunk-parallel (WY) form
// (equal to the steps within FP32 re-association) instead of token order.
//
// Common options: --contract ref|bf16w|fp32 (default ref, the reference's
// all-BF16 arithmetic), --synth[=LAYERS] in place of a weights file (the
// library's seeded random-init model, for runs without a checkpoint).
//
// Differences from the reference drivers:
//  - per_step_tpot_ms is the token-in -> token-out time of the step (H2D,
//    graph, D2H); the independent host checks after it are not included;
//  - --dump-state writes the post-decode state in the reference's GDNSDMP1
//    layout (gdn_eval.cpp:464-491: magic, {stripe beats, ports, head-buffer
//    beats, 0}, the four BF16 state stripes, the packed conv tails) from the
//    host mirrors gdn_sync_host_state refreshes; --save-gdnstate writes the
//    same state as a .gdnstate another decode can start from (no reference
//    counterpart; in --prefill mode --dump-state names the .gdnstate);
//  - --interstep-delay-ms N sleeps N ms after each step, outside the step's
//    tpot (host.cpp:1772-1775);
//  - --ftz (gdn_eval.cpp:536-547) is refused: it sets FTZ/DAZ on the CPU
//    FPU under the reference's native model; this engine computes on the
//    GPU, where the contract alone fixes what flushes (the BF16 products'
//    DAZ/FTZ) and the FP32 arithmetic keeps IEEE subnormals;
//  - --logits-reference also reports the GPU-logit vector gate
//    (host.cpp:77-110) beside the exact-match count.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <string>
#include <thread>
#include <vector>

#include "gdn_amd.h"

namespace {

[[noreturn]] void die(const std::string &msg) {
    std::fprintf(stderr, "gdn_eval_amd: %s\n", msg.c_str());
    std::exit(2);
}

double now_ms() {
    using clk = std::chrono::steady_clock;
    return std::chrono::duration<double, std::milli>(clk::now().time_since_epoch()).count();
}

struct Options {
    std::string weights, fixture, output, state, logits_dump, logits_ref, hidden_dump, dump_state,
        save_gdnstate, bench_tokens, prefill;
    uint32_t interstep_delay_ms = 0;
    uint32_t decode_len = 0, bench_steps = 0, bench_warmup = 64, score_limit = 0, synth_layers = 0;
    // the timed benchmark protocol, with the reference's defaults (host.cpp:208-211)
    uint32_t bench_idle_s = 60, bench_warmup_s = 30, bench_interval_s = 60, bench_intervals = 3;
    uint32_t example = 0;
    bool synth = false, host_check = true, score = false, round_bf16 = false, prefill_chunked = false;
    int contract = GDN_CONTRACT_REF;
};

uint32_t parse_u32(const char *s, const char *what) {
    char *end = nullptr;
    const unsigned long v = std::strtoul(s, &end, 10);
    if (end == s || *end != '\0' || v > 0xffffffffUL) die(std::string("bad value for ") + what + ": " + s);
    return (uint32_t)v;
}

Options parse(int argc, char **argv) {
    Options o;
    std::vector<std::string> pos;
    for (int i = 1; i < argc; ++i) {
        const std::string a = argv[i];
        auto next = [&](const char *what) -> const char * {
            if (i + 1 >= argc) die(std::string(what) + " requires a value");
            return argv[++i];
        };
        if (a == "--decode") {
        } else if (a == "--decode-from-state") o.state = next("--decode-from-state");
        else if (a == "--decode-len") o.decode_len = parse_u32(next("--decode-len"), "--decode-len");
        else if (a == "--logits-dump") o.logits_dump = next("--logits-dump");
        else if (a == "--logits-reference") o.logits_ref = next("--logits-reference");
        else if (a == "--hidden-dump") o.hidden_dump = next("--hidden-dump");
        else if (a == "--dump-state") o.dump_state = next("--dump-state");
        else if (a == "--save-gdnstate") o.save_gdnstate = next("--save-gdnstate");
        else if (a == "--interstep-delay-ms")
            o.interstep_delay_ms = parse_u32(next("--interstep-delay-ms"), "--interstep-delay-ms");
        else if (a == "--ftz")
            die("--ftz is not supported: the reference's flag sets FTZ/DAZ on the CPU FPU that runs its native "
                "model; this engine computes on the GPU, where the contract alone fixes what flushes (the BF16 "
                "products) and FP32 arithmetic keeps IEEE subnormals");
        else if (a == "--no-host-check") o.host_check = false;
        else if (a == "--benchmark-tokens") o.bench_tokens = next("--benchmark-tokens");
        else if (a == "--benchmark-steps") o.bench_steps = parse_u32(next("--benchmark-steps"), "--benchmark-steps");
        else if (a == "--benchmark-warmup") o.bench_warmup = parse_u32(next("--benchmark-warmup"), "--benchmark-warmup");
        else if (a == "--benchmark-idle-seconds")
            o.bench_idle_s = parse_u32(next("--benchmark-idle-seconds"), "--benchmark-idle-seconds");
        else if (a == "--benchmark-warmup-seconds")
            o.bench_warmup_s = parse_u32(next("--benchmark-warmup-seconds"), "--benchmark-warmup-seconds");
        else if (a == "--benchmark-interval-seconds")
            o.bench_interval_s = parse_u32(next("--benchmark-interval-seconds"), "--benchmark-interval-seconds");
        else if (a == "--benchmark-intervals")
            o.bench_intervals = parse_u32(next("--benchmark-intervals"), "--benchmark-intervals");
        else if (a == "--score") o.score = true;
        else if (a == "--prefill") o.prefill = next("--prefill");
        else if (a == "--prefill-chunked") o.prefill_chunked = true;
        else if (a == "--example") o.example = parse_u32(next("--example"), "--example");
        else if (a == "--round-bf16") o.round_bf16 = true;
        else if (a == "--score-doc-limit") o.score_limit = parse_u32(next("--score-doc-limit"), "--score-doc-limit");
        else if (a == "--contract") {
            const std::string c = next("--contract");
            if (c == "ref") o.contract = GDN_CONTRACT_REF;
            else if (c == "bf16w") o.contract = GDN_CONTRACT_BF16W_FP32S;
            else if (c == "fp32") o.contract = GDN_CONTRACT_FP32;
            else die("--contract must be ref, bf16w or fp32");
        } else if (a == "--synth" || a.rfind("--synth=", 0) == 0) {
            o.synth = true;
            o.synth_layers = a.size() > 8 ? parse_u32(a.c_str() + 8, "--synth") : 24;
        } else if (a == "--help" || a == "-h") {
            std::printf(
                "usage:\n"
                "  gdn_eval_amd <weights.gdnw|--synth[=L]> [fixture.gdnreq] [out.json] "
                "--decode-from-state S [--decode-len N] [--logits-dump F] [--logits-reference F] "
                "[--hidden-dump F] [--dump-state F] [--save-gdnstate F] [--interstep-delay-ms N] [--no-host-check]\n"
                "  gdn_eval_amd <weights|--synth[=L]> [out.json] --decode-from-state S --benchmark-tokens T "
                "[--benchmark-idle-seconds N] [--benchmark-warmup-seconds N] [--benchmark-interval-seconds N] "
                "[--benchmark-intervals N]   (or a fixed count: [--benchmark-steps N] [--benchmark-warmup N])\n"
                "  gdn_eval_amd <weights|--synth[=L]> <rolling.gdnreq> [out.json] --score [--score-doc-limit N]\n"
                "  gdn_eval_amd <weights|--synth[=L]> [out.json] --prefill <prompt.txt|ll.gdnreq> [--example N] "
                "--dump-state S [--round-bf16] [--prefill-chunked]\n"
                "  common: --contract ref|bf16w|fp32\n");
            std::exit(0);
        } else if (!a.empty() && a[0] == '-') {
            die("unknown option " + a);
        } else {
            pos.push_back(a);
        }
    }
    // positionals: [weights] [fixture] [output] (gdn_eval.cpp:556-640); with
    // --synth the weights slot is absent, and a lone trailing positional is
    // the output when it ends in .json, else the fixture
    size_t k = 0;
    if (!o.synth) {
        if (pos.empty()) die("a weights file (or --synth) is required; see --help");
        o.weights = pos[k++];
    }
    const size_t rest = pos.size() - k;
    if (rest > 2) die("unexpected argument " + pos[k + 2]);
    if (rest == 2) {
        o.fixture = pos[k];
        o.output = pos[k + 1];
    } else if (rest == 1) {
        const std::string &p = pos[k];
        if (p.size() > 5 && p.compare(p.size() - 5, 5, ".json") == 0) o.output = p;
        else o.fixture = p;
    }
    if (o.score && o.fixture.empty()) die("--score requires a rolling fixture (GDNREQ1, kind 3)");
    if (!o.prefill.empty() && o.dump_state.empty()) die("--prefill requires --dump-state <out.gdnstate>");
    if (!o.score && o.state.empty() && o.prefill.empty())
        die("a mode is required: --decode-from-state S, --score or --prefill P; see --help");
    if (!o.bench_tokens.empty() && o.state.empty()) die("--benchmark-tokens requires --decode-from-state");
    if (!o.bench_tokens.empty() && (!o.dump_state.empty() || !o.save_gdnstate.empty() || o.interstep_delay_ms))
        die("--dump-state, --save-gdnstate and --interstep-delay-ms apply to the decode run, not --benchmark-tokens");
    if (!o.prefill.empty() && (!o.save_gdnstate.empty() || o.interstep_delay_ms))
        die("--save-gdnstate and --interstep-delay-ms apply to the decode run, not --prefill");
    if (!o.bench_tokens.empty() && !o.bench_steps && (o.bench_interval_s == 0 || o.bench_intervals == 0))
        die("--benchmark-interval-seconds and --benchmark-intervals must be positive");
    return o;
}

// GDNREQ1 fixtures (export_gdn_c.py layout): magic, version 1, kind, count.
// Kind 2 (LL, gdn_eval.cpp:77-151): per example ctx_len, cont_len,
// ctx[ctx_len], cont[cont_len].  Kind 3 (rolling, host.cpp:516-550): per
// document word_count, byte_count, n_windows, then n_windows such pairs.
struct Window {
    std::vector<int32_t> ctx, cont;
};
struct Document {
    uint32_t word_count = 0, byte_count = 0;
    std::vector<Window> windows;
};
struct Fixture {
    uint32_t kind = 0;
    std::vector<Document> docs;  // kind 2: one single-window document per example
};

Fixture load_fixture(const std::string &path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) die("cannot open fixture " + path);
    std::vector<char> blob((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
    size_t off = 0;
    auto u32 = [&](const char *what) {
        if (off + 4 > blob.size()) die(std::string("truncated fixture (") + what + ")");
        uint32_t v;
        std::memcpy(&v, blob.data() + off, 4);
        off += 4;
        return v;
    };
    auto window = [&]() {
        Window w;
        const uint32_t cl = u32("ctx_len"), nl = u32("cont_len");
        if ((uint64_t)cl + nl > (blob.size() - off) / 4) die("truncated fixture (tokens)");
        w.ctx.resize(cl);
        w.cont.resize(nl);
        for (auto &t : w.ctx) t = (int32_t)u32("ctx");
        for (auto &t : w.cont) t = (int32_t)u32("cont");
        return w;
    };
    if (blob.size() < 20 || std::memcmp(blob.data(), "GDNREQ1", 7) != 0) die("not a GDNREQ1 fixture: " + path);
    off = 8;
    if (u32("version") != 1) die("unsupported fixture version");
    Fixture fx;
    fx.kind = u32("kind");
    if (fx.kind != 2 && fx.kind != 3) die("fixture kind must be 2 (LL) or 3 (rolling)");
    const uint32_t n = u32("count");
    for (uint32_t e = 0; e < n; ++e) {
        Document d;
        if (fx.kind == 2) {
            d.windows.push_back(window());
        } else {
            d.word_count = u32("word_count");
            d.byte_count = u32("byte_count");
            const uint32_t nw = u32("n_windows");
            for (uint32_t w = 0; w < nw; ++w) d.windows.push_back(window());
        }
        fx.docs.push_back(std::move(d));
    }
    if (off != blob.size()) die("trailing data in fixture " + path);
    return fx;
}

// GDNLOG1 / GDNHID1 dumps: 8-byte magic, u32 version 1, u32 width, u32
// steps, then steps x width FP32 (export_gdn_state.py:238-251).
struct DumpHeader {
    char magic[8];
    uint32_t version, width, steps;
};
static_assert(sizeof(DumpHeader) == 20, "packed dump header");

FILE *open_dump(const std::string &path, const char *magic, uint32_t width, uint32_t steps) {
    FILE *f = std::fopen(path.c_str(), "wb");
    if (!f) die("cannot create " + path);
    DumpHeader h{};
    std::memcpy(h.magic, magic, 8);
    h.version = 1;
    h.width = width;
    h.steps = steps;
    if (std::fwrite(&h, sizeof(h), 1, f) != 1) die("cannot write " + path);
    return f;
}

struct Summary {
    double mean = 0, median = 0, p95 = 0, min = 0, max = 0;
};
Summary summarize(std::vector<double> v) {
    Summary s;
    if (v.empty()) return s;
    std::sort(v.begin(), v.end());
    double sum = 0;
    for (double x : v) sum += x;
    s.mean = sum / v.size();
    s.median = v.size() % 2 ? v[v.size() / 2] : 0.5 * (v[v.size() / 2 - 1] + v[v.size() / 2]);
    s.p95 = v[std::min(v.size() - 1, (size_t)std::ceil(0.95 * v.size()) - 1)];
    s.min = v.front();
    s.max = v.back();
    return s;
}
void write_summary(FILE *o, const Summary &s) {
    std::fprintf(o, "{\"mean_ms\": %.6f, \"median_ms\": %.6f, \"p95_ms\": %.6f, \"min_ms\": %.6f, \"max_ms\": %.6f}",
                 s.mean, s.median, s.p95, s.min, s.max);
}

FILE *open_output(const std::string &path) {
    if (path.empty()) return stdout;
    FILE *f = std::fopen(path.c_str(), "w");
    if (!f) die("cannot create " + path);
    return f;
}

const char *contract_name(int c) {
    return c == GDN_CONTRACT_REF ? "ref" : c == GDN_CONTRACT_BF16W_FP32S ? "bf16w_fp32s" : "fp32";
}

// ------------------------------------------------------------- decode mode

// The post-decode state in the reference's GDNSDMP1 layout
// (gdn_eval.cpp:464-491): 8-byte magic, u32 {stripe beats, ports, head-buffer
// beats, 0}, the BF16 state stripe of each port (the run state's host mirror
// at weight_shards[28 + p] + gdn_weight_shard_beats), then the head buffer
// (the packed conv tails).
void write_state_dump(GDNRunState &rs, const GDNModel &model, const std::string &path) {
    if (gdn_sync_host_state(&rs) != 0) die("cannot read the state back from the device");
    FILE *f = std::fopen(path.c_str(), "wb");
    if (!f) die("cannot create state dump " + path);
    const uint32_t hb_beats = GDN_WSF_HEADBUF / 16u;
    const uint32_t hdr[4] = {GDN_RECURRENT_STATE_STRIPE_BF16_BEATS, GDN_RECURRENT_STATE_PORTS, hb_beats, 0};
    bool ok = std::fwrite("GDNSDMP1", 1, 8, f) == 8 && std::fwrite(hdr, 4, 4, f) == 4;
    const size_t shard_beats = gdn_weight_shard_beats(&model.config);
    for (int p = 0; ok && p < GDN_RECURRENT_STATE_PORTS; ++p)
        ok = std::fwrite(rs.weight_shards[GDN_RECURRENT_STATE_FIRST_PORT + p] + shard_beats, sizeof(Beat512),
                         GDN_RECURRENT_STATE_STRIPE_BF16_BEATS, f) == GDN_RECURRENT_STATE_STRIPE_BF16_BEATS;
    ok = ok && std::fwrite(rs.head_buffer, sizeof(Beat512), hb_beats, f) == hb_beats;
    if (std::fclose(f) != 0 || !ok) die("state dump write failed: " + path);
    std::fprintf(stderr, "[state_dump] wrote %s\n", path.c_str());
}

int run_decode(const Options &o, const Fixture *fx, const GDNModel &model, GDNRunState &rs) {
    const uint32_t V = model.config.vocab_size, H = model.config.hidden_size;
    uint32_t prompt_len = 0;
    int32_t seed = 0;
    if (gdn_load_gdnstate(&rs, &model, o.state.c_str(), &prompt_len, &seed) != 0) die("cannot load " + o.state);
    // decode length: --decode-len, else the first golden continuation of an
    // LL fixture (gdn_eval.cpp:666-677), else 64 (gdn_eval.cpp:278)
    uint32_t n = o.decode_len;
    if (n == 0 && fx) {
        if (fx->kind != 2 || fx->docs.empty()) die("decode-from-state requires an LL fixture with at least 1 example");
        n = (uint32_t)fx->docs[0].windows[0].cont.size();
        if (n == 0) die("decode-from-state: zero decode length");
    }
    if (n == 0) n = 64;
    std::fprintf(stderr, "[progress] decode-from-state N=%u seed=%d prompt_len=%u contract=%s\n", n, seed,
                 prompt_len, contract_name(o.contract));

    std::vector<int32_t> traj(n, 0);
    std::vector<double> tpot(n, 0.0);
    std::vector<float> logits(V), host_logits(V), ref_logits(V), hidden(H);
    traj[0] = seed;
    FILE *ldump = o.logits_dump.empty() ? nullptr : open_dump(o.logits_dump, "GDNLOG1\0", V, n - 1);
    FILE *hdump = o.hidden_dump.empty() ? nullptr : open_dump(o.hidden_dump, "GDNHID1\0", H, n - 1);
    FILE *lref = nullptr;
    if (!o.logits_ref.empty()) {
        lref = std::fopen(o.logits_ref.c_str(), "rb");
        DumpHeader h{};
        if (!lref || std::fread(&h, sizeof(h), 1, lref) != 1 || std::memcmp(h.magic, "GDNLOG1", 7) != 0 ||
            h.version != 1 || h.width != V || h.steps < n - 1)
            die("incompatible logits reference " + o.logits_ref);
    }
    // host check: the engine's logits against the independent scalar LM head
    double max_abs = 0, max_rel = 0;
    uint64_t tol_fail = 0, compared = 0, exact_ref_mismatch = 0;
    uint32_t checked = 0, argmax_mismatch = 0;
    GDNLogitsParity gate;
    gdn_logits_parity_init(&gate);

    for (uint32_t step = 1; step < n; ++step) {
        const double t0 = now_ms();
        if (gdn_decode_step_host(&model, &rs, &traj[step - 1]) != 0) die("decode step failed");
        int32_t tok = 0;
        if (gdn_read_token(&rs, &tok) != 0) die("cannot read the token");
        tpot[step] = now_ms() - t0;
        traj[step] = tok;
        if (gdn_read_logits(&rs, logits.data(), V) != 0) die("cannot read logits");
        if (gdn_strict_argmax(logits.data(), V) != (uint32_t)tok) {
            std::fprintf(stderr, "on-device argmax %d != host scan %u at step %u\n", tok,
                         gdn_strict_argmax(logits.data(), V), step);
            die("the on-device argmax disagrees with the host scan of its logits");
        }
        if (o.host_check || hdump) {
            if (gdn_read_final_hidden(&rs, hidden.data(), H) != 0) die("cannot read the final hidden vector");
        }
        if (hdump && std::fwrite(hidden.data(), 4, H, hdump) != H) die("hidden dump write failed");
        if (o.host_check) {
            gdn_compute_logits(&model, hidden.data(), host_logits.data());
            for (uint32_t v = 0; v < V; ++v) {
                const float a = logits[v], r = host_logits[v];
                const double ad = std::fabs((double)a - (double)r);
                max_abs = std::max(max_abs, ad);
                max_rel = std::max(max_rel, ad / std::max(1.0, std::fabs((double)r)));
                if (std::memcmp(&a, &r, 4) != 0 &&
                    (!std::isfinite(a) || !std::isfinite(r) || ad > 1e-3 + 1e-4 * std::fabs((double)r)))
                    ++tol_fail;
            }
            if (gdn_strict_argmax(host_logits.data(), V) != (uint32_t)tok) ++argmax_mismatch;
            ++checked;
            compared += V;
        }
        if (lref) {
            if (std::fread(ref_logits.data(), 4, V, lref) != V) die("truncated logits reference");
            for (uint32_t v = 0; v < V; ++v)
                if (std::memcmp(&ref_logits[v], &logits[v], 4) != 0) ++exact_ref_mismatch;
            gdn_logits_parity_step(&gate, logits.data(), ref_logits.data(), V, (uint32_t)tok, 0);
        }
        if (ldump && std::fwrite(logits.data(), 4, V, ldump) != V) die("logits dump write failed");
        if (o.interstep_delay_ms) std::this_thread::sleep_for(std::chrono::milliseconds(o.interstep_delay_ms));
    }
    if (ldump) std::fclose(ldump);
    if (hdump) std::fclose(hdump);
    if (lref) std::fclose(lref);
    if (!o.save_gdnstate.empty() &&
        gdn_save_gdnstate(&rs, &model, o.save_gdnstate.c_str(), nullptr, 0, traj[n - 1]) != 0)
        die("cannot write " + o.save_gdnstate);
    if (!o.dump_state.empty()) write_state_dump(rs, model, o.dump_state);
    std::fprintf(stderr,
                 "[logits] steps=%u values=%llu max_abs=%.9g max_rel=%.9g cpu_tol_fail=%llu "
                 "exact_ref_mismatch=%llu argmax_mismatch=%u\n",
                 checked, (unsigned long long)compared, max_abs, max_rel, (unsigned long long)tol_fail,
                 (unsigned long long)exact_ref_mismatch, argmax_mismatch);

    FILE *out = open_output(o.output);
    std::fprintf(out, "{\"kind\": 2, \"decode_len\": %u, \"num_examples\": 1,\n \"examples\": [\n  {\"index\": 0,\n", n);
    const char *keys[2] = {"gen_traj", "tf_argmax"};
    for (const char *key : keys) {
        std::fprintf(out, "   \"%s\": [", key);
        for (uint32_t j = 0; j < n; ++j) std::fprintf(out, "%s%d", j ? ", " : "", traj[j]);
        std::fprintf(out, "],\n");
    }
    std::fprintf(out, "   \"per_step_tpot_ms\": [");
    for (uint32_t j = 0; j < n; ++j) std::fprintf(out, "%s%.6f", j ? ", " : "", tpot[j]);
    std::fprintf(out, "]}\n ],\n");
    std::fprintf(out,
                 " \"logits_parity\": {\"checked_steps\": %u, \"compared_values\": %llu, \"max_abs_error\": %.17g, "
                 "\"max_rel_error\": %.17g, \"cpu_tolerance_failures\": %llu, \"exact_reference_mismatches\": %llu, "
                 "\"argmax_mismatches\": %u}",
                 checked, (unsigned long long)compared, max_abs, max_rel, (unsigned long long)tol_fail,
                 (unsigned long long)exact_ref_mismatch, argmax_mismatch);
    if (!o.logits_ref.empty()) {
        std::fprintf(out,
                     ",\n \"vector_gate\": {\"checked_steps\": %u, \"global_nrmse\": %.9g, \"global_cosine\": %.12g, "
                     "\"worst_step_nrmse\": %.9g, \"min_step_cosine\": %.12g, \"worst_max_abs_over_reference_rms\": "
                     "%.9g, \"max_abs_error\": %.9g, \"min_top5_overlap\": %u, \"argmax_mismatches\": %u, "
                     "\"nonfinite_mismatches\": %llu, \"passes\": %s}",
                     gate.checked_steps, gdn_logits_parity_nrmse(&gate), gdn_logits_parity_cosine(&gate),
                     gate.worst_step_nrmse, gate.min_step_cosine, gate.worst_max_abs_over_reference_rms,
                     gate.max_abs_error, gate.min_top5_overlap, gate.argmax_mismatches,
                     (unsigned long long)gate.nonfinite_mismatches, gdn_logits_gate_passes(&gate) ? "true" : "false");
    }
    std::fprintf(out, ",\n \"engine\": {\"library\": \"libgdn_amd\", \"contract\": \"%s\"}}\n", contract_name(o.contract));
    if (out != stdout) std::fclose(out);
    return (tol_fail == 0 && exact_ref_mismatch == 0 && argmax_mismatch == 0) ? 0 : 1;
}

// ---------------------------------------------------------- benchmark mode

// Whitespace-separated token ids in [0, vocab) (host.cpp:2116-2139).
std::vector<int32_t> load_token_file(const std::string &path, uint32_t V, const char *what) {
    std::ifstream f(path);
    if (!f) die(std::string("cannot open ") + what + " token file " + path);
    std::vector<int32_t> tokens;
    long long v;
    while (f >> v) {
        if (v < 0 || (unsigned long long)v >= V) die(std::string(what) + " token out of vocabulary range");
        tokens.push_back((int32_t)v);
    }
    if (!f.eof()) die(std::string(what) + " token file must hold whitespace-separated integers");
    if (tokens.empty()) die(std::string(what) + " token stream is empty");
    return tokens;
}

double unix_now() {
    return std::chrono::duration<double>(std::chrono::system_clock::now().time_since_epoch()).count();
}

void write_bench_header(FILE *out, const Options &o, size_t stream_len) {
    std::fprintf(out,
                 "{\n  \"schema\": \"gdn-steady-tpot-v1\",\n  \"weights\": \"%s\",\n  \"state\": \"%s\",\n"
                 "  \"token_file\": \"%s\",\n  \"token_stream_length\": %zu,\n  \"teacher_forced\": true,\n"
                 "  \"full_lm_head\": true,\n  \"onchip_argmax\": true,\n  \"full_logits_readback\": false,\n"
                 "  \"contract\": \"%s\",\n",
                 o.synth ? "synthetic" : o.weights.c_str(), o.state.c_str(), o.bench_tokens.c_str(), stream_len,
                 contract_name(o.contract));
}

// One measured interval: its wall-clock bounds (reported), its duration on
// the monotonic clock (the rate; a wall-clock step cannot skew it) and every
// step's token-in -> token-out time (production_tpot) and graph time between
// HIP events (kernel).
struct Interval {
    double start_unix = 0, end_unix = 0;
    std::chrono::steady_clock::time_point t0, t1;
    std::vector<double> outer, inner;
    void begin() {
        start_unix = unix_now();
        t0 = std::chrono::steady_clock::now();
    }
    void end() {
        t1 = std::chrono::steady_clock::now();
        end_unix = unix_now();
    }
    double seconds() const { return std::chrono::duration<double>(t1 - t0).count(); }
};

void write_interval(FILE *out, size_t index, const Interval &iv, bool first) {
    std::fprintf(out, "%s\n    {\"index\": %zu, \"start_unix\": %.6f, \"end_unix\": %.6f, \"steps\": %zu, "
                 "\"tokens_per_second\": %.3f, \"production_tpot\": ",
                 first ? "" : ",", index, iv.start_unix, iv.end_unix, iv.outer.size(),
                 (double)iv.outer.size() / iv.seconds());
    write_summary(out, summarize(iv.outer));
    std::fprintf(out, ", \"kernel\": ");
    write_summary(out, summarize(iv.inner));
    std::fprintf(out, "}");
}

// The steady teacher-forced benchmark (host.cpp:2150-2256): a loaded-idle
// window, a timed warmup, then timed intervals over the cyclic token
// stream, each summarised.  With --benchmark-steps: a fixed warmup count and
// one interval of a fixed step count instead.  The reference's embedding
// write / H2D / launch / token D2H phases have no counterpart: the embedding
// import runs on the device and the token crosses through mapped memory.
int run_benchmark(const Options &o, const GDNModel &model, GDNRunState &rs) {
    const std::vector<int32_t> tokens = load_token_file(o.bench_tokens, model.config.vocab_size, "benchmark");
    uint32_t prompt_len = 0;
    int32_t seed = 0;
    if (gdn_load_gdnstate(&rs, &model, o.state.c_str(), &prompt_len, &seed) != 0) die("cannot load " + o.state);
    if (o.bench_steps) {
        const uint32_t steps = o.bench_steps;
        if (o.bench_warmup && gdn_run_teacher_forced(&rs, tokens.data(), (uint32_t)tokens.size(), o.bench_warmup,
                                                     nullptr, nullptr, nullptr) != 0)
            die("benchmark warmup failed");
        std::vector<float> inner(steps), outer(steps);
        Interval iv;
        iv.begin();
        if (gdn_run_teacher_forced(&rs, tokens.data(), (uint32_t)tokens.size(), steps, nullptr, inner.data(),
                                   outer.data()) != 0)
            die("benchmark failed");
        iv.end();
        iv.outer.assign(outer.begin(), outer.end());
        iv.inner.assign(inner.begin(), inner.end());
        FILE *out = open_output(o.output);
        write_bench_header(out, o, tokens.size());
        std::fprintf(out, "  \"warmup_steps\": %u,\n  \"intervals\": [", o.bench_warmup);
        write_interval(out, 0, iv, true);
        std::fprintf(out, "\n  ]\n}\n");
        if (out != stdout) std::fclose(out);
        return 0;
    }
    size_t next = 0;
    auto one = [&](float *inner, float *outer) {
        const int32_t tok = tokens[next];
        next = (next + 1) % tokens.size();
        if (gdn_run_teacher_forced(&rs, &tok, 1, 1, nullptr, inner, outer) != 0) die("benchmark step failed");
    };
    using clock = std::chrono::steady_clock;
    const double idle_start = unix_now();
    std::fprintf(stderr, "[benchmark] loaded-idle window %us\n", o.bench_idle_s);
    std::this_thread::sleep_for(std::chrono::seconds(o.bench_idle_s));
    const double warmup_start = unix_now();
    uint64_t warmup_steps = 0;
    for (const auto end = clock::now() + std::chrono::seconds(o.bench_warmup_s); clock::now() < end; ++warmup_steps)
        one(nullptr, nullptr);
    const double warmup_end = unix_now();
    std::fprintf(stderr, "[benchmark] warmup complete steps=%llu\n", (unsigned long long)warmup_steps);
    std::vector<Interval> intervals(o.bench_intervals);
    for (uint32_t i = 0; i < o.bench_intervals; ++i) {
        Interval &iv = intervals[i];
        iv.begin();
        for (const auto end = clock::now() + std::chrono::seconds(o.bench_interval_s); clock::now() < end;) {
            float inner = 0.0f, outer = 0.0f;
            one(&inner, &outer);
            iv.inner.push_back(inner);
            iv.outer.push_back(outer);
        }
        iv.end();
        std::fprintf(stderr, "[benchmark] interval %u/%u steps=%zu\n", i + 1, o.bench_intervals, iv.outer.size());
    }
    FILE *out = open_output(o.output);
    write_bench_header(out, o, tokens.size());
    std::fprintf(out,
                 "  \"idle_start_unix\": %.6f,\n  \"warmup_start_unix\": %.6f,\n  \"warmup_end_unix\": %.6f,\n"
                 "  \"warmup_steps\": %llu,\n  \"intervals\": [",
                 idle_start, warmup_start, warmup_end, (unsigned long long)warmup_steps);
    for (size_t i = 0; i < intervals.size(); ++i) write_interval(out, i, intervals[i], i == 0);
    std::fprintf(out, "\n  ]\n}\n");
    if (out != stdout) std::fclose(out);
    return 0;
}

// ------------------------------------------------------------ scoring mode

// Rolling teacher-forced scoring (host.cpp:1943-2070): every window starts
// from a blank recurrent and conv state; position i feeds tokens[i] and, from
// the last context token on, adds log softmax(logits)[tokens[i+1]].
int run_score(const Options &o, const Fixture &fx, const GDNModel &model, GDNRunState &rs) {
    const GDNWeightHeader &c = model.config;
    const uint32_t V = c.vocab_size;
    const size_t rec = (size_t)c.num_layers * c.num_heads * c.head_dim * c.head_dim;
    const size_t conv = (size_t)c.num_layers * 3 * (c.conv_size - 1) * c.hidden_size;
    const std::vector<float> zero_rec(rec, 0.0f), zero_conv(conv, 0.0f);
    std::vector<float> logits(V);
    size_t docs = fx.docs.size();
    if (o.score_limit && o.score_limit < docs) docs = o.score_limit;
    std::fprintf(stderr, "[progress] scoring %zu of %zu documents\n", docs, fx.docs.size());
    double total = 0.0, kernel_ms = 0.0;
    uint64_t scored = 0, windows = 0, words = 0, bytes = 0, steps = 0;
    const double t_start = now_ms();
    for (size_t d = 0; d < docs; ++d) {
        const Document &doc = fx.docs[d];
        for (const Window &w : doc.windows) {
            if (w.ctx.empty() || w.cont.empty()) die("invalid scoring window");
            if (gdn_load_recurrent_state(&rs, zero_rec.data(), rec) != 0 ||
                gdn_load_conv_tails(&rs, zero_conv.data(), conv) != 0)
                die("cannot reset the state");
            std::vector<int32_t> toks(w.ctx);
            toks.insert(toks.end(), w.cont.begin(), w.cont.end());
            for (size_t i = 0; i + 1 < toks.size(); ++i) {
                const double t0 = now_ms();
                if (gdn_decode_step_host(&model, &rs, &toks[i]) != 0) die("scoring step failed (token out of range?)");
                int32_t tok = 0;
                if (gdn_read_token(&rs, &tok) != 0) die("cannot read the token");
                kernel_ms += now_ms() - t0;
                ++steps;
                if (i + 1 < w.ctx.size()) continue;  // still inside the context
                if (gdn_read_logits(&rs, logits.data(), V) != 0) die("cannot read logits");
                const double l = gdn_token_logprob(logits.data(), V, toks[i + 1]);
                if (std::isnan(l) && (toks[i + 1] < 0 || (uint32_t)toks[i + 1] >= V))
                    die("scoring target token out of range");
                total += l;
                ++scored;
            }
            ++windows;
        }
        words += doc.word_count;
        bytes += doc.byte_count;
        std::fprintf(stderr, "[progress] doc %zu/%zu windows=%zu scored_tokens=%llu elapsed=%.0fs\n", d + 1, docs,
                     doc.windows.size(), (unsigned long long)scored, (now_ms() - t_start) / 1000.0);
    }
    const double word_ppl = std::exp(-total / (double)words);
    const double byte_ppl = std::exp(-total / (double)bytes);
    const double bpb = -total / (double)bytes / std::log(2.0);
    const double avg_ms = steps ? kernel_ms / steps : 0.0;
    std::fprintf(stderr,
                 "[score] documents=%zu windows=%llu scored_tokens=%llu words=%llu bytes=%llu total_logprob=%.17g "
                 "word_ppl=%.9g byte_ppl=%.9g bits_per_byte=%.9g step_ms=%.6f\n",
                 docs, (unsigned long long)windows, (unsigned long long)scored, (unsigned long long)words,
                 (unsigned long long)bytes, total, word_ppl, byte_ppl, bpb, avg_ms);
    FILE *out = open_output(o.output);
    std::fprintf(out,
                 "{\n  \"task\": \"wikitext_rolling\",\n  \"fixture\": \"%s\",\n  \"engine\": \"libgdn_amd\",\n"
                 "  \"contract\": \"%s\",\n  \"documents\": %zu,\n  \"windows\": %llu,\n  \"scored_tokens\": %llu,\n"
                 "  \"words\": %llu,\n  \"bytes\": %llu,\n  \"total_logprob\": %.17g,\n  \"word_perplexity\": %.17g,\n"
                 "  \"byte_perplexity\": %.17g,\n  \"bits_per_byte\": %.17g,\n  \"average_step_ms\": %.17g\n}\n",
                 o.fixture.c_str(), contract_name(o.contract), docs, (unsigned long long)windows,
                 (unsigned long long)scored, (unsigned long long)words, (unsigned long long)bytes, total, word_ppl,
                 byte_ppl, bpb, avg_ms);
    if (out != stdout) std::fclose(out);
    return 0;
}

// ----------------------------------------------------------- prefill mode

int run_prefill(const Options &o, const Fixture *fx, const GDNModel &model) {
    const GDNWeightHeader &c = model.config;
    std::vector<int32_t> prompt;
    if (fx) {
        if (fx->kind != 2 || o.example >= fx->docs.size()) die("--prefill needs an LL fixture example (kind 2)");
        prompt = fx->docs[o.example].windows[0].ctx;
        if (prompt.empty()) die("cannot export state for an empty prompt");
        for (int32_t t : prompt)
            if (t < 0 || (uint32_t)t >= c.vocab_size) die("prompt token out of vocabulary range");
    } else {
        prompt = load_token_file(o.prefill, c.vocab_size, "prompt");
    }
    GDNBatchState bs;
    std::memset(&bs, 0, sizeof(bs));
    if (gdn_batch_init(&bs, &model, 1) != 0) die("multi-stream engine init failed (BF16-exact weights needed)");
    std::fprintf(stderr, "[progress] prefill of %zu tokens\n", prompt.size());
    int32_t seed = 0;
    const double t0 = now_ms();
    if (o.prefill_chunked && gdn_batch_set_prefill_mode(&bs, GDN_PREFILL_CHUNKED) != 0) die("prefill mode");
    if (gdn_batch_prefill(&bs, 0, prompt.data(), (uint32_t)prompt.size(), &seed) != 0) die("prefill failed");
    const double ms = now_ms() - t0;
    const size_t rec = (size_t)c.num_layers * c.num_heads * c.head_dim * c.head_dim;
    const size_t conv = (size_t)c.num_layers * 3 * (c.conv_size - 1) * c.hidden_size;
    std::vector<float> r(rec), cv(conv);
    if (gdn_batch_save_stream_state(&bs, 0, r.data(), rec, cv.data(), conv) != 0) die("cannot read the state");
    gdn_batch_free(&bs);
    if (o.round_bf16) {
        for (auto *vec : {&r, &cv})
            for (float &x : *vec) {
                uint32_t b;
                std::memcpy(&b, &x, 4);
                b = (uint32_t)gdn_test_fp32_to_bf16_rne_bits(b) << 16;
                std::memcpy(&x, &b, 4);
            }
    }
    if (gdn_write_gdnstate(&c, o.dump_state.c_str(), r.data(), cv.data(), prompt.data(), (uint32_t)prompt.size(),
                           seed) != 0)
        die("cannot write " + o.dump_state);
    std::fprintf(stderr, "[prefill] prompt_len=%zu seed_token=%d %.1f ms (%.0f tokens/s) -> %s\n", prompt.size(), seed,
                 ms, 1000.0 * prompt.size() / ms, o.dump_state.c_str());
    FILE *out = open_output(o.output);
    std::fprintf(out,
                 "{\"mode\": \"prefill\", \"prompt_len\": %zu, \"seed_token\": %d, \"prefill_ms\": %.3f, "
                 "\"tokens_per_second\": %.1f, \"state\": \"%s\", \"state_rounding\": \"%s\", "
                 "\"engine\": \"libgdn_amd multi-stream prefill\"}\n",
                 prompt.size(), seed, ms, 1000.0 * prompt.size() / ms, o.dump_state.c_str(),
                 o.round_bf16 ? "bf16" : "fp32");
    if (out != stdout) std::fclose(out);
    return 0;
}

}  // namespace

int main(int argc, char **argv) {
    const Options o = parse(argc, argv);
    // the fixture is validated before any weights or device memory are touched
    Fixture fx;
    if (!o.fixture.empty()) fx = load_fixture(o.fixture);
    if (o.score && fx.kind != 3) die("--score requires a rolling fixture (kind 3)");
    GDNModel model;
    std::memset(&model, 0, sizeof(model));
    if (o.synth) {
        GDNWeightHeader cfg;
        gdn_default_config(&cfg, o.synth_layers);
        if (gdn_model_synth(&model, &cfg, 0, 0.02f, o.contract != GDN_CONTRACT_FP32) != 0) die("synthesis failed");
    } else {
        const int rc = (o.contract == GDN_CONTRACT_FP32) ? gdn_model_load_fp32(&model, o.weights.c_str())
                                                          : gdn_model_load(&model, o.weights.c_str());
        if (rc != 0) die("cannot load " + o.weights);
    }
    if (!o.prefill.empty()) {
        const bool is_fixture = o.prefill.size() > 7 && o.prefill.compare(o.prefill.size() - 7, 7, ".gdnreq") == 0;
        Fixture pf;
        if (is_fixture) pf = load_fixture(o.prefill);
        const int rc = run_prefill(o, is_fixture ? &pf : nullptr, model);
        gdn_model_free(&model);
        return rc;
    }
    GDNRunState rs;
    std::memset(&rs, 0, sizeof(rs));
    if (gdn_run_state_init_contract(&rs, &model, model.config.max_seq_len, o.contract) != 0) die("run state init failed");
    int rc;
    if (o.score) rc = run_score(o, fx, model, rs);
    else if (!o.bench_tokens.empty()) rc = run_benchmark(o, model, rs);
    else rc = run_decode(o, o.fixture.empty() ? nullptr : &fx, model, rs);
    gdn_run_state_free(&rs);
    gdn_model_free(&model);
    return rc;
}
