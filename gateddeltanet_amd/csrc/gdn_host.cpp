// gdn_host.cpp -- host-side half of libgdn_amd.so: the .gdnw / .gdnstate
// formats, weight views, the seeded synthetic generator, and the reference's
// host helpers (BF16 rounding hooks, native product, scalar LM head).
//
// Reference behaviour followed (YAMWD/GatedDeltaNet):
//   gdn_model.cpp:1082-1245   header validation, views, .gdnw load
//   gdn_model.cpp:309-325     BF16 RNE / widen
//   gdn_model.cpp:392-467     native BF16 product
//   gdn_model.cpp:3930-3965   gdn_compute_logits
//   gdn_eval.cpp:196-267      .gdnstate reader
//   export_gdn_state.py:340-362  .gdnstate writer
#include "gdn_amd.h"
#include "gdn_internal.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace {

uint32_t f2u(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
float u2f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

int validate_config(const GDNWeightHeader *c) {
    static_assert(sizeof(GDNWeightHeader) == 60, "GDNWeightHeader is 60 bytes");
    if (std::memcmp(c->magic, "GDNWv1", 6) != 0 || c->version != 1) {
        gdn_error("unsupported weight file");
        return -1;
    }
    if (c->num_heads != c->num_v_heads) {
        gdn_error("expected num_heads == num_v_heads");
        return -1;
    }
    if (c->hidden_size != c->num_heads * c->head_dim) {
        gdn_error("expected hidden_size == num_heads * head_dim");
        return -1;
    }
    return 0;
}

size_t layer_stride(const GDNWeightHeader *c) {
    const size_t H = c->hidden_size, nh = c->num_heads, hd = c->head_dim;
    const size_t I = c->intermediate_size, cs = c->conv_size;
    return H + 2 * nh + 3 * H * H + 2 * nh * H + 3 * H * cs + H * H + hd +
           H * H + H + 2 * I * H + H * I;
}

size_t layer_offset(const GDNWeightHeader *c, uint32_t layer) {
    return (size_t)c->vocab_size * c->hidden_size + (size_t)layer * layer_stride(c);
}

// View assignment in the .gdnw payload order (gdn_model.cpp:1102-1159).
void assign_views(GDNModel *m) {
    const GDNWeightHeader *c = &m->config;
    const size_t H = c->hidden_size, nh = c->num_heads, hd = c->head_dim;
    const size_t I = c->intermediate_size, cs = c->conv_size;
    const float *p = m->weight_data;
    m->embeddings = p;
    p += (size_t)c->vocab_size * H;
    for (uint32_t l = 0; l < c->num_layers; ++l) {
        GDNLayerWeights *w = &m->layers[l];
        w->attn_norm = p; p += H;
        w->a_log = p; p += nh;
        w->dt_bias = p; p += nh;
        w->q_proj = p; p += H * H;
        w->k_proj = p; p += H * H;
        w->v_proj = p; p += H * H;
        w->a_proj = p; p += nh * H;
        w->b_proj = p; p += nh * H;
        w->q_conv = p; p += H * cs;
        w->k_conv = p; p += H * cs;
        w->v_conv = p; p += H * cs;
        w->g_proj = p; p += H * H;
        w->o_norm = p; p += hd;
        w->o_proj = p; p += H * H;
        w->mlp_norm = p; p += H;
        w->mlp_gate_proj = p; p += I * H;
        w->mlp_up_proj = p; p += I * H;
        w->mlp_down_proj = p; p += H * I;
    }
    m->final_norm = p;
    p += H;
    m->lm_head = p;
}

int alloc_model(GDNModel *m, const GDNWeightHeader *c) {
    std::memset(m, 0, sizeof(*m));
    m->config = *c;
    const size_t total = gdn_total_weight_floats(c);
    m->weight_data = static_cast<float *>(std::malloc(total * sizeof(float)));
    m->layers = static_cast<GDNLayerWeights *>(
        std::calloc(c->num_layers ? c->num_layers : 1, sizeof(GDNLayerWeights)));
    if (!m->weight_data || !m->layers) {
        gdn_error("model allocation failed");
        gdn_model_free(m);
        return -1;
    }
    assign_views(m);
    return 0;
}

int load_impl(GDNModel *m, const char *path, bool require_bf16) {
    std::memset(m, 0, sizeof(*m));
    FILE *f = std::fopen(path, "rb");
    if (!f) {
        std::perror("fopen weights");
        return -1;
    }
    GDNWeightHeader hdr;
    if (std::fread(&hdr, 1, sizeof(hdr), f) != sizeof(hdr)) {
        gdn_error("failed to read weight header");
        std::fclose(f);
        return -1;
    }
    if (validate_config(&hdr) != 0 || alloc_model(m, &hdr) != 0) {
        std::fclose(f);
        return -1;
    }
    // Validate while reading, chunk by chunk (gdn_model.cpp:1192-1224).
    const size_t total = gdn_total_weight_floats(&hdr);
    const size_t chunk = (size_t)4 << 20;
    for (size_t done = 0; done < total;) {
        const size_t n = total - done < chunk ? total - done : chunk;
        if (std::fread(m->weight_data + done, sizeof(float), n, f) != n) {
            gdn_error("failed to read weight payload");
            std::fclose(f);
            gdn_model_free(m);
            return -1;
        }
        if (require_bf16) {
            for (size_t i = 0; i < n; ++i) {
                const uint32_t b = f2u(m->weight_data[done + i]);
                if ((b & 0xffffu) != 0) {
                    std::fprintf(stderr, "gdn: weight %zu is not BF16-exact (bits=0x%08x)\n",
                                 done + i, b);
                    gdn_error("dense packing requires a BF16-exact FP32-word checkpoint");
                    std::fclose(f);
                    gdn_model_free(m);
                    return -1;
                }
            }
        }
        done += n;
    }
    std::fclose(f);
    return 0;
}

// SplitMix64 finaliser (Steele, Lea, Flood 2014).
inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}
constexpr uint64_t kGolden = 0x9e3779b97f4a7c15ULL;

inline uint64_t stream_key(uint64_t seed, uint64_t stream) {
    return mix64(mix64(seed + kGolden) + kGolden * (stream + 1));
}
inline uint64_t draw(uint64_t key, uint64_t i) { return mix64(key + kGolden * (i + 1)); }
// (0, 1]: 53 random bits, offset by one so log() never sees zero.
inline double unit_open(uint64_t r) { return ((double)(r >> 11) + 1.0) * 0x1.0p-53; }

}  // namespace

extern "C" {

void gdn_error(const char *message) { std::fprintf(stderr, "%s\n", message); }

size_t gdn_total_weight_floats(const GDNWeightHeader *c) {
    return layer_offset(c, c->num_layers) + c->hidden_size +
           (size_t)c->vocab_size * c->hidden_size;
}

void gdn_default_config(GDNWeightHeader *c, uint32_t num_layers) {
    std::memset(c, 0, sizeof(*c));
    std::memcpy(c->magic, "GDNWv1\0\0", 8);
    c->version = 1;
    c->vocab_size = 32000;
    c->hidden_size = 2048;
    c->num_layers = num_layers;
    c->num_heads = 8;
    c->num_v_heads = 8;
    c->head_dim = 256;
    c->intermediate_size = 5632;
    c->conv_size = 4;
    c->max_seq_len = 2048;
    c->bos_token_id = 1;
    c->eos_token_id = 2;
    c->norm_eps = u2f(0x358637bdu);  // 1e-6f, gdn_model.cpp:155
}

int gdn_model_load(GDNModel *model, const char *path) { return load_impl(model, path, true); }
int gdn_model_load_fp32(GDNModel *model, const char *path) { return load_impl(model, path, false); }

void gdn_model_free(GDNModel *model) {
    std::free(model->weight_data);
    std::free(model->layers);
    std::memset(model, 0, sizeof(*model));
}

int gdn_model_save(const GDNModel *model, const char *path) {
    FILE *f = std::fopen(path, "wb");
    if (!f) {
        gdn_error("cannot create weight file");
        return -1;
    }
    const size_t total = gdn_total_weight_floats(&model->config);
    const bool ok = std::fwrite(&model->config, sizeof(GDNWeightHeader), 1, f) == 1 &&
                    std::fwrite(model->weight_data, sizeof(float), total, f) == total;
    std::fclose(f);
    if (!ok) gdn_error("weight file write failed");
    return ok ? 0 : -1;
}

void gdn_tile_bf16(const uint16_t *src, size_t n_rows, size_t k, int rt, uint16_t *dst) {
    const size_t kt_n = k / 32, blocks = n_rows / (16 * (size_t)rt);
#pragma omp parallel for schedule(static)
    for (long long bi = 0; bi < (long long)blocks; ++bi) {
        const size_t b = (size_t)bi;
        for (size_t kt = 0; kt < kt_n; ++kt)
            for (size_t r = 0; r < (size_t)rt; ++r) {
                uint16_t *tile = dst + (((b * kt_n + kt) * rt + r) * 64) * 8;
                for (size_t l = 0; l < 64; ++l) {
                    const uint16_t *row = src + (b * 16 * rt + r * 16 + l % 16) * k + kt * 32 + 8 * (l / 16);
                    std::memcpy(tile + l * 8, row, 16);
                }
            }
    }
}

void gdn_test_tile_bf16(const uint16_t *src, size_t n_rows, size_t k, int rt, uint16_t *dst) {
    gdn_tile_bf16(src, n_rows, k, rt, dst);
}

int gdn_validate_bf16_exact_weights(const float *wd, const GDNWeightHeader *c) {
    const size_t n = gdn_total_weight_floats(c);
    for (size_t i = 0; i < n; ++i) {
        const uint32_t b = f2u(wd[i]);
        if ((b & 0xffffu) != 0) {
            std::fprintf(stderr, "gdn: weight %zu is not BF16-exact (bits=0x%08x)\n", i, b);
            return -1;
        }
    }
    return 0;
}

void gdn_synth_normal(float *out, size_t n, uint64_t seed, uint64_t stream, float mean,
                      float std_, int round_bf16) {
    const uint64_t key = stream_key(seed, stream);
    const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
    for (long long pi = 0; pi < (long long)((n + 1) / 2); ++pi) {
        const uint64_t p = (uint64_t)pi;
        const double u1 = unit_open(draw(key, 2 * p));
        const double u2 = unit_open(draw(key, 2 * p + 1));
        const double r = std::sqrt(-2.0 * std::log(u1));
        const double z[2] = {r * std::cos(two_pi * u2), r * std::sin(two_pi * u2)};
        for (int e = 0; e < 2; ++e) {
            const size_t i = 2 * p + (size_t)e;
            if (i >= n) break;
            float v = (float)((double)mean + (double)std_ * z[e]);
            if (round_bf16) v = gdn_bf16_round_host(v);
            out[i] = v;
        }
    }
}

void gdn_synth_uniform(float *out, size_t n, uint64_t seed, uint64_t stream, float lo, float hi) {
    const uint64_t key = stream_key(seed, stream);
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i) {
        const double u = (double)(draw(key, (uint64_t)i) >> 11) * 0x1.0p-53;  // [0, 1)
        out[i] = (float)((double)lo + ((double)hi - (double)lo) * u);
    }
}

void gdn_synth_tokens(int32_t *out, size_t n, uint64_t seed, uint64_t stream, uint32_t vocab) {
    const uint64_t key = stream_key(seed, stream);
    for (size_t i = 0; i < n; ++i)
        out[i] = (int32_t)(((draw(key, i) >> 32) * (uint64_t)vocab) >> 32);
}

int gdn_model_synth(GDNModel *model, const GDNWeightHeader *config, uint64_t seed, float std_,
                    int bf16) {
    if (validate_config(config) != 0 || alloc_model(model, config) != 0) return -1;
    const GDNWeightHeader *c = &model->config;
    const size_t H = c->hidden_size, nh = c->num_heads, hd = c->head_dim;
    const size_t I = c->intermediate_size, cs = c->conv_size, V = c->vocab_size;
    // (pointer, count, is_norm) in .gdnw order; the ordinal is the stream id.
    struct T { const float *p; size_t n; bool norm; };
    std::vector<T> order;
    order.push_back({model->embeddings, V * H, false});
    for (uint32_t l = 0; l < c->num_layers; ++l) {
        const GDNLayerWeights &w = model->layers[l];
        order.push_back({w.attn_norm, H, true});
        order.push_back({w.a_log, nh, false});
        order.push_back({w.dt_bias, nh, false});
        order.push_back({w.q_proj, H * H, false});
        order.push_back({w.k_proj, H * H, false});
        order.push_back({w.v_proj, H * H, false});
        order.push_back({w.a_proj, nh * H, false});
        order.push_back({w.b_proj, nh * H, false});
        order.push_back({w.q_conv, H * cs, false});
        order.push_back({w.k_conv, H * cs, false});
        order.push_back({w.v_conv, H * cs, false});
        order.push_back({w.g_proj, H * H, false});
        order.push_back({w.o_norm, hd, true});
        order.push_back({w.o_proj, H * H, false});
        order.push_back({w.mlp_norm, H, true});
        order.push_back({w.mlp_gate_proj, I * H, false});
        order.push_back({w.mlp_up_proj, I * H, false});
        order.push_back({w.mlp_down_proj, H * I, false});
    }
    order.push_back({model->final_norm, H, true});
    order.push_back({model->lm_head, V * H, false});
    for (size_t t = 0; t < order.size(); ++t) {
        float *dst = const_cast<float *>(order[t].p);
        if (order[t].norm) {
            for (size_t i = 0; i < order[t].n; ++i) dst[i] = 1.0f;
        } else {
            gdn_synth_normal(dst, order[t].n, seed, t, 0.0f, std_, bf16);
        }
    }
    return 0;
}

// ---- BF16 helpers, gdn_model.cpp:309-325 ----
uint16_t gdn_test_fp32_to_bf16_rne_bits(uint32_t bits) {
    const uint32_t mag = bits & 0x7fffffffu;
    if (mag >= 0x7f800000u) {
        if (mag == 0x7f800000u) return (uint16_t)(bits >> 16);
        return (uint16_t)((bits & 0x80000000u) ? 0xffc0u : 0x7fc0u);
    }
    return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

uint32_t gdn_test_bf16_to_fp32_bits(uint16_t bits) { return (uint32_t)bits << 16; }

float gdn_bf16_round_host(float x) {
    return u2f(gdn_test_bf16_to_fp32_bits(gdn_test_fp32_to_bf16_rne_bits(f2u(x))));
}

// gdn_native_bf16_product_bits, gdn_model.cpp:401-462 (the native model of
// the FPGA multiplier): DAZ inputs, canonical NaN, FTZ below 0x007fc000.
uint16_t gdn_native_product_bits_host(uint16_t w, uint16_t x) {
    const uint32_t ew = (w >> 7) & 0xffu, fw = w & 0x7fu;
    const uint32_t ex = (x >> 7) & 0xffu, fx = x & 0x7fu;
    const bool w_nan = ew == 0xffu && fw, x_nan = ex == 0xffu && fx;
    const bool w_inf = ew == 0xffu && !fw, x_inf = ex == 0xffu && !fx;
    const bool w_zero = ew == 0, x_zero = ex == 0;
    const uint16_t sign = (uint16_t)((w ^ x) & 0x8000u);
    if (w_nan || x_nan || (w_inf && x_zero) || (x_inf && w_zero)) return 0x7fc0u;
    if (w_inf || x_inf) return (uint16_t)(sign | 0x7f80u);
    if (w_zero || x_zero) return sign;
    volatile float prod = u2f((uint32_t)w << 16) * u2f((uint32_t)x << 16);
    const uint32_t pb = f2u(prod), mag = pb & 0x7fffffffu;
    if (mag == 0x7f800000u) return (uint16_t)(pb >> 16);
    if (mag < 0x007fc000u) return (uint16_t)((pb >> 16) & 0x8000u);
    const uint16_t r = (uint16_t)((pb + 0x7fffu + ((pb >> 16) & 1u)) >> 16);
    if ((r & 0x7f80u) == 0) return (uint16_t)(r & 0x8000u);
    return r;
}

void gdn_pack_bf16_daz(const float *src, uint16_t *dst, size_t n, float *min_abs, float *max_abs,
                       int *nonfinite) {
    float mn = INFINITY, mx = 0.0f;
    int bad = 0;
#pragma omp parallel for schedule(static) reduction(min : mn) reduction(max : mx) reduction(| : bad)
    for (long long i = 0; i < (long long)n; ++i) {
        uint16_t b = (uint16_t)(f2u(src[i]) >> 16);
        const uint16_t e = (uint16_t)((b >> 7) & 0xffu);
        if (e == 0) b = (uint16_t)(b & 0x8000u);  // DAZ: subnormal -> signed zero
        if (e == 0xffu) bad = 1;
        dst[i] = b;
        const float a = std::fabs(u2f((uint32_t)b << 16));
        if (e != 0xffu && a > mx) mx = a;
        if (a != 0.0f && a < mn) mn = a;
    }
    *min_abs = mn;
    *max_abs = mx;
    *nonfinite = bad;
}

void gdn_scan_fp32(const float *src, size_t n, float *min_abs, float *max_abs, int *nonfinite) {
    float mn = INFINITY, mx = 0.0f;
    int bad = 0;
#pragma omp parallel for schedule(static) reduction(min : mn) reduction(max : mx) reduction(| : bad)
    for (long long i = 0; i < (long long)n; ++i) {
        const float a = std::fabs(src[i]);
        if (!std::isfinite(a)) {
            bad = 1;
        } else {
            if (a != 0.0f && a < mn) mn = a;
            if (a > mx) mx = a;
        }
    }
    *min_abs = mn;
    *max_abs = mx;
    *nonfinite = bad;
}

float gdn_native_bf16_mul_to_fp32(uint16_t weight, uint16_t activation) {
    return u2f((uint32_t)gdn_native_product_bits_host(weight, activation) << 16);
}

void gdn_compute_logits(const GDNModel *model, const float *hidden, float *logits_out) {
    const uint32_t V = model->config.vocab_size, H = model->config.hidden_size;
    std::vector<uint16_t> act(H);
    for (uint32_t i = 0; i < H; ++i)
        act[i] = gdn_test_fp32_to_bf16_rne_bits(f2u(gdn_bf16_round_host(hidden[i])));
#pragma omp parallel for schedule(static)
    for (long long v = 0; v < (long long)V; ++v) {
        const float *row = model->lm_head + (size_t)v * H;
        float sum = 0.0f;
        for (uint32_t i = 0; i < H; ++i)
            sum += gdn_native_bf16_mul_to_fp32((uint16_t)(f2u(row[i]) >> 16), act[i]);
        logits_out[v] = sum;
    }
}

// ---- .gdnstate, gdn_eval.cpp:196-267 / export_gdn_state.py:340-362 ----
int gdn_load_gdnstate(GDNRunState *state, const GDNModel *model, const char *path,
                      uint32_t *prompt_len, int32_t *seed_token) {
    FILE *f = std::fopen(path, "rb");
    if (!f) {
        gdn_error("cannot open .gdnstate file");
        return -1;
    }
    char magic[8];
    uint32_t v[9];
    auto fail = [&](const char *msg) {
        gdn_error(msg);
        std::fclose(f);
        return -1;
    };
    if (std::fread(magic, 1, 8, f) != 8 || std::memcmp(magic, "GDNSTAT1", 8) != 0)
        return fail(".gdnstate: bad magic (expected GDNSTAT1)");
    if (std::fread(v, sizeof(uint32_t), 9, f) != 9) return fail(".gdnstate: truncated header");
    const GDNWeightHeader *c = &model->config;
    if (v[1] != c->num_layers || v[2] != c->num_heads || v[3] != c->head_dim ||
        v[5] != c->hidden_size || v[6] != c->conv_size)
        return fail(".gdnstate: dims do not match the loaded model");
    if (std::fseek(f, (long)v[7] * (long)sizeof(int32_t), SEEK_CUR) != 0)
        return fail(".gdnstate: cannot skip prompt ids");
    const size_t rec = (size_t)v[1] * v[2] * v[3] * v[4];
    std::vector<float> buf(rec);
    if (std::fread(buf.data(), sizeof(float), rec, f) != rec)
        return fail(".gdnstate: truncated recurrent section");
    if (gdn_load_recurrent_state(state, buf.data(), rec) != 0)
        return fail(".gdnstate: recurrent values rejected");
    const size_t conv = (size_t)v[1] * 3u * (v[6] - 1u) * v[5];
    buf.resize(conv);
    if (std::fread(buf.data(), sizeof(float), conv, f) != conv)
        return fail(".gdnstate: truncated conv section");
    if (gdn_load_conv_tails(state, buf.data(), conv) != 0)
        return fail(".gdnstate: convolution-tail values rejected");
    std::fclose(f);
    if (prompt_len) *prompt_len = v[7];
    if (seed_token) *seed_token = (int32_t)v[8];
    return 0;
}

int gdn_write_gdnstate(const GDNWeightHeader *c, const char *path, const float *recurrent, const float *conv_tails,
                       const int32_t *prompt, uint32_t prompt_len, int32_t seed_token) {
    const size_t rec = (size_t)c->num_layers * c->num_heads * c->head_dim * c->head_dim;
    const size_t conv = (size_t)c->num_layers * 3u * (c->conv_size - 1u) * c->hidden_size;
    FILE *f = std::fopen(path, "wb");
    if (!f) {
        gdn_error("cannot create .gdnstate file");
        return -1;
    }
    const uint32_t v[9] = {1u, c->num_layers, c->num_heads, c->head_dim, c->head_dim,
                           c->hidden_size, c->conv_size, prompt_len, (uint32_t)seed_token};
    bool ok = std::fwrite("GDNSTAT1", 1, 8, f) == 8 && std::fwrite(v, 4, 9, f) == 9;
    if (ok && prompt_len) ok = std::fwrite(prompt, 4, prompt_len, f) == prompt_len;
    ok = ok && std::fwrite(recurrent, 4, rec, f) == rec && std::fwrite(conv_tails, 4, conv, f) == conv;
    ok = (std::fclose(f) == 0) && ok;
    if (!ok) gdn_error(".gdnstate write failed");
    return ok ? 0 : -1;
}

int gdn_save_gdnstate(const GDNRunState *state, const GDNModel *model, const char *path,
                      const int32_t *prompt, uint32_t prompt_len, int32_t seed_token) {
    const GDNWeightHeader *c = &model->config;
    const size_t rec = (size_t)c->num_layers * c->num_heads * c->head_dim * c->head_dim;
    const size_t conv = (size_t)c->num_layers * 3u * (c->conv_size - 1u) * c->hidden_size;
    std::vector<float> r(rec), cv(conv);
    if (gdn_save_recurrent_state(state, r.data(), rec) != 0 ||
        gdn_save_conv_tails(state, cv.data(), conv) != 0)
        return -1;
    return gdn_write_gdnstate(c, path, r.data(), cv.data(), prompt, prompt_len, seed_token);
}

}  // extern "C"
