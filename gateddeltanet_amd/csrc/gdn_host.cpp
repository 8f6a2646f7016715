// gdn_host.cpp -- host-side half of libgdn_amd.so: the .gdnw / .gdnstate
// formats, weight views, the seeded synthetic generator, and the reference's
// host helpers (BF16 rounding hooks, native product, scalar LM head).
//
// Reference behaviour followed (YAMWD/GatedDeltaNet):
//   gdn_model.cpp:1082-1245   .gdnw header rules, view order, payload load
//   gdn_model.cpp:309-325     BF16 RNE / widen
//   gdn_model.cpp:392-467     native BF16 product
//   gdn_model.cpp:3930-3965   gdn_compute_logits
//   gdn_eval.cpp:196-267      .gdnstate reader
//   export_gdn_state.py:340-362  .gdnstate writer
#include "gdn_amd.h"
#include "gdn_internal.h"
#include "gdn_libm.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

namespace {

uint32_t f2u(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
float u2f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

// What is wrong with a .gdnw header, or nullptr when the engine's host side
// accepts it.  The message names the offending fields and their values.
// gdn_total_weight_floats in 128-bit arithmetic, which cannot wrap for any
// 32-bit header fields (the largest term, 3 H^2 L, stays below 2^98).
unsigned __int128 payload_floats_wide(const GDNWeightHeader *c) {
    using u128 = unsigned __int128;
    const u128 H = c->hidden_size, nh = c->num_heads, hd = c->head_dim;
    const u128 I = c->intermediate_size, cs = c->conv_size, V = c->vocab_size, L = c->num_layers;
    const u128 layer = H + 2 * nh + 3 * H * H + 2 * nh * H + 3 * H * cs + H * H + hd + H * H + H + 2 * I * H + H * I;
    return V * H + L * layer + H + V * H;
}

const char *header_problem(const GDNWeightHeader *c, char *buf, size_t n) {
    static_assert(sizeof(GDNWeightHeader) == 60, "GDNWeightHeader is 60 bytes");
    if (std::memcmp(c->magic, "GDNWv1", 6) != 0) {
        std::snprintf(buf, n, "gdn: weight header magic is not GDNWv1");
    } else if (c->version != 1) {
        std::snprintf(buf, n, "gdn: weight header version %u, this library reads version 1", c->version);
    } else if (c->num_heads != c->num_v_heads) {
        std::snprintf(buf, n, "gdn: weight header has %u key heads and %u value heads; they must match",
                      c->num_heads, c->num_v_heads);
    } else if ((uint64_t)c->hidden_size != (uint64_t)c->num_heads * c->head_dim) {
        // (in 64 bits: a 32-bit product that wraps would match a small hidden_size)
        std::snprintf(buf, n, "gdn: hidden_size %u differs from num_heads %u x head_dim %u", c->hidden_size,
                      c->num_heads, c->head_dim);
    } else if (c->vocab_size == 0 || c->hidden_size == 0 || c->intermediate_size == 0 || c->conv_size == 0) {
        // conv_size - 1 sizes the conv tails, the vocabulary the argmax
        std::snprintf(buf, n, "gdn: weight header has a zero dimension (vocab %u, hidden %u, intermediate %u, conv %u)",
                      c->vocab_size, c->hidden_size, c->intermediate_size, c->conv_size);
    } else if (payload_floats_wide(c) > (unsigned __int128)(PTRDIFF_MAX / sizeof(float))) {
        // the size_t payload arithmetic would wrap, and a wrapped total would
        // pass the file-size check with a small file
        std::snprintf(buf, n, "gdn: weight header dimensions describe more payload than this process can address");
    } else {
        return nullptr;
    }
    return buf;
}

int validate_config(const GDNWeightHeader *c) {
    char msg[160];
    if (const char *why = header_problem(c, msg, sizeof(msg))) {
        gdn_error(why);
        return -1;
    }
    return 0;
}

// Index of the first value whose low 16 bits are not zero (a value BF16
// cannot hold), or n when every value is BF16-exact.  Parallel scan.
size_t first_non_bf16(const float *v, size_t n) {
    size_t first = n;
#pragma omp parallel for schedule(static) reduction(min : first)
    for (long long i = 0; i < (long long)n; ++i) {
        uint32_t b;
        std::memcpy(&b, v + i, 4);
        if ((b & 0xffffu) != 0 && (size_t)i < first) first = (size_t)i;
    }
    return first;
}

void report_non_bf16(const char *what, const float *v, size_t i) {
    uint32_t b;
    std::memcpy(&b, v + i, 4);
    std::fprintf(stderr, "gdn: %s value %zu (bits 0x%08x) is not a BF16 number\n", what, i, b);
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

// Reads a .gdnw: the file size is checked against the header's dimensions
// before the payload buffer is allocated, the payload is read in large
// pieces, and (for the BF16 contracts) the whole blob is scanned afterwards.
int load_impl(GDNModel *m, const char *path, bool require_bf16) {
    std::memset(m, 0, sizeof(*m));
    FILE *f = std::fopen(path, "rb");
    if (!f) {
        std::fprintf(stderr, "gdn: cannot open weight file %s\n", path);
        return -1;
    }
    struct Closer {
        FILE *f;
        ~Closer() { std::fclose(f); }
    } closer{f};
    GDNWeightHeader hdr;
    if (std::fread(&hdr, 1, sizeof(hdr), f) != sizeof(hdr)) {
        std::fprintf(stderr, "gdn: %s is shorter than a weight header\n", path);
        return -1;
    }
    if (validate_config(&hdr) != 0) return -1;
    const size_t total = gdn_total_weight_floats(&hdr);
    if (std::fseek(f, 0, SEEK_END) != 0) {
        std::fprintf(stderr, "gdn: cannot seek in %s\n", path);
        return -1;
    }
    const long long have = (long long)std::ftell(f) - (long long)sizeof(hdr);
    if (have < 0 || (unsigned long long)have < total * sizeof(float)) {
        std::fprintf(stderr, "gdn: %s holds %lld payload bytes, its header describes %zu\n", path, have,
                     total * sizeof(float));
        return -1;
    }
    if (std::fseek(f, (long)sizeof(hdr), SEEK_SET) != 0 || alloc_model(m, &hdr) != 0) return -1;
    const size_t piece = (size_t)64 << 20;  // floats per fread
    for (size_t done = 0; done < total; done += piece) {
        const size_t n = std::min(piece, total - done);
        if (std::fread(m->weight_data + done, sizeof(float), n, f) != n) {
            std::fprintf(stderr, "gdn: read error in %s at float %zu\n", path, done);
            gdn_model_free(m);
            return -1;
        }
    }
    if (require_bf16) {
        const size_t bad = first_non_bf16(m->weight_data, total);
        if (bad != total) {
            report_non_bf16("weight", m->weight_data, bad);
            gdn_error("gdn: the BF16 contracts take a BF16-valued checkpoint "
                      "(gdn_model_load_fp32 loads any FP32 payload)");
            gdn_model_free(m);
            return -1;
        }
    }
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
        std::fprintf(stderr, "gdn: cannot create weight file %s\n", path);
        return -1;
    }
    const size_t total = gdn_total_weight_floats(&model->config);
    const bool ok = std::fwrite(&model->config, sizeof(GDNWeightHeader), 1, f) == 1 &&
                    std::fwrite(model->weight_data, sizeof(float), total, f) == total;
    std::fclose(f);
    if (!ok) std::fprintf(stderr, "gdn: writing weight file %s failed\n", path);
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
    const size_t bad = first_non_bf16(wd, n);
    if (bad == n) return 0;
    report_non_bf16("weight", wd, bad);
    return -1;
}

void gdn_report_non_bf16(const char *what, const float *values, size_t index) {
    report_non_bf16(what, values, index);
}

size_t gdn_first_non_bf16(const float *values, size_t n) { return first_non_bf16(values, n); }

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

}  // extern "C"

namespace {

// Outcome counters of the native product (the fields of GDNMixedMulStats).
struct ProductCounts {
    uint64_t calls = 0, special = 0, flushed_in = 0, flushed_out = 0, overflow = 0;
};

// gdn_native_bf16_product_bits, gdn_model.cpp:401-462 (the native model of
// the FPGA multiplier): DAZ inputs, canonical NaN, FTZ below 0x007fc000;
// each outcome is counted as the reference counts it.
inline uint16_t native_product(uint16_t w, uint16_t x, ProductCounts &n) {
    const uint32_t ew = (w >> 7) & 0xffu, fw = w & 0x7fu;
    const uint32_t ex = (x >> 7) & 0xffu, fx = x & 0x7fu;
    const bool w_nan = ew == 0xffu && fw, x_nan = ex == 0xffu && fx;
    const bool w_inf = ew == 0xffu && !fw, x_inf = ex == 0xffu && !fx;
    const bool w_zero = ew == 0, x_zero = ex == 0;
    const uint16_t sign = (uint16_t)((w ^ x) & 0x8000u);
    ++n.calls;
    if (w_nan || x_nan || w_inf || x_inf || w_zero || x_zero) {
        ++n.special;
        if ((w_zero && fw) || (x_zero && fx)) ++n.flushed_in;
    }
    if (w_nan || x_nan || (w_inf && x_zero) || (x_inf && w_zero)) return 0x7fc0u;
    if (w_inf || x_inf) return (uint16_t)(sign | 0x7f80u);
    if (w_zero || x_zero) return sign;
    volatile float prod = u2f((uint32_t)w << 16) * u2f((uint32_t)x << 16);
    const uint32_t pb = f2u(prod), mag = pb & 0x7fffffffu;
    if (mag == 0x7f800000u) {
        ++n.overflow;
        return (uint16_t)(pb >> 16);
    }
    if (mag < 0x007fc000u) {
        ++n.flushed_out;
        return (uint16_t)((pb >> 16) & 0x8000u);
    }
    const uint16_t r = (uint16_t)((pb + 0x7fffu + ((pb >> 16) & 1u)) >> 16);
    if ((r & 0x7f80u) == 0) {
        ++n.flushed_out;
        return (uint16_t)(r & 0x8000u);
    }
    if ((r & 0x7fffu) == 0x7f80u) ++n.overflow;
    return r;
}

// Process-wide product counters (the reference keeps one file-static set,
// gdn_model.cpp:327-336) and the device-counting switch.
std::mutex g_stats_mu;
GDNMixedMulStats g_stats = {};
int g_device_counting = 0;

void stats_add(const ProductCounts &n) {
    std::lock_guard<std::mutex> lock(g_stats_mu);
    g_stats.calls += n.calls;
    g_stats.special_inputs += n.special;
    g_stats.flushed_inputs += n.flushed_in;
    g_stats.flushed_outputs += n.flushed_out;
    g_stats.overflows += n.overflow;
}

}  // namespace

extern "C" {

uint16_t gdn_native_product_bits_host(uint16_t w, uint16_t x) {
    ProductCounts n;
    return native_product(w, x, n);
}

void gdn_reset_mixed_mul_stats(void) {
    std::lock_guard<std::mutex> lock(g_stats_mu);
    g_stats = GDNMixedMulStats{};
    g_device_counting = 1;
}

void gdn_stop_mixed_mul_stats(void) {
    std::lock_guard<std::mutex> lock(g_stats_mu);
    g_device_counting = 0;
}

GDNMixedMulStats gdn_get_mixed_mul_stats(void) {
    std::lock_guard<std::mutex> lock(g_stats_mu);
    return g_stats;
}

int gdn_stats_counting(void) {
    std::lock_guard<std::mutex> lock(g_stats_mu);
    return g_device_counting;
}

void gdn_stats_add(uint64_t calls, uint64_t special, uint64_t flushed_in, uint64_t flushed_out,
                   uint64_t overflow) {
    ProductCounts n;
    n.calls = calls;
    n.special = special;
    n.flushed_in = flushed_in;
    n.flushed_out = flushed_out;
    n.overflow = overflow;
    stats_add(n);
}

void gdn_weight_column_counts(const float *W, size_t rows, size_t K, uint32_t *spec, uint32_t *sub) {
#pragma omp parallel for schedule(static)
    for (long long kk = 0; kk < (long long)K; ++kk) {
        uint32_t a = 0, b = 0;
        for (size_t r = 0; r < rows; ++r) {
            const uint32_t w = f2u(W[r * K + (size_t)kk]) >> 16;
            const uint32_t e = (w >> 7) & 0xffu;
            a += (e == 0 || e == 0xffu) ? 1u : 0u;
            b += (e == 0 && (w & 0x7fu) != 0) ? 1u : 0u;
        }
        spec[kk] += a;
        sub[kk] += b;
    }
}

void gdn_count_native_outcomes(const float *W, size_t rows, size_t K, const uint16_t *xbits, uint64_t *flushed,
                               uint64_t *overflow) {
    uint64_t fo = 0, ov = 0;
#pragma omp parallel for schedule(static) reduction(+ : fo, ov)
    for (long long r = 0; r < (long long)rows; ++r) {
        ProductCounts n;
        for (size_t k = 0; k < K; ++k)
            (void)native_product((uint16_t)(f2u(W[(size_t)r * K + k]) >> 16), xbits[k], n);
        fo += n.flushed_out;
        ov += n.overflow;
    }
    *flushed += fo;
    *overflow += ov;
}

// The reference's BF16 stripe layout of the recurrent state
// (gdn_scatter_recurrent_state, gdn_model.cpp:850-890): value v of 256-value
// row r goes to stripe 2 (v / 128) + (v / 16) % 2, beat 2 r + (v / 64) % 2,
// BF16 lane 16 ((v / 32) % 2) + v % 16.  Values are rounded to BF16 (exact
// for the REF contract's BF16-exact state).
void gdn_pack_state_stripes(const float *rec, size_t rows, Beat512 *const stripes[]) {
#pragma omp parallel for schedule(static)
    for (long long ri = 0; ri < (long long)rows; ++ri) {
        const size_t r = (size_t)ri;
        for (uint32_t v = 0; v < 256; ++v) {
            const uint32_t port = 2 * (v >> 7) + ((v >> 4) & 1u);
            const size_t beat = 2 * r + ((v >> 6) & 1u);
            const uint32_t lane = 16 * ((v >> 5) & 1u) + (v & 15u);
            const uint16_t b = gdn_test_fp32_to_bf16_rne_bits(f2u(rec[r * 256 + v]));
            std::memcpy(stripes[port][beat].bytes + 2 * lane, &b, 2);
        }
    }
}

// The conv tails of n_stripes (layer, q|k|v) stripes, [W-1][hidden] each,
// as BF16 payloads in the first half of each GDN_CONV_TAIL_FLOATS_PER_STRIPE
// reservation of the workspace head buffer, the rest zero
// (gdn_pack_conv_tails_bf16, gdn_model.cpp:892-928).
void gdn_pack_tail_stripes(const float *conv, size_t n_stripes, float *head_buffer) {
    std::memset(head_buffer, 0, (size_t)GDN_WSF_HEADBUF * 4);
    const size_t per = GDN_CONV_TAIL_FLOATS_PER_STRIPE;
    for (size_t st = 0; st < n_stripes; ++st) {
        uint16_t *d = reinterpret_cast<uint16_t *>(head_buffer + st * per);
        for (size_t i = 0; i < per; ++i) d[i] = gdn_test_fp32_to_bf16_rne_bits(f2u(conv[st * per + i]));
    }
}

int gdn_model_wrap(GDNModel *m, const GDNWeightHeader *c, const float *data) {
    std::memset(m, 0, sizeof(*m));
    m->config = *c;
    m->weight_data = const_cast<float *>(data);
    m->layers = static_cast<GDNLayerWeights *>(std::calloc(c->num_layers ? c->num_layers : 1,
                                                            sizeof(GDNLayerWeights)));
    if (!m->layers) {
        gdn_error("gdn: host allocation failed");
        return -1;
    }
    assign_views(m);
    return 0;
}

void gdn_test_libm_array(int which, const float *in, float *out, size_t n) {
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i)
        out[i] = which == 0 ? gdn_libm::gdn_expf(in[i]) : gdn_libm::gdn_log1pf(in[i]);
}

// ---- Beat512 lane accessors, gdn_model.h:207-210 ----
void gdn_test_set_fp32_lane_bits(Beat512 *beat, uint32_t lane, uint32_t bits) {
    std::memcpy(beat->bytes + 4 * (lane & 15u), &bits, 4);
}
uint32_t gdn_test_get_fp32_lane_bits(const Beat512 *beat, uint32_t lane) {
    uint32_t b;
    std::memcpy(&b, beat->bytes + 4 * (lane & 15u), 4);
    return b;
}
void gdn_test_set_bf16_lane_bits(Beat512 *beat, uint32_t lane, uint16_t bits) {
    std::memcpy(beat->bytes + 2 * (lane & 31u), &bits, 2);
}
uint16_t gdn_test_get_bf16_lane_bits(const Beat512 *beat, uint32_t lane) {
    uint16_t b;
    std::memcpy(&b, beat->bytes + 2 * (lane & 31u), 2);
    return b;
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
    ProductCounts n;
    const uint16_t r = native_product(weight, activation, n);
    stats_add(n);
    return u2f((uint32_t)r << 16);
}

void gdn_compute_logits(const GDNModel *model, const float *hidden, float *logits_out) {
    const uint32_t V = model->config.vocab_size, H = model->config.hidden_size;
    std::vector<uint16_t> act(H);
    for (uint32_t i = 0; i < H; ++i)
        act[i] = gdn_test_fp32_to_bf16_rne_bits(f2u(gdn_bf16_round_host(hidden[i])));
#pragma omp parallel
    {
        ProductCounts n;
#pragma omp for schedule(static)
        for (long long v = 0; v < (long long)V; ++v) {
            const float *row = model->lm_head + (size_t)v * H;
            float sum = 0.0f;
            for (uint32_t i = 0; i < H; ++i)
                sum += u2f((uint32_t)native_product((uint16_t)(f2u(row[i]) >> 16), act[i], n) << 16);
            logits_out[v] = sum;
        }
        stats_add(n);
    }
}

// ---- .gdnstate, gdn_eval.cpp:196-267 / export_gdn_state.py:340-362 ----
int gdn_load_gdnstate(GDNRunState *state, const GDNModel *model, const char *path,
                      uint32_t *prompt_len, int32_t *seed_token) {
    FILE *f = std::fopen(path, "rb");
    if (!f) {
        std::fprintf(stderr, "gdn: cannot open state file %s\n", path);
        return -1;
    }
    struct Closer {
        FILE *f;
        ~Closer() { std::fclose(f); }
    } closer{f};
    // "GDNSTAT1", then u32 {version, layers, heads, K, V, hidden, conv width,
    // prompt length, seed token}
    struct {
        char magic[8];
        uint32_t version, layers, heads, dk, dv, hidden, width, prompt_len, seed;
    } h;
    static_assert(sizeof(h) == 44, "packed .gdnstate header");
    if (std::fread(&h, 1, sizeof(h), f) != sizeof(h) || std::memcmp(h.magic, "GDNSTAT1", 8) != 0) {
        std::fprintf(stderr, "gdn: %s has no GDNSTAT1 header\n", path);
        return -1;
    }
    const GDNWeightHeader *c = &model->config;
    if (h.version != 1) {
        std::fprintf(stderr, "gdn: %s is .gdnstate version %u, this library reads version 1\n", path, h.version);
        return -1;
    }
    // Every dimension that sizes a section is checked against the model, the
    // value dimension included (the sections are sized from the file's own
    // header below, so an unchecked one could ask for any allocation).
    if (h.layers != c->num_layers || h.heads != c->num_heads || h.dk != c->head_dim || h.dv != c->head_dim ||
        h.hidden != c->hidden_size || h.width != c->conv_size) {
        std::fprintf(stderr,
                     "gdn: %s describes %u layers x %u heads x %u x %u, hidden %u, conv %u; the model has "
                     "%u x %u x %u x %u, hidden %u, conv %u\n",
                     path, h.layers, h.heads, h.dk, h.dv, h.hidden, h.width, c->num_layers, c->num_heads,
                     c->head_dim, c->head_dim, c->hidden_size, c->conv_size);
        return -1;
    }
    const size_t rec = (size_t)h.layers * h.heads * h.dk * h.dv;
    const size_t conv = (size_t)h.layers * 3u * (h.width - 1u) * h.hidden;
    std::vector<float> buf(rec > conv ? rec : conv);
    // the prompt ids are informational: skip them
    const bool ok = std::fseek(f, (long)sizeof(h) + 4L * (long)h.prompt_len, SEEK_SET) == 0 &&
                    std::fread(buf.data(), sizeof(float), rec, f) == rec;
    if (!ok) {
        std::fprintf(stderr, "gdn: %s ends inside its recurrent-state section\n", path);
        return -1;
    }
    if (gdn_load_recurrent_state(state, buf.data(), rec) != 0) return -1;
    if (std::fread(buf.data(), sizeof(float), conv, f) != conv) {
        std::fprintf(stderr, "gdn: %s ends inside its conv-tail section\n", path);
        return -1;
    }
    if (gdn_load_conv_tails(state, buf.data(), conv) != 0) return -1;
    if (prompt_len) *prompt_len = h.prompt_len;
    if (seed_token) *seed_token = (int32_t)h.seed;
    return 0;
}

int gdn_write_gdnstate(const GDNWeightHeader *c, const char *path, const float *recurrent, const float *conv_tails,
                       const int32_t *prompt, uint32_t prompt_len, int32_t seed_token) {
    const size_t rec = (size_t)c->num_layers * c->num_heads * c->head_dim * c->head_dim;
    const size_t conv = (size_t)c->num_layers * 3u * (c->conv_size - 1u) * c->hidden_size;
    FILE *f = std::fopen(path, "wb");
    if (!f) {
        std::fprintf(stderr, "gdn: cannot create state file %s\n", path);
        return -1;
    }
    const uint32_t v[9] = {1u, c->num_layers, c->num_heads, c->head_dim, c->head_dim,
                           c->hidden_size, c->conv_size, prompt_len, (uint32_t)seed_token};
    bool ok = std::fwrite("GDNSTAT1", 1, 8, f) == 8 && std::fwrite(v, 4, 9, f) == 9;
    if (ok && prompt_len) ok = std::fwrite(prompt, 4, prompt_len, f) == prompt_len;
    ok = ok && std::fwrite(recurrent, 4, rec, f) == rec && std::fwrite(conv_tails, 4, conv, f) == conv;
    ok = (std::fclose(f) == 0) && ok;
    if (!ok) std::fprintf(stderr, "gdn: writing state file %s failed\n", path);
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
