// gdn_tools.cpp -- host-side logit tooling of libgdn_amd.so: the scoring
// log-probability, the strict argmax and the GPU-logit vector gate of the
// reference host (host.cpp), as C-ABI calls shared by the CLI and tests.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>

#include "gdn_amd.h"

namespace {

// Thresholds of the GPU-logit envelope (host.cpp:77-82).
constexpr double kGlobalNrmseMax = 0.01;
constexpr double kWorstStepNrmseMax = 0.04;
constexpr double kMinStepCosine = 0.9995;
constexpr double kWorstMaxOverRms = 0.10;
constexpr double kMaxAbs = 0.50;
constexpr uint32_t kTop5 = 5;

// Indices of the five largest values, descending; a later equal value does
// not displace an earlier one.
void top5(const float *v, uint32_t n, uint32_t *idx) {
    float best[kTop5];
    for (uint32_t r = 0; r < kTop5; ++r) {
        best[r] = std::numeric_limits<float>::lowest();
        idx[r] = n;
    }
    for (uint32_t i = 0; i < n; ++i) {
        const float x = v[i];
        uint32_t r = 0;
        while (r < kTop5 && !(x > best[r])) ++r;
        if (r == kTop5) continue;
        for (uint32_t s = kTop5 - 1; s > r; --s) {
            best[s] = best[s - 1];
            idx[s] = idx[s - 1];
        }
        best[r] = x;
        idx[r] = i;
    }
}

}  // namespace

extern "C" {

uint32_t gdn_strict_argmax(const float *logits, uint32_t n) {
    uint32_t best_i = 0;
    if (n == 0) return 0;
    float best = logits[0];
    for (uint32_t i = 1; i < n; ++i) {
        if (logits[i] > best) {
            best = logits[i];
            best_i = i;
        }
    }
    return best_i;
}

double gdn_token_logprob(const float *logits, uint32_t vocab, int32_t target) {
    if (vocab == 0 || target < 0 || (uint32_t)target >= vocab) return std::nan("");
    double m = logits[0];
    for (uint32_t i = 1; i < vocab; ++i) m = std::max(m, (double)logits[i]);
    double sum = 0.0;
    for (uint32_t i = 0; i < vocab; ++i) sum += std::exp((double)logits[i] - m);
    return ((double)logits[target] - m) - std::log(sum);
}

void gdn_logits_parity_init(GDNLogitsParity *p) {
    std::memset(p, 0, sizeof(*p));
    p->min_top5_overlap = kTop5;
    p->min_step_cosine = 1.0;
}

void gdn_logits_parity_step(GDNLogitsParity *p, const float *actual, const float *reference,
                            uint32_t vocab, uint32_t selected_token, int apply_fp32_tolerance) {
    double se = 0.0, cs = 0.0, rs = 0.0, dot = 0.0, step_max = 0.0;
    for (uint32_t i = 0; i < vocab; ++i) {
        const float a = actual[i], r = reference[i];
        const bool same_bits = std::memcmp(&a, &r, sizeof(float)) == 0;
        if (!same_bits) ++p->exact_mismatches;
        if (!std::isfinite(a) || !std::isfinite(r)) {
            if (!same_bits) {
                ++p->nonfinite_mismatches;
                if (apply_fp32_tolerance) ++p->tolerance_failures;
            }
            continue;
        }
        const double d = (double)a - (double)r, ad = std::fabs(d);
        p->max_abs_error = std::max(p->max_abs_error, ad);
        p->max_rel_error = std::max(p->max_rel_error, ad / std::max(1.0, std::fabs((double)r)));
        step_max = std::max(step_max, ad);
        se += d * d;
        cs += (double)a * a;
        rs += (double)r * r;
        dot += (double)a * r;
        if (apply_fp32_tolerance && ad > 1e-3 + 1e-4 * std::fabs((double)r)) ++p->tolerance_failures;
    }
    uint32_t ta[kTop5], tr[kTop5];
    top5(actual, vocab, ta);
    top5(reference, vocab, tr);
    uint32_t overlap = 0;
    for (uint32_t x = 0; x < kTop5; ++x)
        for (uint32_t y = 0; y < kTop5; ++y)
            if (ta[x] == tr[y]) {
                ++overlap;
                break;
            }
    p->min_top5_overlap = std::min(p->min_top5_overlap, overlap);
    p->squared_error_sum += se;
    p->candidate_squared_sum += cs;
    p->reference_squared_sum += rs;
    p->dot_product_sum += dot;
    if (rs > 0.0) {
        p->worst_step_nrmse = std::max(p->worst_step_nrmse, std::sqrt(se / rs));
        p->worst_max_abs_over_reference_rms =
            std::max(p->worst_max_abs_over_reference_rms, step_max / std::sqrt(rs / vocab));
    }
    const double norms = cs * rs;
    p->min_step_cosine = norms > 0.0 ? std::min(p->min_step_cosine, dot / std::sqrt(norms)) : -1.0;
    ++p->checked_steps;
    p->compared_values += vocab;
    if (gdn_strict_argmax(actual, vocab) != selected_token ||
        gdn_strict_argmax(reference, vocab) != selected_token)
        ++p->argmax_mismatches;
}

double gdn_logits_parity_nrmse(const GDNLogitsParity *p) {
    return p->reference_squared_sum > 0.0 ? std::sqrt(p->squared_error_sum / p->reference_squared_sum)
                                          : std::numeric_limits<double>::infinity();
}

double gdn_logits_parity_cosine(const GDNLogitsParity *p) {
    const double norms = p->candidate_squared_sum * p->reference_squared_sum;
    return norms > 0.0 ? p->dot_product_sum / std::sqrt(norms) : -1.0;
}

int gdn_logits_gate_passes(const GDNLogitsParity *p) {
    return p->nonfinite_mismatches == 0 && p->argmax_mismatches == 0 && p->min_top5_overlap >= kTop5 &&
           gdn_logits_parity_nrmse(p) <= kGlobalNrmseMax && p->worst_step_nrmse <= kWorstStepNrmseMax &&
           p->min_step_cosine >= kMinStepCosine && p->worst_max_abs_over_reference_rms <= kWorstMaxOverRms &&
           p->max_abs_error <= kMaxAbs;
}

}  // extern "C"
