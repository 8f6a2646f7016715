/*
 * gdn_oracle.c -- CPU restatement of the reference's batch-1 decode
 * arithmetic (YAMWD/GatedDeltaNet, c_impl/gdn_model.cpp).
 *
 * TEST INFRASTRUCTURE: the checker for the HIP engine, never the product.
 * Built with -O3 -ffp-contract=off (the reference Makefile:27-34 flag) and
 * without -ffast-math, so every expression rounds where the C source does
 * (vectorised loops perform the same IEEE operations in the same order).
 *
 * What pins each function (tests named after tests/):
 *   orc_rne_bits / orc_widen_bits   the 20 RNE boundary cases and the
 *       exhaustive widen of packed_bf16_test.cpp:219-246 (golden fixture),
 *       an exhaustive 2^32 sweep against an independent integer model
 *       (test_oracle_bf16.py).
 *   orc_native_product_bits         the rule text of the reference
 *       (architecture.md:867-878): an independent double-precision model on
 *       every BF16 weight x 64 structured activations and 2^20 random pairs,
 *       the flush tie 0x007fc000 and the special classes
 *       (test_oracle_bf16.py).
 *   orc_tree16 / orc_tree256        closed forms: powers of two, integer
 *       inputs, and order-sensitive inputs whose result differs under any
 *       other association (test_oracle_ops.py: test_tree16_association,
 *       test_tree256_association).
 *   orc_gemv / orc_gemv_tiny        one-hot activations select the rounded
 *       weight column; integer inputs give exact sums; cancellation vectors
 *       distinguish the bank order (test_gemv_bank_order, test_gemv_tiny_
 *       order); a brute force against a literal Python loop over the stated
 *       formula on random operands with zeros and subnormals
 *       (test_gemv_brute_force_literal_loop).  The rows' branch-free native
 *       product equals orc_native_product_bits on every weight x structured
 *       activations and 2^22 random pairs (test_native_product_select_form).
 *   orc_rmsnorm / residual / output_norm_gate   constant vectors give exact
 *       results; scale invariance; the 16-value chunk / sequential chunk-sum
 *       association is pinned by inputs where a flat sequential sum or a
 *       tree over the chunk sums gives a different result
 *       (test_rmsnorm_sum_is_chunked_then_sequential,
 *       test_output_norm_sum_is_chunked_per_head).
 *   orc_conv_silu                   tap one-hots give silu(x) / silu(t0);
 *       zero tails propagate; tail shift; the left association
 *       ((t0w0 + t1w1) + t2w2) + xw3 by inputs where any other pairing
 *       differs (test_conv_taps_and_shift, test_conv_sum_is_left_associated).
 *   orc_recurrence_head             beta=0, decay=1/beta=1/k=e_j special
 *       cases; plain-IEEE case decay=1 beta=0.5; fp64 textbook recurrence
 *       (chunk.py:688-718 restated) within tolerance (test_oracle_ops.py).
 *   orc_argmax                      ties, -inf, NaN (test_oracle_ops.py).
 *   orc_layer_forward / orc_decode_step   composition only; each piece is
 *       pinned above.  No reference-held vector covers random-init weights
 *       (every committed golden of the reference needs the real checkpoint),
 *       so the end-to-end composition is "parity unpinned" beyond the
 *       per-piece pins and the fp64 cross-check of test_oracle_model.py.
 */
#include "gdn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

void orc_set_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* fp32_to_bf16_rne, gdn_model.cpp:309-320: round half to even on the upper
 * 16 bits, infinities keep their sign, NaNs become the canonical quiet NaN
 * of their sign; subnormals are rounded, not flushed. */
uint16_t orc_rne_bits(uint32_t bits) {
    const uint32_t mag = bits & 0x7fffffffu;
    if (mag >= 0x7f800000u) {
        if (mag == 0x7f800000u) return (uint16_t)(bits >> 16);
        return (uint16_t)((bits & 0x80000000u) ? 0xffc0u : 0x7fc0u);
    }
    return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

/* bf16_to_fp32, gdn_model.cpp:305-307: widening is a 16-bit shift. */
uint32_t orc_widen_bits(uint16_t b) { return (uint32_t)b << 16; }

float orc_bf16_round(float x) {
    return u2f(orc_widen_bits(orc_rne_bits(f2u(x))));
}

/* Contract rounding point: identity in the FP32 control arm. */
static inline float R(int contract, float x) {
    return contract == ORC_FP32 ? x : orc_bf16_round(x);
}

/* gdn_native_bf16_product_bits (native branch), gdn_model.cpp:401-462.
 * Inputs with a zero exponent are zeros (DAZ).  NaN operands, or an
 * infinity times a zero, give the positive canonical NaN; otherwise an
 * infinity operand gives a signed infinity and a zero operand a signed zero.
 * Finite products are formed in FP32 (exact for two 8-bit significands
 * unless they underflow), flushed to a signed zero below the magnitude
 * 0x007fc000, and rounded half-to-even to BF16; a rounded result with a
 * zero exponent is flushed as well. */
uint16_t orc_native_product_bits(uint16_t w, uint16_t x) {
    const uint32_t ew = (w >> 7) & 0xffu, fw = w & 0x7fu;
    const uint32_t ex = (x >> 7) & 0xffu, fx = x & 0x7fu;
    const int w_nan = ew == 0xffu && fw != 0, x_nan = ex == 0xffu && fx != 0;
    const int w_inf = ew == 0xffu && fw == 0, x_inf = ex == 0xffu && fx == 0;
    const int w_zero = ew == 0, x_zero = ex == 0;
    const uint16_t sign = (uint16_t)((w ^ x) & 0x8000u);
    if (w_nan || x_nan || (w_inf && x_zero) || (x_inf && w_zero))
        return 0x7fc0u;
    if (w_inf || x_inf) return (uint16_t)(sign | 0x7f80u);
    if (w_zero || x_zero) return sign;
    volatile float prod = u2f(orc_widen_bits(w)) * u2f(orc_widen_bits(x));
    const uint32_t pb = f2u(prod);
    const uint32_t mag = pb & 0x7fffffffu;
    if (mag == 0x7f800000u) return (uint16_t)(pb >> 16);
    if (mag < 0x007fc000u) return (uint16_t)((pb >> 16) & 0x8000u);
    const uint16_t r = (uint16_t)((pb + 0x7fffu + ((pb >> 16) & 1u)) >> 16);
    if ((r & 0x7f80u) == 0) return (uint16_t)(r & 0x8000u);
    return r;
}

/* ---- transcendentals: gdn_sigmoid / gdn_silu / gdn_softplus,
 *      gdn_model.cpp:1307-1330 ---- */
float orc_expf(float x, int tmode) {
    return tmode == ORC_CR ? (float)exp((double)x) : expf(x);
}

float orc_log1pf(float x, int tmode) {
    return tmode == ORC_CR ? (float)log1p((double)x) : log1pf(x);
}

float orc_sigmoid(float x, int tmode) {
    if (x >= 0.0f) {
        const float z = orc_expf(-x, tmode);
        return 1.0f / (1.0f + z);
    }
    const float z = orc_expf(x, tmode);
    return z / (1.0f + z);
}

float orc_silu(float x, int tmode) { return x * orc_sigmoid(x, tmode); }

float orc_softplus(float x, int tmode) {
    if (x > 20.0f) return x;
    if (x < -20.0f) return orc_expf(x, tmode);
    return orc_log1pf(orc_expf(x, tmode), tmode);
}

/* gemv32_tree16 (gdn_model.cpp:4004-4035) and gdn_tree16 (:1477-1488):
 * balanced pairwise association over 16 contiguous values. */
float orc_tree16(const float *p) {
    const float s0 = p[0] + p[1], s1 = p[2] + p[3];
    const float s2 = p[4] + p[5], s3 = p[6] + p[7];
    const float s4 = p[8] + p[9], s5 = p[10] + p[11];
    const float s6 = p[12] + p[13], s7 = p[14] + p[15];
    const float a0 = s0 + s1, a1 = s2 + s3, a2 = s4 + s5, a3 = s6 + s7;
    const float b0 = a0 + a1, b1 = a2 + a3;
    return b0 + b1;
}

/* gdn_tree_reduce_256, gdn_model.cpp:1336-1374: eight pairwise levels. */
float orc_tree256(const float *a) {
    float buf[256];
    int n = 256;
    memcpy(buf, a, sizeof(buf));
    while (n > 1) {
        for (int i = 0; i < n / 2; ++i) buf[i] = buf[2 * i] + buf[2 * i + 1];
        n /= 2;
    }
    return buf[0];
}

/* The native product of two BF16-exact FP32 words as integer selects: the
 * same IEEE multiply and the same cases as orc_native_product_bits, with
 * its special cases applied last in reverse order of precedence (the last
 * select wins), so that the row loop below vectorises.  Returns the widened
 * product's bits.  tests/test_oracle_bf16.py compares the two forms. */
static inline uint32_t native_bits_sel(uint32_t wb, uint32_t xb) {
    const uint32_t w = wb >> 16, x = xb >> 16;
    const uint32_t ew = (w >> 7) & 0xffu, fw = w & 0x7fu;
    const uint32_t ex = (x >> 7) & 0xffu, fx = x & 0x7fu;
    const uint32_t sign = (w ^ x) & 0x8000u;
    const uint32_t pb = f2u(u2f(w << 16) * u2f(x << 16));
    const uint32_t mag = pb & 0x7fffffffu;
    const uint32_t r = (pb + 0x7fffu + ((pb >> 16) & 1u)) >> 16;
    uint32_t res = (r & 0x7f80u) == 0 ? (r & 0x8000u) : r;
    res = mag < 0x007fc000u ? ((pb >> 16) & 0x8000u) : res;
    res = mag == 0x7f800000u ? (pb >> 16) : res;
    const int w_zero = ew == 0, x_zero = ex == 0;
    const int w_inf = ew == 0xffu && fw == 0, x_inf = ex == 0xffu && fx == 0;
    const int w_nan = ew == 0xffu && fw != 0, x_nan = ex == 0xffu && fx != 0;
    res = (w_zero | x_zero) ? sign : res;
    res = (w_inf | x_inf) ? (sign | 0x7f80u) : res;
    res = (w_nan | x_nan | (w_inf & x_zero) | (x_inf & w_zero)) ? 0x7fc0u : res;
    return res << 16;
}

/* p[i] = the contract's product of w[i] and x[i]: native BF16 (ORC_REF,
 * ORC_BF16W_FP32S) or plain FP32 (ORC_FP32, ORC_BF16X). */
static inline void row_products(int contract, const float *w, const float *x,
                                int n, float *p) {
    if (contract == ORC_FP32 || contract == ORC_BF16X) {
        for (int i = 0; i < n; ++i) p[i] = w[i] * x[i];
        return;
    }
    for (int i = 0; i < n; ++i) {
        uint32_t wb, xb;
        memcpy(&wb, w + i, 4);
        memcpy(&xb, x + i, 4);
        const uint32_t pb = native_bits_sel(wb, xb);
        memcpy(p + i, &pb, 4);
    }
}

#define ORC_KMAX 8192

/* One dense GEMV row, gemv32_cluster2 + gemv32_pair_dot16 +
 * gemv32_reduce_parts (gdn_model.cpp:4037-4059, :4444-4586, :4115-4127).
 * For every 32-column beat b the lower and upper 16 products are each
 * reduced with tree16; four banks (lower/upper x even/odd beat) accumulate
 * those sums in beat order starting from +0.0f; the row result is
 * (even_lo + even_hi) + (odd_lo + odd_hi).  The four tree16 levels run over
 * the whole row at once (level m adds neighbouring pairs of level m - 1),
 * which is tree16 on every 16-product half-beat.  Products are native BF16
 * (ORC_REF, ORC_BF16W_FP32S) or plain FP32 (ORC_FP32, ORC_BF16X).  The row
 * functions are compiled for AVX-512, AVX2 and baseline x86-64 and chosen
 * at load time; every clone performs the same IEEE operations. */
#if defined(__x86_64__) && defined(__GNUC__) && !defined(__clang__)
#define ORC_CLONES __attribute__((target_clones("avx512f", "avx2", "default")))
#else
#define ORC_CLONES
#endif

ORC_CLONES
static float gemv_row(int contract, const float *w, const float *x, int K) {
    float p[ORC_KMAX], s1[ORC_KMAX / 2], s2[ORC_KMAX / 4], s3[ORC_KMAX / 8];
    float t[ORC_KMAX / 16];
    row_products(contract, w, x, K, p);
    for (int i = 0; i < K / 2; ++i) s1[i] = p[2 * i] + p[2 * i + 1];
    for (int i = 0; i < K / 4; ++i) s2[i] = s1[2 * i] + s1[2 * i + 1];
    for (int i = 0; i < K / 8; ++i) s3[i] = s2[2 * i] + s2[2 * i + 1];
    for (int i = 0; i < K / 16; ++i) t[i] = s3[2 * i] + s3[2 * i + 1];
    float bank[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int b = 0; b < K / 32; ++b) {
        const int e = (b & 1) * 2;
        bank[e] = bank[e] + t[2 * b];
        bank[e + 1] = bank[e + 1] + t[2 * b + 1];
    }
    const float s0 = bank[0] + bank[1];
    const float s1v = bank[2] + bank[3];
    return s0 + s1v;
}

/* gdn_compute_logits' row: the same native products, summed sequentially
 * from +0.0f. */
ORC_CLONES
static float seq_native_row(const float *w, const float *x, int K) {
    float p[ORC_KMAX];
    row_products(ORC_REF, w, x, K, p);
    float sum = 0.0f;
    for (int i = 0; i < K; ++i) sum += p[i];
    return sum;
}

void orc_gemv(int contract, const float *W, const float *x, int M, int K,
              float *y) {
    if (K > ORC_KMAX || K % 32 != 0) abort();  /* whole beats, row buffers */
#pragma omp parallel for schedule(static) if (M >= 64)
    for (int r = 0; r < M; ++r)
        y[r] = gemv_row(contract, W + (size_t)r * K, x, K);
}

void orc_gemv_rows(int contract, const float *W, const float *x, int M, int K,
                   float *y) {
    if (K > ORC_KMAX || K % 32 != 0) abort();
    for (int r = 0; r < M; ++r)
        y[r] = gemv_row(contract, W + (size_t)r * K, x, K);
}

/* gdn_gemv_tiny_ab, gdn_model.cpp:1501-1536: plain FP32 products of the
 * operands, per 32-column beat acc = (acc + tree16(lo)) + tree16(hi), beats
 * in order from +0.0f.  The caller applies the BF16 rounding point. */
void orc_gemv_tiny(const float *W, const float *x, int M, int K, float *y) {
    float p[32];
    for (int r = 0; r < M; ++r) {
        float acc = 0.0f;
        for (int b = 0; b < K / 32; ++b) {
            for (int l = 0; l < 32; ++l)
                p[l] = x[32 * b + l] * W[(size_t)r * K + 32 * b + l];
            const float t0 = orc_tree16(p), t1 = orc_tree16(p + 16);
            acc = (acc + t0) + t1;
        }
        y[r] = acc;
    }
}

/* Sum of squares in the norm order: 16-value chunks, each summed
 * sequentially from 0 in lane order, chunk sums added sequentially
 * (gdn_model.cpp:1432-1450, :3413-3431). */
static float chunked_sumsq(const float *x, int n) {
    float sum = 0.0f;
    for (int h = 0; h < n / 16; ++h) {
        float s = 0.0f;
        for (int kk = 0; kk < 16; ++kk) {
            const float v = x[16 * h + kk];
            s += v * v;
        }
        sum += s;
    }
    return sum;
}

/* gdn_rmsnorm_rows_bf16, gdn_model.cpp:1394-1474, one row:
 * scale = 1 / sqrtf(sum / n + eps); out = R((x * scale) * w). */
void orc_rmsnorm(int contract, const float *x, const float *w, int n,
                 float eps, float *out) {
    const float sum = chunked_sumsq(x, n);
    const float scale = 1.0f / sqrtf(sum / (float)n + eps);
    for (int i = 0; i < n; ++i) out[i] = R(contract, x[i] * scale * w[i]);
}

/* gdn_residual_rmsnorm_bf16 + gdn_bf16_add_half, gdn_model.cpp:3351-3450:
 * x' = R(x + y), then the same norm of x'. */
void orc_residual_rmsnorm(int contract, const float *x, const float *y,
                          const float *w, int n, float eps, float *x_out,
                          float *out) {
    for (int i = 0; i < n; ++i) x_out[i] = R(contract, x[i] + y[i]);
    orc_rmsnorm(contract, x_out, w, n, eps, out);
}

/* gdn_output_norm_and_gate, gdn_model.cpp:3226-3349 (production copy
 * gdn_attn_norm_gate :5720-5835): per head, scale = 1/sqrtf(sum/hd + eps),
 * out = R(((a * scale) * w) * g * sigmoid(g)). */
void orc_output_norm_gate(int contract, int tmode, const float *o,
                          const float *g, const float *w, int nh, int hd,
                          float eps, float *out) {
    for (int h = 0; h < nh; ++h) {
        const float *a = o + (size_t)h * hd;
        const float *gh = g + (size_t)h * hd;
        const float sum = chunked_sumsq(a, hd);
        const float scale = 1.0f / sqrtf(sum / (float)hd + eps);
        for (int i = 0; i < hd; ++i) {
            const float normalized = a[i] * scale * w[i];
            const float gv = gh[i];
            out[(size_t)h * hd + i] =
                R(contract, normalized * gv * orc_sigmoid(gv, tmode));
        }
    }
}

/* gdn_depthwise_conv_silu_head_kind, gdn_model.cpp:1543-1667, and the tail
 * update of gemv32_qkvg_consumer (:5043-5130): window [t0, t1, t2, x]
 * (oldest first), s = ((t0*w0 + t1*w1) + t2*w2) + x*w3 without FMA,
 * out = R(silu(s)); the new tail is [t1, t2, x].
 * tails: [3][C], row 0 oldest. conv_w: [C][4]. */
void orc_conv_silu(int contract, int tmode, const float *raw,
                   const float *conv_w, float *tails, int C, float *out) {
    for (int c = 0; c < C; ++c) {
        const float t0 = tails[c], t1 = tails[C + c], t2 = tails[2 * C + c];
        const float x = raw[c];
        const float *w = conv_w + (size_t)c * 4;
        const float s = t0 * w[0] + t1 * w[1] + t2 * w[2] + x * w[3];
        out[c] = R(contract, orc_silu(s, tmode));
        tails[c] = t1;
        tails[C + c] = t2;
        tails[2 * C + c] = x;
    }
}

/* Per-head scalars, gdn_island_prep, gdn_model.cpp:2461-2465:
 * beta = sigmoid(b); decay = expf(-expf(a_log) * softplus(a + dt_bias)). */
void orc_head_scalars(int tmode, float a, float b, float a_log,
                      float dt_bias, float *beta, float *decay) {
    *beta = orc_sigmoid(b, tmode);
    const float decay_in = a + dt_bias;
    const float decay_val =
        -orc_expf(a_log, tmode) * orc_softplus(decay_in, tmode);
    *decay = orc_expf(decay_val, tmode);
}

#define DK 256
#define DV 256

/* The gated delta-rule state pass for one head, gdn_island_prep /
 * gdn_island_read / gdn_island_update / gdn_recurrent_merge_islands
 * (gdn_model.cpp:2376-2933; monolith :1933-2337).
 *   q_inv = 1/sqrtf(tree256(q^2) + 1e-6f), qn = q*q_inv; same for k.
 *   alpha = tree256(qn*kn).
 *   r_i = sum_j S[j][i]*kn_j, p_i = sum_j S[j][i]*qn_j, j = 0..255 in order.
 *   delta_i = beta*(v_i - decay*r_i);  o_i = (1/16)*(decay*p_i + alpha*delta_i)
 *   S'[j][i] = decay*S[j][i] + kn_j*delta_i (BF16-rounded in ORC_REF).
 * This is o = S_t^T q / sqrt(dk) with S_t = decay*S + k (x) delta. */
static void qk_normalize(const float *q, const float *k, float *qn,
                         float *kn, float *alpha) {
    float qs[DK], ks[DK], ap[DK];
    for (int j = 0; j < DK; ++j) {
        qs[j] = q[j] * q[j];
        ks[j] = k[j] * k[j];
    }
    const float q_inv = 1.0f / sqrtf(orc_tree256(qs) + 1e-6f);
    const float k_inv = 1.0f / sqrtf(orc_tree256(ks) + 1e-6f);
    for (int j = 0; j < DK; ++j) {
        qn[j] = q[j] * q_inv;
        kn[j] = k[j] * k_inv;
        ap[j] = qn[j] * kn[j];
    }
    *alpha = orc_tree256(ap);
}

static void state_pass(int contract, const float *qn, const float *kn,
                       float alpha, const float *v, float beta, float decay,
                       float *S, float *o) {
    const float q_scale = 1.0f / sqrtf((float)DK);
    float r[DV], p[DV], delta[DV];
    for (int i = 0; i < DV; ++i) { r[i] = 0.0f; p[i] = 0.0f; }
    for (int j = 0; j < DK; ++j) {
        const float *row = S + (size_t)j * DV;
        for (int i = 0; i < DV; ++i) {
            r[i] = r[i] + row[i] * kn[j];
            p[i] = p[i] + row[i] * qn[j];
        }
    }
    for (int i = 0; i < DV; ++i) {
        delta[i] = beta * (v[i] - decay * r[i]);
        const float out = q_scale * (decay * p[i] + alpha * delta[i]);
        o[i] = R(contract, out);
    }
    for (int j = 0; j < DK; ++j) {
        float *row = S + (size_t)j * DV;
        for (int i = 0; i < DV; ++i) {
            const float decayed = decay * row[i];
            const float written = kn[j] * delta[i];
            const float updated = decayed + written;
            row[i] = contract == ORC_REF ? orc_bf16_round(updated) : updated;
        }
    }
}

void orc_recurrence_head(int contract, int tmode, const float *q,
                         const float *k, const float *v, float a, float b,
                         float a_log, float dt_bias, float *S, float *o) {
    float qn[DK], kn[DK], alpha, beta, decay;
    qk_normalize(q, k, qn, kn, &alpha);
    orc_head_scalars(tmode, a, b, a_log, dt_bias, &beta, &decay);
    state_pass(contract, qn, kn, alpha, v, beta, decay, S, o);
}

/* Same pass with beta and decay given directly (isolated-kernel tests). */
void orc_recurrence_head_scalars(int contract, const float *q, const float *k,
                                 const float *v, float beta, float decay,
                                 float *S, float *o) {
    float qn[DK], kn[DK], alpha;
    qk_normalize(q, k, qn, kn, &alpha);
    state_pass(contract, qn, kn, alpha, v, beta, decay, S, o);
}

/* gemv32_store SwiGLU branch, gdn_model.cpp:4751-4767: h = R(silu(g) * u)
 * on gate/up values that are already at the BF16 rounding point. */
void orc_swiglu(int contract, int tmode, const float *g, const float *u,
                int n, float *h) {
    for (int i = 0; i < n; ++i)
        h[i] = R(contract, orc_silu(g[i], tmode) * u[i]);
}

/* LM-head argmax, gdn_model.cpp:4822-4931: running best from -FLT_MAX at
 * index 0, strict '>' in index order (lowest index wins ties, NaN never
 * wins, a logit equal to -FLT_MAX never replaces the start value). */
int orc_argmax(const float *logits, int n) {
    float best = -3.402823466e38f;
    int idx = 0;
    for (int i = 0; i < n; ++i) {
        if (logits[i] > best) {
            best = logits[i];
            idx = i;
        }
    }
    return idx;
}

/* ---- model level: .gdnw payload order, gdn_assign_weight_views
 *      (gdn_model.cpp:1102-1159) ---- */
static size_t layer_stride(const orc_header *h) {
    const size_t H = h->hidden_size, nh = h->num_heads, hd = h->head_dim;
    const size_t I = h->intermediate_size, cs = h->conv_size;
    return H + 2 * nh + 3 * H * H + 2 * nh * H + 3 * H * cs + H * H + hd +
           H * H + H + 2 * I * H + H * I;
}

size_t orc_layer_offset(const orc_header *h, int layer) {
    return (size_t)h->vocab_size * h->hidden_size +
           (size_t)layer * layer_stride(h);
}

size_t orc_total_weight_floats(const orc_header *h) {
    return orc_layer_offset(h, (int)h->num_layers) + h->hidden_size +
           (size_t)h->vocab_size * h->hidden_size;
}

typedef struct {
    const float *attn_norm, *a_log, *dt_bias, *q, *k, *v, *a_proj, *b_proj;
    const float *q_conv, *k_conv, *v_conv, *g, *o_norm, *o_proj, *mlp_norm;
    const float *gate, *up, *down;
} layer_views;

static layer_views views(const orc_header *h, const float *blob, int layer) {
    const size_t H = h->hidden_size, nh = h->num_heads, hd = h->head_dim;
    const size_t I = h->intermediate_size, cs = h->conv_size;
    const float *p = blob + orc_layer_offset(h, layer);
    layer_views v;
    v.attn_norm = p; p += H;
    v.a_log = p; p += nh;
    v.dt_bias = p; p += nh;
    v.q = p; p += H * H;
    v.k = p; p += H * H;
    v.v = p; p += H * H;
    v.a_proj = p; p += nh * H;
    v.b_proj = p; p += nh * H;
    v.q_conv = p; p += H * cs;
    v.k_conv = p; p += H * cs;
    v.v_conv = p; p += H * cs;
    v.g = p; p += H * H;
    v.o_norm = p; p += hd;
    v.o_proj = p; p += H * H;
    v.mlp_norm = p; p += H;
    v.gate = p; p += I * H;
    v.up = p; p += I * H;
    v.down = p;
    return v;
}

static void round_vec(int contract, float *x, int n) {
    if (contract == ORC_FP32) return;
    for (int i = 0; i < n; ++i) x[i] = orc_bf16_round(x[i]);
}

/* gdn_forward's per-layer sequence, gdn_model.cpp:3741-3843 (the attention
 * norm is evaluated at the layer start; the reference fuses it into the
 * previous layer's residual add, which is the same arithmetic). */
/* gemv_in (optional) receives the layer's four dense-GEMV input vectors in
 * order: the QKVG input [H], the o_proj input [H], the gate/up input [H]
 * and the down input [I] (the native multiplier's activations). */
static void layer_forward_impl(int contract, int tmode, const orc_header *h,
                               const float *blob, int layer, float *x,
                               float *state, float *conv, float *attn_out,
                               float *gemv_in);

void orc_layer_forward(int contract, int tmode, const orc_header *h,
                       const float *blob, int layer, float *x, float *state,
                       float *conv, float *attn_out) {
    layer_forward_impl(contract, tmode, h, blob, layer, x, state, conv, attn_out, NULL);
}

static void layer_forward_impl(int contract, int tmode, const orc_header *h,
                               const float *blob, int layer, float *x,
                               float *state, float *conv, float *attn_out,
                               float *gemv_in) {
    const int H = (int)h->hidden_size, nh = (int)h->num_heads;
    const int hd = (int)h->head_dim, I = (int)h->intermediate_size;
    const float eps = h->norm_eps;
    const layer_views w = views(h, blob, layer);
    float *xn = (float *)malloc(sizeof(float) * (size_t)I);
    float *q = (float *)malloc(sizeof(float) * 4 * (size_t)H);
    float *qc = (float *)malloc(sizeof(float) * 3 * (size_t)H);
    float *o = (float *)malloc(sizeof(float) * (size_t)H);
    float *og = (float *)malloc(sizeof(float) * (size_t)H);
    float *y = (float *)malloc(sizeof(float) * (size_t)H);
    float *xalt = (float *)malloc(sizeof(float) * (size_t)H);
    float *gt = (float *)malloc(sizeof(float) * (size_t)I);
    float *ut = (float *)malloc(sizeof(float) * (size_t)I);
    float *hh = (float *)malloc(sizeof(float) * (size_t)I);
    float a[64], b[64];

    orc_rmsnorm(contract, x, w.attn_norm, H, eps, xn);
    if (gemv_in) memcpy(gemv_in, xn, sizeof(float) * (size_t)H);
    orc_gemv_tiny(w.a_proj, xn, nh, H, a);
    orc_gemv_tiny(w.b_proj, xn, nh, H, b);
    round_vec(contract, a, nh);
    round_vec(contract, b, nh);
    orc_gemv(contract, w.q, xn, H, H, q);
    orc_gemv(contract, w.k, xn, H, H, q + H);
    orc_gemv(contract, w.v, xn, H, H, q + 2 * H);
    orc_gemv(contract, w.g, xn, H, H, q + 3 * H);
    round_vec(contract, q, 4 * H);
    const size_t tail = (size_t)(h->conv_size - 1) * H;
    orc_conv_silu(contract, tmode, q, w.q_conv, conv, H, qc);
    orc_conv_silu(contract, tmode, q + H, w.k_conv, conv + tail, H, qc + H);
    orc_conv_silu(contract, tmode, q + 2 * H, w.v_conv, conv + 2 * tail, H,
                  qc + 2 * H);
#pragma omp parallel for schedule(static)
    for (int hh_ = 0; hh_ < nh; ++hh_) {
        orc_recurrence_head(contract, tmode, qc + (size_t)hh_ * hd,
                            qc + H + (size_t)hh_ * hd,
                            qc + 2 * H + (size_t)hh_ * hd, a[hh_], b[hh_],
                            w.a_log[hh_], w.dt_bias[hh_],
                            state + (size_t)hh_ * hd * hd,
                            o + (size_t)hh_ * hd);
    }
    if (attn_out) memcpy(attn_out, o, sizeof(float) * (size_t)H);
    orc_output_norm_gate(contract, tmode, o, q + 3 * H, w.o_norm, nh, hd, eps,
                         og);
    if (gemv_in) memcpy(gemv_in + H, og, sizeof(float) * (size_t)H);
    orc_gemv(contract, w.o_proj, og, H, H, y);
    round_vec(contract, y, H);
    orc_residual_rmsnorm(contract, x, y, w.mlp_norm, H, eps, xalt, xn);
    if (gemv_in) memcpy(gemv_in + 2 * H, xn, sizeof(float) * (size_t)H);
    orc_gemv(contract, w.gate, xn, I, H, gt);
    orc_gemv(contract, w.up, xn, I, H, ut);
    round_vec(contract, gt, I);
    round_vec(contract, ut, I);
    orc_swiglu(contract, tmode, gt, ut, I, hh);
    if (gemv_in) memcpy(gemv_in + 3 * H, hh, sizeof(float) * (size_t)I);
    orc_gemv(contract, w.down, hh, H, I, y);
    round_vec(contract, y, H);
    for (int i = 0; i < H; ++i) x[i] = R(contract, xalt[i] + y[i]);

    free(xn); free(q); free(qc); free(o); free(og); free(y); free(xalt);
    free(gt); free(ut); free(hh);
}

/* gdn_decode_step_host + gdn_forward, gdn_model.cpp:3716-3734, :3857-3900:
 * the FP32 embedding row is rounded to the contract, run through the
 * layers, normalised with final_norm and multiplied by lm_head into FP32
 * logits (not rounded); the argmax is the returned token. */
static int decode_step_impl(int contract, int tmode, const orc_header *h,
                            const float *blob, float *state, float *conv,
                            int token, float *logits, float *final_hidden,
                            float *gemv_in);

int orc_decode_step(int contract, int tmode, const orc_header *h,
                    const float *blob, float *state, float *conv, int token,
                    float *logits, float *final_hidden) {
    return decode_step_impl(contract, tmode, h, blob, state, conv, token, logits, final_hidden, NULL);
}

/* As orc_decode_step, also writing every dense GEMV's input vector of the
 * step to gemv_in: per layer [H] QKVG, [H] o_proj, [H] gate/up, [I] down,
 * then the LM head's [H] (the final hidden vector). */
int orc_decode_step_trace(int contract, int tmode, const orc_header *h,
                          const float *blob, float *state, float *conv,
                          int token, float *logits, float *final_hidden,
                          float *gemv_in) {
    return decode_step_impl(contract, tmode, h, blob, state, conv, token, logits, final_hidden, gemv_in);
}

static int decode_step_impl(int contract, int tmode, const orc_header *h,
                            const float *blob, float *state, float *conv,
                            int token, float *logits, float *final_hidden,
                            float *gemv_in) {
    const int H = (int)h->hidden_size, L = (int)h->num_layers;
    const size_t layer_state = (size_t)h->num_heads * h->head_dim * h->head_dim;
    const size_t layer_conv = (size_t)3 * (h->conv_size - 1) * H;
    if (token < 0 || (uint32_t)token >= h->vocab_size) return -1;
    float *x = (float *)malloc(sizeof(float) * (size_t)H);
    float *xn = (float *)malloc(sizeof(float) * (size_t)H);
    const float *emb = blob + (size_t)token * H;
    for (int i = 0; i < H; ++i) x[i] = R(contract, emb[i]);
    const size_t per_layer_in = 3 * (size_t)H + h->intermediate_size;
    for (int l = 0; l < L; ++l)
        layer_forward_impl(contract, tmode, h, blob, l, x,
                           state + (size_t)l * layer_state,
                           conv + (size_t)l * layer_conv, NULL,
                           gemv_in ? gemv_in + (size_t)l * per_layer_in : NULL);
    const float *final_norm = blob + orc_layer_offset(h, L);
    const float *lm_head = final_norm + H;
    orc_rmsnorm(contract, x, final_norm, H, h->norm_eps, xn);
    if (final_hidden) memcpy(final_hidden, xn, sizeof(float) * (size_t)H);
    if (gemv_in) memcpy(gemv_in + (size_t)L * per_layer_in, xn, sizeof(float) * (size_t)H);
    orc_gemv(contract, lm_head, xn, (int)h->vocab_size, H, logits);
    free(x);
    free(xn);
    return orc_argmax(logits, (int)h->vocab_size);
}

/* gdn_compute_logits, gdn_model.cpp:3930-3965: the reference's independent
 * scalar LM head -- the same per-product rounding, sequential sum. */
void orc_compute_logits(const orc_header *h, const float *blob,
                        const float *hidden, float *logits) {
    const int H = (int)h->hidden_size;
    const float *lm_head =
        blob + orc_layer_offset(h, (int)h->num_layers) + H;
    float *rounded = (float *)malloc(sizeof(float) * (size_t)H);
    for (int i = 0; i < H; ++i) rounded[i] = orc_bf16_round(hidden[i]);
#pragma omp parallel for schedule(static)
    for (int v = 0; v < (int)h->vocab_size; ++v) {
        logits[v] = seq_native_row(lm_head + (size_t)v * H, rounded, H);
    }
    free(rounded);
}

/* ---- array helpers for the tests (same functions, many inputs) ---- */
void orc_rne_array(const uint32_t *in, uint16_t *out, size_t n) {
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i) out[i] = orc_rne_bits(in[i]);
}

void orc_native_product_array(const uint16_t *w, const uint16_t *x, uint16_t *out, size_t n) {
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i)
        out[i] = orc_native_product_bits(w[i], x[i]);
}

/* The select form used by the GEMV rows, for the test that compares it with
 * orc_native_product_bits. */
void orc_native_product_sel_array(const uint16_t *w, const uint16_t *x, uint16_t *out, size_t n) {
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i)
        out[i] = (uint16_t)(native_bits_sel((uint32_t)w[i] << 16, (uint32_t)x[i] << 16) >> 16);
}

void orc_transcendental_array(int which, int tmode, const float *in, float *out, size_t n) {
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)n; ++i) {
        const float x = in[i];
        switch (which) {
        case 0: out[i] = orc_expf(x, tmode); break;
        case 1: out[i] = orc_log1pf(x, tmode); break;
        case 2: out[i] = orc_sigmoid(x, tmode); break;
        case 3: out[i] = orc_silu(x, tmode); break;
        default: out[i] = orc_softplus(x, tmode); break;
        }
    }
}
