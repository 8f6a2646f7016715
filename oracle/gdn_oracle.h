/*
 * gdn_oracle.h -- CPU restatement of the reference decode arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (gateddeltanet_amd/,
 * include/) may include, link or call this library.  Only tests/, the
 * smoke() check in __graft_entry__.py and the cpu_baseline leg of bench.py
 * use it, and only as the checker.
 *
 * Every function restates one piece of c_impl/gdn_model.cpp of the reference
 * (YAMWD/GatedDeltaNet); the citation is on the definition in gdn_oracle.c.
 *
 * Contracts (one switch for the whole library call):
 *   ORC_REF          gdn_model.cpp exactly: BF16 weights, native BF16-product
 *                    GEMVs, BF16 operator boundaries, BF16 recurrent state.
 *   ORC_BF16W_FP32S  as ORC_REF except the recurrent state stays FP32
 *                    between tokens (the north-star bf16 arm).
 *   ORC_FP32         control arm: FP32 weights/activations/state, plain FP32
 *                    products, no rounding point anywhere, same reduction
 *                    orders.
 *   ORC_BF16X        as ORC_BF16W_FP32S except the dense GEMV products are
 *                    exact FP32 products of the BF16 operands (no product
 *                    rounding): the arithmetic of the multi-stream engine's
 *                    matrix-core projections up to summation order.  Not a
 *                    reference contract.
 *
 * Transcendental modes:
 *   ORC_LIBM  glibc expf/log1pf, as the reference calls them.
 *   ORC_CR    correctly rounded float results computed through double
 *             (float)exp((double)x) and (float)log1p((double)x); this is
 *             the evaluation the HIP kernels use.  Both modes agree except
 *             where glibc's float routines are not correctly rounded.
 *
 * Parity pins (which test checks what) are listed in the header comment
 * of gdn_oracle.c.
 */
#ifndef GDN_ORACLE_H
#define GDN_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_REF = 0, ORC_BF16W_FP32S = 1, ORC_FP32 = 2, ORC_BF16X = 3 };
enum { ORC_LIBM = 0, ORC_CR = 1 };

/* Same 60-byte layout as the reference GDNWeightHeader. */
typedef struct {
    char magic[8];
    uint32_t version;
    uint32_t vocab_size;
    uint32_t hidden_size;
    uint32_t num_layers;
    uint32_t num_heads;
    uint32_t num_v_heads;
    uint32_t head_dim;
    uint32_t intermediate_size;
    uint32_t conv_size;
    uint32_t max_seq_len;
    int32_t bos_token_id;
    int32_t eos_token_id;
    float norm_eps;
} orc_header;

/* ---- scalar helpers ---- */
uint16_t orc_rne_bits(uint32_t fp32_bits);
uint32_t orc_widen_bits(uint16_t bf16_bits);
float orc_bf16_round(float x);          /* RNE to BF16, widened back */
uint16_t orc_native_product_bits(uint16_t w, uint16_t x);
float orc_expf(float x, int tmode);
float orc_log1pf(float x, int tmode);
float orc_sigmoid(float x, int tmode);
float orc_silu(float x, int tmode);
float orc_softplus(float x, int tmode);
float orc_tree16(const float *p);
float orc_tree256(const float *a);

/* ---- operators (arrays are FP32 words; BF16 values are carried
 *      BF16-exact in FP32 slots, as the reference does) ---- */
void orc_gemv(int contract, const float *W, const float *x, int M, int K,
              float *y);
void orc_gemv_rows(int contract, const float *W, const float *x, int M, int K,
                   float *y);     /* single-threaded row loop, same values */
void orc_gemv_tiny(const float *W, const float *x, int M, int K, float *y);
void orc_rmsnorm(int contract, const float *x, const float *w, int n,
                 float eps, float *out);
void orc_residual_rmsnorm(int contract, const float *x, const float *y,
                          const float *w, int n, float eps, float *x_out,
                          float *out);
void orc_output_norm_gate(int contract, int tmode, const float *o,
                          const float *g, const float *w, int nh, int hd,
                          float eps, float *out);
void orc_conv_silu(int contract, int tmode, const float *raw,
                   const float *conv_w, float *tails, int C, float *out);
void orc_head_scalars(int tmode, float a, float b, float a_log,
                      float dt_bias, float *beta, float *decay);
void orc_recurrence_head(int contract, int tmode, const float *q,
                         const float *k, const float *v, float a, float b,
                         float a_log, float dt_bias, float *S, float *o);
void orc_recurrence_head_scalars(int contract, const float *q, const float *k,
                                 const float *v, float beta, float decay,
                                 float *S, float *o);
void orc_swiglu(int contract, int tmode, const float *g, const float *u,
                int n, float *h);
int orc_argmax(const float *logits, int n);

/* ---- model level ---- */
size_t orc_total_weight_floats(const orc_header *h);
size_t orc_layer_offset(const orc_header *h, int layer);

/* One GatedDeltaNet layer on the residual stream x (in/out, H floats).
 * state: this layer's [nh][dk][dv] FP32 recurrent state (in/out).
 * conv:  this layer's [3][W-1][H] conv tails, oldest row first (in/out).
 * attn_out (optional, H floats): the recurrence output o for the layer. */
void orc_layer_forward(int contract, int tmode, const orc_header *h,
                       const float *blob, int layer, float *x, float *state,
                       float *conv, float *attn_out);

/* One decode step of the full model: token in, logits out, argmax returned.
 * state: [L][nh][dk][dv]; conv: [L][3][W-1][H].  final_hidden optional. */
int orc_decode_step(int contract, int tmode, const orc_header *h,
                    const float *blob, float *state, float *conv, int token,
                    float *logits, float *final_hidden);
int orc_decode_step_trace(int contract, int tmode, const orc_header *h,
                          const float *blob, float *state, float *conv,
                          int token, float *logits, float *final_hidden,
                          float *gemv_in);

/* Reference-style independent scalar LM head (gdn_compute_logits). */
void orc_compute_logits(const orc_header *h, const float *blob,
                        const float *hidden, float *logits);

void orc_set_threads(int n);

/* Array forms of the scalar helpers, for exhaustive tests. which: 0 expf,
 * 1 log1pf, 2 sigmoid, 3 silu, 4 softplus. */
void orc_rne_array(const uint32_t *in, uint16_t *out, size_t n);
void orc_native_product_array(const uint16_t *w, const uint16_t *x, uint16_t *out, size_t n);
void orc_native_product_sel_array(const uint16_t *w, const uint16_t *x, uint16_t *out, size_t n);
void orc_transcendental_array(int which, int tmode, const float *in, float *out, size_t n);

#ifdef __cplusplus
}
#endif
#endif
