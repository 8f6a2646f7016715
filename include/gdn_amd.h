/*
 * gdn_amd.h -- C ABI of the MI355X batch-1 GatedDeltaNet-1.3B decode engine
 * (libgdn_amd.so).
 *
 * The declarations mirror the reference's c_impl/gdn_model.h (YAMWD/
 * GatedDeltaNet) so that a caller written against gdn_model.cpp -- its own
 * gdn_eval.cpp, or host.cpp's runner -- links against this library instead.
 * Each entry point cites the reference interface it replaces.  Plain C types
 * and pointers only; no HIP or torch type appears here.
 *
 * Errors: every int-returning entry point returns 0 on success and -1 on
 * failure after printing one line to stderr, as the reference's
 * gdn_print_error does (gdn_model.cpp:487-493).  Nothing throws across this
 * boundary.  Not reentrant per run state, like the reference.
 */
#ifndef GDN_AMD_H
#define GDN_AMD_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- .gdnw header: byte-identical to GDNWeightHeader, gdn_model.h:30-45
 *      (60 bytes, little-endian; written by export_gdn_c.py:27-30). ---- */
typedef struct {
    char magic[8];              /* "GDNWv1\0\0" */
    uint32_t version;           /* 1 */
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
} GDNWeightHeader;

/* ---- workspace layout in FLOATS: identical values to gdn_model.h:54-75.
 *      GDNRunState.workspace is a host buffer of this layout. ---- */
#define GDN_WSF_HID     2048u
#define GDN_WSF_HEAD    16u
#define GDN_WSF_MLP     5632u
#define GDN_WSF_STATE   12582912u
#define GDN_WSF_HEADBUF 442368u
#define GDN_WSF_LOGITS  32000u
#define GDN_WS_OFF_X          ((size_t)0)
#define GDN_WS_OFF_X_NORM     (GDN_WS_OFF_X         + GDN_WSF_HID)
#define GDN_WS_OFF_Q          (GDN_WS_OFF_X_NORM    + GDN_WSF_HID)
#define GDN_WS_OFF_K          (GDN_WS_OFF_Q         + GDN_WSF_HID)
#define GDN_WS_OFF_V          (GDN_WS_OFF_K         + GDN_WSF_HID)
#define GDN_WS_OFF_A          (GDN_WS_OFF_V         + GDN_WSF_HID)
#define GDN_WS_OFF_B          (GDN_WS_OFF_A         + GDN_WSF_HEAD)
#define GDN_WS_OFF_GATE       (GDN_WS_OFF_B         + GDN_WSF_HEAD)
#define GDN_WS_OFF_ATTN       (GDN_WS_OFF_GATE      + GDN_WSF_HID)
#define GDN_WS_OFF_TMP_HIDDEN (GDN_WS_OFF_ATTN      + GDN_WSF_HID)
#define GDN_WS_OFF_MLP_GATE   (GDN_WS_OFF_TMP_HIDDEN + GDN_WSF_HID)
#define GDN_WS_OFF_MLP_UP     (GDN_WS_OFF_MLP_GATE  + GDN_WSF_MLP)
#define GDN_WS_OFF_REC_STATE  (GDN_WS_OFF_MLP_UP    + GDN_WSF_MLP)
#define GDN_WS_OFF_HEAD_BUF   (GDN_WS_OFF_REC_STATE + GDN_WSF_STATE)
#define GDN_WS_OFF_LOGITS     (GDN_WS_OFF_HEAD_BUF  + GDN_WSF_HEADBUF)
#define GDN_WS_FLOATS         (GDN_WS_OFF_LOGITS    + GDN_WSF_LOGITS)

/* ---- arithmetic contracts (the reference implements GDN_CONTRACT_REF) ----
 * GDN_CONTRACT_REF          gdn_model.cpp: BF16 weights, native BF16-product
 *                           GEMVs, BF16 operator boundaries, BF16 state.
 * GDN_CONTRACT_BF16W_FP32S  as REF but the recurrent state stays FP32.
 * GDN_CONTRACT_FP32         FP32 weights/activations/state, FP32 products,
 *                           no rounding points; same reduction orders. */
#define GDN_CONTRACT_REF          0
#define GDN_CONTRACT_BF16W_FP32S  1
#define GDN_CONTRACT_FP32         2

/* Host-side weight views into the .gdnw payload (gdn_model.h:123-142). */
typedef struct {
    const float *attn_norm;
    const float *a_log;
    const float *dt_bias;
    const float *q_proj;
    const float *k_proj;
    const float *v_proj;
    const float *a_proj;
    const float *b_proj;
    const float *q_conv;
    const float *k_conv;
    const float *v_conv;
    const float *g_proj;
    const float *o_norm;
    const float *o_proj;
    const float *mlp_norm;
    const float *mlp_gate_proj;
    const float *mlp_up_proj;
    const float *mlp_down_proj;
} GDNLayerWeights;

/* Host model: gdn_model.h:144-151, unchanged. */
typedef struct {
    GDNWeightHeader config;
    float *weight_data;
    GDNLayerWeights *layers;
    const float *embeddings;
    const float *final_norm;
    const float *lm_head;
} GDNModel;

/* ---- device-format geometry the reference's drivers compute with
 *      (gdn_model.h:22, :84-90, :115-121).  The values are the reference's;
 *      on this engine the 32 weight shards hold no weights (see
 *      gdn_weight_shard_beats) and shards 28..31 are host mirrors of the
 *      BF16 recurrent-state stripes. ---- */
#define GEMV_CHANNELS 32
#define GDN_RECURRENT_STATE_PORTS       4
#define GDN_RECURRENT_STATE_FIRST_PORT 28
#define GDN_RECURRENT_STATE_STRIPE_FLOATS (GDN_WSF_STATE / GDN_RECURRENT_STATE_PORTS)
#define GDN_RECURRENT_STATE_STRIPE_BF16_BEATS (GDN_RECURRENT_STATE_STRIPE_FLOATS / 32u)
#define GDN_CONV_TAIL_STRIPES (24u * 3u)
#define GDN_CONV_TAIL_FLOATS_PER_STRIPE (GDN_WSF_HEADBUF / GDN_CONV_TAIL_STRIPES)
#define GDN_CONV_TAIL_RESERVED_BEATS_PER_STRIPE (GDN_CONV_TAIL_FLOATS_PER_STRIPE / 16u)
#define GDN_CONV_TAIL_BF16_BEATS_PER_STRIPE (GDN_CONV_TAIL_FLOATS_PER_STRIPE / 32u)

/* One 512-bit beat, the reference's Beat512 (ap_uint<512>, gdn_model.h:10-14):
 * 64 bytes, FP32 lane i at bytes 4i..4i+3, BF16 lane i at bytes 2i..2i+1,
 * little-endian. */
typedef struct GDNBeat512 {
    unsigned char bytes[64];
} Beat512;

struct GDNEngine;

/* Run state: the reference's GDNRunState (gdn_model.h:153-160) field for
 * field, with the device engine appended.  Every reference field is HOST
 * memory, so a caller written against gdn_model.cpp reads and writes it as
 * before:
 *   workspace        GDN_WS_FLOATS floats, 64-byte aligned.  After each
 *                    gdn_decode_step_host: X holds the token's FP32
 *                    embedding row and lane 0 of X_NORM the argmax token as
 *                    a float (the reference's token line).  The other slots
 *                    are not refreshed per step (the debug buffers and
 *                    gdn_read_* return device results).
 *   x, recurrent_state, head_buffer   views at GDN_WS_OFF_X / _REC_STATE /
 *                    _HEAD_BUF (the .gdnstate loader reads into
 *                    recurrent_state, as gdn_eval.cpp does)
 *   weight_shards    [0..27] NULL; [28..31] host buffers of
 *                    GDN_RECURRENT_STATE_STRIPE_BF16_BEATS beats holding the
 *                    recurrent state in the reference's BF16 stripe layout,
 *                    written by gdn_scatter_recurrent_state and refreshed
 *                    from the device by gdn_sync_host_state
 *   aux_weights      NULL (the small weights live on the device)
 *   engine           device weights, state, activations, stream and graph */
typedef struct {
    Beat512 *workspace;
    float *x;
    float *recurrent_state;
    float *head_buffer;
    Beat512 *weight_shards[GEMV_CHANNELS];
    Beat512 *aux_weights;
    struct GDNEngine *engine;
} GDNRunState;

/* Product counters of the native BF16 multiplier (gdn_model.h:162-168). */
typedef struct {
    uint64_t calls;
    uint64_t special_inputs;
    uint64_t flushed_inputs;
    uint64_t flushed_outputs;
    uint64_t overflows;
} GDNMixedMulStats;

/* ===== model (host) ===== */

/* gdn_model.h:213 -- read a .gdnw file: 60-byte header, FP32 payload in
 * gdn_assign_weight_views order; rejects bad magic/version,
 * num_heads != num_v_heads, hidden != heads*head_dim and (unless the file
 * is loaded for the FP32 contract) non-BF16-exact values. */
int gdn_model_load(GDNModel *model, const char *path);
/* gdn_model.h:214 */
void gdn_model_free(GDNModel *model);
/* Like gdn_model_load but keeps non-BF16-exact payloads (FP32 contract).
 * No reference counterpart: the reference rejects such files. */
int gdn_model_load_fp32(GDNModel *model, const char *path);
/* Write a .gdnw (export_gdn_c.py:169-210 byte layout). */
int gdn_model_save(const GDNModel *model, const char *path);
/* Seeded synthetic model in .gdnw order: every tensor N(0, std) from
 * gdn_synth_normal with stream = its .gdnw ordinal, norm weights = 1;
 * BF16-rounded when bf16 != 0.  Replaces loading a checkpoint. */
int gdn_model_synth(GDNModel *model, const GDNWeightHeader *config,
                    uint64_t seed, float std, int bf16);
/* gdn_model.h:174-175 */
int gdn_validate_bf16_exact_weights(const float *weight_data,
                                    const GDNWeightHeader *config);
size_t gdn_total_weight_floats(const GDNWeightHeader *config);
/* The GDN-1.3B header (vocab 32000, hidden 2048, 24 layers, 8x256 heads,
 * intermediate 5632, conv 4, max_seq_len 2048, eps 1e-6f). */
void gdn_default_config(GDNWeightHeader *config, uint32_t num_layers);

/* ===== run state (device) ===== */

/* gdn_model.h:216 -- allocate the host workspace and state mirrors, upload
 * the weights to the device in the engine's layout and zero the
 * recurrent/conv state, for the REF contract.  Fails on max_tokens == 0 or
 * > max_seq_len, and on a model shape the kernels are not built for
 * (hidden 2048, 8 x 256 heads, intermediate 5632, conv 4, 1..24 layers,
 * vocab a positive multiple of 8). */
int gdn_run_state_init(GDNRunState *state, const GDNModel *model,
                       uint32_t max_tokens);
/* Same with an explicit contract (GDN_CONTRACT_*). */
int gdn_run_state_init_contract(GDNRunState *state, const GDNModel *model,
                                uint32_t max_tokens, int contract);
/* gdn_model.h:217 */
void gdn_run_state_free(GDNRunState *state);

/* gdn_model.h:264 -- one teacher-forced decode step: the embedding row of
 * *token (host workspace X gets its FP32 copy), every layer against the
 * persistent device state, the LM head and the argmax, which lands as a
 * float in lane 0 of the host workspace's X_NORM.  Returns -1 for a token
 * outside [0, vocab), for a run state that was never initialised, and when
 * the step does not finish within GDN_KERNEL_WAIT_TIMEOUT_MS milliseconds
 * (environment; default 10000) or a kernel's bounded internal wait ran out
 * (the run state then refuses further steps). */
int gdn_decode_step_host(const GDNModel *model, GDNRunState *state,
                         const int32_t *token);
/* ---- the remaining gdn_model.h calls of the reference's gdn_eval.cpp ---- */

/* gdn_model.h:172-173: beats per packed weight shard.  This engine keeps its
 * weights on the device in its own layout, so the shards hold no weight
 * beats: 0 (and 0 bytes), which makes a caller's
 * weight_shards[GDN_RECURRENT_STATE_FIRST_PORT + p] + gdn_weight_shard_beats()
 * the state stripe itself. */
size_t gdn_weight_shard_beats(const GDNWeightHeader *config);
size_t gdn_weight_shard_bytes(const GDNWeightHeader *config);
/* gdn_model.h:176-178: checks the device copy of every weight against the
 * FP32-word blob, value for value in the engine's packing (download and
 * compare; about 3 GB of reads).  `shards` identifies the run state (its
 * weight_shards array).  0 when every value matches. */
int gdn_validate_weight_shards(const float *weight_data, const GDNWeightHeader *config,
                               Beat512 *const shards[]);
/* gdn_model.h:190-192: the recurrent state [L][H][K][V] (FP32 words)
 * written into `state_stripes` in the reference's BF16 stripe layout.  When
 * the stripes are a run state's (weight_shards + GDN_RECURRENT_STATE_FIRST_PORT)
 * the values also go to its engine: under the REF contract they must be
 * BF16-exact, as in the reference, while the FP32-state contracts keep the
 * FP32 values on the device and mirror their BF16 rounding in the stripes.
 * Other stripes are only packed, from BF16-exact values. */
int gdn_scatter_recurrent_state(Beat512 *const state_stripes[], const float *recurrent_state,
                                size_t recurrent_state_floats);
/* gdn_model.h:193-195: the conv tails [L][q,k,v][W-1][hidden] written into
 * `workspace_head_buffer` as BF16 payloads in the first half of each stripe
 * reservation, the rest zeroed.  When it is a run state's head_buffer the
 * values also go to its engine (BF16-exact except under the FP32 contract);
 * any other buffer is only packed, from GDN_WSF_HEADBUF BF16-exact values. */
int gdn_pack_conv_tails_bf16(Beat512 *workspace_head_buffer, const float *conv_tails,
                             size_t conv_tail_floats);
/* gdn_model.h:274: after every gdn_decode_step_host the final normalised
 * hidden vector (hidden_size floats) and the FP32 logits (vocab_size floats)
 * are copied into these caller buffers; NULL stops the copies.  Process-wide,
 * like the reference. */
void gdn_set_native_debug_buffers(float *final_hidden, float *logits);
/* gdn_model.h:203-204: counters of the native BF16 products, process-wide.
 * Host products (gdn_compute_logits, gdn_native_bf16_mul_to_fp32) are
 * counted as they run.  Device products are counted per decode step while
 * counting is on: calls exactly; special and flushed inputs exactly, from
 * each GEMV's input vector and per-column tables of the weights; flushed
 * outputs and overflows exactly, and only where the kernel's fast-path
 * verdict does not already exclude them.  gdn_reset_mixed_mul_stats zeroes
 * the counters and turns device counting on (each counted step also copies
 * the step's GEMV inputs to the host); gdn_get_mixed_mul_stats reads them. */
void gdn_reset_mixed_mul_stats(void);
GDNMixedMulStats gdn_get_mixed_mul_stats(void);
/* Turns device counting off again (no reference counterpart). */
void gdn_stop_mixed_mul_stats(void);
/* Refresh the host mirrors of the run state from the device: the BF16 state
 * stripes in weight_shards[28..31] and the packed conv tails in head_buffer,
 * in the layouts gdn_scatter_recurrent_state / gdn_pack_conv_tails_bf16
 * write.  Call before reading them (e.g. a GDNSDMP1 state dump).  No
 * reference counterpart: the reference's stripes are the device memory. */
int gdn_sync_host_state(GDNRunState *state);
/* gdn_model.h:207-210: lane accessors of a Beat512. */
void gdn_test_set_fp32_lane_bits(Beat512 *beat, uint32_t lane, uint32_t bits);
uint32_t gdn_test_get_fp32_lane_bits(const Beat512 *beat, uint32_t lane);
void gdn_test_set_bf16_lane_bits(Beat512 *beat, uint32_t lane, uint16_t bits);
uint16_t gdn_test_get_bf16_lane_bits(const Beat512 *beat, uint32_t lane);

/* Device results of the last step, copied to host memory. */
int gdn_read_token(const GDNRunState *state, int32_t *token);
int gdn_read_logits(const GDNRunState *state, float *logits, size_t count);
int gdn_read_final_hidden(const GDNRunState *state, float *hidden,
                          size_t count);

/* Recurrent/conv state in the .gdnstate section layouts
 * (gdn_eval.cpp:202-257): recurrent [L][H][K][V] FP32, conv tails
 * [L][q,k,v][W-1 oldest..newest][hidden] FP32.  Loading replaces
 * gdn_scatter_recurrent_state / gdn_pack_conv_tails_bf16 (gdn_model.h:
 * 190-195); for the REF contract values must be BF16-exact. */
int gdn_load_recurrent_state(GDNRunState *state, const float *recurrent,
                             size_t floats);
int gdn_load_conv_tails(GDNRunState *state, const float *conv_tails,
                        size_t floats);
int gdn_save_recurrent_state(const GDNRunState *state, float *recurrent,
                             size_t floats);
int gdn_save_conv_tails(const GDNRunState *state, float *conv_tails,
                        size_t floats);
/* load_gdnstate, gdn_eval.cpp:202-267: read a .gdnstate file into the run
 * state; returns the header fields via the optional out pointers. */
int gdn_load_gdnstate(GDNRunState *state, const GDNModel *model,
                      const char *path, uint32_t *prompt_len,
                      int32_t *seed_token);
/* Write the current state as a .gdnstate file (export_gdn_state.py:
 * 340-362 layout). */
int gdn_save_gdnstate(const GDNRunState *state, const GDNModel *model,
                      const char *path, const int32_t *prompt,
                      uint32_t prompt_len, int32_t seed_token);

/* Write a .gdnstate from host arrays in the section layouts above (the
 * writer of gdn_save_gdnstate; used to export a prefilled stream). */
int gdn_write_gdnstate(const GDNWeightHeader *config, const char *path, const float *recurrent,
                       const float *conv_tails, const int32_t *prompt, uint32_t prompt_len,
                       int32_t seed_token);

/* Steady teacher-forced benchmark, host.cpp:2150-2256: tokens[i % n_tokens]
 * is fed at step i for n_steps steps.  Per step: outer = host token in ->
 * host token out (the token is read and the argmax written through mapped
 * pinned memory around one graph launch); inner = HIP events around the
 * graph on the engine stream, recorded only when inner_ms is given.  Any
 * output pointer may be NULL. */
int gdn_run_teacher_forced(GDNRunState *state, const int32_t *tokens,
                           uint32_t n_tokens, uint32_t n_steps,
                           int32_t *argmax_out, float *inner_ms,
                           float *outer_ms);
/* Average device time (microseconds) per launch of each kernel kind, in
 * the order qkvg, recur, o_proj, gate_up, down, lm_head, argmax; each kind
 * is launched back to back over every layer's weights (HIP events on the
 * engine stream).  Advances the recurrent and conv state.  No reference
 * counterpart: the reference times its FPGA calls with compile-time cycle
 * probes (GDN_CALL_PROBE, gdn_model.h:91-107). */
int gdn_profile_kernels(GDNRunState *state, uint32_t rounds, float *avg_us,
                        uint32_t n_kinds);
/* 0: launch kernels one by one; 1 (default): one captured hipGraph/step. */
int gdn_set_graph_mode(GDNRunState *state, int use_graph);
/* The persistent step: one cooperative launch of 256 one-per-CU workgroups
 * runs the whole token (every layer, the LM head and the argmax), stages
 * handing their outputs over as tagged words in uncached memory read through
 * the scalar path.  Opt-in: a run state has it when the environment sets
 * GDN_PERSIST=1 at gdn_run_state_init, its contract is GDN_CONTRACT_REF or
 * GDN_CONTRACT_BF16W_FP32S, the vocabulary is 32000 (256 x 125 LM-head rows)
 * and the device holds the grid; its steps then replace the captured graph
 * (results are bit-identical; it measured slower than the graph, which is
 * why it is not the default).  gdn_set_persistent(state, 0) switches back to
 * the graph (1 switches again); it returns -1 when the run state has no
 * persistent step.  gdn_get_persistent: 1 if steps run persistent, 0 if not,
 * -1 on a bad run state.  No reference counterpart. */
int gdn_set_persistent(GDNRunState *state, int on);
int gdn_get_persistent(const GDNRunState *state);
int gdn_get_contract(const GDNRunState *state);

/* ===== reference host helpers ===== */

/* gdn_model.h:267 -- the independent scalar LM head (host, CPU). */
void gdn_compute_logits(const GDNModel *model, const float *hidden,
                        float *logits_out);
/* gdn_model.h:200 -- native BF16 product (host model of the contract). */
float gdn_native_bf16_mul_to_fp32(uint16_t weight, uint16_t activation);
/* gdn_model.h:205-206 */
uint16_t gdn_test_fp32_to_bf16_rne_bits(uint32_t bits);
uint32_t gdn_test_bf16_to_fp32_bits(uint16_t bits);

/* ===== seeded synthetic inputs ===== */

/* Counter-based N(mean, std) draws: element i of (seed, stream) is the
 * Box-Muller pair (2*(i/2), +1) of SplitMix64 outputs; deterministic for
 * any thread count.  round_bf16 RNE-rounds every value to BF16. */
void gdn_synth_normal(float *out, size_t n, uint64_t seed, uint64_t stream,
                      float mean, float std, int round_bf16);
/* U[lo, hi) draws on the same counter scheme. */
void gdn_synth_uniform(float *out, size_t n, uint64_t seed, uint64_t stream,
                       float lo, float hi);
/* Uniform token ids in [0, vocab). */
void gdn_synth_tokens(int32_t *out, size_t n, uint64_t seed, uint64_t stream,
                      uint32_t vocab);

/* ===== isolated kernels on host buffers (test hooks, like the reference's
 *       gdn_test_* family; each copies in, runs the engine's kernel, copies
 *       out) ===== */

/* Dense GEMV row results before any rounding point: y[M] (FP32) of W[M][K]
 * and x[K] under the contract's product rule.  K in {2048, 5632}. */
int gdn_test_gemv(int contract, const float *W, const float *x, uint32_t M,
                  uint32_t K, float *y);
/* n_steps of the gated delta-rule kernel on n_heads independent heads.
 * q,k,v [steps][heads][256] (pre-L2-norm conv outputs), a,b,a_log,dt_bias
 * [steps][heads]; S [heads][256][256] FP32 words in/out (BF16-exact for
 * REF); o [steps][heads][256]. */
int gdn_test_recurrence(int contract, uint32_t n_heads, uint32_t n_steps,
                        const float *q, const float *k, const float *v,
                        const float *a, const float *b, const float *a_log,
                        const float *dt_bias, float *S, float *o);
/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid it): the
 * steps of gdn_test_recurrence on caller-owned DEVICE buffers, allocating
 * nothing.  Arguments and layouts as gdn_test_recurrence, all device
 * pointers, except S, which is in the engine's device format: [heads][256][256]
 * BF16 bits (uint16) for GDN_CONTRACT_REF, FP32 otherwise.  The per-step
 * (beta, decay) pairs live in a fixed 128 KiB device array of 16384 pairs that
 * every call on a GPU shares (steps run in chunks that fit it); n_heads above
 * 16384 is rejected.  Work is enqueued on `stream` (a hipStream_t; NULL = the
 * null stream) and not waited for.  Calls that overlap on one GPU race on the
 * shared array. */
int gdn_recurrence_noalloc(int contract, uint32_t n_heads, uint32_t n_steps, const float *q,
                           const float *k, const float *v, const float *a, const float *b,
                           const float *a_log, const float *dt_bias, void *S, float *o, void *stream);
/* The engine's expf (which = 0) or log1pf (which = 1) evaluated on the host
 * over n inputs: the same code the kernels run, a restatement of the methods
 * of the reference's C library (glibc 2.35) that equals it on every input. */
void gdn_test_libm_array(int which, const float *in, float *out, size_t n);
/* Test hook: copies the last step's device buffers to `out` (at most
 * `bytes`): which = 0, the persistent step's exchange area (32-bit words
 * (tag << 16) | payload); which = 1, the per-kernel step's activation
 * buffers (FP32; layout in gateddeltanet_amd/engine.py); which = 2, the
 * persistent step's phase stamps when GDN_PERSIST_STAMPS=1 was set at init
 * (uint64 [256 workgroups][25][16] of the 100 MHz real-time counter);
 * which = 3, the per-kernel step's phase stamps when GDN_GRAPH_STAMPS=1 was
 * set at init (uint64 [122 kernels][256 workgroups][4]: start, input ready,
 * products done, end, from each workgroup's thread 0; kernel 5 l + {0 QKVG,
 * 1 recurrence, 2 o_proj, 3 gate/up, 4 down} of layer l, then the LM head
 * and the argmax; the recurrence fills 128 workgroups, the argmax one, with
 * its slots 0 and 3).  No reference counterpart. */
int gdn_test_step_buffers(const GDNRunState *state, int which, void *out, size_t bytes);
/* Layer `layer` of the run state's model for n_steps teacher-forced residual
 * inputs x_in[step][H] (BF16-exact for the BF16 contracts): the same kernels
 * a decode step runs for that layer, against the run state's persistent
 * recurrent/conv state.  x_out[step][H] receives the layer's residual
 * output. */
int gdn_test_layer(GDNRunState *state, uint32_t layer, uint32_t n_steps,
                   const float *x_in, float *x_out);

/* ===== logit tooling (host only): the reference host's scoring and
 *       GPU-logit vector gate, as reusable calls ===== */

/* Parity of one logit stream against a reference stream, accumulated over
 * decode steps: exact / non-finite / FP32-tolerance mismatches, global and
 * per-step NRMSE and cosine, max |error| and its ratio to the reference RMS,
 * top-5 overlap and argmax agreement (host.cpp:61-110, :1412-1586).  No
 * counterpart in gdn_model.h. */
typedef struct GDNLogitsParity {
    uint32_t checked_steps;
    uint32_t argmax_mismatches;
    uint64_t compared_values;
    uint64_t exact_mismatches;
    uint64_t nonfinite_mismatches;
    uint64_t tolerance_failures;
    uint32_t min_top5_overlap;
    uint32_t reserved;
    double max_abs_error;
    double max_rel_error;
    double squared_error_sum;
    double candidate_squared_sum;
    double reference_squared_sum;
    double dot_product_sum;
    double worst_step_nrmse;
    double min_step_cosine;
    double worst_max_abs_over_reference_rms;
} GDNLogitsParity;

void gdn_logits_parity_init(GDNLogitsParity *parity);
/* One step: actual[vocab] (the engine's logits), reference[vocab], and the
 * token the run selected.  apply_fp32_tolerance counts values outside
 * 1e-3 + 1e-4 |reference| as tolerance failures. */
void gdn_logits_parity_step(GDNLogitsParity *parity, const float *actual,
                            const float *reference, uint32_t vocab,
                            uint32_t selected_token, int apply_fp32_tolerance);
double gdn_logits_parity_nrmse(const GDNLogitsParity *parity);
double gdn_logits_parity_cosine(const GDNLogitsParity *parity);
/* 1 when the accumulated parity meets the GPU-logit envelope (global NRMSE
 * <= 0.01, worst step NRMSE <= 0.04, min step cosine >= 0.9995, worst
 * max|err| / ref RMS <= 0.10, max|err| <= 0.5, top-5 overlap 5, no argmax or
 * non-finite mismatch; host.cpp:77-110). */
int gdn_logits_gate_passes(const GDNLogitsParity *parity);
/* log softmax(logits)[target] in double (host.cpp:1954-1995, :2361-2382);
 * NaN when target is out of range. */
double gdn_token_logprob(const float *logits, uint32_t vocab, int32_t target);
/* First index of the maximum under strict '>' from index 0
 * (host.cpp:2348-2359). */
uint32_t gdn_strict_argmax(const float *logits, uint32_t n);

/* ===== multi-stream decode =====
 * No counterpart in the reference, which decodes one stream (README.md:75-77).
 * Up to GDN_MAX_STREAMS (64) independent streams,
 * each with its own FP32 recurrent state and conv tails, advance one token
 * each per step.  Arithmetic is the BF16W_FP32S contract's except inside the
 * projections, which form exact products of the same BF16 operands and sum
 * them in FP32 on the matrix cores; results agree with gdn_decode_step_host
 * under GDN_CONTRACT_BF16W_FP32S to rounding, not bit for bit.  Stream s's
 * results never depend on the other streams. */
#define GDN_MAX_STREAMS 64

struct GDNBatchEngine;
typedef struct {
    struct GDNBatchEngine *engine;
    uint32_t n_streams;
    uint32_t reserved;
} GDNBatchState;

/* Upload the weights (BF16-exact checkpoint) and zero every stream's state.
 * n_streams in 1..GDN_MAX_STREAMS; the vocabulary must be a multiple of 32. */
int gdn_batch_init(GDNBatchState *state, const GDNModel *model, uint32_t n_streams);
void gdn_batch_free(GDNBatchState *state);
/* One step of every stream: tokens[n_streams] in; the greedy next tokens
 * out (next_tokens may be NULL).  -1 for a token outside [0, vocab). */
int gdn_batch_decode_step(GDNBatchState *state, const int32_t *tokens, int32_t *next_tokens);
int gdn_batch_read_tokens(const GDNBatchState *state, int32_t *tokens);
int gdn_batch_read_logits(const GDNBatchState *state, uint32_t stream, float *logits, size_t count);
int gdn_batch_read_final_hidden(const GDNBatchState *state, uint32_t stream, float *hidden, size_t count);
/* One stream's state in the .gdnstate section layouts (as
 * gdn_load_recurrent_state / gdn_load_conv_tails); either pointer may be
 * NULL.  Sizes must be the full per-stream sizes.  The conv tails are kept
 * as BF16 on the device, so loaded tails must be BF16-exact (-1 otherwise,
 * before anything is written). */
int gdn_batch_load_stream_state(GDNBatchState *state, uint32_t stream, const float *recurrent,
                                size_t recurrent_floats, const float *conv_tails, size_t conv_floats);
int gdn_batch_save_stream_state(const GDNBatchState *state, uint32_t stream, float *recurrent,
                                size_t recurrent_floats, float *conv_tails, size_t conv_floats);
/* Prefill: run n_tokens prompt tokens through one stream's state as
 * n_tokens gdn_batch_decode_step calls would feed them to that stream (the
 * GPU prompt pass that produces a .gdnstate, export_gdn_state.py:157-201,
 * :325-330),
 * in segments of up to 4096 tokens (gdn_batch_set_prefill_segment), each
 * layer by layer: token-parallel projections as GEMMs on the matrix cores,
 * the causal conv across the segment, and the recurrence over chunks of 64
 * tokens -- by default in token order with the state held on chip, so
 * results equal the steps bit for bit; in GDN_PREFILL_CHUNKED mode in the
 * chunk-parallel (WY) form of the gated delta rule (chunk.py:616-686), equal
 * to the steps within FP32 re-association.  *seed_token (may be NULL)
 * receives the argmax of the last position; that position's logits and final
 * hidden vector become the stream's readable ones.  Other streams' states
 * are untouched.  The first prefill allocates the segment's buffers (about
 * 150 KB per segment token, 0.6 GB at 4096), kept until the engine is freed
 * or the segment length changes. */
#define GDN_PREFILL_SCAN 0
#define GDN_PREFILL_CHUNKED 1
/* Selects the prefill's recurrence (GDN_PREFILL_SCAN by default).  No
 * reference counterpart: the reference's GPU prefill is the chunked form
 * only, its C++ decode the scan's arithmetic. */
int gdn_batch_set_prefill_mode(GDNBatchState *state, int mode);
/* Tokens per prefill segment: a multiple of 128 in 128..32768 (default
 * 4096).  Longer prompts run as consecutive segments; the results do not
 * depend on the segment length.  No reference counterpart. */
int gdn_batch_set_prefill_segment(GDNBatchState *state, uint32_t tokens);
int gdn_batch_prefill(GDNBatchState *state, uint32_t stream, const int32_t *prompt, uint32_t n_tokens,
                      int32_t *seed_token);
/* n_steps steps with tokens[step][n_streams] fed; per-step argmax
 * [step][n_streams], inner ms (HIP events around the step graph) and outer
 * ms (host tokens in -> host tokens out).  Output pointers may be NULL. */
int gdn_batch_run_teacher_forced(GDNBatchState *state, const int32_t *tokens, uint32_t n_steps,
                                 int32_t *argmax_out, float *inner_ms, float *outer_ms);
/* Average microseconds per launch of each kernel kind, in the order embed,
 * qkvg, recur, onorm, o_proj, layer_norm, gate_up, down, lm_head, argmax
 * (each kind launched back to back over every layer).  Advances state. */
int gdn_batch_profile_kernels(GDNBatchState *state, uint32_t rounds, float *avg_us, uint32_t n_kinds);
/* 0: launch kernels one by one; 1 (default): one captured hipGraph/step. */
int gdn_batch_set_graph_mode(GDNBatchState *state, int use_graph);
/* Host helper (test hook): the multi-stream GEMM's operand tiling of a
 * row-major BF16 matrix [n_rows][k] (16-row x 32-column tiles of 64 lanes x
 * 8 values; lane l carries row l % 16 and columns 8 (l / 16) .. + 7; tiles
 * ordered by (block of 16 rt rows, k tile, row tile)). */
void gdn_test_tile_bf16(const uint16_t *src, size_t n_rows, size_t k, int rt, uint16_t *dst);
/* Test hook: Y[64][N] = X[64][K] W[N][K]^T on the multi-stream GEMM (no
 * rounding of the sums); W and X BF16-exact, K = 2048 (N % 32 == 0) or
 * K = 5632 (N % 16 == 0). */
int gdn_test_batch_gemm(const float *W, const float *X, uint32_t N, uint32_t K, float *Y);
/* Test hook: the prefill's projection GEMM over T tokens (Y [T][N]) beside
 * the step's GEMM run on each 64-token block (Y_step, split sums added in
 * split order).  kind 0: the q/k/v/g configuration (K 2048); 1: o_proj's
 * (K 2048, 4 splits); 2: down's (K 5632, 4 splits); 3: gate/up + SwiGLU
 * (W = gate [5632][2048] then up rows, N = 5632; Y the BF16 SwiGLU values).
 * N a multiple of 128 for kinds 0-2; W and X BF16-exact. */
int gdn_test_prefill_gemm(int kind, const float *W, const float *X, uint32_t N, uint32_t T, float *Y,
                          float *Y_step);

#ifdef __cplusplus
}
#endif
#endif
