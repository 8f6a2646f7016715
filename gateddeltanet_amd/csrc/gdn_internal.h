// gdn_internal.h -- declarations shared by the host (gdn_host.cpp) and
// device (gdn_engine.hip) halves of libgdn_amd.so.  Not part of the ABI.
#ifndef GDN_INTERNAL_H
#define GDN_INTERNAL_H

#include <stddef.h>
#include <stdint.h>

#include "gdn_amd.h"

#ifdef __cplusplus
extern "C" {
#endif

void gdn_error(const char *message);
float gdn_bf16_round_host(float x);
uint16_t gdn_native_product_bits_host(uint16_t w, uint16_t x);

// Convert n BF16-exact FP32 words to BF16 bits with subnormals flushed to
// signed zero (the native product treats them as zero), and report the
// smallest nonzero and the largest finite magnitude and whether any value is
// not finite.
void gdn_pack_bf16_daz(const float *src, uint16_t *dst, size_t n, float *min_abs, float *max_abs,
                       int *nonfinite);
// Same statistics for an FP32 matrix (no conversion).
void gdn_scan_fp32(const float *src, size_t n, float *min_abs, float *max_abs, int *nonfinite);

// Rearrange a row-major BF16 matrix [n_rows][k] into the operand tiles of
// the multi-stream GEMM (v_mfma_f32_16x16x32_bf16, A operand).  A tile is
// 16 rows x 32 columns stored as 64 lanes x 8 values: lane l carries row
// l % 16, columns 8 (l / 16) .. 8 (l / 16) + 7.  Tiles are ordered by (block
// of 16 * rt rows, 32-column k tile, 16-row tile within the block), so one
// workgroup's rows at one k tile are rt contiguous KiB.  n_rows must be a
// multiple of 16 * rt and k of 32.
void gdn_tile_bf16(const uint16_t *src, size_t n_rows, size_t k, int rt, uint16_t *dst);

// Index of the first value BF16 cannot hold exactly (nonzero low 16 bits),
// or n; and the one-line report of such a value.
size_t gdn_first_non_bf16(const float *values, size_t n);
void gdn_report_non_bf16(const char *what, const float *values, size_t index);

// Native-product counters: whether device counting is on, and adding to the
// process-wide counts.
int gdn_stats_counting(void);
void gdn_stats_add(uint64_t calls, uint64_t special, uint64_t flushed_in, uint64_t flushed_out,
                   uint64_t overflow);
// Adds, per column k of W[rows][K], the rows whose weight has a zero or
// all-ones exponent (spec) and the rows whose weight is subnormal (sub).
void gdn_weight_column_counts(const float *W, size_t rows, size_t K, uint32_t *spec, uint32_t *sub);
// Adds the flushed outputs and overflows of every product W[r][k] x xbits[k].
void gdn_count_native_outcomes(const float *W, size_t rows, size_t K, const uint16_t *xbits, uint64_t *flushed,
                               uint64_t *overflow);

// Host mirrors in the reference's layouts: the recurrent state's BF16
// stripes (four stripe pointers) and the packed conv tails of n_stripes
// stripes in a workspace head buffer.
void gdn_pack_state_stripes(const float *rec, size_t rows, Beat512 *const stripes[]);
void gdn_pack_tail_stripes(const float *conv, size_t n_stripes, float *head_buffer);

// A GDNModel viewing `data` (not owned; free only m->layers).
int gdn_model_wrap(GDNModel *m, const GDNWeightHeader *c, const float *data);

#ifdef __cplusplus
}
#endif
#endif
