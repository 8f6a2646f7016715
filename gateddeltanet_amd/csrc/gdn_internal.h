// gdn_internal.h -- declarations shared by the host (gdn_host.cpp) and
// device (gdn_engine.hip) halves of libgdn_amd.so.  Not part of the ABI.
#ifndef GDN_INTERNAL_H
#define GDN_INTERNAL_H

#include <stddef.h>
#include <stdint.h>

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

#ifdef __cplusplus
}
#endif
#endif
