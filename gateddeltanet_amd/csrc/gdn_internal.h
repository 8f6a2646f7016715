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

#ifdef __cplusplus
}
#endif
#endif
