/*
 * ref_q8_0.c - harness exporting ggml's own Q8_0 routines, compiled from the
 * reference tree where the sources lie (see the Makefile's `ref` target).
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/ to pin the oracle's Q8_0
 * quantiser/dequantiser bit for bit.  Nothing here is product code, and no
 * reference source is copied: the Makefile compiles
 *   third_party/ggml/src/ggml-cpu/arch/x86/quants.c  (quantize_row_q8_0, :302-398)
 *   third_party/ggml/src/ggml-quants.c               (quantize_row_q8_0_ref :276-299,
 *                                                     dequantize_row_q8_0 :553-567)
 * in place and links only these three wrappers (version script + gc-sections).
 */
#include "ggml-quants.h"
#include "quants.h"

void ref_quantize_row_q8_0_x86(const float *x, void *y, int64_t k) { quantize_row_q8_0(x, y, k); }
void ref_quantize_row_q8_0_scalar(const float *x, void *y, int64_t k) { quantize_row_q8_0_ref(x, (block_q8_0 *) y, k); }
void ref_dequantize_row_q8_0(const void *x, float *y, int64_t k) { dequantize_row_q8_0((const block_q8_0 *) x, y, k); }
