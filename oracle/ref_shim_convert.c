/*
 * ref_shim_convert.c -- exposes the reference quantiser (TEST INFRASTRUCTURE).
 *
 * Compiles yuhai-china/hy3's own hy3_convert.c from /root/reference (never
 * copied) with its Makefile flags and exports quantize_row_q4_K
 * (hy3_convert.c:605-651) and fp32_to_fp16 (hy3_convert.c:511-530) under
 * hy3ref_* names, and the converter itself (hy3_convert, :903-1249) on a
 * safetensors directory, which is how the Q8_0 quantiser (inline in it,
 * :1192-1221) is reached. The converter's main() is renamed away. Built only into
 * oracle/_ref/ by oracle/Makefile; used to write golden fixtures and as the
 * benchmark's CPU baseline.
 */
#define main hy3ref_convert_main_unused
#include "hy3_convert.c"
#undef main

void hy3ref_quantize_q4k(const float *x, uint8_t *y, int k) { quantize_row_q4_K(x, y, k); }
uint16_t hy3ref_fp32_to_fp16(float f) { return fp32_to_fp16(f); }
/* quant_type: 8 (Q8_0) or 12 (Q4_K), as `-t` selects in main (:1251-1280). */
int hy3ref_convert(const char *in_dir, const char *out_path, int quant_type) {
  return hy3_convert(in_dir, out_path, quant_type);
}
