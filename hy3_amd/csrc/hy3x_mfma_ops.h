// hy3x_mfma_ops.h -- the Q4_K x fp16 MFMA building blocks shared by the
// grouped-GEMM tile kernels (hy3x_mfma.hip, hy3x_mfma_big.hip): operand
// types, the weight copy, the Q4_K scale unpack, the exact integer weight
// operands and the mins operand.
#pragma once
#include "hy3x_kernels.h"
#include "hy3x_q4k.h"
#include "hy3x_dma.h"

namespace hy3x {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));  // 16 bytes as a native vector
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

// dma16_stream is the weight copy, with the default cache policy (a
// non-temporal one measured ~15% slower).
__device__ __forceinline__ void dma16_stream(const void *sbase, uint32_t voff, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase),
               "{m0}"(lds)
               : "memory");
}

__device__ __forceinline__ uint32_t pk_fma_f16(uint32_t a, h2_t b, h2_t c) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(as_h2(a), b, c));
}

// The 6-bit scales and mins of a Q4_K block (hy3.c:1001-1009) as bytes:
// sc[0] = sc_0..3, sc[1] = sc_4..7, mn[0] = m_0..3, mn[1] = m_4..7.
struct Scales6 {
  uint32_t sc[2], mn[2];
};
__device__ __forceinline__ Scales6 unpack_scales(const u4_t &h) {
  // j < 4: sc_j = s[j] & 63, m_j = s[j+4] & 63
  // j >= 4: sc_j = (s[j+4] & 15) | (s[j-4] >> 6) << 4, m_j = (s[j+4] >> 4) | (s[j] >> 6) << 4
  Scales6 r;
  r.sc[0] = h.y & 0x3F3F3F3Fu;
  r.mn[0] = h.z & 0x3F3F3F3Fu;
  r.sc[1] = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
  r.mn[1] = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
  return r;
}

// fp16 pair of the two bytes of w that `sel` (a v_perm selector placing them
// in bytes 0 and 2, zeros in 1 and 3) picks, values <= 63: the bytes go into
// the mantissa of 1024.0, then 1024 is subtracted (both steps exact).
__device__ __forceinline__ h2_t bytes_h2(uint32_t w, uint32_t sel) {
  const uint32_t v = __builtin_amdgcn_perm(w, w, sel) | 0x64006400u;
  return as_h2(v) + (h2_t){(_Float16)-1024.0f, (_Float16)-1024.0f};
}

// Weight operands of one 8-byte run of qs: the low nibbles (sub-block scale
// sc_lo) and the high nibbles (sc_hi) as exact integers sc*q in fp16
// (sc*q <= 945). Low: 0x6400 | q = 1024 + q, times sc_lo, minus 1024 sc_lo.
// High, left in place: 0x6400 | 16q = 1024 + 16q, times sc_hi/16, minus
// 64 sc_hi. Each is one fused multiply-add whose exact result is
// representable, so it is exact.
__device__ __forceinline__ void dequant_run(u2_t q, h2_t ml, h2_t al, h2_t mh, h2_t ah,
                                            h8_t &w_lo, h8_t &w_hi) {
  const uint32_t mag = 0x64006400u, m_lo = 0x000F000Fu, m_hi = 0x00F000F0u;
  const uint32_t x8 = q.x >> 8, y8 = q.y >> 8;
  u4_t lo, hi;
  lo.x = pk_fma_f16(and_or(q.x, m_lo, mag), ml, al);
  lo.y = pk_fma_f16(and_or(x8, m_lo, mag), ml, al);
  lo.z = pk_fma_f16(and_or(q.y, m_lo, mag), ml, al);
  lo.w = pk_fma_f16(and_or(y8, m_lo, mag), ml, al);
  hi.x = pk_fma_f16(and_or(q.x, m_hi, mag), mh, ah);
  hi.y = pk_fma_f16(and_or(x8, m_hi, mag), mh, ah);
  hi.z = pk_fma_f16(and_or(q.y, m_hi, mag), mh, ah);
  hi.w = pk_fma_f16(and_or(y8, m_hi, mag), mh, ah);
  w_lo = __builtin_bit_cast(h8_t, lo);
  w_hi = __builtin_bit_cast(h8_t, hi);
}

// -dmin * m_j for sub-blocks j = 2g and 2g+1 of this lane's row, each split
// exactly into two fp16 parts (dmin: 11 significant bits, m: 6, so the
// product is exact in fp32 and hi + lo carries it to 22 bits), laid out for
// the mins MFMA: k = 4j' + c, c = (hi, hi, lo, lo) against the staged
// activation sums (Sh, Sl, Sh, Sl): the four cross products of the two splits.
__device__ __forceinline__ h8_t mins_operand(float dmin, uint32_t m2) {
  const float v0 = -dmin * (float)(m2 & 0xFFu), v1 = -dmin * (float)((m2 >> 8) & 0xFFu);
  const _Float16 h0 = (_Float16)v0, h1 = (_Float16)v1;
  const _Float16 l0 = (_Float16)(v0 - (float)h0), l1 = (_Float16)(v1 - (float)h1);
  return (h8_t){h0, h0, l0, l0, h1, h1, l1, l1};
}

// Launch order -> work item, so that consecutive work items run on one XCD
// (workgroups are dealt to the 8 XCDs round-robin): the row tiles of one
// expert tile share its activations in that XCD's L2, and consecutive token
// tiles of one expert share its weights.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  const int q = nblocks >> 3, r = nblocks & 7, x = bid & 7, i = bid >> 3;
  return x * q + (x < r ? x : r) + i;
}

// Launch order -> work item with whole tiles dealt round-robin to the XCDs:
// tile j's nrt row tiles run consecutively on XCD j % 8 (sharing the tile's
// activations in that L2), and neighbouring tiles go to different XCDs. Work
// item w < n_tiles * nrt is block ((w / nrt / 8) * nrt + w % nrt) * 8 +
// (w / nrt) % 8, which is below (n_tiles + 7) * nrt: the grid needs
// XCD_TILE_RR_MARGIN = 7 tiles of margin; blocks whose item is past the work
// leave.
__device__ __forceinline__ int xcd_tile_rr(int bid, int nrt) {
  const int x = bid & 7, i = bid >> 3;
  return ((i / nrt) * 8 + x) * nrt + i % nrt;
}

// fp16 weights (exact q) of 8 consecutive bytes, in the staged activations'
// run order (0, 2, 1, 3, 4, 6, 5, 7).
__device__ __forceinline__ h8_t q8_run(u2_t b) {
  const uint32_t ex = 0x64646464u, a = b.x ^ 0x80808080u, c = b.y ^ 0x80808080u;
  const h2_t m1152 = {(_Float16)-1152.0f, (_Float16)-1152.0f};
  u4_t w;
  w.x = __builtin_bit_cast(uint32_t, as_h2(__builtin_amdgcn_perm(ex, a, 0x04020400u)) + m1152);
  w.y = __builtin_bit_cast(uint32_t, as_h2(__builtin_amdgcn_perm(ex, a, 0x04030401u)) + m1152);
  w.z = __builtin_bit_cast(uint32_t, as_h2(__builtin_amdgcn_perm(ex, c, 0x04020400u)) + m1152);
  w.w = __builtin_bit_cast(uint32_t, as_h2(__builtin_amdgcn_perm(ex, c, 0x04030401u)) + m1152);
  return __builtin_bit_cast(h8_t, w);
}

}  // namespace hy3x
