// hy3x_q4k.h -- per-lane Q4_K super-block arithmetic for the gfx950 kernels.
//
// Lane layout: a lane owns one "group" of a Q4_K row = 64 consecutive weights
// = one sub-block pair (2p, 2p+1) of block b (g = 4b + p). It loads the
// block's 16-byte header and the 32 bytes qs[32p .. 32p+31] (two 16-byte
// loads), so four lanes share a header and a 64-lane wave covers 4096
// weights. Activations arrive pair-staged (hy3x_common.h), 32 dwords per
// group. Nibbles are turned into fp16 with the exponent-bias trick
// (0x6400 | q is 1024 + q exactly; 0x6400 | q<<4 is 1024 + 16q), the bias is
// removed by starting each dot2 chain at -1024 * sum(x), and the Q4_K
// dequantisation  w = d*sc*q - dmin*m  (hy3.c:1036-1037) is applied once per
// sub-block: d*sc*sum(q*x) - dmin*m*sum(x).
#pragma once
#include "hy3x_common.h"

namespace hy3x {

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ h2_t as_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }

// Per-lane constants for unpacking the 6-bit scales/mins of sub-blocks 2p and
// 2p+1 (hy3.c:1001-1009) with the same shifts for every p.
struct ScaleSel {
  int off, hs, mo;
  bool lowpair;
  __device__ __forceinline__ explicit ScaleSel(int p)
      : off((p & 1) * 16), hs(p < 2 ? 4 : 6), mo(p < 2 ? 0 : 4), lowpair(p < 2) {}
};

struct BlockScale {
  float a_lo;  // d * sc_lo
  float a_hi;  // d * sc_hi / 16 (the high-nibble chain carries 16*q)
  float m_lo;  // dmin * m_lo
  float m_hi;  // dmin * m_hi
};

__device__ __forceinline__ uint32_t bfe(uint32_t v, int off, int w) {
  return (v >> off) & ((1u << w) - 1u);
}

__device__ __forceinline__ BlockScale block_scale(const uint4 &hdr, const ScaleSel &s) {
  const float d = fp16_quirk(hdr.x & 0xffffu), dmin = fp16_quirk(hdr.x >> 16);
  const uint32_t s03 = hdr.y, s47 = hdr.z, s811 = hdr.w;
  const uint32_t L1 = s.lowpair ? s03 : s811, M1 = s.lowpair ? s47 : s811;
  const uint32_t sc_lo = bfe(L1, s.off, 4) | (bfe(s03, s.off + s.hs, 2) << 4);
  const uint32_t sc_hi = bfe(L1, s.off + 8, 4) | (bfe(s03, s.off + 8 + s.hs, 2) << 4);
  const uint32_t m_lo = bfe(M1, s.off + s.mo, 4) | (bfe(s47, s.off + s.hs, 2) << 4);
  const uint32_t m_hi = bfe(M1, s.off + 8 + s.mo, 4) | (bfe(s47, s.off + 8 + s.hs, 2) << 4);
  BlockScale r;
  r.a_lo = d * (float)sc_lo;
  r.a_hi = d * (float)sc_hi * 0.0625f;
  r.m_lo = dmin * (float)m_lo;
  r.m_hi = dmin * (float)m_hi;
  return r;
}

// (a & m) | o in one VALU op (v_and_or_b32); the compiler otherwise often
// emits an AND and an OR.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(o));
  return r;
}

// fp16 pairs of the 64 nibbles of one group: P[4j+0..3] pair with X[4j+0..3].
__device__ __forceinline__ void unpack_group(const uint4 &q0, const uint4 &q1, uint32_t (&P)[32]) {
  const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
  const uint32_t mag = 0x64006400u;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint32_t a = w[j], b = a >> 8;
    P[4 * j + 0] = and_or(a, 0x000F000Fu, mag);
    P[4 * j + 1] = and_or(a, 0x00F000F0u, mag);
    P[4 * j + 2] = and_or(b, 0x000F000Fu, mag);
    P[4 * j + 3] = and_or(b, 0x00F000F0u, mag);
  }
}

// Activation sums of one staged group (fixed order), from the fp16 values.
__device__ __forceinline__ void group_sums(const uint32_t (&X)[32], float &s_lo, float &s_hi) {
  const h2_t one = {(_Float16)1.0f, (_Float16)1.0f};
  float lo = 0.0f, hi = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    lo = __builtin_amdgcn_fdot2(as_h2(X[4 * j + 0]), one, lo, false);
    hi = __builtin_amdgcn_fdot2(as_h2(X[4 * j + 1]), one, hi, false);
    lo = __builtin_amdgcn_fdot2(as_h2(X[4 * j + 2]), one, lo, false);
    hi = __builtin_amdgcn_fdot2(as_h2(X[4 * j + 3]), one, hi, false);
  }
  s_lo = lo;
  s_hi = hi;
}

// This lane's contribution to one row-dot: sum over its 64 weights of w * x.
__device__ __forceinline__ float group_dot(const uint32_t (&P)[32], const uint32_t (&X)[32],
                                           float s_lo, float s_hi, const BlockScale &bs) {
  float lo = -1024.0f * s_lo, hi = -1024.0f * s_hi;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    lo = __builtin_amdgcn_fdot2(as_h2(P[4 * j + 0]), as_h2(X[4 * j + 0]), lo, false);
    hi = __builtin_amdgcn_fdot2(as_h2(P[4 * j + 1]), as_h2(X[4 * j + 1]), hi, false);
    lo = __builtin_amdgcn_fdot2(as_h2(P[4 * j + 2]), as_h2(X[4 * j + 2]), lo, false);
    hi = __builtin_amdgcn_fdot2(as_h2(P[4 * j + 3]), as_h2(X[4 * j + 3]), hi, false);
  }
  return bs.a_lo * lo + bs.a_hi * hi - (bs.m_lo * s_lo + bs.m_hi * s_hi);
}

__device__ __forceinline__ void load_group_x(const __half *staged, int g, uint32_t (&X)[32]) {
  const uint4 *src = reinterpret_cast<const uint4 *>(staged + g * 64);
#pragma unroll
  for (int v = 0; v < 8; v++) {
    const uint4 t = src[v];
    X[4 * v + 0] = t.x;
    X[4 * v + 1] = t.y;
    X[4 * v + 2] = t.z;
    X[4 * v + 3] = t.w;
  }
}

// Sub-block sums of one fp16 row of n32 * 32 values, as (Sh, Sl, Sh, Sl) with
// Sh = fp16(sum), Sl = fp16(sum - Sh). One lane per sub-block.
__device__ __forceinline__ void row_subsums(const __half *__restrict__ row, int n32,
                                            __half *__restrict__ dst) {
  for (int j = threadIdx.x; j < n32; j += blockDim.x) {
    const uint4 *src = reinterpret_cast<const uint4 *>(row + 32 * j);
    float sum = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const uint4 q = src[v];
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const h2_t p = as_h2(w[u]);
        sum += (float)p[0];
        sum += (float)p[1];
      }
    }
    const _Float16 hi = (_Float16)sum;
    const _Float16 lo = (_Float16)(sum - (float)hi);
    const h2_t r = {hi, lo};
    *reinterpret_cast<h2_t *>(dst + 4 * j) = r;
    *reinterpret_cast<h2_t *>(dst + 4 * j + 2) = r;
  }
}

}  // namespace hy3x
