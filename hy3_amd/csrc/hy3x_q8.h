// hy3x_q8.h -- the shared expert in hy3's Q8_0, as the library holds it on
// the device, and its per-lane arithmetic.
//
// hy3's Q8_0 block is 36 bytes: an fp32 scale d and 32 int8 q, w = d * q
// (hy3.c:400-403, 1098-1120; hy3_convert.c:1192-1221 writes it for the
// ffn_*_shexp tensors, :684-697). The library repacks every four consecutive
// blocks of a row into one 144-byte super-block of 128 weights:
//   bytes 0..15    d of blocks 0..3 (fp32)
//   bytes 16..143  q of blocks 0..3 (32 int8 each)
// -- the same bytes, and the same 144-byte row-block geometry as Q4_K, so the
// copy machinery of the Q4_K kernels serves both. A 64-weight lane group g of
// a row is half h = g & 1 of super-block g >> 1: scales d[2h], d[2h+1] and
// the 64 bytes at 16 + 64 h.
//
// int8 -> fp16 exactly: (q ^ 0x80) placed under the exponent byte 0x64 is the
// half 1024 + (q + 128) = 1152 + q; the 1152 bias is removed by starting the
// dot2 chain at -1152 * sum(x), as the Q4_K chains start at -1024 * sum(x).
#pragma once
#include "hy3x_q4k.h"

namespace hy3x {

constexpr int Q8K = 128;                                   // weights per super-block
constexpr int Q8_BLOCK = 36;                               // hy3 Q8_0 block bytes
constexpr int64_t Q8_MAT_BYTES = (int64_t)F * D / Q8K * QB;  // 7,077,888 per matrix
constexpr int64_t Q8_EXPERT_BYTES = 3 * Q8_MAT_BYTES;      // gate | up | down

// fp16 pairs (1152 + q) of one lane group: P[4j+0..3] pair with X[4j+0..3]
// of the pair-staged activations (low block: x[4j], x[4j+2] / x[4j+1],
// x[4j+3]; high block: the same at 32 + ...). lo, hi: the 32 bytes of the
// group's low and high block.
__device__ __forceinline__ void unpack_group_q8(const uint4 &lo0, const uint4 &lo1,
                                                const uint4 &hi0, const uint4 &hi1,
                                                uint32_t (&P)[32]) {
  const uint32_t l[8] = {lo0.x, lo0.y, lo0.z, lo0.w, lo1.x, lo1.y, lo1.z, lo1.w};
  const uint32_t h[8] = {hi0.x, hi0.y, hi0.z, hi0.w, hi1.x, hi1.y, hi1.z, hi1.w};
  const uint32_t ex = 0x64646464u;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    const uint32_t a = l[j] ^ 0x80808080u, b = h[j] ^ 0x80808080u;
    P[4 * j + 0] = __builtin_amdgcn_perm(ex, a, 0x04020400u);  // (q0, q2)
    P[4 * j + 1] = __builtin_amdgcn_perm(ex, b, 0x04020400u);
    P[4 * j + 2] = __builtin_amdgcn_perm(ex, a, 0x04030401u);  // (q1, q3)
    P[4 * j + 3] = __builtin_amdgcn_perm(ex, b, 0x04030401u);
  }
}

// This lane's contribution to one row-dot: d_lo * sum(q x) over the low block
// plus d_hi * sum(q x) over the high block.
__device__ __forceinline__ float group_dot_q8(const uint32_t (&P)[32], const uint32_t (&X)[32],
                                              float s_lo, float s_hi, float d_lo, float d_hi) {
  float lo = -1152.0f * s_lo, hi = -1152.0f * s_hi;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    lo = __builtin_amdgcn_fdot2(as_h2(P[4 * j + 0]), as_h2(X[4 * j + 0]), lo, false);
    hi = __builtin_amdgcn_fdot2(as_h2(P[4 * j + 1]), as_h2(X[4 * j + 1]), hi, false);
    lo = __builtin_amdgcn_fdot2(as_h2(P[4 * j + 2]), as_h2(X[4 * j + 2]), lo, false);
    hi = __builtin_amdgcn_fdot2(as_h2(P[4 * j + 3]), as_h2(X[4 * j + 3]), hi, false);
  }
  return d_lo * lo + d_hi * hi;
}

// One lane group of a q8x128 row: the two scales and the 64 bytes.
struct Q8Group {
  uint2 d;     // fp32 bits of d_lo, d_hi
  uint4 q[4];  // low block (q[0], q[1]), high block (q[2], q[3])
};

__device__ __forceinline__ void load_q8_group(const uint8_t *row, int g, Q8Group &o) {
  const uint8_t *sb = row + (size_t)(g >> 1) * QB;
  const int h = g & 1;
  o.d = *reinterpret_cast<const uint2 *>(sb + 8 * h);
  const uint4 *qp = reinterpret_cast<const uint4 *>(sb + 16 + 64 * h);
#pragma unroll
  for (int i = 0; i < 4; i++) o.q[i] = qp[i];
}

__device__ __forceinline__ float q8_group_dot(const Q8Group &gq, const uint32_t (&X)[32],
                                              float slo, float shi) {
  uint32_t P[32];
  unpack_group_q8(gq.q[0], gq.q[1], gq.q[2], gq.q[3], P);
  return group_dot_q8(P, X, slo, shi, __uint_as_float(gq.d.x), __uint_as_float(gq.d.y));
}

// Gate and up rows r0 .. r0 + RPW - 1 of the Q8 shared expert (base wsh) for
// one token, like gateup_rows: lane = 64-weight group, PF rows in flight,
// h = silu(g) * u pair-staged into h16[slot * F + ...] (hy3.c:1296-1300).
template <int RPW, int PF>
struct GateupRowsQ8 {
  // As GateupRows: the constructor puts the first PF rows' loads in flight.
  static constexpr int ROWB = D / Q8K * QB;  // 4608 bytes per gate/up row
  Q8Group ring[PF][2];
  const uint8_t *wsh;
  int slot, r0;
  __device__ __forceinline__ GateupRowsQ8(const uint8_t *__restrict__ wsh_, int slot_, int r0_)
      : wsh(wsh_), slot(slot_), r0(r0_) {
#pragma unroll
    for (int rr = 0; rr < PF && rr < RPW; rr++) issue(rr, ring[rr]);
  }
  __device__ __forceinline__ void issue(int rr, Q8Group (&dst)[2]) const {
    const int lane = threadIdx.x & 63;
    load_q8_group(wsh + (size_t)(r0 + rr) * ROWB, lane, dst[0]);
    load_q8_group(wsh + Q8_MAT_BYTES + (size_t)(r0 + rr) * ROWB, lane, dst[1]);
  }
  __device__ __forceinline__ void finish(const uint32_t (&X)[32], float slo, float shi,
                                         __half *__restrict__ h16) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int rr = 0; rr < RPW; rr++) {
      Q8Group cur[2] = {ring[rr % PF][0], ring[rr % PF][1]};
      if (rr + PF < RPW) issue(rr + PF, ring[rr % PF]);
      const float g = wave_total(q8_group_dot(cur[0], X, slo, shi));
      const float u = wave_total(q8_group_dot(cur[1], X, slo, shi));
      if (lane == 0) h16[(size_t)slot * F + stage_index(r0 + rr)] = swiglu_h(g, u);
    }
  }
};

template <int RPW, int PF>
__device__ __forceinline__ void gateup_rows_q8(const uint8_t *__restrict__ wsh, int slot, int r0,
                                               const uint32_t (&X)[32], float slo, float shi,
                                               __half *__restrict__ h16) {
  GateupRowsQ8<RPW, PF> rows(wsh, slot, r0);
  rows.finish(X, slo, shi, h16);
}

// Down rows r0 .. r0 + 2 PASSES - 1 of the Q8 shared expert for one token,
// one wave, like down_rows: each 32-lane half takes one row per pass (24 of
// its lanes active, one 64-weight group each), PF passes in flight; fn(ps,
// sums) gets the two row sums of pass ps. h: the slot's staged h.
template <int PASSES, int PF, typename Fn>
__device__ __forceinline__ void down_rows_q8(const uint8_t *__restrict__ wsh,
                                             const __half *__restrict__ h, int r0, Fn &&fn) {
  constexpr int G = F / 64, ROWB = F / Q8K * QB;  // 24 groups, 1728 bytes per down row
  const int lane = threadIdx.x & 63, hw = lane >> 5, gl = lane & 31;
  const bool active = gl < G;
  const int glc = active ? gl : G - 1;  // unconditional loads, as down_rows
  const uint8_t *dbase = wsh + 2 * Q8_MAT_BYTES;
  uint32_t X[32];
  load_group_x(h, glc, X);  // h first: loads complete in issue order
  Q8Group ring[PF];
  auto issue = [&](int ps, Q8Group &dst) {
    load_q8_group(dbase + (size_t)(r0 + 2 * ps + hw) * ROWB, glc, dst);
  };
#pragma unroll
  for (int ps = 0; ps < PF && ps < PASSES; ps++) issue(ps, ring[ps]);
  float slo = 0.0f, shi = 0.0f;
  group_sums(X, slo, shi);
#pragma unroll
  for (int ps = 0; ps < PASSES; ps++) {
    const Q8Group cur = ring[ps % PF];
    if (ps + PF < PASSES) issue(ps + PF, ring[ps % PF]);
    const float dv = q8_group_dot(cur, X, slo, shi);
    fn(ps, half_totals(active ? dv : 0.0f));
  }
}

}  // namespace hy3x
