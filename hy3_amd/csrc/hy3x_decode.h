// hy3x_decode.h -- single-token (decode) expert row streaming shared by the
// routing kernel (shared expert) and the routed gate/up kernel.
#pragma once
#include "hy3x_q4k.h"

namespace hy3x {

// Gate and up rows r0 .. r0 + RPW - 1 of expert e for one token: each lane
// owns one 64-weight group of the row (lane = 4 * block + pair), X holds the
// token's staged s for that group and slo/shi its sub-block sums. The rows'
// Q4_K bytes go through a ring of PF rows in flight; the wave reduces each
// row dot with DPP and lane 0 writes h = silu(g) * u, pair-staged, to
// h16[slot * F + ...] (hy3.c:1296-1300 / 1307-1314).
template <int RPW, int PF>
struct GateupRows {
  // Split in two so that a caller can put the first PF rows' loads in flight
  // before it has the activations (the constructor issues them).
  uint4 ring[PF][6];
  const uint8_t *gbase, *ubase;
  int slot, r0;
  __device__ __forceinline__ GateupRows(const uint8_t *__restrict__ wq, int e, int slot_, int r0_)
      : slot(slot_), r0(r0_) {
    const int lane = threadIdx.x & 63, b = lane >> 2;
    gbase = wq + (size_t)e * EXPERT_BYTES + (size_t)b * QB;
    ubase = gbase + MAT_BYTES;
#pragma unroll
    for (int rr = 0; rr < PF && rr < RPW; rr++) issue(rr, ring[rr]);
  }
  __device__ __forceinline__ void issue(int rr, uint4 (&dst)[6]) const {
    const int p = threadIdx.x & 3;
    const uint8_t *gp = gbase + (size_t)(r0 + rr) * (D / QK) * QB;
    const uint8_t *up = ubase + (size_t)(r0 + rr) * (D / QK) * QB;
    dst[0] = *reinterpret_cast<const uint4 *>(gp);
    dst[1] = *reinterpret_cast<const uint4 *>(gp + 16 + 32 * p);
    dst[2] = *reinterpret_cast<const uint4 *>(gp + 32 + 32 * p);
    dst[3] = *reinterpret_cast<const uint4 *>(up);
    dst[4] = *reinterpret_cast<const uint4 *>(up + 16 + 32 * p);
    dst[5] = *reinterpret_cast<const uint4 *>(up + 32 + 32 * p);
  }
  __device__ __forceinline__ void finish(const uint32_t (&X)[32], float slo, float shi,
                                         __half *__restrict__ h16) {
    const int lane = threadIdx.x & 63;
    const ScaleSel sel(lane & 3);
#pragma unroll
    for (int rr = 0; rr < RPW; rr++) {
      uint4 cur[6];
#pragma unroll
      for (int q = 0; q < 6; q++) cur[q] = ring[rr % PF][q];
      if (rr + PF < RPW) issue(rr + PF, ring[rr % PF]);
      uint32_t P[32];
      unpack_group(cur[1], cur[2], P);
      const float gv = group_dot(P, X, slo, shi, block_scale(cur[0], sel));
      unpack_group(cur[4], cur[5], P);
      const float uv = group_dot(P, X, slo, shi, block_scale(cur[3], sel));
      const float g = wave_total(gv), u = wave_total(uv);
      if (lane == 0) h16[(size_t)slot * F + stage_index(r0 + rr)] = swiglu_h(g, u);
    }
  }
};

template <int RPW, int PF>
__device__ __forceinline__ void gateup_rows(const uint8_t *__restrict__ wq, int e, int slot,
                                            int r0, const uint32_t (&X)[32], float slo,
                                            float shi, __half *__restrict__ h16) {
  GateupRows<RPW, PF> rows(wq, e, slot, r0);
  rows.finish(X, slo, shi, h16);
}

// Down rows r0 .. r0 + 2 PASSES - 1 of expert e for one token, one wave:
// each 32-lane half takes one row per pass (lane = one 64-weight group of
// the 1536, 24 of the 32 lanes active), the passes' Q4_K go through a ring of
// PF passes in flight, and fn(ps, sums) gets the two row sums of pass ps
// (row r0 + 2 ps in .x, r0 + 2 ps + 1 in .y, wave-uniform). h: the slot's
// staged h (hy3.c:1316-1317).
template <int PASSES, int PF, typename Expert, typename Fn>
__device__ __forceinline__ void down_rows(const uint8_t *__restrict__ wq, Expert &&expert,
                                          const __half *__restrict__ h, int r0, Fn &&fn) {
  constexpr int G = F / 64;
  const int lane = threadIdx.x & 63, hw = lane >> 5, gl = lane & 31;
  const bool active = gl < G;
  // Every lane loads (the 8 idle lanes of each half re-read group G - 1 and
  // drop it): loads under a lane condition make the compiler wait for the
  // whole ring at every pass, which serialises the passes.
  const int glc = active ? gl : G - 1;
  const int b = glc >> 2, p = glc & 3;
  const ScaleSel sel(p);
  // h first: loads complete in issue order for the wait counters, so h
  // issued after the weight ring would hold the first pass back until the
  // whole ring had landed. The expert id (expert(): a constant, or a load
  // from memory) is read after h's loads are in flight.
  uint32_t X[32];
  load_group_x(h, glc, X);
  asm volatile("" ::: "memory");  // h's loads issue before the id's
  const int e = expert();
  const uint8_t *dbase = wq + (size_t)e * EXPERT_BYTES + 2 * MAT_BYTES + (size_t)b * QB;
  uint4 ring[PF][3];
  auto issue = [&](int ps, uint4 (&dst)[3]) {
    const uint8_t *dp = dbase + (size_t)(r0 + 2 * ps + hw) * (F / QK) * QB;
    dst[0] = *reinterpret_cast<const uint4 *>(dp);
    dst[1] = *reinterpret_cast<const uint4 *>(dp + 16 + 32 * p);
    dst[2] = *reinterpret_cast<const uint4 *>(dp + 32 + 32 * p);
  };
#pragma unroll
  for (int ps = 0; ps < PF && ps < PASSES; ps++) issue(ps, ring[ps]);
  float slo = 0.0f, shi = 0.0f;
  group_sums(X, slo, shi);
#pragma unroll
  for (int ps = 0; ps < PASSES; ps++) {
    uint4 cur[3];
#pragma unroll
    for (int q = 0; q < 3; q++) cur[q] = ring[ps % PF][q];
    if (ps + PF < PASSES) issue(ps + PF, ring[ps % PF]);
    uint32_t P[32];
    unpack_group(cur[1], cur[2], P);
    const float dv = group_dot(P, X, slo, shi, block_scale(cur[0], sel));
    fn(ps, half_totals(active ? dv : 0.0f));
  }
}

// Decode launch shapes (measured on MI355X; the alternatives tried and their
// figures are recorded with the design notes, not as build switches).
constexpr int DEC_RPW = 4;                   // gate/up rows per wave
constexpr int DEC_GU_PF = 2;                 // gate/up rows in flight per wave (4: all of them, 0.3-0.4 us slower)
// Shared gate/up rows per wave of a routing block: two (192 blocks of 8
// rows; each block recomputes s, so fewer blocks also load x and norm_w
// fewer times). C0 per forward, 1 / 2 / 3 / 4 rows per wave: 30.06 / 29.87 /
// 30.7 / 31.3 us (with 16-row blocks and the route blocks' LDS larger, the
// last shared blocks had ended about 1 us after the router chains).
constexpr int DEC_SH_RPW = 2;
constexpr int DEC_RPB = 4 * DEC_SH_RPW;       // shared gate/up rows per routing block (four waves)
static_assert(F % DEC_RPB == 0, "the routing kernel's shared blocks cover every row");
constexpr int DEC_SH_BLOCKS = F / DEC_RPB;   // shared gate/up blocks of the routing kernel (192)
// Waves per routed gate/up block (each block routes the token once, then its
// waves stream DEC_RPW rows each): one, so 3072 blocks of 4 rows (12 per
// CU, all resident). C0 per forward against 4-wave blocks: 29.38 vs 29.75 us;
// 2 waves 29.6, 3 waves 30.1; one wave of 2, 3, 6, 8 rows: 31.2, 31.9, 29.9,
// 30.8.
constexpr int DEC_GU_WAVES = 1;
constexpr int DEC_GU_RPB = DEC_GU_WAVES * DEC_RPW;  // routed gate/up rows per block
static_assert(F % DEC_GU_RPB == 0, "whole blocks per expert");
constexpr int DEC_GU_BLOCKS = F / DEC_GU_RPB;       // routed gate/up blocks per expert
constexpr int DEC_DOWN_RPB = 16;  // down rows per block
constexpr int DEC_DOWN_PF = 2;    // down passes (2 rows each) in flight per wave
// Waves of a down block: one per routed slot, then the shared expert's rows
// split over DEC_DOWN_SH_WAVES waves, so that every SIMD runs the same number
// of passes (with one shared wave, the SIMD holding three waves set the pace).
constexpr int DEC_DOWN_SH_WAVES = 4;
constexpr int DEC_DOWN_WAVES = KMAX + DEC_DOWN_SH_WAVES;
static_assert(DEC_DOWN_RPB % (2 * DEC_DOWN_SH_WAVES) == 0, "whole passes per shared wave");

}  // namespace hy3x
