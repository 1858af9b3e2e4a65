// hy3x_route.h -- the routing contract's device arithmetic (shared by the
// router kernels and the fused decode kernel). Every function body turns FMA
// contraction off: only the explicit fma calls fuse, as the CPU oracle does.
#pragma once
#include "hy3x_common.h"

namespace hy3x {

__device__ __forceinline__ float sig_expf(float xf) {
#pragma clang fp contract(off)
  if (xf != xf) return xf;
  if (xf > 88.72f) return __builtin_huge_valf();
  if (xf < -87.0f) return 0.0f;
  const double x = (double)xf;
  const double kd = __builtin_rint(x * 1.4426950408889634);
  double r = __builtin_fma(kd, -6.93147180369123816490e-01, x);
  r = __builtin_fma(kd, -1.90821492927058770002e-10, r);
  double p = 1.0 / 6227020800.0;
  p = __builtin_fma(p, r, 1.0 / 479001600.0);
  p = __builtin_fma(p, r, 1.0 / 39916800.0);
  p = __builtin_fma(p, r, 1.0 / 3628800.0);
  p = __builtin_fma(p, r, 1.0 / 362880.0);
  p = __builtin_fma(p, r, 1.0 / 40320.0);
  p = __builtin_fma(p, r, 1.0 / 5040.0);
  p = __builtin_fma(p, r, 1.0 / 720.0);
  p = __builtin_fma(p, r, 1.0 / 120.0);
  p = __builtin_fma(p, r, 1.0 / 24.0);
  p = __builtin_fma(p, r, 1.0 / 6.0);
  p = __builtin_fma(p, r, 0.5);
  p = __builtin_fma(p, r, 1.0);
  p = __builtin_fma(p, r, 1.0);
  const long long k = (long long)kd;
  const double sc = __longlong_as_double((long long)((unsigned long long)(k + 1023) << 52));
  return (float)(p * sc);
}

__device__ __forceinline__ float sigmoid_c(float l) {
#pragma clang fp contract(off)
  return 1.0f / (1.0f + sig_expf(-l));
}

// ((c1+c5)+(c3+c7)) + ((c0+c4)+(c2+c6))
__device__ __forceinline__ float tree8(const float (&c)[8]) {
#pragma clang fp contract(off)
  const float t0 = c[0] + c[4], t1 = c[1] + c[5], t2 = c[2] + c[6], t3 = c[3] + c[7];
  const float u0 = t2 + t0, u1 = t3 + t1;
  return u1 + u0;
}

// Same tree over 8 consecutive lanes (lane group g8 = lane & ~7 holds c[0..7]);
// every lane of the group gets the result.
__device__ __forceinline__ float tree8_lanes(float c, int v) {
#pragma clang fp contract(off)
  const float c4 = __shfl_xor(c, 4, 64);           // lanes v<4: c[v+4]
  const float t = c + c4;                            // t_v = c_v + c_{v+4} (v<4)
  const float t2 = __shfl_xor(t, 2, 64);           // v=0: t2 ; v=1: t3
  const float u = t2 + t;                            // u0 = t2+t0 (v=0), u1 = t3+t1 (v=1)
  const float u1 = __shfl_xor(u, 1, 64);           // v=0 gets u1
  const float res = u1 + u;                          // v=0: u1 + u0
  return __shfl(res, (threadIdx.x & 63) & ~7, 64);
}

// Element m (wave-uniform) of lane l's three-value array, as a wave-uniform
// value. Each of the three is read out of lane l first and the choice is made
// between the scalars: a select between the array elements themselves can be
// lowered to an indexed copy through scratch memory.
__device__ __forceinline__ float pick3_lane(const float (&a)[3], int m, int l) {
  const float a0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a[0]), l));
  const float a1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a[1]), l));
  const float a2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a[2]), l));
  return m == 0 ? a0 : (m == 1 ? a1 : a2);
}

// Best candidate of the wave: largest score, ties to the lowest current
// position (key = position * 256 + expert). Every lane returns the winner.
__device__ __forceinline__ void wave_best(float &v, int &key) {
#pragma clang fp contract(off)
#define HY3X_TAKE(CTRL)                                         \
  {                                                             \
    const float ov = dpp<CTRL>(v);                              \
    const int ok = dppi<CTRL>(key);                             \
    if (ov > v || (ov == v && ok < key)) { v = ov; key = ok; }  \
  }
  HY3X_TAKE(DPP_XOR1)
  HY3X_TAKE(DPP_XOR2)
  HY3X_TAKE(DPP_HALF_MIRROR)
  HY3X_TAKE(DPP_MIRROR)
#undef HY3X_TAKE
  float bv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  int bk = __builtin_amdgcn_readlane(key, 0);
#pragma unroll
  for (int r = 16; r < 64; r += 16) {
    const float ov =
        __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), r));
    const int ok = __builtin_amdgcn_readlane(key, r);
    if (ov > bv || (ov == bv && ok < bk)) { bv = ov; bk = ok; }
  }
  v = bv;
  key = bk;
}

// Top-K of one token by one wave (hy3.c:654-666, 1282-1291). Expert e sits
// at lane e % 64, slot e / 64 of sc (biased score) and sg (sigmoid). Selection
// with swaps: step k takes the largest score among positions >= k, ties to
// the lowest current position, a NaN at position k kept, NaNs elsewhere
// never taken; the element at position k moves to the winner's position. Then sum = sigma_sel0 + sigma_sel1 + ... in selection
// order, inv = 1 / (sum + 1e-20), wpre_k = sigma_k * inv, w_k = wpre_k * scale.
// Everything stays in registers; lane k < K writes ids[k], wpre[k], wout[k].
__device__ __forceinline__ void topk_wave_regs(const float (&sc)[3], const float (&sg)[3], int K,
                                               float scale, int32_t *ids, float *wpre,
                                               float *wout) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  int pos[3] = {lane, lane + 64, lane + 128};
  float sum = 0.0f, my_sig = 0.0f;
  int my_e = 0;
  for (int k = 0; k < K; k++) {
    float bv = -__builtin_huge_valf();
    int bk = 0x7fffffff;
#pragma unroll
    for (int m = 0; m < 3; m++) {
      const int key = pos[m] * 256 + lane + 64 * m;
      // the scan starts from the element at position k and only a strictly
      // greater score replaces it: a NaN there is never replaced (+inf wins
      // every tie by its lowest position), a NaN elsewhere never wins (it
      // compares false). Position k is always a candidate, so some element
      // always wins.
      const float v = (pos[m] == k && sc[m] != sc[m]) ? __builtin_huge_valf() : sc[m];
      if (pos[m] >= k && (v > bv || (v == bv && key < bk))) {
        bv = v;
        bk = key;
      }
    }
    wave_best(bv, bk);
    const int be = bk & 255, bp = bk >> 8;
#pragma unroll
    for (int m = 0; m < 3; m++) {
      if (pos[m] == k) pos[m] = bp;               // the element at position k moves
      if (lane + 64 * m == be) pos[m] = k;        // the winner takes position k
    }
    const float s_be = pick3_lane(sg, be >> 6, be & 63);
    sum = sum + s_be;
    if (lane == k) {
      my_e = be;
      my_sig = s_be;
    }
  }
  const float inv = 1.0f / (sum + 1e-20f);
  if (lane < K) {
    const float v = my_sig * inv;
    ids[lane] = my_e;
    wpre[lane] = v;
    wout[lane] = v * scale;
  }
}

// Top-K by one wave as K rounds of wave-wide argmax over the 192 scores (3
// per lane, expert e at lane e % 64, slot e / 64), on order-preserving integer
// keys (-0 folded into +0, so that equal floats give equal keys). While every
// round's maximum is unique the result is the selection order of
// topk_wave_regs; a round with a tied maximum, or a NaN anywhere, returns
// false and the caller falls back to topk_wave_regs, which follows the
// reference's selection with swaps in every case. Lane k < K receives the
// k-th expert and its sigma; sum = sigma_0 + sigma_1 + ... in selection
// order (wave-uniform). K may be smaller than the routing's top-K when only
// the first places are needed: they do not depend on the later ones. No LDS,
// no barrier.
__device__ __forceinline__ bool topk_wave_fast(const float (&sc)[3], const float (&sg)[3], int K,
                                               int &my_e, float &my_sig, float &sum) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  uint32_t key[3];
  bool nan = false;
#pragma unroll
  for (int m = 0; m < 3; m++) {
    nan |= sc[m] != sc[m];
    const uint32_t u = __builtin_bit_cast(uint32_t, sc[m] + 0.0f);
    key[m] = (u & 0x80000000u) ? ~u : (u | 0x80000000u);  // > 0 for every non-NaN
  }
  if (__builtin_amdgcn_ballot_w64(nan)) return false;
  sum = 0.0f;
  my_e = 0;
  my_sig = 0.0f;
  bool tie = false;
  for (int k = 0; k < K; k++) {
    uint32_t v = key[0] > key[1] ? key[0] : key[1];
    v = v > key[2] ? v : key[2];
    // row maxima by DPP, then row 0 into row 1 and row 2 into row 3
    // (row_bcast:15), then lane 31 into rows 2 and 3 (row_bcast:31): lane 63
    // holds the wave maximum
    v = max(v, (uint32_t)dppi<DPP_XOR1>((int)v));
    v = max(v, (uint32_t)dppi<DPP_XOR2>((int)v));
    v = max(v, (uint32_t)dppi<DPP_HALF_MIRROR>((int)v));
    v = max(v, (uint32_t)dppi<DPP_MIRROR>((int)v));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, DPP_BCAST15, 0xA, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, DPP_BCAST31, 0xC, 0xF, false));
    const uint32_t M = (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
    const bool h0 = key[0] == M, h1 = key[1] == M, h2 = key[2] == M;
    const uint64_t b0 = __builtin_amdgcn_ballot_w64(h0);
    const uint64_t b1 = __builtin_amdgcn_ballot_w64(h1);
    const uint64_t b2 = __builtin_amdgcn_ballot_w64(h2);
    // a tie for this place: noted, the rounds go on without a branch
    tie |= __builtin_popcountll(b0) + __builtin_popcountll(b1) + __builtin_popcountll(b2) != 1;
    const int wl = __builtin_ctzll(b0 | b1 | b2);
    // the winner's slot and sigma, chosen in its own lane, then read out once
    // (masked ORs of the three values, not a select between array elements,
    // which the compiler lowers to an indexed memory read)
    const uint32_t sel_sig = (h0 ? __builtin_bit_cast(uint32_t, sg[0]) : 0u) |
                             (h1 ? __builtin_bit_cast(uint32_t, sg[1]) : 0u) |
                             (h2 ? __builtin_bit_cast(uint32_t, sg[2]) : 0u);
    const int sel_e = lane + (h1 ? 64 : 0) + (h2 ? 128 : 0);
    const float s_e = __builtin_bit_cast(float, __builtin_amdgcn_readlane((int)sel_sig, wl));
    const int e_w = __builtin_amdgcn_readlane(sel_e, wl);
    sum = sum + s_e;
    if (lane == k) {
      my_e = e_w;
      my_sig = s_e;
    }
    key[0] = h0 ? 0u : key[0];  // taken
    key[1] = h1 ? 0u : key[1];
    key[2] = h2 ? 0u : key[2];
  }
  return !tie;
}

// Sum of squares of a 4096-vector by a 256-thread block, thread t holding
// float4 a[u] = x[1024u + 4t .. +3] (u = 0..3): per-thread fmaf chain over
// (u, component), then per wave v += dpp xor1, xor2, half-mirror, mirror and
// (v0 + v16) + (v32 + v48), then (W0 + W1) + (W2 + W3). red_l: 4 floats LDS.
// Returns the total to every thread (contains a barrier).
__device__ __forceinline__ float block_sumsq(const float4 (&a)[4], float *red_l) {
#pragma clang fp contract(off)
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < 4; u++) {
    acc = __builtin_fmaf(a[u].x, a[u].x, acc);
    acc = __builtin_fmaf(a[u].y, a[u].y, acc);
    acc = __builtin_fmaf(a[u].z, a[u].z, acc);
    acc = __builtin_fmaf(a[u].w, a[u].w, acc);
  }
  acc = row16_sum(acc);
  const int b = __builtin_bit_cast(int, acc);
  const float w = (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
                   __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16))) +
                  (__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) +
                   __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48)));
  if ((threadIdx.x & 63) == 0) red_l[threadIdx.x >> 6] = w;
  __syncthreads();
  return (red_l[0] + red_l[1]) + (red_l[2] + red_l[3]);
}

__device__ __forceinline__ void stage_store(__half *dst, int j, float v) {
#pragma clang fp contract(off)
  dst[stage_index(j)] = __float2half(v);
}

// Device dispatch, step 0 (in the first kernel of the routing): clear the
// E x ceil(T/32) token-bitmap words that k_topk marks. Part `part` of `nparts` (one
// per block of that kernel) clears its share; a fill by kernels, not a
// memset, so that the forward stays graph-capturable.
__device__ __forceinline__ void dispatch_clear_part(int T, uint32_t *bits, int wt, int part,
                                                    int nparts) {
  const int nw = (T + 31) >> 5;
  for (int f = part * 256 + (int)threadIdx.x; f < E * nw; f += nparts * 256)
    bits[(f / nw) * wt + f % nw] = 0u;
}


}  // namespace hy3x
