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

// Top-K of one token by one wave (hy3.c:1282-1291). Expert e sits at lane
// e % 64, slot e / 64 of sc (biased score) and sg (sigmoid). Selection with
// swaps: step k takes the largest score among positions >= k, ties to the
// lowest current position, and the element at position k moves to the
// winner's position. Then sum = sigma_sel0 + sigma_sel1 + ... in selection
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
      if (pos[m] >= k && (sc[m] > bv || (sc[m] == bv && key < bk))) {
        bv = sc[m];
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
    const int bm = be >> 6;
    const float sv = bm == 0 ? sg[0] : (bm == 1 ? sg[1] : sg[2]);
    const float s_be =
        __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sv), be & 63));
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

// The same from 192-entry arrays sig / score (global or LDS).
__device__ __forceinline__ void topk_wave(const float *sig, const float *score, int K, float scale,
                                          int32_t *ids, float *wpre, float *wout) {
  const int lane = threadIdx.x & 63;
  float sc[3], sg[3];
#pragma unroll
  for (int m = 0; m < 3; m++) {
    sc[m] = score[lane + 64 * m];
    sg[m] = sig[lane + 64 * m];
  }
  topk_wave_regs(sc, sg, K, scale, ids, wpre, wout);
}

// Top-K by a 256-thread block, with the same result as topk_wave_regs.
// Rank of element e = number of scores strictly greater than score[e]: wave w
// holds quarter w (scores 48w .. 48w+47) as wave-uniform values and counts,
// for each of its lanes' three elements (lane + 64 m), how many of them are
// greater; the four partial counts are summed in LDS. With distinct top
// scores, selection with swaps picks in descending score order, so the
// element of rank k is the k-th pick. Any tie among the first K ranks (two
// elements with one rank, or a rank left empty) or a NaN sends wave 0 to the
// sequential selection, which defines the result then.
// sig / score: 192 entries each (global or LDS; visible to the whole block).
// sg_l: LDS float[192]; scratch_l: LDS int[4*192 + 2*KMAX + 2]. ids_l, wpre_l,
// w_l: outputs (LDS or global), valid after the call, which ends with a
// barrier unless kFinalBarrier is false (then the caller's next barrier makes
// them visible). Every thread must call it; after it, no global memory is read.
template <bool kFinalBarrier = true>
__device__ __forceinline__ void topk_block(const float *sig, const float *score, int K, float scale,
                                           int32_t *ids_l, float *wpre_l, float *w_l, float *sg_l,
                                           int32_t *scratch_l,
                                           unsigned long long *trace = nullptr) {
#pragma clang fp contract(off)
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int32_t *part_l = scratch_l, *cnt_l = scratch_l + 4 * E, *flag_l = cnt_l + KMAX,
          *sel_l = flag_l + 1;
  // every load first: the lane's three elements, the wave's quarter, sigma
  float v[3];
#pragma unroll
  for (int m = 0; m < 3; m++) v[m] = score[lane + 64 * m];
  float4 q4[12];
  // waves past the fourth (wider blocks) repeat a quarter and keep no count
  const float4 *qsrc = reinterpret_cast<const float4 *>(score + 48 * (wave & 3));
#pragma unroll
  for (int u = 0; u < 12; u++) q4[u] = qsrc[u];
  // unconditional (a clamped index): a load under a lane condition would wait
  // for the loads issued before it
  const float sgv = sig[tid < E ? tid : E - 1];
  if (tid < KMAX) cnt_l[tid] = 0;
  if (tid == 0) *flag_l = 0;
  int cnt[3] = {0, 0, 0};
#pragma unroll
  for (int u = 0; u < 12; u++) {
    const float qx = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, q4[u].x)));
    const float qy = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, q4[u].y)));
    const float qz = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, q4[u].z)));
    const float qw = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, q4[u].w)));
#pragma unroll
    for (int m = 0; m < 3; m++)
      cnt[m] += (int)(qx > v[m]) + (int)(qy > v[m]) + (int)(qz > v[m]) + (int)(qw > v[m]);
  }
#pragma unroll
  for (int m = 0; m < 3; m++)
    if (wave < 4) part_l[wave * E + lane + 64 * m] = cnt[m];
  if (tid < E) sg_l[tid] = sgv;
  __syncthreads();
  if (trace) trace_point(trace, 4);
  if (tid < E) {
    const int rank = (part_l[tid] + part_l[tid + E]) + (part_l[tid + 2 * E] + part_l[tid + 3 * E]);
    const float sv = wave == 0 ? v[0] : (wave == 1 ? v[1] : v[2]);  // score[tid]
    if (sv != sv) atomicOr(flag_l, 1);
    if (rank < K) {
      atomicAdd(&cnt_l[rank], 1);
      sel_l[rank] = tid;
    }
  }
  __syncthreads();
  if (tid < K && cnt_l[tid] != 1) atomicOr(flag_l, 1);
  __syncthreads();
  if (trace) trace_point(trace, 5);
  if (*flag_l) {
    if (wave == 0) topk_wave(sg_l, score, K, scale, ids_l, wpre_l, w_l);
  } else if (wave == 0) {
    const int e = lane < K ? sel_l[lane] : 0;
    const float se = sg_l[e];
    float sum = 0.0f;
    for (int k = 0; k < K; k++)
      sum = sum + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, se), k));
    const float inv = 1.0f / (sum + 1e-20f);
    if (lane < K) {
      const float wv = se * inv;
      ids_l[lane] = e;
      wpre_l[lane] = wv;
      w_l[lane] = wv * scale;
    }
  }
  if (kFinalBarrier) __syncthreads();
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
// E x ceil(T/32) token-bitmap words of step 1. Part `part` of `nparts` (one
// per block of that kernel) clears its share; a fill by kernels, not a
// memset, so that the forward stays graph-capturable.
__device__ __forceinline__ void dispatch_clear_part(int T, uint32_t *bits, int wt, int part,
                                                    int nparts) {
  const int nw = (T + 31) >> 5;
  for (int f = part * 256 + (int)threadIdx.x; f < E * nw; f += nparts * 256)
    bits[(f / nw) * wt + f % nw] = 0u;
}

// Step 1 (in the top-K kernel, once token t's ids are out): bit t of each of
// its experts' token bitmaps (bits[e * wt + t / 32]). The result is
// independent of the order of the atomics; step 2 counts by popcount.
__device__ __forceinline__ void dispatch_mark(const int32_t *ids_t, int t, int K, uint32_t *bits,
                                              int wt) {
  if ((int)threadIdx.x < K) {
    const int e = ids_t[threadIdx.x];
    if (e >= 0 && e < E) atomicOr(&bits[(size_t)e * wt + (t >> 5)], 1u << (t & 31));
  }
}

}  // namespace hy3x
