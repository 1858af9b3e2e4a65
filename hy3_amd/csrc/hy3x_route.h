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

// Top-K of one token by one wave from its 192 sigmoid values and biased
// scores (hy3.c:1282-1291): selection with swaps (each step takes the largest
// score, ties to the lowest current position, and the element at position k
// moves to the winner's position), then w_k = sigma_k * (1/(sum + 1e-20)).
// Scores sit 3 per lane (expert e at lane e%64, slot e/64). sig_l and
// sel_l are LDS scratch (192 and 8 entries). Lane 0 writes ids/wpre/wout.
__device__ __forceinline__ void topk_wave(const float *sig, const float *score, int K, float scale,
                                          int32_t *ids, float *wpre, float *wout, float *sig_l,
                                          int32_t *sel_l) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  float sc[3];
  int pos[3];
#pragma unroll
  for (int m = 0; m < 3; m++) {
    const int e = lane + 64 * m;
    sc[m] = score[e];
    if (sig_l != sig) sig_l[e] = sig[e];
    pos[m] = e;
  }
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
    if (lane == 0) sel_l[k] = be;
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
  __builtin_amdgcn_wave_barrier();
  if (lane == 0) {
    float sum = 0.0f;
    for (int k = 0; k < K; k++) sum += sig_l[sel_l[k]];
    const float inv = 1.0f / (sum + 1e-20f);
    for (int k = 0; k < K; k++) {
      const int e = sel_l[k];
      const float v = sig_l[e] * inv;
      ids[k] = e;
      wpre[k] = v;
      wout[k] = v * scale;
    }
  }
}

// Order-preserving unsigned key of a float score (-0.0 folded into +0.0 so
// that equal scores have equal keys).
__device__ __forceinline__ uint32_t score_key(float v) {
  const uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ int wave_count_ge(const uint32_t (&key)[3], uint32_t t) {
  return __builtin_popcountll(__ballot(key[0] >= t)) + __builtin_popcountll(__ballot(key[1] >= t)) +
         __builtin_popcountll(__ballot(key[2] >= t));
}

// Top-K by one wave without a sequential selection: bisection on the score
// keys finds the largest threshold with K scores at or above it; the K
// selected scores, if distinct from each other and from every unselected
// score, are picked by selection-with-swaps in descending order, so each one's
// rank among them is its slot. Ties at or above the threshold, or a NaN, use
// the sequential selection (topk_wave), which defines the result then.
// Writes ids/wpre/wout (lane 0) like topk_wave; sig_l, sel_l: LDS scratch.
__device__ __forceinline__ void topk_ballot(const float *sig, const float *score, int K,
                                            float scale, int32_t *ids, float *wpre, float *wout,
                                            float *sig_l, int32_t *sel_l,
                                            unsigned long long *trace = nullptr) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  uint32_t key[3];
  float sg[3];
  bool nan = false;
#pragma unroll
  for (int m = 0; m < 3; m++) {
    const float v = score[lane + 64 * m];
    sg[m] = sig[lane + 64 * m];
    nan |= v != v;
    key[m] = score_key(v);
  }
  if (trace) {
    __builtin_amdgcn_s_waitcnt(0);
    trace_point(trace, 4);
  }
  // largest t with count(key >= t) >= K (count(key >= 0) = 192 >= K holds
  // initially; the interval halves every step, so 32 steps finish it)
  uint64_t lo = 0ull, hi = 0xFFFFFFFFull;
  for (int it = 0; it < 33 && lo < hi; it++) {
    const uint64_t mid = (lo + hi + 1ull) >> 1;
    if (wave_count_ge(key, (uint32_t)mid) >= K) lo = mid; else hi = mid - 1ull;
  }
  const uint32_t thr = (uint32_t)lo;
  if (trace) trace_point(trace, 5);
  const bool exact = wave_count_ge(key, thr) == K && __ballot(nan) == 0ull;
  bool distinct = exact;
  if (exact) {
    // rank of each selected score among the selected ones
#pragma unroll
    for (int m = 0; m < 3; m++) {
      const bool mine = key[m] >= thr;
      int above = 0, equal = 0;
      const unsigned long long selm[3] = {__ballot(key[0] >= thr), __ballot(key[1] >= thr),
                                          __ballot(key[2] >= thr)};
      // compare against every selected key (at most K of them)
      for (int mm = 0; mm < 3; mm++) {
        unsigned long long msk = selm[mm];
        while (msk) {
          const int src = __builtin_ctzll(msk);
          msk &= msk - 1ull;
          const uint32_t kv = (uint32_t)__builtin_amdgcn_readlane((int)key[mm], src);
          above += kv > key[m];
          equal += (kv == key[m]) && !(src == lane && mm == m);
        }
      }
      if (mine) {
        if (equal) distinct = false;
        sel_l[above] = lane + 64 * m;
        sig_l[lane + 64 * m] = sg[m];
      }
    }
    distinct = __ballot(!distinct) == 0ull;
  }
  if (!distinct) {
    topk_wave(sig, score, K, scale, ids, wpre, wout, sig_l, sel_l);
    return;
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
  __builtin_amdgcn_wave_barrier();
  if (lane == 0) {
    float sum = 0.0f;
    for (int k = 0; k < K; k++) sum += sig_l[sel_l[k]];
    const float inv = 1.0f / (sum + 1e-20f);
    for (int k = 0; k < K; k++) {
      const int e = sel_l[k];
      const float v = sig_l[e] * inv;
      ids[k] = e;
      wpre[k] = v;
      wout[k] = v * scale;
    }
  }
}

// Top-K by a 256-thread block: thread t counts, for elements i = t, t+256..
// (i < 192 x 4 comparator quarters), the scores of quarter t/192.. greater
// than score i; the four partial ranks are summed in LDS. With distinct top
// scores, selection-with-swaps picks in descending score order, so the element
// of rank k is the k-th pick. Any tie among the first K ranks (two elements
// with one rank, or a rank left empty) or a NaN sends wave 0 to the
// sequential selection, which defines the result then. sc_l/sg_l: LDS (192
// each); scratch_l: LDS int[4*192 + 2*KMAX + 2]; ids/wpre/w: LDS or global.
// Every thread must call it; it ends with a barrier.
__device__ __forceinline__ void topk_block(const float *sig, const float *score, int K, float scale,
                                           int32_t *ids_l, float *wpre_l, float *w_l,
                                           float *sc_l, float *sg_l, int32_t *scratch_l) {
#pragma clang fp contract(off)
  const int tid = threadIdx.x;
  int32_t *part_l = scratch_l, *cnt_l = scratch_l + 4 * E, *flag_l = cnt_l + KMAX,
          *sel_l = flag_l + 1;
  if (tid < E) {
    sc_l[tid] = score[tid];
    sg_l[tid] = sig[tid];
  }
  if (tid < KMAX) cnt_l[tid] = 0;
  if (tid == 0) *flag_l = 0;
  __syncthreads();
  // (element, quarter) pairs q = tid + 256 j, j < 3: element q % 192, quarter q / 192
#pragma unroll
  for (int j = 0; j < 3; j++) {
    const int q = tid + 256 * j, i = q % E, c = q / E;
    const float s = sc_l[i];
    const float4 *v4 = reinterpret_cast<const float4 *>(sc_l + 48 * c);
    int rank = 0;
#pragma unroll
    for (int u = 0; u < 12; u++) {
      const float4 v = v4[u];
      rank += (v.x > s) + (v.y > s) + (v.z > s) + (v.w > s);
    }
    part_l[q] = rank;
  }
  __syncthreads();
  if (tid < E) {
    const int rank = (part_l[tid] + part_l[tid + E]) + (part_l[tid + 2 * E] + part_l[tid + 3 * E]);
    const float s = sc_l[tid];
    if (s != s) atomicOr(flag_l, 1);
    if (rank < K) {
      atomicAdd(&cnt_l[rank], 1);
      sel_l[rank] = tid;
    }
  }
  __syncthreads();
  if (tid < K && cnt_l[tid] != 1) atomicOr(flag_l, 1);
  __syncthreads();
  if (*flag_l) {
    if (tid < 64) topk_wave(sg_l, sc_l, K, scale, ids_l, wpre_l, w_l, sg_l, sel_l);
  } else if (tid == 0) {
    float sum = 0.0f;
    for (int k = 0; k < K; k++) sum += sg_l[sel_l[k]];
    const float inv = 1.0f / (sum + 1e-20f);
    for (int k = 0; k < K; k++) {
      const int e = sel_l[k];
      const float v = sg_l[e] * inv;
      ids_l[k] = e;
      wpre_l[k] = v;
      w_l[k] = v * scale;
    }
  }
  __syncthreads();
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

}  // namespace hy3x
