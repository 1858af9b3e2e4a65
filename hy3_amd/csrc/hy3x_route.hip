// hy3x_route.hip -- RMSNorm + router + top-K, and the device dispatch.
//
// Routing contract (the reference CPU block hy3.c:1266-1291 as its Makefile
// builds it; restated by the CPU oracle, which the results match bit for bit):
//  * every fp32 sum over the 4096 hidden elements has the order gcc's 8-wide
//    FMA vectorisation gives it: chain v (v = 0..7) accumulates a[8i+v]*b[8i+v]
//    with fmaf for i = 0..511 from 0, then ((c1+c5)+(c3+c7)) + ((c0+c4)+(c2+c6));
//  * ss = sum x^2; r = 1/sqrt(ss/4096 + 1e-5) correctly rounded; s = (x*w)*r
//    (hy3.c:435-444; the build's own r comes from an rsqrt estimate and a
//    Newton step whose last bits depend on the host CPU);
//  * logit_e = sum router[e,:]*s (hy3.c:1269);
//  * sigma = 1/(1 + exp(-logit)) with exp correctly rounded (evaluated in
//    fp64: Cody-Waite reduction, degree-13 Taylor polynomial); score = sigma +
//    bias (hy3.c:1272-1277);
//  * top-K by selection with swaps, strict '>' (hy3.c:654-666), reproduced in
//    parallel: each step takes the largest score, ties to the lowest current
//    position, then swaps it into place;
//  * wpre_k = sigma_k * (1/(sum_k sigma_k + 1e-20)) (k order), w = wpre*scale
//    (hy3.c:1283-1291).
// fp32 division and sqrt are correctly rounded (built with
// -fhip-fp32-correctly-rounded-divide-sqrt) and nothing in this file is
// contracted into FMAs beyond the explicit fmaf calls.
#include "hy3x_common.h"

#pragma clang fp contract(off)

namespace hy3x {

__device__ __forceinline__ float sig_expf(float xf) {
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

__device__ __forceinline__ float sigmoid_c(float l) { return 1.0f / (1.0f + sig_expf(-l)); }

// ((c1+c5)+(c3+c7)) + ((c0+c4)+(c2+c6))
__device__ __forceinline__ float tree8(const float (&c)[8]) {
  const float t0 = c[0] + c[4], t1 = c[1] + c[5], t2 = c[2] + c[6], t3 = c[3] + c[7];
  const float u0 = t2 + t0, u1 = t3 + t1;
  return u1 + u0;
}

// Same tree over 8 consecutive lanes (lane group g8 = lane & ~7 holds c[0..7]);
// every lane of the group gets the result.
__device__ __forceinline__ float tree8_lanes(float c, int v) {
  const float c4 = __shfl_xor(c, 4, 64);           // lanes v<4: c[v+4]
  const float t = c + c4;                            // t_v = c_v + c_{v+4} (v<4)
  const float t2 = __shfl_xor(t, 2, 64);           // v=0: t2 ; v=1: t3
  const float u = t2 + t;                            // u0 = t2+t0 (v=0), u1 = t3+t1 (v=1)
  const float u1 = __shfl_xor(u, 1, 64);           // v=0 gets u1
  const float res = u1 + u;                          // v=0: u1 + u0
  return __shfl(res, (threadIdx.x & 63) & ~7, 64);
}

// Parallel selection-with-swaps top-K over 192 scores held 3 per lane
// (expert e at lane e%64, slot e/64). Lane 0 writes ids[0..K).
__device__ void wave_topk(const float (&sc)[3], int lane, int K, int32_t *ids) {
  int pos[3] = {lane, lane + 64, lane + 128};
  bool sel[3] = {false, false, false};
  for (int k = 0; k < K; k++) {
    float bv = -__builtin_huge_valf();
    int bp = 0x7fffffff, be = -1;
#pragma unroll
    for (int m = 0; m < 3; m++) {
      if (!sel[m] && (sc[m] > bv || (sc[m] == bv && pos[m] < bp))) {
        bv = sc[m];
        bp = pos[m];
        be = lane + 64 * m;
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(bv, o, 64);
      const int op = __shfl_xor(bp, o, 64), oe = __shfl_xor(be, o, 64);
      if (ov > bv || (ov == bv && op < bp)) {
        bv = ov;
        bp = op;
        be = oe;
      }
    }
#pragma unroll
    for (int m = 0; m < 3; m++) {
      if (!sel[m] && pos[m] == k) pos[m] = bp;  // the element at position k moves
      if (lane + 64 * m == be) {
        sel[m] = true;
        pos[m] = k;
      }
    }
    if (lane == 0) ids[k] = be;
  }
}

// sigmoid, biased scores, top-K and weights of one token by one wave.
__device__ void route_from_logits(const float *lg, const float *bias, int has_bias, int K,
                                  float scale, int32_t *ids, float *wpre, float *wout,
                                  float *sg_l, int32_t *sel_ids) {
  const int lane = threadIdx.x & 63;
  float sc[3];
#pragma unroll
  for (int m = 0; m < 3; m++) {
    const int e = lane + 64 * m;
    const float sgm = sigmoid_c(lg[e]);
    sg_l[e] = sgm;
    sc[m] = has_bias ? sgm + bias[e] : sgm;
  }
  wave_topk(sc, lane, K, sel_ids);
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
  __builtin_amdgcn_wave_barrier();
  if (lane == 0) {
    float sum = 0.0f;
    for (int k = 0; k < K; k++) sum += sg_l[sel_ids[k]];
    const float inv = 1.0f / (sum + 1e-20f);
    for (int k = 0; k < K; k++) {
      const float v = sg_l[sel_ids[k]] * inv;
      ids[k] = sel_ids[k];
      wpre[k] = v;
      wout[k] = v * scale;
    }
  }
}

__device__ __forceinline__ void stage_store(__half *dst, int j, float v) {
  dst[stage_index(j)] = __float2half(v);
}

// ---------------------------------------------------------------------------
// Small T (decode): grid (192, T), one wave per (expert, token). The wave
// stages x, norm_w and the router row in LDS transposed by chain
// (buf[v][i] = a[8i+v]), lanes 0..7 run the eight sum-of-squares chains, then
// the eight logit chains. The last block of a token (atomic ticket) runs the
// top-K and resets the ticket, so the kernel can be relaunched or replayed
// without clearing memory. Block (0, t) also stages s for the expert kernels.
__global__ __launch_bounds__(64) void k_router_small(
    const float *__restrict__ x, const float *__restrict__ norm_w,
    const float *__restrict__ router, const float *__restrict__ bias, int has_bias, int K,
    float scale, float *logits, __half *__restrict__ s16, float *__restrict__ s32,
    int32_t *__restrict__ ids, float *__restrict__ wpre, float *__restrict__ wout,
    unsigned *__restrict__ tickets) {
  constexpr int NI = D / 8;  // 512 steps per chain
  __shared__ float4 xs[8][NI / 4], ws[8][NI / 4], rs[8][NI / 4];
  const int e = blockIdx.x, t = blockIdx.y, lane = threadIdx.x;
  const float4 *xg = reinterpret_cast<const float4 *>(x + (size_t)t * D);
  const float4 *wg = reinterpret_cast<const float4 *>(norm_w);
  const float4 *rg = reinterpret_cast<const float4 *>(router + (size_t)e * D);
  float *xsf = &xs[0][0].x, *wsf = &ws[0][0].x, *rsf = &rs[0][0].x;
#pragma unroll 4
  for (int q = lane; q < D / 4; q += 64) {
    const float4 a = xg[q], b = wg[q], c = rg[q];
    const int j = 4 * q, v = j & 7, i = j >> 3;  // j..j+3 share i; v = 0 or 4
    xsf[(v + 0) * NI + i] = a.x; xsf[(v + 1) * NI + i] = a.y;
    xsf[(v + 2) * NI + i] = a.z; xsf[(v + 3) * NI + i] = a.w;
    wsf[(v + 0) * NI + i] = b.x; wsf[(v + 1) * NI + i] = b.y;
    wsf[(v + 2) * NI + i] = b.z; wsf[(v + 3) * NI + i] = b.w;
    rsf[(v + 0) * NI + i] = c.x; rsf[(v + 1) * NI + i] = c.y;
    rsf[(v + 2) * NI + i] = c.z; rsf[(v + 3) * NI + i] = c.w;
  }
  __syncthreads();
  __shared__ float r_sh;
  if (lane < 8) {  // sum-of-squares chain `lane`
    float acc = 0.0f;
    const float4 *xv = xs[lane];
#pragma unroll 8
    for (int q = 0; q < NI / 4; q++) {
      const float4 a = xv[q];
      acc = __builtin_fmaf(a.x, a.x, acc);
      acc = __builtin_fmaf(a.y, a.y, acc);
      acc = __builtin_fmaf(a.z, a.z, acc);
      acc = __builtin_fmaf(a.w, a.w, acc);
    }
    const float ss = tree8_lanes(acc, lane);
    if (lane == 0) r_sh = 1.0f / __builtin_sqrtf(ss / 4096.0f + 1e-5f);
  }
  __syncthreads();
  const float r = r_sh;
  // s = (x*w)*r, in place over xs (chain-transposed)
  for (int q = lane; q < D; q += 64) xsf[q] = (xsf[q] * wsf[q]) * r;
  __syncthreads();
  if (e == 0) {  // stage s for the expert kernels (fp16 pair-staged and fp32)
    for (int j = lane; j < D; j += 64) {
      const float sv = xsf[(j & 7) * NI + (j >> 3)];
      stage_store(s16 + (size_t)t * D, j, sv);
      s32[(size_t)t * D + j] = sv;
    }
  }
  if (lane < 8) {  // logit chain `lane`
    float acc = 0.0f;
    const float4 *sv = xs[lane], *rv = rs[lane];
#pragma unroll 8
    for (int q = 0; q < NI / 4; q++) {
      const float4 a = rv[q], b = sv[q];
      acc = __builtin_fmaf(a.x, b.x, acc);
      acc = __builtin_fmaf(a.y, b.y, acc);
      acc = __builtin_fmaf(a.z, b.z, acc);
      acc = __builtin_fmaf(a.w, b.w, acc);
    }
    const float lg = tree8_lanes(acc, lane);
    if (lane == 0) {
      logits[(size_t)t * E + e] = lg;
      __threadfence();
    }
  }
  __shared__ int is_last;
  if (lane == 0) {
    const unsigned prev = __hip_atomic_fetch_add(&tickets[t], 1u, __ATOMIC_ACQ_REL,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    is_last = (prev == gridDim.x - 1);
  }
  __syncthreads();
  if (!is_last) return;
  __atomic_thread_fence(__ATOMIC_ACQUIRE);
  __shared__ float sg_l[E], lg_l[E];
  __shared__ int32_t sel_ids[KMAX];
  for (int ee = lane; ee < E; ee += 64) lg_l[ee] = logits[(size_t)t * E + ee];
  __syncthreads();
  route_from_logits(lg_l, bias, has_bias, K, scale, ids + (size_t)t * K, wpre + (size_t)t * K,
                    wout + (size_t)t * K, sg_l, sel_ids);
  if (lane == 0) tickets[t] = 0u;
}

// ---------------------------------------------------------------------------
// Large T: (1) RMSNorm per token, one wave per token (chains over LDS);
// (2) router GEMM, LDS-tiled SIMT, each output keeping its eight chains;
// (3) top-K, one wave per token.
__global__ __launch_bounds__(64) void k_rmsnorm(const float *__restrict__ x,
                                                const float *__restrict__ norm_w,
                                                __half *__restrict__ s16,
                                                float *__restrict__ s32) {
  constexpr int NI = D / 8;
  __shared__ float4 xs[8][NI / 4];
  const int t = blockIdx.x, lane = threadIdx.x;
  const float4 *xg = reinterpret_cast<const float4 *>(x + (size_t)t * D);
  float *xsf = &xs[0][0].x;
  for (int q = lane; q < D / 4; q += 64) {
    const float4 a = xg[q];
    const int j = 4 * q, v = j & 7, i = j >> 3;
    xsf[(v + 0) * NI + i] = a.x; xsf[(v + 1) * NI + i] = a.y;
    xsf[(v + 2) * NI + i] = a.z; xsf[(v + 3) * NI + i] = a.w;
  }
  __syncthreads();
  __shared__ float r_sh;
  if (lane < 8) {
    float acc = 0.0f;
    const float4 *xv = xs[lane];
#pragma unroll 8
    for (int q = 0; q < NI / 4; q++) {
      const float4 a = xv[q];
      acc = __builtin_fmaf(a.x, a.x, acc);
      acc = __builtin_fmaf(a.y, a.y, acc);
      acc = __builtin_fmaf(a.z, a.z, acc);
      acc = __builtin_fmaf(a.w, a.w, acc);
    }
    const float ss = tree8_lanes(acc, lane);
    if (lane == 0) r_sh = 1.0f / __builtin_sqrtf(ss / 4096.0f + 1e-5f);
  }
  __syncthreads();
  const float r = r_sh;
  for (int j = lane; j < D; j += 64) {
    const float sv = (x[(size_t)t * D + j] * norm_w[j]) * r;
    s32[(size_t)t * D + j] = sv;
    stage_store(s16 + (size_t)t * D, j, sv);
  }
}

// logits[T x 192] = s[T x 4096] . router^T, block tile 32 tokens x 64 experts,
// thread tile 4 tokens x 2 experts x 8 chains. K is walked in chunks of 64
// elements (8 chain steps) staged in LDS; every chain runs i ascending.
__global__ __launch_bounds__(256) void k_router_gemm(const float *__restrict__ s32,
                                                     const float *__restrict__ router, int T,
                                                     float *__restrict__ logits) {
  constexpr int TT = 32, TE = 64, KC = 64;
  __shared__ float4 sl[TT][KC / 4 + 1], wl[TE][KC / 4 + 1];
  const int t0 = blockIdx.x * TT, e0 = blockIdx.y * TE;
  const int tid = threadIdx.x, tg = tid & 7, eg = tid >> 3;  // 8 token groups x 32 expert groups
  float acc[4][2][8];
#pragma unroll
  for (int a = 0; a < 4; a++)
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
      for (int v = 0; v < 8; v++) acc[a][b][v] = 0.0f;
  for (int k0 = 0; k0 < D; k0 += KC) {
    // stage: 32x64 s (512 float4) and 64x64 router (1024 float4)
    for (int q = tid; q < TT * KC / 4; q += 256) {
      const int rr = q / (KC / 4), cc = q % (KC / 4), tt = t0 + rr;
      sl[rr][cc] = tt < T ? reinterpret_cast<const float4 *>(s32 + (size_t)tt * D + k0)[cc]
                          : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    for (int q = tid; q < TE * KC / 4; q += 256) {
      const int rr = q / (KC / 4), cc = q % (KC / 4);
      wl[rr][cc] = reinterpret_cast<const float4 *>(router + (size_t)(e0 + rr) * D + k0)[cc];
    }
    __syncthreads();
#pragma unroll
    for (int ii = 0; ii < KC / 8; ii++) {  // chain step: elements 8ii .. 8ii+7 of the chunk
      float4 sa[4][2], wb[2][2];
#pragma unroll
      for (int a = 0; a < 4; a++) {
        sa[a][0] = sl[tg + 8 * a][2 * ii];
        sa[a][1] = sl[tg + 8 * a][2 * ii + 1];
      }
#pragma unroll
      for (int b = 0; b < 2; b++) {
        wb[b][0] = wl[eg + 32 * b][2 * ii];
        wb[b][1] = wl[eg + 32 * b][2 * ii + 1];
      }
#pragma unroll
      for (int a = 0; a < 4; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) {
          acc[a][b][0] = __builtin_fmaf(wb[b][0].x, sa[a][0].x, acc[a][b][0]);
          acc[a][b][1] = __builtin_fmaf(wb[b][0].y, sa[a][0].y, acc[a][b][1]);
          acc[a][b][2] = __builtin_fmaf(wb[b][0].z, sa[a][0].z, acc[a][b][2]);
          acc[a][b][3] = __builtin_fmaf(wb[b][0].w, sa[a][0].w, acc[a][b][3]);
          acc[a][b][4] = __builtin_fmaf(wb[b][1].x, sa[a][1].x, acc[a][b][4]);
          acc[a][b][5] = __builtin_fmaf(wb[b][1].y, sa[a][1].y, acc[a][b][5]);
          acc[a][b][6] = __builtin_fmaf(wb[b][1].z, sa[a][1].z, acc[a][b][6]);
          acc[a][b][7] = __builtin_fmaf(wb[b][1].w, sa[a][1].w, acc[a][b][7]);
        }
    }
    __syncthreads();
  }
#pragma unroll
  for (int a = 0; a < 4; a++)
#pragma unroll
    for (int b = 0; b < 2; b++) {
      const int tt = t0 + tg + 8 * a, ee = e0 + eg + 32 * b;
      if (tt < T) logits[(size_t)tt * E + ee] = tree8(acc[a][b]);
    }
}

__global__ __launch_bounds__(64) void k_topk(const float *__restrict__ logits,
                                             const float *__restrict__ bias, int has_bias, int K,
                                             float scale, int32_t *__restrict__ ids,
                                             float *__restrict__ wpre, float *__restrict__ wout) {
  const int t = blockIdx.x;
  __shared__ float sg_l[E], lg_l[E];
  __shared__ int32_t sel_ids[KMAX];
  for (int e = threadIdx.x; e < E; e += 64) lg_l[e] = logits[(size_t)t * E + e];
  __syncthreads();
  route_from_logits(lg_l, bias, has_bias, K, scale, ids + (size_t)t * K, wpre + (size_t)t * K,
                    wout + (size_t)t * K, sg_l, sel_ids);
}

// Device dispatch: per-expert slot lists and the work-tile list, one block.
// Slots: s < T*K is (token s/K, rank s%K) of a routed expert; s = T*K + t is
// token t of the shared expert (index E), which every token uses.
// tiles[i] = {expert, first list index, count <= NT, 0}.
__global__ __launch_bounds__(1024) void k_dispatch(const int32_t *__restrict__ ids, int T, int K,
                                                   int NT, int32_t *__restrict__ list,
                                                   int4 *__restrict__ tiles,
                                                   int32_t *__restrict__ n_tiles, int max_tiles,
                                                   int32_t *__restrict__ counts_out,
                                                   unsigned long long *__restrict__ stats) {
  __shared__ int cnt[E + 1], off[E + 2], cur[E + 1], toff[E + 2];
  const int tid = threadIdx.x, n = T * K;
  for (int e = tid; e <= E; e += blockDim.x) {
    cnt[e] = 0;
    cur[e] = 0;
  }
  __syncthreads();
  for (int i = tid; i < n; i += blockDim.x) {
    const int e = ids[i];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  if (tid == 0) cnt[E] = T;
  __syncthreads();
  if (tid == 0) {
    int a = 0, b = 0;
    for (int e = 0; e <= E; e++) {
      off[e] = a;
      toff[e] = b;
      a += cnt[e];
      b += (cnt[e] + NT - 1) / NT;
    }
    off[E + 1] = a;
    toff[E + 1] = b;
    *n_tiles = b < max_tiles ? b : max_tiles;
    if (stats) {  // forwards, experts touched (shared included)
      int active = 0;
      for (int e = 0; e <= E; e++) active += cnt[e] > 0;
      stats[0] += 1ull;
      stats[1] += (unsigned long long)active;
    }
  }
  __syncthreads();
  for (int i = tid; i < n; i += blockDim.x) {
    const int e = ids[i];
    if (e >= 0 && e < E) list[off[e] + atomicAdd(&cur[e], 1)] = i;
  }
  for (int t = tid; t < T; t += blockDim.x) list[off[E] + t] = n + t;
  for (int e = tid; e <= E; e += blockDim.x) {
    if (counts_out) counts_out[e] = cnt[e];
    const int c = cnt[e];
    for (int j = 0, ti = toff[e]; j * NT < c && ti < max_tiles; j++, ti++)
      tiles[ti] = make_int4(e, off[e] + j * NT, min(NT, c - j * NT), 0);
  }
}

}  // namespace hy3x
