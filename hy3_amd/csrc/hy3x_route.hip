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
#include "hy3x_route.h"

#pragma clang fp contract(off)

namespace hy3x {

// Chain-transposed LDS rows: buf[v*RS + i] = a[8i+v]. RS = 512 + 4 keeps the
// eight chains' float4 reads on distinct banks.
constexpr int NI = D / 8;  // 512 steps per chain
constexpr int RS = NI + 4;

__device__ __forceinline__ void load_transposed(const float *src, float *buf, int lane,
                                                int nthreads) {
  const float4 *g = reinterpret_cast<const float4 *>(src);
#pragma unroll 4
  for (int q = lane; q < D / 4; q += nthreads) {
    const float4 a = g[q];
    const int j = 4 * q, v = j & 7, i = j >> 3;  // j..j+3 share i; v = 0 or 4
    buf[(v + 0) * RS + i] = a.x;
    buf[(v + 1) * RS + i] = a.y;
    buf[(v + 2) * RS + i] = a.z;
    buf[(v + 3) * RS + i] = a.w;
  }
}

// One fmaf chain over a chain-transposed row pair (512 steps).
__device__ __forceinline__ float chain_dot(const float *a, const float *b) {
  const float4 *av = reinterpret_cast<const float4 *>(a);
  const float4 *bv = reinterpret_cast<const float4 *>(b);
  float acc = 0.0f;
#pragma unroll 16
  for (int q = 0; q < NI / 4; q++) {
    const float4 x = av[q], y = bv[q];
    acc = __builtin_fmaf(x.x, y.x, acc);
    acc = __builtin_fmaf(x.y, y.y, acc);
    acc = __builtin_fmaf(x.z, y.z, acc);
    acc = __builtin_fmaf(x.w, y.w, acc);
  }
  return acc;
}

// ---------------------------------------------------------------------------
// Small T (decode): grid (192, T), one wave per (expert, token). The wave
// stages x, norm_w and the router row in LDS transposed by chain
// (buf[v][i] = a[8i+v]), lanes 0..7 run the eight sum-of-squares chains, then
// the eight logit chains. The last block of a token (atomic ticket) runs the
// top-K and resets the ticket, so the kernel can be relaunched or replayed
// without clearing memory. Block (0, t) also stages s for the expert kernels.
__global__ __launch_bounds__(256) void k_router_logits(
    const float *__restrict__ x, const float *__restrict__ norm_w,
    const float *__restrict__ router, const float *__restrict__ bias, int has_bias,
    float *__restrict__ logits, float *__restrict__ sig, float *__restrict__ score,
    __half *__restrict__ s16, float *__restrict__ s32, unsigned long long *trace) {
  __shared__ __attribute__((aligned(16))) float xsf[8 * RS], wsf[8 * RS], rsf[8 * RS];
  const int e = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
  trace_point(trace, 0);
  float r_blk;
  {  // every load in flight at once: 4 float4 of each row per thread
    const float4 *xg = reinterpret_cast<const float4 *>(x + (size_t)t * D);
    const float4 *wg = reinterpret_cast<const float4 *>(norm_w);
    const float4 *rg = reinterpret_cast<const float4 *>(router + (size_t)e * D);
    float4 a[4], b[4], c[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      a[u] = xg[tid + 256 * u];
      b[u] = wg[tid + 256 * u];
      c[u] = rg[tid + 256 * u];
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int j = 4 * (tid + 256 * u), v = j & 7, i = j >> 3;
      xsf[(v + 0) * RS + i] = a[u].x; xsf[(v + 1) * RS + i] = a[u].y;
      xsf[(v + 2) * RS + i] = a[u].z; xsf[(v + 3) * RS + i] = a[u].w;
      wsf[(v + 0) * RS + i] = b[u].x; wsf[(v + 1) * RS + i] = b[u].y;
      wsf[(v + 2) * RS + i] = b[u].z; wsf[(v + 3) * RS + i] = b[u].w;
      rsf[(v + 0) * RS + i] = c[u].x; rsf[(v + 1) * RS + i] = c[u].y;
      rsf[(v + 2) * RS + i] = c[u].z; rsf[(v + 3) * RS + i] = c[u].w;
    }
    __shared__ float red_l[4];
    const float ss = block_sumsq(a, red_l);  // contains the barrier for the LDS rows
    r_blk = 1.0f / __builtin_sqrtf(ss / 4096.0f + 1e-5f);
  }
  trace_point(trace, 1);
  const float r = r_blk;
  for (int q = tid; q < 8 * RS; q += 256) xsf[q] = (xsf[q] * wsf[q]) * r;  // s, in place
  __syncthreads();
  if (tid < 8) {  // logit chain `tid`
    const float lg = tree8_lanes(chain_dot(rsf + tid * RS, xsf + tid * RS), tid);
    if (tid == 0) {
      const float sg = sigmoid_c(lg);
      logits[(size_t)t * E + e] = lg;
      sig[(size_t)t * E + e] = sg;
      score[(size_t)t * E + e] = has_bias ? sg + bias[e] : sg;
    }
    trace_point(trace, 3);
  } else if (e == 0) {  // stage s for the expert kernels (fp16 pair-staged and fp32)
    for (int j = tid - 8; j < D; j += 248) {
      const float sv = xsf[(j & 7) * RS + (j >> 3)];
      stage_store(s16 + (size_t)t * D, j, sv);
      s32[(size_t)t * D + j] = sv;
    }
  }
}

// ---------------------------------------------------------------------------
// Large T: (1) RMSNorm per token, one wave per token (chains over LDS);
// (2) router GEMM, LDS-tiled SIMT, each output keeping its eight chains;
// (3) top-K, one wave per token.
__global__ __launch_bounds__(256) void k_rmsnorm(const float *__restrict__ x,
                                                 const float *__restrict__ norm_w,
                                                 __half *__restrict__ s16,
                                                 float *__restrict__ s32) {
  const int t = blockIdx.x, tid = threadIdx.x;
  const float4 *xg = reinterpret_cast<const float4 *>(x + (size_t)t * D);
  const float4 *wg = reinterpret_cast<const float4 *>(norm_w);
  float4 a[4];
#pragma unroll
  for (int u = 0; u < 4; u++) a[u] = xg[tid + 256 * u];
  __shared__ float red_l[4];
  const float r = 1.0f / __builtin_sqrtf(block_sumsq(a, red_l) / 4096.0f + 1e-5f);
#pragma unroll
  for (int u = 0; u < 4; u++) {
    const float4 w = wg[tid + 256 * u];
    const int j = 4 * (tid + 256 * u);
    const float4 sv = make_float4((a[u].x * w.x) * r, (a[u].y * w.y) * r, (a[u].z * w.z) * r,
                                  (a[u].w * w.w) * r);
    reinterpret_cast<float4 *>(s32 + (size_t)t * D)[tid + 256 * u] = sv;
    stage_store(s16 + (size_t)t * D, j + 0, sv.x);
    stage_store(s16 + (size_t)t * D, j + 1, sv.y);
    stage_store(s16 + (size_t)t * D, j + 2, sv.z);
    stage_store(s16 + (size_t)t * D, j + 3, sv.w);
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

// Routing of one token per block (large-T path): sigmoid and scores of the
// 192 logits, then the top-K.
__global__ __launch_bounds__(256) void k_topk(const float *__restrict__ logits,
                                              const float *__restrict__ bias, int has_bias, int K,
                                              float scale, int32_t *__restrict__ ids,
                                              float *__restrict__ wpre, float *__restrict__ wout) {
  const int t = blockIdx.x;
  __shared__ __attribute__((aligned(16))) float sg[E], sc[E], sc_l[E], sg_l[E];
  __shared__ int32_t scratch_l[4 * E + 2 * KMAX + 2];
  for (int e = threadIdx.x; e < E; e += 256) {
    const float v = sigmoid_c(logits[(size_t)t * E + e]);
    sg[e] = v;
    sc[e] = has_bias ? v + bias[e] : v;
  }
  __syncthreads();
  topk_block(sg, sc, K, scale, ids + (size_t)t * K, wpre + (size_t)t * K, wout + (size_t)t * K,
             sc_l, sg_l, scratch_l);
}

// Device dispatch: per-expert slot lists and the work-tile list, one block of
// 256 threads (four waves; expert e is handled by thread e).
// Slots: s < T*K is (token s/K, rank s%K) of a routed expert; s = T*K + t is
// token t of the shared expert (index E), which every token uses.
// tiles[i] = {expert, first list index, count <= NT, 0}.
__device__ __forceinline__ int block_exclusive_scan256(int v, int *tmp) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  if (lane == 63) tmp[wave] = incl;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; w++) base += tmp[w];
  __syncthreads();
  return base + incl - v;
}

__global__ __launch_bounds__(256) void k_dispatch(const int32_t *__restrict__ ids, int T, int K,
                                                  int NT, int32_t *__restrict__ list,
                                                  int4 *__restrict__ tiles,
                                                  int32_t *__restrict__ n_tiles, int max_tiles,
                                                  int32_t *__restrict__ counts_out,
                                                  unsigned long long *__restrict__ stats) {
  __shared__ int cnt[256], cur[256], tmp[8];
  const int tid = threadIdx.x, n = T * K;
  cnt[tid] = 0;
  cur[tid] = 0;
  __syncthreads();
  for (int i = tid; i < n; i += 256) {
    const int e = ids[i];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  const int c = tid < E ? cnt[tid] : (tid == E ? T : 0);
  const int off = block_exclusive_scan256(c, tmp);
  const int nt = (c + NT - 1) / NT;
  const int toff = block_exclusive_scan256(nt, tmp);
  const int active = block_exclusive_scan256(c > 0 ? 1 : 0, tmp);
  if (tid == 255) {
    *n_tiles = toff < max_tiles ? toff : max_tiles;
    if (stats) {  // forwards, experts touched (shared included)
      stats[0] += 1ull;
      stats[1] += (unsigned long long)active;
    }
  }
  __shared__ int offs[256];
  offs[tid] = off;
  __syncthreads();
  for (int i = tid; i < n; i += 256) {
    const int e = ids[i];
    if (e >= 0 && e < E) list[offs[e] + atomicAdd(&cur[e], 1)] = i;
  }
  for (int t = tid; t < T; t += 256) list[offs[E] + t] = n + t;
  if (tid <= E) {
    if (counts_out) counts_out[tid] = c;
    for (int j = 0, ti = toff; j * NT < c && ti < max_tiles; j++, ti++)
      tiles[ti] = make_int4(tid, off + j * NT, min(NT, c - j * NT), 0);
  }
}

}  // namespace hy3x
