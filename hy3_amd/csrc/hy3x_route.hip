// hy3x_route.hip -- RMSNorm + router + top-K for T >= 2, and the device
// dispatch (the single-token router launch is hy3x_route_decode.hip).
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
#include "hy3x_kernels.h"
#include "hy3x_route.h"
#include "hy3x_router_block.h"
#include "hy3x_q4k.h"

#pragma clang fp contract(off)

namespace hy3x {

__global__ __launch_bounds__(256) void k_router_logits(
    const float *__restrict__ x, const float *__restrict__ xadd, const float *__restrict__ norm_w,
    const float *__restrict__ router, const float *__restrict__ bias, int has_bias,
    float *__restrict__ logits, float *__restrict__ sig, float *__restrict__ score,
    __half *__restrict__ s16, float *__restrict__ s32, unsigned long long *trace, int T,
    uint32_t *__restrict__ bits, int wt, const float *__restrict__ r_in) {
  if (bits) dispatch_clear_part(T, bits, wt, blockIdx.y * E + blockIdx.x, E * T);
  router_block(blockIdx.x, blockIdx.y, x, xadd, norm_w, router, bias, has_bias, logits, sig,
               score, s16, s32, trace, r_in);
}

// ---------------------------------------------------------------------------
// Large T: (1) RMSNorm per token, one wave per token (chains over LDS);
// (2) router GEMM, LDS-tiled SIMT, each output keeping its eight chains;
// (3) top-K, one wave per token.
__global__ __launch_bounds__(256) void k_rmsnorm(const float *__restrict__ x,
                                                 const float *__restrict__ xadd,
                                                 const float *__restrict__ norm_w,
                                                 __half *__restrict__ s16,
                                                 float *__restrict__ s32,
                                                 __half *__restrict__ s16m,
                                                 __half *__restrict__ ssum, int T,
                                                 uint32_t *__restrict__ bits, int wt,
                                                 const float *__restrict__ r_in) {
  const int t = blockIdx.x, tid = threadIdx.x;
  if (bits) dispatch_clear_part(T, bits, wt, t, T);
  const float *xt = x + (size_t)t * D, *at = xadd ? xadd + (size_t)t * D : nullptr;
  const float4 *wg = reinterpret_cast<const float4 *>(norm_w);
  float4 a[4];
#pragma unroll
  for (int u = 0; u < 4; u++) a[u] = load_x4(xt, at, tid + 256 * u);
  __shared__ float red_l[4];
  const float ss = block_sumsq(a, red_l);
  const float r = r_in ? r_in[t] : 1.0f / __builtin_sqrtf(ss / 4096.0f + 1e-5f);
#pragma unroll
  for (int u = 0; u < 4; u++) {
    const float4 w = wg[tid + 256 * u];
    const int j = 4 * (tid + 256 * u);
    const float4 sv = make_float4((a[u].x * w.x) * r, (a[u].y * w.y) * r, (a[u].z * w.z) * r,
                                  (a[u].w * w.w) * r);
    reinterpret_cast<float4 *>(s32 + (size_t)t * D)[tid + 256 * u] = sv;
    if (s16) {
      stage_store(s16 + (size_t)t * D, j + 0, sv.x);
      stage_store(s16 + (size_t)t * D, j + 1, sv.y);
      stage_store(s16 + (size_t)t * D, j + 2, sv.z);
      stage_store(s16 + (size_t)t * D, j + 3, sv.w);
    }
    if (s16m) {  // fp16 in the MFMA run order (perm8: j + (0, 2, 1, 3)), one 8-byte store
      const __half2 a01 = __halves2half2(__float2half(sv.x), __float2half(sv.z));
      const __half2 a23 = __halves2half2(__float2half(sv.y), __float2half(sv.w));
      uint2 v;
      v.x = __builtin_bit_cast(uint32_t, a01);
      v.y = __builtin_bit_cast(uint32_t, a23);
      *reinterpret_cast<uint2 *>(s16m + (size_t)t * D + j) = v;
    }
  }
  if (s16m) {  // and its sub-block sums
    __syncthreads();
    row_subsums(s16m + (size_t)t * D, D / 32, ssum + (size_t)t * (D / 32) * 4);
  }
}

// logits[T x 192] = s[T x 4096] . router^T for T > 8, in the router's fixed
// summation order: 8 chains per output, chain v = fmaf over elements 8i + v
// with i ascending, then tree8 (the order of hy3.c's vectorised fast-math
// mul_mat_f32, hy3.c:1076-1085). A thread runs ONE chain v for an MT x ME
// micro-tile of (token, expert) outputs; the 8 chains of a micro-tile sit in
// 8 neighbouring lanes and are combined with tree8_lanes. Block tile:
// TT = MT*TG tokens x TE = ME*EG experts, K walked in chunks of KC staged
// k-major in LDS (double-buffered, next chunk prefetched into registers). The
// chunk is large (few blocks run at small T, so each K step's load latency is
// paid in sequence: the fewer steps, the better).
template <int MT, int ME, int TG, int EG, int KC, int R>
__global__ __launch_bounds__(256) void k_router_gemm(const float *__restrict__ s32,
                                                     const float *__restrict__ router, int T,
                                                     float *__restrict__ logits) {
  static_assert(8 * TG * EG == 256, "256 threads");
  static_assert(D % KC == 0 && KC % 8 == 0, "K chunks");
  constexpr int NCH = D / KC;
  static_assert(R >= 1 && NCH % R == 0, "whole rounds of the fetch ring");
  constexpr int TT = MT * TG, TE = ME * EG;
  constexpr int SP = TT + 4, WP = TE + 4;        // padded LDS rows (floats)
  constexpr int NS = TT * KC / 4 / 256, NW = TE * KC / 4 / 256;  // float4 per thread
  static_assert(NS >= 1 && NW >= 1, "staging split");
  __shared__ float sl[2][KC][SP], wl[2][KC][WP];
  const int t0 = blockIdx.x * TT, e0 = blockIdx.y * TE;
  const int tid = threadIdx.x, v = tid & 7, mt = tid >> 3, tg = mt % TG, eg = mt / TG;
  // a register ring of R chunks in flight (the loop is unrolled by R so that
  // the ring slots stay static)
  float4 sn[R][NS], wn[R][NW];
  // Loads are unconditional (rows past T read row T - 1 and are zeroed when
  // staged; fetches past the end re-read the last chunk), so that the wait
  // counters stay exact through the ring and no fetch waits on a later one.
  auto fetch = [&](int k0, float4(&sd)[NS], float4(&wd)[NW]) {
#pragma unroll
    for (int u = 0; u < NS; u++) {
      const int q = tid + 256 * u, r = q % TT, c = q / TT, tt = t0 + r;
      sd[u] = reinterpret_cast<const float4 *>(s32 + (size_t)(tt < T ? tt : T - 1) * D + k0)[c];
    }
#pragma unroll
    for (int u = 0; u < NW; u++) {
      const int q = tid + 256 * u, r = q % TE, c = q / TE;
      wd[u] = reinterpret_cast<const float4 *>(router + (size_t)(e0 + r) * D + k0)[c];
    }
  };
  auto stage = [&](int buf, const float4(&sd)[NS], const float4(&wd)[NW]) {
#pragma unroll
    for (int u = 0; u < NS; u++) {  // neighbouring lanes write neighbouring words
      const int q = tid + 256 * u, r = q % TT, c = q / TT;
      const bool in = t0 + r < T;
      sl[buf][4 * c + 0][r] = in ? sd[u].x : 0.0f;
      sl[buf][4 * c + 1][r] = in ? sd[u].y : 0.0f;
      sl[buf][4 * c + 2][r] = in ? sd[u].z : 0.0f;
      sl[buf][4 * c + 3][r] = in ? sd[u].w : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < NW; u++) {
      const int q = tid + 256 * u, r = q % TE, c = q / TE;
      wl[buf][4 * c + 0][r] = wd[u].x;
      wl[buf][4 * c + 1][r] = wd[u].y;
      wl[buf][4 * c + 2][r] = wd[u].z;
      wl[buf][4 * c + 3][r] = wd[u].w;
    }
  };
  float acc[MT][ME];
#pragma unroll
  for (int a = 0; a < MT; a++)
#pragma unroll
    for (int b = 0; b < ME; b++) acc[a][b] = 0.0f;
#pragma unroll
  for (int r = 0; r < R; r++) fetch(r * KC, sn[r], wn[r]);
  for (int it0 = 0; it0 < NCH; it0 += R) {
#pragma unroll
    for (int r = 0; r < R; r++) {
      const int it = it0 + r, buf = it & 1;
      stage(buf, sn[r], wn[r]);
      __syncthreads();  // buf staged; the other buffer is no longer read
      fetch((it + R < NCH ? it + R : NCH - 1) * KC, sn[r], wn[r]);
#pragma unroll 4
      for (int ii = 0; ii < KC / 8; ii++) {
        const int k = 8 * ii + v;
        float sv[MT], wv[ME];
#pragma unroll
        for (int a = 0; a < MT; a++) sv[a] = sl[buf][k][MT * tg + a];
#pragma unroll
        for (int b = 0; b < ME; b++) wv[b] = wl[buf][k][ME * eg + b];
#pragma unroll
        for (int a = 0; a < MT; a++)
#pragma unroll
          for (int b = 0; b < ME; b++) acc[a][b] = __builtin_fmaf(wv[b], sv[a], acc[a][b]);
      }
    }
  }
#pragma unroll
  for (int a = 0; a < MT; a++)
#pragma unroll
    for (int b = 0; b < ME; b++) {
      const float lg = tree8_lanes(acc[a][b], v);
      const int tt = t0 + MT * tg + a, ee = e0 + ME * eg + b;
      if (v == 0 && tt < T) logits[(size_t)tt * E + ee] = lg;
    }
}
template __global__ void HY3X_ROUTER_GEMM(TINY)(const float *, const float *, int, float *);
template __global__ void HY3X_ROUTER_GEMM(MID)(const float *, const float *, int, float *);
template __global__ void HY3X_ROUTER_GEMM(LARGE)(const float *, const float *, int, float *);
template __global__ void HY3X_ROUTER_GEMM(XL)(const float *, const float *, int, float *);
template __global__ void HY3X_ROUTER_GEMM(XXL)(const float *, const float *, int, float *);

// Routing of one token per wave (T > 1 paths), a block holding 1 or 4 waves: sigmoid and
// score of the 192 logits (expert lane + 64 m in slot m), the top-K in
// registers (topk_wave_fast, or topk_wave_regs on a tie or NaN), then the
// token's bit in each of its experts' dispatch bitmaps.
__global__ __launch_bounds__(256) void k_topk(const float *__restrict__ logits,
                                              const float *__restrict__ bias, int has_bias, int K,
                                              float scale, int T, int32_t *__restrict__ ids,
                                              float *__restrict__ wpre, float *__restrict__ wout,
                                              uint32_t *__restrict__ bits, int wt,
                                              uint8_t *__restrict__ ranks) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (t >= T) return;  // whole waves
  float sg[3], sc[3];
#pragma unroll
  for (int m = 0; m < 3; m++) {
    const int e = lane + 64 * m;
    sg[m] = sigmoid_c(logits[(size_t)t * E + e]);
    sc[m] = has_bias ? sg[m] + bias[e] : sg[m];
  }
  int32_t *ids_t = ids + (size_t)t * K;
  int my_e;
  float my_sig, sum;
  if (topk_wave_fast(sc, sg, K, my_e, my_sig, sum)) {
    if (lane < K) {
      const float inv = 1.0f / (sum + 1e-20f);
      const float v = my_sig * inv;
      ids_t[lane] = my_e;
      wpre[(size_t)t * K + lane] = v;
      wout[(size_t)t * K + lane] = v * scale;
    }
  } else {
    topk_wave_regs(sc, sg, K, scale, ids_t, wpre + (size_t)t * K, wout + (size_t)t * K);
    my_e = lane < K ? ids_t[lane] : 0;  // this lane's own store: program order
  }
  if (bits && lane < K) {
    atomicOr(&bits[(size_t)my_e * wt + (t >> 5)], 1u << (t & 31));
    ranks[(size_t)my_e * wt * 32 + t] = (uint8_t)lane;  // lane k holds place k
  }
}

// Device dispatch: per-expert slot lists and the work-tile list.
// Slots: s < T*K is (token s/K, rank s%K) of a routed expert; s = T*K + t is
// token t of the shared expert (index E), which every token uses. Each
// expert's slots are listed in token order, so the lists (and the tiles, and
// every result computed from them) do not depend on scheduling.
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

// Dispatch lists from the bitmaps k_topk marked, one block per expert (E + 1
// blocks, the last is the shared expert): list offset and first tile from exclusive scans of all counts, the expert's
// tiles, and its slots in token order from its bitmap (popcount prefix sums).
// Block E also writes the tile count, the per-expert counts and the stats.
__global__ __launch_bounds__(256) void k_dispatch_list(
    const uint8_t *__restrict__ ranks, int T, int K, int NT, const uint32_t *__restrict__ bits,
    int wt, int32_t *__restrict__ list,
    int4 *__restrict__ tiles, int32_t *__restrict__ n_tiles, int max_tiles,
    int32_t *__restrict__ counts_out, unsigned long long *__restrict__ stats) {
  __shared__ int tmp[8], off_l, toff_l, ce_l;
  const int e = blockIdx.x, tid = threadIdx.x;
  const int nw = (T + 31) >> 5;
  // expert tid's count: the popcount of its token bitmap (every block forms
  // all counts itself; no counter atomics in the marking step)
  int c = tid == E ? T : 0;
  if (tid < E) {  // rows are 16-byte aligned (wt % 4 == 0); words past nw are not counted
    const uint4 *row = reinterpret_cast<const uint4 *>(bits + (size_t)tid * wt);
    for (int q = 0; 4 * q < nw; q++) {
      const uint4 v = row[q];
      const int w = 4 * q;
      c += __popc(v.x) + (w + 1 < nw ? __popc(v.y) : 0) + (w + 2 < nw ? __popc(v.z) : 0) +
           (w + 3 < nw ? __popc(v.w) : 0);
    }
  }
  const int off = block_exclusive_scan256(c, tmp);
  const int nt = (c + NT - 1) / NT;
  const int toff = block_exclusive_scan256(nt, tmp);
  if (tid == e) {
    off_l = off;
    toff_l = toff;
    ce_l = c;
  }
  if (e == E) {
    const int active = block_exclusive_scan256(c > 0 ? 1 : 0, tmp);
    if (tid == 255) {
      *n_tiles = toff < max_tiles ? toff : max_tiles;
      if (stats) {  // forwards, experts touched (shared included)
        stats[0] += 1ull;
        stats[1] += (unsigned long long)active;
      }
    }
    if (counts_out && tid <= E) counts_out[tid] = c;
  }
  __syncthreads();
  const int eoff = off_l, etoff = toff_l, ce = ce_l;
  for (int j = tid; j * NT < ce; j += 256)
    if (etoff + j < max_tiles) tiles[etoff + j] = make_int4(e, eoff + j * NT, min(NT, ce - j * NT), 0);
  if (e == E) {
    for (int t = tid; t < T; t += 256) list[eoff + t] = T * K + t;
    return;
  }
  int base = 0;
  for (int w0 = 0; w0 < nw; w0 += 256) {  // rounds of 256 bitmap words, in order
    const int w = w0 + tid;
    uint32_t word = w < nw ? bits[(size_t)e * wt + w] : 0u;
    // the word's 32 tokens' places of e (k_topk's rank bytes; read only where
    // the bit is set), in two 16-byte loads issued with the bitmap word's
    uint4 rk[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
    if (word) {
      const uint4 *rp = reinterpret_cast<const uint4 *>(ranks + (size_t)e * wt * 32 + 32 * w);
      rk[0] = rp[0];
      rk[1] = rp[1];
    }
    const int pos = base + block_exclusive_scan256(__popc(word), tmp);
    int r = 0;
    while (word) {
      const int b = __ffs(word) - 1;
      word &= word - 1u;
      const int t = 32 * w + b;
      // byte b of the 32 (a select chain: an indexed read of a register
      // array would go through scratch memory)
      const int q = b >> 2;
      const uint4 h = q < 4 ? rk[0] : rk[1];
      const int qq = q & 3;
      const uint32_t wsel = qq == 0 ? h.x : qq == 1 ? h.y : qq == 2 ? h.z : h.w;
      const int k = (int)((wsel >> (8 * (b & 3))) & 0xffu);
      list[eoff + pos + r] = t * K + k;
      r++;
    }
    if (tid == 255) tmp[4] = pos + r;  // round total (tmp[0..3] belong to the scan)
    __syncthreads();
    base = tmp[4];
    __syncthreads();
  }
}

}  // namespace hy3x
