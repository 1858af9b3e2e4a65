// hy3x_router_block.h -- one router logit of one token per block, in the
// routing contract's exact order (the 8 fmaf chains and tree8 of
// hy3x_route.h), shared by the 2-8 token router (k_router_logits,
// hy3x_route.hip) and the single-token router launch (k_route_decode,
// hy3x_route_decode.hip).
#pragma once
#include "hy3x_kernels.h"
#include "hy3x_route.h"

namespace hy3x {

// Chain-transposed LDS rows: buf[v*RS + i] = a[8i+v]. RS = 512 + 4 keeps the
// eight chains' float4 reads on distinct banks.
constexpr int NI = D / 8;  // 512 steps per chain
constexpr int RS = NI + 4;

// The eight fmaf chains of one logit over chain-transposed row pairs (512
// steps each, i ascending), with their operands in registers spread over a
// whole wave: lane 8 g + v holds steps [64 g, 64 g + 64) of chain v (64
// router and 64 s values). The wave runs 8 rounds of 64 FMAs; in round g the
// lanes of segment g continue chain v from the accumulator the lanes of
// segment g - 1 left (moved up 8 lanes between rounds); the other lanes'
// results are discarded. The chain is bound by the dependent FMA latency, and
// no FMA waits on LDS (8 lanes each running a whole chain from LDS took about
// 1.5 times as long). Returns chain v's total in lane 56 + v.
__device__ __forceinline__ float chain_lanes(const float *rs, const float *xs, int lane) {
  const int v = lane & 7, seg = lane >> 3;
  float a[64], b[64];
  const float4 *av = reinterpret_cast<const float4 *>(rs + v * RS + 64 * seg);
  const float4 *bv = reinterpret_cast<const float4 *>(xs + v * RS + 64 * seg);
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const float4 p = av[j], q = bv[j];
    a[4 * j] = p.x; a[4 * j + 1] = p.y; a[4 * j + 2] = p.z; a[4 * j + 3] = p.w;
    b[4 * j] = q.x; b[4 * j + 1] = q.y; b[4 * j + 2] = q.z; b[4 * j + 3] = q.w;
  }
  float acc = 0.0f;
#pragma unroll 1
  for (int g = 0; g < 8; g++) {
#pragma unroll
    for (int j = 0; j < 64; j++) acc = __builtin_fmaf(a[j], b[j], acc);
    const float up = __shfl_up(acc, 8, 64);
    if (seg == g + 1) acc = up;
  }
  return acc;
}

// ---------------------------------------------------------------------------
// Small T: one block per (expert, token). The block stages x, norm_w and the
// router row in LDS transposed by chain (buf[v][i] = a[8i+v]), reduces the
// sum of squares in the fixed block order, then wave 0 runs the eight logit
// chains (chain_lanes). Block (0, t) also stages s for the expert kernels.
__device__ __forceinline__ void router_block(
    int e, int t, const float *__restrict__ x, const float *__restrict__ xadd,
    const float *__restrict__ norm_w, const float *__restrict__ router,
    const float *__restrict__ bias, int has_bias, float *__restrict__ logits,
    float *__restrict__ sig, float *__restrict__ score, __half *__restrict__ s16,
    float *__restrict__ s32, unsigned long long *trace, const float *__restrict__ r_in) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) float xsf[8 * RS], rsf[8 * RS];
  const int tid = threadIdx.x;
  trace_point(trace, 0);
  {  // every load in flight at once: 4 float4 of each row per thread
    const float *xt = x + (size_t)t * D, *at = xadd ? xadd + (size_t)t * D : nullptr;
    const float4 *wg = reinterpret_cast<const float4 *>(norm_w);
    const float4 *rg = reinterpret_cast<const float4 *>(router + (size_t)e * D);
    float4 a[4], b[4], c[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      a[u] = load_x4(xt, at, tid + 256 * u);
      b[u] = wg[tid + 256 * u];
      c[u] = rg[tid + 256 * u];
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int j = 4 * (tid + 256 * u), v = j & 7, i = j >> 3;
      rsf[(v + 0) * RS + i] = c[u].x; rsf[(v + 1) * RS + i] = c[u].y;
      rsf[(v + 2) * RS + i] = c[u].z; rsf[(v + 3) * RS + i] = c[u].w;
    }
    __shared__ float red_l[4];
    const float ss = block_sumsq(a, red_l);  // contains a barrier
    const float r = r_in ? r_in[t] : 1.0f / __builtin_sqrtf(ss / 4096.0f + 1e-5f);
    trace_point(trace, 1);
    // s = (x * norm_w) * r, formed in registers and stored chain-transposed
    // (norm_w is not staged: the block holds 2 rows in LDS, not 3, so that
    // three blocks fit a CU)
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int j = 4 * (tid + 256 * u), v = j & 7, i = j >> 3;
      xsf[(v + 0) * RS + i] = (a[u].x * b[u].x) * r; xsf[(v + 1) * RS + i] = (a[u].y * b[u].y) * r;
      xsf[(v + 2) * RS + i] = (a[u].z * b[u].z) * r; xsf[(v + 3) * RS + i] = (a[u].w * b[u].w) * r;
    }
  }
  __syncthreads();
  if (tid < 64) {  // the eight logit chains in wave 0
    // the chain wave first at its SIMD's issue while the chains run: the shared
    // expert's gate/up waves of the same launch compete for it (C0 29.9 ->
    // 29.75 us; the whole router block at raised priority measured the same)
    __builtin_amdgcn_s_setprio(3);
    const float lg = tree8_lanes(chain_lanes(rsf, xsf, tid), tid & 7);
    __builtin_amdgcn_s_setprio(0);
    if (tid == 56) {
      const float sg = sigmoid_c(lg);
      logits[(size_t)t * E + e] = lg;
      sig[(size_t)t * E + e] = sg;
      score[(size_t)t * E + e] = has_bias ? sg + bias[e] : sg;
    }
    trace_point(trace, 3);
  } else if (e == 0 && tid >= 64) {
    // stage s for the expert kernels (fp16 pair-staged and fp32) from the
    // waves that run no chain
    for (int j = tid - 64; j < D; j += 192) {
      const float sv = xsf[(j & 7) * RS + (j >> 3)];
      stage_store(s16 + (size_t)t * D, j, sv);
      s32[(size_t)t * D + j] = sv;
    }
  }
}

}  // namespace hy3x
