// hy3x_route.hip -- fused RMSNorm + router + top-K, and the device dispatch.
//
// Routing contract (shared with the CPU oracle, which restates it):
//  * every fp32 reduction over the 4096 hidden elements uses one fixed order:
//    lane l of a 64-lane wave accumulates a[256i+4l+c]*b[256i+4l+c] with fmaf
//    over (i, c) lexicographically from 0, then an xor-butterfly over the lanes;
//  * ss = sum x^2 in that order; r = 1/sqrt(ss/4096 + 1e-5); s = (x*r)*w
//    (hy3.c:435-444);
//  * logit_e = sum router[e,:]*s in that order (hy3.c:1269);
//  * sigma = 1/(1 + exp(-logit)) with exp from Cody-Waite reduction and a
//    degree-7 Taylor polynomial; score = sigma + bias (hy3.c:1272-1277);
//  * top-K by selection with swaps, strict '>' (hy3.c:654-666), reproduced in
//    parallel: each step takes the largest score, ties to the lowest current
//    position, then swaps it into place;
//  * w_k = sigma_k * (1/(sum_k sigma_k + 1e-20)) (k order), times the scale
//    (hy3.c:1283-1291). wpre is the value before the scale.
// fp32 division and sqrt are correctly rounded (built with
// -fhip-fp32-correctly-rounded-divide-sqrt), and no a*b+c outside the explicit
// fmaf calls is contracted in this file, so the results are bit-identical to
// the oracle's.
#include "hy3x_common.h"

#pragma clang fp contract(off)

namespace hy3x {

__device__ __forceinline__ float sig_expf(float x) {
  if (x != x) return x;
  if (x > 88.72f) return __builtin_huge_valf();
  if (x < -87.0f) return 0.0f;
  const float kf = __builtin_rintf(x * 1.44269502f);
  float r = __builtin_fmaf(kf, -0.693145751953125f, x);
  r = __builtin_fmaf(kf, -1.428606765330187e-06f, r);
  float p = 1.98412701e-4f;
  p = __builtin_fmaf(p, r, 1.38888892e-3f);
  p = __builtin_fmaf(p, r, 8.33333377e-3f);
  p = __builtin_fmaf(p, r, 4.16666679e-2f);
  p = __builtin_fmaf(p, r, 1.66666672e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int k = (int)kf;
  const int k1 = k / 2, k2 = k - k1;
  const float s1 = __uint_as_float((uint32_t)(k1 + 127) << 23);
  const float s2 = __uint_as_float((uint32_t)(k2 + 127) << 23);
  return (p * s1) * s2;
}

// Loads this lane's 64 elements of a 4096-vector: v[i][c] = a[256i + 4l + c].
__device__ __forceinline__ void load_lane64(const float *a, int lane, float4 (&v)[16]) {
  const float4 *p = reinterpret_cast<const float4 *>(a) + lane;
#pragma unroll
  for (int i = 0; i < 16; i++) v[i] = p[64 * i];
}

__device__ __forceinline__ float lane_dot64(const float4 (&a)[16], const float4 (&b)[16]) {
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    acc = __builtin_fmaf(a[i].x, b[i].x, acc);
    acc = __builtin_fmaf(a[i].y, b[i].y, acc);
    acc = __builtin_fmaf(a[i].z, b[i].z, acc);
    acc = __builtin_fmaf(a[i].w, b[i].w, acc);
  }
  return acc;
}

// s = (x * r) * w for this lane's elements, r from the contract's sum of squares.
__device__ __forceinline__ void lane_rmsnorm(const float *x, const float *nw, int lane,
                                             float4 (&s)[16]) {
  float4 xv[16], wv[16];
  load_lane64(x, lane, xv);
  load_lane64(nw, lane, wv);
  const float ss = wave_sum(lane_dot64(xv, xv));
  const float r = 1.0f / __builtin_sqrtf(ss / 4096.0f + 1e-5f);
#pragma unroll
  for (int i = 0; i < 16; i++) {
    s[i].x = xv[i].x * r * wv[i].x;
    s[i].y = xv[i].y * r * wv[i].y;
    s[i].z = xv[i].z * r * wv[i].z;
    s[i].w = xv[i].w * r * wv[i].w;
  }
}

// Parallel selection-with-swaps top-K over 192 scores held 3 per lane
// (expert e at lane e%64, slot e/64). Writes ids[K] (lane 0).
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

// Router for small T: grid (48, T), 4 waves per block, one expert per wave.
// The last block to finish a token (atomic ticket) runs the top-K for it and
// resets the ticket, so the kernel can be relaunched (or graph-replayed)
// without clearing memory.
__global__ __launch_bounds__(256) void k_router_gemv(
    const float *__restrict__ x, const float *__restrict__ norm_w,
    const float *__restrict__ router, const float *__restrict__ bias, int has_bias, int K,
    float scale, float *logits, __half *__restrict__ s16, int32_t *__restrict__ ids,
    float *__restrict__ wpre, float *__restrict__ wout, unsigned *__restrict__ tickets) {
  const int t = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blockIdx.x * 4 + wave;
  const float *xt = x + (size_t)t * D;
  float4 s[16];
  lane_rmsnorm(xt, norm_w, lane, s);
  if (blockIdx.x == 0) {  // stage s (fp16, pair-staged) for the expert kernels
    __half *dst = s16 + (size_t)t * D;
#pragma unroll
    for (int i = 4 * wave; i < 4 * wave + 4; i++) {
      const int j = 256 * i + 4 * lane;
      dst[stage_index(j + 0)] = __float2half(s[i].x);
      dst[stage_index(j + 1)] = __float2half(s[i].y);
      dst[stage_index(j + 2)] = __float2half(s[i].z);
      dst[stage_index(j + 3)] = __float2half(s[i].w);
    }
  }
  float4 wr[16];
  load_lane64(router + (size_t)e * D, lane, wr);
  const float lg = wave_sum(lane_dot64(wr, s));
  if (lane == 0) {
    logits[(size_t)t * E + e] = lg;
    __threadfence();
  }

  __shared__ int is_last;
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned prev = __hip_atomic_fetch_add(&tickets[t], 1u, __ATOMIC_ACQ_REL,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    is_last = (prev == gridDim.x - 1);
  }
  __syncthreads();
  if (!is_last || wave != 0) return;
  __atomic_thread_fence(__ATOMIC_ACQUIRE);  // agent scope: see every block's logits
  __shared__ float sg_l[E];
  float sc[3];
#pragma unroll
  for (int m = 0; m < 3; m++) {
    const int ee = lane + 64 * m;
    const float l = logits[(size_t)t * E + ee];
    const float sgm = 1.0f / (1.0f + sig_expf(-l));
    sg_l[ee] = sgm;
    sc[m] = has_bias ? sgm + bias[ee] : sgm;
  }
  __shared__ int32_t sel_ids[KMAX];
  wave_topk(sc, lane, K, sel_ids);
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup");
  __builtin_amdgcn_wave_barrier();
  if (lane == 0) {
    float sum = 0.0f;
    for (int k = 0; k < K; k++) sum += sg_l[sel_ids[k]];
    const float inv = 1.0f / (sum + 1e-20f);
    for (int k = 0; k < K; k++) {
      const float v = sg_l[sel_ids[k]] * inv;
      ids[(size_t)t * K + k] = sel_ids[k];
      wpre[(size_t)t * K + k] = v;
      wout[(size_t)t * K + k] = v * scale;
    }
    tickets[t] = 0u;
  }
}

// Device dispatch: per-expert slot lists and the work-tile list, one block.
// Slots: s < T*K is (token s/K, rank s%K) of a routed expert; s = T*K + t is
// token t of the shared expert (index E), which every token uses.
// tiles[i] = {expert, first list index, count <= NT, 0}.
__global__ __launch_bounds__(1024) void k_dispatch(const int32_t *__restrict__ ids, int T, int K,
                                                   int NT, int32_t *__restrict__ list,
                                                   int4 *__restrict__ tiles,
                                                   int32_t *__restrict__ n_tiles, int max_tiles,
                                                   int32_t *__restrict__ counts_out) {
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
