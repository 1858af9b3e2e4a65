// hy3x_gemv.hip -- grouped wavefront-reduction GEMV expert kernels (decode)
// and the weighted combine + residual.
//
// Work comes from the device tile list (k_dispatch_list): a tile is one expert and
// up to NT of its slots. The weights of a tile are streamed from HBM once,
// with 16-byte loads (each lane: the block header + 32 bytes of nibbles), and
// dotted against the NT staged activations held in registers. Replaces
// moe_matmul_q4k_id_gate_up_kernel / silu_mul_kernel / moe_matmul_q4k_id_kernel
// / moe_combine_id_kernel / add_kernel (hy3_gpu.cu:96-130, 140-142, 461-463)
// and the CPU loops hy3.c:1293-1325.
#include "hy3x_q4k.h"
#include "hy3x_decode.h"
#include "hy3x_route.h"
#include "hy3x_q8.h"

namespace hy3x {

// Slot -> token: routed slots are t*K + k, shared-expert slots T*K + t.
__device__ __forceinline__ int slot_token(int slot, int T, int K) {
  return slot < T * K ? slot / K : slot - T * K;
}

// gate/up + SwiGLU. Block = 4 waves x 4 rows = 16 rows of the 1536; a wave
// covers one 4096-wide row (64 groups, one per lane). h = silu(g) * u is
// written pair-staged (fp16) for the down kernel.
template <int NT>
__global__ __launch_bounds__(256) void k_gateup_gemv(const uint8_t *__restrict__ wq,
                                                     const __half *__restrict__ s16,
                                                     const int32_t *__restrict__ list,
                                                     const int4 *__restrict__ tiles,
                                                     const int32_t *__restrict__ n_tiles, int T,
                                                     int K, __half *__restrict__ h16) {
  constexpr int RPWAVE = 4, RPB = 16, CH = F / RPB;
  const int tile = blockIdx.x / CH, rc = blockIdx.x % CH;
  if (tile >= *n_tiles) return;
  const int4 td = tiles[tile];
  const int e = td.x, o = td.y, n = td.z;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = lane >> 2, p = lane & 3;
  const ScaleSel sel(p);

  uint32_t X[NT][32];
  float slo[NT], shi[NT];
  int slot[NT];
#pragma unroll
  for (int tt = 0; tt < NT; tt++) {
    slot[tt] = 0;
    slo[tt] = shi[tt] = 0.0f;
    if (tt < n) {
      slot[tt] = list[o + tt];
      load_group_x(s16 + (size_t)slot_token(slot[tt], T, K) * D, lane, X[tt]);
      group_sums(X[tt], slo[tt], shi[tt]);
    } else {
#pragma unroll
      for (int j = 0; j < 32; j++) X[tt][j] = 0u;
    }
  }
  const uint8_t *gbase = wq + (size_t)e * EXPERT_BYTES + (size_t)b * QB;
  const uint8_t *ubase = gbase + MAT_BYTES;
  const int r0 = rc * RPB + wave * RPWAVE;
#pragma unroll
  for (int rr = 0; rr < RPWAVE; rr++) {
    const int r = r0 + rr;
    const uint8_t *gp = gbase + (size_t)r * (D / QK) * QB;
    const uint8_t *up = ubase + (size_t)r * (D / QK) * QB;
    const uint4 gh = *reinterpret_cast<const uint4 *>(gp);
    const uint4 g0 = *reinterpret_cast<const uint4 *>(gp + 16 + 32 * p);
    const uint4 g1 = *reinterpret_cast<const uint4 *>(gp + 32 + 32 * p);
    const uint4 uh = *reinterpret_cast<const uint4 *>(up);
    const uint4 u0 = *reinterpret_cast<const uint4 *>(up + 16 + 32 * p);
    const uint4 u1 = *reinterpret_cast<const uint4 *>(up + 32 + 32 * p);
    const BlockScale gs = block_scale(gh, sel), us = block_scale(uh, sel);
    uint32_t P[32];
    float gv[NT], uv[NT];
    unpack_group(g0, g1, P);
#pragma unroll
    for (int tt = 0; tt < NT; tt++) gv[tt] = group_dot(P, X[tt], slo[tt], shi[tt], gs);
    unpack_group(u0, u1, P);
#pragma unroll
    for (int tt = 0; tt < NT; tt++) uv[tt] = group_dot(P, X[tt], slo[tt], shi[tt], us);
#pragma unroll
    for (int tt = 0; tt < NT; tt++) {
      const float g = wave_total(gv[tt]), u = wave_total(uv[tt]);
      if (lane == 0 && tt < n) h16[(size_t)slot[tt] * F + stage_index(r)] = swiglu_h(g, u);
    }
  }
}

// down: [4096 x 1536] per expert; a row is 24 groups, so each 32-lane half of
// a wave takes one row (lanes 24..31 idle). Block = 4 waves x 8 rows = 32 rows.
// out[slot][row] fp32.
template <int NT>
__global__ __launch_bounds__(256) void k_down_gemv(const uint8_t *__restrict__ wq,
                                                   const __half *__restrict__ h16,
                                                   const int32_t *__restrict__ list,
                                                   const int4 *__restrict__ tiles,
                                                   const int32_t *__restrict__ n_tiles,
                                                   float *__restrict__ out) {
  constexpr int RPWAVE = 8, RPB = 32, CH = D / RPB, G = F / 64;
  const int tile = blockIdx.x / CH, rc = blockIdx.x % CH;
  if (tile >= *n_tiles) return;
  const int4 td = tiles[tile];
  const int e = td.x, o = td.y, n = td.z;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hw = lane >> 5, gl = lane & 31;
  const bool active = gl < G;
  const int b = gl >> 2, p = gl & 3;
  const ScaleSel sel(p);

  uint32_t X[NT][32];
  float slo[NT], shi[NT];
  int slot[NT];
#pragma unroll
  for (int tt = 0; tt < NT; tt++) {
    slot[tt] = 0;
    slo[tt] = shi[tt] = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) X[tt][j] = 0u;
    if (tt < n) {
      slot[tt] = list[o + tt];
      if (active) {
        load_group_x(h16 + (size_t)slot[tt] * F, gl, X[tt]);
        group_sums(X[tt], slo[tt], shi[tt]);
      }
    }
  }
  const uint8_t *dbase = wq + (size_t)e * EXPERT_BYTES + 2 * MAT_BYTES + (size_t)b * QB;
  const int r0 = rc * RPB + wave * RPWAVE;
#pragma unroll
  for (int it = 0; it < RPWAVE / 2; it++) {
    const int r = r0 + 2 * it + hw;
    float dv[NT];
#pragma unroll
    for (int tt = 0; tt < NT; tt++) dv[tt] = 0.0f;
    if (active) {
      const uint8_t *dp = dbase + (size_t)r * (F / QK) * QB;
      const uint4 hd = *reinterpret_cast<const uint4 *>(dp);
      const uint4 q0 = *reinterpret_cast<const uint4 *>(dp + 16 + 32 * p);
      const uint4 q1 = *reinterpret_cast<const uint4 *>(dp + 32 + 32 * p);
      const BlockScale bs = block_scale(hd, sel);
      uint32_t P[32];
      unpack_group(q0, q1, P);
#pragma unroll
      for (int tt = 0; tt < NT; tt++) dv[tt] = group_dot(P, X[tt], slo[tt], shi[tt], bs);
    }
#pragma unroll
    for (int tt = 0; tt < NT; tt++) {
      const float2 v2 = half_totals(dv[tt]);
      if (gl == 0 && tt < n) out[(size_t)slot[tt] * D + r] = hw ? v2.y : v2.x;
    }
  }
}

// ---------------------------------------------------------------------------
// Decode fast path (T = 1): no dispatch. Slot k < K is routed expert ids[k],
// slot K the shared expert; the expert id is one load away from the weights.

// Routed gate/up of a single token: block = DEC_GU_RPB rows (DEC_GU_WAVES
// waves x DEC_RPW) of routed slot blockIdx.x / DEC_GU_BLOCKS. Every wave routes the
// token itself from the 192 sigmoid values / scores (the routing contract,
// identical in every wave and block: topk_wave_fast, or topk_wave_regs on a
// tie) and takes the expert of its slot; block 0 publishes the routing and
// the stats. All blocks are resident at once.
__global__ __launch_bounds__(64 * DEC_GU_WAVES) void k_gateup_decode(
    const uint8_t *__restrict__ wq, const __half *__restrict__ s16,
    const float *__restrict__ sig, const float *__restrict__ score, int K, float scale,
    int32_t *__restrict__ ids, float *__restrict__ wpre, float *__restrict__ wout,
    unsigned long long *__restrict__ stats, __half *__restrict__ h16,
    unsigned long long *trace) {
  trace_point(trace, 0);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int slot = blockIdx.x / DEC_GU_BLOCKS, rc = blockIdx.x % DEC_GU_BLOCKS;
  // the token's staged s, once per block (the block's waves read it from LDS),
  // loaded together with the routing inputs
  const int tid = threadIdx.x;
  constexpr int NT = 64 * DEC_GU_WAVES, NS = (D / 8 + NT - 1) / NT;  // 16-byte pieces per thread
  constexpr bool EXACT = NS * NT == D / 8;
  uint4 sv[NS];
#pragma unroll
  for (int i = 0; i < NS; i++)
    sv[i] = EXACT || tid + NT * i < D / 8 ? reinterpret_cast<const uint4 *>(s16)[tid + NT * i]
                                          : make_uint4(0u, 0u, 0u, 0u);
  // the routing inputs: expert lane + 64 m's score and sigma
  float sc[3], sg[3];
#pragma unroll
  for (int m = 0; m < 3; m++) {
    sc[m] = score[lane + 64 * m];
    sg[m] = sig[lane + 64 * m];
  }
  __shared__ __attribute__((aligned(16))) __half s_l[D];
  __shared__ int32_t sids[KMAX];
  __shared__ float swp[KMAX], sw[KMAX];
#pragma unroll
  for (int i = 0; i < NS; i++)
    if (EXACT || tid + NT * i < D / 8) reinterpret_cast<uint4 *>(s_l)[tid + NT * i] = sv[i];
  // every wave routes the token itself, in registers (the same arithmetic in
  // every wave and block, so the outcome is block-uniform)
  int my_e;
  float my_sig, sum;
  // a block needs the first slot + 1 places only (block 0, which publishes
  // the routing, all K): places before a tie are the same in every method.
  // (Issuing the first weight loads before the activation reads below, as
  // the shared-expert blocks do, measured 4 us slower here.)
  const bool fast = topk_wave_fast(sc, sg, blockIdx.x == 0 ? K : slot + 1, my_e, my_sig, sum);
  __syncthreads();  // s_l staged
  int e;
  if (fast) {
    e = __builtin_amdgcn_readlane(my_e, slot);
    if (blockIdx.x == 0 && threadIdx.x < K) {
      const float inv = 1.0f / (sum + 1e-20f);
      const float v = my_sig * inv;
      ids[threadIdx.x] = my_e;
      wpre[threadIdx.x] = v;
      wout[threadIdx.x] = v * scale;
    }
  } else {  // a tie or a NaN among the scores: the reference's selection with swaps
    if (wave == 0) topk_wave_regs(sc, sg, K, scale, sids, swp, sw);
    __syncthreads();
    e = sids[slot];
    if (blockIdx.x == 0 && threadIdx.x < K) {
      ids[threadIdx.x] = sids[threadIdx.x];
      wpre[threadIdx.x] = swp[threadIdx.x];
      wout[threadIdx.x] = sw[threadIdx.x];
    }
  }
  uint32_t X[32];
  load_group_x(s_l, lane, X);
  float slo, shi;
  group_sums(X, slo, shi);
  trace_point(trace, 1);
  if (blockIdx.x == 0 && threadIdx.x == 0 && stats) {  // forwards, experts touched (shared included)
    stats[0] += 1ull;
    stats[1] += (unsigned long long)(K + 1);
  }
  gateup_rows<DEC_RPW, DEC_GU_PF>(wq, e, slot, rc * DEC_GU_RPB + wave * DEC_RPW, X, slo, shi,
                                  h16);
  trace_point(trace, 3);
}

// Down of a single token for rows blockIdx.x*RPB .. +RPB, fused with the
// combine y = x + (shared + sum_k w_k * down_k), k in selection order
// (hy3.c:1302, 1318-1319, 1324-1325). Wave k < K owns routed slot k, waves
// KMAX .. KMAX + 3 a quarter of the rows each of the shared expert (waves
// K .. KMAX - 1 are idle): their passes of 2 rows stream through a register
// ring of DEC_DOWN_PF passes (down_rows; 2 measured best), the row sums go
// to LDS, and DEC_DOWN_RPB threads combine them. wsh != nullptr: the shared
// expert is the layer's Q8 one (down_rows_q8). A variant that copied each
// wave's 16 rows into LDS with every copy in flight at once measured faster
// in back-to-back replays of this kernel alone but slower inside the
// forward (decode 32.9 vs 32.1 us, 79-layer stack 2.87 vs 2.82 ms): its
// 157 KB of LDS per block keeps a block off a CU until the CU is empty.
__global__ __launch_bounds__(64 * DEC_DOWN_WAVES) void k_down_decode(
    const uint8_t *__restrict__ wq, const __half *__restrict__ h16,
    const int32_t *__restrict__ ids, const float *__restrict__ w, int K,
    float *__restrict__ x, const float *__restrict__ xadd, const uint8_t *__restrict__ wsh,
    unsigned long long *trace) {
  constexpr int RPB = DEC_DOWN_RPB, SH_ROWS = RPB / DEC_DOWN_SH_WAVES;
  __shared__ float out_l[KMAX + 1][RPB];  // [KMAX]: the shared expert
  trace_point(trace, 0);
  const int lane = threadIdx.x & 63, k = threadIdx.x >> 6;
  const int r0 = blockIdx.x * RPB;
  // the combine's inputs (residual row, gate weights), loaded before the
  // weight streams so that they are in registers when the row sums are
  // (raw values: an add here would wait for the loads)
  float xv = 0.0f, xav = 0.0f, wv = 0.0f;
  if (k == 0) {
    const int r = r0 + (lane < RPB ? lane : 0);
    xv = x[r];
    if (xadd) xav = xadd[r];
    wv = w[lane < K ? lane : 0];  // lane kk holds w[kk]
  }
  if (k >= KMAX) {  // a quarter of the block's rows of the shared expert
    const int q = k - KMAX;
    auto keep = [&](int ps, float2 t) {
      if (lane == 0) {
        out_l[KMAX][q * SH_ROWS + 2 * ps] = t.x;
        out_l[KMAX][q * SH_ROWS + 2 * ps + 1] = t.y;
      }
    };
    if (wsh)
      down_rows_q8<SH_ROWS / 2, DEC_DOWN_PF>(wsh, h16 + (size_t)K * F, r0 + q * SH_ROWS, keep);
    else
      down_rows<SH_ROWS / 2, DEC_DOWN_PF>(wq, [] { return E; }, h16 + (size_t)K * F,
                                          r0 + q * SH_ROWS, keep);
  } else if (k < K) {
    auto keep = [&](int ps, float2 t) {
      if (lane == 0) {
        out_l[k][2 * ps] = t.x;
        out_l[k][2 * ps + 1] = t.y;
      }
    };
    const int ku = __builtin_amdgcn_readfirstlane(k);  // a scalar load of the id
    down_rows<RPB / 2, DEC_DOWN_PF>(wq, [&] { return ids[ku]; }, h16 + (size_t)k * F, r0, keep);
  }
  __syncthreads();
  trace_point(trace, 2);
  if (threadIdx.x < RPB) {
    const int r = r0 + threadIdx.x;
    float eo = 0.0f;
    for (int kk = 0; kk < K; kk++)
      eo = __builtin_fmaf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(
                              __builtin_bit_cast(int, wv), kk)),
                          out_l[kk][threadIdx.x], eo);
    const float xr = xadd ? xv + xav : xv;
    x[r] = xr + (out_l[KMAX][threadIdx.x] + eo);
  }
  trace_point(trace, 3);
}

// y = x + (shared + sum_k w_k * routed_k), k in selection order (hy3.c:1302,
// 1318-1319, 1324-1325). Block (c, t): elements 1024 c .. 1024 c + 1023 of
// token t, four per thread; every slot's row is loaded before the FMA chain.
__global__ __launch_bounds__(256) void k_combine(float *__restrict__ x,
                                                 const float *__restrict__ xadd,
                                                 const float *__restrict__ out,
                                                 const float *__restrict__ w, int T, int K) {
  const int t = blockIdx.y, i = blockIdx.x * 1024 + 4 * threadIdx.x;
  float4 r[KMAX];
  float wk[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; k++)
    if (k < K) {
      r[k] = *reinterpret_cast<const float4 *>(out + (size_t)(t * K + k) * D + i);
      wk[k] = w[t * K + k];
    }
  const float4 sh = *reinterpret_cast<const float4 *>(out + (size_t)(T * K + t) * D + i);
  float4 xv = load_x4(x + (size_t)t * D, xadd ? xadd + (size_t)t * D : nullptr, i / 4);
  float4 eo = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int k = 0; k < KMAX; k++)
    if (k < K) {
      eo.x = __builtin_fmaf(wk[k], r[k].x, eo.x);
      eo.y = __builtin_fmaf(wk[k], r[k].y, eo.y);
      eo.z = __builtin_fmaf(wk[k], r[k].z, eo.z);
      eo.w = __builtin_fmaf(wk[k], r[k].w, eo.w);
    }
  xv.x = xv.x + (sh.x + eo.x);
  xv.y = xv.y + (sh.y + eo.y);
  xv.z = xv.z + (sh.z + eo.z);
  xv.w = xv.w + (sh.w + eo.w);
  *reinterpret_cast<float4 *>(x + (size_t)t * D + i) = xv;
}

template __global__ void k_gateup_gemv<1>(const uint8_t *, const __half *, const int32_t *,
                                          const int4 *, const int32_t *, int, int, __half *);
template __global__ void k_gateup_gemv<4>(const uint8_t *, const __half *, const int32_t *,
                                          const int4 *, const int32_t *, int, int, __half *);
template __global__ void k_down_gemv<1>(const uint8_t *, const __half *, const int32_t *,
                                        const int4 *, const int32_t *, float *);
template __global__ void k_down_gemv<4>(const uint8_t *, const __half *, const int32_t *,
                                        const int4 *, const int32_t *, float *);

}  // namespace hy3x
