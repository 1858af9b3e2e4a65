// hy3x_route_decode.hip -- the single-token (decode) router launch: the 192
// router logits and the shared expert's gate/up rows in one kernel. Its own
// translation unit so that it can be scheduled with LLVM's iterative-ILP
// strategy (hy3_amd/build.py), which helps this launch and slows the
// multi-token router kernels of hy3x_route.hip. The routing contract is the
// one stated at the top of hy3x_route.hip.
#include "hy3x_kernels.h"
#include "hy3x_route.h"
#include "hy3x_router_block.h"
#include "hy3x_decode.h"
#include "hy3x_q8.h"

#pragma clang fp contract(off)

namespace hy3x {

// Single token: router logits and the shared expert's gate/up in one launch.
// Blocks 0..191 compute router logit e (router_block; block 0 also stages s).
// Blocks 192.. need no routing: they compute s themselves (the same RMSNorm
// arithmetic as router_block) and stream the shared expert's gate/up rows,
// 16 per block, into h16 slot K (wsh != nullptr: the shared expert is the
// layer's Q8 one, hy3x_q8.h). The top-K runs in the routed gate/up blocks
// (k_gateup_decode). Publishing it from here -- the last router block to
// arrive on a device-scope counter routes once -- measured slower: this
// kernel grew by 3.2 us (coherent stores and a relaxed count) or 5 us
// (acquire-release count), gate/up shrank by 0.6 us.
__global__ __launch_bounds__(256) void k_route_decode(
    const float *__restrict__ x, const float *__restrict__ xadd, const float *__restrict__ norm_w,
    const float *__restrict__ router, const float *__restrict__ bias, int has_bias, int K,
    float *__restrict__ logits, float *__restrict__ sig, float *__restrict__ score,
    __half *__restrict__ s16, float *__restrict__ s32, const uint8_t *__restrict__ wq,
    const uint8_t *__restrict__ wsh, __half *__restrict__ h16, unsigned long long *trace,
    const float *__restrict__ r_in) {
  const int tid = threadIdx.x;
  if (blockIdx.x < E) {
    router_block(blockIdx.x, 0, x, xadd, norm_w, router, bias, has_bias, logits, sig, score, s16,
                 s32, trace, r_in);
    return;
  }
  // shared expert: s = rmsnorm(x) * norm_w, pair-staged fp16 in LDS. The
  // loads of x and norm_w go first, then the rows' weight loads (they need no
  // s), so the weights stream in while the block reduces and stages s.
  trace_point(trace, 0);
  __shared__ __attribute__((aligned(16))) __half s_l[D];
  __shared__ float red_l[4];
  const float4 *wg = reinterpret_cast<const float4 *>(norm_w);
  float4 a[4], ad[4], w4[4];
#pragma unroll
  for (int u = 0; u < 4; u++) {  // x + xadd as load_x4, the add deferred
    a[u] = reinterpret_cast<const float4 *>(x)[tid + 256 * u];
    ad[u] = reinterpret_cast<const float4 *>(xadd ? xadd : x)[tid + 256 * u];
    w4[u] = wg[tid + 256 * u];
  }
  const int lane = tid & 63, wave = tid >> 6, sb = blockIdx.x - E;
  const int r0 = sb * DEC_RPB + wave * DEC_SH_RPW;
  auto stage_s = [&](uint32_t (&X)[32], float &slo, float &shi) {
    if (xadd) {
#pragma unroll
      for (int u = 0; u < 4; u++)
        a[u] = make_float4(a[u].x + ad[u].x, a[u].y + ad[u].y, a[u].z + ad[u].z,
                           a[u].w + ad[u].w);
    }
    const float ss = block_sumsq(a, red_l);
    const float r = r_in ? r_in[0] : 1.0f / __builtin_sqrtf(ss / 4096.0f + 1e-5f);
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int j = 4 * (tid + 256 * u);
      stage_store(s_l, j + 0, (a[u].x * w4[u].x) * r);
      stage_store(s_l, j + 1, (a[u].y * w4[u].y) * r);
      stage_store(s_l, j + 2, (a[u].z * w4[u].z) * r);
      stage_store(s_l, j + 3, (a[u].w * w4[u].w) * r);
    }
    __syncthreads();
    load_group_x(s_l, lane, X);
    group_sums(X, slo, shi);
    trace_point(trace, 1);
  };
  uint32_t X[32];
  float slo, shi;
  if (wsh) {
    GateupRowsQ8<DEC_SH_RPW, 2> rows(wsh, K, r0);
    stage_s(X, slo, shi);
    rows.finish(X, slo, shi, h16);
  } else {
    GateupRows<DEC_SH_RPW, DEC_SH_RPW> rows(wq, E, K, r0);
    stage_s(X, slo, shi);
    rows.finish(X, slo, shi, h16);
  }
  trace_point(trace, 3);
}

}  // namespace hy3x
