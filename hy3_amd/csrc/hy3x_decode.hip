// hy3x_decode.hip -- single-token forward, first launch: RMSNorm, the router,
// the top-K and every gate/up row (the shared expert's and the K routed
// experts') in one kernel. The second launch is k_down_decode (down rows of
// the nine experts fused with the weighted combine and the residual).
//
// The reference runs router GEMV, top-K kernel, then the routed and shared
// FFNs (hy3_gpu.cu:706-738) as separate launches on the critical path; the
// CPU engine does the same steps in sequence (hy3.c:1266-1325). Here the
// routed gate/up blocks do not wait for the router's exact fp32 chains:
//
//  * router block e (e < 192) computes the logit twice from the same fp32 s:
//    first as an fp64 dot product V with A = sum |w_i s_i| (a few hundred
//    cycles after its loads), then as the routing contract's eight 512-step
//    fp32 FMA chains (about 2 us of dependent FMAs). For the chained result l,
//    |l - V| <= gamma_515 * A + (fp64 rounding) < 3.2e-5 * A (recursive
//    summation bound, n = 512 FMAs + 3 tree adds per term). sigmoid_c and the
//    fp32 add of the bias are monotone, so the exact score lies in
//    [score(V - d), score(V + d)], d = 3.2e-5 A (bounds rounded outward);
//  * the routing takes the K experts with the largest lower bounds. If
//    the K-th lower bound is strictly above every other expert's upper bound,
//    the exact top-K is that set (proof: each selection step of hy3.c's
//    selection sort takes the largest remaining exact score, which lies in
//    the set while it has members left), so the routed waves stream their slots'
//    expert at once. Otherwise (a near-tie, a NaN) it waits for the exact
//    top-K. Only the set matters for gate/up: the slot order it used is
//    published (spec_ids) and the down kernel combines in the exact order;
//  * one leader wave (block 0, wave 1) reads the bounds, decides, and
//    publishes the slots' experts; every other routed wave polls one word.
//    When the set is not certain the leader waits for the 192 exact sigmas
//    and runs the exact top-K itself. The down launch runs the exact top-K
//    as hy3.c does and publishes ids, wpre and w.
//
// Cross-block hand-offs use tagged 64-bit words (value | forward tag << 32)
// written and read with agent-scope relaxed atomics: a word is valid for this
// forward when its tag equals this forward's, so nothing needs clearing. The
// tag is epoch + 1; the launch's last block advances the epoch once every
// block has read it (each block writes its tag to started[b] first). All
// waits are bounded (kSpinLimit polls): on expiry the wave goes on with what
// it has and counts the event in stats[3]; no kernel can hang. Blocks only
// wait on lower-numbered blocks (router blocks wait on none; the routed
// waves on router blocks and block 0; the last block on every block's
// start), and workgroups
// are dispatched in order, so every awaited block is running or done.
#include "hy3x_kernels.h"
#include "hy3x_route.h"
#include "hy3x_decode.h"
#include "hy3x_q8.h"

#pragma clang fp contract(off)

namespace hy3x {

// Polls per wait before a wave gives up (each poll is one round trip to
// memory, about 1 us: the limit is far beyond any real wait).
constexpr int kSpinLimit = 1 << 18;

__device__ __forceinline__ uint64_t tagged(float v, uint32_t tag) {
  return (uint64_t)__builtin_bit_cast(uint32_t, v) | ((uint64_t)tag << 32);
}
__device__ __forceinline__ void publish(uint64_t *p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t fetch(const uint64_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Words w[lane + 64 m] (m < M, index < n) loaded until every one of them
// carries tag (whole wave). False when the spin limit ran out.
template <int M>
__device__ __forceinline__ bool poll_tagged(const uint64_t *w, int n, uint32_t tag,
                                            uint64_t (&v)[M]) {
  const int lane = threadIdx.x & 63;
  for (int it = 0; it < kSpinLimit; it++) {
    bool ok = true;
#pragma unroll
    for (int m = 0; m < M; m++) {
      const int i = lane + 64 * m;
      if (i < n) {
        v[m] = fetch(&w[i]);
        ok &= (uint32_t)(v[m] >> 32) == tag;
      }
    }
    if (__builtin_amdgcn_ballot_w64(!ok) == 0) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}

// Order-preserving key of a non-NaN float (-0 folded into +0; every key > 0).
__device__ __forceinline__ uint32_t okey(float f) {
  const uint32_t u = __builtin_bit_cast(uint32_t, f + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Wave maximum of v, wave-uniform.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)dppi<DPP_XOR1>((int)v));
  v = max(v, (uint32_t)dppi<DPP_XOR2>((int)v));
  v = max(v, (uint32_t)dppi<DPP_HALF_MIRROR>((int)v));
  v = max(v, (uint32_t)dppi<DPP_MIRROR>((int)v));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, DPP_BCAST15, 0xA, 0xF, false));
  v = max(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, DPP_BCAST31, 0xC, 0xF, false));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// The certified top-K set from score bounds (expert lane + 64 m in slot m):
// K rounds of wave argmax on the lower bounds; lane k < K gets the k-th
// expert. True when the set is certain: no NaN, no tied maximum in a round,
// and the K-th lower bound strictly above the largest upper bound of the
// experts left out.
__device__ __forceinline__ bool certified_topk(const float (&lo)[3], const float (&hi)[3], int K,
                                               int &my_e) {
  const int lane = threadIdx.x & 63;
  uint32_t kl[3], kh[3];
  bool nan = false;
#pragma unroll
  for (int m = 0; m < 3; m++) {
    nan |= lo[m] != lo[m] || hi[m] != hi[m];
    kl[m] = okey(lo[m]);
    kh[m] = okey(hi[m]);
  }
  my_e = 0;
  if (__builtin_amdgcn_ballot_w64(nan)) return false;
  bool tie = false;
  uint32_t M = 0;
  for (int k = 0; k < K; k++) {
    uint32_t v = kl[0] > kl[1] ? kl[0] : kl[1];
    v = v > kl[2] ? v : kl[2];
    M = wave_max_u32(v);
    const bool h0 = kl[0] == M, h1 = kl[1] == M, h2 = kl[2] == M;
    const uint64_t b0 = __builtin_amdgcn_ballot_w64(h0);
    const uint64_t b1 = __builtin_amdgcn_ballot_w64(h1);
    const uint64_t b2 = __builtin_amdgcn_ballot_w64(h2);
    tie |= __builtin_popcountll(b0) + __builtin_popcountll(b1) + __builtin_popcountll(b2) != 1;
    const int wl = __builtin_ctzll(b0 | b1 | b2);
    const int e_w = __builtin_amdgcn_readlane(lane + (h1 ? 64 : 0) + (h2 ? 128 : 0), wl);
    if (lane == k) my_e = e_w;
    // taken: out of the later rounds and of the upper-bound maximum below
    kl[0] = h0 ? 0u : kl[0];
    kl[1] = h1 ? 0u : kl[1];
    kl[2] = h2 ? 0u : kl[2];
    kh[0] = h0 ? 0u : kh[0];
    kh[1] = h1 ? 0u : kh[1];
    kh[2] = h2 ? 0u : kh[2];
  }
  uint32_t v = kh[0] > kh[1] ? kh[0] : kh[1];
  v = v > kh[2] ? v : kh[2];
  return !tie && M > wave_max_u32(v);
}

// float nearest below / above a double (the bounds are rounded outward).
__device__ __forceinline__ float f32_step(float f, bool up) {
  if (f == 0.0f) return up ? 1.4e-45f : -1.4e-45f;
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  return __builtin_bit_cast(float, (f > 0.0f) == up ? u + 1u : u - 1u);
}
__device__ __forceinline__ float f32_down(double d) {
  const float f = (float)d;
  return (double)f > d ? f32_step(f, false) : f;
}
__device__ __forceinline__ float f32_up(double d) {
  const float f = (float)d;
  return (double)f < d ? f32_step(f, true) : f;
}

// Sum over the wave's 64 lanes of a double in a fixed order (DPP within rows
// of 16, then the four row sums in order), wave-uniform.
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xF, 0xF, false);
  return __builtin_bit_cast(double, (uint64_t)(uint32_t)lo | ((uint64_t)(uint32_t)hi << 32));
}
__device__ __forceinline__ double readlane_f64(double v, int l) {
  const uint64_t u = __builtin_bit_cast(uint64_t, v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, l);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), l);
  return __builtin_bit_cast(double, (uint64_t)lo | ((uint64_t)hi << 32));
}
__device__ __forceinline__ double wave_sum_f64(double v) {
  v += dpp_f64<DPP_XOR1>(v);
  v += dpp_f64<DPP_XOR2>(v);
  v += dpp_f64<DPP_HALF_MIRROR>(v);
  v += dpp_f64<DPP_MIRROR>(v);
  return (readlane_f64(v, 0) + readlane_f64(v, 16)) + (readlane_f64(v, 32) + readlane_f64(v, 48));
}

// A bound on the routing contract's sigmoid_c (correctly rounded exp, IEEE
// add and division: within 1.8e-7 relative of the true sigmoid) at x, from
// below (up = false) or above: the hardware exp2 and reciprocal (each within
// 1 ulp; the rounded argument -x*log2(e) adds |x| 6e-8 relative), widened by
// 4e-6 + |x| 2e-7 relative -- over twice the sum of those errors -- and by
// 1e-37 absolute (results in the subnormal range). The true sigmoid is
// monotone, so a lower bound at a lower bound of the logit stays one.
__device__ __forceinline__ float sigmoid_bound(float x, bool up) {
  const float e = __builtin_amdgcn_exp2f(-x * 1.44269504f);
  const float sg = __builtin_amdgcn_rcpf(1.0f + e);
  const float m = 4e-6f + __builtin_fabsf(x) * 2e-7f;
  return up ? sg * (1.0f + m) + 1e-37f : sg * (1.0f - m) - 1e-37f;
}

// Bound on |chained fp32 logit - fp64 dot| relative to sum |w_i s_i|:
// gamma_515 = 515 u / (1 - 515 u) = 3.0697e-5 (u = 2^-24), plus the fp64 sum's
// own rounding (< 1e-12), rounded up.
constexpr double kLogitBound = 3.2e-5;

__global__ __launch_bounds__(256, 3) void k_decode_gateup(
    const float *__restrict__ x, const float *__restrict__ xadd,
    const float *__restrict__ norm_w, const float *__restrict__ router,
    const float *__restrict__ bias, int has_bias, int K, float scale,
    const uint8_t *__restrict__ wq, const uint8_t *__restrict__ wsh, DecodeSync sync,
    float *__restrict__ logits, float *__restrict__ sig, float *__restrict__ score,
    int32_t *__restrict__ ids, float *__restrict__ wpre, float *__restrict__ wout,
    __half *__restrict__ h16, unsigned long long *__restrict__ stats,
    unsigned long long *trace, const float *__restrict__ r_in) {
  __shared__ __attribute__((aligned(16))) float xsf[8 * RS], rsf[8 * RS];
  __shared__ __attribute__((aligned(16))) __half s_l[D];
  __shared__ float red_l[4];
  __shared__ double redd_l[8];
  __shared__ int32_t sids[KMAX], slot_l[KMAX];
  __shared__ float swp[KMAX], sw[KMAX];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, b = blockIdx.x;
  trace_point(trace, 0);
  // this forward's tag (every lane loads the epoch word, coherently)
  const uint32_t tag =
      (uint32_t)__builtin_amdgcn_readfirstlane(
          (int)__hip_atomic_load(sync.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) + 1u;
  if (tid == 0)
    __hip_atomic_store(&sync.started[b], tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const bool is_router = b < E;
  const bool is_shared = b >= E && b < E + DEC_SH_BLOCKS;
  const int slot = b / DEC_GU_BLOCKS, rc = b % DEC_GU_BLOCKS;
  const bool is_routed = slot < K;
  // (with K < 8 the blocks of slots K .. 7 outside the router and shared
  // ranges have nothing to do but, for the last block, advance the epoch)
  const bool idle = !is_router && !is_shared && !is_routed;

  if (idle) goto advance;
  {
  // x (+ the residual addend), norm_w and, for a router block, its router row
  float4 a[4], w4[4], rv[4];
  // a router block's bias and RMSNorm override, loaded with its rows
  const float bias_b = is_router && has_bias ? bias[b] : 0.0f;
  const float r_sub = r_in ? r_in[0] : 0.0f;
#pragma unroll
  for (int u = 0; u < 4; u++) {
    a[u] = load_x4(x, xadd, tid + 256 * u);
    w4[u] = reinterpret_cast<const float4 *>(norm_w)[tid + 256 * u];
    rv[u] = is_router ? reinterpret_cast<const float4 *>(router + (size_t)b * D)[tid + 256 * u]
                      : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }

  // s = rmsnorm(x) * norm_w (the routing contract's order), pair-staged fp16
  // in s_l; a router block also keeps it chain-transposed for its chains and
  // publishes its score bounds. load_group(): a wave's 64-weight group of s
  // from s_l (after the router chains, whose operands fill the registers).
  uint32_t X[32];
  float slo, shi;
  auto load_group = [&]() {
    load_group_x(s_l, lane, X);
    group_sums(X, slo, shi);
  };
  auto stage_s = [&]() {
    const float ss = block_sumsq(a, red_l);
    trace_point(trace, 7);
    const float r = r_in ? r_sub : 1.0f / __builtin_sqrtf(ss / 4096.0f + 1e-5f);
    float4 s4[4];
#pragma unroll
    for (int u = 0; u < 4; u++)
      s4[u] = make_float4((a[u].x * w4[u].x) * r, (a[u].y * w4[u].y) * r,
                          (a[u].z * w4[u].z) * r, (a[u].w * w4[u].w) * r);
    if (is_router) {
      // fp64 dot and absolute sum (products of two floats are exact in fp64)
      double p = 0.0, q = 0.0;
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const float sv[4] = {s4[u].x, s4[u].y, s4[u].z, s4[u].w};
        const float wv[4] = {rv[u].x, rv[u].y, rv[u].z, rv[u].w};
#pragma unroll
        for (int c = 0; c < 4; c++) {
          const double d = (double)wv[c] * (double)sv[c];
          p += d;
          q += __builtin_fabs(d);
        }
      }
      p = wave_sum_f64(p);
      q = wave_sum_f64(q);
      if (lane == 0) {
        redd_l[wave] = p;
        redd_l[4 + wave] = q;
      }
    }
    __syncthreads();
    if (is_router && tid < 2) {
      // the score bounds, published before the block stages anything: lane 0
      // the lower, lane 1 the upper
      const double V = (redd_l[0] + redd_l[1]) + (redd_l[2] + redd_l[3]);
      const double A = (redd_l[4] + redd_l[5]) + (redd_l[6] + redd_l[7]);
      // (+ 1e-35: room for flushed subnormals, 512 x 2^-126, in the chains)
      const double dl = A * kLogitBound + 1e-35;
      const bool up = tid == 1;
      const float lb = up ? f32_up(V + dl) : f32_down(V - dl);
      const float sg = sigmoid_bound(lb, up);
      const float sc = has_bias ? sg + bias_b : sg;
      publish(up ? &sync.bound_hi[b] : &sync.bound_lo[b], tagged(sc, tag));
      trace_point(trace, 4);
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int j = 4 * (tid + 256 * u);
      stage_store(s_l, j + 0, s4[u].x);
      stage_store(s_l, j + 1, s4[u].y);
      stage_store(s_l, j + 2, s4[u].z);
      stage_store(s_l, j + 3, s4[u].w);
      if (is_router) {  // chain-transposed copies for the exact chains
        const int v = j & 7, i = j >> 3;
        xsf[(v + 0) * RS + i] = s4[u].x; xsf[(v + 1) * RS + i] = s4[u].y;
        xsf[(v + 2) * RS + i] = s4[u].z; xsf[(v + 3) * RS + i] = s4[u].w;
        rsf[(v + 0) * RS + i] = rv[u].x; rsf[(v + 1) * RS + i] = rv[u].y;
        rsf[(v + 2) * RS + i] = rv[u].z; rsf[(v + 3) * RS + i] = rv[u].w;
      }
    }
    __syncthreads();
    trace_point(trace, 1);
  };

  // the shared expert's gate/up: one row per wave of blocks E .. E + 383
  // (they need no routing: before the routing is known)
  auto shared_rows = [&]() {
    const int r0 = (b - E) * DEC_RPB + wave * DEC_SH_RPW;
    load_group();
    if (wsh)
      gateup_rows_q8<DEC_SH_RPW, DEC_SH_RPW>(wsh, K, r0, X, slo, shi, h16);
    else
      gateup_rows<DEC_SH_RPW, DEC_SH_RPW>(wq, E, K, r0, X, slo, shi, h16);
  };
  stage_s();
#ifndef HY3X_V_SHEND
  if (is_shared) shared_rows();
#endif

  unsigned long long timeouts = 0;
  // router block, wave 0: the exact logit (the contract's eight chains; the
  // down launch takes the exact top-K from these sigmas)
  if (is_router && wave == 0) {
    __builtin_amdgcn_s_setprio(3);
#ifdef HY3X_V_NOCHAIN
    const float lg = xsf[lane];
#else
    const float lg = tree8_lanes(chain_lanes(rsf, xsf, lane), lane & 7);
#endif
    __builtin_amdgcn_s_setprio(0);
    const float sg = sigmoid_c(lg);
    if (lane == 56) {
      logits[b] = lg;
      sig[b] = sg;
      score[b] = has_bias ? sg + bias[b] : sg;
      publish(&sync.sig[b], tagged(sg, tag));
    }
    trace_point(trace, 5);
  }

  if (is_routed) {
    if (b == 0 && wave == 1) {
      // the routing leader: the slots' experts, certified from the score
      // bounds, else the exact top-K; published for every routed wave (one
      // wave reads the 384 bound words, the others poll one word each:
      // measured faster than a reader wave per block)
      // both arrays polled together: [0, E) the lower bounds, [E, 2E) the upper
      // (contiguous in the scratch)
      uint64_t bw[6] = {0, 0, 0, 0, 0, 0};
      if (!poll_tagged<6>(sync.bound_lo, 2 * E, tag, bw)) timeouts++;
      float lo[3], hi[3];
#pragma unroll
      for (int m = 0; m < 3; m++) {
        lo[m] = __builtin_bit_cast(float, (uint32_t)bw[m]);
        hi[m] = __builtin_bit_cast(float, (uint32_t)bw[3 + m]);
      }
      int my_e;
      const bool certain = certified_topk(lo, hi, K, my_e);
      // the exact top-K from the 192 exact sigmas (hy3.c:1272-1291), into
      // sids / swp (pre-scale) / sw (final) in LDS (this wave's own stores)
      auto exact_topk = [&]() {
        uint64_t v[3] = {0, 0, 0};
        if (!poll_tagged<3>(sync.sig, E, tag, v)) timeouts++;
        float sgv[3], scv[3];
#pragma unroll
        for (int m = 0; m < 3; m++) {
          sgv[m] = __builtin_bit_cast(float, (uint32_t)v[m]);
          scv[m] = has_bias ? sgv[m] + bias[lane + 64 * m] : sgv[m];
        }
        int xe;
        float my_sig, sum;
        if (topk_wave_fast(scv, sgv, K, xe, my_sig, sum)) {
          if (lane < K) {
            const float inv = 1.0f / (sum + 1e-20f);
            const float wv = my_sig * inv;
            sids[lane] = xe;
            swp[lane] = wv;
            sw[lane] = wv * scale;
          }
        } else {
          topk_wave_regs(scv, sgv, K, scale, sids, swp, sw);
        }
      };
      if (!certain) {
        exact_topk();  // the same set; the slots take the exact order
        if (lane < K) {
          my_e = sids[lane];
          slot_l[lane] = lane;
        }
      }
      if (lane < K) {
        sync.spec_ids[lane] = my_e;
        publish(&sync.spec[lane], tagged(__builtin_bit_cast(float, my_e), tag));
      }
      if (certain) {
        // the exact order of the certified set, for the down launch: the
        // exact sigmas of the K slot experts; with distinct scores hy3.c's
        // selection order is the set sorted by score, descending (a slot's
        // place = the slots scoring higher); a tie or a NaN among them: the
        // full selection with swaps
        const int ek = lane < K ? my_e : 0;
        const float bk = has_bias ? bias[ek] : 0.0f;
        float sgk = 0.0f;
        bool got = false;
        for (int it = 0; it < kSpinLimit && !got; it++) {
          bool ok = true;
          if (lane < K) {
            const uint64_t w = fetch(&sync.sig[ek]);
            ok = (uint32_t)(w >> 32) == tag;
            sgk = __builtin_bit_cast(float, (uint32_t)w);
          }
          got = __builtin_amdgcn_ballot_w64(!ok) == 0;
          if (!got) __builtin_amdgcn_s_sleep(1);
        }
        if (!got) timeouts++;
        const float sck = has_bias ? sgk + bk : sgk;
        int rank = 0;
        bool odd = lane < K && sck != sck;
        for (int j = 0; j < K; j++) {
          const float o =
              __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sck), j));
          rank += o > sck ? 1 : 0;
          odd |= lane < K && j != lane && o == sck;
        }
        if (__builtin_amdgcn_ballot_w64(odd) == 0) {
          if (lane < K) {
            sids[rank] = ek;
            swp[rank] = sgk;
            slot_l[rank] = lane;
          }
          float sum = 0.0f;
          for (int r = 0; r < K; r++) sum = sum + swp[r];  // in selection order
          const float inv = 1.0f / (sum + 1e-20f);
          if (lane < K) {
            const float wv = swp[lane] * inv;
            swp[lane] = wv;
            sw[lane] = wv * scale;
          }
        } else {
          exact_topk();
          if (lane < K) {
            const int idv = sids[lane];
            int pj = -1;  // a place missing from the slots (never, unless a wait expired)
            for (int j = 0; j < K; j++)
              if (__builtin_amdgcn_readlane(my_e, j) == idv) pj = j;
            slot_l[lane] = pj;
          }
        }
      }
      if (lane < K) {
        ids[lane] = sids[lane];
        wpre[lane] = swp[lane];
        wout[lane] = sw[lane];
        sync.perm[lane] = slot_l[lane];
      }
      if (lane == 0 && stats) {  // forwards, experts touched, uncertified routings
        stats[0] += 1ull;
        stats[1] += (unsigned long long)(K + 1);
        stats[2] += certain ? 0ull : 1ull;
      }
    }
    // this slot's expert
    uint64_t v[1] = {0};
#ifdef HY3X_V_NOPOLL
    v[0] = (uint64_t)(slot * 23 + 5);
#else
    if (!poll_tagged<1>(sync.spec + slot, 1, tag, v)) timeouts++;
#endif
    int e = __builtin_amdgcn_readfirstlane((int)(uint32_t)v[0]);
    e = e < 0 || e >= E ? 0 : e;  // only after an expired wait
    trace_point(trace, 2);
    load_group();
    gateup_rows<DEC_RPW, DEC_GU_PF>(wq, e, slot, rc * DEC_GU_RPB + wave * DEC_RPW, X, slo, shi,
                                    h16);
  }
#ifdef HY3X_V_SHEND
  if (is_shared) shared_rows();
#endif
  if (timeouts && lane == 0 && stats) atomicAdd(&stats[3], timeouts);
  trace_point(trace, 3);
  }

advance:
  // the last block advances the epoch once every block has read it
  if (b == DEC_BLOCKS - 1) {
    __syncthreads();
    if (wave == 0) {
      constexpr int M = (DEC_BLOCKS + 63) / 64;
      bool done = false;
      for (int it = 0; it < kSpinLimit && !done; it++) {
        bool ok = true;
#pragma unroll
        for (int m = 0; m < M; m++) {
          const int i = lane + 64 * m;
          if (i < DEC_BLOCKS)
            ok &= __hip_atomic_load(&sync.started[i], __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT) == tag;
        }
        done = __builtin_amdgcn_ballot_w64(!ok) == 0;
        if (!done) __builtin_amdgcn_s_sleep(1);
      }
      if (lane == 0) {
        if (!done && stats) atomicAdd(&stats[3], 1ull);
        __hip_atomic_store(sync.epoch, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      trace_point(trace, 6);
    }
  }
}

}  // namespace hy3x
