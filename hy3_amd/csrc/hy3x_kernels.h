// hy3x_kernels.h -- kernel declarations shared by the translation units.
#pragma once
#include "hy3x_common.h"

namespace hy3x {

__global__ void k_router_logits(const float *x, const float *xadd, const float *norm_w,
                                const float *router,
                                const float *bias, int has_bias, float *logits, float *sig,
                                float *score, __half *s16, float *s32,
                                unsigned long long *trace, int T, uint32_t *bits, int wt,
                                const float *r_in);
__global__ void k_rmsnorm(const float *x, const float *xadd, const float *norm_w, __half *s16,
                          float *s32,
                          __half *s16m, __half *ssum, int T, uint32_t *bits, int wt,
                          const float *r_in);
// K chunk of the router GEMM (floats per LDS stage) and chunks in flight
// (register ring) per tile size: 4 x 8 (tiny), 8 x 16 (mid) and the larger
// tiles. Few blocks run at small T, so each chunk's load latency must hide
// behind the previous chunks' FMAs.
// The largest tile (32 x 32, T > 512) runs 64-wide chunks, four in flight
// (router stage at 4096 tokens 205 -> 182 us; at 512 tokens, 16 x 16 tiles,
// the same ring measured 54 -> 60 us, so that tile keeps 128-wide chunks).
constexpr int ROUTER_KC_TINY = 256, ROUTER_KC_MID = 256, ROUTER_KC_LARGE = 128, ROUTER_KC_XL = 64;
constexpr int ROUTER_R_TINY = 2, ROUTER_R_MID = 2, ROUTER_R_LARGE = 1, ROUTER_R_XL = 4;
template <int MT, int ME, int TG, int EG, int KC, int R>
__global__ __launch_bounds__(256) void k_router_gemm(const float *s32, const float *router, int T,
                                                     float *logits);
extern template __global__ void k_router_gemm<2, 2, 4, 8, ROUTER_KC_MID, ROUTER_R_MID>(
    const float *, const float *, int, float *);
extern template __global__ void k_router_gemm<8, 4, 4, 8, ROUTER_KC_XL, ROUTER_R_XL>(
    const float *, const float *, int, float *);
extern template __global__ void k_router_gemm<1, 1, 4, 8, ROUTER_KC_TINY, ROUTER_R_TINY>(
    const float *, const float *, int, float *);
extern template __global__ void k_router_gemm<4, 2, 4, 8, ROUTER_KC_LARGE, ROUTER_R_LARGE>(
    const float *, const float *, int, float *);
__global__ void k_topk(const float *logits, const float *bias, int has_bias, int K, float scale,
                       int T, int32_t *ids, float *wpre, float *wout, uint32_t *bits, int wt);
__global__ void k_dispatch_list(const int32_t *ids, int T, int K, int NT, const uint32_t *bits,
                                int wt, int32_t *list, int4 *tiles,
                                int32_t *n_tiles, int max_tiles, int32_t *counts_out,
                                unsigned long long *stats);
template <int NT>
__global__ void k_gateup_gemv(const uint8_t *wq, const __half *s16, const int32_t *list,
                              const int4 *tiles, const int32_t *n_tiles, int T, int K,
                              __half *h16);
template <int NT>
__global__ void k_down_gemv(const uint8_t *wq, const __half *h16, const int32_t *list,
                            const int4 *tiles, const int32_t *n_tiles, float *out);
__global__ void k_gateup_decode(const uint8_t *wq, const __half *s16, const float *sig,
                                const float *score, int K, float scale, int32_t *ids,
                                float *wpre, float *wout, unsigned long long *stats,
                                __half *h16, unsigned long long *trace);
__global__ void k_route_decode(const float *x, const float *xadd, const float *norm_w,
                               const float *router,
                               const float *bias, int has_bias, int K, float *logits,
                               float *sig, float *score, __half *s16, float *s32,
                               const uint8_t *wq, const uint8_t *wsh, __half *h16,
                               unsigned long long *trace, const float *r_in);
__global__ void k_down_decode(const uint8_t *wq, const __half *h16, const int32_t *ids,
                              const float *w, int K, float *x, const float *xadd,
                              const uint8_t *wsh,
                              unsigned long long *trace);
__global__ void k_stream_read(const uint4 *p, int64_t n16, uint32_t *sink);
__global__ void k_repack_q8x128(const uint8_t *src, uint8_t *dst, int64_t n_super);
__global__ void k_synth_q8_0(uint8_t *dst, int64_t nblocks, uint64_t key, const float *src);
__global__ void k_combine(float *x, const float *xadd, const float *out, const float *w, int T,
                          int K);

extern template __global__ void k_gateup_gemv<1>(const uint8_t *, const __half *, const int32_t *,
                                                 const int4 *, const int32_t *, int, int,
                                                 __half *);
extern template __global__ void k_gateup_gemv<4>(const uint8_t *, const __half *, const int32_t *,
                                                 const int4 *, const int32_t *, int, int,
                                                 __half *);
extern template __global__ void k_down_gemv<1>(const uint8_t *, const __half *, const int32_t *,
                                               const int4 *, const int32_t *, float *);
extern template __global__ void k_down_gemv<4>(const uint8_t *, const __half *, const int32_t *,
                                               const int4 *, const int32_t *, float *);

// The MFMA grouped GEMMs in two shapes (hy3x_mfma.hip, compiled once per
// shape). A work tile has ROWS_GU = 16 WAVES RGU gate/up rows (per matrix) or
// twice as many down rows and up to TOKENS tokens; each wave takes 16 RGU
// gate/up rows or 32 RGU down rows:
//   narrow: 32 tokens, 4 waves -- two workgroups per CU; the shape for few
//           tokens per expert;
//   wide:   64 tokens, 8 waves -- one workgroup per CU, half the per-token
//           dequantisation work; the shape for long prefills.
#define HY3X_DECLARE_MFMA(NS, TOK, WV, RGU_)                                                  \
  namespace NS {                                                                            \
  constexpr int TOKENS = TOK, WAVES = WV, RGU = RGU_, ROWS_GU = 16 * WV * RGU_;             \
  template <bool GATEUP>                                                                    \
  __global__ __launch_bounds__(64 * WV) void k_moe_mfma(                                    \
      const uint8_t *wq, const uint8_t *wsh, const __half *act, const __half *act_sum,      \
      const int32_t *list, const int4 *tiles, const int32_t *n_tiles, int T, int K,         \
      __half *h16m, float *out);                                                            \
  extern template __global__ void k_moe_mfma<true>(                                         \
      const uint8_t *, const uint8_t *, const __half *, const __half *, const int32_t *,    \
      const int4 *, const int32_t *, int, int, __half *, float *);                          \
  extern template __global__ void k_moe_mfma<false>(                                        \
      const uint8_t *, const uint8_t *, const __half *, const __half *, const int32_t *,    \
      const int4 *, const int32_t *, int, int, __half *, float *);                          \
  }
HY3X_DECLARE_MFMA(mfma_narrow, 32, 4, 1)
HY3X_DECLARE_MFMA(mfma_wide, 64, 8, 1)
#undef HY3X_DECLARE_MFMA
// 128-token tiles for experts holding many tokens (hy3x_mfma_big.hip): the
// MFMA tiles' arithmetic, each wave's dequantised
// weights reused over up to eight 16-token column groups.
constexpr int BIG_TOKENS = 128, BIG_WAVES = 8;
namespace mfma_big {
template <bool GATEUP>
__global__ __launch_bounds__(64 * BIG_WAVES) void k_moe_big(
    const uint8_t *wq, const uint8_t *wsh, const __half *act, const __half *act_sum,
    const int32_t *list, const int4 *tiles, const int32_t *n_tiles, int T, int K, __half *h16m,
    float *out);
extern template __global__ void k_moe_big<true>(const uint8_t *, const uint8_t *, const __half *,
                                                const __half *,
                                                const int32_t *, const int4 *, const int32_t *,
                                                int, int, __half *, float *);
extern template __global__ void k_moe_big<false>(const uint8_t *, const uint8_t *,
                                                 const __half *, const __half *,
                                                 const int32_t *, const int4 *, const int32_t *,
                                                 int, int, __half *, float *);
}  // namespace mfma_big
__global__ void k_stage_mfma(const float *s32, __half *s16m, __half *ssum);
__global__ void k_hsums(const __half *h16m, __half *hsum);

__global__ void k_synth_q4k(uint8_t *dst, int64_t nblocks, uint64_t seed, uint32_t layer,
                            const float *src);

}  // namespace hy3x
