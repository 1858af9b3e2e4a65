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
// Router GEMM tile shapes by token count (k_router_gemm<MT, ME, 4, 8, KC,
// R>): a thread holds MT x ME (token, expert) outputs of one chain, a block
// 4 MT tokens x 8 ME experts; K is walked in chunks of KC floats with R
// chunks in flight. Few blocks run at small T, so there each chunk's load
// latency must hide behind the previous chunks' FMAs; at large T the tile
// sets the LDS reads per FMA and the block count per CU. Measured on MI355X
// (router stage, RMSNorm + GEMM + top-K; the shape replaced in brackets):
//   TINY  T <= 64:   4 x 8,   KC 256, R 2 (T = 32: 21.4 us; 4 x 16: 25.1, 4 x 24: 31.0)
//   MID   T <= 256:  8 x 16,  KC 256, R 2 (T = 96 / 160 / 256: 28.5 / 28.8 / 36.4 us;
//                    KC 128: 29.5 / 29.6 / 34.3, 8 x 24: 33.7 / 33.9 / 34.5)
//   LARGE T <= 1536: 16 x 24, KC 128, R 1 (T = 512: 42.8 us [16 x 16: 49.3],
//                    T = 1024: 62.4 us [32 x 32: 93.7], T = 1536: 86.3 [103.0];
//                    T = 2048: 113.7 against 108.6 for 32 x 32)
//   XL    T <= 2560: 32 x 32, KC 64,  R 4 (T = 2560: 115.0 us; 32 x 48: 138.5)
//   XXL   T > 2560:  32 x 48, KC 64,  R 4 (T = 3072: 140.9 us [32 x 32: 147.2],
//                    T = 4096: 155.9 [165.7])
#define HY3X_RCFG(NAME, MT, ME, KC, R)                                                         \
  constexpr int ROUTER_MT_##NAME = MT, ROUTER_ME_##NAME = ME, ROUTER_KC_##NAME = KC,        \
                ROUTER_R_##NAME = R;
#ifndef HY3X_RCFG_TINY
#define HY3X_RCFG_TINY 1, 1, 256, 2
#endif
#ifndef HY3X_RCFG_MID
#define HY3X_RCFG_MID 2, 2, 256, 2
#endif
#ifndef HY3X_RCFG_LARGE
#define HY3X_RCFG_LARGE 4, 3, 128, 1
#endif
#ifndef HY3X_RCFG_XL
#define HY3X_RCFG_XL 8, 4, 64, 4
#endif
#ifndef HY3X_RCFG_XXL
#define HY3X_RCFG_XXL 8, 6, 64, 4
#endif
#define HY3X_RCFG_(NAME, ...) HY3X_RCFG(NAME, __VA_ARGS__)
HY3X_RCFG_(TINY, HY3X_RCFG_TINY)
HY3X_RCFG_(MID, HY3X_RCFG_MID)
HY3X_RCFG_(LARGE, HY3X_RCFG_LARGE)
HY3X_RCFG_(XL, HY3X_RCFG_XL)
HY3X_RCFG_(XXL, HY3X_RCFG_XXL)
#undef HY3X_RCFG_
#undef HY3X_RCFG
template <int MT, int ME, int TG, int EG, int KC, int R>
__global__ __launch_bounds__(256) void k_router_gemm(const float *s32, const float *router, int T,
                                                     float *logits);
#define HY3X_ROUTER_GEMM(NAME)                                                                 \
  k_router_gemm<ROUTER_MT_##NAME, ROUTER_ME_##NAME, 4, 8, ROUTER_KC_##NAME, ROUTER_R_##NAME>
extern template __global__ void HY3X_ROUTER_GEMM(TINY)(const float *, const float *, int, float *);
extern template __global__ void HY3X_ROUTER_GEMM(MID)(const float *, const float *, int, float *);
extern template __global__ void HY3X_ROUTER_GEMM(LARGE)(const float *, const float *, int, float *);
extern template __global__ void HY3X_ROUTER_GEMM(XL)(const float *, const float *, int, float *);
extern template __global__ void HY3X_ROUTER_GEMM(XXL)(const float *, const float *, int, float *);
__global__ void k_topk(const float *logits, const float *bias, int has_bias, int K, float scale,
                       int T, int32_t *ids, float *wpre, float *wout, uint32_t *bits, int wt,
                       uint8_t *ranks);
__global__ void k_dispatch_list(const uint8_t *ranks, int T, int K, int NT, const uint32_t *bits,
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

// Tiles of grid margin for the kernels that deal whole tiles round-robin to
// the XCDs (xcd_tile_rr, hy3x_mfma_ops.h).
constexpr int XCD_TILE_RR_MARGIN = 7;
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
