// hy3x_mfma.hip -- grouped Q4_K x fp16 GEMMs on the matrix cores (prefill).
//
// A work tile is one expert, a slice of its weight matrix -- 64 rows of gate
// and of up (four waves x 16 rows), or 128 rows of down (four waves x 2 x 16
// rows) -- and up to 64 of its tokens (the dispatch tile list with NT = 64).
// Per Q4_K block column (256 of K) every lane turns the 8-element runs of its
// rows that the MFMA A operand needs into exact integers sc*q in fp16,
// straight from the GGUF bytes (q via the 0x6400 exponent-bias trick, one
// packed fp16 FMA with the sub-block scale), while the block's activations for
// the column sit in LDS. v_mfma_f32_16x16x32_f16 accumulates each block in
// fp32 (one MFMA spans exactly one Q4_K sub-block of 32); d, dmin and the
// mins are applied per block (see mfma_tile).
//
// Operand layouts (16x16x32): lane l holds A[l%16][8(l/16) .. +7] (row, k),
// B[8(l/16) .. +7][l%16] (k, token) and D[4(l/16) + i][l%16], i = 0..3. Within
// each run of 8 the k order is (0,2,1,3,4,6,5,7), the order the nibble unpack
// produces; activations are staged in that order (perm8).
#include "hy3x_kernels.h"
#include "hy3x_q4k.h"

namespace hy3x {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));  // 16 bytes as a native vector
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

constexpr int MT_TOK = 64;      // tokens per tile (dispatch NT)
constexpr int BT_STRIDE = 264;  // fp16 per staged token row (256 + 8 pad: conflict-free reads)
constexpr int BM_STRIDE = 24;   // fp16 per staged token sub-block-sum row (16 + 8 pad)

__device__ __forceinline__ uint32_t pk_fma_f16(uint32_t a, uint32_t b, uint32_t c) {
  const h2_t r = __builtin_elementwise_fma(as_h2(a), as_h2(b), as_h2(c));
  return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ uint32_t h2_splat(float v) {
  const _Float16 h = (_Float16)v;
  const h2_t r = {h, h};
  return __builtin_bit_cast(uint32_t, r);
}

// 6-bit scale and min of sub-block j of a Q4_K header (hy3.c:1001-1009).
__device__ __forceinline__ void scale_min(const u4_t &hdr, int j, uint32_t &sc, uint32_t &m) {
  const uint32_t s03 = hdr.y, s47 = hdr.z, s811 = hdr.w;
  if (j < 4) {
    sc = bfe(s03, 8 * j, 6);
    m = bfe(s47, 8 * j, 6);
  } else {
    sc = bfe(s811, 8 * (j - 4), 4) | (bfe(s03, 8 * (j - 4) + 6, 2) << 4);
    m = bfe(s811, 8 * (j - 4) + 4, 4) | (bfe(s47, 8 * (j - 4) + 6, 2) << 4);
  }
}

// A operand for sub-block 2p (hi = false) or 2p+1 (hi = true) with scale sc:
// the exact integers sc*q in fp16 (sc*q <= 945), from the 8 bytes
// qs[32p + 8g .. +7]. (1024 + q)*sc - 1024*sc is one fused multiply-add whose
// exact result is representable, so it is exact.
__device__ __forceinline__ h8_t dequant_a(u2_t q, bool hi, uint32_t sc) {
  const uint32_t mag = 0x64006400u, mask = 0x000F000Fu;
  const uint32_t sc2 = h2_splat((float)sc), nb2 = h2_splat(-1024.0f * (float)sc);
  const int sh = hi ? 4 : 0;
  u4_t p;
  p.x = pk_fma_f16(and_or(q.x >> sh, mask, mag), sc2, nb2);
  p.y = pk_fma_f16(and_or(q.x >> (8 + sh), mask, mag), sc2, nb2);
  p.z = pk_fma_f16(and_or(q.y >> sh, mask, mag), sc2, nb2);
  p.w = pk_fma_f16(and_or(q.y >> (8 + sh), mask, mag), sc2, nb2);
  return __builtin_bit_cast(h8_t, p);
}

template <bool GATEUP>
struct MfmaCfg {
  static constexpr int KD = GATEUP ? D : F;      // reduction length
  static constexpr int NROWS = GATEUP ? F : D;   // weight rows
  static constexpr int RG = GATEUP ? 1 : 2;      // 16-row groups per wave
  static constexpr int TROWS = 64 * RG;          // weight rows per tile
  static constexpr int NRT = NROWS / TROWS;      // row tiles
  static constexpr int NKB = KD / QK;            // Q4_K block columns
  static constexpr int NSUB = KD / 32;           // sub-blocks per activation row
  static constexpr int NMAT = GATEUP ? 2 : 1;    // gate and up, or down
};

struct MfmaSmem {
  _Float16 bt[2][MT_TOK][BT_STRIDE];  // activations of one block column (double-buffered)
  _Float16 bm[2][MT_TOK][BM_STRIDE];  // their sub-block sums as (hi, lo) fp16 pairs
  int32_t slot[MT_TOK], arow[MT_TOK];
};

// One work tile with NTT token tiles of 16 (n <= 16 * NTT tokens).
//
// Per block column: Dblk = sum over the 8 sub-blocks of MFMA(sc*q, x) (exact
// integer weights, fp16 activations, fp32 accumulation), Dmin = MFMA of the
// 6-bit mins against the tokens' sub-block sums of x (each sum carried as two
// fp16 parts), and acc += d * Dblk - dmin * Dmin with d, dmin of the D rows in
// fp32 -- the Q4_K identity sum_k w_k x_k = d sum_j sc_j sum_{k in j} q_k x_k
// - dmin sum_j m_j sum_{k in j} x_k (hy3.c:1036-1037).
//
// Pipeline: the weights (registers) and activations (registers, then the LDS
// buffer of the next column) of column kb+1 are fetched while column kb runs;
// one barrier per column.
template <bool GATEUP, int NTT>
__device__ __forceinline__ void mfma_tile(MfmaSmem &sm, const uint8_t *__restrict__ wq,
                                          const __half *__restrict__ act,
                                          const __half *__restrict__ act_sum, int e, int n,
                                          int rt, __half *__restrict__ h16m,
                                          float *__restrict__ out) {
  using C = MfmaCfg<GATEUP>;
  constexpr int RG = C::RG, NMAT = C::NMAT, NKB = C::NKB, KD = C::KD;
  constexpr int NTOK = 16 * NTT;
  constexpr int BU = NTOK / 8;  // B uint4 per thread: tokens (tid >> 5) + 8u
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, g = lane >> 4;

  const uint8_t *abase[RG][NMAT];
#pragma unroll
  for (int rg = 0; rg < RG; rg++)
#pragma unroll
    for (int m = 0; m < NMAT; m++)
      abase[rg][m] = wq + (size_t)e * EXPERT_BYTES + (size_t)(GATEUP ? m : 2) * MAT_BYTES +
                     (size_t)(rt * C::TROWS + 16 * (wave * RG + rg) + lr) * NKB * QB;

  // B staging: thread tid moves 16-byte chunk (tid & 31) of tokens (tid >> 5) + 8u,
  // and threads below 2 * NTOK half of one token's sub-block sums. Token slots
  // past n re-load token 0's row (its D columns are never stored), so every
  // prefetch register is written unconditionally.
  const int bc = tid & 31, bt0 = tid >> 5;
  const int arow0 = sm.arow[0];
  const u4_t *bsrc[BU];
#pragma unroll
  for (int u = 0; u < BU; u++) {
    const int ar = sm.arow[bt0 + 8 * u];
    bsrc[u] = reinterpret_cast<const u4_t *>(act + (size_t)(ar >= 0 ? ar : arow0) * KD) + bc;
  }
  const bool s_mover = tid < 2 * NTOK;
  const int ars = s_mover ? sm.arow[tid >> 1] : -1;
  const u4_t *ssrc =
      reinterpret_cast<const u4_t *>(act_sum + (size_t)(ars >= 0 ? ars : arow0) * C::NSUB * 2) +
      (tid & 1);

  u4_t bnext[BU];
  u4_t snext = {0u, 0u, 0u, 0u};
  u4_t hnext[RG][NMAT];
  u2_t qnext[RG][NMAT][4];
  // fetch column 0
#pragma unroll
  for (int u = 0; u < BU; u++) bnext[u] = bsrc[u][0];
  if (s_mover) snext = ssrc[0];
#pragma unroll
  for (int rg = 0; rg < RG; rg++)
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
      hnext[rg][m] = *reinterpret_cast<const u4_t *>(abase[rg][m]);
#pragma unroll
      for (int p = 0; p < 4; p++)
        qnext[rg][m][p] = *reinterpret_cast<const u2_t *>(abase[rg][m] + 16 + 32 * p + 8 * g);
    }

  f4_t acc[RG][NMAT][NTT];
#pragma unroll
  for (int rg = 0; rg < RG; rg++)
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
      for (int t = 0; t < NTT; t++) acc[rg][m][t] = (f4_t){0.f, 0.f, 0.f, 0.f};
  const f4_t zero4 = {0.f, 0.f, 0.f, 0.f};
  h8_t zero8;
#pragma unroll
  for (int u = 0; u < 8; u++) zero8[u] = (_Float16)0.0f;

  for (int kb = 0; kb < NKB; kb++) {
    const int buf = kb & 1;
#pragma unroll
    for (int u = 0; u < BU; u++) *reinterpret_cast<u4_t *>(&sm.bt[buf][bt0 + 8 * u][8 * bc]) = bnext[u];
    if (s_mover) *reinterpret_cast<u4_t *>(&sm.bm[buf][tid >> 1][8 * (tid & 1)]) = snext;
    u4_t hdr[RG][NMAT];
    u2_t qv[RG][NMAT][4];
#pragma unroll
    for (int rg = 0; rg < RG; rg++)
#pragma unroll
      for (int m = 0; m < NMAT; m++) {
        hdr[rg][m] = hnext[rg][m];
#pragma unroll
        for (int p = 0; p < 4; p++) qv[rg][m][p] = qnext[rg][m][p];
      }
    __syncthreads();  // buf is staged; buf ^ 1 is no longer read (column kb - 1 is done)
    // fetch column kb + 1 (the last iteration re-fetches column kb: harmless, no branch)
    const int kn = kb + 1 < NKB ? kb + 1 : kb;
#pragma unroll
    for (int u = 0; u < BU; u++) bnext[u] = bsrc[u][kn * (QK / 8)];
    if (s_mover) snext = ssrc[kn * 2];
#pragma unroll
    for (int rg = 0; rg < RG; rg++)
#pragma unroll
      for (int m = 0; m < NMAT; m++) {
        const uint8_t *bp = abase[rg][m] + (size_t)kn * QB;
        hnext[rg][m] = *reinterpret_cast<const u4_t *>(bp);
#pragma unroll
        for (int p = 0; p < 4; p++)
          qnext[rg][m][p] = *reinterpret_cast<const u2_t *>(bp + 16 + 32 * p + 8 * g);
      }
    f4_t dblk[RG][NMAT][NTT];
#pragma unroll
    for (int sb = 0; sb < 8; sb++) {
      h8_t a[RG][NMAT];
#pragma unroll
      for (int rg = 0; rg < RG; rg++)
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
          uint32_t sc, mn;
          scale_min(hdr[rg][m], sb, sc, mn);
          a[rg][m] = dequant_a(qv[rg][m][sb >> 1], sb & 1, sc);
        }
#pragma unroll
      for (int t = 0; t < NTT; t++) {
        const h8_t b = *reinterpret_cast<const h8_t *>(&sm.bt[buf][16 * t + lr][32 * sb + 8 * g]);
#pragma unroll
        for (int rg = 0; rg < RG; rg++)
#pragma unroll
          for (int m = 0; m < NMAT; m++)
            dblk[rg][m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                a[rg][m], b, sb == 0 ? zero4 : dblk[rg][m][t], 0, 0, 0);
      }
    }
    // mins term and per-block scales
#pragma unroll
    for (int rg = 0; rg < RG; rg++)
#pragma unroll
      for (int m = 0; m < NMAT; m++) {
        const u4_t h = hdr[rg][m];
        const float d_own = fp16_quirk(h.x & 0xffffu), dm_own = fp16_quirk(h.x >> 16);
        float dr[4], dmr[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {  // d, dmin of D rows 4g + i live in lanes 4g + i
          dr[i] = __shfl(d_own, 4 * g + i, 64);
          dmr[i] = __shfl(dm_own, 4 * g + i, 64);
        }
        h8_t am = zero8;  // A of the mins MFMA: k = 2j + h (h: hi/lo part), k < 16
        if (g < 2) {
#pragma unroll
          for (int u = 0; u < 4; u++) {
            uint32_t sc, mn;
            scale_min(h, 4 * g + u, sc, mn);
            am[2 * u] = (_Float16)(float)mn;
            am[2 * u + 1] = (_Float16)(float)mn;
          }
        }
#pragma unroll
        for (int t = 0; t < NTT; t++) {
          const h8_t bmv =
              g < 2 ? *reinterpret_cast<const h8_t *>(&sm.bm[buf][16 * t + lr][8 * g]) : zero8;
          const f4_t dmin4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(am, bmv, zero4, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; i++)
            acc[rg][m][t][i] = __builtin_fmaf(dr[i], dblk[rg][m][t][i],
                                              __builtin_fmaf(-dmr[i], dmin4[i], acc[rg][m][t][i]));
        }
      }
  }
  // epilogue: lane holds D[4g + i][lr] of token tile t, row group rg
#pragma unroll
  for (int t = 0; t < NTT; t++) {
    const int tok = 16 * t + lr;
    if (tok < n) {
      const int slot = sm.slot[tok];
#pragma unroll
      for (int rg = 0; rg < RG; rg++) {
        const int r0 = rt * C::TROWS + 16 * (wave * RG + rg) + 4 * g;
        if constexpr (GATEUP) {
          float hv[4];
#pragma unroll
          for (int i = 0; i < 4; i++) hv[i] = silu(acc[rg][0][t][i]) * acc[rg][NMAT - 1][t][i];
          // rows r0 .. r0+3 sit at perm8 positions r0, r0+2, r0+1, r0+3
          const h4_t v = {(_Float16)hv[0], (_Float16)hv[2], (_Float16)hv[1], (_Float16)hv[3]};
          *reinterpret_cast<h4_t *>(&h16m[(size_t)slot * F + r0]) = v;
        } else {
          *reinterpret_cast<float4 *>(&out[(size_t)slot * D + r0]) =
              make_float4(acc[rg][0][t][0], acc[rg][0][t][1], acc[rg][0][t][2], acc[rg][0][t][3]);
        }
      }
    }
  }
}

// Launch order -> work item, so that consecutive work items run on one XCD
// (workgroups are dealt to the 8 XCDs round-robin): the row tiles of one
// expert tile share its activations in that XCD's L2, and consecutive token
// tiles of one expert share its weights.
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
  const int q = nblocks >> 3, r = nblocks & 7, x = bid & 7, i = bid >> 3;
  return x * q + (x < r ? x : r) + i;
}

// Grouped GEMM over the tile list. GATEUP: A = gate and up rows of the expert
// (K = 4096), B = staged s, epilogue h = silu(g) * u -> h16m[slot][perm8(row)]
// (fp16). Otherwise A = down rows (K = 1536), B = h16m, out[slot][row] fp32.
// act_sum: sub-block sums of each activation row as (hi, lo) fp16 pairs.
template <bool GATEUP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_moe_mfma(
    const uint8_t *__restrict__ wq, const __half *__restrict__ act,
    const __half *__restrict__ act_sum, const int32_t *__restrict__ list,
    const int4 *__restrict__ tiles, const int32_t *__restrict__ n_tiles, int T, int K,
    __half *__restrict__ h16m, float *__restrict__ out) {
  using C = MfmaCfg<GATEUP>;
  const int w = xcd_remap(blockIdx.x, gridDim.x);
  const int tile = w / C::NRT, rt = w % C::NRT;
  if (tile >= *n_tiles) return;
  const int4 td = tiles[tile];
  const int e = td.x, o = td.y, n = td.z;
  __shared__ __attribute__((aligned(16))) MfmaSmem sm;
  const int tid = threadIdx.x;
  if (tid < MT_TOK) {
    const int s = tid < n ? list[o + tid] : -1;
    sm.slot[tid] = s;
    // activation row: gate/up reads s of the token, down reads h of the slot
    sm.arow[tid] = s < 0 ? -1 : (GATEUP ? (s < T * K ? s / K : s - T * K) : s);
  }
  __syncthreads();
  switch ((n + 15) >> 4) {
    case 1: mfma_tile<GATEUP, 1>(sm, wq, act, act_sum, e, n, rt, h16m, out); break;
    case 2: mfma_tile<GATEUP, 2>(sm, wq, act, act_sum, e, n, rt, h16m, out); break;
    case 3: mfma_tile<GATEUP, 3>(sm, wq, act, act_sum, e, n, rt, h16m, out); break;
    default: mfma_tile<GATEUP, 4>(sm, wq, act, act_sum, e, n, rt, h16m, out); break;
  }
}

// Sub-block sums of one fp16 row of n32 * 32 values, as (hi, lo) fp16 pairs:
// hi = fp16(sum), lo = fp16(sum - hi). One lane per sub-block.
__device__ __forceinline__ void row_subsums(const __half *__restrict__ row, int n32,
                                            __half *__restrict__ dst) {
  for (int j = threadIdx.x; j < n32; j += blockDim.x) {
    const uint4 *src = reinterpret_cast<const uint4 *>(row + 32 * j);
    float sum = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const uint4 q = src[v];
      const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const h2_t p = as_h2(w[u]);
        sum += (float)p[0];
        sum += (float)p[1];
      }
    }
    const _Float16 hi = (_Float16)sum;
    const _Float16 lo = (_Float16)(sum - (float)hi);
    const h2_t r = {hi, lo};
    *reinterpret_cast<h2_t *>(dst + 2 * j) = r;
  }
}

// fp16 copy of s in the MFMA run order (perm8) for the gate/up B operand, and
// its 128 sub-block sums.
__global__ __launch_bounds__(256) void k_stage_mfma(const float *__restrict__ s32,
                                                    __half *__restrict__ s16m,
                                                    __half *__restrict__ ssum) {
  const int t = blockIdx.x;
  for (int j = threadIdx.x; j < D; j += 256)
    s16m[(size_t)t * D + perm8(j)] = __float2half(s32[(size_t)t * D + j]);
  __syncthreads();
  row_subsums(s16m + (size_t)t * D, D / 32, ssum + (size_t)t * (D / 32) * 2);
}

// The 48 sub-block sums of every h row (down-GEMM mins operand); one wave per slot.
__global__ __launch_bounds__(64) void k_hsums(const __half *__restrict__ h16m,
                                              __half *__restrict__ hsum) {
  const int slot = blockIdx.x;
  row_subsums(h16m + (size_t)slot * F, F / 32, hsum + (size_t)slot * (F / 32) * 2);
}

template __global__ void k_moe_mfma<true>(const uint8_t *, const __half *, const __half *,
                                          const int32_t *, const int4 *, const int32_t *, int,
                                          int, __half *, float *);
template __global__ void k_moe_mfma<false>(const uint8_t *, const __half *, const __half *,
                                           const int32_t *, const int4 *, const int32_t *, int,
                                           int, __half *, float *);

}  // namespace hy3x
