// hy3x_mfma.hip -- grouped Q4_K x fp16 GEMMs on the matrix cores (prefill).
//
// A work tile is one expert, a slice of its weight matrix -- 64 rows of gate
// and of up (four waves x 16 rows), or 128 rows of down (four waves x 2 x 16
// rows) -- and up to 64 of its tokens (the dispatch tile list with NT = 64).
// Per Q4_K block column (256 of K) every lane turns the 8-element runs of its
// weight row that the MFMA needs into exact integers sc*q in fp16, straight
// from the GGUF bytes (q via the 0x6400 exponent-bias trick, one packed fp16
// FMA with the sub-block scale), while the block's activations for the column
// sit in LDS. v_mfma_f32_16x16x32_f16 accumulates each block in fp32 (one MFMA
// spans exactly one Q4_K sub-block of 32); d, dmin and the mins are applied
// per block (see mfma_tile).
//
// Operand layouts (16x16x32): lane l holds A[l%16][8(l/16) .. +7] (row, k),
// B[8(l/16) .. +7][l%16] (k, column) and D[4(l/16) + i][l%16], i = 0..3. Here
// A = activations (rows = tokens) and B = weights (columns = weight rows), so
// a lane's D values all belong to ONE weight row (its own: l%16) and four
// tokens. Within each run of 8 the k order is (0,2,1,3,4,6,5,7), the order
// the nibble unpack produces; activations are staged in that order (perm8).
#include "hy3x_kernels.h"
#include "hy3x_q4k.h"

namespace hy3x {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));  // 16 bytes as a native vector
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

constexpr int MT_TOK = 64;      // tokens per tile (dispatch NT)
constexpr int BT_STRIDE = 264;  // fp16 per staged token row (256 + 8 pad: conflict-free reads)
constexpr int BM_STRIDE = 40;   // fp16 per staged token mins row (32 + 8 pad)

__device__ __forceinline__ uint32_t pk_fma_f16(uint32_t a, h2_t b, h2_t c) {
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(as_h2(a), b, c));
}

// The 6-bit scales and mins of a Q4_K block (hy3.c:1001-1009) as bytes:
// sc[0] = sc_0..3, sc[1] = sc_4..7, mn[0] = m_0..3, mn[1] = m_4..7.
struct Scales6 {
  uint32_t sc[2], mn[2];
};
__device__ __forceinline__ Scales6 unpack_scales(const u4_t &h) {
  // j < 4: sc_j = s[j] & 63, m_j = s[j+4] & 63
  // j >= 4: sc_j = (s[j+4] & 15) | (s[j-4] >> 6) << 4, m_j = (s[j+4] >> 4) | (s[j] >> 6) << 4
  Scales6 r;
  r.sc[0] = h.y & 0x3F3F3F3Fu;
  r.mn[0] = h.z & 0x3F3F3F3Fu;
  r.sc[1] = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
  r.mn[1] = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
  return r;
}

// fp16 pair (byte J0 of w, byte J1 of w) (values <= 63): the bytes go into the
// mantissa of 1024.0, then 1024 is subtracted (both steps exact).
template <int J0, int J1>
__device__ __forceinline__ h2_t bytes_h2(uint32_t w) {
  constexpr uint32_t sel = 0x0C000C00u | ((uint32_t)J1 << 16) | (uint32_t)J0;  // 0x0C: zero byte
  const uint32_t v = __builtin_amdgcn_perm(w, w, sel) | 0x64006400u;
  return as_h2(v) + (h2_t){(_Float16)-1024.0f, (_Float16)-1024.0f};
}

// Weight operands of sub-blocks 2p (lo) and 2p+1 (hi) from the 8 bytes
// qs[32p + 8g .. +7] of this lane's row: the exact integers sc*q in fp16
// (sc*q <= 945). sc = (sc_lo, sc_hi). Low nibbles: 0x6400 | q = 1024 + q,
// times sc_lo, minus 1024 sc_lo. High nibbles, left in place: 0x6400 | 16q =
// 1024 + 16q, times sc_hi/16, minus 64 sc_hi. Each is one fused multiply-add
// whose exact result is representable, so it is exact.
__device__ __forceinline__ void dequant_pair(u2_t q, h2_t sc, h8_t &w_lo, h8_t &w_hi) {
  const uint32_t mag = 0x64006400u, m_lo = 0x000F000Fu, m_hi = 0x00F000F0u;
  const h2_t mul = sc * (h2_t){(_Float16)1.0f, (_Float16)0.0625f};     // (sc_lo, sc_hi/16)
  const h2_t add = sc * (h2_t){(_Float16)-1024.0f, (_Float16)-64.0f};  // (-1024 sc_lo, -64 sc_hi)
  const h2_t ml = {mul[0], mul[0]}, al = {add[0], add[0]};
  const h2_t mh = {mul[1], mul[1]}, ah = {add[1], add[1]};
  const uint32_t x8 = q.x >> 8, y8 = q.y >> 8;
  u4_t lo, hi;
  lo.x = pk_fma_f16(and_or(q.x, m_lo, mag), ml, al);
  lo.y = pk_fma_f16(and_or(x8, m_lo, mag), ml, al);
  lo.z = pk_fma_f16(and_or(q.y, m_lo, mag), ml, al);
  lo.w = pk_fma_f16(and_or(y8, m_lo, mag), ml, al);
  hi.x = pk_fma_f16(and_or(q.x, m_hi, mag), mh, ah);
  hi.y = pk_fma_f16(and_or(x8, m_hi, mag), mh, ah);
  hi.z = pk_fma_f16(and_or(q.y, m_hi, mag), mh, ah);
  hi.w = pk_fma_f16(and_or(y8, m_hi, mag), mh, ah);
  w_lo = __builtin_bit_cast(h8_t, lo);
  w_hi = __builtin_bit_cast(h8_t, hi);
}

// -dmin * m_j for sub-blocks j = 2g and 2g+1 of this lane's row, each split
// exactly into two fp16 parts (dmin: 11 significant bits, m: 6, so the
// product is exact in fp32 and hi + lo carries it to 22 bits), laid out for
// the mins MFMA: k = 4j' + c, c = (hi, hi, lo, lo) against the staged
// activation sums (Sh, Sl, Sh, Sl): the four cross products of the two splits.
__device__ __forceinline__ h8_t mins_operand(float dmin, uint32_t m2) {
  const float v0 = -dmin * (float)(m2 & 0xFFu), v1 = -dmin * (float)((m2 >> 8) & 0xFFu);
  const _Float16 h0 = (_Float16)v0, h1 = (_Float16)v1;
  const _Float16 l0 = (_Float16)(v0 - (float)h0), l1 = (_Float16)(v1 - (float)h1);
  return (h8_t){h0, h0, l0, l0, h1, h1, l1, l1};
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
  _Float16 bm[2][MT_TOK][BM_STRIDE];  // their sub-block sums as (Sh, Sl, Sh, Sl) per sub-block
  int32_t slot[MT_TOK], arow[MT_TOK];
};

// One work tile with NTT token tiles of 16 (n <= 16 * NTT tokens).
//
// Per block column, for each (token tile, weight row group, matrix):
//   Dblk = sum over the 8 sub-blocks of MFMA(x, sc*q)   (exact integer weights)
//   acc = MFMA(S, -dmin*m, acc)                         (mins term)
//   acc += d * Dblk                                     (fp32, d of the lane's row)
// -- the Q4_K identity sum_k w_k x_k = d sum_j sc_j sum_{k in j} q_k x_k
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
  constexpr int BU = NTOK / 8;  // activation uint4 per thread: tokens (tid >> 5) + 8u
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, g = lane >> 4;

  const uint8_t *abase[RG][NMAT];
#pragma unroll
  for (int rg = 0; rg < RG; rg++)
#pragma unroll
    for (int m = 0; m < NMAT; m++)
      abase[rg][m] = wq + (size_t)e * EXPERT_BYTES + (size_t)(GATEUP ? m : 2) * MAT_BYTES +
                     (size_t)(rt * C::TROWS + 16 * (wave * RG + rg) + lr) * NKB * QB;

  // Activation staging: thread tid moves 16-byte chunk (tid & 31) of tokens
  // (tid >> 5) + 8u, and threads below 4 * NTOK a quarter of one token's sums
  // row. Token slots past n re-load token 0's row (their D rows are never
  // stored), so every prefetch register is written unconditionally.
  const int bc = tid & 31, bt0 = tid >> 5;
  const int arow0 = sm.arow[0];
  const u4_t *bsrc[BU];
#pragma unroll
  for (int u = 0; u < BU; u++) {
    const int ar = sm.arow[bt0 + 8 * u];
    bsrc[u] = reinterpret_cast<const u4_t *>(act + (size_t)(ar >= 0 ? ar : arow0) * KD) + bc;
  }
  const bool s_mover = tid < 4 * NTOK;
  const int ars = s_mover ? sm.arow[tid >> 2] : -1;
  const u4_t *ssrc =
      reinterpret_cast<const u4_t *>(act_sum + (size_t)(ars >= 0 ? ars : arow0) * C::NSUB * 4) +
      (tid & 3);

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
  const f4_t zero4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int rg = 0; rg < RG; rg++)
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
      for (int t = 0; t < NTT; t++) acc[rg][m][t] = zero4;

  for (int kb = 0; kb < NKB; kb++) {
    const int buf = kb & 1;
#pragma unroll
    for (int u = 0; u < BU; u++) *reinterpret_cast<u4_t *>(&sm.bt[buf][bt0 + 8 * u][8 * bc]) = bnext[u];
    if (s_mover) *reinterpret_cast<u4_t *>(&sm.bm[buf][tid >> 2][8 * (tid & 3)]) = snext;
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
    if (s_mover) snext = ssrc[kn * 4];
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

    Scales6 sc6[RG][NMAT];
#pragma unroll
    for (int rg = 0; rg < RG; rg++)
#pragma unroll
      for (int m = 0; m < NMAT; m++) sc6[rg][m] = unpack_scales(hdr[rg][m]);
    f4_t dblk[RG][NMAT][NTT];
#pragma unroll
    for (int p = 0; p < 4; p++) {  // sub-blocks 2p and 2p+1
      h8_t wf[2][RG][NMAT];
#pragma unroll
      for (int rg = 0; rg < RG; rg++)
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
          const uint32_t w = sc6[rg][m].sc[p >> 1];
          const h2_t sc = (p & 1) ? bytes_h2<2, 3>(w) : bytes_h2<0, 1>(w);
          dequant_pair(qv[rg][m][p], sc, wf[0][rg][m], wf[1][rg][m]);
        }
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int sb = 2 * p + h;
#pragma unroll
        for (int t = 0; t < NTT; t++) {
          const h8_t x =
              *reinterpret_cast<const h8_t *>(&sm.bt[buf][16 * t + lr][32 * sb + 8 * g]);
#pragma unroll
          for (int rg = 0; rg < RG; rg++)
#pragma unroll
            for (int m = 0; m < NMAT; m++)
              dblk[rg][m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                  x, wf[h][rg][m], sb == 0 ? zero4 : dblk[rg][m][t], 0, 0, 0);
        }
      }
    }
    // per-block scale d (of this lane's row) and the mins MFMA
    h8_t sv[NTT];
#pragma unroll
    for (int t = 0; t < NTT; t++)
      sv[t] = *reinterpret_cast<const h8_t *>(&sm.bm[buf][16 * t + lr][8 * g]);
#pragma unroll
    for (int rg = 0; rg < RG; rg++)
#pragma unroll
      for (int m = 0; m < NMAT; m++) {
        const u4_t hd = hdr[rg][m];
        const float d = fp16_quirk(hd.x & 0xffffu), dmin = fp16_quirk(hd.x >> 16);
        // m_{2g}, m_{2g+1}: bytes 2(g & 1), 2(g & 1) + 1 of mn[g >> 1]
        const uint32_t mw = (g >> 1) ? sc6[rg][m].mn[1] : sc6[rg][m].mn[0];
        const h8_t mo = mins_operand(dmin, (g & 1) ? (mw >> 16) : mw);
#pragma unroll
        for (int t = 0; t < NTT; t++) {
          acc[rg][m][t] =
              __builtin_amdgcn_mfma_f32_16x16x32_f16(sv[t], mo, acc[rg][m][t], 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; i++)
            acc[rg][m][t][i] = __builtin_fmaf(d, dblk[rg][m][t][i], acc[rg][m][t][i]);
        }
      }
  }
  // epilogue: lane holds D[token 16t + 4g + i][row] for its own weight row
#pragma unroll
  for (int rg = 0; rg < RG; rg++) {
    const int r = rt * C::TROWS + 16 * (wave * RG + rg) + lr;
#pragma unroll
    for (int t = 0; t < NTT; t++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int tok = 16 * t + 4 * g + i;
        if (tok < n) {
          const int slot = sm.slot[tok];
          if constexpr (GATEUP) {
            h16m[(size_t)slot * F + perm8(r)] =
                __float2half(silu(acc[rg][0][t][i]) * acc[rg][1][t][i]);
          } else {
            out[(size_t)slot * D + r] = acc[rg][0][t][i];
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

// Grouped GEMM over the tile list. GATEUP: weights = gate and up rows of the
// expert (K = 4096), activations = staged s, epilogue h = silu(g) * u ->
// h16m[slot][perm8(row)] (fp16). Otherwise weights = down rows (K = 1536),
// activations = h16m, out[slot][row] fp32. act_sum: sub-block sums of each
// activation row as (Sh, Sl, Sh, Sl) fp16 quadruples.
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

// Sub-block sums of one fp16 row of n32 * 32 values, as (Sh, Sl, Sh, Sl) with
// Sh = fp16(sum), Sl = fp16(sum - Sh). One lane per sub-block.
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
    *reinterpret_cast<h2_t *>(dst + 4 * j) = r;
    *reinterpret_cast<h2_t *>(dst + 4 * j + 2) = r;
  }
}

// fp16 copy of s in the MFMA run order (perm8) for the gate/up activations,
// and its 128 sub-block sums.
__global__ __launch_bounds__(256) void k_stage_mfma(const float *__restrict__ s32,
                                                    __half *__restrict__ s16m,
                                                    __half *__restrict__ ssum) {
  const int t = blockIdx.x;
  for (int j = threadIdx.x; j < D; j += 256)
    s16m[(size_t)t * D + perm8(j)] = __float2half(s32[(size_t)t * D + j]);
  __syncthreads();
  row_subsums(s16m + (size_t)t * D, D / 32, ssum + (size_t)t * (D / 32) * 4);
}

// The 48 sub-block sums of every h row (down-GEMM mins operand); one wave per slot.
__global__ __launch_bounds__(64) void k_hsums(const __half *__restrict__ h16m,
                                              __half *__restrict__ hsum) {
  const int slot = blockIdx.x;
  row_subsums(h16m + (size_t)slot * F, F / 32, hsum + (size_t)slot * (F / 32) * 4);
}

template __global__ void k_moe_mfma<true>(const uint8_t *, const __half *, const __half *,
                                          const int32_t *, const int4 *, const int32_t *, int,
                                          int, __half *, float *);
template __global__ void k_moe_mfma<false>(const uint8_t *, const __half *, const __half *,
                                           const int32_t *, const int4 *, const int32_t *, int,
                                           int, __half *, float *);

}  // namespace hy3x
