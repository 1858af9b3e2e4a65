// hy3x_mfma.hip -- grouped Q4_K x fp16 GEMMs on the matrix cores (prefill).
//
// A work tile is one expert, a 64-row slice of its weight matrix (gate and up
// together, or down), and up to 64 of its tokens (the dispatch tile list with
// NT = 64). Four waves each own 16 weight rows. Per Q4_K block column (256 of
// K) every lane dequantises the 8-element runs of its row that the MFMA A
// operand needs -- straight from the GGUF bytes into fp16 registers:
//   w = d*sc*q - dmin*m  (hy3.c:1036-1037), q from the 0x6400 exponent-bias
// trick minus 1024 (exact), then one packed fp16 FMA with the sub-block's
// scale and min -- while the block stages the tokens' fp16 activations for the
// column in LDS. v_mfma_f32_16x16x32_f16 then accumulates in fp32 over the
// whole K. One 16x16x32 MFMA spans exactly one Q4_K sub-block.
//
// Operand layouts (16x16x32): lane l holds A[l%16][8(l/16) .. +7] (row, k),
// B[8(l/16) .. +7][l%16] (k, token) and D[4(l/16) + i][l%16], i = 0..3. Within
// each run of 8 the k order is (0,2,1,3,4,6,5,7), the order the nibble unpack
// produces; activations are staged in that order (perm8).
#include "hy3x_kernels.h"
#include "hy3x_q4k.h"

namespace hy3x {

typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

constexpr int MT_ROWS = 64;   // weight rows per tile
constexpr int MT_TOK = 64;    // tokens per tile (dispatch NT)
constexpr int BT_STRIDE = 264; // fp16 per staged token row (256 + 8 pad)

__device__ __forceinline__ uint32_t pk_add_f16(uint32_t a, uint32_t b) {
  return __builtin_bit_cast(uint32_t, as_h2(a) + as_h2(b));
}
__device__ __forceinline__ uint32_t pk_fma_f16(uint32_t a, uint32_t b, uint32_t c) {
  const h2_t r = __builtin_elementwise_fma(as_h2(a), as_h2(b), as_h2(c));
  return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ uint32_t h2_splat(float v) {
  const _Float16 h = (_Float16)v;
  const h2_t r = {h, h};
  return __builtin_bit_cast(uint32_t, r);
}

// Per-lane state of one Q4_K block of one row: fp16 pairs (sc_j, sc_j) and
// (-1024 sc_j, -1024 sc_j) for the 8 sub-blocks, and the 6-bit mins. All
// exact in fp16.
struct BlockI16 {
  uint32_t sc2[8], nb2[8];
  uint32_t m[8];
};

__device__ __forceinline__ BlockI16 block_i16(const uint4 &hdr) {
  const uint32_t s03 = hdr.y, s47 = hdr.z, s811 = hdr.w;
  BlockI16 r;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    uint32_t sc, m;
    if (j < 4) {
      sc = bfe(s03, 8 * j, 6);
      m = bfe(s47, 8 * j, 6);
    } else {
      sc = bfe(s811, 8 * (j - 4), 4) | (bfe(s03, 8 * (j - 4) + 6, 2) << 4);
      m = bfe(s811, 8 * (j - 4) + 4, 4) | (bfe(s47, 8 * (j - 4) + 6, 2) << 4);
    }
    r.sc2[j] = h2_splat((float)sc);
    r.nb2[j] = h2_splat(-1024.0f * (float)sc);
    r.m[j] = m;
  }
  return r;
}

// A operand for sub-block 2p (hi = false) or 2p+1 (hi = true): the exact
// integers sc*q in fp16 (sc*q <= 945), from the 8 bytes qs[32p + 8g .. +7].
// (1024 + q)*sc - 1024*sc is computed by one fused multiply-add whose exact
// result is representable, so it is exact.
__device__ __forceinline__ h8_t dequant_a(uint2 q, bool hi, uint32_t sc2, uint32_t nb2) {
  const uint32_t mag = 0x64006400u, mask = 0x000F000Fu;
  const int sh = hi ? 4 : 0;
  uint32_t p[4];
  p[0] = and_or(q.x >> sh, mask, mag);
  p[1] = and_or(q.x >> (8 + sh), mask, mag);
  p[2] = and_or(q.y >> sh, mask, mag);
  p[3] = and_or(q.y >> (8 + sh), mask, mag);
#pragma unroll
  for (int i = 0; i < 4; i++) p[i] = pk_fma_f16(p[i], sc2, nb2);
  return __builtin_bit_cast(h8_t, *reinterpret_cast<uint4 *>(p));
}

// Grouped GEMM over the tile list. GATEUP: A = gate and up rows of the expert
// (K = 4096), B = staged s, epilogue h = silu(g) * u -> h16m[slot][perm8(row)]
// (fp16). Otherwise A = down rows (K = 1536), B = h16m, out[slot][row] fp32.
//
// Per block column: Dblk = sum over the 8 sub-blocks of MFMA(sc*q, x) (exact
// integer weights, fp16 activations, fp32 accumulation), Dmin = MFMA of the
// 6-bit mins against the tokens' sub-block sums of x (each sum split into two
// fp16 parts), and acc += d * Dblk - dmin * Dmin with d, dmin of the D rows in
// fp32 -- the Q4_K identity sum_k w_k x_k = d sum_j sc_j sum_{k in j} q_k x_k
// - dmin sum_j m_j sum_{k in j} x_k.
template <bool GATEUP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void k_moe_mfma(const uint8_t *__restrict__ wq,
                                                  const __half *__restrict__ act,
                                                  const int32_t *__restrict__ list,
                                                  const int4 *__restrict__ tiles,
                                                  const int32_t *__restrict__ n_tiles, int T,
                                                  int K, __half *__restrict__ h16m,
                                                  float *__restrict__ out) {
  constexpr int KD = GATEUP ? D : F;          // reduction length
  constexpr int NROWS = GATEUP ? F : D;        // weight rows
  constexpr int NRT = NROWS / MT_ROWS;         // row tiles
  constexpr int NKB = KD / QK;                 // Q4_K block columns
  constexpr int NMAT = GATEUP ? 2 : 1;
  const int tile = blockIdx.x / NRT, rt = blockIdx.x % NRT;
  if (tile >= *n_tiles) return;
  const int4 td = tiles[tile];
  const int e = td.x, o = td.y, n = td.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, g = lane >> 4;

  __shared__ __attribute__((aligned(16))) _Float16 bt[MT_TOK][BT_STRIDE];
  __shared__ __attribute__((aligned(16))) _Float16 bm[MT_TOK][16];  // sub-block sums (hi, lo)
  __shared__ int32_t slot_l[MT_TOK], arow_l[MT_TOK];
  if (tid < MT_TOK) {
    const int s = tid < n ? list[o + tid] : -1;
    slot_l[tid] = s;
    // activation row of the token: gate/up reads s by token, down reads h by slot
    arow_l[tid] = s < 0 ? -1 : (GATEUP ? (s < T * K ? s / K : s - T * K) : s);
  }
  const int ntt = (n + 15) >> 4;  // token tiles of 16 in use

  const int row = rt * MT_ROWS + 16 * wave + lr;  // this lane's A row
  const uint8_t *abase[NMAT];
#pragma unroll
  for (int m = 0; m < NMAT; m++)
    abase[m] = wq + (size_t)e * EXPERT_BYTES + (size_t)(GATEUP ? m : 2) * MAT_BYTES +
               (size_t)row * NKB * QB;

  f4_t acc[NMAT][4];
#pragma unroll
  for (int m = 0; m < NMAT; m++)
#pragma unroll
    for (int t = 0; t < 4; t++) acc[m][t] = (f4_t){0.f, 0.f, 0.f, 0.f};
  const f4_t zero4 = {0.f, 0.f, 0.f, 0.f};

  __syncthreads();
  for (int kb = 0; kb < NKB; kb++) {
    // this lane's A bytes for block column kb (issued before the B staging)
    uint4 hdr[NMAT];
    uint2 qv[NMAT][4];
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
      const uint8_t *bp = abase[m] + (size_t)kb * QB;
      hdr[m] = *reinterpret_cast<const uint4 *>(bp);
#pragma unroll
      for (int p = 0; p < 4; p++) qv[m][p] = *reinterpret_cast<const uint2 *>(bp + 16 + 32 * p + 8 * g);
    }
    // stage B: tokens x 256 fp16 of this column (32 uint4 per token)
    for (int q = tid; q < MT_TOK * 32; q += 256) {
      const int t = q >> 5, c = q & 31;
      uint4 v = make_uint4(0u, 0u, 0u, 0u);
      const int ar = arow_l[t];
      if (ar >= 0) v = reinterpret_cast<const uint4 *>(act + (size_t)ar * KD + kb * QK)[c];
      *reinterpret_cast<uint4 *>(&bt[t][8 * c]) = v;
    }
    __syncthreads();
    // sub-block sums of the staged activations, split into two fp16 parts
    for (int q = tid; q < MT_TOK * 8; q += 256) {
      const int t = q >> 3, j = q & 7;
      const h8_t *src = reinterpret_cast<const h8_t *>(&bt[t][32 * j]);
      const h2_t one = {(_Float16)1.0f, (_Float16)1.0f};
      float sum = 0.0f;
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const h8_t v = src[u];
        sum = __builtin_amdgcn_fdot2((h2_t){v[0], v[1]}, one, sum, false);
        sum = __builtin_amdgcn_fdot2((h2_t){v[2], v[3]}, one, sum, false);
        sum = __builtin_amdgcn_fdot2((h2_t){v[4], v[5]}, one, sum, false);
        sum = __builtin_amdgcn_fdot2((h2_t){v[6], v[7]}, one, sum, false);
      }
      const _Float16 hi = (_Float16)sum;
      const _Float16 lo = (_Float16)(sum - (float)hi);
      bm[t][2 * j] = hi;
      bm[t][2 * j + 1] = lo;
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
      const BlockI16 bi = block_i16(hdr[m]);
      // d, dmin of the D rows 4g + i (row lr of this lane's A is row 4g+i of another lane)
      const float d_own = fp16_quirk(hdr[m].x & 0xffffu), dm_own = fp16_quirk(hdr[m].x >> 16);
      float dr[4], dmr[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        dr[i] = __shfl(d_own, 4 * g + i, 64);
        dmr[i] = __shfl(dm_own, 4 * g + i, 64);
      }
      // mins operand: k = 2j + h (h: hi/lo part of the sum), k < 16
      h8_t am;
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const _Float16 mv = g < 2 ? (_Float16)(float)bi.m[4 * g + u] : (_Float16)0.0f;
        am[2 * u] = mv;
        am[2 * u + 1] = mv;
      }
      f4_t dblk[4];
#pragma unroll
      for (int sb = 0; sb < 8; sb++) {
        const h8_t a = dequant_a(qv[m][sb >> 1], sb & 1, bi.sc2[sb], bi.nb2[sb]);
#pragma unroll
        for (int t = 0; t < 4; t++) {
          if (t < ntt) {
            const h8_t b = *reinterpret_cast<const h8_t *>(&bt[16 * t + lr][32 * sb + 8 * g]);
            dblk[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, sb == 0 ? zero4 : dblk[t], 0,
                                                             0, 0);
          }
        }
      }
#pragma unroll
      for (int t = 0; t < 4; t++) {
        if (t < ntt) {
          h8_t bmv;
          if (g < 2) {
            bmv = *reinterpret_cast<const h8_t *>(&bm[16 * t + lr][8 * g]);
          } else {
#pragma unroll
            for (int u = 0; u < 8; u++) bmv[u] = (_Float16)0.0f;
          }
          const f4_t dmin4 = __builtin_amdgcn_mfma_f32_16x16x32_f16(am, bmv, zero4, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; i++)
            acc[m][t][i] = __builtin_fmaf(dr[i], dblk[t][i], __builtin_fmaf(-dmr[i], dmin4[i], acc[m][t][i]));
        }
      }
    }
    __syncthreads();
  }
  // epilogue: D[4g + i][lr] of token tile t
#pragma unroll
  for (int t = 0; t < 4; t++) {
    const int tok = 16 * t + lr;
    if (t < ntt && tok < n) {
      const int slot = slot_l[tok];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int r = rt * MT_ROWS + 16 * wave + 4 * g + i;
        if (GATEUP) {
          const float h = silu(acc[0][t][i]) * acc[NMAT - 1][t][i];
          h16m[(size_t)slot * F + perm8(r)] = __float2half(h);
        } else {
          out[(size_t)slot * D + r] = acc[0][t][i];
        }
      }
    }
  }
}

// fp16 copy of s in the MFMA run order (perm8) for the gate/up B operand.
__global__ __launch_bounds__(256) void k_stage_mfma(const float *__restrict__ s32,
                                                    __half *__restrict__ s16m) {
  const int t = blockIdx.x;
  for (int j = threadIdx.x; j < D; j += 256)
    s16m[(size_t)t * D + perm8(j)] = __float2half(s32[(size_t)t * D + j]);
}

template __global__ void k_moe_mfma<true>(const uint8_t *, const __half *, const int32_t *,
                                          const int4 *, const int32_t *, int, int, __half *,
                                          float *);
template __global__ void k_moe_mfma<false>(const uint8_t *, const __half *, const int32_t *,
                                           const int4 *, const int32_t *, int, int, __half *,
                                           float *);

}  // namespace hy3x
