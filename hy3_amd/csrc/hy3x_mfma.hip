// hy3x_mfma.hip -- grouped Q4_K x fp16 GEMMs on the matrix cores (prefill).
//
// A work tile is one expert, a slice of its weight matrix -- 16 WAVES
// rows of gate and of up, or 32 WAVES rows of down (each wave 16 or
// 2 x 16 rows) -- and up to TOKENS (32 or 64) of its tokens (the dispatch
// tile list with NT = TOKENS), in 16-token MFMA column groups (NTT of them).
//
// Per Q4_K block column (256 of K):
//  * the tile's 256 row-blocks (144 B each) are copied from HBM straight into
//    LDS with coalesced 16-byte global->LDS loads (every row's block is 9
//    consecutive chunks), through a ring of A_STAGES columns;
//  * every lane turns 64 of its row's 256 weights into exact integers sc*q in
//    fp16 (q via the 0x6400 exponent-bias trick, one packed fp16 FMA with the
//    sub-block scale) -- the MFMA operands;
//  * v_mfma_f32_16x16x32_f16 accumulates the block in fp32 against the
//    tokens' activations (also copied global->LDS, double-buffered), then d,
//    dmin and the mins are applied per block (see mfma_step).
// All loads inside the column loop are these global->LDS copies, issued from
// inline assembly: their completion is tracked by hand (s_waitcnt vmcnt on
// the known number of copies in flight, then a barrier), which the compiler's
// own wait insertion cannot do for LDS copies.
//
// Operand layouts (16x16x32): lane l holds A[l%16][8(l/16) .. +7] (row, k),
// B[8(l/16) .. +7][l%16] (k, column) and D[4(l/16) + i][l%16], i = 0..3. Here
// A = activations (rows = tokens) and B = weights (columns = weight rows), so
// a lane's D values all belong to ONE weight row (its own: l%16) and four
// tokens.
//
// k order inside a block: an MFMA only needs the A and B operands to agree on
// which k each lane-slot carries, and the sub-block scales are folded into
// the weights, so one MFMA may mix sub-blocks of one block. Lane group g
// (= l/16) takes two contiguous 16-byte pieces of the block's 128 qs bytes,
// [16g, 16g+16) and [64+16g, 64+16g+16) -- i.e. half (g&1) of qs chunks
// p = g>>1 and p = 2 + (g>>1) -- and MFMA i = 4 piece + 2 h + u of the block
// uses, from piece `piece`, bytes [8u, 8u+8): their low (h = 0) or high
// (h = 1) nibbles, elements 16(g&1) + 8u .. +7 of sub-block 2p + h
// (hy3.c:1030-1040). Within each run of 8 the element order is
// (0,2,1,3,4,6,5,7), the order the nibble unpack produces; activations are
// staged in that order (perm8).
#include "hy3x_mfma_ops.h"
#include "hy3x_q8.h"

namespace hy3x {

// This file is compiled twice: as the narrow shape (namespace mfma_narrow)
// and, with HY3X_MFMA_WIDE defined (hy3x_mfma_wide.hip), as the wide one.
#ifdef HY3X_MFMA_WIDE
namespace mfma_wide {
#else
namespace mfma_narrow {
#endif

constexpr int MT_TOK = TOKENS;             // tokens per tile (dispatch NT for this path)
static_assert(MT_TOK == 32 || MT_TOK == 64, "tile tokens");
constexpr int MT_WAVES = WAVES;            // waves per workgroup
constexpr int MT_THREADS = 64 * MT_WAVES;
constexpr int MT_RGU = RGU;                // 16-row gate/up groups per wave (down: twice)
constexpr int RB = 32 * MT_WAVES * MT_RGU; // row-blocks per tile and block column
constexpr int RB_HALF = RB / 2;            // gate/up: gate row-blocks, then up
constexpr int RB_CHUNKS = 9;    // 16-byte chunks per row-block (144 B)
constexpr int A_CHUNKS = RB * RB_CHUNKS;              // 2304 per column
constexpr int A_CHUNKS_WAVE = A_CHUNKS / MT_WAVES;    // 288 per wave (32 row-blocks)
constexpr int A_DMA = (A_CHUNKS_WAVE + 63) / 64;      // 5 copies per wave (last one half)
constexpr int A_STAGES = 2;                           // weight ring stages
constexpr int A_AHEAD = A_STAGES - 1;                 // weight columns copied ahead
constexpr int B_DMA = MT_TOK * 32 / 64 / MT_WAVES;    // activation copies per wave
constexpr int S_LANES = MT_TOK * 4 / MT_WAVES;        // lanes per wave copying sums
// At the top of column kb's step, the weight copies of kb+1 .. kb+A_AHEAD-1
// (issued last, A_DMA each) may still be in flight.
constexpr int VM_IN_FLIGHT = (A_AHEAD - 1) * A_DMA;

// LDS: the weight ring, the activations of a column (token rows of 32
// 16-byte chunks, chunk c of row r at position c ^ (r & 15) so that the 16
// rows an MFMA operand read touches hit 16 different bank groups) and their
// sub-block sums (rows of 4 chunks, chunk p of row r at position
// p ^ ((r >> 2) & 3)), both double-buffered, and the tile's slots.
__shared__ __attribute__((aligned(16))) u4_t a_ring[A_STAGES][A_CHUNKS];
__shared__ __attribute__((aligned(16))) u4_t bt_st[2][MT_TOK][32];
__shared__ __attribute__((aligned(16))) u4_t bm_st[2][MT_TOK][4];
__shared__ int32_t t_slot[MT_TOK], t_arow[MT_TOK];

template <bool GATEUP>
struct MfmaCfg {
  static constexpr int KD = GATEUP ? D : F;        // reduction length
  static constexpr int NROWS = GATEUP ? F : D;     // weight rows
  static constexpr int RG = GATEUP ? MT_RGU : 2 * MT_RGU;  // 16-row groups per wave
  static constexpr int TROWS = 16 * MT_WAVES * RG; // weight rows per tile
  static constexpr int NRT = NROWS / TROWS;        // row tiles
  static constexpr int NKB = KD / QK;              // Q4_K block columns (16 / 6)
  static constexpr int NSUB = KD / 32;             // sub-blocks per activation row
  static constexpr int NMAT = GATEUP ? 2 : 1;      // gate and up, or down
  static_assert(TROWS * NMAT == RB, "row-blocks per tile");
};

// Weight copy schedule. OWN_COPIES (the wide shape): each wave copies
// exactly the row-blocks it reads, so it needs no barrier for its weights
// and issues column kb + 1 into the stage its own reads of kb - 1 used
// before it waits for kb -- two weight columns in flight (measured: 512
// tokens 643 -> 633 us; the narrow shape, two workgroups per CU, 290 -> 298
// us at 32 tokens, so it keeps the split copies issued after the barrier).
#ifdef HY3X_MFMA_WIDE
constexpr bool OWN_COPIES = true;
#else
constexpr bool OWN_COPIES = false;
#endif
// LDS position (row-block index) of the lane's row-block of 16-row group rg,
// matrix m. OWN_COPIES: each wave's own row-blocks are contiguous (wave, then
// matrix, then group); otherwise gate rows, then up rows, in row order.
template <bool GATEUP>
__device__ __forceinline__ int rb_pos(int wave, int m, int rg, int lr) {
  using C = MfmaCfg<GATEUP>;
  if (!OWN_COPIES) return (GATEUP ? m * RB_HALF : 0) + 16 * (C::RG * wave + rg) + lr;
  return 16 * (C::RG * C::NMAT * wave + C::RG * m + rg) + lr;
}
// Byte offset, within an expert's (or the shared expert's) matrices of stride
// mat_bytes, of local weight chunk cl (< A_CHUNKS_WAVE) of this wave's copy
// of a column: LDS chunk A_CHUNKS_WAVE * wave + cl = row-block (in rb_pos
// order) / 9, 16-byte piece % 9.
template <bool GATEUP>
__device__ __forceinline__ uint32_t a_src(int wave, int cl, int rt, int64_t mat_bytes, int nkb) {
  using C = MfmaCfg<GATEUP>;
  if (!OWN_COPIES) {
    int c = A_CHUNKS_WAVE * wave + cl;
    if (c >= A_CHUNKS) c = A_CHUNKS - 1;
    const int rb = c / RB_CHUNKS, pc = c % RB_CHUNKS;
    const int m = GATEUP ? rb / RB_HALF : 2, lrow = GATEUP ? rb % RB_HALF : rb;
    return (uint32_t)(m * mat_bytes + (int64_t)(rt * C::TROWS + lrow) * nkb * QB + 16 * pc);
  }
  if (cl >= A_CHUNKS_WAVE) cl = A_CHUNKS_WAVE - 1;  // inactive lanes of the last copy
  const int j = cl / RB_CHUNKS, pc = cl % RB_CHUNKS;
  const int m = GATEUP ? j / (16 * C::RG) : 2, jr = j % (16 * C::RG);
  const int row = rt * C::TROWS + 16 * C::RG * wave + jr;
  return (uint32_t)(m * mat_bytes + (int64_t)row * nkb * QB + 16 * pc);
}

// Copy sources of one work tile: wave-uniform bases (scalar registers) plus
// per-lane byte offsets, so that a copy costs no vector instruction. Column
// kb adds kb blocks to the bases.
template <bool GATEUP, int NTT>
struct TileState {
  using C = MfmaCfg<GATEUP>;
  static constexpr int RG = C::RG, NMAT = C::NMAT;
  const uint8_t *abase;         // the expert's weights (uniform)
  uint32_t aoff[A_DMA];         // weight chunks, from abase
  bool a_last;                  // the half-used last weight copy is active in this lane
  const uint8_t *bbase;         // activations (uniform)
  uint32_t boff[B_DMA];         // activation chunks, from bbase
  const uint8_t *sbase;         // sums (uniform)
  uint32_t soff;                // sums chunk (lanes below S_LANES), from sbase
  f4_t acc[RG][NMAT][NTT];
  // the last column's block sums and scales d, added to acc (acc += d * pend)
  // in the next column, where the adds overlap that column's MFMAs
  f4_t pend[RG][NMAT][NTT];
  float pend_d[RG][NMAT];
};

// acc += d * Dblk of the previous column (zeros before the first).
template <bool GATEUP, int NTT>
__device__ __forceinline__ void apply_pending(TileState<GATEUP, NTT> &st) {
#pragma unroll
  for (int rg = 0; rg < TileState<GATEUP, NTT>::RG; rg++)
#pragma unroll
    for (int m = 0; m < TileState<GATEUP, NTT>::NMAT; m++)
#pragma unroll
      for (int t = 0; t < NTT; t++)
#pragma unroll
        for (int i = 0; i < 4; i++)
          st.acc[rg][m][t][i] = __builtin_fmaf(st.pend_d[rg][m], st.pend[rg][m][t][i],
                                               st.acc[rg][m][t][i]);
}

// Copies of column kb: activations and sums into buffer kb & 1, then weights
// of column ka into ring stage ka % 3 -- always B_DMA + 1 + A_DMA copies per
// wave, weights last.
template <bool GATEUP, int NTT>
__device__ __forceinline__ void issue_b(const TileState<GATEUP, NTT> &st, int kb) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int buf = kb & 1;
  const uint8_t *bb = st.bbase + (size_t)kb * QK * 2;
  // only the token rows the tile's NTT token tiles read: a copy covers two
  // rows (copy j of wave w: rows 2 (B_DMA w + j), +1), a wave's sums lanes
  // S_LANES / 4 rows (the skip is wave-uniform)
#pragma unroll
  for (int j = 0; j < B_DMA; j++)
    if (2 * (B_DMA * wave + j) < 16 * NTT)
      dma16_s(bb, st.boff[j], lds_addr(&bt_st[buf][0][0] + 64 * (B_DMA * wave + j)));
  if (lane < S_LANES && S_LANES * wave / 4 < 16 * NTT)
    dma16_s(st.sbase + (size_t)kb * 64, st.soff,
            lds_addr(&bm_st[buf][0][0] + S_LANES * wave));
}
template <class State>  // TileState or TileStateQ8: the weight copies are the same
__device__ __forceinline__ void issue_a(const State &st, int ka) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const u4_t *dst = &a_ring[ka % A_STAGES][0] + A_CHUNKS_WAVE * wave;
  const uint8_t *ab = st.abase + (size_t)ka * QB;
#pragma unroll
  for (int j = 0; j < A_DMA; j++)
    if (j < A_DMA - 1 || st.a_last) dma16_stream(ab, st.aoff[j], lds_addr(dst + 64 * j));
}

// One block column kb. Its copies were issued one (activations) and A_AHEAD
// (weights) columns earlier; once they are in, the copies of kb + 1 and
// kb + A_AHEAD are issued into the buffers column kb - 1 used, and kb is
// computed.
// Per (token tile, weight row group, matrix):
//   Dblk = sum of the 8 MFMAs of the block (exact integer weights sc*q)
//   acc  = MFMA(S, -dmin*m, acc) + d * Dblk      (d, dmin of the lane's row)
// -- the Q4_K identity sum_k w_k x_k = d sum_j sc_j sum_{k in j} q_k x_k
// - dmin sum_j m_j sum_{k in j} x_k (hy3.c:1036-1037).
template <bool GATEUP, int NTT>
__device__ __forceinline__ void mfma_step(TileState<GATEUP, NTT> &st, int kb) {
  using C = MfmaCfg<GATEUP>;
  constexpr int RG = C::RG, NMAT = C::NMAT, NKB = C::NKB;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, g = lane >> 4;
  const int buf = kb & 1;
  // this wave's copies of column kb have landed (only the weights of
  // kb + 1 .. kb + A_AHEAD - 1, the last copies issued, may be in flight) and
  // its reads of kb - 1 are done; after the barrier the same holds for every
  // wave
  if (OWN_COPIES) {
    // this wave's weights of kb + 1 go into the stage its own reads of kb - 1
    // used (a wave reads only the row-blocks it copies), before the wait: two
    // weight columns in flight
    issue_a(st, kb + 1 < NKB ? kb + 1 : NKB - 1);  // past the end: a harmless re-copy
    wait_copies_and_barrier<A_DMA>();
    issue_b(st, kb + 1 < NKB ? kb + 1 : NKB - 1);
  } else {
    wait_copies_and_barrier<VM_IN_FLIGHT>();
    issue_b(st, kb + 1 < NKB ? kb + 1 : NKB - 1);  // past the end: a harmless re-copy
    issue_a(st, kb + A_AHEAD < NKB ? kb + A_AHEAD : NKB - 1);
  }

  const u4_t *as = &a_ring[kb % A_STAGES][0];
  // byte selector of this lane group's sub-block pairs, activation chunk offset
  const uint32_t sel =
      0x0C000C00u | ((uint32_t)(2 * (g >> 1) + 1) << 16) | (uint32_t)(2 * (g >> 1));
  const int gch = 8 * (g >> 1) + 2 * (g & 1);  // chunk (8 fp16) of k offset 64(g>>1) + 16(g&1)
  const f4_t zero4 = {0.f, 0.f, 0.f, 0.f};

  // All LDS reads of the column first (weights: header and two qs pieces per
  // row-block; activations: 8 fragments per token tile; sums), so that their
  // latency is covered by the dequantisation below, not paid per MFMA.
  u4_t hdr[RG][NMAT], pv[RG][NMAT][2];
#pragma unroll
  for (int rg = 0; rg < RG; rg++)
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
      const int rb = rb_pos<GATEUP>(wave, m, rg, lr);
      hdr[rg][m] = as[rb * RB_CHUNKS];
      pv[rg][m][0] = as[rb * RB_CHUNKS + 1 + g];
      pv[rg][m][1] = as[rb * RB_CHUNKS + 5 + g];
    }
  h8_t x[NTT][8], sv[NTT];
#pragma unroll
  for (int t = 0; t < NTT; t++) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      // MFMA i = 4 piece + 2 h + u: k0 = 128 piece + 32 h + 8 u + 64 (g>>1) + 16 (g&1)
      const int c = 16 * (i >> 2) + 4 * ((i >> 1) & 1) + (i & 1) + gch;
      x[t][i] = __builtin_bit_cast(h8_t, bt_st[buf][16 * t + lr][c ^ lr]);
    }
    sv[t] = __builtin_bit_cast(h8_t, bm_st[buf][16 * t + lr][g ^ ((lr >> 2) & 3)]);
  }

  // the previous column's d * Dblk, in the same order on acc as if it had
  // been added there (mins MFMA of kb - 1, then this): bit-identical
  apply_pending(st);
  f4_t dblk[RG][NMAT][NTT];
#pragma unroll
  for (int piece = 0; piece < 2; piece++) {
    h8_t wf[RG][NMAT][4];  // [2h + u]
#pragma unroll
    for (int rg = 0; rg < RG; rg++)
#pragma unroll
      for (int m = 0; m < NMAT; m++) {
        const Scales6 s6 = unpack_scales(hdr[rg][m]);
        const h2_t sc = bytes_h2(s6.sc[piece], sel);                         // (sc_lo, sc_hi)
        const h2_t mul = sc * (h2_t){(_Float16)1.0f, (_Float16)0.0625f};     // (sc_lo, sc_hi/16)
        const h2_t add = sc * (h2_t){(_Float16)-1024.0f, (_Float16)-64.0f};  // (-1024 sc_lo, -64 sc_hi)
        const h2_t ml = {mul[0], mul[0]}, al = {add[0], add[0]};
        const h2_t mh = {mul[1], mul[1]}, ah = {add[1], add[1]};
        dequant_run(pv[rg][m][piece].xy, ml, al, mh, ah, wf[rg][m][0], wf[rg][m][2]);
        dequant_run(pv[rg][m][piece].zw, ml, al, mh, ah, wf[rg][m][1], wf[rg][m][3]);
      }
#pragma unroll
    for (int hu = 0; hu < 4; hu++) {  // 2h + u
      const int i = 4 * piece + hu;
#pragma unroll
      for (int t = 0; t < NTT; t++)
#pragma unroll
        for (int rg = 0; rg < RG; rg++)
#pragma unroll
          for (int m = 0; m < NMAT; m++)
            dblk[rg][m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                x[t][i], wf[rg][m][hu], i == 0 ? zero4 : dblk[rg][m][t], 0, 0, 0);
    }
  }
  // per-block scale d (of this lane's row) and the mins MFMA
#pragma unroll
  for (int rg = 0; rg < RG; rg++)
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
      const u4_t hd = hdr[rg][m];
      const float d = fp16_quirk(hd.x & 0xffffu), dmin = fp16_quirk(hd.x >> 16);
      const Scales6 s6 = unpack_scales(hd);
      // m_{2g}, m_{2g+1}: bytes 2(g & 1), 2(g & 1) + 1 of mn[g >> 1]
      const uint32_t mw = (g >> 1) ? s6.mn[1] : s6.mn[0];
      const h8_t mo = mins_operand(dmin, (g & 1) ? (mw >> 16) : mw);
#pragma unroll
      for (int t = 0; t < NTT; t++) {
        st.acc[rg][m][t] =
            __builtin_amdgcn_mfma_f32_16x16x32_f16(sv[t], mo, st.acc[rg][m][t], 0, 0, 0);
        st.pend[rg][m][t] = dblk[rg][m][t];
      }
      st.pend_d[rg][m] = d;
    }
}

// Epilogue: lane holds D[token 16t + 4g + i][row] for its own weight row.
// GATEUP: h = silu(gate) * up -> h16m[slot][perm8(row)]; else out[slot][row].
template <bool GATEUP, int NTT>
__device__ __forceinline__ void store_tile(
    const f4_t (&acc)[MfmaCfg<GATEUP>::RG][MfmaCfg<GATEUP>::NMAT][NTT], int n, int rt,
    __half *__restrict__ h16m, float *__restrict__ out) {
  using C = MfmaCfg<GATEUP>;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, lr = lane & 15, g = lane >> 4;
#pragma unroll
  for (int rg = 0; rg < C::RG; rg++) {
    const int r = rt * C::TROWS + 16 * (C::RG * wave + rg) + lr;
#pragma unroll
    for (int t = 0; t < NTT; t++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int tok = 16 * t + 4 * g + i;
        if (tok < n) {
          const int slot = t_slot[tok];
          if constexpr (GATEUP) {
            h16m[(size_t)slot * F + perm8(r)] =
                swiglu_h(acc[rg][0][t][i], acc[rg][1][t][i]);
          } else {
            out[(size_t)slot * D + r] = acc[rg][0][t][i];
          }
        }
      }
  }
}

// One work tile with NTT token tiles of 16 (n <= 16 * NTT tokens).
template <bool GATEUP, int NTT>
__device__ __forceinline__ void mfma_tile(const uint8_t *__restrict__ wq,
                                          const __half *__restrict__ act,
                                          const __half *__restrict__ act_sum, int e, int n,
                                          int rt, __half *__restrict__ h16m,
                                          float *__restrict__ out) {
  using C = MfmaCfg<GATEUP>;
  constexpr int RG = C::RG, NMAT = C::NMAT, NKB = C::NKB, KD = C::KD;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lr = lane & 15, g = lane >> 4;
  TileState<GATEUP, NTT> st;

  // weights: wave w copies LDS chunks [288 w, 288 w + 288) of the column
  // (row-block c / 9 in rb_pos order, 16-byte piece c % 9), 64 per copy
  st.abase = wq + (size_t)__builtin_amdgcn_readfirstlane(e) * EXPERT_BYTES;
#pragma unroll
  for (int j = 0; j < A_DMA; j++)
    st.aoff[j] = a_src<GATEUP>(wave, 64 * j + lane, rt, MAT_BYTES, NKB);
  st.a_last = 64 * (A_DMA - 1) + lane < A_CHUNKS_WAVE;
  // activations: copy j of wave w fills positions q = 64 (B_DMA w + j) + lane
  // of the 32 x 32 chunk tile: row r = q / 32, position q % 32 holds chunk
  // (q % 32) ^ (r & 15). Sums: lane (< S_LANES) of wave w fills position
  // q = S_LANES w + lane of the 32 x 4 tile: row q / 4, position q % 4 holds
  // part (q % 4) ^ ((row >> 2) & 3). Rows past n copy token 0's row (their D
  // rows are never stored).
  const int arow0 = t_arow[0];
  st.bbase = reinterpret_cast<const uint8_t *>(act);
  st.sbase = reinterpret_cast<const uint8_t *>(act_sum);
#pragma unroll
  for (int j = 0; j < B_DMA; j++) {
    const int q = 64 * (B_DMA * wave + j) + lane, r = q >> 5;
    const int ar = t_arow[r] >= 0 ? t_arow[r] : arow0;
    st.boff[j] = (uint32_t)(2 * (ar * KD + 8 * ((q & 31) ^ (r & 15))));
  }
  {
    const int q = S_LANES * wave + (lane & (S_LANES - 1)), r = q >> 2;
    const int ar = t_arow[r] >= 0 ? t_arow[r] : arow0;
    st.soff = (uint32_t)(2 * (ar * C::NSUB * 4 + 8 * ((q & 3) ^ ((r >> 2) & 3))));
  }
  const f4_t zero4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int rg = 0; rg < RG; rg++)
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
      for (int t = 0; t < NTT; t++) st.acc[rg][m][t] = st.pend[rg][m][t] = zero4;
#pragma unroll
  for (int rg = 0; rg < RG; rg++)
#pragma unroll
    for (int m = 0; m < NMAT; m++) st.pend_d[rg][m] = 0.0f;

  // prologue: weights of column 0, activations of column 0, weights of
  // columns 1 .. A_AHEAD - 1
  issue_a(st, 0);
  issue_b(st, 0);
#pragma unroll
  for (int c = 1; c < A_AHEAD; c++) issue_a(st, c < NKB ? c : NKB - 1);
  // two columns per iteration (512 tokens: gate/up 355 -> 351 us, down 201
  // -> 199; four per iteration measured no better)
#pragma unroll 2
  for (int kb = 0; kb < NKB; kb++) mfma_step(st, kb);
  apply_pending(st);  // the last column's d * Dblk
  // drain the trailing re-copies before the workgroup's LDS is released
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  store_tile<GATEUP, NTT>(st.acc, n, rt, h16m, out);
}

// ---------------------------------------------------------------------------
// The shared expert in Q8 (q8x128 super-blocks, hy3x_q8.h). A column is one
// 144-byte super-block per row = 128 k = four 32-weight blocks, each exactly
// one 16x16x32 MFMA, so the weight copies are the Q4_K path's (issue_a).
// Activations: 16 chunks per token per column in bt_st[buf] viewed as
// [MT_TOK tokens][16 chunks], chunk c of row r at position c ^ (r & 15). The
// weights are the exact integers q in fp16 ((1152 + q) from the byte
// permute, minus 1152) and each block's MFMA result is scaled by its d in
// fp32: acc += d_b * (x_b . q_b) -- sum d*q*x as mul_mat_f32 case 8
// (hy3.c:1098-1120).
constexpr int B8_DMA = MT_TOK * 16 / 64 / MT_WAVES;  // activation copies per wave

template <bool GATEUP, int NTT>
struct TileStateQ8 {
  using C = MfmaCfg<GATEUP>;
  static constexpr int RG = C::RG, NMAT = C::NMAT, NKB = C::KD / Q8K;
  const uint8_t *abase;   // the shared expert's Q8 matrices (uniform)
  uint32_t aoff[A_DMA];   // weight chunks, from abase
  bool a_last;            // the half-used last weight copy is active in this lane
  const uint8_t *bbase;   // activations (uniform)
  uint32_t boff[B8_DMA];  // activation chunks, from bbase
  f4_t acc[RG][NMAT][NTT];
};

template <bool GATEUP, int NTT>
__device__ __forceinline__ void issue_b_q8(const TileStateQ8<GATEUP, NTT> &st, int kb) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const u4_t *dst = &bt_st[kb & 1][0][0];
  const uint8_t *bb = st.bbase + (size_t)kb * Q8K * 2;
#pragma unroll
  for (int j = 0; j < B8_DMA; j++)  // a copy covers four rows; only the rows the NTT tiles read
    if (4 * (B8_DMA * wave + j) < 16 * NTT)
      dma16_s(bb, st.boff[j], lds_addr(dst + 64 * (B8_DMA * wave + j)));
}

template <bool GATEUP, int NTT>
__device__ __forceinline__ void mfma_step_q8(TileStateQ8<GATEUP, NTT> &st, int kb) {
  using S = TileStateQ8<GATEUP, NTT>;
  constexpr int RG = S::RG, NMAT = S::NMAT, NKB = S::NKB;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lr = lane & 15, g = lane >> 4;
  if (OWN_COPIES) {  // as mfma_step
    issue_a(st, kb + 1 < NKB ? kb + 1 : NKB - 1);
    wait_copies_and_barrier<A_DMA>();
    issue_b_q8(st, kb + 1 < NKB ? kb + 1 : NKB - 1);
  } else {
    wait_copies_and_barrier<VM_IN_FLIGHT>();
    issue_b_q8(st, kb + 1 < NKB ? kb + 1 : NKB - 1);
    issue_a(st, kb + A_AHEAD < NKB ? kb + A_AHEAD : NKB - 1);
  }
  const u4_t *as = &a_ring[kb % A_STAGES][0];
  const u4_t *bt = &bt_st[kb & 1][0][0];
  // LDS reads first: per row-block the four scales and this lane's 8 bytes of
  // each block; per token tile the four activation fragments
  f4_t dsc[RG][NMAT];
  u2_t qb[RG][NMAT][4];
#pragma unroll
  for (int rg = 0; rg < RG; rg++)
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
      const int rb = rb_pos<GATEUP>(wave, m, rg, lr);
      dsc[rg][m] = __builtin_bit_cast(f4_t, as[rb * RB_CHUNKS]);
      const u2_t *qp = reinterpret_cast<const u2_t *>(as + rb * RB_CHUNKS + 1);
#pragma unroll
      for (int b = 0; b < 4; b++) qb[rg][m][b] = qp[4 * b + g];
    }
  h8_t x[NTT][4];
#pragma unroll
  for (int t = 0; t < NTT; t++)
#pragma unroll
    for (int b = 0; b < 4; b++)
      x[t][b] = __builtin_bit_cast(h8_t, bt[16 * (16 * t + lr) + ((4 * b + g) ^ lr)]);
  const f4_t zero4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int b = 0; b < 4; b++) {
    h8_t wf[RG][NMAT];
#pragma unroll
    for (int rg = 0; rg < RG; rg++)
#pragma unroll
      for (int m = 0; m < NMAT; m++) wf[rg][m] = q8_run(qb[rg][m][b]);
#pragma unroll
    for (int t = 0; t < NTT; t++)
#pragma unroll
      for (int rg = 0; rg < RG; rg++)
#pragma unroll
        for (int m = 0; m < NMAT; m++) {
          const f4_t p = __builtin_amdgcn_mfma_f32_16x16x32_f16(x[t][b], wf[rg][m], zero4, 0, 0, 0);
          const float d = dsc[rg][m][b];
#pragma unroll
          for (int i = 0; i < 4; i++) st.acc[rg][m][t][i] = __builtin_fmaf(d, p[i], st.acc[rg][m][t][i]);
        }
  }
}

template <bool GATEUP, int NTT>
__device__ __forceinline__ void mfma_tile_q8(const uint8_t *__restrict__ wsh,
                                             const __half *__restrict__ act, int n, int rt,
                                             __half *__restrict__ h16m, float *__restrict__ out) {
  using S = TileStateQ8<GATEUP, NTT>;
  using C = MfmaCfg<GATEUP>;
  constexpr int RG = S::RG, NMAT = S::NMAT, NKB = S::NKB, KD = C::KD;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  S st;
  st.abase = wsh;
#pragma unroll
  for (int j = 0; j < A_DMA; j++)
    st.aoff[j] = a_src<GATEUP>(wave, 64 * j + lane, rt, Q8_MAT_BYTES, NKB);
  st.a_last = 64 * (A_DMA - 1) + lane < A_CHUNKS_WAVE;
  // activations: copy j of wave w fills positions q = 64 (B8_DMA w + j) + lane
  // of the 32 x 16 chunk tile: row r = q / 16, position q % 16 holds chunk
  // (q % 16) ^ (r & 15). Rows past n copy token 0's row.
  const int arow0 = t_arow[0];
  st.bbase = reinterpret_cast<const uint8_t *>(act);
#pragma unroll
  for (int j = 0; j < B8_DMA; j++) {
    const int q = 64 * (B8_DMA * wave + j) + lane, r = q >> 4;
    const int ar = t_arow[r] >= 0 ? t_arow[r] : arow0;
    st.boff[j] = (uint32_t)(2 * (ar * KD + 8 * ((q & 15) ^ (r & 15))));
  }
  const f4_t zero4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int rg = 0; rg < RG; rg++)
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
      for (int t = 0; t < NTT; t++) st.acc[rg][m][t] = zero4;
  issue_a(st, 0);
  issue_b_q8(st, 0);
#pragma unroll
  for (int c = 1; c < A_AHEAD; c++) issue_a(st, c < NKB ? c : NKB - 1);
  for (int kb = 0; kb < NKB; kb++) mfma_step_q8(st, kb);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  store_tile<GATEUP, NTT>(st.acc, n, rt, h16m, out);
}

// Grouped GEMM over the tile list (tiles of at most MT_TOK tokens). GATEUP:
// weights = gate and up rows of the expert (K = 4096), activations = staged
// s, epilogue h = silu(g) * u -> h16m[slot][perm8(row)] (fp16). Otherwise
// weights = down rows (K = 1536), activations = h16m, out[slot][row] fp32.
// act_sum: sub-block sums of each activation row as (Sh, Sl, Sh, Sl) fp16.
// wsh != nullptr: the shared expert's tiles use its Q8 matrices (mfma_tile_q8).
template <bool GATEUP>
__global__ __launch_bounds__(MT_THREADS) void k_moe_mfma(
    const uint8_t *__restrict__ wq, const uint8_t *__restrict__ wsh,
    const __half *__restrict__ act, const __half *__restrict__ act_sum,
    const int32_t *__restrict__ list, const int4 *__restrict__ tiles,
    const int32_t *__restrict__ n_tiles, int T, int K, __half *__restrict__ h16m,
    float *__restrict__ out) {
  using C = MfmaCfg<GATEUP>;
  // The grid is sized for the most tiles T tokens can make; the blocks past
  // this forward's work leave at once, and the work items are dealt over the
  // real blocks only, so that every XCD gets an even share.
  const int nreal = *n_tiles * C::NRT;
  // each XCD on a contiguous run of the work (the token tiles of an expert
  // share its weights in L2; whole tiles dealt round-robin measured equal at
  // 32 tokens and 0.7 % slower at 512)
  if ((int)blockIdx.x >= nreal) return;
  const int w = xcd_remap(blockIdx.x, nreal);
  const int tile = w / C::NRT, rt = w % C::NRT;
  const int4 td = tiles[tile];
  const int e = td.x, o = td.y, n = td.z;
  const int tid = threadIdx.x;
  if (tid < MT_TOK) {
    const int s = tid < n ? list[o + tid] : -1;
    t_slot[tid] = s;
    // activation row: gate/up reads s of the token, down reads h of the slot
    t_arow[tid] = s < 0 ? -1 : (GATEUP ? (s < T * K ? s / K : s - T * K) : s);
  }
  __syncthreads();
  if (wsh && e == E) {
    if constexpr (MT_TOK > 32) {
      if (n > 48) {
        mfma_tile_q8<GATEUP, 4>(wsh, act, n, rt, h16m, out);
        return;
      }
      if (n > 32) {
        mfma_tile_q8<GATEUP, 3>(wsh, act, n, rt, h16m, out);
        return;
      }
    }
    if (n > 16)
      mfma_tile_q8<GATEUP, 2>(wsh, act, n, rt, h16m, out);
    else
      mfma_tile_q8<GATEUP, 1>(wsh, act, n, rt, h16m, out);
    return;
  }
  if constexpr (MT_TOK > 32) {
    if (n > 48) {
      mfma_tile<GATEUP, 4>(wq, act, act_sum, e, n, rt, h16m, out);
      return;
    }
    if (n > 32) {
      mfma_tile<GATEUP, 3>(wq, act, act_sum, e, n, rt, h16m, out);
      return;
    }
  }
  if (n > 16)
    mfma_tile<GATEUP, 2>(wq, act, act_sum, e, n, rt, h16m, out);
  else
    mfma_tile<GATEUP, 1>(wq, act, act_sum, e, n, rt, h16m, out);
}

template __global__ void k_moe_mfma<true>(const uint8_t *, const uint8_t *, const __half *,
                                          const __half *, const int32_t *, const int4 *,
                                          const int32_t *, int, int, __half *, float *);
template __global__ void k_moe_mfma<false>(const uint8_t *, const uint8_t *, const __half *,
                                           const __half *, const int32_t *, const int4 *,
                                           const int32_t *, int, int, __half *, float *);

}  // namespace mfma_narrow / mfma_wide

#ifndef HY3X_MFMA_WIDE

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

#endif  // !HY3X_MFMA_WIDE

}  // namespace hy3x
