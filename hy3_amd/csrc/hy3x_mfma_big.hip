// hy3x_mfma_big.hip -- grouped Q4_K x fp16 GEMMs for experts holding many
// tokens (long prefills): 128-token work tiles.
//
// The arithmetic is the MFMA tiles' (hy3x_mfma.hip: exact integer weights
// sc*q from the same nibble unpack, the same k order and per-block d / mins
// MFMA), with each wave's dequantised weights reused over up to eight 16-token
// MFMA column groups instead of four, which halves the dequantisation per
// MFMA on hot experts. To fit 128 tokens' activations in LDS next to the
// weight ring, the activations are staged half a block column (128 of K) at a
// time: a block column takes two steps, step h computing piece h (the MFMAs
// whose k lies in [128h, 128h + 128)).
//
// Workgroup: 8 waves; a wave owns 16 gate and the same 16 up rows (gate/up)
// or 32 down rows of the tile for the whole reduction.
//   weights   a_ring[2]: the tile's 256 row-blocks of a column (as the MFMA
//             tiles), copied one column ahead;
//   act       bx[2]: 128 token rows x 16 chunks of a half column, chunk c of
//             row r at position c ^ (r & 15), copied one step ahead;
//   sums      bs[2]: 128 token rows x 4 chunks of a column's sub-block sums,
//             part p of row r at p ^ ((r >> 2) & 3), copied one column ahead.
// Copies at step s (after its barrier): activations of step s + 1, then at
// h = 0 the weights of column kb + 1, at h = 1 the sums of column kb + 1.
#include "hy3x_mfma_ops.h"
#include "hy3x_q8.h"

namespace hy3x {
namespace mfma_big {

constexpr int BW = BIG_WAVES;              // waves per workgroup
constexpr int B_THREADS = 64 * BW;
constexpr int RB = 256;                    // row-blocks per tile and block column
constexpr int RB_CHUNKS = 9;               // 16-byte chunks per row-block
constexpr int A_CHUNKS = RB * RB_CHUNKS;   // 2304 per column
constexpr int A_CHUNKS_WAVE = A_CHUNKS / BW;         // 288
constexpr int A_DMA = (A_CHUNKS_WAVE + 63) / 64;     // 5 (the last one half used)
constexpr int X_DMA = BIG_TOKENS * 16 / 64 / BW;     // 4 activation copies per wave and step
constexpr int S_DMA = BIG_TOKENS * 4 / 64 / BW;      // 1 sums copy per wave and column
static_assert(X_DMA * 64 * BW == BIG_TOKENS * 16 && S_DMA * 64 * BW == BIG_TOKENS * 4, "copies");

__shared__ __attribute__((aligned(16))) u4_t a_ring[2][A_CHUNKS];
__shared__ __attribute__((aligned(16))) u4_t bx[2][BIG_TOKENS * 16];
__shared__ __attribute__((aligned(16))) u4_t bs[2][BIG_TOKENS * 4];
__shared__ int32_t t_slot[BIG_TOKENS], t_arow[BIG_TOKENS];

template <bool GATEUP>
struct Cfg {
  static constexpr int KD = GATEUP ? D : F;
  static constexpr int NROWS = GATEUP ? F : D;
  static constexpr int RG = GATEUP ? 1 : 2;       // 16-row groups per wave
  static constexpr int NMAT = GATEUP ? 2 : 1;
  static constexpr int TROWS = 16 * BW * RG;      // weight rows per tile (per matrix)
  static constexpr int NRT = NROWS / TROWS;
  static constexpr int NKB = KD / QK;
  static constexpr int NSUB = KD / 32;
  static_assert(TROWS * NMAT == RB && NROWS % TROWS == 0, "tile rows");
};

template <bool GATEUP, int NTT>
struct State {
  using C = Cfg<GATEUP>;
  const uint8_t *abase;
  uint32_t aoff[A_DMA];
  bool a_last;
  const uint8_t *xbase, *sbase;
  uint32_t xoff[X_DMA];
  uint32_t soff;
  f4_t acc[C::RG][C::NMAT][NTT];
  f4_t dblk[C::RG][C::NMAT][NTT];  // the current column's block sums
  u4_t hdr[C::RG][C::NMAT];        // the current column's row-block headers
};

// Weight copy sources of the tile's row tile rt: wave w copies chunks
// [288 w, 288 w + 288) of the column's (row-block c / 9, 16-byte piece c % 9),
// 64 per copy. A column is one 144-byte block per row: Q4_K (256 of K) or the
// shared expert's Q8 super-block (128 of K); mat_bytes is the matrix stride.
template <bool GATEUP, int NTT>
__device__ __forceinline__ void set_weights(State<GATEUP, NTT> &st, const uint8_t *base,
                                            int64_t mat_bytes, int rt) {
  using C = Cfg<GATEUP>;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int ncol = mat_bytes / ((int64_t)C::NROWS * QB);  // columns per row
  st.abase = base;
#pragma unroll
  for (int j = 0; j < A_DMA; j++) {
    int c = A_CHUNKS_WAVE * wave + 64 * j + lane;
    if (c >= A_CHUNKS) c = A_CHUNKS - 1;  // inactive lanes of the last copy
    const int rb = c / RB_CHUNKS, pc = c % RB_CHUNKS;
    const int m = GATEUP ? rb / (RB / 2) : 2, lrow = GATEUP ? rb % (RB / 2) : rb;
    st.aoff[j] = (uint32_t)(m * mat_bytes + (int64_t)(rt * C::TROWS + lrow) * ncol * QB + 16 * pc);
  }
  st.a_last = 64 * (A_DMA - 1) + lane < A_CHUNKS_WAVE;
}

// Copies (wave-uniform counts): weights A_DMA, activations X_DMA (those
// covering rows past the tile's 16 NTT are skipped), sums S_DMA (idem).
template <bool GATEUP, int NTT>
__device__ __forceinline__ void issue_w(const State<GATEUP, NTT> &st, int kb) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const u4_t *dst = &a_ring[kb & 1][0] + A_CHUNKS_WAVE * wave;
  const uint8_t *ab = st.abase + (size_t)kb * QB;
#pragma unroll
  for (int j = 0; j < A_DMA; j++)
    if (j < A_DMA - 1 || st.a_last) dma16_stream(ab, st.aoff[j], lds_addr(dst + 64 * j));
}
template <bool GATEUP, int NTT>
__device__ __forceinline__ void issue_x(const State<GATEUP, NTT> &st, int s) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint8_t *xb = st.xbase + (size_t)(s >> 1) * QK * 2 + (s & 1) * 256;
#pragma unroll
  for (int j = 0; j < X_DMA; j++)  // copy j of wave w: rows 4 (X_DMA w + j) .. +3
    if (4 * (X_DMA * wave + j) < 16 * NTT)
      dma16_s(xb, st.xoff[j], lds_addr(&bx[s & 1][0] + 64 * (X_DMA * wave + j)));
}
template <bool GATEUP, int NTT>
__device__ __forceinline__ void issue_s(const State<GATEUP, NTT> &st, int kb) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
#pragma unroll
  for (int j = 0; j < S_DMA; j++)  // rows 16 (S_DMA w + j) .. +15
    if (16 * (S_DMA * wave + j) < 16 * NTT)
      dma16_s(st.sbase + (size_t)kb * 64, st.soff,
              lds_addr(&bs[kb & 1][0] + 64 * (S_DMA * wave + j)));
}

// Step s = 2 kb + h of the tile.
template <bool GATEUP, int NTT>
__device__ __forceinline__ void big_step(State<GATEUP, NTT> &st, int s) {
  using C = Cfg<GATEUP>;
  constexpr int RG = C::RG, NMAT = C::NMAT, NKB = C::NKB;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lr = lane & 15, g = lane >> 4;
  const int kb = s >> 1, h = s & 1;
  // copies needed now: at h = 1 the activations issued at step s - 1 (the
  // weights issued after them may still fly); at h = 0 everything
  if (h)
    wait_copies_and_barrier<A_DMA>();
  else
    wait_copies_and_barrier<0>();
  const int sn = s + 1 < 2 * NKB ? s + 1 : 2 * NKB - 1;  // past the end: a harmless re-copy
  issue_x(st, sn);
  if (h == 0)
    issue_w(st, kb + 1 < NKB ? kb + 1 : NKB - 1);
  else
    issue_s(st, kb + 1 < NKB ? kb + 1 : NKB - 1);

  const u4_t *as = &a_ring[kb & 1][0];
  const u4_t *xs = &bx[s & 1][0];
  const uint32_t sel =
      0x0C000C00u | ((uint32_t)(2 * (g >> 1) + 1) << 16) | (uint32_t)(2 * (g >> 1));
  const int gch = 8 * (g >> 1) + 2 * (g & 1);
  const f4_t zero4 = {0.f, 0.f, 0.f, 0.f};
  u4_t pv[RG][NMAT];
#pragma unroll
  for (int rg = 0; rg < RG; rg++)
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
      const int rb = (GATEUP ? m * (RB / 2) : 0) + 16 * (RG * wave + rg) + lr;
      if (h == 0) st.hdr[rg][m] = as[rb * RB_CHUNKS];
      pv[rg][m] = as[rb * RB_CHUNKS + 1 + 4 * h + g];
    }
  h8_t wf[RG][NMAT][4];  // [2 hi + u] of this piece
#pragma unroll
  for (int rg = 0; rg < RG; rg++)
#pragma unroll
    for (int m = 0; m < NMAT; m++) {
      const Scales6 s6 = unpack_scales(st.hdr[rg][m]);
      const h2_t sc = bytes_h2(h ? s6.sc[1] : s6.sc[0], sel);
      const h2_t mul = sc * (h2_t){(_Float16)1.0f, (_Float16)0.0625f};
      const h2_t add = sc * (h2_t){(_Float16)-1024.0f, (_Float16)-64.0f};
      const h2_t ml = {mul[0], mul[0]}, al = {add[0], add[0]};
      const h2_t mh = {mul[1], mul[1]}, ah = {add[1], add[1]};
      dequant_run(pv[rg][m].xy, ml, al, mh, ah, wf[rg][m][0], wf[rg][m][2]);
      dequant_run(pv[rg][m].zw, ml, al, mh, ah, wf[rg][m][1], wf[rg][m][3]);
    }
  // k run outer, token groups inner: an MFMA's accumulator was last written
  // 2 NTT MFMAs earlier, so the chains do not wait on each other
#pragma unroll
  for (int hu = 0; hu < 4; hu++) {
    // chunk of k offset 32 hi + 8 u + 64 (g >> 1) + 16 (g & 1) within the half
    const int c = 4 * ((hu >> 1) & 1) + (hu & 1) + gch;
#pragma unroll
    for (int t = 0; t < NTT; t++) {
      const h8_t x = __builtin_bit_cast(h8_t, xs[16 * (16 * t + lr) + (c ^ lr)]);
#pragma unroll
      for (int rg = 0; rg < RG; rg++)
#pragma unroll
        for (int m = 0; m < NMAT; m++)
          st.dblk[rg][m][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              x, wf[rg][m][hu], (h == 0 && hu == 0) ? zero4 : st.dblk[rg][m][t], 0, 0, 0);
    }
  }
  if (h) {  // the column's mins MFMA, then acc += d * Dblk (the MFMA tiles' order)
#pragma unroll
    for (int rg = 0; rg < RG; rg++)
#pragma unroll
      for (int m = 0; m < NMAT; m++) {
        const u4_t hd = st.hdr[rg][m];
        const float d = fp16_quirk(hd.x & 0xffffu), dmin = fp16_quirk(hd.x >> 16);
        const Scales6 s6 = unpack_scales(hd);
        const uint32_t mw = (g >> 1) ? s6.mn[1] : s6.mn[0];
        const h8_t mo = mins_operand(dmin, (g & 1) ? (mw >> 16) : mw);
#pragma unroll
        for (int t = 0; t < NTT; t++) {
          const h8_t sv = __builtin_bit_cast(
              h8_t, bs[kb & 1][4 * (16 * t + lr) + (g ^ ((lr >> 2) & 3))]);
          f4_t a = __builtin_amdgcn_mfma_f32_16x16x32_f16(sv, mo, st.acc[rg][m][t], 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 4; i++) a[i] = __builtin_fmaf(d, st.dblk[rg][m][t][i], a[i]);
          st.acc[rg][m][t] = a;
        }
      }
  }
}


// The shared expert in Q8 (q8x128 super-blocks, hy3x_q8.h): a column is one
// 144-byte super-block per row (128 of K), i.e. one activation step of the
// Q4_K tiles, so the copies are the same (issue_w / issue_x with step = Q8
// column). Per column and row: four 32-weight blocks, each one 16x16x32 MFMA of
// the exact integers q against the activations, scaled by its d in fp32:
// acc += d_b * (x_b . q_b) -- the order of the MFMA tiles' mfma_step_q8.
// Copies of column c + 1 are issued after the barrier of column c.
template <bool GATEUP, int NTT>
__device__ __forceinline__ void big_tile_q8_columns(State<GATEUP, NTT> &st) {
  using C = Cfg<GATEUP>;
  constexpr int RG = C::RG, NMAT = C::NMAT, NC = C::KD / Q8K;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lr = lane & 15, g = lane >> 4;
  const f4_t zero4 = {0.f, 0.f, 0.f, 0.f};
  issue_w(st, 0);
  issue_x(st, 0);
  for (int c = 0; c < NC; c++) {
    wait_copies_and_barrier<0>();
    issue_w(st, c + 1 < NC ? c + 1 : NC - 1);  // past the end: a harmless re-copy
    issue_x(st, c + 1 < NC ? c + 1 : NC - 1);
    const u4_t *as = &a_ring[c & 1][0];
    const u4_t *xs = &bx[c & 1][0];
    f4_t dsc[RG][NMAT];
    u2_t qb[RG][NMAT][4];
#pragma unroll
    for (int rg = 0; rg < RG; rg++)
#pragma unroll
      for (int m = 0; m < NMAT; m++) {
        const int rb = (GATEUP ? m * (RB / 2) : 0) + 16 * (RG * wave + rg) + lr;
        dsc[rg][m] = __builtin_bit_cast(f4_t, as[rb * RB_CHUNKS]);
        const u2_t *qp = reinterpret_cast<const u2_t *>(as + rb * RB_CHUNKS + 1);
#pragma unroll
        for (int b = 0; b < 4; b++) qb[rg][m][b] = qp[4 * b + g];
      }
#pragma unroll
    for (int b = 0; b < 4; b++) {
      h8_t wf[RG][NMAT];
#pragma unroll
      for (int rg = 0; rg < RG; rg++)
#pragma unroll
        for (int m = 0; m < NMAT; m++) wf[rg][m] = q8_run(qb[rg][m][b]);
#pragma unroll
      for (int t = 0; t < NTT; t++) {
        const h8_t x =
            __builtin_bit_cast(h8_t, xs[16 * (16 * t + lr) + ((4 * b + g) ^ lr)]);
#pragma unroll
        for (int rg = 0; rg < RG; rg++)
#pragma unroll
          for (int m = 0; m < NMAT; m++) {
            const f4_t p = __builtin_amdgcn_mfma_f32_16x16x32_f16(x, wf[rg][m], zero4, 0, 0, 0);
            const float d = dsc[rg][m][b];
#pragma unroll
            for (int i = 0; i < 4; i++)
              st.acc[rg][m][t][i] = __builtin_fmaf(d, p[i], st.acc[rg][m][t][i]);
          }
      }
    }
  }
}

template <bool GATEUP, int NTT>
__device__ __forceinline__ void big_tile(const uint8_t *__restrict__ wq,
                                         const uint8_t *__restrict__ wsh,
                                         const __half *__restrict__ act,
                                         const __half *__restrict__ act_sum, int e, int n,
                                         int rt, __half *__restrict__ h16m,
                                         float *__restrict__ out) {
  using C = Cfg<GATEUP>;
  constexpr int RG = C::RG, NMAT = C::NMAT, NKB = C::NKB, KD = C::KD;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lr = lane & 15, g = lane >> 4;
  State<GATEUP, NTT> st;
  const bool q8 = wsh != nullptr && e == E;  // the shared expert in Q8 (uniform)
  if (q8)
    set_weights(st, wsh, Q8_MAT_BYTES, rt);
  else
    set_weights(st, wq + (size_t)__builtin_amdgcn_readfirstlane(e) * EXPERT_BYTES, MAT_BYTES, rt);
  // activations: copy j of wave w fills positions q = 64 (X_DMA w + j) + lane
  // of the 128 x 16 half-column tile: row r = q / 16, position q % 16 holds
  // chunk (q % 16) ^ (r & 15) of the half. Sums: positions q = 64 (S_DMA w +
  // j) + lane of the 128 x 4 tile: row q / 4, position q % 4 holds part
  // (q % 4) ^ ((row >> 2) & 3). Rows past n copy token 0's row.
  const int arow0 = t_arow[0];
  st.xbase = reinterpret_cast<const uint8_t *>(act);
  st.sbase = reinterpret_cast<const uint8_t *>(act_sum);
#pragma unroll
  for (int j = 0; j < X_DMA; j++) {
    const int q = 64 * (X_DMA * wave + j) + lane, r = q >> 4;
    const int ar = t_arow[r] >= 0 ? t_arow[r] : arow0;
    st.xoff[j] = (uint32_t)(2 * (ar * KD + 8 * ((q & 15) ^ (r & 15))));
  }
  {
    const int q = 64 * S_DMA * wave + lane, r = q >> 2;  // S_DMA == 1
    const int ar = t_arow[r] >= 0 ? t_arow[r] : arow0;
    st.soff = (uint32_t)(2 * (ar * C::NSUB * 4 + 8 * ((q & 3) ^ ((r >> 2) & 3))));
  }
  static_assert(S_DMA == 1, "one sums copy per wave");
  const f4_t zero4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int rg = 0; rg < RG; rg++)
#pragma unroll
    for (int m = 0; m < NMAT; m++)
#pragma unroll
      for (int t = 0; t < NTT; t++) st.acc[rg][m][t] = zero4;

  if (q8) {
    big_tile_q8_columns(st);
  } else {
    // prologue: the copies step 0 needs (weights and sums of column 0,
    // activations of half 0)
    issue_w(st, 0);
    issue_s(st, 0);
    issue_x(st, 0);
    // two steps per iteration: the half h is a constant in each
#pragma unroll 2
    for (int s = 0; s < 2 * NKB; s++) big_step(st, s);
  }
  // drain the trailing re-copies before the workgroup's LDS is released
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // epilogue: lane holds D[token 16t + 4g + i][row] for its own weight row
#pragma unroll
  for (int rg = 0; rg < RG; rg++) {
    const int r = rt * C::TROWS + 16 * (RG * wave + rg) + lr;
#pragma unroll
    for (int t = 0; t < NTT; t++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int tok = 16 * t + 4 * g + i;
        if (tok < n) {
          const int slot = t_slot[tok];
          if constexpr (GATEUP)
            h16m[(size_t)slot * F + perm8(r)] = swiglu_h(st.acc[rg][0][t][i], st.acc[rg][1][t][i]);
          else
            out[(size_t)slot * D + r] = st.acc[rg][0][t][i];
        }
      }
  }
}

// Grouped GEMM over a tile list of at most BIG_TOKENS tokens per tile,
// operands and outputs as k_moe_mfma; wsh != nullptr: the shared expert's
// tiles use its Q8 matrices.
template <bool GATEUP>
__global__ __launch_bounds__(B_THREADS) void k_moe_big(
    const uint8_t *__restrict__ wq, const uint8_t *__restrict__ wsh, const __half *__restrict__ act,
    const __half *__restrict__ act_sum, const int32_t *__restrict__ list,
    const int4 *__restrict__ tiles, const int32_t *__restrict__ n_tiles, int T, int K,
    __half *__restrict__ h16m, float *__restrict__ out) {
  using C = Cfg<GATEUP>;
  const int nreal = *n_tiles * C::NRT;
  // gate/up: whole tiles dealt round-robin to the XCDs, a tile's row tiles
  // consecutive on one (sharing its activations in L2; the grid carries
  // XCD_TILE_RR_MARGIN tiles of margin); down: work items round-robin, as the
  // workgroups are. Measured at 4096 tokens, Zipf routing, against one
  // contiguous run of work per XCD: gate/up 1320 -> 1297 and 1296 -> 1268 us
  // (items round-robin: 1329), down 757 -> 740 us (tiles round-robin: 764).
  int w;
  if constexpr (GATEUP) {
    w = xcd_tile_rr(blockIdx.x, C::NRT);
  } else {
    w = blockIdx.x;
  }
  if (w >= nreal) return;
  const int tile = w / C::NRT, rt = w % C::NRT;
  const int4 td = tiles[tile];
  const int e = td.x, o = td.y, n = td.z;
  const int tid = threadIdx.x;
  if (tid < BIG_TOKENS) {
    const int s = tid < n ? list[o + tid] : -1;
    t_slot[tid] = s;
    t_arow[tid] = s < 0 ? -1 : (GATEUP ? (s < T * K ? s / K : s - T * K) : s);
  }
  __syncthreads();
  // as many 16-token column groups as the tile's tokens fill (measured
  // against even counts only: 4096 tokens with Zipf routing, gate/up -1.7 %,
  // down -2 %; 1152 and 1536 tokens -3 to -4 %)
  if (n > 112)
    big_tile<GATEUP, 8>(wq, wsh, act, act_sum, e, n, rt, h16m, out);
  else if (n > 96)
    big_tile<GATEUP, 7>(wq, wsh, act, act_sum, e, n, rt, h16m, out);
  else if (n > 80)
    big_tile<GATEUP, 6>(wq, wsh, act, act_sum, e, n, rt, h16m, out);
  else if (n > 64)
    big_tile<GATEUP, 5>(wq, wsh, act, act_sum, e, n, rt, h16m, out);
  else if (n > 48)
    big_tile<GATEUP, 4>(wq, wsh, act, act_sum, e, n, rt, h16m, out);
  else if (n > 32)
    big_tile<GATEUP, 3>(wq, wsh, act, act_sum, e, n, rt, h16m, out);
  else if (n > 16)
    big_tile<GATEUP, 2>(wq, wsh, act, act_sum, e, n, rt, h16m, out);
  else
    big_tile<GATEUP, 1>(wq, wsh, act, act_sum, e, n, rt, h16m, out);
}

template __global__ void k_moe_big<true>(const uint8_t *, const uint8_t *, const __half *, const __half *,
                                         const int32_t *, const int4 *, const int32_t *, int,
                                         int, __half *, float *);
template __global__ void k_moe_big<false>(const uint8_t *, const uint8_t *, const __half *, const __half *,
                                          const int32_t *, const int4 *, const int32_t *, int,
                                          int, __half *, float *);

}  // namespace mfma_big
}  // namespace hy3x
