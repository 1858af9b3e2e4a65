// hy3x_common.h -- shared constants and device helpers for the gfx950 MoE block.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace hy3x {

constexpr int D = 4096;        // hidden size
constexpr int F = 1536;        // expert intermediate size
constexpr int E = 192;         // routed experts; expert index E is the shared expert
constexpr int KMAX = 8;        // top-K upper bound
constexpr int QK = 256;        // weights per Q4_K super-block
constexpr int QB = 144;        // bytes per Q4_K super-block
constexpr int64_t MAT_BYTES = 3538944;          // one 1536x4096 matrix in Q4_K
constexpr int64_t EXPERT_BYTES = 3 * MAT_BYTES;  // gate | up | down
constexpr int WAVE = 64;

// fp16 -> fp32 exactly as hy3.c:354-369 decodes Q4_K d/dmin: exponent 0
// (zero and subnormal halves) becomes 2^-15 * (1 + mant/1024).
__device__ __forceinline__ float fp16_quirk(uint32_t h) {
  const uint32_t ex = (h >> 10) & 31u;
  const uint32_t e32 = ex == 0u ? 112u : (ex == 31u ? 255u : ex + 112u);
  return __uint_as_float(((h & 0x8000u) << 16) | (e32 << 23) | ((h & 0x3ffu) << 13));
}

// Activation staging for the Q4_K dot kernels ("pair-staged" fp16 layout).
// A length-K vector is split into groups of 64 elements (group g = Q4_K block
// g/4, sub-block pair g%4: elements 0..31 are the low-nibble sub-block,
// 32..63 the high-nibble one). Each group is 32 dwords of fp16 pairs so that
// dword j of the weights' qs, unpacked with two masks and one shift, meets its
// activations in dot2 order:
//   dword 4j+0 = (x[4j+0],    x[4j+2]   )   low nibbles of bytes 0,2
//   dword 4j+1 = (x[32+4j+0], x[32+4j+2])   high nibbles of bytes 0,2
//   dword 4j+2 = (x[4j+1],    x[4j+3]   )   low nibbles of bytes 1,3
//   dword 4j+3 = (x[32+4j+1], x[32+4j+3])   high nibbles of bytes 1,3
// Returns the fp16 (half-word) index of element i within the staged vector.
__host__ __device__ __forceinline__ int stage_index(int i) {
  const int g = i >> 6, r = i & 63, hi = r >> 5, l = r & 31;
  const int j = l >> 2, e = l & 3;
  return g * 64 + 2 * (4 * j + hi + ((e & 1) << 1)) + (e >> 1);
}

// Position of element k inside its run of 8 in the MFMA-staged fp16 layout:
// the run holds k order (0,2,1,3,4,6,5,7), the order the nibble unpack of the
// Q4_K bytes produces.
__host__ __device__ __forceinline__ int perm8(int k) {
  const int lo = k & 7;
  const int p = lo == 1 ? 2 : lo == 2 ? 1 : lo == 5 ? 6 : lo == 6 ? 5 : lo;
  return (k & ~7) | p;
}

// 64-lane xor-butterfly sum (every lane ends with the total). The addition
// order is fixed: v_l += v_{l^o} for o = 32, 16, 8, 4, 2, 1.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Sum over each 32-lane half (lanes 0..31 and 32..63 reduced separately).
__device__ __forceinline__ float half_sum(float v) {
#pragma unroll
  for (int o = 16; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// DPP moves (gfx9 encodings): quad_perm [1,0,3,2] / [2,3,0,1], row_half_mirror,
// row_mirror, row_bcast:15, row_bcast:31.
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140,
              DPP_BCAST15 = 0x142, DPP_BCAST31 = 0x143;

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dppi(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

// Sum over each row of 16 lanes; every lane of the row receives the row sum:
// v += xor1, v += xor2, v += half-mirror (lane i <-> 7-i in each 8), v +=
// mirror (i <-> 15-i in each 16), in that fixed order.
__device__ __forceinline__ float row16_sum(float v) {
#pragma clang fp contract(off)
  v += dpp<DPP_XOR1>(v);
  v += dpp<DPP_XOR2>(v);
  v += dpp<DPP_HALF_MIRROR>(v);
  v += dpp<DPP_MIRROR>(v);
  return v;
}

// Sum over the 64 lanes, returned as a wave-uniform value.
__device__ __forceinline__ float wave_total(float v) {
  v = row16_sum(v);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32)) +
         __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
}

// Sums over each 32-lane half: .x = lanes 0..31, .y = lanes 32..63 (uniform).
__device__ __forceinline__ float2 half_totals(float v) {
  v = row16_sum(v);
  const int b = __builtin_bit_cast(int, v);
  return make_float2(__builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)) +
                         __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16)),
                     __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)) +
                         __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48)));
}

// Optional per-block timestamps for diagnostics (REALTIME counter, 100 MHz):
// when trace_buf is non-null, thread 0 of block b writes checkpoint i to
// trace_buf[b * 8 + i].
__device__ __forceinline__ void trace_point(unsigned long long *trace_buf, int i) {
  if (trace_buf && threadIdx.x == 0) {
    const unsigned long long t = __builtin_amdgcn_s_memrealtime();
    __hip_atomic_store(&trace_buf[blockIdx.x * 8 + i], t, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + __expf(-v)); }

// The staged fp16 h = silu(g) * u: the product rounded to fp32, then to fp16.
// The empty asm pins the fp32 product in a register: otherwise the backend
// fuses the multiply into the conversion (v_fma_mix, one rounding) for some
// accumulator elements and not others, and a token's h then depends on its
// row in the MFMA tile. Every kernel and element now rounds the same way.
__device__ __forceinline__ __half swiglu_h(float g, float u) {
  float h = silu(g) * u;
  asm volatile("" : "+v"(h));
  return __float2half(h);
}

// Four elements of the residual stream x, plus the addend xadd when the
// forward carries one (x + attn_out, the residual add of hy3.c:1264 and of
// add_rmsnorm_kernel, hy3_gpu.cu:453-460; the same fp32 add in every reader).
// Branch-free, so that a caller's other loads stay in flight: without an
// addend the second load re-reads x (a cache hit) and its sum is discarded.
__device__ __forceinline__ float4 load_x4(const float *x, const float *xadd, size_t i4) {
  const float4 v = reinterpret_cast<const float4 *>(x)[i4];
  const float4 a = reinterpret_cast<const float4 *>(xadd ? xadd : x)[i4];
  const float4 s = make_float4(v.x + a.x, v.y + a.y, v.z + a.z, v.w + a.w);
  return xadd ? s : v;
}

}  // namespace hy3x
