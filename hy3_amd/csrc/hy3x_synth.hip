// hy3x_synth.hip -- seeded synthetic Hy3 MoE layers (benchmark/test inputs).
//
// Not part of the MoE forward. Generates the configurations' expert weights
// directly in device memory and quantises them to Q4_K with the arithmetic of
// hy3_convert.c:605-651 as the reference Makefile compiles it (-O3
// -ffast-math): constant divisions become multiplies by rounded reciprocals,
// 1/(max/63) is folded to 62.999996f/max, and each "v/d + 0.5" is
// fmaf(v, 1/d, 0.5) before the truncating cast. fp32 -> fp16 truncates
// (hy3_convert.c:511-530).
//
// Values: SplitMix64 counter RNG keyed by (seed, layer, tensor kind, expert);
// an approximate N(0, sigma) value is the Irwin-Hall sum of twelve 16-bit
// uniforms, exact in integers, then one float multiply.
#include <math.h>
#include <string.h>

#include "hy3x_kernels.h"
#include "hy3x_q8.h"

#pragma clang fp contract(off)

namespace hy3x {

__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__host__ __device__ __forceinline__ uint64_t tensor_key(uint64_t seed, uint32_t layer,
                                                        uint32_t kind, uint32_t index) {
  const uint64_t tid =
      ((uint64_t)layer << 32) | ((uint64_t)(kind & 0xFFu) << 24) | (index & 0xFFFFFFu);
  return splitmix64(seed ^ splitmix64(tid));
}

__host__ __device__ __forceinline__ float synth_normal(uint64_t key, uint64_t i, float sigma) {
  int32_t s = 0;
  for (int j = 0; j < 3; j++) {
    const uint64_t r = splitmix64(key + 3 * i + (uint64_t)j);
    for (int h = 0; h < 4; h++) s += 2 * (int32_t)((r >> (16 * h)) & 0xFFFFu) + 1;
  }
  return (float)(s - 786432) * (sigma * (1.0f / 131072.0f));
}

__device__ __forceinline__ uint16_t fp32_to_fp16_trunc(float f) {
  const uint32_t x = __float_as_uint(f);
  const uint32_t sign = (x >> 31) & 1u, ex = (x >> 23) & 0xffu, man = x & 0x7fffffu;
  if (ex == 0) return (uint16_t)(sign << 15);
  if (ex == 0xff) return (uint16_t)((sign << 15) | 0x7c00u | (man ? 1u : 0u));
  const int ne = (int)ex - 112;
  if (ne >= 31) return (uint16_t)((sign << 15) | 0x7c00u);
  if (ne <= 0) return (uint16_t)((sign << 15) | (((man | 0x800000u) >> (1 - ne)) >> 13));
  return (uint16_t)((sign << 15) | ((uint32_t)ne << 10) | (man >> 13));
}

// (int)v as the reference's x86 build executes it: truncation, and INT_MIN
// for NaN or values outside the int range (the GPU's own conversion would
// saturate instead).
__device__ __forceinline__ int cvt_trunc_x86(float v) {
  return (v >= -2147483648.0f && v < 2147483648.0f) ? (int)v : (int)0x80000000u;
}

// One wave per Q4_K block; lane L holds elements 4L..4L+3 (sub-block L/8).
// src == nullptr: generate the block of the whole-layer arena (193 experts x
// gate|up|down, contiguous) from (seed, layer); otherwise quantise src.
__global__ __launch_bounds__(256) void k_synth_q4k(uint8_t *dst, int64_t nblocks, uint64_t seed,
                                                   uint32_t layer, const float *src) {
  const int64_t bi = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (bi >= nblocks) return;
  const int lane = threadIdx.x & 63;
  float v[4];
  if (src) {
    const float4 t = reinterpret_cast<const float4 *>(src + bi * QK)[lane];
    v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
  } else {
    const int64_t per_mat = MAT_BYTES / QB;  // 24576 blocks
    const int64_t em = bi / per_mat, lb = bi - em * per_mat;
    const uint32_t e = (uint32_t)(em / 3), m = (uint32_t)(em % 3);
    const uint64_t key = tensor_key(seed, layer, 5u + m, e);
#pragma unroll
    for (int c = 0; c < 4; c++) v[c] = synth_normal(key, (uint64_t)(lb * QK + 4 * lane + c), 0.02f);
  }
  float mn = fminf(fminf(v[0], v[1]), fminf(v[2], v[3]));
  float mx = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
#pragma unroll
  for (int o = 1; o <= 4; o <<= 1) {
    mn = fminf(mn, __shfl_xor(mn, o, 64));
    mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  }
  const float inv15 = 1.0f / 15.0f, inv63 = 1.0f / 63.0f, c63 = 1.0f / inv63;
  const float sub_scale = (mx - mn) * inv15;
  const float sub_min = mn < 0 ? -mn : 0.0f;
  float max_s = sub_scale, max_m = sub_min;
#pragma unroll
  for (int o = 8; o <= 32; o <<= 1) {
    max_s = fmaxf(max_s, __shfl_xor(max_s, o, 64));
    max_m = fmaxf(max_m, __shfl_xor(max_m, o, 64));
  }
  if (max_s < 1e-10f) max_s = 1e-10f;
  if (max_m < 1e-10f) max_m = 1e-10f;
  const float d = max_s * inv63, dmin = max_m * inv63;
  const float rd = c63 / max_s, rdm = c63 / max_m;
  int ls = cvt_trunc_x86(__builtin_fmaf(sub_scale, rd, 0.5f));
  int lm = cvt_trunc_x86(__builtin_fmaf(sub_min, rdm, 0.5f));
  ls = ls < 0 ? 0 : (ls > 63 ? 63 : ls);
  lm = lm < 0 ? 0 : (lm > 63 ? 63 : lm);
  const float eff_d = d * (float)ls, eff_dm = dmin * (float)lm;
  const float rq = 1.0f / (eff_d > 1e-10f ? eff_d : 1e-10f);
  uint32_t packed = 0;
#pragma unroll
  for (int c = 0; c < 4; c++) {
    int q = cvt_trunc_x86(__builtin_fmaf(v[c] + eff_dm, rq, 0.5f));
    q = q < 0 ? 0 : (q > 15 ? 15 : q);
    packed |= (uint32_t)q << (8 * c);
  }
  const uint32_t hi = __shfl_down(packed, 8, 64);
  uint8_t *blk = dst + bi * QB;
  const int j = lane >> 3;  // sub-block of this lane
  if ((j & 1) == 0) {       // even sub-block: low nibbles; partner lane L+8 gives the high ones
    const int l = 4 * (lane & 7);
    *reinterpret_cast<uint32_t *>(blk + 16 + 32 * (j >> 1) + l) = packed | (hi << 4);
  }
  int lsv[8], lmv[8];
#pragma unroll
  for (int s = 0; s < 8; s++) {
    lsv[s] = __shfl(ls, 8 * s, 64);
    lmv[s] = __shfl(lm, 8 * s, 64);
  }
  if (lane == 0) {
    uint8_t sc[12];
    for (int s = 0; s < 12; s++) sc[s] = 0;
    for (int s = 0; s < 8; s++) {
      if (s < 4) {
        sc[s] = (uint8_t)lsv[s];
        sc[s + 4] = (uint8_t)lmv[s];
      } else {
        sc[s + 4] = (uint8_t)((lsv[s] & 0xF) | ((lmv[s] & 0xF) << 4));
        sc[s - 4] |= (uint8_t)((lsv[s] >> 4) << 6);
        sc[s] |= (uint8_t)((lmv[s] >> 4) << 6);
      }
    }
    uint4 h;
    h.x = (uint32_t)fp32_to_fp16_trunc(d) | ((uint32_t)fp32_to_fp16_trunc(dmin) << 16);
    h.y = sc[0] | (sc[1] << 8) | (sc[2] << 16) | ((uint32_t)sc[3] << 24);
    h.z = sc[4] | (sc[5] << 8) | (sc[6] << 16) | ((uint32_t)sc[7] << 24);
    h.w = sc[8] | (sc[9] << 8) | (sc[10] << 16) | ((uint32_t)sc[11] << 24);
    *reinterpret_cast<uint4 *>(blk) = h;
  }
}

// hy3 Q8_0 (36-byte blocks, hy3.c:400-403) -> q8x128 super-blocks (hy3x_q8.h):
// one thread per super-block of 4 source blocks. Source blocks are 4-byte
// aligned, so everything moves as dwords.
__global__ __launch_bounds__(256) void k_repack_q8x128(const uint8_t *__restrict__ src,
                                                       uint8_t *__restrict__ dst,
                                                       int64_t n_super) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n_super) return;
  const uint32_t *s = reinterpret_cast<const uint32_t *>(src + i * 4 * Q8_BLOCK);
  uint32_t *o = reinterpret_cast<uint32_t *>(dst + i * QB);
#pragma unroll
  for (int b = 0; b < 4; b++) {
    o[b] = s[9 * b];
#pragma unroll
    for (int w = 0; w < 8; w++) o[4 + 8 * b + w] = s[9 * b + 1 + w];
  }
}

// hy3_convert.c:1192-1221 on the device, one thread per 32-weight block:
// d = amax * (1/127) (the reference build's reciprocal multiply), floored at
// 1e-10; q = x * (1/d) rounded half away from zero, clamped to +-127. src ==
// nullptr: the block's values are the synthetic normals of matrix `key`
// (element index 32 b + k, sigma 0.02); otherwise src[32 b + k].
__global__ __launch_bounds__(256) void k_synth_q8_0(uint8_t *__restrict__ dst, int64_t nblocks,
                                                    uint64_t key, const float *__restrict__ src) {
#pragma clang fp contract(off)
  const int64_t b = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (b >= nblocks) return;
  float v[32];
#pragma unroll
  for (int k = 0; k < 32; k++)
    v[k] = src ? src[b * 32 + k] : synth_normal(key, (uint64_t)(b * 32 + k), 0.02f);
  float amax = 0.0f;
#pragma unroll
  for (int k = 0; k < 32; k++) amax = fmaxf(amax, fabsf(v[k]));
  float d = amax * (1.0f / 127.0f);
  if (d < 1e-10f) d = 1e-10f;
  const float id = 1.0f / d;
  uint32_t *o = reinterpret_cast<uint32_t *>(dst + b * Q8_BLOCK);
  o[0] = __float_as_uint(d);
#pragma unroll
  for (int w = 0; w < 8; w++) {
    uint32_t word = 0;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const float t = v[4 * w + c] * id;
      int q = (int)(t + (t >= 0.0f ? 0.5f : -0.5f));
      q = q > 127 ? 127 : (q < -127 ? -127 : q);
      word |= (uint32_t)(uint8_t)(int8_t)q << (8 * c);
    }
    o[1 + w] = word;
  }
}

// Diagnostics: a plain streaming read of n16 16-byte words (a grid-stride
// loop, eight loads in flight per thread), the reference point for what a
// launch reading that many bytes can achieve. The XOR of the data is kept
// live through a store that never happens for real inputs.
__global__ __launch_bounds__(256) void k_stream_read(const uint4 *__restrict__ p, int64_t n16,
                                                     uint32_t *__restrict__ sink) {
  int64_t i = (int64_t)blockIdx.x * 256 * 8 + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * 256 * 8;
  uint32_t acc = 0;
  for (; i < n16; i += stride) {
    uint4 v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) v[u] = i + 256 * u < n16 ? p[i + 256 * u] : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < 8; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

}  // namespace hy3x

using namespace hy3x;

extern "C" {

uint64_t hy3x_synth_key(uint64_t seed, uint32_t layer, uint32_t kind, uint32_t index) {
  return tensor_key(seed, layer, kind, index);
}

void hy3x_synth_normal(float *dst, int64_t n, uint64_t key, uint64_t first, float sigma,
                       float offset) {
  for (int64_t k = 0; k < n; k++) dst[k] = offset + synth_normal(key, first + (uint64_t)k, sigma);
}

void hy3x_synth_uniform_sym(float *dst, int64_t n, uint64_t key, float a) {
  for (int64_t k = 0; k < n; k++) {
    const uint32_t u = (uint32_t)(splitmix64(key + (uint64_t)k) >> 40);
    const float t = (float)((int32_t)(2u * u + 1u) - (1 << 24)) * (1.0f / 16777216.0f);
    dst[k] = t * a;
  }
}

void hy3x_synth_zipf_bias(float *dst, int n_expert, uint64_t seed) {
  int perm[1024];
  if (n_expert > 1024) n_expert = 1024;
  const uint64_t key = tensor_key(seed, 0, 4, 0xFFFFFu);
  for (int i = 0; i < n_expert; i++) perm[i] = i;
  for (int i = n_expert - 1; i > 0; i--) {
    const int j = (int)(splitmix64(key + (uint64_t)i) % (uint64_t)(i + 1));
    const int t = perm[i];
    perm[i] = perm[j];
    perm[j] = t;
  }
  for (int r = 0; r < n_expert; r++) dst[perm[r]] = (float)(0.5 * pow(1.0 / (double)(r + 1), 0.8));
}

}  // extern "C"
