/*
 * hy3_oracle.c -- CPU restatement of the Hy3 MoE FFN block.
 *
 * TEST INFRASTRUCTURE ONLY: this file is the checker for the HIP kernels in
 * hy3_amd/csrc and the CPU baseline of the benchmark. The product path never
 * links or calls it.
 *
 * Build: strict IEEE (-O2 -fno-fast-math -ffp-contract=off -fopenmp), see
 * oracle/Makefile. Every fmaf below is intentional; every other a*b+c is two
 * roundings, exactly as written.
 */
#include "hy3_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ======================================================================== */
/* Synthetic inputs                                                          */
/* ======================================================================== */

/* SplitMix64 (Steele, Lea, Flood 2014; constants as published by Vigna). */
uint64_t hy3o_splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

uint64_t hy3o_tensor_key(uint64_t seed, uint32_t layer, uint32_t kind, uint32_t index) {
  uint64_t tid = ((uint64_t)layer << 32) | ((uint64_t)(kind & 0xFFu) << 24) | (index & 0xFFFFFFu);
  return hy3o_splitmix64(seed ^ hy3o_splitmix64(tid));
}

static inline int32_t irwin_hall_sum(uint64_t key, uint64_t i) {
  int32_t s = 0;
  for (int j = 0; j < 3; j++) {
    uint64_t r = hy3o_splitmix64(key + 3 * i + (uint64_t)j);
    for (int h = 0; h < 4; h++) s += 2 * (int32_t)((r >> (16 * h)) & 0xFFFFu) + 1;
  }
  return s - 786432; /* 12 * 65536 */
}

float hy3o_normal(uint64_t key, uint64_t i, float sigma) {
  const float scale = sigma * (1.0f / 131072.0f); /* exact: power-of-two scaling */
  return (float)irwin_hall_sum(key, i) * scale;
}

float hy3o_uniform_sym(uint64_t key, uint64_t i, float a) {
  uint32_t u = (uint32_t)(hy3o_splitmix64(key + i) >> 40);
  float t = (float)((int32_t)(2u * u + 1u) - (1 << 24)) * (1.0f / 16777216.0f);
  return t * a;
}

void hy3o_fill_normal(float *dst, size_t n, uint64_t key, uint64_t first, float sigma,
                      float offset) {
#pragma omp parallel for schedule(static)
  for (long long k = 0; k < (long long)n; k++)
    dst[k] = offset + hy3o_normal(key, first + (uint64_t)k, sigma);
}

void hy3o_fill_uniform_sym(float *dst, size_t n, uint64_t key, float a) {
  for (size_t k = 0; k < n; k++) dst[k] = hy3o_uniform_sym(key, k, a);
}

void hy3o_zipf_bias(float *dst, int n_expert, uint64_t seed) {
  int perm[1024];
  uint64_t key = hy3o_tensor_key(seed, 0, HY3O_T_BIAS, 0xFFFFFu);
  for (int i = 0; i < n_expert; i++) perm[i] = i;
  for (int i = n_expert - 1; i > 0; i--) {
    int j = (int)(hy3o_splitmix64(key + (uint64_t)i) % (uint64_t)(i + 1));
    int t = perm[i]; perm[i] = perm[j]; perm[j] = t;
  }
  for (int r = 0; r < n_expert; r++)
    dst[perm[r]] = (float)(0.5 * pow(1.0 / (double)(r + 1), 0.8));
}

/* ======================================================================== */
/* fp16 and Q4_K                                                             */
/* ======================================================================== */

/* hy3.c:354-369. exp==0 (zero and subnormal halves) decodes as
 * 2^-15 * (1 + mant/1024) with the sign applied: the reference's quirk. */
float hy3o_fp16_to_fp32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15), ex = (uint32_t)((h >> 10) & 0x1f), man = h & 0x3ffu;
  uint32_t bits;
  if (ex == 0) bits = (sign << 31) | ((uint32_t)(127 - 15) << 23) | (man << 13);
  else if (ex == 31) bits = (sign << 31) | 0x7f800000u | (man << 13);
  else bits = (sign << 31) | ((ex + 112u) << 23) | (man << 13);
  float r;
  memcpy(&r, &bits, 4);
  return r;
}

/* hy3_convert.c:511-530: truncating conversion; fp32 exp==0 -> signed zero. */
uint16_t hy3o_fp32_to_fp16_trunc(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  uint32_t sign = (x >> 31) & 1u, ex = (x >> 23) & 0xffu, man = x & 0x7fffffu;
  if (ex == 0) return (uint16_t)(sign << 15);
  if (ex == 0xff) return (uint16_t)((sign << 15) | 0x7c00u | (man ? 1u : 0u));
  int ne = (int)ex - 112;
  if (ne >= 31) return (uint16_t)((sign << 15) | 0x7c00u);
  if (ne <= 0) return (uint16_t)((sign << 15) | (((man | 0x800000u) >> (1 - ne)) >> 13));
  return (uint16_t)((sign << 15) | ((uint32_t)ne << 10) | (man >> 13));
}

/* hy3.c:1001-1009: 6-bit scale and min of sub-block j from the 12 packed bytes. */
void hy3o_q4k_scale_min(int j, const uint8_t *q, uint8_t *sc, uint8_t *m) {
  if (j < 4) {
    *sc = q[j] & 63;
    *m = q[j + 4] & 63;
  } else {
    *sc = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
    *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
  }
}

/* hy3.c:1019-1043. Chunk c (64 weights) reads qs[32c..32c+31]: the low nibble
 * is sub-block 2c, the high nibble sub-block 2c+1. */
void hy3o_dequant_q4k(float *dst, const uint8_t *src, int64_t n) {
  int64_t nb = n / HY3O_QK;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < nb; i++) {
    const uint8_t *b = src + i * HY3O_BLOCK_BYTES;
    uint16_t hd, hm;
    memcpy(&hd, b, 2);
    memcpy(&hm, b + 2, 2);
    const float d = hy3o_fp16_to_fp32(hd), dmin = hy3o_fp16_to_fp32(hm);
    const uint8_t *sc = b + 4, *q = b + 16;
    float *y = dst + i * HY3O_QK;
    for (int c = 0; c < 4; c++) {
      uint8_t s1, m1, s2, m2;
      hy3o_q4k_scale_min(2 * c, sc, &s1, &m1);
      hy3o_q4k_scale_min(2 * c + 1, sc, &s2, &m2);
      const float d1 = d * (float)s1, dm1 = dmin * (float)m1;
      const float d2 = d * (float)s2, dm2 = dmin * (float)m2;
      for (int l = 0; l < 32; l++) y[l] = d1 * (float)(q[l] & 0xF) - dm1;
      for (int l = 0; l < 32; l++) y[32 + l] = d2 * (float)(q[l] >> 4) - dm2;
      y += 64;
      q += 32;
    }
  }
}

/* (int)v as the reference's x86 build executes it (cvttss2si): truncation, and
 * INT_MIN for NaN or anything outside the int range (C leaves that undefined;
 * the quantiser reaches it for constant blocks, where 1/max(eff_d, 1e-10)
 * scales values past 2^31). */
static inline int cvt_trunc_x86(float v) {
  return (v >= -2147483648.0f && v < 2147483648.0f) ? (int)v : (int)0x80000000u;
}

/* hy3_convert.c:605-651 as its Makefile builds it (-O3 -ffast-math): the
 * divisions by the constants 15 and 63 become multiplies by their rounded
 * reciprocals, 1/d is folded to 62.999996f/max_s, each remaining division v/d
 * becomes v * (1/d), and every
 * "v * r + 0.5" is one fused multiply-add before the truncating int cast.
 * This reproduces the compiled reference quantiser bit for bit (pinned by the
 * golden fixtures); a literal IEEE reading of the source differs from it in
 * about 6 of 10,000 blocks. */
static void quantize_block_q4k(const float *xb, uint8_t *out) {
  const float inv15 = 1.0f / 15.0f, inv63 = 1.0f / 63.0f;
  float sub_scale[8], sub_min[8];
  uint8_t L[HY3O_QK];
  for (int j = 0; j < 8; j++) {
    float smin = FLT_MAX, smax = -FLT_MAX;
    for (int l = 0; l < 32; l++) {
      float v = xb[32 * j + l];
      if (v < smin) smin = v;
      if (v > smax) smax = v;
    }
    sub_scale[j] = (smax - smin) * inv15;
    sub_min[j] = smin < 0 ? -smin : 0;
  }
  float max_s = 0, max_m = 0;
  for (int j = 0; j < 8; j++) {
    if (sub_scale[j] > max_s) max_s = sub_scale[j];
    if (sub_min[j] > max_m) max_m = sub_min[j];
  }
  if (max_s < 1e-10f) max_s = 1e-10f;
  if (max_m < 1e-10f) max_m = 1e-10f;
  const float d = max_s * inv63, dmin = max_m * inv63;
  /* 1/(max*(1/63)) is folded to (1/(1/63))/max = 62.999996f/max. */
  const float c63 = 1.0f / inv63;
  const float rd = c63 / max_s, rdm = c63 / max_m;
  uint16_t hd = hy3o_fp32_to_fp16_trunc(d), hm = hy3o_fp32_to_fp16_trunc(dmin);
  memcpy(out, &hd, 2);
  memcpy(out + 2, &hm, 2);
  uint8_t *scales = out + 4;
  memset(scales, 0, 12);
  for (int j = 0; j < 8; j++) {
    int ls = cvt_trunc_x86(fmaf(sub_scale[j], rd, 0.5f));
    int lm = cvt_trunc_x86(fmaf(sub_min[j], rdm, 0.5f));
    if (ls < 0) ls = 0;
    if (ls > 63) ls = 63;
    if (lm < 0) lm = 0;
    if (lm > 63) lm = 63;
    if (j < 4) {
      scales[j] = (uint8_t)ls;
      scales[j + 4] = (uint8_t)lm;
    } else {
      scales[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
      scales[j - 4] |= (uint8_t)((ls >> 4) << 6);
      scales[j] |= (uint8_t)((lm >> 4) << 6);
    }
    const float eff_d = d * (float)ls, eff_dm = dmin * (float)lm;
    const float rq = 1.0f / (eff_d > 1e-10f ? eff_d : 1e-10f);
    for (int i = 0; i < 32; i++) {
      int q = cvt_trunc_x86(fmaf(xb[32 * j + i] + eff_dm, rq, 0.5f));
      if (q < 0) q = 0;
      if (q > 15) q = 15;
      L[32 * j + i] = (uint8_t)q;
    }
  }
  uint8_t *qs = out + 16;
  for (int j = 0; j < HY3O_QK; j += 64) {
    for (int l = 0; l < 32; l++) qs[l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
    qs += 32;
  }
}

void hy3o_quantize_q4k(const float *x, uint8_t *dst, int64_t n) {
  int64_t nb = n / HY3O_QK;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < nb; i++)
    quantize_block_q4k(x + i * HY3O_QK, dst + i * HY3O_BLOCK_BYTES);
}

void hy3o_gen_q4k_matrix(uint8_t *dst, int rows, int cols, uint64_t key, float sigma) {
  int64_t nb = (int64_t)rows * cols / HY3O_QK;
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < nb; b++) {
    float xb[HY3O_QK];
    for (int k = 0; k < HY3O_QK; k++) xb[k] = hy3o_normal(key, (uint64_t)(b * HY3O_QK + k), sigma);
    quantize_block_q4k(xb, dst + b * HY3O_BLOCK_BYTES);
  }
}

/* hy3_convert.c:1192-1221: d = amax / 127 (the build multiplies by the fp32
 * reciprocal of 127), floored at 1e-10; q = v rounded half away from zero,
 * v = x * (1/d), clamped to [-127, 127]; stored as f32 d then 32 int8. */
static void quantize_block_q8_0(const float *xb, uint8_t *out) {
  float amax = 0.0f;
  for (int k = 0; k < 32; k++) {
    const float a = fabsf(xb[k]);
    if (a > amax) amax = a;
  }
  float d = amax * (1.0f / 127.0f);
  if (d < 1e-10f) d = 1e-10f;
  const float id = 1.0f / d;
  memcpy(out, &d, 4);
  for (int k = 0; k < 32; k++) {
    const float v = xb[k] * id;
    int q = (int)(v + (v >= 0.0f ? 0.5f : -0.5f));
    if (q > 127) q = 127;
    if (q < -127) q = -127;
    out[4 + k] = (uint8_t)(int8_t)q;
  }
}

void hy3o_quantize_q8_0(const float *x, uint8_t *dst, int64_t n) {
  const int64_t nb = n / 32;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < nb; i++) quantize_block_q8_0(x + i * 32, dst + i * HY3O_Q8_BLOCK);
}

void hy3o_dequant_q8_0(float *dst, const uint8_t *src, int64_t n) {
  for (int64_t i = 0; i < n / 32; i++) {
    float d;
    memcpy(&d, src + i * HY3O_Q8_BLOCK, 4);
    const int8_t *q = (const int8_t *)(src + i * HY3O_Q8_BLOCK + 4);
    for (int k = 0; k < 32; k++) dst[i * 32 + k] = d * (float)q[k];
  }
}

void hy3o_gen_q8_0_matrix(uint8_t *dst, int rows, int cols, uint64_t key, float sigma) {
  const int64_t nb = (int64_t)rows * cols / 32;
#pragma omp parallel for schedule(static)
  for (int64_t b = 0; b < nb; b++) {
    float xb[32];
    for (int k = 0; k < 32; k++) xb[k] = hy3o_normal(key, (uint64_t)(b * 32 + k), sigma);
    quantize_block_q8_0(xb, dst + b * HY3O_Q8_BLOCK);
  }
}

/* ======================================================================== */
/* Routing contract                                                          */
/* ======================================================================== */

/* The reduction order the reference's build gives these sums (gcc -O3
 * -ffast-math, 8-wide FMA vectors): eight chains, chain v accumulating
 * a[8i+v]*b[8i+v] with fmaf for i ascending from 0, then the horizontal tree
 * ((a1+a5)+(a3+a7)) + ((a0+a4)+(a2+a6)). */
static float tree8(const float *a) {
  const float t0 = a[0] + a[4], t1 = a[1] + a[5], t2 = a[2] + a[6], t3 = a[3] + a[7];
  const float u0 = t2 + t0, u1 = t3 + t1;
  return u1 + u0;
}

float hy3o_dot8(const float *a, const float *b, int n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int i = 0; i < n / 8; i++)
    for (int v = 0; v < 8; v++) acc[v] = fmaf(a[8 * i + v], b[8 * i + v], acc[v]);
  return tree8(acc);
}

/* exp(x) rounded to fp32 from a double-precision evaluation: Cody-Waite
 * reduction x = k*ln2 + r (two-part ln2 in double), a degree-13 Taylor
 * polynomial for e^r (|r| <= 0.35, truncation < 1e-17 relative) and exact
 * scaling by 2^k. The double result is within a few ulp(double) of e^x, so the
 * final rounding gives the correctly rounded float except in cases closer to a
 * rounding boundary than ~1e-15 relative. Used only for the router sigmoid;
 * inputs below -87 return 0 (1 + e^x rounds to 1 there anyway). */
float hy3o_sig_expf(float xf) {
  if (xf != xf) return xf;
  if (xf > 88.72f) return INFINITY;
  if (xf < -87.0f) return 0.0f;
  const double x = (double)xf;
  const double kd = rint(x * 1.4426950408889634);
  double r = fma(kd, -6.93147180369123816490e-01, x);
  r = fma(kd, -1.90821492927058770002e-10, r);
  double p = 1.0 / 6227020800.0;
  p = fma(p, r, 1.0 / 479001600.0);
  p = fma(p, r, 1.0 / 39916800.0);
  p = fma(p, r, 1.0 / 3628800.0);
  p = fma(p, r, 1.0 / 362880.0);
  p = fma(p, r, 1.0 / 40320.0);
  p = fma(p, r, 1.0 / 5040.0);
  p = fma(p, r, 1.0 / 720.0);
  p = fma(p, r, 1.0 / 120.0);
  p = fma(p, r, 1.0 / 24.0);
  p = fma(p, r, 1.0 / 6.0);
  p = fma(p, r, 0.5);
  p = fma(p, r, 1.0);
  p = fma(p, r, 1.0);
  const int64_t k = (int64_t)kd;
  uint64_t bits = (uint64_t)(k + 1023) << 52;
  double s;
  memcpy(&s, &bits, 8);
  return (float)(p * s);
}

/* RMSNorm (hy3.c:435-444) with n = 4096: ss in the block order above, r =
 * 1/sqrt(ss/n + eps) correctly rounded (the build uses an rsqrt estimate
 * refined by one Newton step, whose last bits depend on the host CPU), out =
 * (x * w) * r (the build's reassociation of x * r * w). */
/* Sum of squares over 4096 elements in the order of a 256-thread block:
 * thread t accumulates x[1024i + 4t + c]^2 with fmaf for i = 0..3 (outer),
 * c = 0..3 (inner) from 0; each 64-thread wave reduces with v[l] += v[l^1],
 * v[l] += v[l^2], v[l] += v[mirror8(l)], v[l] += v[mirror16(l)], its total is
 * (v[0] + v[16]) + (v[32] + v[48]); the block total is (W0 + W1) + (W2 + W3).
 * (The reference build's r comes from an rsqrt estimate whose bits depend on
 * the host CPU, so no summation order reproduces it; this one is fast on the
 * GPU and restated exactly here.) */
float hy3o_sumsq_block(const float *x) {
  float W[4];
  for (int w = 0; w < 4; w++) {
    float v[64], u[64];
    for (int l = 0; l < 64; l++) {
      const int t = 64 * w + l;
      float acc = 0.0f;
      for (int i = 0; i < 4; i++)
        for (int c = 0; c < 4; c++) {
          const float a = x[1024 * i + 4 * t + c];
          acc = fmaf(a, a, acc);
        }
      v[l] = acc;
    }
    for (int l = 0; l < 64; l++) u[l] = v[l] + v[l ^ 1];
    for (int l = 0; l < 64; l++) v[l] = u[l] + u[l ^ 2];
    for (int l = 0; l < 64; l++) u[l] = v[l] + v[(l & ~7) | (7 - (l & 7))];
    for (int l = 0; l < 64; l++) v[l] = u[l] + u[(l & ~15) | (15 - (l & 15))];
    W[w] = (v[0] + v[16]) + (v[32] + v[48]);
  }
  return (W[0] + W[1]) + (W[2] + W[3]);
}

static float rms_scale(const float *x, int n) {
  const float ss = hy3o_sumsq_block(x);
  return 1.0f / sqrtf(ss / (float)n + HY3O_RMS_EPS);
}

void hy3o_rms_norm(float *out, const float *x, const float *w, int n) {
  const float r = rms_scale(x, n);
  for (int i = 0; i < n; i++) out[i] = (x[i] * w[i]) * r;
}

/* hy3.c:654-666. */
void hy3o_topk_select(float *vals, int *inds, const float *scores, int n, int k) {
  int idx[1024];
  float val[1024];
  for (int i = 0; i < n; i++) {
    idx[i] = i;
    val[i] = scores[i];
  }
  for (int i = 0; i < k && i < n; i++) {
    int best = i;
    for (int j = i + 1; j < n; j++)
      if (val[j] > val[best]) best = j;
    float tv = val[i]; val[i] = val[best]; val[best] = tv;
    int ti = idx[i]; idx[i] = idx[best]; idx[best] = ti;
  }
  for (int i = 0; i < k && i < n; i++) {
    vals[i] = val[i];
    inds[i] = idx[i];
  }
}

/* hy3.c:1266-1291 (routing half of the MoE block). r_override > 0 replaces
 * the RMSNorm scale (test hook: feed the reference build's own r). */
void hy3o_route_token_r(const float *x, const float *norm_w, const float *router,
                        const float *bias, int has_bias, int K, float scale, float r_override,
                        float *s_out, float *logits, float *sigm, float *score,
                        int32_t *ids, float *wpre, float *w) {
  float s[HY3O_D], lg[HY3O_E], sg[HY3O_E], sc[HY3O_E], tv[HY3O_KMAX];
  int ti[HY3O_KMAX];
  const float r = r_override > 0.0f ? r_override : rms_scale(x, HY3O_D);
  for (int i = 0; i < HY3O_D; i++) s[i] = (x[i] * norm_w[i]) * r;
  for (int e = 0; e < HY3O_E; e++) {
    lg[e] = hy3o_dot8(router + (size_t)e * HY3O_D, s, HY3O_D);
    sg[e] = 1.0f / (1.0f + hy3o_sig_expf(-lg[e]));
    sc[e] = sg[e];
    if (has_bias && bias) sc[e] += bias[e];
  }
  hy3o_topk_select(tv, ti, sc, HY3O_E, K);
  float sum = 0.0f;
  for (int k = 0; k < K; k++) sum += sg[ti[k]];
  const float inv = 1.0f / (sum + 1e-20f);
  for (int k = 0; k < K; k++) {
    const float v = sg[ti[k]] * inv;
    if (ids) ids[k] = ti[k];
    if (wpre) wpre[k] = v;
    if (w) w[k] = v * scale;
  }
  if (s_out) memcpy(s_out, s, sizeof(s));
  if (logits) memcpy(logits, lg, sizeof(lg));
  if (sigm) memcpy(sigm, sg, sizeof(sg));
  if (score) memcpy(score, sc, sizeof(sc));
}

void hy3o_route_token(const float *x, const float *norm_w, const float *router,
                      const float *bias, int has_bias, int K, float scale, float *s_out,
                      float *logits, float *sigm, float *score, int32_t *ids, float *wpre,
                      float *w) {
  hy3o_route_token_r(x, norm_w, router, bias, has_bias, K, scale, 0.0f, s_out, logits, sigm,
                     score, ids, wpre, w);
}

/* ======================================================================== */
/* MoE block                                                                 */
/* ======================================================================== */

void hy3o_mul_mat_q4k(float *dst, const uint8_t *w, const float *x, int m, int n) {
  float *tmp = (float *)malloc((size_t)m * n * sizeof(float));
  hy3o_dequant_q4k(tmp, w, (int64_t)m * n);
#pragma omp parallel for schedule(static)
  for (int i = 0; i < m; i++) {
    float sum = 0.0f;
    const float *row = tmp + (size_t)i * n;
    for (int j = 0; j < n; j++) sum += row[j] * x[j];
    dst[i] = sum;
  }
  free(tmp);
}

void hy3o_mul_mat_q8_0(float *dst, const uint8_t *w, const float *x, int m, int n) {
  const int nb = n / 32;
#pragma omp parallel for schedule(static)
  for (int i = 0; i < m; i++) {
    float sum = 0.0f;
    const uint8_t *row = w + (size_t)i * nb * HY3O_Q8_BLOCK;
    for (int j = 0; j < nb; j++) {
      float d;
      memcpy(&d, row + (size_t)j * HY3O_Q8_BLOCK, 4);
      const int8_t *q = (const int8_t *)(row + (size_t)j * HY3O_Q8_BLOCK + 4);
      for (int l = 0; l < 32; l++) sum += d * (float)q[l] * x[(size_t)j * 32 + l];
    }
    dst[i] = sum;
  }
}

/* The shared expert's matrices in their own type (index E). */
static void mul_mat_shared(const hy3o_layer *L, float *dst, const uint8_t *w, const float *x,
                           int m, int n) {
  if (L->shared_type == HY3O_TYPE_Q8_0) hy3o_mul_mat_q8_0(dst, w, x, m, n);
  else hy3o_mul_mat_q4k(dst, w, x, m, n);
}

static inline float silu_f(float v) { return v / (1.0f + expf(-v)); } /* hy3.c:446-448 */

void hy3o_moe_token(const hy3o_layer *L, float *x, int K, float scale, int32_t *ids,
                    float *wpre, float *w) {
  float s[HY3O_D], sh_g[HY3O_F], sh_u[HY3O_F], g[HY3O_F], u[HY3O_F], dn[HY3O_D];
  float eo[HY3O_D], shd[HY3O_D], ww[HY3O_KMAX], wp[HY3O_KMAX];
  int32_t id[HY3O_KMAX];
  hy3o_route_token(x, L->norm_w, L->router, L->bias, L->bias != NULL, K, scale, s, NULL,
                   NULL, NULL, id, wp, ww);
  /* shared expert (hy3.c:1293-1300) */
  mul_mat_shared(L, sh_g, L->gate[HY3O_E], s, HY3O_F, HY3O_D);
  mul_mat_shared(L, sh_u, L->up[HY3O_E], s, HY3O_F, HY3O_D);
  for (int i = 0; i < HY3O_F; i++) sh_g[i] = silu_f(sh_g[i]) * sh_u[i];
  /* routed experts (hy3.c:1302-1320) */
  memset(eo, 0, sizeof(eo));
  for (int k = 0; k < K; k++) {
    const int e = id[k];
    hy3o_mul_mat_q4k(g, L->gate[e], s, HY3O_F, HY3O_D);
    hy3o_mul_mat_q4k(u, L->up[e], s, HY3O_F, HY3O_D);
    for (int i = 0; i < HY3O_F; i++) g[i] = silu_f(g[i]) * u[i];
    hy3o_mul_mat_q4k(dn, L->down[e], g, HY3O_D, HY3O_F);
    for (int i = 0; i < HY3O_D; i++) eo[i] += ww[k] * dn[i];
  }
  /* shared down + residual (hy3.c:1322-1325) */
  mul_mat_shared(L, shd, L->down[HY3O_E], sh_g, HY3O_D, HY3O_F);
  for (int i = 0; i < HY3O_D; i++) x[i] += shd[i] + eo[i];
  for (int k = 0; k < K; k++) {
    if (ids) ids[k] = id[k];
    if (wpre) wpre[k] = wp[k];
    if (w) w[k] = ww[k];
  }
}

void hy3o_moe_forward(const hy3o_layer *L, float *x, int T, int K, float scale, int32_t *ids,
                      float *wpre, float *w) {
  for (int t = 0; t < T; t++)
    hy3o_moe_token(L, x + (size_t)t * HY3O_D, K, scale, ids ? ids + (size_t)t * K : NULL,
                   wpre ? wpre + (size_t)t * K : NULL, w ? w + (size_t)t * K : NULL);
}

/* fp64 yardstick: same block bits, same routing (ids_in), fp64 arithmetic. */
static void mul_mat_q4k_f64(double *dst, const uint8_t *w, const double *x, int m, int n) {
  const int nb = n / HY3O_QK;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < m; r++) {
    double acc = 0.0;
    for (int b = 0; b < nb; b++) {
      const uint8_t *blk = w + ((size_t)r * nb + b) * HY3O_BLOCK_BYTES;
      uint16_t hd, hm;
      memcpy(&hd, blk, 2);
      memcpy(&hm, blk + 2, 2);
      const double d = hy3o_fp16_to_fp32(hd), dmin = hy3o_fp16_to_fp32(hm);
      const uint8_t *q = blk + 16;
      for (int c = 0; c < 4; c++) {
        uint8_t s1, m1, s2, m2;
        hy3o_q4k_scale_min(2 * c, blk + 4, &s1, &m1);
        hy3o_q4k_scale_min(2 * c + 1, blk + 4, &s2, &m2);
        const double *xb = x + (size_t)b * HY3O_QK + 64 * c;
        for (int l = 0; l < 32; l++) {
          acc += (d * s1 * (q[32 * c + l] & 0xF) - dmin * m1) * xb[l];
          acc += (d * s2 * (q[32 * c + l] >> 4) - dmin * m2) * xb[32 + l];
        }
      }
    }
    dst[r] = acc;
  }
}

static void mul_mat_q8_0_f64(double *dst, const uint8_t *w, const double *x, int m, int n) {
  const int nb = n / 32;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < m; r++) {
    double acc = 0.0;
    for (int b = 0; b < nb; b++) {
      const uint8_t *blk = w + ((size_t)r * nb + b) * HY3O_Q8_BLOCK;
      float d;
      memcpy(&d, blk, 4);
      const int8_t *q = (const int8_t *)(blk + 4);
      for (int l = 0; l < 32; l++) acc += (double)d * q[l] * x[(size_t)b * 32 + l];
    }
    dst[r] = acc;
  }
}

void hy3o_moe_token_f64(const hy3o_layer *L, const float *x, double *y, int K, float scale,
                        const int32_t *ids_in) {
  double s[HY3O_D], g[HY3O_F], u[HY3O_F], dn[HY3O_D], acc[HY3O_D];
  double ss = 0.0;
  for (int i = 0; i < HY3O_D; i++) ss += (double)x[i] * x[i];
  const double r = 1.0 / sqrt(ss / HY3O_D + 1e-5);
  for (int i = 0; i < HY3O_D; i++) s[i] = x[i] * r * L->norm_w[i];
  /* weights from the same ids; sigmoid in fp64 */
  double sg[HY3O_KMAX], sum = 0.0;
  for (int k = 0; k < K; k++) {
    const float *row = L->router + (size_t)ids_in[k] * HY3O_D;
    double l = 0.0;
    for (int j = 0; j < HY3O_D; j++) l += row[j] * s[j];
    sg[k] = 1.0 / (1.0 + exp(-l));
    sum += sg[k];
  }
  for (int i = 0; i < HY3O_D; i++) acc[i] = 0.0;
  for (int k = 0; k <= K; k++) {
    const int e = k < K ? ids_in[k] : HY3O_E;
    const double wk = k < K ? sg[k] / sum * (double)scale : 1.0;
    void (*mm)(double *, const uint8_t *, const double *, int, int) =
        (e == HY3O_E && L->shared_type == HY3O_TYPE_Q8_0) ? mul_mat_q8_0_f64 : mul_mat_q4k_f64;
    mm(g, L->gate[e], s, HY3O_F, HY3O_D);
    mm(u, L->up[e], s, HY3O_F, HY3O_D);
    for (int i = 0; i < HY3O_F; i++) g[i] = g[i] / (1.0 + exp(-g[i])) * u[i];
    mm(dn, L->down[e], g, HY3O_D, HY3O_F);
    for (int i = 0; i < HY3O_D; i++) acc[i] += wk * dn[i];
  }
  for (int i = 0; i < HY3O_D; i++) y[i] = x[i] + acc[i];
}

int hy3o_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void hy3o_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}
