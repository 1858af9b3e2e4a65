/*
 * hy3_oracle.h -- CPU restatement of the Hy3 MoE FFN block (TEST INFRASTRUCTURE).
 *
 * This library is the checker for the HIP path, never the product: only tests,
 * the smoke entry point and the benchmark's CPU-baseline leg may load it.
 *
 * Contents
 *  - the synthetic-input specification (counter-based RNG, seeded tensors);
 *  - GGUF Q4_K block helpers (fp16 decode with the reference's exp==0 quirk,
 *    6-bit scale/min unpack, row dequantisation) and the Q4_K quantiser;
 *  - the routing contract (RMSNorm, fp32 router GEMV in a fixed reduction order,
 *    sigmoid, biased top-K by selection-with-swaps, renormalised weights);
 *  - the MoE block forward exactly as the reference CPU engine computes it
 *    (whole-matrix dequantisation then fp32 GEMV, one token at a time).
 *
 * Reference citations are to yuhai-china/hy3 (hy3.c, hy3_convert.c, hy3_gpu.cu).
 */
#ifndef HY3_ORACLE_H
#define HY3_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HY3O_D 4096          /* hidden size            (hy3.h:33) */
#define HY3O_F 1536          /* expert intermediate    (hy3.h:42) */
#define HY3O_E 192           /* routed experts         (hy3.h:39) */
#define HY3O_KMAX 8          /* n_expert_used default  (hy3.h:40) */
#define HY3O_QK 256          /* weights per Q4_K super-block */
#define HY3O_BLOCK_BYTES 144 /* sizeof(block_q4_K)     (hy3.c:405-410) */
#define HY3O_Q8_BLOCK 36     /* hy3's Q8_0: f32 d + 32 int8 (hy3.c:200, 400-403) */
#define HY3O_TYPE_Q8_0 8
#define HY3O_TYPE_Q4_K 12
#define HY3O_RMS_EPS 1e-5f   /* hy3.c:25 */
#define HY3O_ROUTE_SCALE 2.826f /* hy3.c:1289 */

/* ---- synthetic inputs -------------------------------------------------- */
enum {
  HY3O_T_X = 1,      /* layer input activations  [T x D]   ~N(0,1)      */
  HY3O_T_NORM = 2,   /* ffn_norm weight          [D]       1+N(0,0.02)  */
  HY3O_T_ROUTER = 3, /* router (ffn_gate_inp)    [E x D]   ~N(0,0.02)   */
  HY3O_T_BIAS = 4,   /* expert_bias              [E]       U(-0.1,0.1)  */
  HY3O_T_GATE = 5,   /* expert gate [F x D], expert index 192 = shared    */
  HY3O_T_UP = 6,     /* expert up   [F x D]                               */
  HY3O_T_DOWN = 7    /* expert down [D x F]                               */
};

uint64_t hy3o_splitmix64(uint64_t z);
uint64_t hy3o_tensor_key(uint64_t seed, uint32_t layer, uint32_t kind, uint32_t index);
/* Approximate standard normal from 12 uniform 16-bit draws (Irwin-Hall), scaled
 * by sigma: value = (float)(S - 786432) * (sigma / 131072). Exact integer sum,
 * one rounding; bit-identical on every IEEE platform. */
float hy3o_normal(uint64_t key, uint64_t i, float sigma);
/* Uniform in (-a, a): (float)(2u+1-2^24) * 2^-24 * a with u a 24-bit draw. */
float hy3o_uniform_sym(uint64_t key, uint64_t i, float a);
void hy3o_fill_normal(float *dst, size_t n, uint64_t key, uint64_t first, float sigma, float offset);
void hy3o_fill_uniform_sym(float *dst, size_t n, uint64_t key, float a);
/* Zipf-like skewed bias: bias_e = 0.5*(1/(rank_e+1))^0.8 over a seeded
 * Fisher-Yates permutation rank_e of the experts. */
void hy3o_zipf_bias(float *dst, int n_expert, uint64_t seed);

/* ---- fp16 / Q4_K -------------------------------------------------------- */
float hy3o_fp16_to_fp32(uint16_t h);          /* hy3.c:354-369 (exp==0 quirk kept) */
uint16_t hy3o_fp32_to_fp16_trunc(float f);    /* hy3_convert.c:511-530 */
void hy3o_q4k_scale_min(int j, const uint8_t *q, uint8_t *sc, uint8_t *m); /* hy3.c:1001-1009 */
void hy3o_dequant_q4k(float *dst, const uint8_t *src, int64_t n);          /* hy3.c:1019-1043 */
void hy3o_quantize_q4k(const float *x, uint8_t *dst, int64_t n);           /* hy3_convert.c:605-651 */
/* Generate an [rows x cols] matrix from the spec and quantise it (OpenMP). */
void hy3o_gen_q4k_matrix(uint8_t *dst, int rows, int cols, uint64_t key, float sigma);
/* hy3's Q8_0 (36-byte blocks). The quantiser follows hy3_convert.c:1192-1221
 * as its Makefile build computes it (amax/127 becomes a multiply by the fp32
 * reciprocal under -ffast-math); d*q is the block's dequantisation
 * (hy3.c:1114-1116). */
void hy3o_quantize_q8_0(const float *x, uint8_t *dst, int64_t n);
void hy3o_dequant_q8_0(float *dst, const uint8_t *src, int64_t n);
void hy3o_gen_q8_0_matrix(uint8_t *dst, int rows, int cols, uint64_t key, float sigma);

/* ---- routing contract --------------------------------------------------- */
/* Fixed-order fp32 dot product (n a multiple of 8): eight fmaf chains over
 * j = 8i+v, then ((a1+a5)+(a3+a7)) + ((a0+a4)+(a2+a6)). */
float hy3o_dot8(const float *a, const float *b, int n);
float hy3o_sig_expf(float x);                 /* exp for the router sigmoid */
/* Sum of squares of 4096 values in the GPU block's fixed order. */
float hy3o_sumsq_block(const float *x);                 /* exp for the router sigmoid */
void hy3o_rms_norm(float *out, const float *x, const float *w, int n);
/* Full routing for one token: s (normalised input) is written to s_out if
 * non-NULL; logits/sigmoid/score (E each) if non-NULL; ids[K], wpre[K] (before
 * the x2.826 scale) and w[K] always. */
void hy3o_route_token(const float *x, const float *norm_w, const float *router,
                      const float *bias, int has_bias, int K, float scale,
                      float *s_out, float *logits, float *sigm, float *score,
                      int32_t *ids, float *wpre, float *w);
void hy3o_route_token_r(const float *x, const float *norm_w, const float *router,
                        const float *bias, int has_bias, int K, float scale, float r_override,
                        float *s_out, float *logits, float *sigm, float *score,
                        int32_t *ids, float *wpre, float *w);
/* Selection sort with swaps, strict '>' (hy3.c:654-666). */
void hy3o_topk_select(float *vals, int *inds, const float *scores, int n, int k);

/* ---- MoE block forward (reference semantics) ---------------------------- */
typedef struct {
  const float *norm_w;             /* [D] */
  const float *router;             /* [E x D] */
  const float *bias;               /* [E] or NULL */
  const uint8_t *gate[HY3O_E + 1]; /* Q4_K [F x D]; index E = shared expert */
  const uint8_t *up[HY3O_E + 1];   /* Q4_K [F x D] */
  const uint8_t *down[HY3O_E + 1]; /* Q4_K [D x F] */
  int shared_type;                 /* index E: HY3O_TYPE_Q4_K (or 0) or HY3O_TYPE_Q8_0 */
} hy3o_layer;

/* Q4_K matrix-vector product as the reference computes it: dequantise the whole
 * [m x n] matrix to fp32, then per-row fp32 sums (hy3.c:1122-1135). */
void hy3o_mul_mat_q4k(float *dst, const uint8_t *w, const float *x, int m, int n);
/* Q8_0 matrix-vector product (hy3.c:1098-1120): per row, one fp32 sum of
 * d * q * x over the blocks in order. */
void hy3o_mul_mat_q8_0(float *dst, const uint8_t *w, const float *x, int m, int n);
/* One token through the MoE block: x[D] is updated in place (residual).
 * ids/wpre/w (K each) receive the routing when non-NULL. hy3.c:1266-1325. */
void hy3o_moe_token(const hy3o_layer *L, float *x, int K, float scale,
                    int32_t *ids, float *wpre, float *w);
/* T tokens, one at a time (the reference engine has no batched MoE). */
void hy3o_moe_forward(const hy3o_layer *L, float *x, int T, int K, float scale,
                      int32_t *ids, float *wpre, float *w);
/* Same block with fp64 accumulation everywhere (tolerance yardstick). */
void hy3o_moe_token_f64(const hy3o_layer *L, const float *x, double *y, int K,
                        float scale, const int32_t *ids_in);

int hy3o_num_threads(void);
void hy3o_set_num_threads(int n);

#ifdef __cplusplus
}
#endif
#endif
