/*
 * ref_shim_hy3.c -- drives the reference CPU MoE block (TEST INFRASTRUCTURE).
 *
 * Compiles yuhai-china/hy3's own hy3.c from /root/reference (never copied)
 * with its Makefile flags and exports:
 *  - hy3ref_fp16_to_fp32, hy3ref_dequant_q4k, hy3ref_topk_select,
 *    hy3ref_mul_mat: thin wrappers over the static helpers
 *    (hy3.c:354-369, 1019-1043, 654-666, 1073-1155);
 *  - hy3ref_moe_forward: runs the reference's forward_layer_moe (hy3.c:1219)
 *    once per token on a one-layer in-memory hy3_model whose attention half
 *    contributes exactly +0 (its q/k/v/o projections carry an unsupported
 *    ggml type, for which mul_mat_f32 writes zeros, hy3.c:1149-1152). The MoE
 *    half (hy3.c:1266-1325) is the reference's code, unmodified. After each
 *    token the router scores sigmoid+bias (scratch2[0..191], written at
 *    hy3.c:1272-1277 and not overwritten later) are copied out;
 *  - hy3ref_model_load / hy3ref_model_moe / hy3ref_model_free: the engine's
 *    own GGUF loader (hy3.c:805) and forward_layer_moe on the model it loads,
 *    so the GPU drop-in can be initialised from the very hy3_model the
 *    engine would hand it.
 */
#include "hy3.c"

#include <limits.h>

float hy3ref_fp16_to_fp32(uint16_t h) { return fp16_to_fp32(h); }
void hy3ref_dequant_q4k(float *dst, const uint8_t *src, int n) { dequantize_row_q4_K(dst, src, n); }
void hy3ref_topk_select(float *vals, int *inds, const float *scores, int n, int k) {
  topk_select(vals, inds, scores, n, k);
}
void hy3ref_mul_mat(float *dst, const uint8_t *w, uint32_t type, const float *x, int m, int n) {
  mul_mat_f32(dst, w, type, x, m, n);
}
void hy3ref_set_threads(int n) { omp_set_num_threads(n); }

/* The RMSNorm scale r = 1/sqrt(mean(x^2) + eps) as the reference build
 * computes it (hy3.c:435-439: an rsqrt estimate plus one Newton step under
 * -ffast-math, so the last bits depend on the host CPU). */
float hy3ref_rms_r(const float *x, int n) { return rms_norm_val(x, n, HY3_RMS_EPS); }

/* hy3.c:1266-1277 through the reference's own static helpers: s = rms_norm,
 * logits = mul_mat_f32 (F32 router), scores = sigmoid (+ bias). Used to check
 * that hy3ref_rms_r sees the same arithmetic as forward_layer_moe. */
/* The sigmoid loop of forward_layer_moe compiles to scalar expf calls and an
 * exact division; keep this copy scalar too (a plain loop would be vectorised
 * with vector expf and reciprocal estimates). */
__attribute__((optimize("no-tree-vectorize"))) static void shim_sigmoid(
    const float *logits, const float *bias, int has_bias, float *scores) {
  for (int i = 0; i < HY3_N_EXPERT; i++) {
    float sg = 1.0f / (1.0f + expf(-logits[i]));
    scores[i] = has_bias ? sg + bias[i] : sg;
  }
}

void hy3ref_router_scores(const float *x, const float *norm_w, const float *router,
                          const float *bias, int has_bias, float *s_out, float *logits,
                          float *scores) {
  rms_norm(s_out, x, norm_w, HY3_N_EMBD, HY3_RMS_EPS);
  mul_mat_f32(logits, (const uint8_t *)router, 0, s_out, HY3_N_EXPERT, HY3_N_EMBD);
  shim_sigmoid(logits, bias, has_bias, scores);
}

static hy3_tensor_info ti_f32 = {0}, ti_q4k = {0}, ti_none = {0};

/* x: [T x 4096] updated in place. gate/up/down: 193 host pointers each (index
 * 192 = shared expert). scores_out: [T x 192] or NULL. quiet: silence the
 * attention half's "unsupported ggml_type" diagnostics. Returns 0. */
static hy3_tensor_info ti_shared = {0};

/* shared_type: the shared expert's ggml type (12 Q4_K, or 8 for hy3's Q8_0,
 * the type hy3_convert.c:684-697 forces for ffn_*_shexp). */
int hy3ref_moe_forward_t(float *x, int T, int K, const float *norm_w, const float *router,
                         const float *bias, int has_bias, const uint8_t *const *gate,
                         const uint8_t *const *up, const uint8_t *const *down,
                         float *scores_out, int quiet, uint32_t shared_type) {
  ti_f32.ggml_type = 0;
  ti_q4k.ggml_type = 12;
  ti_shared.ggml_type = shared_type;
  ti_none.ggml_type = 0x7fffffff;
  hy3_model *m = (hy3_model *)calloc(1, sizeof(hy3_model));
  static float ones[HY3_N_EMBD];
  for (int i = 0; i < HY3_N_EMBD; i++) ones[i] = 1.0f;
  m->n_expert_used = K;
  m->scratch = (float *)calloc(1 << 16, sizeof(float));
  m->scratch2 = (float *)calloc(1 << 16, sizeof(float));
  m->cache_k = (float *)calloc((size_t)4 * HY3_N_KV_HEAD * HY3_HEAD_DIM, sizeof(float));
  m->cache_v = (float *)calloc((size_t)4 * HY3_N_KV_HEAD * HY3_HEAD_DIM, sizeof(float));
  m->rope_attn_factor = 1.0f;
  m->rope_pos_stride = 1;
  m->rope_pos_jump_at = INT_MAX;
  hy3_layer_weights *l = &m->w.layers[1];
  l->attn_norm.t = &ti_f32; l->attn_norm.data = (const uint8_t *)ones;
  l->attn_q.t = &ti_none; l->attn_k.t = &ti_none; l->attn_v.t = &ti_none;
  l->attn_output.t = &ti_none;
  l->ffn_norm.t = &ti_f32; l->ffn_norm.data = (const uint8_t *)norm_w;
  l->ffn_gate_inp.t = &ti_f32; l->ffn_gate_inp.data = (const uint8_t *)router;
  for (int e = 0; e < HY3_N_EXPERT; e++) {
    l->ffn_gate_exps[e].t = &ti_q4k; l->ffn_gate_exps[e].data = gate[e];
    l->ffn_up_exps[e].t = &ti_q4k; l->ffn_up_exps[e].data = up[e];
    l->ffn_down_exps[e].t = &ti_q4k; l->ffn_down_exps[e].data = down[e];
    l->expert_bias[e] = has_bias ? bias[e] : 0.0f;
  }
  l->has_expert_bias = has_bias ? true : false;
  l->ffn_gate_shexp.t = &ti_shared; l->ffn_gate_shexp.data = gate[HY3_N_EXPERT];
  l->ffn_up_shexp.t = &ti_shared; l->ffn_up_shexp.data = up[HY3_N_EXPERT];
  l->ffn_down_shexp.t = &ti_shared; l->ffn_down_shexp.data = down[HY3_N_EXPERT];

  int saved = -1;
  if (quiet) {
    fflush(stderr);
    saved = dup(2);
    int devnull = open("/dev/null", O_WRONLY);
    if (devnull >= 0) { dup2(devnull, 2); close(devnull); }
  }
  for (int t = 0; t < T; t++) {
    m->embed = x + (size_t)t * HY3_N_EMBD;
    m->cache_len = 0;
    forward_layer_moe(m, 1, 0);
    if (scores_out) memcpy(scores_out + (size_t)t * HY3_N_EXPERT, m->scratch2, HY3_N_EXPERT * sizeof(float));
  }
  if (quiet && saved >= 0) { fflush(stderr); dup2(saved, 2); close(saved); }
  free(m->scratch); free(m->scratch2); free(m->cache_k); free(m->cache_v); free(m);
  return 0;
}

int hy3ref_moe_forward(float *x, int T, int K, const float *norm_w, const float *router,
                       const float *bias, int has_bias, const uint8_t *const *gate,
                       const uint8_t *const *up, const uint8_t *const *down,
                       float *scores_out, int quiet) {
  return hy3ref_moe_forward_t(x, T, K, norm_w, router, bias, has_bias, gate, up, down,
                              scores_out, quiet, 12);
}

/* ---- the reference's own loader (hy3.c:805-914) --------------------------
 * hy3ref_model_load maps a GGUF file with hy3_model_load, exactly as the
 * engine does, and adds the KV cache that the engine's context set-up would
 * (hy3_model_load leaves cache_k / cache_v NULL; forward_layer_moe writes one
 * position per call). k > 0 overrides n_expert_used like HY3_TOP_K_EXPERTS
 * (hy3.c:824-833). The whole-file prefault (hy3.c:856-867) is skipped: it is
 * a residency measure for zero-copy GPU mappings, not part of the numerics.
 * Returns the hy3_model (opaque to the caller) or NULL. */
void *hy3ref_model_load(const char *path, int n_threads, int k) {
  setenv("HY3_NO_PREFAULT", "1", 1);
  hy3_model *m = NULL;
  if (hy3_model_load(&m, path, n_threads) != 0 || !m) return NULL;
  if (k >= 1 && k <= HY3_N_EXPERT_USED) m->n_expert_used = k;
  m->cache_k = (float *)calloc((size_t)4 * HY3_N_KV_HEAD * HY3_HEAD_DIM, sizeof(float));
  m->cache_v = (float *)calloc((size_t)4 * HY3_N_KV_HEAD * HY3_HEAD_DIM, sizeof(float));
  return m;
}

/* Runs forward_layer_moe(m, il, 0) (hy3.c:1219) on each of T rows of x in
 * place, with an empty KV cache per row, so a file whose attention weights
 * are zero contributes exactly +0 from the attention half. scores_out: [T x
 * 192] sigmoid+bias router scores or NULL. Returns 0, -1 on a bad layer. */
int hy3ref_model_moe(void *mp, int il, float *x, int T, float *scores_out) {
  hy3_model *m = (hy3_model *)mp;
  if (!m || il < HY3_N_LAYER_DENSE || il >= HY3_N_LAYER) return -1;
  float *saved = m->embed;
  for (int t = 0; t < T; t++) {
    m->embed = x + (size_t)t * HY3_N_EMBD;
    m->cache_len = 0;
    forward_layer_moe(m, il, 0);
    if (scores_out) memcpy(scores_out + (size_t)t * HY3_N_EXPERT, m->scratch2, HY3_N_EXPERT * sizeof(float));
  }
  m->embed = saved;
  return 0;
}

int hy3ref_model_n_expert_used(void *mp) { return ((hy3_model *)mp)->n_expert_used; }

/* hy3_model_free (hy3.c:924-949); the GPU context must be released first. */
void hy3ref_model_free(void *mp) { hy3_model_free((hy3_model *)mp); }
