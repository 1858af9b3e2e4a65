/*
 * hy3_gpu_moe.c -- hy3's GPU entry points for the MoE half of the model
 * (include/hy3_gpu_moe.h), over the MI355X MoE block library libhy3x.so.
 * Built by the engine against its own hy3.h (hy3_amd/engine/Makefile).
 *
 * The context bound to m->gpu_ctx holds one hy3x_layer per MoE layer. The
 * layers share one forward scratch (hy3x_layer_create_shared), as the
 * reference's single set of MoE buffers serves every layer
 * (hy3_gpu.cu:616-621): the engine runs its layers one after another.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "hy3_gpu_moe.h"
#include "hy3x_moe.h"

#define MOE_LAYER_SLOTS 82 /* hy3_weights.layers[82], hy3.h:153 */
#define MOE_MAX_GPU_LAYERS 81 /* hy3_gpu.cu:555 */
#define GGML_F32 0
#define GGML_Q8_0 8
#define GGML_Q4_K 12

typedef struct {
  int n_layers;     /* layers [0, n_layers) considered, as m->gpu_layers */
  int max_tokens;   /* tokens per forward (longer calls run in chunks) */
  hy3x_layer *layer[MOE_LAYER_SLOTS]; /* NULL for dense layers */
  float *x_stage;   /* device staging of hy3_gpu_ffn_moe_host, max_tokens rows */
} moe_ctx;

static int check_weight(const hy3_weight *w, uint32_t type, uint64_t rows, uint64_t elements,
                        int il, const char *what, int e) {
  char name[96];
  if (e >= 0)
    snprintf(name, sizeof name, "blk.%d.%s.%d", il, what, e);
  else
    snprintf(name, sizeof name, "blk.%d.%s", il, what);
  if (!w->t || !w->data) {
    fprintf(stderr, "hy3_gpu: %s is missing\n", name);
    return -1;
  }
  if (w->t->ggml_type != type || w->t->elements != elements ||
      (rows && (w->t->ndim < 1 || w->t->dim[0] != rows))) {
    fprintf(stderr,
            "hy3_gpu: %s has type %u, %llu elements, dim0 %llu; expected type %u, %llu "
            "elements, dim0 %llu\n",
            name, w->t->ggml_type, (unsigned long long)w->t->elements,
            (unsigned long long)(w->t->ndim ? w->t->dim[0] : 0), type,
            (unsigned long long)elements, (unsigned long long)rows);
    return -1;
  }
  return 0;
}

/* Every MoE tensor of one layer, before anything is uploaded
 * (hy3_layer_weights, hy3.h:120-150; shapes as the converter writes them,
 * dim[0] = rows). */
static int check_layer(const hy3_layer_weights *l, int il) {
  const uint64_t D = HY3X_D_MODEL, F = HY3X_D_FF;
  if (check_weight(&l->ffn_norm, GGML_F32, 0, D, il, "ffn_norm", -1) ||
      check_weight(&l->ffn_gate_inp, GGML_F32, HY3X_N_EXPERT, HY3X_N_EXPERT * D, il,
                   "ffn_gate_inp", -1))
    return -1;
  for (int e = 0; e < HY3X_N_EXPERT; e++)
    if (check_weight(&l->ffn_gate_exps[e], GGML_Q4_K, F, F * D, il, "ffn_gate_exps", e) ||
        check_weight(&l->ffn_up_exps[e], GGML_Q4_K, F, F * D, il, "ffn_up_exps", e) ||
        check_weight(&l->ffn_down_exps[e], GGML_Q4_K, D, D * F, il, "ffn_down_exps", e))
      return -1;
  const uint32_t st = l->ffn_gate_shexp.t ? l->ffn_gate_shexp.t->ggml_type : GGML_Q4_K;
  if (st != GGML_Q4_K && st != GGML_Q8_0) {
    fprintf(stderr, "hy3_gpu: blk.%d.ffn_gate_shexp has type %u (Q4_K or Q8_0 expected)\n", il,
            st);
    return -1;
  }
  if (check_weight(&l->ffn_gate_shexp, st, F, F * D, il, "ffn_gate_shexp", -1) ||
      check_weight(&l->ffn_up_shexp, st, F, F * D, il, "ffn_up_shexp", -1) ||
      check_weight(&l->ffn_down_shexp, st, D, D * F, il, "ffn_down_shexp", -1))
    return -1;
  return 0;
}

static int upload_layer(hy3x_layer *L, const hy3_layer_weights *l) {
  int rc = hy3x_layer_set_router(L, (const float *)l->ffn_norm.data,
                                 (const float *)l->ffn_gate_inp.data,
                                 l->has_expert_bias ? l->expert_bias : NULL);
  for (int e = 0; e < HY3X_N_EXPERT && rc == 0; e++)
    rc = hy3x_layer_set_expert_q4k(L, e, l->ffn_gate_exps[e].data, l->ffn_up_exps[e].data,
                                   l->ffn_down_exps[e].data, 0);
  if (rc == 0) {
    if (l->ffn_gate_shexp.t->ggml_type == GGML_Q8_0)
      rc = hy3x_layer_set_shared_q8_0(L, l->ffn_gate_shexp.data, l->ffn_up_shexp.data,
                                      l->ffn_down_shexp.data, 0);
    else
      rc = hy3x_layer_set_expert_q4k(L, HY3X_N_EXPERT, l->ffn_gate_shexp.data,
                                     l->ffn_up_shexp.data, l->ffn_down_shexp.data, 0);
  }
  return rc;
}

static void destroy_ctx(moe_ctx *c) {
  if (!c) return;
  for (int i = 0; i < MOE_LAYER_SLOTS; i++)
    if (c->layer[i]) hy3x_layer_destroy(c->layer[i]);
  if (c->x_stage) (void)hipFree(c->x_stage);
  free(c);
}

int hy3_gpu_init(hy3_model *m, int n_gpu_layers) {
  if (!m) return -1;
  if (m->gpu_ctx) hy3_gpu_free(m);
  if (n_gpu_layers <= 0 || n_gpu_layers > MOE_MAX_GPU_LAYERS) n_gpu_layers = MOE_MAX_GPU_LAYERS;
  if (n_gpu_layers <= HY3_N_LAYER_DENSE) {
    /* [HY3_N_LAYER_DENSE, n_gpu_layers) holds no MoE layer: nothing would run
     * on the GPU, so report failure and let the caller stay on the CPU */
    fprintf(stderr, "hy3_gpu: n_gpu_layers %d covers no MoE layer (the first is layer %d)\n",
            n_gpu_layers, HY3_N_LAYER_DENSE);
    return -1;
  }
  for (int il = HY3_N_LAYER_DENSE; il < n_gpu_layers; il++)
    if (check_layer(&m->w.layers[il], il)) return -1;
  moe_ctx *c = (moe_ctx *)calloc(1, sizeof(moe_ctx));
  if (!c) return -1;
  // tokens per forward: a whole long prompt per call where it fits (from 2048
  // tokens the library runs its 128-token tiles: one 4096-token forward takes
  // about 2.5 ms against 8 x 0.65 ms in 512-token chunks)
  const char *chunk = getenv("HY3_PREFILL_CHUNK");
  c->max_tokens = (chunk && atoi(chunk) > 0) ? atoi(chunk) : 4096;
  c->n_layers = n_gpu_layers;
  hy3x_layer *first = NULL;
  for (int il = HY3_N_LAYER_DENSE; il < n_gpu_layers; il++) {
    int rc = first ? hy3x_layer_create_shared(&c->layer[il], first)
                   : hy3x_layer_create(&c->layer[il], c->max_tokens);
    if (rc == 0) rc = upload_layer(c->layer[il], &m->w.layers[il]);
    if (rc != 0) {
      fprintf(stderr, "hy3_gpu: MoE layer %d: %s\n", il, hy3x_last_error());
      destroy_ctx(c);
      return -1;
    }
    if (!first) first = c->layer[il];
  }
  if (hipMalloc((void **)&c->x_stage, (size_t)c->max_tokens * HY3X_D_MODEL * sizeof(float)) !=
      hipSuccess) {
    c->x_stage = NULL;
    fprintf(stderr, "hy3_gpu: staging allocation failed\n");
    destroy_ctx(c);
    return -1;
  }
  m->gpu_layers = n_gpu_layers;
  m->gpu_ctx = c;
  fprintf(stderr, "hy3_gpu: MoE initialized (%d layers, %d tokens per forward)\n",
          n_gpu_layers - HY3_N_LAYER_DENSE, c->max_tokens);
  return 0;
}

void hy3_gpu_free(hy3_model *m) {
  if (!m || !m->gpu_ctx) return;
  destroy_ctx((moe_ctx *)m->gpu_ctx);
  m->gpu_ctx = NULL;
}

static hy3x_layer *bound_layer(hy3_model *m, int il, moe_ctx **ctx) {
  moe_ctx *c = m ? (moe_ctx *)m->gpu_ctx : NULL;
  if (!c) return NULL;
  *ctx = c;
  if (il < 0 || il >= c->n_layers) return NULL;
  return c->layer[il];
}

static int route_k(const hy3_model *m) {
  int k = m->n_expert_used; /* hy3.c:824-833 keeps it in [1, 8] */
  return k < 1 ? 1 : k > HY3X_K_MAX ? HY3X_K_MAX : k;
}

int hy3_gpu_ffn_moe(hy3_model *m, int il, float *x, int T, void *stream) {
  moe_ctx *c = NULL;
  hy3x_layer *L = bound_layer(m, il, &c);
  if (!L || !x || T < 1) return -1;
  const int K = route_k(m);
  for (int t0 = 0; t0 < T; t0 += c->max_tokens) {
    const int n = T - t0 < c->max_tokens ? T - t0 : c->max_tokens;
    if (hy3x_layer_forward(L, x + (size_t)t0 * HY3X_D_MODEL, n, K, HY3X_ROUTE_SCALE, stream)) {
      fprintf(stderr, "hy3_gpu: MoE layer %d: %s\n", il, hy3x_last_error());
      return -1;
    }
  }
  return 0;
}

int hy3_gpu_ffn_moe_host(hy3_model *m, int il, float *x, int T) {
  moe_ctx *c = NULL;
  hy3x_layer *L = bound_layer(m, il, &c);
  if (!L || !x || T < 1) return -1;
  const int K = route_k(m);
  for (int t0 = 0; t0 < T; t0 += c->max_tokens) {
    const int n = T - t0 < c->max_tokens ? T - t0 : c->max_tokens;
    const size_t bytes = (size_t)n * HY3X_D_MODEL * sizeof(float);
    float *xh = x + (size_t)t0 * HY3X_D_MODEL;
    if (hipMemcpy(c->x_stage, xh, bytes, hipMemcpyHostToDevice) != hipSuccess ||
        hy3x_layer_forward(L, c->x_stage, n, K, HY3X_ROUTE_SCALE, NULL) != 0 ||
        hipMemcpy(xh, c->x_stage, bytes, hipMemcpyDeviceToHost) != hipSuccess) {
      fprintf(stderr, "hy3_gpu: MoE layer %d (host buffers): %s\n", il, hy3x_last_error());
      return -1;
    }
  }
  return 0;
}
