/*
 * adapter_check.c -- drives the engine-side drop-in (include/hy3_gpu_moe.h)
 * the way hy3's engine does: a hy3_model (hy3.h:173-217) whose layer weights
 * point at host buffers laid out as the GGUF tensors hy3_model_load binds
 * (hy3.c:736-790), then hy3_gpu_init / hy3_gpu_ffn_moe / hy3_gpu_free.
 *
 *   adapter_check validate   no GPU: malformed models are refused (-1,
 *                            m->gpu_ctx left NULL), calls without a context fail
 *   adapter_check run        GPU: MoE layers 1 (Q4_K shared expert) and 2 (hy3
 *                            Q8_0 shared expert) computed through the drop-in
 *                            equal, bit for bit, the same layers run directly
 *                            through libhy3x.so (hy3x_layer_forward), on device
 *                            and host buffers, at K = 8 and 4, and with
 *                            prefill chunking
 *
 * Prints one line per check; exit status 0 when all pass.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "hy3_gpu_moe.h"
#include "hy3x_moe.h"

#define D HY3X_D_MODEL
#define F HY3X_D_FF
#define E HY3X_N_EXPERT
#define SEED 0xC0ull
/* tensor kinds of the synthetic-input specification */
#define K_X 1
#define K_NORM 2
#define K_ROUTER 3
#define K_BIAS 4
#define K_GATE 5

static int failures = 0;
#define CHECK(cond, ...)                    \
  do {                                      \
    if (cond) {                             \
      printf("ok   ");                      \
    } else {                                \
      printf("FAIL ");                      \
      failures++;                           \
    }                                       \
    printf(__VA_ARGS__);                    \
    printf("\n");                           \
    fflush(stdout);                         \
  } while (0)

#define HIP_OK(call)                                                      \
  do {                                                                    \
    if ((call) != hipSuccess) {                                           \
      printf("FAIL %s (%s:%d)\n", #call, __FILE__, __LINE__);             \
      exit(1);                                                            \
    }                                                                     \
  } while (0)
#define HY3X_OK_(call)                                                    \
  do {                                                                    \
    if ((call) != 0) {                                                    \
      printf("FAIL %s: %s\n", #call, hy3x_last_error());                  \
      exit(1);                                                            \
    }                                                                     \
  } while (0)

/* tensor infos of one layer, kept alive with the model */
typedef struct {
  hy3_tensor_info norm, router, gate[E + 1], up[E + 1], down[E + 1];
} layer_infos;

static void info(hy3_tensor_info *t, uint32_t type, uint64_t rows, uint64_t cols) {
  memset(t, 0, sizeof *t);
  t->ndim = cols ? 2 : 1;
  t->dim[0] = rows;
  t->dim[1] = cols;
  t->ggml_type = type;
  t->elements = cols ? rows * cols : rows;
}

/* Points layer il of m at the given buffers (experts[e][0..2], e = 192 shared). */
static void bind_layer(hy3_model *m, int il, layer_infos *li, const float *norm,
                       const float *router, const float *bias, uint8_t *experts[E + 1][3],
                       uint32_t shared_type) {
  hy3_layer_weights *l = &m->w.layers[il];
  info(&li->norm, 0, D, 0);
  info(&li->router, 0, E, D);
  l->ffn_norm.t = &li->norm;
  l->ffn_norm.data = (const uint8_t *)norm;
  l->ffn_gate_inp.t = &li->router;
  l->ffn_gate_inp.data = (const uint8_t *)router;
  for (int e = 0; e <= E; e++) {
    const uint32_t ty = e == E ? shared_type : 12;
    info(&li->gate[e], ty, F, D);
    info(&li->up[e], ty, F, D);
    info(&li->down[e], ty, D, F);
    hy3_weight *g = e == E ? &l->ffn_gate_shexp : &l->ffn_gate_exps[e];
    hy3_weight *u = e == E ? &l->ffn_up_shexp : &l->ffn_up_exps[e];
    hy3_weight *d = e == E ? &l->ffn_down_shexp : &l->ffn_down_exps[e];
    g->t = &li->gate[e];
    u->t = &li->up[e];
    d->t = &li->down[e];
    g->data = experts[e][0];
    u->data = experts[e][1];
    d->data = experts[e][2];
  }
  memcpy(l->expert_bias, bias, sizeof(float) * E);
  l->has_expert_bias = true;
}

static hy3_model *new_model(void) {
  hy3_model *m = (hy3_model *)calloc(1, sizeof(hy3_model));
  m->n_expert_used = HY3_N_EXPERT_USED;
  m->w.n_layer = 3;
  return m;
}

/* ------------------------------------------------------------ validate */
static int validate(void) {
  static uint8_t dummy[16];
  static float small[E * D];
  uint8_t *ex[E + 1][3];
  for (int e = 0; e <= E; e++) ex[e][0] = ex[e][1] = ex[e][2] = dummy;
  layer_infos *li = (layer_infos *)calloc(1, sizeof(layer_infos));
  hy3_model *m = new_model();

  bind_layer(m, 1, li, small, small, small, ex, 12);
  li->gate[5].ggml_type = 2; /* Q4_0 instead of Q4_K */
  CHECK(hy3_gpu_init(m, 2) == -1 && m->gpu_ctx == NULL, "expert of the wrong type refused");

  bind_layer(m, 1, li, small, small, small, ex, 12);
  li->down[17].dim[0] = F; /* transposed down matrix */
  CHECK(hy3_gpu_init(m, 2) == -1 && m->gpu_ctx == NULL, "transposed down matrix refused");

  bind_layer(m, 1, li, small, small, small, ex, 12);
  m->w.layers[1].ffn_up_shexp.data = NULL;
  CHECK(hy3_gpu_init(m, 2) == -1 && m->gpu_ctx == NULL, "missing shared expert refused");

  bind_layer(m, 1, li, small, small, small, ex, 1 /* F16 shared expert */);
  CHECK(hy3_gpu_init(m, 2) == -1 && m->gpu_ctx == NULL, "shared expert of type F16 refused");

  bind_layer(m, 1, li, small, small, small, ex, 12);
  li->router.elements = (uint64_t)E * D - 1;
  CHECK(hy3_gpu_init(m, 2) == -1 && m->gpu_ctx == NULL, "short router refused");

  bind_layer(m, 1, li, small, small, small, ex, 12);
  CHECK(hy3_gpu_init(m, 3) == -1 && m->gpu_ctx == NULL,
        "layer 2 without MoE tensors refused (n_gpu_layers 3)");

  bind_layer(m, 1, li, small, small, small, ex, 12);
  CHECK(hy3_gpu_init(m, 1) == -1 && m->gpu_ctx == NULL,
        "n_gpu_layers 1 covers only the dense layer: refused");

  float x[D];
  CHECK(hy3_gpu_ffn_moe(m, 1, x, 1, NULL) == -1, "forward without a context fails");
  CHECK(hy3_gpu_ffn_moe_host(m, 1, x, 1) == -1, "host forward without a context fails");
  hy3_gpu_free(m);
  hy3_gpu_free(NULL);
  CHECK(m->gpu_ctx == NULL, "free without a context is a no-op");
  free(m);
  free(li);
  return failures ? 1 : 0;
}

/* ------------------------------------------------------------ run */
typedef struct {
  hy3x_layer *direct; /* the same layer through libhy3x.so */
  float *norm, *router, *bias;
  uint8_t *ex[E + 1][3];
  layer_infos li;
} layer_src;

static void make_source(layer_src *s, int il, int shared_q8) {
  HY3X_OK_(hy3x_layer_create(&s->direct, 1024));
  HY3X_OK_(hy3x_synth_layer_experts(s->direct, SEED, (uint32_t)il));
  s->norm = (float *)malloc(sizeof(float) * D);
  s->router = (float *)malloc(sizeof(float) * E * D);
  s->bias = (float *)malloc(sizeof(float) * E);
  hy3x_synth_normal(s->norm, D, hy3x_synth_key(SEED, il, K_NORM, 0), 0, 0.02f, 1.0f);
  hy3x_synth_normal(s->router, (int64_t)E * D, hy3x_synth_key(SEED, il, K_ROUTER, 0), 0, 0.02f,
                    0.0f);
  hy3x_synth_uniform_sym(s->bias, E, hy3x_synth_key(SEED, il, K_BIAS, 0), 0.1f);
  HY3X_OK_(hy3x_layer_set_router(s->direct, s->norm, s->router, s->bias));
  for (int e = 0; e <= E; e++)
    for (int k = 0; k < 3; k++) {
      void *p = NULL;
      s->ex[e][k] = (uint8_t *)malloc(HY3X_Q8_0_MATRIX_BYTES);
      HY3X_OK_(hy3x_layer_expert_ptr(s->direct, e, k, &p));
      HIP_OK(hipMemcpy(s->ex[e][k], p, HY3X_Q4K_MATRIX_BYTES, hipMemcpyDeviceToHost));
    }
  if (shared_q8) { /* the shared expert's fp32 values in hy3's Q8_0 */
    float *src = (float *)malloc(sizeof(float) * F * D), *dsrc = NULL;
    uint8_t *dq = NULL;
    HIP_OK(hipMalloc((void **)&dsrc, sizeof(float) * F * D));
    HIP_OK(hipMalloc((void **)&dq, HY3X_Q8_0_MATRIX_BYTES));
    for (int k = 0; k < 3; k++) {
      hy3x_synth_normal(src, (int64_t)F * D, hy3x_synth_key(SEED, il, K_GATE + k, E), 0, 0.02f,
                        0.0f);
      HIP_OK(hipMemcpy(dsrc, src, sizeof(float) * F * D, hipMemcpyHostToDevice));
      HY3X_OK_(hy3x_synth_quantize_q8_0(dsrc, dq, (int64_t)F * D, NULL));
      HIP_OK(hipMemcpy(s->ex[E][k], dq, HY3X_Q8_0_MATRIX_BYTES, hipMemcpyDeviceToHost));
    }
    HY3X_OK_(hy3x_layer_set_shared_q8_0(s->direct, s->ex[E][0], s->ex[E][1], s->ex[E][2], 0));
    (void)hipFree(dsrc);
    (void)hipFree(dq);
    free(src);
  }
}

static float *inputs(int T, uint64_t seed) {
  float *x = (float *)malloc(sizeof(float) * (size_t)T * D);
  hy3x_synth_normal(x, (int64_t)T * D, hy3x_synth_key(seed, 0, K_X, 0), 0, 1.0f, 0.0f);
  return x;
}

/* The drop-in on device and host buffers vs the direct layer, chunked as the
 * drop-in chunks (chunk tokens per forward). */
static void compare(hy3_model *m, layer_src *s, int il, int T, int K, int chunk, uint64_t seed) {
  const size_t bytes = sizeof(float) * (size_t)T * D;
  float *x = inputs(T, seed), *a = (float *)malloc(bytes), *b = (float *)malloc(bytes);
  float *h = (float *)malloc(bytes);
  memcpy(h, x, bytes);
  float *xa = NULL, *xb = NULL;
  HIP_OK(hipMalloc((void **)&xa, bytes));
  HIP_OK(hipMalloc((void **)&xb, bytes));
  HIP_OK(hipMemcpy(xa, x, bytes, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(xb, x, bytes, hipMemcpyHostToDevice));
  m->n_expert_used = K;
  const int rc = hy3_gpu_ffn_moe(m, il, xa, T, NULL);
  for (int t0 = 0; t0 < T; t0 += chunk) {
    const int n = T - t0 < chunk ? T - t0 : chunk;
    HY3X_OK_(hy3x_layer_forward(s->direct, xb + (size_t)t0 * D, n, K, HY3X_ROUTE_SCALE, NULL));
  }
  const int rch = hy3_gpu_ffn_moe_host(m, il, h, T);
  HIP_OK(hipDeviceSynchronize());
  HIP_OK(hipMemcpy(a, xa, bytes, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(b, xb, bytes, hipMemcpyDeviceToHost));
  int moved = 0;
  for (size_t i = 0; i < (size_t)T * D; i++) moved |= a[i] != x[i];
  CHECK(rc == 0 && moved && memcmp(a, b, bytes) == 0,
        "layer %d, T=%d, K=%d: hy3_gpu_ffn_moe equals hy3x_layer_forward bit for bit", il, T, K);
  CHECK(rch == 0 && memcmp(h, b, bytes) == 0,
        "layer %d, T=%d, K=%d: hy3_gpu_ffn_moe_host equals it too", il, T, K);
  (void)hipFree(xa);
  (void)hipFree(xb);
  free(x);
  free(a);
  free(b);
  free(h);
}

static int run(void) {
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) {
    printf("FAIL no GPU\n");
    return 1;
  }
  static layer_src src[3];
  make_source(&src[1], 1, 0);
  make_source(&src[2], 2, 1);
  hy3_model *m = new_model();
  bind_layer(m, 1, &src[1].li, src[1].norm, src[1].router, src[1].bias, src[1].ex, 12);
  bind_layer(m, 2, &src[2].li, src[2].norm, src[2].router, src[2].bias, src[2].ex, 8);

  setenv("HY3_PREFILL_CHUNK", "256", 1);
  CHECK(hy3_gpu_init(m, 3) == 0 && m->gpu_ctx != NULL && m->gpu_layers == 3,
        "hy3_gpu_init(m, 3): layers 1-2 bound");
  compare(m, &src[1], 1, 1, 8, 256, 0xE0);
  compare(m, &src[1], 1, 40, 8, 256, 0xE1);
  compare(m, &src[1], 1, 300, 8, 256, 0xE2); /* two chunks: 256 + 44 */
  compare(m, &src[1], 1, 7, 4, 256, 0xE3);
  compare(m, &src[2], 2, 1, 8, 256, 0xE4);
  compare(m, &src[2], 2, 64, 8, 256, 0xE5);
  float x[D] = {0};
  CHECK(hy3_gpu_ffn_moe(m, 0, x, 1, NULL) == -1, "dense layer 0 is not a MoE layer");
  CHECK(hy3_gpu_ffn_moe(m, 3, x, 1, NULL) == -1, "layer 3 is beyond n_gpu_layers");
  hy3_gpu_free(m);
  CHECK(m->gpu_ctx == NULL, "hy3_gpu_free clears gpu_ctx");
  hy3_gpu_free(m);

  unsetenv("HY3_PREFILL_CHUNK");
  CHECK(hy3_gpu_init(m, 0) == -1 && m->gpu_ctx == NULL,
        "hy3_gpu_init(m, 0) means 81 layers: layer 3 has no MoE tensors, refused");
  CHECK(hy3_gpu_init(m, 2) == 0 && m->gpu_layers == 2, "hy3_gpu_init(m, 2) again after free");
  compare(m, &src[1], 1, 600, 8, 4096, 0xE6); /* default chunk 4096: one forward */
  hy3_gpu_free(m);
  for (int il = 1; il <= 2; il++) hy3x_layer_destroy(src[il].direct);
  free(m);
  return failures ? 1 : 0;
}

int main(int argc, char **argv) {
  const char *mode = argc > 1 ? argv[1] : "";
  int rc;
  if (!strcmp(mode, "validate"))
    rc = validate();
  else if (!strcmp(mode, "run"))
    rc = run();
  else {
    fprintf(stderr, "usage: adapter_check validate|run\n");
    return 2;
  }
  printf("adapter_check %s: %s\n", mode, rc ? "FAILED" : "OK");
  return rc;
}
