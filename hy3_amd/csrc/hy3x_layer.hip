// hy3x_layer.hip -- the layer object and the C ABI (include/hy3x_moe.h).
//
// Device memory of a layer:
//   wq       193 experts x [gate | up | down] Q4_K, 10,616,832 B per expert, in
//            the unchanged GGUF block layout (row r of a matrix = blocks
//            [r*C/256, (r+1)*C/256)); expert 192 is the shared expert;
//   norm_w, router, bias   fp32 as in GGUF;
//   scratch  per token: staged s (8 KB), logits, routing; per slot (T*(K+1)):
//            staged h (3 KB) and the expert output row (16 KB).
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/hy3x_moe.h"
#include "hy3x_kernels.h"
#include "hy3x_decode.h"
#include "hy3x_q8.h"

using namespace hy3x;

// Expert path of a forward: single-token fused GEMVs, MFMA grouped GEMM over
// dispatch tiles, or GEMV over dispatch tiles.
enum class Mode { DECODE, MFMA, GEMV };

// Per-forward device scratch for up to max_tokens tokens: routing (logits,
// sigmoid, scores, ids, weights), the staged activations s and h in the
// layouts their kernels read, the expert output rows and the dispatch lists.
// One allocation (or the library's static array, hy3x_layer_forward_static),
// carved by scratch_layout.
struct Scratch {
  int max_tokens = 0;
  int wt = 0;         // bitmap words per expert (max_tokens / 32, rounded up to 4)
  int max_tiles = 0;  // dispatch tiles the tile array holds
  float *logits = nullptr, *sig = nullptr, *score = nullptr, *wpre = nullptr, *w = nullptr;
  float *out = nullptr, *s32 = nullptr;
  __half *s16 = nullptr, *h16 = nullptr, *s16m = nullptr, *h16m = nullptr;
  __half *ssum = nullptr, *hsum = nullptr;  // sub-block sums (hi, lo) of s16m / h16m rows
  int32_t *ids = nullptr, *list = nullptr, *n_tiles = nullptr, *counts = nullptr;
  int4 *tiles = nullptr;
  uint32_t *bits = nullptr;  // dispatch: per-expert token bitmaps [E][wt]
  uint8_t *ranks = nullptr;  // dispatch: [E][32 wt] token t's place of expert e where t's bit is set
};

// A scratch allocation and the number of layers using it.
struct ScratchMem {
  uint8_t *mem = nullptr;
  int max_tokens = 0;
  int refs = 1;
  const hy3x_layer *owner = nullptr;  // the layer whose forward ran on it last
};
static std::mutex g_scratch_mu;

struct hy3x_layer {
  int device = 0;
  int max_tokens = 0;
  uint8_t *wq = nullptr;
  uint8_t *wsh = nullptr;      // the shared expert in Q8 (q8x128 layout), when set
  int shared_q8 = 0;           // 1: the forward uses wsh for the shared expert
  float *norm_w = nullptr, *router = nullptr, *bias = nullptr;
  int has_bias = 0, router_set = 0;
  ScratchMem *scratch_mem = nullptr;  // the scratch allocation (shared by layers made
                                      // with hy3x_layer_create_shared)
  Scratch own;                 // carved from scratch_mem
  unsigned long long *stats = nullptr;
  float *rms_r = nullptr;      // diagnostics: RMSNorm scales substituted per token
  int rms_n = 0;               // tokens rms_r covers (0: compute r)
  int last_T = 0, last_K = 0;
  struct Forward {  // launch parameters of the current / last forward
    float *x = nullptr;
    const float *xadd = nullptr;  // residual addend (hy3x_layer_forward_residual) or null
    int T = 0, K = 0, nt = 4, mt = 0;
    float scale = 1.0f;
    Mode mode = Mode::GEMV;
    bool wide = false;  // MFMA mode: the wide tile shape (mfma_wide)
    bool big = false;   // MFMA mode: 128-token tiles (mfma_big)
    const float *r_in = nullptr;  // substituted RMSNorm scales, or null
    Scratch sc;         // the scratch this forward runs on
    const hy3x_layer **owner = nullptr;  // that scratch's last-forward owner slot
  } cur;
  hipStream_t last_stream = nullptr;
  int path = 0;
  unsigned long long *trace[3] = {nullptr, nullptr, nullptr};
  // per-kernel timing (diagnostics): events recorded around every stage
  int timing = 0;
  std::vector<hipEvent_t> ev_pool;
  std::vector<int> ev_stage;  // stage of the interval that ends at event i (-1: start)
  size_t ev_used = 0;
  int n_timed = 0;
};

static int record_stage(hy3x_layer *L, hipStream_t st, int stage) {
  if (!L->timing) return 0;
  if (L->ev_used == L->ev_pool.size()) {
    hipEvent_t ev;
    if (hipEventCreate(&ev) != hipSuccess) return -1;
    L->ev_pool.push_back(ev);
    L->ev_stage.push_back(-1);
  }
  L->ev_stage[L->ev_used] = stage;
  return hipEventRecord(L->ev_pool[L->ev_used++], st) == hipSuccess ? 0 : -1;
}

static thread_local std::string g_err;

static int fail(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
static int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

// The error channel for the library's other translation units (GGUF loader).
namespace hy3x {
int set_error(int code, const char *msg) { return fail(code, "%s", msg); }
}  // namespace hy3x

#define HIP_TRY(call)                                                                  \
  do {                                                                                 \
    hipError_t e_ = (call);                                                            \
    if (e_ != hipSuccess)                                                              \
      return fail(HY3X_E_HIP, "%s failed: %s (%s:%d)", #call, hipGetErrorString(e_), \
                  __FILE__, __LINE__);                                                 \
  } while (0)

// Two timing events, destroyed on every return path.
struct EventPair {
  hipEvent_t a = nullptr, b = nullptr;
  ~EventPair() {
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
  }
  hipError_t create() {
    hipError_t e = hipEventCreate(&a);
    return e != hipSuccess ? e : hipEventCreate(&b);
  }
};

template <class P>
static int dalloc(P **p, size_t bytes) {
  if (hipMalloc((void **)p, bytes) != hipSuccess) {
    *p = nullptr;
    (void)hipGetLastError();
    return fail(HY3X_E_NOMEM, "hipMalloc(%zu) failed", bytes);
  }
  return HY3X_OK;
}

// Up to this many tokens the router runs as one wave per (expert, token);
// above it as RMSNorm + LDS-tiled GEMM + per-token top-K.
constexpr int kSmallRouterT = 8;
// Router GEMM tile classes by token count (shapes and measurements with
// ROUTER_*_TINY ... XXL): TINY up to kTinyRouterT tokens, MID up to
// kMidRouterT, LARGE up to kLargeRouterT, XL up to kXLRouterT, XXL above.
#ifndef HY3X_ROUTER_CLASS_T
#define HY3X_ROUTER_CLASS_T 64, 256, 1536, 2560
#endif
constexpr int kRouterClassT[4] = {HY3X_ROUTER_CLASS_T};
constexpr int kTinyRouterT = kRouterClassT[0];
constexpr int kMidRouterT = kRouterClassT[1];
constexpr int kLargeRouterT = kRouterClassT[2];
constexpr int kXLRouterT = kRouterClassT[3];
// From this many tokens the experts run as MFMA grouped GEMMs. Measured on MI355X the
// MFMA tiles beat the wavefront-reduction GEMV tiles at every T >= 2 (T=2: 51 vs 66 us,
// T=32: 442 vs 550 us for gate/up + down), so the GEMV tiles only run when selected
// explicitly (hy3x_layer_set_path 1); T = 1 keeps the fused decode kernels.
constexpr int kMfmaMinT = 2;
// From this many tokens the MFMA GEMMs use the wide tile shape (64 tokens, 8 waves).
// Measured on MI355X (ms per layer, narrow vs wide): 32 tokens 0.32 vs 0.37,
// 128: 0.43 vs 0.48, 256: 0.503 vs 0.517, 320: 0.556 vs 0.554, 384: 0.598 vs
// 0.585, 448: 0.642 vs 0.607, 512: 0.69 vs 0.65, 4096 (Zipf routing): 3.36 vs
// 2.62 -- with few tokens per expert the tiles are mostly empty and one
// workgroup per CU hides less latency than two.
constexpr int kMfmaWideMinT = 320;
// From this many tokens the MFMA GEMMs use 128-token tiles
// (mfma_big). Measured on MI355X (ms per layer, wide vs 128-token tiles):
// 1024 tokens 0.923 vs 0.928, 1152: 1.002 vs 0.984, 1280: 1.047 vs 1.037,
// 1536: 1.222 vs 1.179, 2048: 1.489 vs 1.417, 3072: 2.05 vs 1.97, 4096: 2.60
// vs 2.46, 4096 with Zipf routing: 2.58 vs 2.34-2.38.
constexpr int kMfmaBigMinT = 1152;

static constexpr int max_tiles_for(int T, int K, int NT) {
  const int n = T * K;
  return n / NT + std::min(E, n) + (T + NT - 1) / NT + 1;
}

// The pieces of a forward's scratch, in carving order, and their bytes for
// max_tokens tokens (slots = tokens x (K_MAX routed + 1 shared)).
enum ScratchPiece {
  SP_LOGITS, SP_SIG, SP_SCORE, SP_WPRE, SP_W, SP_IDS, SP_S16, SP_S32, SP_S16M, SP_H16M,
  SP_SSUM, SP_HSUM, SP_H16, SP_OUT, SP_LIST, SP_TILES, SP_NTILES, SP_COUNTS, SP_BITS, SP_RANKS,
  SP_COUNT
};
constexpr int bitmap_words(int max_tokens) { return ((max_tokens + 31) / 32 + 3) & ~3; }
constexpr size_t piece_bytes(int max_tokens, int piece) {
  const size_t T = (size_t)max_tokens, slots = T * (KMAX + 1);
  switch (piece) {
    case SP_LOGITS: case SP_SIG: case SP_SCORE: return T * E * sizeof(float);
    case SP_WPRE: case SP_W: return T * KMAX * sizeof(float);
    case SP_IDS: return T * KMAX * sizeof(int32_t);
    case SP_S16: case SP_S16M: return T * D * sizeof(__half);
    case SP_S32: return T * D * sizeof(float);
    case SP_H16M: case SP_H16: return slots * F * sizeof(__half);
    case SP_SSUM: return T * (D / 32) * 4 * sizeof(__half);
    case SP_HSUM: return slots * (F / 32) * 4 * sizeof(__half);
    case SP_OUT: return slots * D * sizeof(float);
    case SP_LIST: return slots * sizeof(int32_t);
    case SP_TILES: return (size_t)max_tiles_for(max_tokens, KMAX, 1) * sizeof(int4);
    case SP_NTILES: return sizeof(int32_t);
    case SP_COUNTS: return (E + 1) * sizeof(int32_t);
    case SP_BITS: return (size_t)E * bitmap_words(max_tokens) * sizeof(uint32_t);
    case SP_RANKS: return (size_t)E * bitmap_words(max_tokens) * 32;
  }
  return 0;
}
constexpr size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }
constexpr size_t scratch_bytes(int max_tokens) {
  size_t off = 0;
  for (int i = 0; i < SP_COUNT; i++) off += align256(piece_bytes(max_tokens, i));
  return off;
}

// Carves the scratch of max_tokens tokens out of base (scratch_bytes(max_tokens)
// bytes, 256-byte aligned; every piece 256-byte aligned).
static Scratch scratch_layout(int max_tokens, uint8_t *base) {
  Scratch S;
  void *p[SP_COUNT];
  size_t off = 0;
  for (int i = 0; i < SP_COUNT; i++) {
    p[i] = base + off;
    off += align256(piece_bytes(max_tokens, i));
  }
  S.logits = (float *)p[SP_LOGITS];
  S.sig = (float *)p[SP_SIG];
  S.score = (float *)p[SP_SCORE];
  S.wpre = (float *)p[SP_WPRE];
  S.w = (float *)p[SP_W];
  S.ids = (int32_t *)p[SP_IDS];
  S.s16 = (__half *)p[SP_S16];
  S.s32 = (float *)p[SP_S32];
  S.s16m = (__half *)p[SP_S16M];
  S.h16m = (__half *)p[SP_H16M];
  S.ssum = (__half *)p[SP_SSUM];
  S.hsum = (__half *)p[SP_HSUM];
  S.h16 = (__half *)p[SP_H16];
  S.out = (float *)p[SP_OUT];
  S.list = (int32_t *)p[SP_LIST];
  S.tiles = (int4 *)p[SP_TILES];
  S.n_tiles = (int32_t *)p[SP_NTILES];
  S.counts = (int32_t *)p[SP_COUNTS];
  S.bits = (uint32_t *)p[SP_BITS];
  S.ranks = (uint8_t *)p[SP_RANKS];
  S.max_tokens = max_tokens;
  S.wt = bitmap_words(max_tokens);
  S.max_tiles = max_tiles_for(max_tokens, KMAX, 1);
  return S;
}

// The no-allocation entry point's scratch: one array per GPU, sized for
// HY3X_STATIC_MAX_TOKENS tokens, held by every GPU the library runs on until
// the process ends. Host code never passes `scratch` itself to a kernel (on
// the host it names a stand-in, not device memory): static_scratch_ptr()
// looks up this device's copy once with hipGetSymbolAddress and every use
// goes through that address.
constexpr size_t kStaticScratchBytes = scratch_bytes(HY3X_STATIC_MAX_TOKENS);
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_static_mu;
static uint8_t *g_static_ptr[kMaxDevices];
static const hy3x_layer *g_static_owner[kMaxDevices];  // last layer to run on `scratch`

// This device's address of `scratch` (looked up on the device's first call).
static int static_scratch_ptr(int device, uint8_t **out) {
  if (device < 0 || device >= kMaxDevices)
    return fail(HY3X_E_ARG, "device %d outside [0,%d)", device, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_static_mu);
  if (!g_static_ptr[device]) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(HY3X_E_HIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", device,
                  hipGetErrorString(e));
    g_static_ptr[device] = (uint8_t *)ptr;
  }
  *out = g_static_ptr[device];
  return HY3X_OK;
}

extern "C" {

const char *hy3x_last_error(void) { return g_err.c_str(); }

int hy3x_set_device(int device) {
  HIP_TRY(hipSetDevice(device));
  return HY3X_OK;
}

static void release_scratch(ScratchMem *m) {
  if (!m) return;
  int left;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    left = --m->refs;
  }
  if (left == 0) {
    if (m->mem) (void)hipFree(m->mem);
    delete m;
  }
}

int hy3x_layer_destroy(hy3x_layer *L) {
  if (!L) return HY3X_OK;
  void *ptrs[] = {L->wq, L->wsh, L->norm_w, L->router, L->bias, L->stats, L->rms_r};
  for (void *p : ptrs)
    if (p) (void)hipFree(p);
  release_scratch(L->scratch_mem);
  for (hipEvent_t ev : L->ev_pool) (void)hipEventDestroy(ev);
  delete L;
  return HY3X_OK;
}

// A layer with its weights and counters; its scratch is `share`'s (one more
// user) or, with share == null, a new allocation for max_tokens tokens.
static int create_layer(hy3x_layer **out, int max_tokens, ScratchMem *share) {
  if (!out) return fail(HY3X_E_ARG, "out is NULL");
  *out = nullptr;
  if (max_tokens < 1 || max_tokens > (1 << 16))
    return fail(HY3X_E_ARG, "max_tokens %d out of range [1, 65536]", max_tokens);
  hy3x_layer *L = new hy3x_layer();
  const hipError_t gerr = hipGetDevice(&L->device);
  if (gerr != hipSuccess) {
    delete L;
    return fail(HY3X_E_HIP, "hipGetDevice failed: %s", hipGetErrorString(gerr));
  }
  L->max_tokens = max_tokens;
  if (share) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    share->refs++;
    L->scratch_mem = share;
  } else {
    L->scratch_mem = new ScratchMem();
    L->scratch_mem->max_tokens = max_tokens;
  }
  int rc = HY3X_OK;
  if ((rc = dalloc(&L->wq, (size_t)(E + 1) * EXPERT_BYTES)) ||
      (rc = dalloc(&L->norm_w, D * sizeof(float))) ||
      (rc = dalloc(&L->router, (size_t)E * D * sizeof(float))) ||
      (rc = dalloc(&L->bias, E * sizeof(float))) ||
      (!share && (rc = dalloc(&L->scratch_mem->mem, scratch_bytes(max_tokens)))) ||
      (rc = dalloc(&L->stats, 2 * sizeof(unsigned long long)))) {
    hy3x_layer_destroy(L);
    return rc;
  }
  L->own = scratch_layout(max_tokens, L->scratch_mem->mem);
  if (hipMemset(L->bias, 0, E * sizeof(float)) != hipSuccess ||
      hipMemset(L->stats, 0, 2 * sizeof(unsigned long long)) != hipSuccess) {
    hy3x_layer_destroy(L);
    return fail(HY3X_E_HIP, "hipMemset failed");
  }
  *out = L;
  return HY3X_OK;
}

int hy3x_layer_create(hy3x_layer **out, int max_tokens) {
  return create_layer(out, max_tokens, nullptr);
}

int hy3x_layer_create_shared(hy3x_layer **out, hy3x_layer *scratch_from) {
  if (!scratch_from) return fail(HY3X_E_ARG, "scratch_from is NULL");
  int dev = -1;
  HIP_TRY(hipGetDevice(&dev));
  if (dev != scratch_from->device)
    return fail(HY3X_E_ARG, "scratch_from lives on device %d, the current device is %d",
                scratch_from->device, dev);
  return create_layer(out, scratch_from->scratch_mem->max_tokens, scratch_from->scratch_mem);
}

int hy3x_layer_set_router(hy3x_layer *L, const float *norm_w, const float *router,
                          const float *expert_bias) {
  if (!L || !norm_w || !router) return fail(HY3X_E_ARG, "NULL argument");
  HIP_TRY(hipMemcpy(L->norm_w, norm_w, D * sizeof(float), hipMemcpyHostToDevice));
  HIP_TRY(hipMemcpy(L->router, router, (size_t)E * D * sizeof(float), hipMemcpyHostToDevice));
  if (expert_bias) HIP_TRY(hipMemcpy(L->bias, expert_bias, E * sizeof(float), hipMemcpyHostToDevice));
  L->has_bias = expert_bias != nullptr;
  L->router_set = 1;
  return HY3X_OK;
}

int hy3x_layer_expert_ptr(hy3x_layer *L, int expert, int matrix, void **ptr) {
  if (!L || !ptr) return fail(HY3X_E_ARG, "NULL argument");
  if (expert < 0 || expert > E || matrix < 0 || matrix > 2)
    return fail(HY3X_E_ARG, "expert %d / matrix %d out of range", expert, matrix);
  *ptr = L->wq + (size_t)expert * EXPERT_BYTES + (size_t)matrix * MAT_BYTES;
  return HY3X_OK;
}

int hy3x_layer_set_expert_q4k(hy3x_layer *L, int expert, const void *gate, const void *up,
                              const void *down, int src_on_device) {
  if (!L || !gate || !up || !down) return fail(HY3X_E_ARG, "NULL argument");
  if (expert < 0 || expert > E) return fail(HY3X_E_ARG, "expert %d out of range [0,192]", expert);
  const hipMemcpyKind kind = src_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice;
  uint8_t *dst = L->wq + (size_t)expert * EXPERT_BYTES;
  HIP_TRY(hipMemcpy(dst, gate, MAT_BYTES, kind));
  HIP_TRY(hipMemcpy(dst + MAT_BYTES, up, MAT_BYTES, kind));
  HIP_TRY(hipMemcpy(dst + 2 * MAT_BYTES, down, MAT_BYTES, kind));
  if (expert == E) L->shared_q8 = 0;  // the shared expert is this Q4_K one again
  return HY3X_OK;
}

static int ensure_wsh(hy3x_layer *L) {
  if (L->wsh) return HY3X_OK;
  if (hipMalloc(&L->wsh, Q8_EXPERT_BYTES) != hipSuccess)
    return fail(HY3X_E_NOMEM, "hipMalloc of %lld bytes (Q8 shared expert) failed",
                (long long)Q8_EXPERT_BYTES);
  return HY3X_OK;
}

// hy3 Q8_0 matrix (device, 36-byte blocks) -> matrix m of wsh (q8x128).
static int repack_q8(hy3x_layer *L, const uint8_t *src_dev, int m) {
  const int64_t n_super = (int64_t)F * D / Q8K;
  k_repack_q8x128<<<(unsigned)((n_super + 255) / 256), 256>>>(src_dev, L->wsh + m * Q8_MAT_BYTES,
                                                              n_super);
  HIP_TRY(hipGetLastError());
  return HY3X_OK;
}

int hy3x_layer_set_shared_q8_0(hy3x_layer *L, const void *gate, const void *up, const void *down,
                               int src_on_device) {
  if (!L || !gate || !up || !down) return fail(HY3X_E_ARG, "NULL argument");
  int rc = ensure_wsh(L);
  if (rc) return rc;
  const void *src[3] = {gate, up, down};
  uint8_t *stage = nullptr;
  if (!src_on_device && hipMalloc(&stage, HY3X_Q8_0_MATRIX_BYTES) != hipSuccess)
    return fail(HY3X_E_NOMEM, "hipMalloc of the Q8_0 staging buffer failed");
  for (int m = 0; m < 3 && rc == HY3X_OK; m++) {
    const uint8_t *s = (const uint8_t *)src[m];
    if (stage) {
      if (hipMemcpy(stage, s, HY3X_Q8_0_MATRIX_BYTES, hipMemcpyHostToDevice) != hipSuccess) {
        rc = fail(HY3X_E_HIP, "hipMemcpy of the Q8_0 shared expert failed");
        break;
      }
      s = stage;
    }
    rc = repack_q8(L, s, m);
  }
  if (rc == HY3X_OK && hipDeviceSynchronize() != hipSuccess)
    rc = fail(HY3X_E_HIP, "Q8_0 repack failed");
  if (stage) (void)hipFree(stage);
  if (rc == HY3X_OK) L->shared_q8 = 1;
  return rc;
}

int hy3x_layer_set_rms_scale(hy3x_layer *L, const float *r, int n) {
  if (!L || n < 0 || n > L->max_tokens || (n && !r))
    return fail(HY3X_E_ARG, "bad RMSNorm scale override");
  if (n && !L->rms_r) {
    int rc = dalloc(&L->rms_r, (size_t)L->max_tokens * sizeof(float));
    if (rc) return rc;
  }
  if (n) HIP_TRY(hipMemcpy(L->rms_r, r, (size_t)n * sizeof(float), hipMemcpyHostToDevice));
  L->rms_n = n;
  return HY3X_OK;
}

int hy3x_layer_set_path(hy3x_layer *L, int path) {
  if (!L || path < 0 || path > 5) return fail(HY3X_E_ARG, "bad path");
  L->path = path;
  return HY3X_OK;
}

int hy3x_layer_last_path(const hy3x_layer *L, int *path) {
  if (!L || !path) return fail(HY3X_E_ARG, "NULL argument");
  if (!L->last_T) return fail(HY3X_E_STATE, "no forward yet");
  const auto &c = L->cur;
  *path = c.mode == Mode::DECODE ? 0 : c.mode == Mode::GEMV ? 1 : c.big ? 5 : c.wide ? 4 : 3;
  return HY3X_OK;
}

// Kernels of one stage for the forward described by L->cur (shared by the
// forward and the kernel replay used for timing).
static void launch_stage(hy3x_layer *L, int stage, hipStream_t st) {
  const auto &c = L->cur;
  const Scratch &S = c.sc;
  const int T = c.T, K = c.K, mt = c.mt;
  float *x = c.x;
  switch (stage) {
    case HY3X_STAGE_ROUTER:
      if (c.mode == Mode::DECODE) {
        k_route_decode<<<E + DEC_SH_BLOCKS, 256, 0, st>>>(
            x, c.xadd, L->norm_w, L->router, L->bias, L->has_bias, K, S.logits, S.sig, S.score,
            S.s16, S.s32, L->wq, L->shared_q8 ? L->wsh : nullptr, S.h16, L->trace[0], c.r_in);
        break;
      }
      // the routing kernels also clear (first kernel) and fill (top-K) the
      // dispatch bitmaps; for T > 8 the RMSNorm kernel stages the MFMA operand
      if (T <= kSmallRouterT) {
        k_router_logits<<<dim3(E, T), 256, 0, st>>>(x, c.xadd, L->norm_w, L->router, L->bias,
                                                    L->has_bias, S.logits, S.sig, S.score,
                                                    S.s16, S.s32, L->trace[0], T, S.bits,
                                                    S.wt, c.r_in);
      } else {
        const bool mf = c.mode == Mode::MFMA;
        k_rmsnorm<<<T, 256, 0, st>>>(x, c.xadd, L->norm_w, mf ? nullptr : S.s16, S.s32,
                                     mf ? S.s16m : nullptr, S.ssum, T, S.bits, S.wt,
                                     c.r_in);
#define HY3X_LAUNCH_ROUTER(NAME)                                                           \
  HY3X_ROUTER_GEMM(NAME)<<<dim3((T + 4 * ROUTER_MT_##NAME - 1) / (4 * ROUTER_MT_##NAME),     \
                                E / (8 * ROUTER_ME_##NAME)),                                  \
                           256, 0, st>>>(S.s32, L->router, T, S.logits)
        if (T <= kTinyRouterT)
          HY3X_LAUNCH_ROUTER(TINY);
        else if (T <= kMidRouterT)
          HY3X_LAUNCH_ROUTER(MID);
        else if (T <= kLargeRouterT)
          HY3X_LAUNCH_ROUTER(LARGE);
        else if (T <= kXLRouterT)
          HY3X_LAUNCH_ROUTER(XL);
        else
          HY3X_LAUNCH_ROUTER(XXL);
#undef HY3X_LAUNCH_ROUTER
      }
      {
        // one wave per token; up to 256 tokens one wave per block, so that
        // few tokens still spread over many CUs
        const int wpb = T <= 256 ? 1 : 4;
        k_topk<<<(T + wpb - 1) / wpb, 64 * wpb, 0, st>>>(S.logits, L->bias, L->has_bias, K,
                                                         c.scale, T, S.ids, S.wpre, S.w,
                                                         S.bits, S.wt, S.ranks);
      }
      break;
    case HY3X_STAGE_DISPATCH:
      if (c.mode == Mode::MFMA && T <= kSmallRouterT)
        k_stage_mfma<<<T, 256, 0, st>>>(S.s32, S.s16m, S.ssum);
      if (c.mode != Mode::DECODE) {
        k_dispatch_list<<<E + 1, 256, 0, st>>>(S.ranks, T, K, c.nt, S.bits, S.wt,
                                               S.list, S.tiles, S.n_tiles, mt, S.counts,
                                               L->stats);
      }
      break;
    case HY3X_STAGE_GATEUP:
      if (c.mode == Mode::DECODE)
        k_gateup_decode<<<K * DEC_GU_BLOCKS, 64 * DEC_GU_WAVES, 0, st>>>(L->wq, S.s16, S.sig, S.score, K,
                                                          c.scale, S.ids, S.wpre, S.w,
                                                          L->stats, S.h16, L->trace[1]);
      else if (c.mode == Mode::MFMA && c.big)
        mfma_big::k_moe_big<true><<<(mt + XCD_TILE_RR_MARGIN) * (F / (16 * BIG_WAVES)), 64 * BIG_WAVES, 0, st>>>(
            L->wq, L->shared_q8 ? L->wsh : nullptr, S.s16m, S.ssum, S.list, S.tiles, S.n_tiles, T, K, S.h16m, nullptr);
      else if (c.mode == Mode::MFMA && c.wide)
        mfma_wide::k_moe_mfma<true>
            <<<mt * (F / mfma_wide::ROWS_GU), 64 * mfma_wide::WAVES, 0, st>>>(
                L->wq, L->shared_q8 ? L->wsh : nullptr, S.s16m, S.ssum, S.list, S.tiles,
                S.n_tiles, T, K, S.h16m, nullptr);
      else if (c.mode == Mode::MFMA)
        mfma_narrow::k_moe_mfma<true>
            <<<mt * (F / mfma_narrow::ROWS_GU), 64 * mfma_narrow::WAVES, 0, st>>>(
                L->wq, L->shared_q8 ? L->wsh : nullptr, S.s16m, S.ssum, S.list, S.tiles,
                S.n_tiles, T, K, S.h16m, nullptr);
      else
        k_gateup_gemv<4><<<mt * (F / 16), 256, 0, st>>>(L->wq, S.s16, S.list, S.tiles,
                                                        S.n_tiles, T, K, S.h16);
      break;
    case HY3X_STAGE_DOWN:
      if (c.mode == Mode::DECODE)
        k_down_decode<<<D / DEC_DOWN_RPB, 64 * DEC_DOWN_WAVES, 0, st>>>(
            L->wq, S.h16, S.ids, S.w, K, x, c.xadd, L->shared_q8 ? L->wsh : nullptr,
            L->trace[2]);
      else if (c.mode == Mode::MFMA) {
        k_hsums<<<T * (K + 1), 64, 0, st>>>(S.h16m, S.hsum);
        const uint8_t *wsh = L->shared_q8 ? L->wsh : nullptr;
        if (c.big)
          mfma_big::k_moe_big<false><<<mt * (D / (32 * BIG_WAVES)), 64 * BIG_WAVES, 0, st>>>(
              L->wq, wsh, S.h16m, S.hsum, S.list, S.tiles, S.n_tiles, T, K, nullptr, S.out);
        else if (c.wide)
          mfma_wide::k_moe_mfma<false>
              <<<mt * (D / (2 * mfma_wide::ROWS_GU)), 64 * mfma_wide::WAVES, 0, st>>>(
                  L->wq, wsh, S.h16m, S.hsum, S.list, S.tiles, S.n_tiles, T, K, nullptr,
                  S.out);
        else
          mfma_narrow::k_moe_mfma<false>
              <<<mt * (D / (2 * mfma_narrow::ROWS_GU)), 64 * mfma_narrow::WAVES, 0, st>>>(
                  L->wq, wsh, S.h16m, S.hsum, S.list, S.tiles, S.n_tiles, T, K, nullptr,
                  S.out);
      }
      else
        k_down_gemv<4><<<mt * (D / 32), 256, 0, st>>>(L->wq, S.h16, S.list, S.tiles,
                                                      S.n_tiles, S.out);
      break;
    case HY3X_STAGE_COMBINE:
      if (c.mode != Mode::DECODE) k_combine<<<dim3(D / 1024, T), 256, 0, st>>>(x, c.xadd, S.out, S.w, T, K);
      break;
  }
}

static int forward_impl(hy3x_layer *L, const Scratch *sc, const hy3x_layer **owner, float *x,
                        const float *xadd, int T, int K, float scale, void *stream);

int hy3x_layer_forward(hy3x_layer *L, float *x, int T, int K, float scale, void *stream) {
  return forward_impl(L, L ? &L->own : nullptr, L ? &L->scratch_mem->owner : nullptr, x,
                      nullptr, T, K, scale, stream);
}

int hy3x_layer_forward_static(hy3x_layer *L, float *x, int T, int K, float scale, void *stream) {
  if (!L) return fail(HY3X_E_ARG, "NULL layer");
  if (T < 1 || T > HY3X_STATIC_MAX_TOKENS)
    return fail(HY3X_E_ARG, "T=%d outside [1,%d] (the static scratch's maximum)", T,
                HY3X_STATIC_MAX_TOKENS);
  int dev = -1;
  HIP_TRY(hipGetDevice(&dev));
  if (dev != L->device)
    return fail(HY3X_E_ARG, "the layer lives on device %d, the current device is %d", L->device,
                dev);
  uint8_t *base = nullptr;
  const int rc = static_scratch_ptr(dev, &base);
  if (rc) return rc;
  const Scratch sc = scratch_layout(HY3X_STATIC_MAX_TOKENS, base);
  return forward_impl(L, &sc, &g_static_owner[dev], x, nullptr, T, K, scale, stream);
}

int hy3x_layer_forward_residual(hy3x_layer *L, float *x, const float *attn_out, int T, int K,
                                float scale, void *stream) {
  if (!attn_out) return fail(HY3X_E_ARG, "NULL attn_out");
  if (x && T > 0) {
    // the kernels read x and attn_out through restrict pointers: no overlap at all
    const uintptr_t a0 = (uintptr_t)x, b0 = (uintptr_t)attn_out;
    const uintptr_t n = (uintptr_t)T * D * sizeof(float);
    if (a0 < b0 + n && b0 < a0 + n) return fail(HY3X_E_ARG, "attn_out overlaps x");
  }
  return forward_impl(L, L ? &L->own : nullptr, L ? &L->scratch_mem->owner : nullptr, x,
                      attn_out, T, K, scale, stream);
}

static int forward_impl(hy3x_layer *L, const Scratch *sc, const hy3x_layer **owner, float *x,
                        const float *xadd, int T, int K, float scale, void *stream) {
  if (!L || !x || !sc || !owner) return fail(HY3X_E_ARG, "NULL argument");
  if (T < 1 || T > sc->max_tokens)
    return fail(HY3X_E_ARG, "T=%d outside [1,%d]", T, sc->max_tokens);
  if (K < 1 || K > KMAX) return fail(HY3X_E_ARG, "K=%d outside [1,8]", K);
  if (!L->router_set) return fail(HY3X_E_STATE, "router not set");
  hipStream_t st = (hipStream_t)stream;
  auto &c = L->cur;
  c.x = x;
  c.xadd = xadd;
  c.T = T;
  c.K = K;
  c.scale = scale;
  c.sc = *sc;
  c.r_in = L->rms_n >= T ? L->rms_r : nullptr;
  L->rms_n = 0;  // a substituted scale serves one forward only
  if (T == 1 && L->path == 0)
    c.mode = Mode::DECODE;
  else if (L->path >= 2 || (L->path == 0 && T >= kMfmaMinT))
    c.mode = Mode::MFMA;
  else
    c.mode = Mode::GEMV;
  if (L->shared_q8 && c.mode == Mode::GEMV)
    return fail(HY3X_E_STATE, "the GEMV tile path needs a Q4_K shared expert");
  c.big = c.mode == Mode::MFMA &&
          (L->path == 5 || ((L->path == 0 || L->path == 2) && T >= kMfmaBigMinT));
  c.wide = c.mode == Mode::MFMA && !c.big &&
           (L->path == 4 || (L->path != 3 && T >= kMfmaWideMinT));
  // tokens per work tile
  c.nt = c.mode != Mode::MFMA ? 4
         : c.big              ? BIG_TOKENS
         : c.wide             ? mfma_wide::TOKENS
                              : mfma_narrow::TOKENS;
  c.mt = std::min(max_tiles_for(T, K, c.nt), sc->max_tiles);
  record_stage(L, st, -1);
  for (int stage = HY3X_STAGE_ROUTER; stage <= HY3X_STAGE_COMBINE; stage++) {
    if (c.mode == Mode::DECODE && (stage == HY3X_STAGE_DISPATCH || stage == HY3X_STAGE_COMBINE))
      continue;
    launch_stage(L, stage, st);
    record_stage(L, st, stage);
  }
  if (L->timing) L->n_timed++;
  HIP_TRY(hipGetLastError());
  L->last_T = T;
  L->last_K = K;
  L->last_stream = st;
  c.owner = owner;
  *owner = L;
  return HY3X_OK;
}

int hy3x_layers_time_stage(hy3x_layer *const *layers, int n, int stage, int reps, void *stream,
                           float *us) {
  if (!layers || n < 1 || !us || reps < 1) return fail(HY3X_E_ARG, "bad argument");
  if (stage < HY3X_STAGE_ROUTER || stage > HY3X_STAGE_COMBINE)
    return fail(HY3X_E_ARG, "stage %d outside [0,4]", stage);
  for (int i = 0; i < n; i++) {
    if (!layers[i]) return fail(HY3X_E_ARG, "layer %d is NULL", i);
    if (!layers[i]->last_T) return fail(HY3X_E_STATE, "layer %d: no forward yet", i);
  }
  hipStream_t st = (hipStream_t)stream;
  EventPair ev;
  HIP_TRY(ev.create());
  HIP_TRY(hipEventRecord(ev.a, st));
  for (int i = 0; i < reps; i++) launch_stage(layers[i % n], stage, st);
  HIP_TRY(hipEventRecord(ev.b, st));
  HIP_TRY(hipEventSynchronize(ev.b));
  float ms = 0.0f;
  HIP_TRY(hipEventElapsedTime(&ms, ev.a, ev.b));
  HIP_TRY(hipGetLastError());
  *us = ms * 1e3f / reps;
  return HY3X_OK;
}

int hy3x_layer_time_stage(hy3x_layer *L, int stage, int reps, void *stream, float *us) {
  return hy3x_layers_time_stage(&L, 1, stage, reps, stream, us);
}

int hy3x_layer_set_timing(hy3x_layer *L, int enable) {
  if (!L) return fail(HY3X_E_ARG, "NULL layer");
  L->timing = enable ? 1 : 0;
  L->ev_used = 0;
  L->n_timed = 0;
  return HY3X_OK;
}

int hy3x_layer_stage_times(hy3x_layer *L, float *ms, int n_stages, int *n_forwards) {
  if (!L || !ms || n_stages < 1) return fail(HY3X_E_ARG, "bad argument");
  for (int i = 0; i < n_stages; i++) ms[i] = 0.0f;
  if (L->ev_used) HIP_TRY(hipEventSynchronize(L->ev_pool[L->ev_used - 1]));
  for (size_t i = 1; i < L->ev_used; i++) {
    const int stg = L->ev_stage[i];
    if (stg < 0 || stg >= n_stages) continue;
    float t = 0.0f;
    HIP_TRY(hipEventElapsedTime(&t, L->ev_pool[i - 1], L->ev_pool[i]));
    ms[stg] += t;
  }
  if (n_forwards) *n_forwards = L->n_timed;
  L->ev_used = 0;
  L->n_timed = 0;
  return HY3X_OK;
}

int hy3x_layer_stats(hy3x_layer *L, uint64_t *forwards, uint64_t *experts_touched, int reset) {
  if (!L) return fail(HY3X_E_ARG, "NULL layer");
  unsigned long long h[2];
  HIP_TRY(hipDeviceSynchronize());
  HIP_TRY(hipMemcpy(h, L->stats, sizeof(h), hipMemcpyDeviceToHost));
  if (forwards) *forwards = h[0];
  if (experts_touched) *experts_touched = h[1];
  if (reset) HIP_TRY(hipMemset(L->stats, 0, sizeof(h)));
  return HY3X_OK;
}

int hy3x_layer_set_trace(hy3x_layer *L, int stage, void *buf) {
  if (!L || stage < 0 || stage > 2) return fail(HY3X_E_ARG, "bad argument");
  L->trace[stage] = (unsigned long long *)buf;
  return HY3X_OK;
}

int hy3x_layer_last_shape(const hy3x_layer *L, int *T, int *K) {
  if (!L || !T || !K) return fail(HY3X_E_ARG, "NULL argument");
  if (!L->last_T) return fail(HY3X_E_STATE, "no forward yet");
  *T = L->last_T;
  *K = L->last_K;
  return HY3X_OK;
}

int hy3x_layer_last_routing(hy3x_layer *L, int32_t *ids, float *wpre, float *w,
                            int64_t capacity) {
  if (!L) return fail(HY3X_E_ARG, "NULL layer");
  if (!L->last_T) return fail(HY3X_E_STATE, "no forward yet");
  const int64_t n = (int64_t)L->last_T * L->last_K;
  if (capacity < n)
    return fail(HY3X_E_ARG, "routing buffers hold %lld entries, the last forward has %d x %d",
                (long long)capacity, L->last_T, L->last_K);
  if (!L->cur.owner || *L->cur.owner != L)
    return fail(HY3X_E_STATE,
                "the scratch of this layer's last forward has since run another layer's forward");
  HIP_TRY(hipStreamSynchronize(L->last_stream));
  const Scratch &S = L->cur.sc;
  if (ids) HIP_TRY(hipMemcpy(ids, S.ids, n * sizeof(int32_t), hipMemcpyDeviceToHost));
  if (wpre) HIP_TRY(hipMemcpy(wpre, S.wpre, n * sizeof(float), hipMemcpyDeviceToHost));
  if (w) HIP_TRY(hipMemcpy(w, S.w, n * sizeof(float), hipMemcpyDeviceToHost));
  return HY3X_OK;
}

int hy3x_synth_layer_experts(hy3x_layer *L, uint64_t seed, uint32_t layer_index) {
  if (!L) return fail(HY3X_E_ARG, "NULL layer");
  const int64_t nblocks = (int64_t)(E + 1) * EXPERT_BYTES / QB;
  k_synth_q4k<<<(unsigned)((nblocks + 3) / 4), 256>>>(L->wq, nblocks, seed, layer_index, nullptr);
  HIP_TRY(hipGetLastError());
  HIP_TRY(hipDeviceSynchronize());
  return HY3X_OK;
}

int hy3x_synth_shared_q8_0(hy3x_layer *L, uint64_t seed, uint32_t layer_index) {
  if (!L) return fail(HY3X_E_ARG, "NULL layer");
  int rc = ensure_wsh(L);
  if (rc) return rc;
  uint8_t *stage = nullptr;
  if (hipMalloc(&stage, HY3X_Q8_0_MATRIX_BYTES) != hipSuccess)
    return fail(HY3X_E_NOMEM, "hipMalloc of the Q8_0 staging buffer failed");
  const int64_t nblocks = (int64_t)F * D / 32;
  for (int m = 0; m < 3 && rc == HY3X_OK; m++) {  // kinds gate 5, up 6, down 7; expert 192
    k_synth_q8_0<<<(unsigned)((nblocks + 255) / 256), 256>>>(
        stage, nblocks, hy3x_synth_key(seed, layer_index, 5u + m, (uint32_t)E), nullptr);
    if (hipGetLastError() != hipSuccess) rc = fail(HY3X_E_HIP, "k_synth_q8_0 launch failed");
    else rc = repack_q8(L, stage, m);
  }
  if (rc == HY3X_OK && hipDeviceSynchronize() != hipSuccess)
    rc = fail(HY3X_E_HIP, "Q8_0 synthesis failed");
  (void)hipFree(stage);
  if (rc == HY3X_OK) L->shared_q8 = 1;
  return rc;
}

int hy3x_synth_quantize_q8_0(const float *src, void *dst, int64_t n, void *stream) {
  if (!src || !dst || n <= 0 || n % 32) return fail(HY3X_E_ARG, "bad quantize arguments");
  const int64_t nblocks = n / 32;
  k_synth_q8_0<<<(unsigned)((nblocks + 255) / 256), 256, 0, (hipStream_t)stream>>>(
      (uint8_t *)dst, nblocks, 0, src);
  HIP_TRY(hipGetLastError());
  return HY3X_OK;
}

int hy3x_synth_quantize_q4k(const float *src, void *dst, int64_t n, void *stream) {
  if (!src || !dst || n <= 0 || n % QK) return fail(HY3X_E_ARG, "bad quantize arguments");
  const int64_t nblocks = n / QK;
  k_synth_q4k<<<(unsigned)((nblocks + 3) / 4), 256, 0, (hipStream_t)stream>>>(
      (uint8_t *)dst, nblocks, 0, 0, src);
  HIP_TRY(hipGetLastError());
  return HY3X_OK;
}

int hy3x_diag_read_rate(const void *pool, int64_t pool_bytes, int64_t bytes, int reps,
                        void *stream, float *us) {
  if (!pool || !us || bytes < 16 || bytes % 16 || pool_bytes < bytes || reps < 1)
    return fail(HY3X_E_ARG, "bad read-rate arguments");
  hipStream_t st = (hipStream_t)stream;
  struct Sink {
    uint32_t *p = nullptr;
    ~Sink() {
      if (p) (void)hipFree(p);
    }
  } sink;
  HIP_TRY(hipMalloc(&sink.p, 64));
  const int64_t slots = pool_bytes / bytes, n16 = bytes / 16;
  const unsigned grid = 2048;
  auto launch = [&](int i) {
    const uint4 *p = (const uint4 *)((const uint8_t *)pool + (i % slots) * bytes);
    k_stream_read<<<grid, 256, 0, st>>>(p, n16, sink.p);
  };
  for (int i = 0; i < 10; i++) launch(i);
  EventPair ev;
  HIP_TRY(ev.create());
  HIP_TRY(hipEventRecord(ev.a, st));
  for (int i = 0; i < reps; i++) launch(i);
  HIP_TRY(hipEventRecord(ev.b, st));
  HIP_TRY(hipEventSynchronize(ev.b));
  float ms = 0.0f;
  HIP_TRY(hipEventElapsedTime(&ms, ev.a, ev.b));
  HIP_TRY(hipGetLastError());
  *us = ms * 1e3f / reps;
  return HY3X_OK;
}

}  // extern "C"
