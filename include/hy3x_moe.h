/*
 * hy3x_moe.h -- C ABI of the MI355X (gfx950) Hy3 MoE FFN block.
 *
 * One library, libhy3x.so, built by hipcc for gfx950. Plain C types only.
 * Every call returns 0 on success or a negative HY3X_E* code; the message of
 * the last failure on the calling thread is available from hy3x_last_error().
 * Nothing in this library calls exit() (the reference aborts the process on
 * any CUDA error, hy3_gpu.cu:17-20).
 *
 * Reference interface replaced (yuhai-china/hy3):
 *  - gpu_ffn_moe()          hy3_gpu.cu:706-738  -> hy3x_layer_forward()
 *    (router GEMV + router_topk_kernel + routed gate_up/silu/down kernels +
 *    shared-expert GEMMs + moe_combine_id_kernel, one token per call), and
 *    the per-token prefill loop around it, hy3_gpu.cu:836-837, which the
 *    batched forward (T tokens per call) replaces;
 *  - the MoE part of hy3_gpu_init(), hy3_gpu.cu:580-595 (router/bias upload,
 *    Q4_K expert upload through upload_q4k_compressed hy3_gpu.cu:515, device
 *    pointer tables) -> hy3x_layer_create / hy3x_layer_set_router /
 *    hy3x_layer_set_expert_q4k;
 *  - the MoE scratch of hy3_gpu_init(), hy3_gpu.cu:616-621 -> owned by the
 *    layer object, sized by max_tokens;
 *  - the CPU MoE block forward_layer_moe(), hy3.c:1266-1325, whose semantics
 *    (RMSNorm, sigmoid + expert_bias top-K, renormalised weights x2.826,
 *    shared expert, combine, residual) this forward computes.
 */
#ifndef HY3X_MOE_H
#define HY3X_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HY3X_OK 0
#define HY3X_E_ARG (-1)     /* bad argument (NULL, range, size)            */
#define HY3X_E_HIP (-2)     /* HIP runtime error                           */
#define HY3X_E_NOMEM (-3)   /* device allocation failed                    */
#define HY3X_E_STATE (-4)   /* call out of order (e.g. weights not set)    */

#define HY3X_D_MODEL 4096   /* HY3_N_EMBD       hy3.h:33 */
#define HY3X_D_FF 1536      /* HY3_MOE_INTERMED hy3.h:42 */
#define HY3X_N_EXPERT 192   /* HY3_N_EXPERT     hy3.h:39 */
#define HY3X_K_MAX 8        /* HY3_N_EXPERT_USED hy3.h:40 */
#define HY3X_Q4K_BLOCK 144  /* sizeof(block_q4_K) hy3.c:405-410 */
/* Q4_K bytes of one [1536 x 4096] or [4096 x 1536] matrix. */
#define HY3X_Q4K_MATRIX_BYTES 3538944
/* hy3's Q8_0 (f32 d + 32 int8 = 36 bytes per 32 weights, hy3.c:200, 400-403):
 * bytes of one [1536 x 4096] or [4096 x 1536] matrix. */
#define HY3X_Q8_0_BLOCK 36
#define HY3X_Q8_0_MATRIX_BYTES 7077888
#define HY3X_ROUTE_SCALE 2.826f /* hy3.c:1289, hy3_gpu.cu:717 */

typedef struct hy3x_layer hy3x_layer;

/* Message for the last failed call on this thread ("" if none). */
const char *hy3x_last_error(void);

/* Select the HIP device for subsequent calls on this thread. */
int hy3x_set_device(int device);

/* Create one MoE layer on the current device, with scratch for up to
 * max_tokens tokens per forward. Replaces the MoE allocations of
 * hy3_gpu_init (hy3_gpu.cu:580-595, 616-621). Device memory: 193 experts x
 * 3 matrices of Q4_K (2.05 GB) + router (3 MB) + scratch (~36 KB/token). */
int hy3x_layer_create(hy3x_layer **out, int max_tokens);
int hy3x_layer_destroy(hy3x_layer *layer);

/* Another layer (own weights, router and counters) that shares the forward
 * scratch of `scratch_from` (same max_tokens, same device; the allocation is
 * freed with the last layer using it, in any destroy order). For an engine
 * that runs its MoE layers one after another on one stream, as the
 * reference's single set of MoE buffers (hy3_gpu.cu:616-621) serves all of
 * hy3_gpu_init's layers: one scratch instead of one per layer. Forwards of
 * layers sharing a scratch must not overlap. */
int hy3x_layer_create_shared(hy3x_layer **out, hy3x_layer *scratch_from);

/* Router-side tensors, host pointers, copied to the device:
 * norm_w[4096] (ffn_norm, F32), router[192 x 4096] (ffn_gate_inp, F32,
 * row-major as in GGUF), expert_bias[192] or NULL when the layer has no bias
 * (has_expert_bias == false, hy3.c:781-787). Mirrors hy3_gpu.cu:580,589. */
int hy3x_layer_set_router(hy3x_layer *layer, const float *norm_w, const float *router,
                          const float *expert_bias);

/* Q4_K expert matrices in the unchanged GGUF block layout (the bytes
 * hy3_weight.data points at for ffn_{gate,up,down}_exps[e], hy3.h:137-139):
 * gate/up [1536 x 4096], down [4096 x 1536], HY3X_Q4K_MATRIX_BYTES each.
 * expert in [0,192) is a routed expert; expert == 192 is the shared expert
 * (ffn_{gate,up,down}_shexp) in Q4_K. src_on_device != 0: the pointers are
 * device pointers. Replaces upload_q4k_compressed (hy3_gpu.cu:515,590). */
int hy3x_layer_set_expert_q4k(hy3x_layer *layer, int expert, const void *gate, const void *up,
                              const void *down, int src_on_device);

/* The shared expert in hy3's Q8_0, the type real checkpoints carry for
 * ffn_{gate,up,down}_shexp (hy3_convert.c:684-697 forces it): gate/up
 * [1536 x 4096], down [4096 x 1536], HY3X_Q8_0_MATRIX_BYTES each, in the
 * unchanged GGUF block layout (36-byte blocks). Replaces the shared-expert
 * upload of hy3_gpu_init (hy3_gpu.cu:581-588), which inflates these to F16
 * (37.7 MB per layer); the layer keeps them as Q8_0 (21.2 MB, repacked into
 * 144-byte super-blocks of 128 weights on the device) and computes
 * sum d*q*x like mul_mat_f32 case 8 (hy3.c:1098-1120). From this call on the
 * forward uses them; hy3x_layer_set_expert_q4k(layer, 192, ...) switches back
 * to a Q4_K shared expert. Allocates 21.2 MB of device memory on first use.
 * src_on_device != 0: the pointers are device pointers. */
int hy3x_layer_set_shared_q8_0(hy3x_layer *layer, const void *gate, const void *up,
                               const void *down, int src_on_device);

/* The MoE tensors of layer `layer_index` straight from a hy3 GGUF file (the
 * converter's names, hy3_convert.c:960-1035, bound as hy3.c:740-787 binds
 * them): blk.N.ffn_norm.weight (F32), blk.N.ffn_gate_inp.weight (F32
 * [192 x 4096]), blk.N.ffn_gate_exps_b.bias (F32 [192], optional: no bias
 * when absent, hy3.c:781-787), blk.N.ffn_{gate,up,down}_exps.E.{gate,up,
 * down}_proj.weight (Q4_K) for E in 0..191, and blk.N.ffn_{gate,up,
 * down}_shexp.weight (hy3 Q8_0, or Q4_K). The file is memory-mapped
 * read-only and parsed with bounds checks (GGUF v2/v3, general.alignment);
 * every tensor's type and shape is checked before anything is uploaded.
 * Replaces the MoE part of hy3_model_load's binding and of hy3_gpu_init's
 * upload (hy3.c:740-787; hy3_gpu.cu:580-595). Errors: HY3X_E_ARG with the
 * offending tensor named in hy3x_last_error(). */
int hy3x_layer_load_gguf(hy3x_layer *layer, const char *path, int layer_index);
/* The same checks without a layer or a GPU: 0 if the file holds every MoE
 * tensor of layer `layer_index` with the expected type and shape;
 * *shared_type (may be NULL) receives the shared expert's ggml type (8 or 12). */
int hy3x_gguf_check_layer(const char *path, int layer_index, int *shared_type);

/* Device address of expert e's matrix m (0 gate, 1 up, 2 down) inside the
 * layer's weight arena, for callers that fill the arena directly. */
int hy3x_layer_expert_ptr(hy3x_layer *layer, int expert, int matrix, void **ptr);

/* The MoE block for T tokens, in place on device memory:
 *   s = rmsnorm(x) * norm_w;  route (sigmoid + bias, top-K, renorm, x scale);
 *   x += shared(s) + sum_k w_k * expert_k(s)
 * x: device pointer to [T x 4096] fp32. 1 <= T <= max_tokens, 1 <= K <= 8.
 * stream: a hipStream_t (NULL = default stream). Asynchronous: returns after
 * enqueueing. Calls on one layer must not overlap (shared scratch), as with
 * the reference's ctx singleton buffers (hy3_gpu.cu:483, 616-621). */
int hy3x_layer_forward(hy3x_layer *layer, float *x, int T, int K, float scale, void *stream);

/* The largest T hy3x_layer_forward_static accepts. */
#define HY3X_STATIC_MAX_TOKENS 64

/* hy3x_layer_forward without any allocation at all, for callers that cannot
 * call hipMalloc (code under HIP graph capture, tight serving loops,
 * harnesses that forbid it). No counterpart in the reference. The forward's
 * scratch (routing, staged activations, expert outputs, dispatch lists; about
 * 15 MB) lives in one static device array per GPU instead of the layer's own
 * buffers; each GPU the library runs on holds it until the process ends.
 * 1 <= T <= HY3X_STATIC_MAX_TOKENS (HY3X_E_ARG beyond), K and scale as
 * hy3x_layer_forward, same result bit for bit. Call it with the layer's
 * device current. Every call on one GPU shares that GPU's array, whatever the
 * layer: calls that overlap on one GPU (other streams, other threads) race,
 * and hy3x_layer_last_routing of a layer refuses (HY3X_E_STATE) once another
 * layer's static call has run. Calls no hipMalloc, hipFree or allocating library routine. */
int hy3x_layer_forward_static(hy3x_layer *layer, float *x, int T, int K, float scale,
                              void *stream);

/* The residual add before the block fused into it: x += attn_out, then the
 * MoE block on the new x, i.e. hy3.c:1264-1266 (x[i] += s2[i]; rms_norm...)
 * and the GPU engine's add_rmsnorm_kernel + gpu_ffn_moe (hy3_gpu.cu:453-460,
 * 761-762), without the separate add kernel and its 16 KB-per-token round
 * trip: every kernel that reads x forms x + attn_out itself (the same fp32
 * add), and the final write is (x + attn_out) + (shared + sum_k w_k expert_k).
 * attn_out: device [T x 4096] fp32, read only, must not alias x. Otherwise
 * as hy3x_layer_forward (its result equals forward on x + attn_out bit for
 * bit). */
int hy3x_layer_forward_residual(hy3x_layer *layer, float *x, const float *attn_out, int T, int K,
                                float scale, void *stream);

/* Token and expert counts (T, K) of the last forward. */
int hy3x_layer_last_shape(const hy3x_layer *layer, int *T, int *K);

/* Routing of the last forward, copied to host buffers (synchronises on the
 * stream): ids[T x K] int32 in selection order, wpre[T x K] = sigma / sum
 * (before the scale), w[T x K] (after). Any pointer may be NULL. capacity:
 * the number of entries each non-NULL buffer holds; HY3X_E_ARG if it is
 * below T x K of the last forward (nothing is copied then). HY3X_E_STATE when
 * the scratch that forward ran on has since run another layer's forward
 * (layers made with hy3x_layer_create_shared, or hy3x_layer_forward_static
 * calls of other layers): the routing it held is gone. */
int hy3x_layer_last_routing(hy3x_layer *layer, int32_t *ids, float *wpre, float *w,
                            int64_t capacity);

/* Per-stage timing (diagnostics, no counterpart in the reference beyond its
 * HY3_TIMING wall clocks, hy3.c:1532-1563): while enabled, every forward
 * records HIP events on its stream between its kernel stages.
 * hy3x_layer_stage_times() synchronises, returns the accumulated milliseconds
 * per stage (index HY3X_STAGE_*) and the number of forwards timed, and resets
 * the accumulators. Enabling also resets. */
#define HY3X_STAGE_ROUTER 0   /* RMSNorm + router GEMV + top-K        */
#define HY3X_STAGE_DISPATCH 1 /* per-expert lists and work tiles      */
#define HY3X_STAGE_GATEUP 2   /* gate/up GEMV or GEMM + SwiGLU         */
#define HY3X_STAGE_DOWN 3     /* down GEMV or GEMM                     */
#define HY3X_STAGE_COMBINE 4  /* weighted combine + residual           */
#define HY3X_N_STAGES 8
int hy3x_layer_set_timing(hy3x_layer *layer, int enable);
int hy3x_layer_stage_times(hy3x_layer *layer, float *ms, int n_stages, int *n_forwards);

/* Diagnostics: relaunches the kernels of one stage (HY3X_STAGE_*) of the last
 * forward `reps` times back to back on `stream`, bracketed by two HIP events,
 * and returns the mean microseconds per launch in *us (synchronises). Inputs
 * are those of the last forward, so the x buffer it named must still be live;
 * the down stage of a single-token forward adds its output into x again, so x
 * is modified. No reference counterpart (measurement only). */
int hy3x_layer_time_stage(hy3x_layer *layer, int stage, int reps, void *stream, float *us);
/* The same over n layers in rotation (launch i replays layers[i % n]'s stage),
 * so that with n layers whose weights together exceed the last-level cache
 * every launch streams its weights from HBM. */
int hy3x_layers_time_stage(hy3x_layer *const *layers, int n, int stage, int reps, void *stream,
                           float *us);

/* Diagnostics: the reference point for the roofline fractions. Mean
 * microseconds per launch of a plain streaming-read kernel reading `bytes`
 * (multiple of 16) from the device buffer `pool`, successive launches taking
 * successive `bytes`-sized slots of the pool so that a pool larger than the
 * last-level cache defeats reuse; reps launches back to back between two HIP
 * events (synchronises). No reference counterpart (measurement only). */
int hy3x_diag_read_rate(const void *pool, int64_t pool_bytes, int64_t bytes, int reps,
                        void *stream, float *us);

/* Device-side counters since the last reset: forwards run and the sum over
 * forwards of the experts touched (shared expert included), i.e. the "U" of
 * the algorithmic byte count. Synchronises the device. */
int hy3x_layer_stats(hy3x_layer *layer, uint64_t *forwards, uint64_t *experts_touched,
                     int reset);

/* Diagnostics: per-block timestamps of the decode kernels (stage 0 router,
 * 1 gate/up, 2 down). buf: device memory of 8 x 64-bit words per block, or
 * NULL to stop: stage 0 has 384 blocks (192 router logits, then 192 shared
 * gate/up blocks), stage 1 K x 384, stage 2 256. Each block writes
 * REALTIME-counter (100 MHz) checkpoints. */
int hy3x_layer_set_trace(hy3x_layer *layer, int stage, void *buf);

/* Diagnostics: substitute the RMSNorm scale for ONE forward. The next forward
 * of this layer, if it has T <= n tokens, uses r[t] (host array of n floats,
 * copied) as token t's 1/sqrt(mean(x^2) + 1e-5) instead of computing it;
 * s = (x * norm_w) * r[t] as before. That forward consumes the override
 * (whatever its T): every later forward computes the scale again, so a
 * forgotten override cannot leak into production routing. n = 0 cancels a
 * pending override. No reference
 * counterpart: it lets a test feed the reference CPU build's own r (from the
 * host's rsqrt estimate and a Newton step, hy3.c:435-444 as compiled) and
 * compare the rest of the routing to it. */
int hy3x_layer_set_rms_scale(hy3x_layer *layer, const float *r, int n);

/* Execution-path override for tests: 0 = automatic (by T), 1 = force the
 * wavefront-GEMV expert path, 2 = force the MFMA grouped-GEMM path (tile
 * shape by T), 3 = MFMA with the narrow tile shape (32 tokens), 4 = MFMA with
 * the wide tile shape (64 tokens), 5 = MFMA with 128-token tiles. */
int hy3x_layer_set_path(hy3x_layer *layer, int path);

/* Which expert path the last forward ran: 0 = the fused single-token decode
 * kernels, 1 = wavefront-GEMV tiles, 3 = MFMA with the narrow tile shape,
 * 4 = MFMA with the wide one, 5 = MFMA with 128-token tiles (diagnostics and benchmarks: the kernel whose
 * roofline a benchmark reports). */
int hy3x_layer_last_path(const hy3x_layer *layer, int *path);

/* ---- synthetic inputs (test / benchmark data, not part of the MoE path) ----
 * Device-side generator + Q4_K quantiser for the seeded synthetic layers the
 * benchmark configurations describe. The quantiser reproduces hy3_convert.c's
 * quantize_row_q4_K (hy3_convert.c:605-651) as built by its Makefile. */
/* Fill every expert (0..192) of the layer from (seed, layer_index). */
int hy3x_synth_layer_experts(hy3x_layer *layer, uint64_t seed, uint32_t layer_index);
/* Quantise n fp32 values (device pointers; n multiple of 256) to Q4_K. */
int hy3x_synth_quantize_q4k(const float *src, void *dst, int64_t n, void *stream);
/* The shared expert in hy3's Q8_0 from (seed, layer_index): the same fp32
 * values as expert 192 of hy3x_synth_layer_experts, quantised by the Q8_0
 * quantiser of hy3_convert.c:1192-1221 as its Makefile build computes it,
 * then set as by hy3x_layer_set_shared_q8_0. */
int hy3x_synth_shared_q8_0(hy3x_layer *layer, uint64_t seed, uint32_t layer_index);
/* Quantise n fp32 values (device pointers; n multiple of 32) to hy3's Q8_0. */
int hy3x_synth_quantize_q8_0(const float *src, void *dst, int64_t n, void *stream);
/* Host-side generators for the small tensors (bit-identical to the spec). */
uint64_t hy3x_synth_key(uint64_t seed, uint32_t layer, uint32_t kind, uint32_t index);
void hy3x_synth_normal(float *dst, int64_t n, uint64_t key, uint64_t first, float sigma,
                       float offset);
void hy3x_synth_uniform_sym(float *dst, int64_t n, uint64_t key, float a);
void hy3x_synth_zipf_bias(float *dst, int n_expert, uint64_t seed);

#ifdef __cplusplus
}
#endif
#endif
