/*
 * hy3_gpu_moe.h -- the engine-side drop-in: hy3's GPU entry points for the
 * MoE half of the model, over libhy3x.so (include/hy3x_moe.h).
 *
 * This header and hy3_amd/engine/hy3_gpu_moe.c are compiled by the engine,
 * against its own hy3.h (the hy3_model / hy3_layer_weights / hy3_weight
 * types, hy3.h:107-217), into libhy3gpu_moe.so. The engine's sources need
 * edits to use it; they do NOT link unchanged:
 *  - hy3.c built with -DHY3_CUDA calls hy3_eval_gpu (hy3.c:1368-1371), the
 *    whole-token GPU engine (attention, KV cache, LM head), which this library
 *    does not export, and would hand it a gpu_ctx of another type. Build the
 *    engine WITHOUT HY3_CUDA;
 *  - without HY3_CUDA, hy3_cli.c (:278-285) and hy3_agent.c (:591-592) never
 *    call hy3_gpu_init and hy3_model_free (hy3.c:926-929) never calls
 *    hy3_gpu_free: the application calls hy3_gpu_init after hy3_model_load
 *    and hy3_gpu_free before hy3_model_free itself;
 *  - forward_layer_moe (hy3.c:1264-1266) gets one line that hands its MoE half
 *    to hy3_gpu_ffn_moe_host when m->gpu_ctx is set.
 * The exact edits are listed where this library's integration is documented.
 *
 * Reference interface replaced (yuhai-china/hy3):
 *  - hy3_gpu_init   hy3_gpu.cu:544 (prototype hy3_gpu.h:6, hy3.c:1359,
 *                   hy3_cli.c:11): the same signature and return contract
 *                   (0, or -1 with m->gpu_ctx left NULL so the CLI falls back to
 *                   the CPU, hy3_cli.c:280-281). n_gpu_layers <= 0 or > 81
 *                   means 81 (hy3_gpu.cu:555); m->gpu_layers is set. It uploads
 *                   the MoE tensors of the layers [HY3_N_LAYER_DENSE,
 *                   n_gpu_layers): ffn_norm, ffn_gate_inp, expert_bias (when
 *                   has_expert_bias), the 192 Q4_K experts (hy3_gpu.cu:589-595)
 *                   and the shared expert, Q8_0 or Q4_K (hy3_gpu.cu:581-588),
 *                   after checking every tensor's type and shape. Errors are
 *                   reported on stderr and returned; nothing calls exit().
 *  - hy3_gpu_free   hy3_gpu.cu:632: the same signature; idempotent.
 *  - gpu_ffn_moe    hy3_gpu.cu:706-738 (static in the reference, one token per
 *                   call) and the per-token MoE loop of a prefill chunk
 *                   (hy3_gpu.cu:836-837) -> hy3_gpu_ffn_moe: T tokens per call
 *                   on device memory.
 *  - the MoE half of forward_layer_moe, hy3.c:1266-1325 (the CPU engine) ->
 *    hy3_gpu_ffn_moe_host: the same block on host memory, for a CPU engine
 *    that keeps attention on the host.
 * Not covered: hy3_eval_gpu (hy3_gpu.cu:844), the rest of the GPU engine
 * (attention, KV cache, dense layer 0, embeddings, LM head); its MoE call
 * site is the place hy3_gpu_ffn_moe goes.
 */
#ifndef HY3_GPU_MOE_H
#define HY3_GPU_MOE_H

#include "hy3.h"

#ifdef __cplusplus
extern "C" {
#endif

/* hy3_gpu.cu:544. 0 on success; -1 on any error, with m->gpu_ctx NULL. An
 * n_gpu_layers of 1 .. HY3_N_LAYER_DENSE (no MoE layer in range) is an error:
 * the caller keeps the CPU path. */
int hy3_gpu_init(hy3_model *m, int n_gpu_layers);

/* hy3_gpu.cu:632. Frees everything hy3_gpu_init made; m->gpu_ctx = NULL. */
void hy3_gpu_free(hy3_model *m);

/* The MoE block of layer il for T tokens, in place: x (device memory,
 * [T x 4096] fp32) += shared(s) + sum_k w_k expert_k(s), s = rmsnorm(x) *
 * ffn_norm, with K = m->n_expert_used (clamped to [1, 8]) and the 2.826
 * route scale (hy3.c:1266-1325). Any T >= 1: tokens beyond the forward's
 * capacity (HY3_PREFILL_CHUNK at init, else 4096) run in consecutive chunks.
 * stream: a hipStream_t, or NULL. Asynchronous. 0, or -1 when there is no
 * context, il is not a bound MoE layer, or a HIP call fails. */
int hy3_gpu_ffn_moe(hy3_model *m, int il, float *x, int T, void *stream);

/* The same on host memory x[T x 4096] (copied in and out; synchronous). */
int hy3_gpu_ffn_moe_host(hy3_model *m, int il, float *x, int T);

#ifdef __cplusplus
}
#endif
#endif
