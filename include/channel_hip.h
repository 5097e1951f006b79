/*
 * channel_hip.h -- C-ABI of the MI355X (gfx950) backend for Channel's
 * quantized inference hot path.
 *
 * Plain C: opaque handles, raw pointers and sizes, no C++ or torch types.
 * Device pointers come from chn_alloc().  Every compute entry point only
 * enqueues work on the context's single HIP stream and returns; results are
 * visible after chn_sync() or a blocking chn_download().  A context, like the
 * reference's GpuEngine, is not thread-safe: one thread drives it.
 *
 * Status codes: 0 = OK, negative = error; chn_last_error() describes the
 * last failure on a context.  Each declaration names the reference
 * interface (Sullux/channel, file:line) it replaces.
 *
 * Q4 weight layout (src/quant.zig:54-98, kept bit-for-bit): each row of K
 * weights is K/32 blocks of 5 little-endian u32 words (20 bytes); word 0 =
 * f16 scale | f16 min << 16, words 1..4 = 32 nibbles, element 8w+n in bits
 * 4n..4n+3 of word 1+w.  Every kernel dequantizes scale*(q-8) and ignores
 * the min half, as the reference's live shaders do.  K % 32 == 0 is
 * required (shaders/gemv_q4.wgsl:37).
 */
#ifndef CHANNEL_HIP_H
#define CHANNEL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes: mirror the reference's Zig error names ------------- */
#define CHN_OK 0
#define CHN_E_INVALID (-1)          /* bad argument / shape                 */
#define CHN_E_HIP (-2)              /* HIP runtime failure (VkQueueSubmitFailed, ...) */
#define CHN_E_NO_DEVICE (-3)        /* error.NoVulkanDevices (src/gpu/context.zig:29) */
#define CHN_E_OUT_OF_MEMORY (-4)    /* error.VkMemoryAllocFailed (src/gpu/buffer.zig:82) */
#define CHN_E_BATCH_TOO_LARGE (-5)  /* error.BatchTooLarge (src/gpu/batch_dispatch.zig:42) */
#define CHN_E_UNSUPPORTED (-6)      /* shape outside what the kernels support */

typedef struct chn_ctx chn_ctx;

/* ======================================================================
 * Runtime (replaces the Vulkan runtime, src/gpu/context.zig,
 * src/gpu/buffer.zig)
 * ==================================================================== */

/* Number of visible HIP devices (context.zig:25-29 device enumeration). */
int chn_device_count(int *count);

/* GpuContext.init (src/gpu/context.zig:17-107): bind device `device`,
 * create one stream.  CHN_E_NO_DEVICE when no device is visible. */
int chn_init(int device, chn_ctx **out);

/* GpuContext.deinit (src/gpu/context.zig:109). Waits for queued work. */
void chn_destroy(chn_ctx *ctx);

/* Text of the last error on `ctx` ("" if none).  With ctx == NULL: the last
 * error of a failed chn_init on this thread. */
const char *chn_last_error(const chn_ctx *ctx);

/* GpuBuffer.init (src/gpu/buffer.zig:57-97): device allocation, 256-byte
 * aligned.  Unlike the reference's host-visible UMA buffers the memory is
 * device-local; host access goes through chn_upload/chn_download. */
int chn_alloc(chn_ctx *ctx, size_t bytes, void **dptr);

/* GpuBuffer.deinit (src/gpu/buffer.zig:99-106). */
int chn_free(chn_ctx *ctx, void *dptr);

/* Writes through GpuBuffer.asSlice (src/gpu/buffer.zig:108-111), made
 * explicit: host -> device copy, ordered on the context stream, returns
 * once the source may be reused. */
int chn_upload(chn_ctx *ctx, void *dst_dev, const void *src_host, size_t bytes);

/* Reads through GpuBuffer.asSlice, made explicit: waits for queued work,
 * then device -> host copy. */
int chn_download(chn_ctx *ctx, void *dst_host, const void *src_dev, size_t bytes);

/* Device -> device copy on the stream (vkCmdCopyBuffer,
 * src/gpu/batch_dispatch.zig:146). */
int chn_copy(chn_ctx *ctx, void *dst_dev, const void *src_dev, size_t bytes);

/* Fill `count` u32 words with `value` by a kernel (graph-capture safe). */
int chn_fill_u32(chn_ctx *ctx, void *dst_dev, uint32_t value, size_t count);

/* vkWaitForFences on the context's queue (src/gpu/kernels.zig:193). */
int chn_sync(chn_ctx *ctx);

/* Stream timer: chn_timer_start records an event, chn_timer_stop records a
 * second one, waits for it and returns the elapsed milliseconds.  Has no
 * reference counterpart (the reference has no GPU timers); it times work on
 * the stream the kernels run on. */
int chn_timer_start(chn_ctx *ctx);
int chn_timer_stop(chn_ctx *ctx, float *ms);

/* ======================================================================
 * Decode matvecs (GpuEngine.record*, src/gpu/kernels.zig:89-126)
 * ==================================================================== */

/* y[M] = W[M x K] (Q4) . x[K], fp32 accumulate.
 * recordGemv / recordGemvMlp (src/gpu/kernels.zig:89-92,107-110) +
 * shaders/gemv_q4.wgsl.  x must be 16-byte aligned. */
int chn_gemv_q4(chn_ctx *ctx, const uint32_t *W, const float *x, float *y,
                uint32_t M, uint32_t K);

/* q = Wq.x, k = Wk.x, v = Wv.x in one launch over the concatenated row
 * space [q_dim | kv_dim | kv_dim].  recordFusedQkv
 * (src/gpu/kernels.zig:93-100) + shaders/fused_qkv_q4.wgsl. */
int chn_fused_qkv_q4(chn_ctx *ctx, const uint32_t *Wq, const uint32_t *Wk,
                     const uint32_t *Wv, const float *x, float *q, float *k,
                     float *v, uint32_t q_dim, uint32_t kv_dim, uint32_t K);

/* act[r] = gelu_tanh(Wg[r].x) * (Wu[r].x), r < M.  recordGateUpSwiGlu
 * (src/gpu/kernels.zig:123-126) + shaders/fused_mlp_q4.wgsl. */
int chn_fused_mlp_q4(chn_ctx *ctx, const uint32_t *Wg, const uint32_t *Wu,
                     const float *x, float *act, uint32_t M, uint32_t K);

/* ======================================================================
 * Prefill contractions (src/gpu/batch_dispatch.zig:70-81,108-130)
 * ==================================================================== */

/* Y[t][r] = sum_k X[t][k] * W[r][k] for t < n_tok, r < M: X fp32 [n_tok][K]
 * (16-byte aligned), W Q4 [M][K], Y fp32 [n_tok][M].  Operands are rounded
 * to bf16 (X) and bf16(scale*(q-8)) (W, dequantized in LDS) for MFMA with
 * fp32 accumulation; results match the fp32 contraction within 1e-2
 * relative.  The reference's push constants call n_tok "N" and the output
 * rows "M".  batch_gemm_q4 (shaders/batch_gemm_q4.wgsl; the unreferenced
 * batch_gemm_q4_tiled.wgsl computes the same contraction). */
int chn_batch_gemm_q4(chn_ctx *ctx, const uint32_t *W, const float *X, float *Y,
                      uint32_t n_tok, uint32_t M, uint32_t K);

/* Y[t][r] = gelu_tanh(G[t][r]) * U[t][r] with G, U as chn_batch_gemm_q4 over
 * Wg, Wu.  batch_fused_mlp_q4 (shaders/batch_fused_mlp_q4.wgsl,
 * src/gpu/batch_dispatch.zig:121-123). */
int chn_batch_fused_mlp_q4(chn_ctx *ctx, const uint32_t *Wg, const uint32_t *Wu,
                           const float *X, float *Y, uint32_t n_tok, uint32_t M, uint32_t K);

/* ======================================================================
 * Attention, RoPE and norms (src/gpu/kernels.zig:131-164)
 * ==================================================================== */

/* Per-head RMSNorm * weight and RoPE for q (into q_out) and k, unit RMSNorm
 * for v; k and v land in the caches at slot_idx * (num_kv_heads*head_dim).
 * step_params is DEVICE memory holding {clock, slot_idx} (the reference's
 * Step_params[0..1]), so a recorded graph can be replayed per token.
 * recordQkvRope (src/gpu/kernels.zig:159-164) + shaders/qkv_rope.wgsl. */
int chn_qkv_rope(chn_ctx *ctx, const float *q_in, const float *k_in, const float *v_in,
                 const float *q_norm_w, const float *k_norm_w, float *q_out,
                 float *k_cache, float *v_cache, const uint32_t *step_params,
                 uint32_t num_q_heads, uint32_t num_kv_heads, uint32_t head_dim,
                 uint32_t rotary_dim, int k_eq_v, float theta, float eps);

/* Softmax attention of each query head over the slot list slots[0..S),
 * S = *n_slots (DEVICE memory, clamped to max_slots <= 4096): the reference's
 * Active_slots + Step_params[2] (global) or Active_slots + 4096 +
 * Step_params[3] (sliding).  Query head h reads KV head h / gqa_ratio at
 * cache row slot * kv_dim.  scale multiplies q.k (the reference passes 1.0).
 * head_dim 256 or 512.  recordDecodeAttn (src/gpu/kernels.zig:147-152) +
 * shaders/decode_attn.wgsl. */
int chn_decode_attn(chn_ctx *ctx, const float *q, const float *k_cache, const float *v_cache,
                    const uint32_t *slots, const uint32_t *n_slots, uint32_t max_slots,
                    uint32_t num_q_heads, uint32_t head_dim, uint32_t kv_dim,
                    uint32_t gqa_ratio, float scale, float *out);

/* y = x * rsqrt(mean(x^2) + eps) * w over dim (dim % 4 == 0).
 * recordRmsNorm (src/gpu/kernels.zig:139-142) + shaders/rmsnorm.wgsl. */
int chn_rmsnorm(chn_ctx *ctx, const float *x, const float *w, float *y, uint32_t dim, float eps);

/* x = (x + r) * scalar (in place), then y = rmsnorm(x) * w.
 * recordAddRmsNorm (src/gpu/kernels.zig:131-134) + shaders/add_rmsnorm.wgsl. */
int chn_add_rmsnorm(chn_ctx *ctx, float *x, const float *r, const float *w, float *y,
                    uint32_t dim, float eps, float scalar);

/* Row-wise versions over n_tok rows of dim (prefill): shaders/batch_rmsnorm.wgsl,
 * shaders/batch_add_rmsnorm.wgsl (src/gpu/batch_dispatch.zig:64-67,117-119). */
int chn_batch_rmsnorm(chn_ctx *ctx, const float *X, const float *w, float *Y, uint32_t n_tok,
                      uint32_t dim, float eps);
int chn_batch_add_rmsnorm(chn_ctx *ctx, float *X, const float *R, const float *w, float *Y,
                          uint32_t n_tok, uint32_t dim, float eps, float scalar);

/* ======================================================================
 * Seeded synthetic inputs (no reference counterpart: benchmark and test
 * inputs generated in place on the device; the same counter-based hash is
 * restated on the host, so any block can be regenerated for checking)
 * ==================================================================== */

/* Q4 matrix [rows x K], codes uniform 0..15, f16 scales U(smin, smax). */
int chn_synth_q4(chn_ctx *ctx, uint32_t *W, uint32_t rows, uint32_t K,
                 uint64_t seed, float smin, float smax);

/* Q8_0 matrix [rows x K], int8 uniform, f32 scales U(smin, smax). */
int chn_synth_q8(chn_ctx *ctx, uint32_t *W, uint32_t rows, uint32_t K,
                 uint64_t seed, float smin, float smax);

/* n floats ~ N(0, stddev^2) (Box-Muller on one hash per element). */
int chn_synth_normal(chn_ctx *ctx, float *dst, size_t n, uint64_t seed,
                     float stddev);

#ifdef __cplusplus
}
#endif
#endif /* CHANNEL_HIP_H */
