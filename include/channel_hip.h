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
typedef struct chn_model chn_model;

/* ======================================================================
 * Runtime (replaces the Vulkan runtime, src/gpu/context.zig,
 * src/gpu/buffer.zig)
 * ==================================================================== */

/* Number of visible HIP devices (context.zig:25-29 device enumeration). */
int chn_device_count(int *count);

/* GpuContext.init (src/gpu/context.zig:17-107): bind device `device`,
 * create one stream.  CHN_E_NO_DEVICE when no device is visible. */
int chn_init(int device, chn_ctx **out);

/* GpuContext.device_name (src/gpu/context.zig:17-107; checked by the
 * reference's context test, src/gpu.zig:24-30): the bound device's name and
 * gfx target, never empty for a live context ("" for NULL). */
const char *chn_device_name(const chn_ctx *ctx);

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

/* Recordings: the reference's pre-recorded command buffers (GpuEngine.record*
 * into a VkCommandBuffer, then submitPreRecorded, src/gpu/kernels.zig:89-194;
 * recordForwardGraph, src/gpu/model_dispatch.zig:103-126).  Between
 * chn_record_begin and chn_record_end the kernel-level calls on ctx (matvecs,
 * contractions, attention, norms, logits, chn_copy, chn_fill_u32) are
 * recorded into a HIP graph instead of run; chn_submit enqueues the recording
 * on the context stream (chn_sync waits, as submitPreRecorded's fence wait
 * does) and may be called any number of times.
 *  - A recording holds the device pointers and sizes it was made with: the
 *    buffers must stay allocated while it is used, and their contents at
 *    submission are what the kernels read.
 *  - Calls that copy to or from the host, synchronize, or would grow the
 *    context workspace fail while recording (CHN_E_UNSUPPORTED for the
 *    workspace: make one unrecorded call of the same shapes first, or use
 *    chn_decode_attn_noalloc); a failed call can invalidate the recording,
 *    which chn_record_end then reports.
 *  - chn_submit refuses a recording made before the workspace was last
 *    reallocated (it would read freed memory), and one from another context.
 * chn_recording_free waits for the context stream, then releases it;
 * chn_destroy releases the recordings still live on its context (they must
 * not be used or freed afterwards). */
typedef struct chn_recording chn_recording;
int chn_record_begin(chn_ctx *ctx);
int chn_record_end(chn_ctx *ctx, chn_recording **out);
int chn_submit(chn_ctx *ctx, const chn_recording *rec);
void chn_recording_free(chn_recording *rec);

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

/* ======================================================================
 * Repacked Q4 ("Q4R"): the layout the model keeps in HBM.  Per matrix of
 * rows x K: [rows][K/32] 16-byte words of nibbles, each nibble XOR 8 (the
 * two's-complement value q - 8), then [rows][K/32] f16 scales; 18 bytes per
 * 32 weights (the reference's unused f16 min half-word is dropped).  A pure
 * bit permutation of the reference layout, so products are unchanged.  No
 * reference counterpart: these replace the same recorders as the entries
 * above (src/gpu/kernels.zig:89-126) over weights that model ingest
 * (GpuModelContext.init, src/gpu/model_gpu.zig:68) repacks once.
 * ==================================================================== */

#define CHN_Q4R_BYTES(rows, K) ((size_t)(rows) * ((K) / 32) * 18)

/* Reference-layout Q4 (device) -> Q4R (device, 16-byte aligned, CHN_Q4R_BYTES). */
int chn_q4_repack(chn_ctx *ctx, const uint32_t *W, uint32_t rows, uint32_t K, void *dst);

/* As chn_gemv_q4 / chn_fused_qkv_q4 / chn_fused_mlp_q4 over Q4R weights;
 * K % 32 == 0, K <= 16384. */
int chn_gemv_q4r(chn_ctx *ctx, const void *W, const float *x, float *y, uint32_t M, uint32_t K);
int chn_fused_qkv_q4r(chn_ctx *ctx, const void *Wq, const void *Wk, const void *Wv, const float *x,
                      float *q, float *k, float *v, uint32_t q_dim, uint32_t kv_dim, uint32_t K);
int chn_fused_mlp_q4r(chn_ctx *ctx, const void *Wg, const void *Wu, const float *x, float *act,
                      uint32_t M, uint32_t K);

/* Activation digit planes: the form in which every matvec above reads its
 * input x (K values in K/32 blocks).  Per block b of nb = K/32: an exponent
 * e with |x_i| < 2^e, X_i = rint(x_i * 2^(18 - e)) split into five signed
 * hex digits, stored as plane words [(p*4 + w)*nb + b] (p < 5 digit, w < 4
 * eight-value group, 4-bit digits XOR 8), then nb float scales 2^(e - 18).
 * Producing the planes once lets several matvecs share them; the model's
 * norm and attention kernels write them directly.  No reference
 * counterpart (the reference multiplies by f32 x in every shader). */
#define CHN_XPLANES_BYTES(K) ((size_t)((K) / 32) * 21 * 4)
int chn_xplanes(chn_ctx *ctx, const float *x, uint32_t K, uint32_t *planes);

/* chn_gemv_q4r / chn_fused_mlp_q4r reading planes of x (chn_xplanes)
 * instead of x.  With act_planes != NULL (M % 32 == 0, not aliasing planes)
 * the gate/up matvec also writes the planes of act, the down projection's
 * input, in the same pass; bit-identical to chn_xplanes(act). */
int chn_gemv_q4r_xp(chn_ctx *ctx, const void *W, const uint32_t *planes, float *y, uint32_t M, uint32_t K);
int chn_fused_mlp_q4r_xp(chn_ctx *ctx, const void *Wg, const void *Wu, const uint32_t *planes, float *act,
                         uint32_t *act_planes, uint32_t M, uint32_t K);

/* The decode step's pre-FFN block in one launch, as the model runs it:
 * r' = rmsnorm(r) * post_w (post_w != NULL; else r' = r), x_out = x_in + r',
 * normed = rmsnorm(x_out) * pre_w (written to normed_out if non-NULL),
 * act[m] = gelu_tanh(Wg[m].normed) * (Wu[m].normed) over Q4R weights, and the
 * digit planes of act (chn_xplanes layout, CHN_XPLANES_BYTES(M)) for the down
 * projection.  recordRmsNorm + recordAddRmsNorm + recordGateUpSwiGlu
 * (src/gpu/model_dispatch.zig:33-40) fused.  K <= 4096, M % 32 == 0;
 * vectors 16-byte aligned; x_out must not alias x_in. */
int chn_ffn_gate_up_q4r(chn_ctx *ctx, const void *Wg, const void *Wu, const float *x_in, const float *r,
                        const float *post_w, const float *pre_w, float *x_out, float *normed_out, float *act,
                        uint32_t *act_planes, uint32_t M, uint32_t K, float eps);

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

/* The same contractions over Q4R weights (chn_q4_repack), the ones
 * chn_prefill runs (which keeps the K-split partial sums of o and down in
 * separate buffers for its norm chains to add; these entries return their
 * sum in Y): chn_batch_gemm_q4r as the o and down projections
 * (src/gpu/batch_dispatch.zig:108-109,129-130),
 * chn_batch_qkv_q4r as q, k and v in one launch over the same activations
 * (:70-81), chn_batch_fused_mlp_q4r as gate/up with the product written as
 * fp32 (Y) or as bf16 bits (Y_bf16, the form the down projection reads;
 * exactly one of the two) (:121-123).  X fp32 [n_tok][K], 16-byte aligned;
 * weights 16-byte aligned. */
int chn_batch_gemm_q4r(chn_ctx *ctx, const void *W, const float *X, float *Y, uint32_t n_tok, uint32_t M,
                       uint32_t K);
int chn_batch_qkv_q4r(chn_ctx *ctx, const void *Wq, const void *Wk, const void *Wv, const float *X,
                      float *Yq, float *Yk, float *Yv, uint32_t n_tok, uint32_t q_dim, uint32_t kv_dim,
                      uint32_t K);
int chn_batch_fused_mlp_q4r(chn_ctx *ctx, const void *Wg, const void *Wu, const float *X, float *Y,
                            uint16_t *Y_bf16, uint32_t n_tok, uint32_t M, uint32_t K);

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
 * S = *n_slots (DEVICE memory, clamped to max_slots <= 4096).  The list
 * buffer holds max_slots entries: entries at S and beyond are read (with
 * the count, in one round trip) but never used.  List and count are the
 * reference's Active_slots + Step_params[2] (global) or Active_slots +
 * 4096 + Step_params[3] (sliding).  Query head h reads KV head h / gqa_ratio at
 * cache row slot * kv_dim.  scale multiplies q.k (the reference passes 1.0).
 * head_dim 256 or 512.  recordDecodeAttn (src/gpu/kernels.zig:147-152) +
 * shaders/decode_attn.wgsl. */
int chn_decode_attn(chn_ctx *ctx, const float *q, const float *k_cache, const float *v_cache,
                    const uint32_t *slots, const uint32_t *n_slots, uint32_t max_slots,
                    uint32_t num_q_heads, uint32_t head_dim, uint32_t kv_dim,
                    uint32_t gqa_ratio, float scale, float *out);

/* chn_decode_attn without any allocation.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops).  The split partials live in a 2 MiB
 * file-scope device array per GPU (held until the process ends) instead of
 * the context workspace, which chn_decode_attn may grow with hipMalloc.
 * The partials take min(ceil(max_slots / 16), 32) * num_q_heads *
 * (head_dim + 2) * 4 bytes; shapes above 2 MiB (at max_slots > 496:
 * num_q_heads * (head_dim + 2) > 16384, e.g. 32 query heads at head_dim
 * 512) return CHN_E_UNSUPPORTED.  All
 * calls on one GPU share the array: calls that overlap on one GPU (two
 * contexts or threads on the same device) race.  Results are bit-identical
 * to chn_decode_attn. */
int chn_decode_attn_noalloc(chn_ctx *ctx, const float *q, const float *k_cache, const float *v_cache,
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

/* Prefill RoPE over n_tok tokens: token t uses clock start_clock + t and
 * writes K/V at slot slots[slot_offset + t]; q/k/v rows are [t][dim].
 * batch_qkv_rope (shaders/batch_qkv_rope.wgsl, src/gpu/batch_dispatch.zig:84-95). */
int chn_batch_qkv_rope(chn_ctx *ctx, const float *q_in, const float *k_in, const float *v_in,
                       const float *q_norm_w, const float *k_norm_w, float *q_out,
                       float *k_cache, float *v_cache, const uint32_t *slots,
                       uint32_t slot_offset, uint32_t start_clock, uint32_t n_tok,
                       uint32_t num_q_heads, uint32_t num_kv_heads, uint32_t head_dim,
                       uint32_t rotary_dim, int k_eq_v, float theta, float eps);

/* Prefill attention: token t (query rows [t][num_q_heads*head_dim]) attends
 * over slots[start .. num_prev_slots + t] of the list, start = S - window
 * when window > 0 and S > window (the reference uses window 1024 on sliding
 * layers, 0 = whole list on full layers).  batch_causal_attn
 * (shaders/batch_causal_attn.wgsl, src/gpu/batch_dispatch.zig:97-106). */
int chn_batch_causal_attn(chn_ctx *ctx, const float *q, const float *k_cache, const float *v_cache,
                          const uint32_t *slots, uint32_t n_tok, uint32_t num_prev_slots,
                          uint32_t num_q_heads, uint32_t head_dim, uint32_t kv_dim,
                          uint32_t gqa_ratio, float scale, uint32_t window, float *out);

/* ======================================================================
 * Logits, selection, quantization
 * ==================================================================== */

/* y[M] = W[M x K] (Q8_0: f32 scale + 32 int8 per 36-byte block) . x[K];
 * K % 128 == 0, K <= 4096.  recordGemvLogits (src/gpu/kernels.zig:119-122) +
 * shaders/gemv_q8.wgsl. */
int chn_gemv_q8(chn_ctx *ctx, const uint32_t *W, const float *x, float *y, uint32_t M, uint32_t K);

/* Q8R: the Q8_0 blocks of W [rows x K] repacked into dst (rows * K / 32 * 36
 * bytes, 16-byte aligned) for coalesced streaming: per row, the first 16
 * codes of each of its blocks in block order, then the last 16 codes of
 * each; after all rows, the f32 scales in block order.  The model holds its
 * tied embedding this way.  Counterpart of chn_q4_repack for the logits table; the
 * reference keeps the Q8_0 layout (src/quant.zig:54-98). */
int chn_q8_repack(chn_ctx *ctx, const uint32_t *W, uint32_t rows, uint32_t K, void *dst);

/* chn_gemv_q8 over Q8R weights (chn_q8_repack): identical results to
 * chn_gemv_q8 on the same weights.  gemv_q8 (shaders/gemv_q8.wgsl) as the
 * model's logits run it. */
int chn_gemv_q8r(chn_ctx *ctx, const void *R, const float *x, float *y, uint32_t M, uint32_t K);

/* Global top-64 of 30*tanh(logit/30), sorted descending, ties by lower
 * index; ids/vals are device arrays of 64.  V <= 262144.  recordTopK
 * (src/gpu/kernels.zig:178-184) + shaders/topk_pass1.wgsl, topk_pass2.wgsl. */
int chn_topk64(chn_ctx *ctx, const float *logits, uint32_t V, uint32_t *ids, float *vals);

/* bf16 rows (device) -> Q4 / Q8_0 words (device), bit-exact with
 * quantizeRowQ4_0 / quantizeRowQ8_0 (src/quant.zig:21-98).  cols % 32 == 0. */
int chn_quantize_q4(chn_ctx *ctx, const uint16_t *src_bf16, uint32_t *dst, uint32_t rows, uint32_t cols);
int chn_quantize_q8(chn_ctx *ctx, const uint16_t *src_bf16, uint32_t *dst, uint32_t rows, uint32_t cols);

/* fp32 -> bf16 bits with the reference's rounding (bf16.fromF32,
 * src/tensor.zig:7-13), device to device. */
int chn_to_bf16_bits(chn_ctx *ctx, const float *src, uint16_t *dst, size_t n);

/* ======================================================================
 * Model level (GpuModelContext, src/gpu/model_gpu.zig:30-216; decode,
 * src/gpu/model_dispatch.zig:128-153; prefill, src/gpu/batch_dispatch.zig:27-172)
 * ==================================================================== */

/* ModelConfig (src/model/types.zig:43-61) fields the GPU path uses. */
typedef struct chn_model_config {
    uint32_t hidden_size, intermediate_size, vocab_size, num_layers;
    uint32_t num_heads, num_kv_heads, head_dim, rotary_dim;
    /* full-attention layers: global_head_dim / num_global_key_value_heads
     * (0 = same as head_dim / num_kv_heads); such layers rotate their whole
     * head (src/model/loader.zig:37-41) */
    uint32_t global_head_dim, num_global_kv_heads;
    float rms_norm_eps, rope_theta, rope_theta_full;
    uint32_t sliding_window;       /* informational: slot lists come from the caller */
    uint32_t k_eq_v;               /* attention_k_eq_v */
    uint32_t max_prefill_tokens;   /* BatchPrefillContext max_tokens (model_gpu.zig:178) */
    uint8_t layer_full[64];        /* 1 = full_attention, 0 = sliding_attention */
    /* GpuModelContext.init's quiescence_thresh (model_gpu.zig:68,198): > 0
     * gates layers >= num_layers / 3 of the decode steps that return logits
     * (model_dispatch.zig:47-126, shaders/quiescence_gate.wgsl): a layer whose
     * input stream's mean squared change since the previous such step is
     * below it runs none of its work (no K/V write either); 0 = off. */
    float quiescence_thresh;
    /* Prefill attention window of sliding layers: 0 = 1024, the reference's
     * fixed value (shaders/batch_causal_attn.wgsl:53); sliding_window makes
     * prefill agree with decode. */
    uint32_t prefill_window;
} chn_model_config;

/* LayerWeights (src/model/types.zig:13-41): host bf16 tensors, row-major
 * [out][in]; NULL v_proj uses k_proj; NULL norms read as 1.0; NULL post
 * norms are skipped. */
typedef struct chn_layer_weights {
    const uint16_t *input_layernorm, *q_proj, *k_proj, *v_proj, *o_proj, *q_norm, *k_norm;
    const uint16_t *post_attention_layernorm, *pre_feedforward_layernorm;
    const uint16_t *gate_proj, *up_proj, *down_proj, *post_feedforward_layernorm;
    float layer_scalar;
    int has_layer_scalar;
} chn_layer_weights;

/* ProgressFn (src/gpu/batch_dispatch.zig:25). */
typedef void (*chn_progress_fn)(size_t layer_idx, size_t total_layers, void *ctx);

/* GpuModelContext.init: quantize bf16 weights on the device (Q4 for the
 * layers, Q8 for the tied embedding), allocate KV caches (4096 slots per
 * layer), record the decode graphs.  The caller may drop its bf16 pages
 * afterwards. */
int chn_model_create(chn_ctx *ctx, const chn_model_config *cfg, const chn_layer_weights *layers,
                     const uint16_t *embed_bf16, const uint16_t *final_norm_bf16, chn_model **out);

/* Same, with seeded synthetic weights generated in HBM (codes uniform,
 * f16 scales U(0.005, 0.02), norms 1.0, bf16 embedding ~ N(0, 0.02) kept on
 * the device for the input gather).  No reference counterpart. */
int chn_model_create_synthetic(chn_ctx *ctx, const chn_model_config *cfg, uint64_t seed, chn_model **out);

/* GpuModelContext.deinit (src/gpu/model_gpu.zig:203-215). */
void chn_model_destroy(chn_model *m);

int chn_model_get_config(const chn_model *m, chn_model_config *cfg);

/* Decode launch mode: enabled != 0 (default) replays the recorded graph;
 * 0 launches the same kernels one by one on the stream (for tools that do
 * not follow graph launches).  No reference counterpart. */
int chn_model_set_graph(chn_model *m, int enabled);

/* Device pointer to the model's bf16 embedding table (vocab x hidden). */
int chn_model_embedding_bf16(chn_model *m, const uint16_t **table);

/* gpuDispatchForwardToken (src/gpu/model_dispatch.zig:128-153): x[hidden]
 * (host), the global and sliding slot lists (host, <= 4096 each), clock and
 * the slot receiving this token's K/V.  With topk_ids != NULL the logits
 * graph runs and 64 candidates are returned; *token_out = ids[0] (the
 * reference's return value).  Returns a status; the reference's "return 0
 * on submit failure" is the caller's choice. */
int chn_decode_step(chn_model *m, const float *x, uint32_t clock, uint32_t slot_idx,
                    const uint32_t *active, uint32_t n_active, const uint32_t *sliding,
                    uint32_t n_sliding, uint32_t *topk_ids, float *topk_vals, uint32_t *token_out);

/* forwardToken's embedding step (src/model/forward.zig:35-37) on the
 * device (gather from the model's bf16 embedding), then chn_decode_step. */
int chn_decode_token(chn_model *m, uint32_t token, uint32_t clock, uint32_t slot_idx,
                     const uint32_t *active, uint32_t n_active, const uint32_t *sliding,
                     uint32_t n_sliding, uint32_t *topk_ids, float *topk_vals, uint32_t *token_out);

/* The state of the reference's KV ring (DynamicRingBuffer,
 * src/ring_buffer.zig:17-355) that decides a decode step's slot lists when
 * every clock so far was written and nothing was evicted.  The ring holds
 * 4096 slots: anchors [0, num_anchors) keep clocks 0..num_anchors-1, the FIFO
 * window [num_anchors, 3968) takes clock c at slot
 * num_anchors + (c - num_anchors) mod (3968 - num_anchors)
 * (getSlotIndexLayer, :117-122), the recall tier [3968, 4096) holds
 * retrieved entries (writeRecallKV, :277-285). */
#define CHN_RECALL_NONE 0xFFFFFFFFu
typedef struct chn_ring_state {
    uint32_t num_anchors;            /* <= 3904 (setNumAnchors' cap, :101-103) */
    uint32_t num_boundaries;         /* turn boundaries, <= 1024 (markBoundary, :79-90) */
    const uint32_t *boundaries;      /* host, oldest first; snapToBoundary (:92-100) moves
                                        the global window's start to the first one at or
                                        after it */
    const uint32_t *recall_clocks;   /* host, 128 entries: the clock held by recall slot
                                        3968 + r, or CHN_RECALL_NONE; NULL = none active */
} chn_ring_state;

/* n_steps (<= 4096) greedy decode steps without host round trips: the
 * server's decode loop (src/server/decode.zig:7-27) over forwardToken's GPU
 * branch (src/model/forward.zig:41-47) with the slot lists generated on the
 * device.  Step i runs at clock + i with slot_idx = getSlotIndexLayer(clock
 * + i), the global list = getActiveSlotsLayer(layer 0, full) = the anchors,
 * the window clocks from the snapped start of the newest 3968 - num_anchors,
 * then the recall slots whose clock is <= clock + i; the sliding list = the
 * newest cfg.sliding_window clocks (anchors included, no recall)
 * (src/ring_buffer.zig:291-333).  Step i feeds token (i = 0) or step i-1's
 * argmax; tokens_out[i] = step i's argmax.  ring NULL = no anchors, no
 * boundaries, no recall.  Equivalent to n calls of chn_decode_token with
 * those lists.  No direct reference counterpart. */
int chn_decode_greedy(chn_model *m, uint32_t token, uint32_t clock, uint32_t n_steps,
                      const chn_ring_state *ring, uint32_t *tokens_out);

/* gpuDispatchPrefillBatch: n <= max_prefill_tokens tokens (else
 * CHN_E_BATCH_TOO_LARGE); slots[0..n_slots) lists num_prev_slots earlier
 * slots then one slot per new token; embed_bf16 is the host table
 * (vocab x hidden) or NULL to use the model's device table.  Synchronizes
 * every 4 layers and calls progress.  logits_out (host, vocab floats) and
 * topk_ids/topk_vals (host, 64) may be NULL. */
int chn_prefill(chn_model *m, const uint32_t *tokens, uint32_t n, const uint16_t *embed_bf16,
                const uint32_t *slots, uint32_t n_slots, uint32_t start_clock, uint32_t num_prev_slots,
                float *logits_out, uint32_t *topk_ids, float *topk_vals, chn_progress_fn progress,
                void *progress_ctx);

/* KV cache access replacing the UMA reads/writes of buf_k_cache/buf_v_cache
 * (src/snapshot.zig:95-98,171-174, src/memory.zig:104-107,
 * src/hippocampus.zig:166-169, src/model/memory_inject.zig:14-30): n slots
 * from slot_begin of one layer, each that layer's kv_dim floats. */
int chn_kv_read(chn_model *m, uint32_t layer, uint32_t slot_begin, uint32_t n, float *k_out, float *v_out);
int chn_kv_write(chn_model *m, uint32_t layer, uint32_t slot_begin, uint32_t n, const float *k_in,
                 const float *v_in);

/* Reads of buf_x / buf_normed_x (src/server/decode.zig:13,
 * src/model/memory_inject.zig:56): hidden state and last normed row.  Both
 * start at zero when the model is created (what src/server.zig:76-81 sets
 * them to). */
int chn_model_read_state(chn_model *m, float *x_out, float *normed_out);

/* Reads of buf_logits (src/gpu/model_gpu.zig:30-216; zeroed by
 * src/server.zig:77): the fp32 logits (vocab floats, host) of the last decode
 * step or prefill that computed them; zero at creation. */
int chn_model_read_logits(chn_model *m, float *logits_out);

/* GpuEngine.submitPreRecorded(cmd_buf_decode) (src/gpu/kernels.zig:189-194,
 * called by src/model/bench.zig:12-15): runs the recorded decode step once
 * more on the inputs already on the device -- the stream x as the last step
 * left it, and the slot lists, clock and slot_idx of the last decode call --
 * and waits for it, as the reference waits on its fence.  with_logits != 0
 * runs the logits step (cmd_buf_decode) and, when topk_ids / topk_vals
 * (host, 64 each) are set, returns its top-64; 0 runs the step without
 * logits (topk pointers must be NULL).  The same kernels as chn_decode_step,
 * so the results equal a chn_decode_step call with x = the device stream and
 * the same lists. */
int chn_model_replay(chn_model *m, int with_logits, uint32_t *topk_ids, float *topk_vals);

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
