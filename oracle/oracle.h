/*
 * CPU oracle for the Q4 inference hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Results are checked against this library: it is linked or
 * loaded by tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline
 * leg, never by the product library (channel_amd/).  It restates, in plain
 * C99 with fp32 arithmetic (built with -ffp-contract=off, so every product
 * and sum is rounded where the source shows it), the semantics of the
 * reference's CPU helpers and of the WGSL kernels its GPU path runs.
 *
 * Each function cites the reference file:line it follows.  How each one is
 * pinned (golden vectors, closed forms, brute force) is listed in
 * tests/test_oracle.py; parity of the transcendental functions (tanh, exp,
 * pow, sin, cos) is pinned only to libm precision, because the reference runs
 * them through an unpinned shader compiler and driver.
 */
#ifndef CHANNEL_ORACLE_H
#define CHANNEL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar conversions (src/tensor.zig:4-28) ------------------------- */
uint16_t orc_f32_to_f16(float v);          /* IEEE RNE, as Zig @floatCast  */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_bf16_from_f32(float v);       /* bias trick, tensor.zig:7-13 */
float orc_bf16_to_f32(uint16_t b);

/* ---- quantizers (src/quant.zig:21-98) --------------------------------- */
void orc_quantize_row_q4(uint32_t *dst_words, const uint16_t *src_bf16, size_t n);
void orc_quantize_row_q8(uint32_t *dst_words, const uint16_t *src_bf16, size_t n);
void orc_quantize_matrix_q4(uint32_t *dst, const uint16_t *src, size_t rows, size_t cols);
void orc_quantize_matrix_q8(uint32_t *dst, const uint16_t *src, size_t rows, size_t cols);
/* dequant used by every live Q4 kernel: scale*(q-8), min half ignored */
void orc_dequant_q4(float *dst, const uint32_t *W, size_t rows, size_t K);
void orc_dequant_q8(float *dst, const uint32_t *W, size_t rows, size_t K);

/* ---- decode matvecs (shaders/gemv_q4.wgsl, fused_qkv_q4.wgsl,
 *      fused_mlp_q4.wgsl, gemv_q8.wgsl) ---------------------------------- */
float orc_gelu_tanh(float x);
void orc_gemv_q4(const uint32_t *W, const float *x, float *y, uint32_t M, uint32_t K);
void orc_fused_qkv_q4(const uint32_t *Wq, const uint32_t *Wk, const uint32_t *Wv,
                      const float *x, float *q, float *k, float *v,
                      uint32_t q_dim, uint32_t kv_dim, uint32_t K);
void orc_fused_mlp_q4(const uint32_t *Wg, const uint32_t *Wu, const float *x,
                      float *act, uint32_t M, uint32_t K);
void orc_gemv_q8(const uint32_t *W, const float *x, float *y, uint32_t M, uint32_t K);

/* ---- prefill (shaders/batch_gemm_q4.wgsl, batch_fused_mlp_q4.wgsl) ----- */
void orc_batch_gemm_q4(const uint32_t *W, const float *X, float *Y,
                       uint32_t n_tok, uint32_t M, uint32_t K);
void orc_batch_fused_mlp_q4(const uint32_t *Wg, const uint32_t *Wu, const float *X,
                            float *Y, uint32_t n_tok, uint32_t M, uint32_t K);
/* same contraction with X and the dequantized weights rounded to bf16
 * (RNE) before an fp32-accumulated product: the MFMA prefill's operands */
void orc_batch_gemm_q4_bf16(const uint32_t *W, const float *X, float *Y,
                            uint32_t n_tok, uint32_t M, uint32_t K);

/* ---- attention and norms (shaders/decode_attn.wgsl, qkv_rope.wgsl,
 *      rmsnorm.wgsl, add_rmsnorm.wgsl) ----------------------------------- */
void orc_decode_attn(const float *Q, const float *Kc, const float *Vc,
                     const uint32_t *slots, uint32_t S, uint32_t num_q_heads,
                     uint32_t head_dim, uint32_t kv_dim, uint32_t gqa_ratio,
                     float scale, float *out);
void orc_qkv_rope(const float *q_in, const float *k_in, const float *v_in,
                  const float *q_norm_w, const float *k_norm_w, float *q_out,
                  float *k_cache, float *v_cache, uint32_t num_q_heads,
                  uint32_t num_kv_heads, uint32_t head_dim, uint32_t rotary_dim,
                  int k_eq_v, float theta, float eps, uint32_t clock,
                  uint32_t slot_idx);
void orc_rmsnorm(const float *x, const float *w, float *y, uint32_t dim, float eps);
void orc_add_rmsnorm(float *x, const float *r, const float *w, float *y,
                     uint32_t dim, float eps, float scalar);

/* ---- batched prefill helpers (shaders/batch_rmsnorm.wgsl,
 *      batch_add_rmsnorm.wgsl, batch_qkv_rope.wgsl,
 *      batch_causal_attn.wgsl) ------------------------------------------- */
void orc_batch_causal_attn(const float *Q, const float *Kc, const float *Vc,
                           const uint32_t *slots, uint32_t n_tok,
                           uint32_t num_prev_slots, uint32_t num_q_heads,
                           uint32_t head_dim, uint32_t kv_dim, uint32_t gqa_ratio,
                           float scale, uint32_t window, float *out);

/* ---- logits selection (shaders/topk_pass1.wgsl, topk_pass2.wgsl,
 *      src/kernels.zig:133-143) ------------------------------------------ */
float orc_softcap(float v);
void orc_topk64(const float *logits, uint32_t V, uint32_t *ids, float *vals);
uint32_t orc_argmax(const float *v, uint32_t n);

/* ---- seeded synthetic inputs (counter-based, identical on any host) ---- */
uint64_t orc_mix64(uint64_t seed, uint64_t idx);
void orc_synth_q4(uint32_t *W, uint32_t rows, uint32_t K, uint64_t seed,
                  float smin, float smax);
void orc_synth_q8(uint32_t *W, uint32_t rows, uint32_t K, uint64_t seed,
                  float smin, float smax);
void orc_synth_normal(float *dst, size_t n, uint64_t seed, float stddev);

/* ---- quiescence gate (shaders/quiescence_gate.wgsl): returns 1 when the
 *      layer runs; x_prev <- x ------------------------------------------- */
int orc_quiescence_gate(const float *x, float *x_prev, uint32_t H, float thresh, float *mean_out);

/* ---- threaded CPU baseline (src/kernels.zig:53-99 scheme) ------------- */
void orc_gemv_q4_mt(const uint32_t *W, const float *x, float *y, uint32_t M,
                    uint32_t K, int nthreads);
void orc_fused_mlp_step_mt(const uint32_t *Wg, const uint32_t *Wu,
                           const uint32_t *Wd, const float *x, float *act,
                           float *y, uint32_t H, uint32_t I, int nthreads);
void orc_gemv_q8_mt(const uint32_t *W, const float *x, float *y, uint32_t M,
                    uint32_t K, int nthreads);

/* ---- threaded forms for checking at full sizes (bit-identical to the
 *      serial routines: rows split over threads, each row's order kept) --- */
void orc_quantize_matrix_q4_mt(uint32_t *dst, const uint16_t *src, size_t rows, size_t cols, int nthreads);
void orc_quantize_matrix_q8_mt(uint32_t *dst, const uint16_t *src, size_t rows, size_t cols, int nthreads);
void orc_batch_gemm_q4_bf16_mt(const uint32_t *W, const float *X, float *Y, uint32_t n_tok, uint32_t M,
                               uint32_t K, int nthreads);
void orc_fused_mlp_q4_mt(const uint32_t *Wg, const uint32_t *Wu, const float *x, float *act, uint32_t M,
                         uint32_t K, int nthreads);
void orc_batch_causal_attn_mt(const float *Q, const float *Kc, const float *Vc, const uint32_t *slots,
                              uint32_t n_tok, uint32_t num_prev_slots, uint32_t num_q_heads, uint32_t head_dim,
                              uint32_t kv_dim, uint32_t gqa_ratio, float scale, uint32_t window, float *out,
                              int nthreads);
void orc_gelu_tanh_vec(const float *x, float *y, size_t n);
void orc_softcap_vec(const float *x, float *y, size_t n);

#ifdef __cplusplus
}
#endif
#endif
