/*
 * CPU oracle for the Q4 inference hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library; the product library never links it.  Built with
 * -ffp-contract=off so that fp32 expressions round exactly where written.
 * Citations are to the reference checkout (Sullux/channel).
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

/* ======================================================================
 * Scalar conversions
 * ==================================================================== */

/* Zig's @floatCast(f32 -> f16) is IEEE round-to-nearest-even
 * (src/tensor.zig:26-28, used by src/quant.zig:76-77). */
uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) /* inf / nan */
        return (uint16_t)(sign | 0x7c00u | (man ? (0x200u | (man >> 13)) : 0u));
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        int shift = 14 - e;
        uint32_t h = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)h;
}

/* WGSL unpack2x16float(...).x / Zig @floatCast(f16 -> f32): exact. */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t man = (uint32_t)h & 0x3ffu;
    uint32_t out;
    if (exp == 0) {
        if (man == 0) {
            out = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do { man <<= 1; e++; } while (!(man & 0x400u));
            man &= 0x3ffu;
            out = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1f) {
        out = sign | 0x7f800000u | (man << 13);
    } else {
        out = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &out, 4);
    return f;
}

/* bf16.fromF32: add 0x7FFF + lsb, keep the high half (src/tensor.zig:7-13). */
uint16_t orc_bf16_from_f32(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    uint32_t bias = 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)((u + bias) >> 16);
}

/* bf16.toF32 (src/tensor.zig:15-18). */
float orc_bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* ======================================================================
 * Quantizers
 * ==================================================================== */

/* Zig std.math.round: half away from zero, same as C roundf. */
static inline int32_t zig_round_to_i32(float v) { return (int32_t)roundf(v); }

static inline int32_t clamp_i32(int32_t v, int32_t lo, int32_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

/* quantizeRowQ4_0 (src/quant.zig:58-98): per 32-block d = amax/8,
 * id = 1/d, q = clamp(round(v*id + 8), 0, 15); word0 = f16(d) | f16(-8d)<<16;
 * element 8w+n is nibble n (bits 4n..4n+3) of word 1+w. */
void orc_quantize_row_q4(uint32_t *dst, const uint16_t *src, size_t n) {
    size_t nb = n / 32;
    for (size_t b = 0; b < nb; ++b) {
        const uint16_t *s = src + b * 32;
        uint32_t *o = dst + b * 5;
        float vals[32];
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) {
            vals[i] = orc_bf16_to_f32(s[i]);
            float a = fabsf(vals[i]);
            if (a > amax) amax = a;
        }
        float d = amax / 8.0f;
        float id = d > 0.0f ? 1.0f / d : 0.0f;
        uint16_t sc = orc_f32_to_f16(d);
        uint16_t mn = orc_f32_to_f16(-8.0f * d);
        o[0] = (uint32_t)sc | ((uint32_t)mn << 16);
        uint8_t nib[32];
        for (int i = 0; i < 32; ++i) {
            float t = vals[i] * id;
            t = t + 8.0f;
            nib[i] = (uint8_t)clamp_i32(zig_round_to_i32(t), 0, 15);
        }
        for (int w = 0; w < 4; ++w) {
            uint32_t word = 0;
            for (int k = 0; k < 8; ++k) word |= (uint32_t)nib[w * 8 + k] << (4 * k);
            o[1 + w] = word;
        }
    }
}

/* quantizeRowQ8_0 (src/quant.zig:21-52): d = amax/127 stored as raw f32,
 * q = clamp(round(v * 127/amax), -128, 127), 32 int8 little-endian in
 * words 1..8. */
void orc_quantize_row_q8(uint32_t *dst, const uint16_t *src, size_t n) {
    size_t nb = n / 32;
    for (size_t b = 0; b < nb; ++b) {
        const uint16_t *s = src + b * 32;
        uint32_t *o = dst + b * 9;
        float vals[32];
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) {
            vals[i] = orc_bf16_to_f32(s[i]);
            float a = fabsf(vals[i]);
            if (a > amax) amax = a;
        }
        float d = amax / 127.0f;
        float id = amax > 0.0f ? 127.0f / amax : 0.0f;
        memcpy(&o[0], &d, 4);
        uint8_t bytes[32];
        for (int i = 0; i < 32; ++i) {
            int32_t q = clamp_i32(zig_round_to_i32(vals[i] * id), -128, 127);
            bytes[i] = (uint8_t)(int8_t)q;
        }
        for (int w = 0; w < 8; ++w)
            o[1 + w] = (uint32_t)bytes[4 * w] | ((uint32_t)bytes[4 * w + 1] << 8) |
                       ((uint32_t)bytes[4 * w + 2] << 16) | ((uint32_t)bytes[4 * w + 3] << 24);
    }
}

/* quantizeMatrix row loop (src/quant.zig:100-170); row stride =
 * getQuantizedRowWords (src/quant.zig:172-179). */
void orc_quantize_matrix_q4(uint32_t *dst, const uint16_t *src, size_t rows, size_t cols) {
    size_t rw = ((cols + 31) / 32) * 5;
    for (size_t r = 0; r < rows; ++r) orc_quantize_row_q4(dst + r * rw, src + r * cols, cols);
}

void orc_quantize_matrix_q8(uint32_t *dst, const uint16_t *src, size_t rows, size_t cols) {
    size_t rw = ((cols + 31) / 32) * 9;
    for (size_t r = 0; r < rows; ++r) orc_quantize_row_q8(dst + r * rw, src + r * cols, cols);
}

/* scale*(q-8) with the f16 scale in the low half of word 0 and the min
 * half ignored (shaders/gemv_q4.wgsl:15-26,47). */
void orc_dequant_q4(float *dst, const uint32_t *W, size_t rows, size_t K) {
    size_t nb = K / 32;
    for (size_t r = 0; r < rows; ++r)
        for (size_t b = 0; b < nb; ++b) {
            const uint32_t *blk = W + (r * nb + b) * 5;
            float s = orc_f16_to_f32((uint16_t)(blk[0] & 0xffffu));
            for (int w = 0; w < 4; ++w)
                for (int n = 0; n < 8; ++n) {
                    float q = (float)((blk[1 + w] >> (4 * n)) & 0xfu) - 8.0f;
                    dst[r * K + b * 32 + w * 8 + n] = s * q;
                }
        }
}

/* Q8 dequant: raw f32 scale * int8 (shaders/gemv_q8.wgsl:41-55). */
void orc_dequant_q8(float *dst, const uint32_t *W, size_t rows, size_t K) {
    size_t nb = K / 32;
    for (size_t r = 0; r < rows; ++r)
        for (size_t b = 0; b < nb; ++b) {
            const uint32_t *blk = W + (r * nb + b) * 9;
            float s;
            memcpy(&s, &blk[0], 4);
            for (int i = 0; i < 32; ++i) {
                int8_t q = (int8_t)((blk[1 + i / 4] >> (8 * (i % 4))) & 0xffu);
                dst[r * K + b * 32 + i] = s * (float)q;
            }
        }
}

/* ======================================================================
 * Decode matvecs
 * ==================================================================== */

/* gelu_tanh (shaders/fused_mlp_q4.wgsl:15-18 = src/kernels.zig:7-10). */
float orc_gelu_tanh(float x) {
    float c = 0.044715f * x; /* WGSL evaluates 0.044715 * x * x * x left to right */
    c = c * x;
    c = c * x;
    float inner = x + c;
    inner = 0.7978845608f * inner;
    float t = 1.0f + tanhf(inner);
    float h = 0.5f * x;
    return h * t;
}

/* unpack_dot2 (shaders/gemv_q4.wgsl:15-26): nibbles 0..3 against v_a,
 * 4..7 against v_b, summed left to right. */
static inline float unpack_dot2(uint32_t w, const float *xa) {
    float acc = 0.0f;
    for (int n = 0; n < 8; ++n) {
        float q = (float)((w >> (4 * n)) & 0xfu) - 8.0f;
        float p = q * xa[n];
        acc = (n == 0) ? p : acc + p;
    }
    return acc;
}

/* One output row of gemv_q4 in the shader's order: 32 lanes, lane l takes
 * blocks l, l+32, ...; acc += s*(ud(w0)+ud(w1)+ud(w2)+ud(w3)); then a
 * 16/8/4/2/1 tree (shaders/gemv_q4.wgsl:41-92). */
static float gemv_q4_row(const uint32_t *Wrow, const float *x, uint32_t nb) {
    float lanes[32];
    for (uint32_t lane = 0; lane < 32; ++lane) {
        float acc = 0.0f;
        for (uint32_t b = lane; b < nb; b += 32) {
            const uint32_t *blk = Wrow + b * 5;
            float s = orc_f16_to_f32((uint16_t)(blk[0] & 0xffffu));
            const float *xb = x + b * 32;
            float d = unpack_dot2(blk[1], xb);
            d = d + unpack_dot2(blk[2], xb + 8);
            d = d + unpack_dot2(blk[3], xb + 16);
            d = d + unpack_dot2(blk[4], xb + 24);
            acc = acc + s * d;
        }
        lanes[lane] = acc;
    }
    for (uint32_t off = 16; off >= 1; off >>= 1)
        for (uint32_t l = 0; l < off; ++l) lanes[l] = lanes[l] + lanes[l + off];
    return lanes[0];
}

void orc_gemv_q4(const uint32_t *W, const float *x, float *y, uint32_t M, uint32_t K) {
    uint32_t nb = K / 32;
    for (uint32_t r = 0; r < M; ++r) y[r] = gemv_q4_row(W + (size_t)r * nb * 5, x, nb);
}

/* fused_qkv_q4: rows [0,q) from Wq, [q,q+kv) from Wk, rest from Wv, each
 * exactly a gemv_q4 row (shaders/fused_qkv_q4.wgsl:37-154). */
void orc_fused_qkv_q4(const uint32_t *Wq, const uint32_t *Wk, const uint32_t *Wv,
                      const float *x, float *q, float *k, float *v,
                      uint32_t q_dim, uint32_t kv_dim, uint32_t K) {
    orc_gemv_q4(Wq, x, q, q_dim, K);
    orc_gemv_q4(Wk, x, k, kv_dim, K);
    orc_gemv_q4(Wv, x, v, kv_dim, K);
}

/* fused_mlp_q4: gate and up rows reduced as in gemv_q4, then
 * act = gelu_tanh(gate) * up (shaders/fused_mlp_q4.wgsl:33-127). */
void orc_fused_mlp_q4(const uint32_t *Wg, const uint32_t *Wu, const float *x,
                      float *act, uint32_t M, uint32_t K) {
    uint32_t nb = K / 32;
    for (uint32_t r = 0; r < M; ++r) {
        float g = gemv_q4_row(Wg + (size_t)r * nb * 5, x, nb);
        float u = gemv_q4_row(Wu + (size_t)r * nb * 5, x, nb);
        act[r] = orc_gelu_tanh(g) * u;
    }
}

/* gemv_q8 (shaders/gemv_q8.wgsl:20-86): 32 lanes; lane = (block-in-8,
 * word-pair); acc += s * sum of 8 int8*x; 16..1 tree.  The shader reads
 * blocks base+0..7 without a bound; here blocks >= K/32 are skipped (all
 * live calls have K/32 % 8 == 0, where the two agree). */
static float gemv_q8_row(const uint32_t *Wrow, const float *x, uint32_t nb) {
    float lanes[32];
    for (uint32_t lane = 0; lane < 32; ++lane) {
        uint32_t bi = lane >> 2, sub = lane & 3u;
        float acc = 0.0f;
        for (uint32_t base = 0; base < nb; base += 8) {
            uint32_t b = base + bi;
            if (b >= nb) continue;
            const uint32_t *blk = Wrow + b * 9;
            float s;
            memcpy(&s, &blk[0], 4);
            uint32_t wa = blk[1 + sub * 2], wb = blk[2 + sub * 2];
            const float *xv = x + b * 32 + sub * 8;
            float sum = 0.0f;
            for (int i = 0; i < 8; ++i) {
                uint32_t w = i < 4 ? wa : wb;
                float q = (float)(int8_t)((w >> (8 * (i & 3))) & 0xffu);
                float p = q * xv[i];
                sum = (i == 0) ? p : sum + p;
            }
            acc = acc + s * sum;
        }
        lanes[lane] = acc;
    }
    for (uint32_t off = 16; off >= 1; off >>= 1)
        for (uint32_t l = 0; l < off; ++l) lanes[l] = lanes[l] + lanes[l + off];
    return lanes[0];
}

void orc_gemv_q8(const uint32_t *W, const float *x, float *y, uint32_t M, uint32_t K) {
    uint32_t nb = K / 32;
    for (uint32_t r = 0; r < M; ++r) y[r] = gemv_q8_row(W + (size_t)r * nb * 9, x, nb);
}

/* ======================================================================
 * Prefill contractions
 * ==================================================================== */

/* vec4 dot of (q-8) nibbles against x (batch_gemm_q4.wgsl:18-24). */
static inline float unpack_dot2_vec(uint32_t w, const float *xa) {
    float na[8];
    for (int n = 0; n < 8; ++n) na[n] = (float)((w >> (4 * n)) & 0xfu) - 8.0f;
    float a = na[0] * xa[0];
    a = a + na[1] * xa[1];
    a = a + na[2] * xa[2];
    a = a + na[3] * xa[3];
    float b = na[4] * xa[4];
    b = b + na[5] * xa[5];
    b = b + na[6] * xa[6];
    b = b + na[7] * xa[7];
    return a + b;
}

/* Y[t*M + r] = sum_b s_b * (ud(w1)+ud(w2)+ud(w3)+ud(w4)), blocks in order,
 * one accumulator per (t, r) (shaders/batch_gemm_q4.wgsl:26-159).  The
 * reference's push constants name tokens N and output rows M. */
void orc_batch_gemm_q4(const uint32_t *W, const float *X, float *Y,
                       uint32_t n_tok, uint32_t M, uint32_t K) {
    uint32_t nb = K / 32;
    for (uint32_t t = 0; t < n_tok; ++t) {
        const float *x = X + (size_t)t * K;
        for (uint32_t r = 0; r < M; ++r) {
            const uint32_t *Wrow = W + (size_t)r * nb * 5;
            float acc = 0.0f;
            for (uint32_t b = 0; b < nb; ++b) {
                const uint32_t *blk = Wrow + b * 5;
                float s = orc_f16_to_f32((uint16_t)(blk[0] & 0xffffu));
                const float *xb = x + b * 32;
                float d = unpack_dot2_vec(blk[1], xb);
                d = d + unpack_dot2_vec(blk[2], xb + 8);
                d = d + unpack_dot2_vec(blk[3], xb + 16);
                d = d + unpack_dot2_vec(blk[4], xb + 24);
                acc = acc + s * d;
            }
            Y[(size_t)t * M + r] = acc;
        }
    }
}

/* Y = gelu_tanh(G) * U per (t, r) (shaders/batch_fused_mlp_q4.wgsl:33-195). */
void orc_batch_fused_mlp_q4(const uint32_t *Wg, const uint32_t *Wu, const float *X,
                            float *Y, uint32_t n_tok, uint32_t M, uint32_t K) {
    float *G = (float *)malloc((size_t)n_tok * M * sizeof(float));
    float *U = (float *)malloc((size_t)n_tok * M * sizeof(float));
    orc_batch_gemm_q4(Wg, X, G, n_tok, M, K);
    orc_batch_gemm_q4(Wu, X, U, n_tok, M, K);
    for (size_t i = 0; i < (size_t)n_tok * M; ++i) Y[i] = orc_gelu_tanh(G[i]) * U[i];
    free(G);
    free(U);
}

/* MFMA operand model: w = bf16(s*(q-8)), x = bf16(x), fp32 sum of exact
 * products (bf16*bf16 fits fp32), K ascending. */
void orc_batch_gemm_q4_bf16(const uint32_t *W, const float *X, float *Y,
                            uint32_t n_tok, uint32_t M, uint32_t K) {
    float *Wd = (float *)malloc((size_t)M * K * sizeof(float));
    float *Xb = (float *)malloc((size_t)n_tok * K * sizeof(float));
    orc_dequant_q4(Wd, W, M, K);
    for (size_t i = 0; i < (size_t)M * K; ++i) Wd[i] = orc_bf16_to_f32(orc_bf16_from_f32(Wd[i]));
    for (size_t i = 0; i < (size_t)n_tok * K; ++i) Xb[i] = orc_bf16_to_f32(orc_bf16_from_f32(X[i]));
    for (uint32_t t = 0; t < n_tok; ++t)
        for (uint32_t r = 0; r < M; ++r) {
            const float *w = Wd + (size_t)r * K, *x = Xb + (size_t)t * K;
            float acc = 0.0f;
            for (uint32_t k = 0; k < K; ++k) acc = acc + w[k] * x[k];
            Y[(size_t)t * M + r] = acc;
        }
    free(Wd);
    free(Xb);
}

/* ======================================================================
 * Attention, RoPE, norms
 * ==================================================================== */

/* Softmax-weighted sum over a slot list, shared by the decode and the
 * batched prefill kernels: scores = (q.K)*scale; max starts at -1e9; 32
 * lanes stride the slots, then a 16..1 tree; inv = 1/(sum + 1e-9);
 * out = sum_i p_i V_i accumulated in bursts of 8
 * (shaders/decode_attn.wgsl:49-217, shaders/batch_causal_attn.wgsl:55-222). */
static void attn_one_head(const float *q, const float *Kc, const float *Vc,
                          const uint32_t *slots, uint32_t start, uint32_t S,
                          uint32_t head_dim, uint32_t kv_dim, uint32_t kv_h,
                          float scale, float *out, float *scores) {
    for (uint32_t i = start; i < S; ++i) {
        const float *k = Kc + (size_t)slots[i] * kv_dim + (size_t)kv_h * head_dim;
        float dot = 0.0f;
        for (uint32_t d = 0; d < head_dim; d += 16) {
            float part = 0.0f;
            for (uint32_t j = 0; j < 16; j += 4) {
                float v4 = q[d + j] * k[d + j];
                v4 = v4 + q[d + j + 1] * k[d + j + 1];
                v4 = v4 + q[d + j + 2] * k[d + j + 2];
                v4 = v4 + q[d + j + 3] * k[d + j + 3];
                part = (j == 0) ? v4 : part + v4;
            }
            dot = dot + part;
        }
        scores[i] = dot * scale;
    }
    float lane_max[32], lane_sum[32];
    for (uint32_t l = 0; l < 32; ++l) {
        float m = -1e9f;
        for (uint32_t i = start + l; i < S; i += 32)
            if (scores[i] > m) m = scores[i];
        lane_max[l] = m;
    }
    for (uint32_t off = 16; off >= 1; off >>= 1)
        for (uint32_t l = 0; l < off; ++l)
            if (lane_max[l + off] > lane_max[l]) lane_max[l] = lane_max[l + off];
    float mx = lane_max[0];
    for (uint32_t l = 0; l < 32; ++l) {
        float s = 0.0f;
        for (uint32_t i = start + l; i < S; i += 32) {
            float e = expf(scores[i] - mx);
            scores[i] = e;
            s = s + e;
        }
        lane_sum[l] = s;
    }
    for (uint32_t off = 16; off >= 1; off >>= 1)
        for (uint32_t l = 0; l < off; ++l) lane_sum[l] = lane_sum[l] + lane_sum[l + off];
    float inv = 1.0f / (lane_sum[0] + 1e-9f);
    for (uint32_t i = start; i < S; ++i) scores[i] = scores[i] * inv;
    for (uint32_t d = 0; d < head_dim; ++d) out[d] = 0.0f;
    uint32_t s = start;
    for (; s + 8 <= S; s += 8)
        for (uint32_t d = 0; d < head_dim; ++d) {
            float burst = 0.0f;
            for (uint32_t j = 0; j < 8; ++j) {
                const float *v = Vc + (size_t)slots[s + j] * kv_dim + (size_t)kv_h * head_dim;
                float p = scores[s + j] * v[d];
                burst = (j == 0) ? p : burst + p;
            }
            out[d] = out[d] + burst;
        }
    for (; s < S; ++s) {
        const float *v = Vc + (size_t)slots[s] * kv_dim + (size_t)kv_h * head_dim;
        for (uint32_t d = 0; d < head_dim; ++d) out[d] = out[d] + scores[s] * v[d];
    }
}

/* decode_attn (shaders/decode_attn.wgsl:24-218): q head h reads kv head
 * h / gqa_ratio; S = 0 leaves a zero output. */
void orc_decode_attn(const float *Q, const float *Kc, const float *Vc,
                     const uint32_t *slots, uint32_t S, uint32_t num_q_heads,
                     uint32_t head_dim, uint32_t kv_dim, uint32_t gqa_ratio,
                     float scale, float *out) {
    float *scores = (float *)malloc((S ? S : 1) * sizeof(float));
    for (uint32_t h = 0; h < num_q_heads; ++h)
        attn_one_head(Q + (size_t)h * head_dim, Kc, Vc, slots, 0, S, head_dim, kv_dim,
                      h / gqa_ratio, scale, out + (size_t)h * head_dim, scores);
    free(scores);
}

/* batch_causal_attn (shaders/batch_causal_attn.wgsl:25-223): token t sees
 * slots [start, prev+t+1) of the list, start = S - window when window > 0
 * and S > window (the reference hard-codes window 1024 for sliding layers,
 * line 53). */
void orc_batch_causal_attn(const float *Q, const float *Kc, const float *Vc,
                           const uint32_t *slots, uint32_t n_tok,
                           uint32_t num_prev_slots, uint32_t num_q_heads,
                           uint32_t head_dim, uint32_t kv_dim, uint32_t gqa_ratio,
                           float scale, uint32_t window, float *out) {
    uint32_t q_dim = num_q_heads * head_dim;
    float *scores = (float *)malloc((size_t)(num_prev_slots + n_tok) * sizeof(float));
    for (uint32_t t = 0; t < n_tok; ++t) {
        uint32_t S = num_prev_slots + t + 1;
        uint32_t start = (window > 0 && S > window) ? S - window : 0;
        for (uint32_t h = 0; h < num_q_heads; ++h)
            attn_one_head(Q + (size_t)t * q_dim + (size_t)h * head_dim, Kc, Vc, slots, start, S,
                          head_dim, kv_dim, h / gqa_ratio, scale,
                          out + (size_t)t * q_dim + (size_t)h * head_dim, scores);
    }
    free(scores);
}

/* 32-lane strided sum of squares, lane 0 sums the 32 partials in order
 * (shaders/qkv_rope.wgsl:42-61). */
static float head_inv_rms(const float *v, uint32_t D, float eps) {
    float lanes[32];
    for (uint32_t l = 0; l < 32; ++l) {
        float s = 0.0f;
        for (uint32_t d = l; d < D; d += 32) s = s + v[d] * v[d];
        lanes[l] = s;
    }
    float total = 0.0f;
    for (uint32_t l = 0; l < 32; ++l) total = total + lanes[l];
    return 1.0f / sqrtf(total / (float)D + eps);
}

/* RMSNorm * weight then RoPE over pairs (d, d + rot/2),
 * freq = 1/pow(theta, 2d/rot), angle = clock*freq; suffix past rot copied
 * normed (shaders/qkv_rope.wgsl:63-91). */
static void norm_rope_head(const float *in, const float *w, float *out, uint32_t D,
                           uint32_t rot, float theta, float eps, uint32_t clock) {
    float inv = head_inv_rms(in, D, eps);
    uint32_t half = rot / 2;
    for (uint32_t d = 0; d < half; ++d) {
        float v0 = in[d] * inv;
        v0 = v0 * w[d];
        float v1 = in[d + half] * inv;
        v1 = v1 * w[d + half];
        float fe = (2.0f * (float)d) / (float)rot;
        float freq = 1.0f / powf(theta, fe);
        float ang = (float)clock * freq;
        float c = cosf(ang), s = sinf(ang);
        float a = v0 * c;
        a = a - v1 * s;
        float b = v0 * s;
        b = b + v1 * c;
        out[d] = a;
        out[d + half] = b;
    }
    for (uint32_t d = rot; d < D; ++d) {
        float v = in[d] * inv;
        out[d] = v * w[d];
    }
}

/* qkv_rope (shaders/qkv_rope.wgsl:25-180): q heads normed+roped into q_out;
 * k heads normed+roped and v heads unit-RMS-normed into the caches at
 * slot_idx*kv_dim + kv_head*D (kv_dim = num_kv_heads*D). */
void orc_qkv_rope(const float *q_in, const float *k_in, const float *v_in,
                  const float *q_norm_w, const float *k_norm_w, float *q_out,
                  float *k_cache, float *v_cache, uint32_t num_q_heads,
                  uint32_t num_kv_heads, uint32_t D, uint32_t rot,
                  int k_eq_v, float theta, float eps, uint32_t clock,
                  uint32_t slot_idx) {
    uint32_t kv_dim = num_kv_heads * D;
    for (uint32_t h = 0; h < num_q_heads; ++h)
        norm_rope_head(q_in + (size_t)h * D, q_norm_w, q_out + (size_t)h * D, D, rot, theta, eps,
                       clock);
    for (uint32_t h = 0; h < num_kv_heads; ++h) {
        const float *k = k_in + (size_t)h * D;
        const float *v = k_eq_v ? k : v_in + (size_t)h * D;
        float *kc = k_cache + (size_t)slot_idx * kv_dim + (size_t)h * D;
        float *vc = v_cache + (size_t)slot_idx * kv_dim + (size_t)h * D;
        norm_rope_head(k, k_norm_w, kc, D, rot, theta, eps, clock);
        float inv = head_inv_rms(v, D, eps);
        for (uint32_t d = 0; d < D; ++d) vc[d] = v[d] * inv;
    }
}

/* rmsnorm (shaders/rmsnorm.wgsl): 256 threads x vec4 strided sum of
 * dot(v,v), 128..1 tree, y = (x * inverseSqrt(mean + eps)) * w. */
static float norm_sumsq_256(const float *x, uint32_t dim) {
    float lanes[256];
    uint32_t dv = dim / 4;
    for (uint32_t t = 0; t < 256; ++t) {
        float s = 0.0f;
        for (uint32_t i = t; i < dv; i += 256) {
            const float *v = x + 4 * i;
            float d = v[0] * v[0];
            d = d + v[1] * v[1];
            d = d + v[2] * v[2];
            d = d + v[3] * v[3];
            s = s + d;
        }
        lanes[t] = s;
    }
    for (uint32_t off = 128; off >= 1; off >>= 1)
        for (uint32_t l = 0; l < off; ++l) lanes[l] = lanes[l] + lanes[l + off];
    return lanes[0];
}

void orc_rmsnorm(const float *x, const float *w, float *y, uint32_t dim, float eps) {
    float r = 1.0f / sqrtf(norm_sumsq_256(x, dim) / (float)dim + eps);
    for (uint32_t i = 0; i < dim; ++i) {
        float v = x[i] * r;
        y[i] = v * w[i];
    }
}

/* add_rmsnorm (shaders/add_rmsnorm.wgsl): x = (x + r) * scalar in place,
 * then y = rmsnorm(x) * w. */
void orc_add_rmsnorm(float *x, const float *r, const float *w, float *y,
                     uint32_t dim, float eps, float scalar) {
    for (uint32_t i = 0; i < dim; ++i) {
        float s = x[i] + r[i];
        x[i] = s * scalar;
    }
    orc_rmsnorm(x, w, y, dim, eps);
}

/* ======================================================================
 * Logits selection
 * ==================================================================== */

/* softcap (shaders/topk_pass1.wgsl:17-19). */
float orc_softcap(float v) {
    float t = tanhf(v * (1.0f / 30.0f));
    return 30.0f * t;
}

typedef struct { float v; uint32_t i; } vi_t;

static int vi_cmp(const void *a, const void *b) {
    const vi_t *x = (const vi_t *)a, *y = (const vi_t *)b;
    if (x->v > y->v) return -1;
    if (x->v < y->v) return 1;
    return x->i < y->i ? -1 : (x->i > y->i ? 1 : 0);
}

/* Global top-64 of softcap(logits), sorted descending
 * (shaders/topk_pass1.wgsl + topk_pass2.wgsl).  Equal values order by
 * ascending index (the bitonic network leaves ties unspecified). */
void orc_topk64(const float *logits, uint32_t V, uint32_t *ids, float *vals) {
    vi_t *a = (vi_t *)malloc((size_t)V * sizeof(vi_t));
    for (uint32_t i = 0; i < V; ++i) { a[i].v = orc_softcap(logits[i]); a[i].i = i; }
    qsort(a, V, sizeof(vi_t), vi_cmp);
    for (uint32_t k = 0; k < 64; ++k) {
        if (k < V) { ids[k] = a[k].i; vals[k] = a[k].v; }
        else { ids[k] = 0; vals[k] = -1e30f; }
    }
    free(a);
}

/* sampleArgmax: first maximum (src/kernels.zig:133-143). */
uint32_t orc_argmax(const float *v, uint32_t n) {
    uint32_t best = 0;
    float bv = v[0];
    for (uint32_t i = 1; i < n; ++i)
        if (v[i] > bv) { bv = v[i]; best = i; }
    return best;
}

/* ======================================================================
 * Seeded synthetic inputs
 * ==================================================================== */

/* splitmix64 output function over a counter. */
uint64_t orc_mix64(uint64_t seed, uint64_t idx) {
    uint64_t z = seed + (idx + 1u) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Q4 block (row r, block b) = counter base (r*nb + b)*3: hash 0 -> scale
 * fma(u24 * 2^-24, smax - smin, smin) -> f16, min half f16(-8*s);
 * hashes 1, 2 -> the four nibble words (low half first). */
void orc_synth_q4(uint32_t *W, uint32_t rows, uint32_t K, uint64_t seed,
                  float smin, float smax) {
    uint32_t nb = K / 32;
    float range = smax - smin;
    for (uint64_t blk = 0; blk < (uint64_t)rows * nb; ++blk) {
        uint32_t *o = W + blk * 5;
        uint64_t h0 = orc_mix64(seed, blk * 3), h1 = orc_mix64(seed, blk * 3 + 1),
                 h2 = orc_mix64(seed, blk * 3 + 2);
        float u = (float)(uint32_t)(h0 >> 40) * (1.0f / 16777216.0f);
        float s = fmaf(u, range, smin);
        o[0] = (uint32_t)orc_f32_to_f16(s) | ((uint32_t)orc_f32_to_f16(-8.0f * s) << 16);
        o[1] = (uint32_t)h1;
        o[2] = (uint32_t)(h1 >> 32);
        o[3] = (uint32_t)h2;
        o[4] = (uint32_t)(h2 >> 32);
    }
}

/* Q8 block = counter base blk*5: hash 0 -> raw f32 scale, hashes 1..4 ->
 * the eight int8x4 words. */
void orc_synth_q8(uint32_t *W, uint32_t rows, uint32_t K, uint64_t seed,
                  float smin, float smax) {
    uint32_t nb = K / 32;
    float range = smax - smin;
    for (uint64_t blk = 0; blk < (uint64_t)rows * nb; ++blk) {
        uint32_t *o = W + blk * 9;
        uint64_t h0 = orc_mix64(seed, blk * 5);
        float u = (float)(uint32_t)(h0 >> 40) * (1.0f / 16777216.0f);
        float s = fmaf(u, range, smin);
        memcpy(&o[0], &s, 4);
        for (int j = 0; j < 4; ++j) {
            uint64_t h = orc_mix64(seed, blk * 5 + 1 + (uint64_t)j);
            o[1 + 2 * j] = (uint32_t)h;
            o[2 + 2 * j] = (uint32_t)(h >> 32);
        }
    }
}

/* Box-Muller on one hash per element: u1 = (hi24 + 1) * 2^-24 in (0, 1],
 * u2 = mid24 * 2^-24; z = sqrt(-2 ln u1) cos(2 pi u2) in double. */
void orc_synth_normal(float *dst, size_t n, uint64_t seed, float stddev) {
    for (size_t i = 0; i < n; ++i) {
        uint64_t h = orc_mix64(seed, i);
        double u1 = ((double)(h >> 40) + 1.0) * (1.0 / 16777216.0);
        double u2 = (double)((h >> 16) & 0xffffffu) * (1.0 / 16777216.0);
        double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        dst[i] = (float)(z * (double)stddev);
    }
}

/* ======================================================================
 * Threaded CPU baseline: rows in chunks of max(1, rows/(threads+1)),
 * workers pull chunks, the caller works too (src/kernels.zig:53-99).
 * ==================================================================== */

typedef struct {
    const uint32_t *W, *W2;
    const float *x;
    float *y;
    uint32_t rows, nb, chunk;
    int mode;   /* 0 Q4 matvec, 1 fused gate/up, 2 Q8 matvec */
    atomic_uint next;
} pool_job_t;

static void run_chunks(pool_job_t *j) {
    for (;;) {
        uint32_t c = atomic_fetch_add(&j->next, 1u);
        uint64_t s = (uint64_t)c * j->chunk;
        if (s >= j->rows) return;
        uint32_t e = (uint32_t)(s + j->chunk < j->rows ? s + j->chunk : j->rows);
        for (uint32_t r = (uint32_t)s; r < e; ++r) {
            if (j->mode == 2) {
                j->y[r] = gemv_q8_row(j->W + (size_t)r * j->nb * 9, j->x, j->nb);
                continue;
            }
            float g = gemv_q4_row(j->W + (size_t)r * j->nb * 5, j->x, j->nb);
            if (j->mode == 1) {
                float u = gemv_q4_row(j->W2 + (size_t)r * j->nb * 5, j->x, j->nb);
                j->y[r] = orc_gelu_tanh(g) * u;
            } else {
                j->y[r] = g;
            }
        }
    }
}

static void *pool_worker(void *arg) {
    run_chunks((pool_job_t *)arg);
    return NULL;
}

static void run_pool(pool_job_t *j, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    uint32_t chunk = j->rows / (uint32_t)(nthreads + 1);
    j->chunk = chunk > 0 ? chunk : 1;
    atomic_store(&j->next, 0u);
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nthreads);
    int spawned = 0;
    for (int t = 0; t < nthreads; ++t)
        if (pthread_create(&th[spawned], NULL, pool_worker, j) == 0) spawned++;
    run_chunks(j);
    for (int t = 0; t < spawned; ++t) pthread_join(th[t], NULL);
    free(th);
}

void orc_gemv_q4_mt(const uint32_t *W, const float *x, float *y, uint32_t M,
                    uint32_t K, int nthreads) {
    pool_job_t j;
    memset(&j, 0, sizeof(j));
    j.W = W; j.x = x; j.y = y; j.rows = M; j.nb = K / 32; j.mode = 0;
    run_pool(&j, nthreads);
}

void orc_fused_mlp_step_mt(const uint32_t *Wg, const uint32_t *Wu,
                           const uint32_t *Wd, const float *x, float *act,
                           float *y, uint32_t H, uint32_t I, int nthreads) {
    pool_job_t j;
    memset(&j, 0, sizeof(j));
    j.W = Wg; j.W2 = Wu; j.x = x; j.y = act; j.rows = I; j.nb = H / 32; j.mode = 1;
    run_pool(&j, nthreads);
    orc_gemv_q4_mt(Wd, act, y, H, I, nthreads);
}

void orc_gemv_q8_mt(const uint32_t *W, const float *x, float *y, uint32_t M,
                    uint32_t K, int nthreads) {
    pool_job_t j;
    memset(&j, 0, sizeof(j));
    j.W = W; j.x = x; j.y = y; j.rows = M; j.nb = K / 32; j.mode = 2;
    run_pool(&j, nthreads);
}

/* ======================================================================
 * Threaded forms for checking at full model sizes.  Each output element
 * is computed by exactly the serial routine's code, in the same order, so
 * every result is bit-identical to the serial one; threads only split the
 * independent rows.
 * ==================================================================== */

typedef void (*rows_fn)(void *arg, size_t r0, size_t r1);
typedef struct {
    rows_fn fn;
    void *arg;
    size_t r0, r1;
} rows_job_t;

static void *rows_worker(void *p) {
    rows_job_t *j = (rows_job_t *)p;
    j->fn(j->arg, j->r0, j->r1);
    return NULL;
}

/* fn over [0, n) in nthreads contiguous ranges, the caller taking the last. */
static void par_rows(size_t n, int nthreads, rows_fn fn, void *arg) {
    if (nthreads < 1) nthreads = 1;
    if ((size_t)nthreads > n) nthreads = n ? (int)n : 1;
    rows_job_t *jobs = (rows_job_t *)malloc(sizeof(rows_job_t) * (size_t)nthreads);
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nthreads);
    int *ok = (int *)calloc((size_t)nthreads, sizeof(int));
    for (int t = 0; t < nthreads; ++t) {
        jobs[t].fn = fn;
        jobs[t].arg = arg;
        jobs[t].r0 = n * (size_t)t / (size_t)nthreads;
        jobs[t].r1 = n * (size_t)(t + 1) / (size_t)nthreads;
    }
    for (int t = 0; t + 1 < nthreads; ++t) ok[t] = pthread_create(&th[t], NULL, rows_worker, &jobs[t]) == 0;
    for (int t = 0; t + 1 < nthreads; ++t)
        if (!ok[t]) rows_worker(&jobs[t]);     /* no thread: run it here */
    rows_worker(&jobs[nthreads - 1]);
    for (int t = 0; t + 1 < nthreads; ++t)
        if (ok[t]) pthread_join(th[t], NULL);
    free(ok);
    free(th);
    free(jobs);
}

typedef struct {
    uint32_t *dst;
    const uint16_t *src;
    size_t cols;
    int q8;
} quant_job_t;

static void quant_rows(void *p, size_t r0, size_t r1) {
    quant_job_t *j = (quant_job_t *)p;
    size_t rw = ((j->cols + 31) / 32) * (j->q8 ? 9 : 5);
    for (size_t r = r0; r < r1; ++r) {
        if (j->q8) orc_quantize_row_q8(j->dst + r * rw, j->src + r * j->cols, j->cols);
        else orc_quantize_row_q4(j->dst + r * rw, j->src + r * j->cols, j->cols);
    }
}

void orc_quantize_matrix_q4_mt(uint32_t *dst, const uint16_t *src, size_t rows, size_t cols, int nthreads) {
    quant_job_t j = {dst, src, cols, 0};
    par_rows(rows, nthreads, quant_rows, &j);
}

void orc_quantize_matrix_q8_mt(uint32_t *dst, const uint16_t *src, size_t rows, size_t cols, int nthreads) {
    quant_job_t j = {dst, src, cols, 1};
    par_rows(rows, nthreads, quant_rows, &j);
}

typedef struct {
    const uint32_t *W;
    const float *X;
    float *Wd, *Xb, *Y;
    uint32_t n_tok, M, K;
} bgemm_job_t;

static void bgemm_dequant_rows(void *p, size_t r0, size_t r1) {
    bgemm_job_t *j = (bgemm_job_t *)p;
    size_t nb = j->K / 32;
    orc_dequant_q4(j->Wd + r0 * j->K, j->W + r0 * nb * 5, r1 - r0, j->K);
    for (size_t i = r0 * j->K; i < r1 * j->K; ++i) j->Wd[i] = orc_bf16_to_f32(orc_bf16_from_f32(j->Wd[i]));
}

/* Blocks of 8 rows x 4 tokens: the token tile is transposed to [k][4] and
 * each row keeps a 4-lane vector of sums (one lane per token; lane-wise
 * multiply, then add, each rounded as the scalar code rounds it), so the
 * weights of a row block stay in cache across tokens and eight
 * independent sums are in flight.  Every sum runs over k in ascending
 * order, as in orc_batch_gemm_q4_bf16. */
typedef float f32x4 __attribute__((vector_size(16)));

static void bgemm_rows(void *p, size_t r0, size_t r1) {
    bgemm_job_t *j = (bgemm_job_t *)p;
    const uint32_t K = j->K;
    f32x4 *xt = (f32x4 *)aligned_alloc(16, (size_t)K * sizeof(f32x4));
    for (uint32_t t0 = 0; t0 < j->n_tok; t0 += 4) {
        const uint32_t nt = j->n_tok - t0 < 4 ? j->n_tok - t0 : 4;
        for (uint32_t k = 0; k < K; ++k)
            for (uint32_t c = 0; c < 4; ++c) xt[k][c] = c < nt ? j->Xb[(size_t)(t0 + c) * K + k] : 0.0f;
        for (size_t r = r0; r < r1; r += 8) {
            const size_t nr = r1 - r < 8 ? r1 - r : 8;
            const float *w[8];
            for (size_t i = 0; i < 8; ++i) w[i] = j->Wd + (r + (i < nr ? i : 0)) * K;
            f32x4 acc[8];
            for (int i = 0; i < 8; ++i) acc[i] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
            for (uint32_t k = 0; k < K; ++k) {
                const f32x4 x = xt[k];
                for (int i = 0; i < 8; ++i) {
                    const f32x4 prod = x * w[i][k];
                    acc[i] = acc[i] + prod;
                }
            }
            for (size_t i = 0; i < nr; ++i)
                for (uint32_t c = 0; c < nt; ++c) j->Y[(size_t)(t0 + c) * j->M + r + i] = acc[i][c];
        }
    }
    free(xt);
}

/* orc_batch_gemm_q4_bf16 over threads (output rows split). */
void orc_batch_gemm_q4_bf16_mt(const uint32_t *W, const float *X, float *Y, uint32_t n_tok, uint32_t M,
                               uint32_t K, int nthreads) {
    bgemm_job_t j = {W, X, NULL, NULL, Y, n_tok, M, K};
    j.Wd = (float *)malloc((size_t)M * K * sizeof(float));
    j.Xb = (float *)malloc((size_t)n_tok * K * sizeof(float));
    for (size_t i = 0; i < (size_t)n_tok * K; ++i) j.Xb[i] = orc_bf16_to_f32(orc_bf16_from_f32(X[i]));
    par_rows(M, nthreads, bgemm_dequant_rows, &j);
    par_rows(M, nthreads, bgemm_rows, &j);
    free(j.Wd);
    free(j.Xb);
}

typedef struct {
    const uint32_t *Wg, *Wu;
    const float *x;
    float *act;
    uint32_t nb;
} mlp_job_t;

static void mlp_rows(void *p, size_t r0, size_t r1) {
    mlp_job_t *j = (mlp_job_t *)p;
    for (size_t r = r0; r < r1; ++r) {
        float g = gemv_q4_row(j->Wg + r * j->nb * 5, j->x, j->nb);
        float u = gemv_q4_row(j->Wu + r * j->nb * 5, j->x, j->nb);
        j->act[r] = orc_gelu_tanh(g) * u;
    }
}

/* orc_fused_mlp_q4 over threads. */
void orc_fused_mlp_q4_mt(const uint32_t *Wg, const uint32_t *Wu, const float *x, float *act, uint32_t M,
                         uint32_t K, int nthreads) {
    mlp_job_t j = {Wg, Wu, x, act, K / 32};
    par_rows(M, nthreads, mlp_rows, &j);
}

/* Elementwise forms of the scalar routines over arrays. */
void orc_gelu_tanh_vec(const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = orc_gelu_tanh(x[i]);
}

void orc_softcap_vec(const float *x, float *y, size_t n) {
    for (size_t i = 0; i < n; ++i) y[i] = orc_softcap(x[i]);
}

typedef struct {
    const float *Q, *Kc, *Vc;
    const uint32_t *slots;
    uint32_t num_prev_slots, num_q_heads, head_dim, kv_dim, gqa_ratio, window;
    float scale;
    float *out;
} cattn_job_t;

static void cattn_rows(void *p, size_t t0, size_t t1) {
    cattn_job_t *j = (cattn_job_t *)p;
    const uint32_t q_dim = j->num_q_heads * j->head_dim;
    float *scores = (float *)malloc((size_t)(j->num_prev_slots + t1) * sizeof(float));
    for (size_t t = t0; t < t1; ++t) {
        uint32_t S = j->num_prev_slots + (uint32_t)t + 1;
        uint32_t start = (j->window > 0 && S > j->window) ? S - j->window : 0;
        for (uint32_t h = 0; h < j->num_q_heads; ++h)
            attn_one_head(j->Q + t * q_dim + (size_t)h * j->head_dim, j->Kc, j->Vc, j->slots, start, S, j->head_dim,
                          j->kv_dim, h / j->gqa_ratio, j->scale, j->out + t * q_dim + (size_t)h * j->head_dim,
                          scores);
    }
    free(scores);
}

/* orc_batch_causal_attn over threads (tokens split). */
void orc_batch_causal_attn_mt(const float *Q, const float *Kc, const float *Vc, const uint32_t *slots,
                              uint32_t n_tok, uint32_t num_prev_slots, uint32_t num_q_heads, uint32_t head_dim,
                              uint32_t kv_dim, uint32_t gqa_ratio, float scale, uint32_t window, float *out,
                              int nthreads) {
    cattn_job_t j = {Q, Kc, Vc, slots, num_prev_slots, num_q_heads, head_dim, kv_dim, gqa_ratio, window, scale, out};
    par_rows(n_tok, nthreads, cattn_rows, &j);
}

/* ======================================================================
 * Quiescence gate (shaders/quiescence_gate.wgsl:17-62, wired in
 * src/gpu/model_dispatch.zig:47-126): 32 lanes stride the hidden vector
 * summing (x - x_prev)^2 in order and copying x into x_prev, then a
 * 16/8/4/2 tree and s[0] + s[1]; the layer runs when the mean is at least
 * the threshold (or the threshold is not positive).
 * ==================================================================== */
int orc_quiescence_gate(const float *x, float *x_prev, uint32_t H, float thresh, float *mean_out) {
    float s[32];
    for (uint32_t lane = 0; lane < 32; ++lane) {
        float acc = 0.0f;
        for (uint32_t i = lane; i < H; i += 32) {
            const float d = x[i] - x_prev[i];
            acc = acc + d * d;
            x_prev[i] = x[i];
        }
        s[lane] = acc;
    }
    for (uint32_t off = 16; off >= 2; off >>= 1)
        for (uint32_t l = 0; l < off; ++l) s[l] = s[l] + s[l + off];
    const float mean_sq = (s[0] + s[1]) / (float)H;
    if (mean_out) *mean_out = mean_sq;
    return (mean_sq >= thresh) || (thresh <= 0.0f);
}
