// Decode attention over the ring-buffer slot list (shaders/decode_attn.wgsl)
// and the per-head RMSNorm + RoPE + KV-cache write (shaders/qkv_rope.wgsl).
//
// Decode attention is split over the slot list ("flash-decoding"): a
// workgroup takes one KV head and a chunk of 64 slots, serves all of that
// head's GQA query heads from one pass over K and V (1 KB contiguous rows,
// one coalesced 16-byte load per lane per row), and leaves a partial
// (max m, sum l, sum p*V) per query head; a second kernel merges the
// chunks.  The merged result equals the reference's two-pass softmax
// p_i = exp(s_i - max) / (sum exp(s_j - max) + 1e-9) up to rounding.  The
// slot count is read from device memory, so a captured graph can be
// replayed with a new count.
#include "chn_internal.h"

namespace chn {

constexpr int kAttnChunk = 64;   // slots per workgroup
constexpr float kNegBig = -1e30f;

typedef float f4 __attribute__((ext_vector_type(4)));

__host__ __device__ inline size_t attn_ws_bytes(uint32_t num_q_heads, uint32_t head_dim, uint32_t max_slots) {
    const size_t nsplit = (max_slots + kAttnChunk - 1) / kAttnChunk;
    return nsplit * num_q_heads * ((size_t)head_dim + 2) * 4;
}

// Partials: acc [nsplit][num_q_heads][D], then m and l [nsplit][num_q_heads].
template <int DV, int GQA>
__global__ __launch_bounds__(256) void k_attn_split(const float *__restrict__ Q, const float *__restrict__ Kc,
                                                    const float *__restrict__ Vc,
                                                    const uint32_t *__restrict__ slots,
                                                    const uint32_t *__restrict__ n_slots, uint32_t max_slots,
                                                    uint32_t num_q_heads, uint32_t kv_dim, float scale,
                                                    float *__restrict__ ws) {
    constexpr int D = DV * 256;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t split = blockIdx.x, kvh = blockIdx.y;
    uint32_t S = *n_slots;
    if (S > max_slots) S = max_slots;
    const uint32_t s0 = split * kAttnChunk;
    if (s0 >= S) return;
    const uint32_t cnt = (S - s0 < (uint32_t)kAttnChunk) ? S - s0 : kAttnChunk;
    const uint32_t nsplit = (max_slots + kAttnChunk - 1) / kAttnChunk;

    __shared__ float sc[GQA][kAttnChunk];
    __shared__ f4 pacc[4][GQA][DV * 64];

    // q for this KV head's query heads: lane holds 4 consecutive dims per DV
    f4 q[GQA][DV];
#pragma unroll
    for (int h = 0; h < GQA; ++h)
#pragma unroll
        for (int v = 0; v < DV; ++v)
            q[h][v] = *(const f4 *)(Q + (size_t)(kvh * GQA + h) * D + 4 * (lane + 64 * v));

    // ---- scores: wave w takes slots w*16 .. w*16+15 of the chunk
    const uint32_t base = s0 + wave * 16;
    float part[16 * GQA];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        f4 k[DV];
        const bool ok = (uint32_t)(wave * 16 + i) < cnt;
        const uint32_t ps = ok ? slots[base + i] : 0u;
        const float *kr = Kc + (size_t)ps * kv_dim + (size_t)kvh * D;
#pragma unroll
        for (int v = 0; v < DV; ++v) k[v] = ok ? *(const f4 *)(kr + 4 * (lane + 64 * v)) : f4{0, 0, 0, 0};
#pragma unroll
        for (int h = 0; h < GQA; ++h) {
            float d = 0.0f;
#pragma unroll
            for (int v = 0; v < DV; ++v) {
                d = fmaf(q[h][v].x, k[v].x, d);
                d = fmaf(q[h][v].y, k[v].y, d);
                d = fmaf(q[h][v].z, k[v].z, d);
                d = fmaf(q[h][v].w, k[v].w, d);
            }
            part[i * GQA + h] = d;
        }
    }
    // reduce the 16*GQA partial dots over the wave, at most 64 values per
    // butterfly: value v = i*GQA + h lands in lanes with lane >> (6 - LV) == v
    {
        constexpr int NG = (16 * GQA <= 64) ? 16 : 64 / GQA;   // slots per round
        constexpr int NV = NG * GQA;
        constexpr int LV = ilog2_c<NV>();
#pragma unroll
        for (int r = 0; r < 16 / NG; ++r) {
            float vals[NV];
#pragma unroll
            for (int i = 0; i < NV; ++i) vals[i] = part[r * NV + i];
            const float s = wave_reduce_v<NV>(vals, lane);
            const int v = lane >> (6 - LV);
            if ((lane & ((64 >> LV) - 1)) == 0) sc[v % GQA][wave * 16 + r * NG + v / GQA] = s * scale;
        }
    }
    __syncthreads();

    // ---- chunk-local softmax statistics; every wave computes them (cheap)
    float m[GQA], l[GQA], p[GQA];
#pragma unroll
    for (int h = 0; h < GQA; ++h) {
        const float s = (uint32_t)lane < cnt ? sc[h][lane] : kNegBig;
        float mm = s;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) mm = fmaxf(mm, __shfl_xor(mm, off, 64));
        const float e = (uint32_t)lane < cnt ? expf(s - mm) : 0.0f;
        float ll = e;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) ll += __shfl_xor(ll, off, 64);
        m[h] = mm;
        l[h] = ll;
        p[h] = e;
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int h = 0; h < GQA; ++h) sc[h][lane] = p[h];
    }
    __syncthreads();

    // ---- weighted V sum: wave w takes its 16 slots
    f4 acc[GQA][DV];
#pragma unroll
    for (int h = 0; h < GQA; ++h)
#pragma unroll
        for (int v = 0; v < DV; ++v) acc[h][v] = f4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const uint32_t li = wave * 16 + i;
        if (li < cnt) {
            const float *vr = Vc + (size_t)slots[base + i] * kv_dim + (size_t)kvh * D;
#pragma unroll
            for (int v = 0; v < DV; ++v) {
                const f4 vv = *(const f4 *)(vr + 4 * (lane + 64 * v));
#pragma unroll
                for (int h = 0; h < GQA; ++h) acc[h][v] += sc[h][li] * vv;
            }
        }
    }
#pragma unroll
    for (int h = 0; h < GQA; ++h)
#pragma unroll
        for (int v = 0; v < DV; ++v) pacc[wave][h][lane + 64 * v] = acc[h][v];
    __syncthreads();

    // ---- combine the four waves (fixed order) and write the partial
    float *wacc = ws;
    float *wm = ws + (size_t)nsplit * num_q_heads * D;
    float *wl = wm + (size_t)nsplit * num_q_heads;
    for (int idx = threadIdx.x; idx < GQA * DV * 64; idx += 256) {
        const int h = idx / (DV * 64), c = idx % (DV * 64);
        const f4 t = ((pacc[0][h][c] + pacc[1][h][c]) + pacc[2][h][c]) + pacc[3][h][c];
        const uint32_t qh = kvh * GQA + h;
        *(f4 *)(wacc + ((size_t)split * num_q_heads + qh) * D + 4 * c) = t;
    }
    if (threadIdx.x < GQA) {
        const uint32_t qh = kvh * GQA + threadIdx.x;
        wm[(size_t)split * num_q_heads + qh] = m[threadIdx.x];
        wl[(size_t)split * num_q_heads + qh] = l[threadIdx.x];
    }
}

// One workgroup per query head: merge the chunk partials.
__global__ __launch_bounds__(128) void k_attn_combine(const float *__restrict__ ws,
                                                      const uint32_t *__restrict__ n_slots, uint32_t max_slots,
                                                      uint32_t num_q_heads, uint32_t head_dim,
                                                      float *__restrict__ out) {
    const uint32_t qh = blockIdx.x;
    uint32_t S = *n_slots;
    if (S > max_slots) S = max_slots;
    const uint32_t nsplit_max = (max_slots + kAttnChunk - 1) / kAttnChunk;
    const uint32_t ns = (S + kAttnChunk - 1) / kAttnChunk;
    const float *wacc = ws;
    const float *wm = ws + (size_t)nsplit_max * num_q_heads * head_dim;
    const float *wl = wm + (size_t)nsplit_max * num_q_heads;
    float M = -1e9f;  // the reference's running-max seed
    for (uint32_t j = 0; j < ns; ++j) M = fmaxf(M, wm[(size_t)j * num_q_heads + qh]);
    float L = 0.0f;
    for (uint32_t j = 0; j < ns; ++j) L += expf(wm[(size_t)j * num_q_heads + qh] - M) * wl[(size_t)j * num_q_heads + qh];
    const float inv = 1.0f / (L + 1e-9f);
    for (uint32_t c = threadIdx.x; c < head_dim / 4; c += blockDim.x) {
        f4 t = f4{0, 0, 0, 0};
        for (uint32_t j = 0; j < ns; ++j) {
            const float w = expf(wm[(size_t)j * num_q_heads + qh] - M);
            t += w * *(const f4 *)(wacc + ((size_t)j * num_q_heads + qh) * head_dim + 4 * c);
        }
        *(f4 *)(out + (size_t)qh * head_dim + 4 * c) = t * inv;
    }
}

int launch_decode_attn(chn_ctx *ctx, const float *q, const float *kc, const float *vc, const uint32_t *slots,
                       const uint32_t *n_slots, uint32_t max_slots, uint32_t num_q_heads, uint32_t head_dim,
                       uint32_t kv_dim, uint32_t gqa, float scale, float *out, float *ws) {
    const uint32_t nsplit = (max_slots + kAttnChunk - 1) / kAttnChunk;
    const uint32_t num_kv = num_q_heads / gqa;
    dim3 grid(nsplit, num_kv);
    hipStream_t s = ctx->stream;
#define CHN_ATTN(DV, G) \
    k_attn_split<DV, G><<<grid, 256, 0, s>>>(q, kc, vc, slots, n_slots, max_slots, num_q_heads, kv_dim, scale, ws)
    if (head_dim == 256) {
        switch (gqa) {
        case 1: CHN_ATTN(1, 1); break;
        case 2: CHN_ATTN(1, 2); break;
        case 4: CHN_ATTN(1, 4); break;
        case 8: CHN_ATTN(1, 8); break;
        default: return set_err(ctx, CHN_E_UNSUPPORTED, "gqa ratio %u unsupported", gqa);
        }
    } else if (head_dim == 512) {
        switch (gqa) {
        case 1: CHN_ATTN(2, 1); break;
        case 2: CHN_ATTN(2, 2); break;
        case 4: CHN_ATTN(2, 4); break;
        default: return set_err(ctx, CHN_E_UNSUPPORTED, "gqa ratio %u unsupported at head_dim 512", gqa);
        }
    } else {
        return set_err(ctx, CHN_E_UNSUPPORTED, "head_dim %u unsupported (256 or 512)", head_dim);
    }
#undef CHN_ATTN
    CHN_LAUNCHED(ctx, "k_attn_split");
    k_attn_combine<<<num_q_heads, 128, 0, s>>>(ws, n_slots, max_slots, num_q_heads, head_dim, out);
    CHN_LAUNCHED(ctx, "k_attn_combine");
    return CHN_OK;
}

// ---------------------------------------------------------------------
// qkv_rope: one 64-lane workgroup per head.
// ---------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// RMSNorm * w, then RoPE on pairs (d, d + rot/2) at `clock`, suffix past
// rot copied (shaders/qkv_rope.wgsl:42-91).
__device__ void norm_rope_head(const float *__restrict__ in, const float *__restrict__ w, float *__restrict__ out,
                               uint32_t D, uint32_t rot, float theta, float eps, uint32_t clock, float *buf) {
    const int lane = threadIdx.x;
    float ss = 0.0f;
    for (uint32_t d = lane; d < D; d += 64) ss += in[d] * in[d];
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)D + eps);
    for (uint32_t d = lane; d < D; d += 64) buf[d] = (in[d] * inv) * w[d];
    __syncthreads();
    const uint32_t half = rot / 2;
    for (uint32_t d = lane; d < half; d += 64) {
        const float v0 = buf[d], v1 = buf[d + half];
        const float fe = (2.0f * (float)d) / (float)rot;
        const float freq = 1.0f / powf(theta, fe);
        const float ang = (float)clock * freq;
        const float c = cosf(ang), s = sinf(ang);
        out[d] = v0 * c - v1 * s;
        out[d + half] = v0 * s + v1 * c;
    }
    for (uint32_t d = rot + lane; d < D; d += 64) out[d] = buf[d];
}

__global__ __launch_bounds__(64) void k_qkv_rope(const float *__restrict__ q_in, const float *__restrict__ k_in,
                                                 const float *__restrict__ v_in, const float *__restrict__ qw,
                                                 const float *__restrict__ kw, float *__restrict__ q_out,
                                                 float *__restrict__ k_cache, float *__restrict__ v_cache,
                                                 const uint32_t *__restrict__ step, uint32_t num_q,
                                                 uint32_t num_kv, uint32_t D, uint32_t rot, int k_eq_v,
                                                 float theta, float eps) {
    __shared__ float buf[512];
    const uint32_t head = blockIdx.x;
    const uint32_t clock = step[0], slot = step[1];
    if (head < num_q) {
        norm_rope_head(q_in + (size_t)head * D, qw, q_out + (size_t)head * D, D, rot, theta, eps, clock, buf);
        return;
    }
    const uint32_t h = head - num_q;
    if (h >= num_kv) return;
    const size_t kv_dim = (size_t)num_kv * D;
    const float *k = k_in + (size_t)h * D;
    const float *v = k_eq_v ? k : v_in + (size_t)h * D;
    norm_rope_head(k, kw, k_cache + (size_t)slot * kv_dim + (size_t)h * D, D, rot, theta, eps, clock, buf);
    // V: unit RMSNorm (no weight)
    const int lane = threadIdx.x;
    float ss = 0.0f;
    for (uint32_t d = lane; d < D; d += 64) ss += v[d] * v[d];
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)D + eps);
    float *vo = v_cache + (size_t)slot * kv_dim + (size_t)h * D;
    for (uint32_t d = lane; d < D; d += 64) vo[d] = v[d] * inv;
}

}  // namespace chn

using namespace chn;

extern "C" int chn_qkv_rope(chn_ctx *ctx, const float *q_in, const float *k_in, const float *v_in,
                            const float *q_norm_w, const float *k_norm_w, float *q_out, float *k_cache,
                            float *v_cache, const uint32_t *step_params, uint32_t num_q_heads,
                            uint32_t num_kv_heads, uint32_t head_dim, uint32_t rotary_dim, int k_eq_v,
                            float theta, float eps) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, q_in && k_in && (v_in || k_eq_v) && q_norm_w && k_norm_w && q_out && k_cache && v_cache &&
                    step_params, "NULL argument");
    CHN_REQUIRE(ctx, head_dim > 0 && head_dim <= 512, "head_dim %u must be in 1..512", head_dim);
    CHN_REQUIRE(ctx, rotary_dim <= head_dim && rotary_dim % 2 == 0, "rotary_dim %u must be even and <= head_dim",
                rotary_dim);
    const uint32_t nh = num_q_heads + num_kv_heads;
    if (!nh) return CHN_OK;
    k_qkv_rope<<<nh, 64, 0, ctx->stream>>>(q_in, k_in, v_in, q_norm_w, k_norm_w, q_out, k_cache, v_cache,
                                           step_params, num_q_heads, num_kv_heads, head_dim, rotary_dim, k_eq_v,
                                           theta, eps);
    CHN_LAUNCHED(ctx, "k_qkv_rope");
    return CHN_OK;
}

extern "C" int chn_decode_attn(chn_ctx *ctx, const float *q, const float *k_cache, const float *v_cache,
                               const uint32_t *slots, const uint32_t *n_slots, uint32_t max_slots,
                               uint32_t num_q_heads, uint32_t head_dim, uint32_t kv_dim, uint32_t gqa_ratio,
                               float scale, float *out) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, q && k_cache && v_cache && slots && n_slots && out, "NULL argument");
    CHN_REQUIRE(ctx, gqa_ratio > 0 && num_q_heads % gqa_ratio == 0, "num_q_heads %u not a multiple of gqa %u",
                num_q_heads, gqa_ratio);
    CHN_REQUIRE(ctx, kv_dim >= (num_q_heads / gqa_ratio) * head_dim && kv_dim % 4 == 0,
                "kv_dim %u too small for %u kv heads of %u", kv_dim, num_q_heads / gqa_ratio, head_dim);
    CHN_REQUIRE(ctx, aligned(q, 16) && aligned(k_cache, 16) && aligned(v_cache, 16) && aligned(out, 16),
                "q, caches and out must be 16-byte aligned");
    CHN_REQUIRE(ctx, max_slots > 0, "max_slots must be > 0");
    if (!num_q_heads) return CHN_OK;
    int rc = ensure_workspace(ctx, attn_ws_bytes(num_q_heads, head_dim, max_slots));
    if (rc) return rc;
    return launch_decode_attn(ctx, q, k_cache, v_cache, slots, n_slots, max_slots, num_q_heads, head_dim,
                              kv_dim, gqa_ratio, scale, out, (float *)ctx->ws);
}
