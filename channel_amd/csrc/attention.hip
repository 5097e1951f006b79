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

size_t attn_ws_bytes(uint32_t num_q_heads, uint32_t head_dim, uint32_t max_slots) {
    const size_t nsplit = (max_slots + kAttnChunk - 1) / kAttnChunk;
    return nsplit * num_q_heads * ((size_t)head_dim + 2) * 4;
}

// Sum over the 16 lanes of each DPP row; every lane of the row gets the sum.
__device__ __forceinline__ float row16_sum(float v) {
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true)); // quad_perm [1,0,3,2]
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true)); // quad_perm [2,3,0,1]
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x124, 0xF, 0xF, true)); // row_ror:4
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xF, 0xF, true)); // row_ror:8
    return v;
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x124, 0xF, 0xF, true)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xF, 0xF, true)));
    return v;
}
// Whole-wave sum / max: row reductions, then the four row results.
__device__ __forceinline__ float wave_sum64(float v) {
    v = row16_sum(v);
    return (__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16))) +
           (__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32)) +
            __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48)));
}
__device__ __forceinline__ float wave_max64(float v) {
    v = row16_max(v);
    return fmaxf(fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0)),
                       __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16))),
                 fmaxf(__builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32)),
                       __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48))));
}

// Running softmax state of one lane: lane row r = lane / 16 holds slots
// r, r+4, r+8, r+12 of each wave's 16, column c = lane % 16 holds 16*DV
// consecutive dims, so one slot's row (1 KB at D = 256) is read by a
// 16-lane row as 64 contiguous bytes per lane and its score reduces inside
// the row with DPP.
template <int DV, int GQA>
struct AttnState {
    float M[GQA], l[GQA];
    f4 acc[GQA][4 * DV];
};

// One 64-slot chunk [c0, c0 + cnt) of the list for KV head kvh: scores,
// running max / sum update (rescaling the accumulators), p-weighted V.
template <int DV, int GQA>
__device__ __forceinline__ void attn_chunk(AttnState<DV, GQA> &st, const f4 (&q)[GQA][4 * DV],
                                           const float *__restrict__ Kc, const float *__restrict__ Vc,
                                           const uint32_t *__restrict__ slots, uint32_t c0, uint32_t cnt,
                                           uint32_t kv_dim, uint32_t kvh, float scale, float (&sc)[GQA][kAttnChunk]) {
    constexpr int D = DV * 256;
    constexpr int NF = 4 * DV;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane >> 4, c = lane & 15;
    const uint32_t base = c0 + wave * 16;
    const uint32_t nval = cnt > (uint32_t)(wave * 16) ? cnt - wave * 16 : 0;
    const uint32_t my_slot = (uint32_t)lane < nval && lane < 16 ? slots[base + lane] : 0u;
    const size_t dim0 = (size_t)kvh * D + (size_t)c * NF * 4;

    f4 kr[4][NF], vr[4][NF];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = r + 4 * u;
        const uint32_t ps = (uint32_t)__shfl(my_slot, i, 64);
        const bool ok = (uint32_t)i < nval;
        const float *kp = Kc + (size_t)ps * kv_dim + dim0;
#pragma unroll
        for (int f = 0; f < NF; ++f) kr[u][f] = ok ? *(const f4 *)(kp + 4 * f) : f4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = r + 4 * u;
        const uint32_t ps = (uint32_t)__shfl(my_slot, i, 64);
        const bool ok = (uint32_t)i < nval;
        const float *vp = Vc + (size_t)ps * kv_dim + dim0;
#pragma unroll
        for (int f = 0; f < NF; ++f) vr[u][f] = ok ? *(const f4 *)(vp + 4 * f) : f4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int h = 0; h < GQA; ++h) {
            float d = 0.0f;
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                d = fmaf(q[h][f].x, kr[u][f].x, d);
                d = fmaf(q[h][f].y, kr[u][f].y, d);
                d = fmaf(q[h][f].z, kr[u][f].z, d);
                d = fmaf(q[h][f].w, kr[u][f].w, d);
            }
            d = row16_sum(d);
            if (c == 0) sc[h][wave * 16 + r + 4 * u] = d * scale;
        }
    __syncthreads();
    float p[GQA];
#pragma unroll
    for (int h = 0; h < GQA; ++h) {
        const float sv = (uint32_t)lane < cnt ? sc[h][lane] : kNegBig;
        const float Mn = fmaxf(st.M[h], wave_max64(sv));
        const float e = (uint32_t)lane < cnt ? expf(sv - Mn) : 0.0f;
        const float rs = expf(st.M[h] - Mn);
        st.l[h] = st.l[h] * rs + wave_sum64(e);
#pragma unroll
        for (int f = 0; f < NF; ++f) st.acc[h][f] *= rs;
        st.M[h] = Mn;
        p[h] = e;
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int h = 0; h < GQA; ++h) sc[h][lane] = p[h];
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = r + 4 * u;
        if ((uint32_t)i < nval) {
#pragma unroll
            for (int h = 0; h < GQA; ++h) {
                const float pw = sc[h][wave * 16 + i];
#pragma unroll
                for (int f = 0; f < NF; ++f) st.acc[h][f] += pw * vr[u][f];
            }
        }
    }
    __syncthreads();   // sc is rewritten by the next chunk
}

// Sum the 16 (wave, row) partial accumulators of each head in a fixed order
// and hand each finished float4 column to `emit(head, column, value)`.
template <int DV, int GQA, typename Emit>
__device__ __forceinline__ void attn_reduce(const AttnState<DV, GQA> &st, f4 (*pacc)[GQA < 2 ? GQA : 2][64 * DV],
                                            Emit emit) {
    constexpr int NF = 4 * DV;
    constexpr int HC = GQA < 2 ? GQA : 2;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane >> 4, c = lane & 15;
#pragma unroll
    for (int h0 = 0; h0 < GQA; h0 += HC) {
#pragma unroll
        for (int hh = 0; hh < HC; ++hh)
#pragma unroll
            for (int f = 0; f < NF; ++f) pacc[wave * 4 + r][hh][c * NF + f] = st.acc[h0 + hh][f];
        __syncthreads();
        for (int idx = threadIdx.x; idx < HC * 16 * NF; idx += 256) {
            const int hh = idx / (16 * NF), col = idx % (16 * NF);
            f4 t = pacc[0][hh][col];
#pragma unroll
            for (int j = 1; j < 16; ++j) t += pacc[j][hh][col];
            emit(h0 + hh, col, t);
        }
        __syncthreads();
    }
}

template <int DV, int GQA>
__device__ __forceinline__ void load_q(f4 (&q)[GQA][4 * DV], const float *__restrict__ Q, uint32_t qh0) {
    constexpr int D = DV * 256;
    const int c = threadIdx.x & 15;
#pragma unroll
    for (int h = 0; h < GQA; ++h)
#pragma unroll
        for (int f = 0; f < 4 * DV; ++f) q[h][f] = *(const f4 *)(Q + (size_t)(qh0 + h) * D + c * 16 * DV + 4 * f);
}

// Decode: one workgroup per (64-slot chunk, KV head) writes a partial
// (m, l, sum p*V) per query head: acc [nsplit][num_q_heads][D], then m and l.
template <int DV, int GQA>
__global__ __launch_bounds__(256) void k_attn_split(const float *__restrict__ Q, const float *__restrict__ Kc,
                                                    const float *__restrict__ Vc,
                                                    const uint32_t *__restrict__ slots,
                                                    const uint32_t *__restrict__ n_slots, uint32_t max_slots,
                                                    uint32_t num_q_heads, uint32_t kv_dim, float scale,
                                                    float *__restrict__ ws) {
    constexpr int D = DV * 256;
    const uint32_t split = blockIdx.x, kvh = blockIdx.y;
    uint32_t S = *n_slots;
    if (S > max_slots) S = max_slots;
    const uint32_t s0 = split * kAttnChunk;
    if (s0 >= S) return;
    const uint32_t cnt = (S - s0 < (uint32_t)kAttnChunk) ? S - s0 : kAttnChunk;
    const uint32_t nsplit = (max_slots + kAttnChunk - 1) / kAttnChunk;
    __shared__ float sc[GQA][kAttnChunk];
    __shared__ f4 pacc[16][GQA < 2 ? GQA : 2][64 * DV];

    f4 q[GQA][4 * DV];
    load_q<DV, GQA>(q, Q, kvh * GQA);
    AttnState<DV, GQA> st;
#pragma unroll
    for (int h = 0; h < GQA; ++h) {
        st.M[h] = -1e9f;
        st.l[h] = 0.0f;
#pragma unroll
        for (int f = 0; f < 4 * DV; ++f) st.acc[h][f] = f4{0, 0, 0, 0};
    }
    attn_chunk<DV, GQA>(st, q, Kc, Vc, slots, s0, cnt, kv_dim, kvh, scale, sc);
    float *wacc = ws;
    float *wm = ws + (size_t)nsplit * num_q_heads * D;
    float *wl = wm + (size_t)nsplit * num_q_heads;
    attn_reduce<DV, GQA>(st, pacc, [&](int h, int col, f4 t) {
        *(f4 *)(wacc + ((size_t)split * num_q_heads + kvh * GQA + h) * D + 4 * col) = t;
    });
    if (threadIdx.x < GQA) {
        const uint32_t qh = kvh * GQA + threadIdx.x;
        wm[(size_t)split * num_q_heads + qh] = st.M[threadIdx.x];
        wl[(size_t)split * num_q_heads + qh] = st.l[threadIdx.x];
    }
}

// Prefill (shaders/batch_causal_attn.wgsl): one workgroup per (token, KV
// head) walks slots [start, prev + t + 1) of the list in 64-slot chunks with
// an online softmax; start = S - window for window > 0 and S > window.
template <int DV, int GQA>
__global__ __launch_bounds__(256) void k_prefill_attn(const float *__restrict__ Q, const float *__restrict__ Kc,
                                                      const float *__restrict__ Vc,
                                                      const uint32_t *__restrict__ slots, uint32_t num_prev,
                                                      uint32_t num_q_heads, uint32_t kv_dim, float scale,
                                                      uint32_t window, float *__restrict__ out) {
    constexpr int D = DV * 256;
    const uint32_t t = blockIdx.x, kvh = blockIdx.y;
    const uint32_t S = num_prev + t + 1;
    const uint32_t start = (window > 0 && S > window) ? S - window : 0;
    __shared__ float sc[GQA][kAttnChunk];
    __shared__ f4 pacc[16][GQA < 2 ? GQA : 2][64 * DV];
    const size_t q_row = (size_t)t * num_q_heads * D;
    f4 q[GQA][4 * DV];
    load_q<DV, GQA>(q, Q + q_row, kvh * GQA);
    AttnState<DV, GQA> st;
#pragma unroll
    for (int h = 0; h < GQA; ++h) {
        st.M[h] = -1e9f;
        st.l[h] = 0.0f;
#pragma unroll
        for (int f = 0; f < 4 * DV; ++f) st.acc[h][f] = f4{0, 0, 0, 0};
    }
    for (uint32_t c0 = start; c0 < S; c0 += kAttnChunk) {
        const uint32_t cnt = (S - c0 < (uint32_t)kAttnChunk) ? S - c0 : kAttnChunk;
        attn_chunk<DV, GQA>(st, q, Kc, Vc, slots, c0, cnt, kv_dim, kvh, scale, sc);
    }
    float inv[GQA];
#pragma unroll
    for (int h = 0; h < GQA; ++h) inv[h] = 1.0f / (st.l[h] + 1e-9f);
    attn_reduce<DV, GQA>(st, pacc, [&](int h, int col, f4 v) {
        *(f4 *)(out + q_row + (size_t)(kvh * GQA + h) * D + 4 * col) = v * inv[h];
    });
}

// One 256-thread workgroup per query head merges the chunk partials: chunk
// weights exp(m_j - M) are computed once, then wave w sums chunks
// j = w, w + 4, ... for every column with loads batched four at a time, and
// the four wave sums are added in a fixed order.
__global__ __launch_bounds__(256) void k_attn_combine(const float *__restrict__ ws,
                                                      const uint32_t *__restrict__ n_slots, uint32_t max_slots,
                                                      uint32_t num_q_heads, uint32_t head_dim,
                                                      float *__restrict__ out) {
    __shared__ float ew[64];
    __shared__ float sinv;
    __shared__ f4 part[4][128];
    const uint32_t qh = blockIdx.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    uint32_t S = *n_slots;
    if (S > max_slots) S = max_slots;
    const uint32_t nsplit_max = (max_slots + kAttnChunk - 1) / kAttnChunk;
    const uint32_t ns = (S + kAttnChunk - 1) / kAttnChunk;     // <= 64
    const float *wacc = ws;
    const float *wm = ws + (size_t)nsplit_max * num_q_heads * head_dim;
    const float *wl = wm + (size_t)nsplit_max * num_q_heads;
    if (wave == 0) {
        const float mj = (uint32_t)lane < ns ? wm[(size_t)lane * num_q_heads + qh] : -1e9f;
        float M = mj;  // seeded at the reference's -1e9 by the padding lanes / the max below
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
        M = fmaxf(M, -1e9f);
        const float e = (uint32_t)lane < ns ? expf(mj - M) : 0.0f;
        float L = (uint32_t)lane < ns ? e * wl[(size_t)lane * num_q_heads + qh] : 0.0f;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) L += __shfl_xor(L, off, 64);
        ew[lane] = e;
        if (lane == 0) sinv = 1.0f / (L + 1e-9f);
    }
    __syncthreads();
    const uint32_t ncol = head_dim / 4;          // float4 columns, <= 128
    for (uint32_t c = lane; c < ncol; c += 64) {
        f4 t = f4{0, 0, 0, 0};
        uint32_t j = wave;
        for (; j + 12 < ns; j += 16) {
            f4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u)
                v[u] = *(const f4 *)(wacc + ((size_t)(j + 4 * u) * num_q_heads + qh) * head_dim + 4 * c);
#pragma unroll
            for (int u = 0; u < 4; ++u) t += ew[j + 4 * u] * v[u];
        }
        for (; j < ns; j += 4) t += ew[j] * *(const f4 *)(wacc + ((size_t)j * num_q_heads + qh) * head_dim + 4 * c);
        part[wave][c] = t;
    }
    __syncthreads();
    for (uint32_t c = threadIdx.x; c < ncol; c += 256)
        *(f4 *)(out + (size_t)qh * head_dim + 4 * c) = (((part[0][c] + part[1][c]) + part[2][c]) + part[3][c]) * sinv;
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
    k_attn_combine<<<num_q_heads, 256, 0, s>>>(ws, n_slots, max_slots, num_q_heads, head_dim, out);
    CHN_LAUNCHED(ctx, "k_attn_combine");
    return CHN_OK;
}

int launch_prefill_attn(hipStream_t st, const float *q, const float *kc, const float *vc, const uint32_t *slots,
                        uint32_t n_tok, uint32_t num_prev, uint32_t num_q_heads, uint32_t head_dim, uint32_t kv_dim,
                        uint32_t gqa, float scale, uint32_t window, float *out) {
    dim3 grid(n_tok, num_q_heads / gqa);
#define CHN_PATTN(DV, G) \
    k_prefill_attn<DV, G><<<grid, 256, 0, st>>>(q, kc, vc, slots, num_prev, num_q_heads, kv_dim, scale, window, out)
    if (head_dim == 256) {
        switch (gqa) {
        case 1: CHN_PATTN(1, 1); break;
        case 2: CHN_PATTN(1, 2); break;
        case 4: CHN_PATTN(1, 4); break;
        case 8: CHN_PATTN(1, 8); break;
        default: return CHN_E_UNSUPPORTED;
        }
    } else if (head_dim == 512) {
        switch (gqa) {
        case 1: CHN_PATTN(2, 1); break;
        case 2: CHN_PATTN(2, 2); break;
        case 4: CHN_PATTN(2, 4); break;
        default: return CHN_E_UNSUPPORTED;
        }
    } else {
        return CHN_E_UNSUPPORTED;
    }
#undef CHN_PATTN
    return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
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

// batch_qkv_rope (shaders/batch_qkv_rope.wgsl): token t uses clock
// start_clock + t and writes its K/V at slot slots[slot_offset + t].
__global__ __launch_bounds__(64) void k_batch_qkv_rope(const float *__restrict__ q_in, const float *__restrict__ k_in,
                                                       const float *__restrict__ v_in, const float *__restrict__ qw,
                                                       const float *__restrict__ kw, float *__restrict__ q_out,
                                                       float *__restrict__ k_cache, float *__restrict__ v_cache,
                                                       const uint32_t *__restrict__ slots, uint32_t slot_offset,
                                                       uint32_t start_clock, uint32_t num_q, uint32_t num_kv,
                                                       uint32_t D, uint32_t rot, int k_eq_v, float theta, float eps) {
    __shared__ float buf[512];
    const uint32_t head = blockIdx.x, t = blockIdx.y;
    const uint32_t clock = start_clock + t, slot = slots[slot_offset + t];
    const size_t q_dim = (size_t)num_q * D, kv_dim = (size_t)num_kv * D;
    if (head < num_q) {
        norm_rope_head(q_in + t * q_dim + (size_t)head * D, qw, q_out + t * q_dim + (size_t)head * D, D, rot, theta,
                       eps, clock, buf);
        return;
    }
    const uint32_t h = head - num_q;
    if (h >= num_kv) return;
    const float *k = k_in + t * kv_dim + (size_t)h * D;
    const float *v = k_eq_v ? k : v_in + t * kv_dim + (size_t)h * D;
    norm_rope_head(k, kw, k_cache + (size_t)slot * kv_dim + (size_t)h * D, D, rot, theta, eps, clock, buf);
    const int lane = threadIdx.x;
    float ss = 0.0f;
    for (uint32_t d = lane; d < D; d += 64) ss += v[d] * v[d];
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)D + eps);
    float *vo = v_cache + (size_t)slot * kv_dim + (size_t)h * D;
    for (uint32_t d = lane; d < D; d += 64) vo[d] = v[d] * inv;
}

int launch_qkv_rope(hipStream_t st, const float *q_in, const float *k_in, const float *v_in, const float *qw,
                    const float *kw, float *q_out, float *kc, float *vc, const uint32_t *step, uint32_t num_q,
                    uint32_t num_kv, uint32_t D, uint32_t rot, int k_eq_v, float theta, float eps) {
    k_qkv_rope<<<num_q + num_kv, 64, 0, st>>>(q_in, k_in, v_in, qw, kw, q_out, kc, vc, step, num_q, num_kv, D, rot,
                                              k_eq_v, theta, eps);
    return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
}

int launch_batch_qkv_rope(hipStream_t st, const float *q_in, const float *k_in, const float *v_in, const float *qw,
                          const float *kw, float *q_out, float *kc, float *vc, const uint32_t *slots,
                          uint32_t slot_offset, uint32_t start_clock, uint32_t n_tok, uint32_t num_q, uint32_t num_kv,
                          uint32_t D, uint32_t rot, int k_eq_v, float theta, float eps) {
    dim3 grid(num_q + num_kv, n_tok);
    k_batch_qkv_rope<<<grid, 64, 0, st>>>(q_in, k_in, v_in, qw, kw, q_out, kc, vc, slots, slot_offset, start_clock,
                                          num_q, num_kv, D, rot, k_eq_v, theta, eps);
    return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
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
    launch_qkv_rope(ctx->stream, q_in, k_in, v_in, q_norm_w, k_norm_w, q_out, k_cache, v_cache, step_params,
                    num_q_heads, num_kv_heads, head_dim, rotary_dim, k_eq_v, theta, eps);
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
    CHN_REQUIRE(ctx, max_slots > 0 && max_slots <= 4096, "max_slots %u must be in 1..4096", max_slots);
    if (!num_q_heads) return CHN_OK;
    int rc = ensure_workspace(ctx, attn_ws_bytes(num_q_heads, head_dim, max_slots));
    if (rc) return rc;
    return launch_decode_attn(ctx, q, k_cache, v_cache, slots, n_slots, max_slots, num_q_heads, head_dim,
                              kv_dim, gqa_ratio, scale, out, (float *)ctx->ws);
}

extern "C" int chn_batch_qkv_rope(chn_ctx *ctx, const float *q_in, const float *k_in, const float *v_in,
                                  const float *q_norm_w, const float *k_norm_w, float *q_out, float *k_cache,
                                  float *v_cache, const uint32_t *slots, uint32_t slot_offset, uint32_t start_clock,
                                  uint32_t n_tok, uint32_t num_q_heads, uint32_t num_kv_heads, uint32_t head_dim,
                                  uint32_t rotary_dim, int k_eq_v, float theta, float eps) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, q_in && k_in && (v_in || k_eq_v) && q_norm_w && k_norm_w && q_out && k_cache && v_cache && slots,
                "NULL argument");
    CHN_REQUIRE(ctx, head_dim > 0 && head_dim <= 512, "head_dim %u must be in 1..512", head_dim);
    CHN_REQUIRE(ctx, rotary_dim <= head_dim && rotary_dim % 2 == 0, "rotary_dim %u must be even and <= head_dim",
                rotary_dim);
    if (!n_tok || !(num_q_heads + num_kv_heads)) return CHN_OK;
    launch_batch_qkv_rope(ctx->stream, q_in, k_in, v_in, q_norm_w, k_norm_w, q_out, k_cache, v_cache, slots,
                          slot_offset, start_clock, n_tok, num_q_heads, num_kv_heads, head_dim, rotary_dim, k_eq_v,
                          theta, eps);
    CHN_LAUNCHED(ctx, "k_batch_qkv_rope");
    return CHN_OK;
}

extern "C" int chn_batch_causal_attn(chn_ctx *ctx, const float *q, const float *k_cache, const float *v_cache,
                                     const uint32_t *slots, uint32_t n_tok, uint32_t num_prev_slots,
                                     uint32_t num_q_heads, uint32_t head_dim, uint32_t kv_dim, uint32_t gqa_ratio,
                                     float scale, uint32_t window, float *out) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, q && k_cache && v_cache && slots && out, "NULL argument");
    CHN_REQUIRE(ctx, gqa_ratio > 0 && num_q_heads % gqa_ratio == 0, "num_q_heads %u not a multiple of gqa %u",
                num_q_heads, gqa_ratio);
    CHN_REQUIRE(ctx, kv_dim >= (num_q_heads / gqa_ratio) * head_dim && kv_dim % 4 == 0, "kv_dim %u too small", kv_dim);
    CHN_REQUIRE(ctx, aligned(q, 16) && aligned(k_cache, 16) && aligned(v_cache, 16) && aligned(out, 16),
                "q, caches and out must be 16-byte aligned");
    if (!n_tok || !num_q_heads) return CHN_OK;
    int rc = launch_prefill_attn(ctx->stream, q, k_cache, v_cache, slots, n_tok, num_prev_slots, num_q_heads, head_dim,
                                 kv_dim, gqa_ratio, scale, window, out);
    if (rc == CHN_E_UNSUPPORTED)
        return set_err(ctx, rc, "head_dim %u / gqa %u unsupported", head_dim, gqa_ratio);
    CHN_LAUNCHED(ctx, "k_prefill_attn");
    return CHN_OK;
}
