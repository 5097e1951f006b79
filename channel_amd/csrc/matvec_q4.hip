// Batch-1 decode matvecs over the reference's Q4 layout on gfx950:
// gemv_q4 (shaders/gemv_q4.wgsl), fused_qkv_q4 (shaders/fused_qkv_q4.wgsl)
// and fused_mlp_q4 (shaders/fused_mlp_q4.wgsl).
//
// Design (HBM-bound, no MFMA):
//  * lane <-> one 32-weight block: a wave covers 64 consecutive blocks of
//    a row, so the wave's weight loads are one contiguous run of 64*20
//    bytes (one dwordx4 + one dword per lane, dword-aligned);
//  * the lane keeps its 32 activations in registers and reuses them for
//    RPW rows (and for the gate and up matrices), so x is read once per
//    RPW rows instead of once per row;
//  * the dot uses sum (q-8)x = sum q*x - 8*sum x per block: a nibble word
//    is masked twice (low / high nibbles of each byte) and each byte goes
//    through v_cvt_f32_ubyteN, i.e. ~2.3 VALU ops per weight; the high
//    nibbles come out multiplied by 16, so the odd-position activations are
//    pre-scaled by 1/16 (an exact power-of-two scaling);
//  * WPR waves of a workgroup split the column passes of the same rows
//    (split-K inside the workgroup), and the partial sums are reduced
//    through LDS in a fixed order, so results are deterministic.
#include "chn_internal.h"

namespace chn {

enum MatvecMode { MV_GEMV = 0, MV_QKV = 1, MV_MLP = 2 };

struct MatvecArgs {
    const uint32_t *W0, *W1, *W2;  // GEMV: W0. QKV: Wq, Wk, Wv. MLP: Wg, Wu.
    float *y0, *y1, *y2;           // GEMV: y0. QKV: q, k, v. MLP: act.
    const float *x;
    uint32_t M;                    // output rows (QKV: q_dim + 2 kv_dim)
    uint32_t seg1, seg2;           // QKV: q_dim, q_dim + kv_dim
    uint32_t nb;                   // K / 32
};

template <int MODE>
__device__ __forceinline__ const uint32_t *row_base(const MatvecArgs &a, uint32_t row, int mat) {
    const size_t rw = (size_t)a.nb * 5;
    if (MODE == MV_QKV) {
        if (row < a.seg1) return a.W0 + (size_t)row * rw;
        if (row < a.seg2) return a.W1 + (size_t)(row - a.seg1) * rw;
        return a.W2 + (size_t)(row - a.seg2) * rw;
    }
    if (MODE == MV_MLP && mat == 1) return a.W1 + (size_t)row * rw;
    return a.W0 + (size_t)row * rw;
}

__device__ __forceinline__ float ub(uint32_t v, int j) {
    return (float)((v >> (8 * j)) & 0xffu);
}

// sum_{i<32} q_i * x_i for one block, x split into even positions (xe) and
// odd positions pre-divided by 16 (xo).
__device__ __forceinline__ float block_dot(const u32x4_a4 q, const float *xe, const float *xo) {
    float d = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t lo = opaque_u32(q[w] & 0x0F0F0F0Fu);
        const uint32_t hi = opaque_u32(q[w] & 0xF0F0F0F0u);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            d = fmaf(ub(lo, j), xe[4 * w + j], d);
            d = fmaf(ub(hi, j), xo[4 * w + j], d);
        }
    }
    return d;
}

template <int MODE, int RPW, int WPR>
__global__ __launch_bounds__(256) void k_matvec_q4(MatvecArgs a) {
    constexpr int NMAT = (MODE == MV_MLP) ? 2 : 1;
    constexpr int V = RPW * NMAT;     // dot products per lane
    constexpr int G = 4 / WPR;        // row groups per workgroup
    constexpr int NOUT = G * V;
    constexpr int TPO = 256 / NOUT;   // threads per output in the reduction
    static_assert(NOUT >= 4 && TPO <= 64, "reduction needs >= 4 outputs per workgroup");

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int grp = wave / WPR, part = wave % WPR;
    const uint32_t row0 = (blockIdx.x * G + grp) * RPW;
    const uint32_t nb = a.nb;

    const uint32_t *rp[V];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            const uint32_t row = row0 + r;
            rp[r * NMAT + m] = row_base<MODE>(a, row < a.M ? row : 0, m);
        }

    float acc[V];
#pragma unroll
    for (int v = 0; v < V; ++v) acc[v] = 0.0f;

    for (uint32_t c = part; c * 64 < nb; c += WPR) {
        const uint32_t b = c * 64 + lane;
        if (b < nb) {
            uint32_t w0[V];
            u32x4_a4 q[V];
#pragma unroll
            for (int v = 0; v < V; ++v) {
                if (row0 + v / NMAT < a.M) {
                    const uint32_t *p = rp[v] + (size_t)b * 5;
                    w0[v] = p[0];
                    q[v] = *(const u32x4_a4 *)(p + 1);
                } else {
                    w0[v] = 0;
                    q[v] = u32x4_a4{0u, 0u, 0u, 0u};
                }
            }
            const float4 *xv = (const float4 *)(a.x + (size_t)b * 32);
            float xe[16], xo[16];
            float sx = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float4 t = xv[j];
                sx += (t.x + t.y) + (t.z + t.w);
                // word w = j/2 covers x[8w..8w+7]; even/odd positions
                xe[2 * j + 0] = t.x;
                xe[2 * j + 1] = t.z;
                xo[2 * j + 0] = t.y * 0.0625f;
                xo[2 * j + 1] = t.w * 0.0625f;
            }
#pragma unroll
            for (int v = 0; v < V; ++v) {
                const float d = block_dot(q[v], xe, xo);
                acc[v] = fmaf(f16_lo_to_f32(w0[v]), fmaf(-8.0f, sx, d), acc[v]);
            }
        }
    }

    // ---- fixed-order reduction: [v][wave][lane] in LDS ----------------
    __shared__ float red[V * 4 * 64];
    __shared__ float outv[NOUT];
#pragma unroll
    for (int v = 0; v < V; ++v) red[(v * 4 + wave) * 64 + lane] = acc[v];
    __syncthreads();
    {
        const int t = threadIdx.x;
        const int o = t / TPO, sub = t % TPO;
        const int g = o / V, v = o % V;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < V; ++i) {  // WPR*64 partials / TPO threads == V
            const int p = sub + i * TPO;
            s += red[(v * 4 + g * WPR + (p >> 6)) * 64 + (p & 63)];
        }
#pragma unroll
        for (int off = TPO / 2; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
        if (sub == 0) outv[o] = s;
    }
    __syncthreads();
    if (threadIdx.x < G * RPW) {
        const int g = threadIdx.x / RPW, r = threadIdx.x % RPW;
        const uint32_t row = (blockIdx.x * G + g) * RPW + r;
        if (row < a.M) {
            const float v0 = outv[g * V + r * NMAT];
            if (MODE == MV_GEMV) {
                a.y0[row] = v0;
            } else if (MODE == MV_QKV) {
                if (row < a.seg1) a.y0[row] = v0;
                else if (row < a.seg2) a.y1[row - a.seg1] = v0;
                else a.y2[row - a.seg2] = v0;
            } else {
                a.y0[row] = gelu_tanh(v0) * outv[g * V + r * NMAT + 1];
            }
        }
    }
}

template <int MODE, int RPW, int WPR>
static void launch_one(const MatvecArgs &a, uint32_t grid, hipStream_t s) {
    k_matvec_q4<MODE, RPW, WPR><<<dim3(grid), dim3(256), 0, s>>>(a);
}

template <int MODE, int WPR>
static bool launch_rpw(int rpw, const MatvecArgs &a, uint32_t grid, hipStream_t s) {
    constexpr int NMAT = (MODE == MV_MLP) ? 2 : 1;
    constexpr int G = 4 / WPR;
    switch (rpw) {
    case 1:
        if constexpr (G * 1 * NMAT >= 4) { launch_one<MODE, 1, WPR>(a, grid, s); return true; }
        return false;
    case 2:
        if constexpr (G * 2 * NMAT >= 4) { launch_one<MODE, 2, WPR>(a, grid, s); return true; }
        return false;
    case 4:
        launch_one<MODE, 4, WPR>(a, grid, s);
        return true;
    case 8:
        if constexpr (NMAT == 1) { launch_one<MODE, 8, WPR>(a, grid, s); return true; }
        return false;
    }
    return false;
}

// Picks the launch shape: WPR waves split the column passes of a row group
// when a row has several 64-block passes; RPW (rows per wave) is the
// largest that still puts >= 3072 waves on the 1024 SIMDs.
int launch_matvec(chn_ctx *ctx, int mode, const MatvecArgs &a) {
    const uint32_t passes = (a.nb + 63) / 64;
    const int wpr = passes >= 4 ? 4 : (passes >= 2 ? 2 : 1);
    const int G = 4 / wpr;
    const int nmat = (mode == MV_MLP) ? 2 : 1;
    int rpw = 0;
    const int cands[4] = {8, 4, 2, 1};
    for (int i = 0; i < 4; ++i) {
        const int r = cands[i];
        if (r * nmat > 8) continue;
        if (G * r * nmat < 4) continue;
        const uint64_t waves = (uint64_t)((a.M + G * r - 1) / (G * r)) * 4;
        if (waves >= 3072) { rpw = r; break; }
    }
    if (!rpw) {  // small problem: smallest legal tile
        for (int i = 3; i >= 0; --i) {
            const int r = cands[i];
            if (r * nmat <= 8 && G * r * nmat >= 4) { rpw = r; break; }
        }
    }
    const uint32_t grid = (a.M + G * rpw - 1) / (G * rpw);
    bool ok = false;
    hipStream_t s = ctx->stream;
    switch (mode) {
    case MV_GEMV:
        ok = wpr == 1 ? launch_rpw<MV_GEMV, 1>(rpw, a, grid, s)
           : wpr == 2 ? launch_rpw<MV_GEMV, 2>(rpw, a, grid, s)
                      : launch_rpw<MV_GEMV, 4>(rpw, a, grid, s);
        break;
    case MV_QKV:
        ok = wpr == 1 ? launch_rpw<MV_QKV, 1>(rpw, a, grid, s)
           : wpr == 2 ? launch_rpw<MV_QKV, 2>(rpw, a, grid, s)
                      : launch_rpw<MV_QKV, 4>(rpw, a, grid, s);
        break;
    default:
        ok = wpr == 1 ? launch_rpw<MV_MLP, 1>(rpw, a, grid, s)
           : wpr == 2 ? launch_rpw<MV_MLP, 2>(rpw, a, grid, s)
                      : launch_rpw<MV_MLP, 4>(rpw, a, grid, s);
        break;
    }
    if (!ok) return set_err(ctx, CHN_E_UNSUPPORTED, "no matvec tile for M=%u nb=%u", a.M, a.nb);
    CHN_LAUNCHED(ctx, "k_matvec_q4");
    return CHN_OK;
}

static int check_common(chn_ctx *ctx, const float *x, uint32_t K) {
    CHN_REQUIRE(ctx, K > 0 && K % 32 == 0, "K=%u must be a positive multiple of 32", K);
    CHN_REQUIRE(ctx, x && aligned(x, 16), "x must be non-NULL and 16-byte aligned");
    return CHN_OK;
}

}  // namespace chn

using namespace chn;

extern "C" int chn_gemv_q4(chn_ctx *ctx, const uint32_t *W, const float *x, float *y,
                           uint32_t M, uint32_t K) {
    if (!ctx) return CHN_E_INVALID;
    int rc = check_common(ctx, x, K);
    if (rc) return rc;
    CHN_REQUIRE(ctx, W && y && aligned(W, 4), "W/y must be non-NULL, W 4-byte aligned");
    if (M == 0) return CHN_OK;
    MatvecArgs a{W, nullptr, nullptr, y, nullptr, nullptr, x, M, M, M, K / 32};
    return launch_matvec(ctx, MV_GEMV, a);
}

extern "C" int chn_fused_qkv_q4(chn_ctx *ctx, const uint32_t *Wq, const uint32_t *Wk,
                                const uint32_t *Wv, const float *x, float *q, float *k,
                                float *v, uint32_t q_dim, uint32_t kv_dim, uint32_t K) {
    if (!ctx) return CHN_E_INVALID;
    int rc = check_common(ctx, x, K);
    if (rc) return rc;
    CHN_REQUIRE(ctx, Wq && Wk && Wv && q && k && v, "NULL matrix or output");
    CHN_REQUIRE(ctx, aligned(Wq, 4) && aligned(Wk, 4) && aligned(Wv, 4), "weights must be 4-byte aligned");
    const uint64_t M = (uint64_t)q_dim + 2ull * kv_dim;
    CHN_REQUIRE(ctx, M < (1ull << 31), "q_dim + 2*kv_dim too large");
    if (M == 0) return CHN_OK;
    MatvecArgs a{Wq, Wk, Wv, q, k, v, x, (uint32_t)M, q_dim, q_dim + kv_dim, K / 32};
    return launch_matvec(ctx, MV_QKV, a);
}

extern "C" int chn_fused_mlp_q4(chn_ctx *ctx, const uint32_t *Wg, const uint32_t *Wu,
                                const float *x, float *act, uint32_t M, uint32_t K) {
    if (!ctx) return CHN_E_INVALID;
    int rc = check_common(ctx, x, K);
    if (rc) return rc;
    CHN_REQUIRE(ctx, Wg && Wu && act && aligned(Wg, 4) && aligned(Wu, 4), "NULL/misaligned argument");
    if (M == 0) return CHN_OK;
    MatvecArgs a{Wg, Wu, nullptr, act, nullptr, nullptr, x, M, M, M, K / 32};
    return launch_matvec(ctx, MV_MLP, a);
}
