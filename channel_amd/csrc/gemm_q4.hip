// Batched prefill contractions over Q4 weights on gfx950 MFMA:
// batch_gemm_q4 (shaders/batch_gemm_q4.wgsl) and batch_fused_mlp_q4
// (shaders/batch_fused_mlp_q4.wgsl).
//
//   Y[t, n] = sum_k X[t, k] * W[n, k]        (t < n_tok, n < M)
//
// The contraction is dense (arithmetic intensity ~800 FLOP/byte at 512
// tokens), so it runs on v_mfma_f32_16x16x32_bf16:
//  * activations are rounded to bf16 (RNE) once, by a pre-pass;
//  * each workgroup owns a 128-token x 128-feature output tile and walks K
//    in steps of 64 (two Q4 blocks); its threads dequantize the weight tile
//    to bf16(scale * (q - 8)) straight into LDS (one 20-byte block per
//    thread), so Q4 bytes are read from HBM once per token tile;
//  * the four waves each compute a 64 x 64 sub-tile (4 x 4 MFMA tiles),
//    reading fragments with ds_read_b128 from rows padded to 144 bytes;
//  * the next K step's global loads are in flight while the current step
//    computes.
// Accumulation is fp32; the only roundings beyond fp32 are the two bf16
// operand roundings.
#include "chn_internal.h"

namespace chn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

constexpr int GT = 128;          // tokens per workgroup tile
constexpr int GN = 128;          // features per workgroup tile
constexpr int GK = 64;           // K per step (two Q4 blocks)
constexpr int LROW = GK * 2 + 16; // LDS row stride in bytes (padded)

__global__ __launch_bounds__(256) void k_to_bf16(const float *__restrict__ x, __bf16 *__restrict__ y, size_t n) {
    size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
    const size_t stride = (size_t)gridDim.x * blockDim.x * 4;
    for (; i < n; i += stride) {
        if (i + 4 <= n) {
            const float4 v = *(const float4 *)(x + i);
            bf16x2 a = {(__bf16)v.x, (__bf16)v.y}, b = {(__bf16)v.z, (__bf16)v.w};
            *(bf16x2 *)(y + i) = a;
            *(bf16x2 *)(y + i + 2) = b;
        } else {
            for (size_t j = i; j < n; ++j) y[j] = (__bf16)x[j];
        }
    }
}

struct GemmArgs {
    const __bf16 *X;       // [n_tok][K] bf16
    const uint32_t *W0, *W1; // Q4 [M][K/32][5], or Q4R (W1: up matrix for the fused MLP)
    float *Y;              // [n_tok][M]
    uint32_t n_tok, M, K;
};

typedef uint32_t u32x4g __attribute__((ext_vector_type(4)));

// Dequantize one Q4 block (5 words) to 32 bf16 = 4 x 16 bytes.
__device__ __forceinline__ void dequant_block_bf16(const uint32_t w0, const u32x4v q, u32x4v (&out)[4]) {
    const float s = f16_lo_to_f32(w0);
    const float ms = -8.0f * s;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint32_t lo = opaque_u32(q[w] & 0x0F0F0F0Fu);
        const uint32_t hi = opaque_u32((q[w] >> 4) & 0x0F0F0F0Fu);
        // element 8w + n is nibble n: even n from lo byte n/2, odd from hi
        float v[8];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[2 * j] = fmaf((float)((lo >> (8 * j)) & 0xffu), s, ms);
            v[2 * j + 1] = fmaf((float)((hi >> (8 * j)) & 0xffu), s, ms);
        }
        u32x4v o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            bf16x2 p = {(__bf16)v[2 * j], (__bf16)v[2 * j + 1]};
            o[j] = __builtin_bit_cast(uint32_t, p);
        }
        out[w] = o;
    }
}

// REP: weights in the repacked layout (16-byte nibble words, each nibble
// XOR 8, then f16 scales), un-XORed here so the dequantization is shared.
template <int NMAT, bool REP>
__global__ __launch_bounds__(256, 2) void k_q4gemm(GemmArgs a) {
    __shared__ __attribute__((aligned(16))) unsigned char lx[GT * LROW];
    __shared__ __attribute__((aligned(16))) unsigned char lw[NMAT][GN * LROW];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wr = wave >> 1, wc = wave & 1;           // wave's 64x64 sub-tile
    const uint32_t n0 = blockIdx.x * GN, t0 = blockIdx.y * GT;
    const uint32_t nb = a.K / 32;
    const uint32_t steps = (a.K + GK - 1) / GK;

    // global -> register staging for one K step
    u32x4v xr[4];                  // 4 x 16 B of X per thread
    uint32_t ww0[NMAT];
    u32x4v wq[NMAT];
    const int w_row = tid >> 1, w_blk = tid & 1;       // weight block handled by this thread

    auto gload = [&](uint32_t ks) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + 256 * i;               // 1024 chunks of 16 B
            const int row = c >> 3, col = c & 7;       // 8 chunks per 64-wide row
            const uint32_t t = t0 + row;
            const uint32_t k = ks * GK + col * 8;
            xr[i] = (t < a.n_tok && k < a.K) ? *(const u32x4v *)(a.X + (size_t)t * a.K + k) : u32x4v{0, 0, 0, 0};
        }
        const uint32_t n = n0 + w_row;
        const uint32_t b = ks * 2 + w_blk;
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            const uint32_t *W = m == 0 ? a.W0 : a.W1;
            if (n < a.M && b < nb) {
                if (REP) {
                    const size_t i = (size_t)n * nb + b;
                    const u32x4g qv = ((const u32x4g *)W)[i];
                    wq[m] = u32x4v{qv[0] ^ 0x88888888u, qv[1] ^ 0x88888888u, qv[2] ^ 0x88888888u,
                                   qv[3] ^ 0x88888888u};
                    ww0[m] = ((const uint16_t *)((const unsigned char *)W + (size_t)a.M * nb * 16))[i];
                } else {
                    const uint32_t *p = W + ((size_t)n * nb + b) * 5;
                    ww0[m] = p[0];
                    wq[m] = *(const u32x4_a4 *)(p + 1);
                }
            } else {
                ww0[m] = 0;
                wq[m] = u32x4v{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
            }
        }
    };

    f32x4 acc[NMAT][4][4];
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[m][i][j] = f32x4{0, 0, 0, 0};

    gload(0);
    for (uint32_t ks = 0; ks < steps; ++ks) {
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + 256 * i;
            *(u32x4v *)(lx + (c >> 3) * LROW + (c & 7) * 16) = xr[i];
        }
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            u32x4v d[4];
            dequant_block_bf16(ww0[m], wq[m], d);
            unsigned char *dst = lw[m] + w_row * LROW + w_blk * 64;
#pragma unroll
            for (int w = 0; w < 4; ++w) *(u32x4v *)(dst + 16 * w) = d[w];
        }
        __syncthreads();
        if (ks + 1 < steps) gload(ks + 1);

#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int koff = (kk * 32 + (lane >> 4) * 8) * 2;
            bf16x8 af[4], bfm[NMAT][4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
                af[mt] = *(const bf16x8 *)(lx + (wr * 64 + mt * 16 + (lane & 15)) * LROW + koff);
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
#pragma unroll
                for (int nt = 0; nt < 4; ++nt)
                    bfm[m][nt] = *(const bf16x8 *)(lw[m] + (wc * 64 + nt * 16 + (lane & 15)) * LROW + koff);
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                    for (int nt = 0; nt < 4; ++nt)
                        acc[m][mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt], bfm[m][nt], acc[m][mt][nt],
                                                                                  0, 0, 0);
        }
    }

    // epilogue: lane holds rows (tokens) (lane>>4)*4 + i, column (feature) lane & 15
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            const uint32_t n = n0 + wc * 64 + nt * 16 + (lane & 15);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t t = t0 + wr * 64 + mt * 16 + (lane >> 4) * 4 + i;
                if (t < a.n_tok && n < a.M) {
                    float v = acc[0][mt][nt][i];
                    if (NMAT == 2) v = gelu_tanh(v) * acc[NMAT - 1][mt][nt][i];
                    a.Y[(size_t)t * a.M + n] = v;
                }
            }
        }
}

int launch_q4gemm(chn_ctx *ctx, int nmat, const float *X, const uint32_t *W0, const uint32_t *W1, float *Y,
                  uint32_t n_tok, uint32_t M, uint32_t K, __bf16 *xb, bool repacked) {
    const size_t n = (size_t)n_tok * K;
    unsigned g = (unsigned)((n / 4 + 255) / 256);
    if (g > 8192) g = 8192;
    if (g == 0) g = 1;
    k_to_bf16<<<g, 256, 0, ctx->stream>>>(X, xb, n);
    CHN_LAUNCHED(ctx, "k_to_bf16");
    GemmArgs a{xb, W0, W1, Y, n_tok, M, K};
    dim3 grid((M + GN - 1) / GN, (n_tok + GT - 1) / GT);
    if (repacked) {
        if (nmat == 1) k_q4gemm<1, true><<<grid, 256, 0, ctx->stream>>>(a);
        else k_q4gemm<2, true><<<grid, 256, 0, ctx->stream>>>(a);
    } else {
        if (nmat == 1) k_q4gemm<1, false><<<grid, 256, 0, ctx->stream>>>(a);
        else k_q4gemm<2, false><<<grid, 256, 0, ctx->stream>>>(a);
    }
    CHN_LAUNCHED(ctx, "k_q4gemm");
    return CHN_OK;
}

static int gemm_common(chn_ctx *ctx, int nmat, const uint32_t *W0, const uint32_t *W1, const float *X, float *Y,
                       uint32_t n_tok, uint32_t M, uint32_t K) {
    CHN_REQUIRE(ctx, W0 && X && Y && (nmat == 1 || W1), "NULL argument");
    CHN_REQUIRE(ctx, K > 0 && K % 32 == 0, "K=%u must be a positive multiple of 32", K);
    CHN_REQUIRE(ctx, K % 8 == 0 && aligned(X, 16), "X must be 16-byte aligned");
    CHN_REQUIRE(ctx, aligned(W0, 4) && (!W1 || aligned(W1, 4)), "weights must be 4-byte aligned");
    if (!n_tok || !M) return CHN_OK;
    int rc = ensure_workspace(ctx, (size_t)n_tok * K * 2);
    if (rc) return rc;
    return launch_q4gemm(ctx, nmat, X, W0, W1, Y, n_tok, M, K, (__bf16 *)ctx->ws, false);
}

}  // namespace chn

using namespace chn;

extern "C" int chn_batch_gemm_q4(chn_ctx *ctx, const uint32_t *W, const float *X, float *Y, uint32_t n_tok,
                                 uint32_t M, uint32_t K) {
    if (!ctx) return CHN_E_INVALID;
    return gemm_common(ctx, 1, W, nullptr, X, Y, n_tok, M, K);
}

extern "C" int chn_batch_fused_mlp_q4(chn_ctx *ctx, const uint32_t *Wg, const uint32_t *Wu, const float *X,
                                      float *Y, uint32_t n_tok, uint32_t M, uint32_t K) {
    if (!ctx) return CHN_E_INVALID;
    return gemm_common(ctx, 2, Wg, Wu, X, Y, n_tok, M, K);
}
