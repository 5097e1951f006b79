// Seeded synthetic inputs generated in place on the device.  The hash is a
// splitmix64 output function over a counter, so the host can regenerate any
// block bit-for-bit (integer codes and fma-then-RNE f16 scales) to check it.
#include "chn_internal.h"

namespace chn {

// Q4 block blk = row * nb + b: hash 3*blk -> scale, hashes 3*blk+1, +2 ->
// nibble words 1..4 (low 32 bits first).
__global__ void k_synth_q4(uint32_t *W, uint64_t nblk, uint64_t seed, float smin, float range) {
    uint64_t blk = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (; blk < nblk; blk += stride) {
        const uint64_t h0 = mix64(seed, blk * 3), h1 = mix64(seed, blk * 3 + 1),
                       h2 = mix64(seed, blk * 3 + 2);
        const float u = (float)(uint32_t)(h0 >> 40) * (1.0f / 16777216.0f);
        const float s = fmaf(u, range, smin);
        const _Float16 hs = (_Float16)s, hm = (_Float16)(-8.0f * s);
        uint32_t *o = W + blk * 5;
        o[0] = (uint32_t)__builtin_bit_cast(unsigned short, hs) |
               ((uint32_t)__builtin_bit_cast(unsigned short, hm) << 16);
        o[1] = (uint32_t)h1;
        o[2] = (uint32_t)(h1 >> 32);
        o[3] = (uint32_t)h2;
        o[4] = (uint32_t)(h2 >> 32);
    }
}

// Q8_0 block: hash 5*blk -> raw f32 scale, hashes 5*blk+1..4 -> words 1..8.
__global__ void k_synth_q8(uint32_t *W, uint64_t nblk, uint64_t seed, float smin, float range) {
    uint64_t blk = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (; blk < nblk; blk += stride) {
        const uint64_t h0 = mix64(seed, blk * 5);
        const float u = (float)(uint32_t)(h0 >> 40) * (1.0f / 16777216.0f);
        const float s = fmaf(u, range, smin);
        uint32_t *o = W + blk * 9;
        o[0] = __builtin_bit_cast(uint32_t, s);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint64_t h = mix64(seed, blk * 5 + 1 + j);
            o[1 + 2 * j] = (uint32_t)h;
            o[2 + 2 * j] = (uint32_t)(h >> 32);
        }
    }
}

__global__ void k_synth_normal(float *dst, uint64_t n, uint64_t seed, float stddev) {
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) {
        const uint64_t h = mix64(seed, i);
        const double u1 = ((double)(h >> 40) + 1.0) * (1.0 / 16777216.0);
        const double u2 = (double)((h >> 16) & 0xffffffu) * (1.0 / 16777216.0);
        const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        dst[i] = (float)(z * (double)stddev);
    }
}

static unsigned grid_for(uint64_t n) {
    uint64_t g = (n + 255) / 256;
    return (unsigned)(g > 65536 ? 65536 : (g ? g : 1));
}

}  // namespace chn

using namespace chn;

extern "C" int chn_synth_q4(chn_ctx *ctx, uint32_t *W, uint32_t rows, uint32_t K,
                            uint64_t seed, float smin, float smax) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, W && aligned(W, 4), "W must be non-NULL and 4-byte aligned");
    CHN_REQUIRE(ctx, K % 32 == 0, "K=%u must be a multiple of 32", K);
    const uint64_t nblk = (uint64_t)rows * (K / 32);
    if (!nblk) return CHN_OK;
    k_synth_q4<<<grid_for(nblk), 256, 0, ctx->stream>>>(W, nblk, seed, smin, smax - smin);
    CHN_LAUNCHED(ctx, "k_synth_q4");
    return CHN_OK;
}

extern "C" int chn_synth_q8(chn_ctx *ctx, uint32_t *W, uint32_t rows, uint32_t K,
                            uint64_t seed, float smin, float smax) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, W && aligned(W, 4), "W must be non-NULL and 4-byte aligned");
    CHN_REQUIRE(ctx, K % 32 == 0, "K=%u must be a multiple of 32", K);
    const uint64_t nblk = (uint64_t)rows * (K / 32);
    if (!nblk) return CHN_OK;
    k_synth_q8<<<grid_for(nblk), 256, 0, ctx->stream>>>(W, nblk, seed, smin, smax - smin);
    CHN_LAUNCHED(ctx, "k_synth_q8");
    return CHN_OK;
}

extern "C" int chn_synth_normal(chn_ctx *ctx, float *dst, size_t n, uint64_t seed, float stddev) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, dst || !n, "dst is NULL");
    if (!n) return CHN_OK;
    k_synth_normal<<<grid_for(n), 256, 0, ctx->stream>>>(dst, n, seed, stddev);
    CHN_LAUNCHED(ctx, "k_synth_normal");
    return CHN_OK;
}
