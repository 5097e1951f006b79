// RMSNorm (shaders/rmsnorm.wgsl, shaders/batch_rmsnorm.wgsl) and the fused
// residual add + RMSNorm (shaders/add_rmsnorm.wgsl,
// shaders/batch_add_rmsnorm.wgsl): one 256-thread workgroup per row,
// float4 accesses, sum of squares reduced wave-then-LDS in a fixed order.
#include "chn_internal.h"

namespace chn {

typedef float f4n __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float block_sum_256(float v, float *sh) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) sh[wave] = v;
    __syncthreads();
    const float t = (sh[0] + sh[1]) + (sh[2] + sh[3]);
    __syncthreads();
    return t;
}

// y = x * rsqrt(mean(x^2) + eps) * w; with ADD, x = (x + r) * scalar first
// and written back.  Row n of x / r / y is at n * dim.
template <bool ADD>
__global__ __launch_bounds__(256) void k_rmsnorm(float *__restrict__ x, const float *__restrict__ r,
                                                 const float *__restrict__ w, float *__restrict__ y,
                                                 uint32_t dim, float eps, float scalar) {
    __shared__ float sh[4];
    const size_t off = (size_t)blockIdx.x * dim;
    f4n *xr = (f4n *)(x + off);
    const f4n *rr = (const f4n *)(r + off);
    const f4n *wr = (const f4n *)w;
    f4n *yr = (f4n *)(y + off);
    const uint32_t dv = dim / 4;
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < dv; i += 256) {
        f4n v = xr[i];
        if (ADD) {
            v = (v + rr[i]) * scalar;
            xr[i] = v;
        }
        ss += ((v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w));
    }
    ss = block_sum_256(ss, sh);
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    for (uint32_t i = threadIdx.x; i < dv; i += 256) yr[i] = (xr[i] * inv) * wr[i];
}

int launch_rmsnorm(hipStream_t s, float *x, const float *r, const float *w, float *y, uint32_t dim,
                   uint32_t rows, float eps, float scalar, bool add) {
    if (add) k_rmsnorm<true><<<rows, 256, 0, s>>>(x, r, w, y, dim, eps, scalar);
    else k_rmsnorm<false><<<rows, 256, 0, s>>>(x, r, w, y, dim, eps, scalar);
    return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
}

static int check_norm(chn_ctx *ctx, const void *x, const void *w, const void *y, uint32_t dim) {
    CHN_REQUIRE(ctx, x && w && y, "NULL argument");
    CHN_REQUIRE(ctx, dim > 0 && dim % 4 == 0, "dim %u must be a positive multiple of 4", dim);
    CHN_REQUIRE(ctx, aligned(x, 16) && aligned(w, 16) && aligned(y, 16), "buffers must be 16-byte aligned");
    return CHN_OK;
}

}  // namespace chn

using namespace chn;

extern "C" int chn_rmsnorm(chn_ctx *ctx, const float *x, const float *w, float *y, uint32_t dim, float eps) {
    if (!ctx) return CHN_E_INVALID;
    int rc = check_norm(ctx, x, w, y, dim);
    if (rc) return rc;
    k_rmsnorm<false><<<1, 256, 0, ctx->stream>>>((float *)x, nullptr, w, y, dim, eps, 1.0f);
    CHN_LAUNCHED(ctx, "k_rmsnorm");
    return CHN_OK;
}

extern "C" int chn_add_rmsnorm(chn_ctx *ctx, float *x, const float *r, const float *w, float *y, uint32_t dim,
                               float eps, float scalar) {
    if (!ctx) return CHN_E_INVALID;
    int rc = check_norm(ctx, x, w, y, dim);
    if (rc) return rc;
    CHN_REQUIRE(ctx, r && aligned(r, 16), "r must be non-NULL and 16-byte aligned");
    k_rmsnorm<true><<<1, 256, 0, ctx->stream>>>(x, r, w, y, dim, eps, scalar);
    CHN_LAUNCHED(ctx, "k_add_rmsnorm");
    return CHN_OK;
}

extern "C" int chn_batch_rmsnorm(chn_ctx *ctx, const float *X, const float *w, float *Y, uint32_t n_tok,
                                 uint32_t dim, float eps) {
    if (!ctx) return CHN_E_INVALID;
    int rc = check_norm(ctx, X, w, Y, dim);
    if (rc) return rc;
    if (!n_tok) return CHN_OK;
    k_rmsnorm<false><<<n_tok, 256, 0, ctx->stream>>>((float *)X, nullptr, w, Y, dim, eps, 1.0f);
    CHN_LAUNCHED(ctx, "k_batch_rmsnorm");
    return CHN_OK;
}

extern "C" int chn_batch_add_rmsnorm(chn_ctx *ctx, float *X, const float *R, const float *w, float *Y,
                                     uint32_t n_tok, uint32_t dim, float eps, float scalar) {
    if (!ctx) return CHN_E_INVALID;
    int rc = check_norm(ctx, X, w, Y, dim);
    if (rc) return rc;
    CHN_REQUIRE(ctx, R && aligned(R, 16), "R must be non-NULL and 16-byte aligned");
    if (!n_tok) return CHN_OK;
    k_rmsnorm<true><<<n_tok, 256, 0, ctx->stream>>>(X, R, w, Y, dim, eps, scalar);
    CHN_LAUNCHED(ctx, "k_batch_add_rmsnorm");
    return CHN_OK;
}
