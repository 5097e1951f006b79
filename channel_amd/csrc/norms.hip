// RMSNorm (shaders/rmsnorm.wgsl, shaders/batch_rmsnorm.wgsl) and the fused
// residual add + RMSNorm (shaders/add_rmsnorm.wgsl,
// shaders/batch_add_rmsnorm.wgsl): one 256-thread workgroup per row,
// float4 accesses, sum of squares reduced wave-then-LDS in a fixed order.
#include "chn_internal.h"

namespace chn {

typedef float f4n __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

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

// The prefill's norm chain on one row per workgroup: the post-norm of the
// branch (k_rmsnorm<false> on r with post_w), the residual add
// (k_rmsnorm<true>) and the input norm of the next contraction, whose
// result is written as bf16 (the contraction's operand) and optionally as
// fp32.  The per-thread partial sums, their reduction and every product
// are those of the two k_rmsnorm passes, so x and y are bit-identical to
// them (r' is formed where it is added, never stored).  POST needs ADD.
// NP: the branch is the sum of NP partial outputs r + p * ps of a split
// contraction, added here in index order instead of through atomics into
// one zeroed buffer.
template <int NP>
__device__ __forceinline__ f4n branch_sum(const f4n (&v)[NP]) {
    f4n b = v[0];
#pragma unroll
    for (int p = 1; p < NP; ++p) b = b + v[p];
    return b;
}
template <bool POST, bool ADD, int NP>
__global__ __launch_bounds__(256) void k_rmsnorm_chain(float *__restrict__ x, const float *__restrict__ r, size_t ps,
                                                       const float *__restrict__ pw, const float *__restrict__ w,
                                                       __bf16 *__restrict__ yb, float *__restrict__ y, uint32_t dim,
                                                       float eps, float scalar) {
    __shared__ float sh[4];
    const size_t off = (size_t)blockIdx.x * dim;
    f4n *xr = (f4n *)(x + off);
    const f4n *pwr = (const f4n *)pw;
    const f4n *wr = (const f4n *)w;
    const uint32_t dv = dim / 4;
    auto branch = [&](uint32_t i) {
        f4n v[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) v[p] = ((const f4n *)(r + p * ps + off))[i];
        return branch_sum<NP>(v);
    };
    float inv_r = 1.0f;
    if (POST) {
        float ss = 0.0f;
        for (uint32_t i = threadIdx.x; i < dv; i += 256) {
            const f4n v = branch(i);
            ss += ((v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w));
        }
        ss = block_sum_256(ss, sh);
        inv_r = 1.0f / sqrtf(ss / (float)dim + eps);
    }
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < dv; i += 256) {
        f4n v = xr[i];
        if (ADD) {
            f4n b = branch(i);
            if (POST) b = (b * inv_r) * pwr[i];
            v = (v + b) * scalar;
            xr[i] = v;
        }
        ss += ((v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w));
    }
    ss = block_sum_256(ss, sh);
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    for (uint32_t i = threadIdx.x; i < dv; i += 256) {
        const f4n o = (xr[i] * inv) * wr[i];
        bf16x2 lo = {(__bf16)o.x, (__bf16)o.y}, hi = {(__bf16)o.z, (__bf16)o.w};
        *(bf16x2 *)(yb + off + 4 * (size_t)i) = lo;
        *(bf16x2 *)(yb + off + 4 * (size_t)i + 2) = hi;
        if (y) *(f4n *)(y + off + 4 * (size_t)i) = o;
    }
}

// The same chain with the row held in registers (dim <= 4096: four float4
// per thread): every input is requested at once, so the row costs one
// memory round trip instead of three, and each element is read once.
// Thread i handles float4s i, i + 256, ... in that order, so every sum and
// product is the loop form's.
template <bool POST, bool ADD, int NP>
__global__ __launch_bounds__(256) void k_rmsnorm_chain_r(float *__restrict__ x, const float *__restrict__ r, size_t ps,
                                                         const float *__restrict__ pw, const float *__restrict__ w,
                                                         __bf16 *__restrict__ yb, float *__restrict__ y, uint32_t dim,
                                                         float eps, float scalar) {
    constexpr int NPT = 4;
    __shared__ float sh[4];
    const size_t off = (size_t)blockIdx.x * dim;
    f4n *xr = (f4n *)(x + off);
    const f4n *pwr = (const f4n *)pw;
    const f4n *wr = (const f4n *)w;
    const uint32_t dv = dim / 4;
    f4n xv[NPT], rv[NPT], pv[NPT], wv[NPT];
    f4n rp[NPT][NP];
#pragma unroll
    for (int k = 0; k < NPT; ++k) {
        const uint32_t i = threadIdx.x + 256 * k;
        const bool ok = i < dv;
        xv[k] = ok ? xr[i] : f4n{0, 0, 0, 0};
        if (ADD)
#pragma unroll
            for (int p = 0; p < NP; ++p) rp[k][p] = ok ? ((const f4n *)(r + p * ps + off))[i] : f4n{0, 0, 0, 0};
        if (POST) pv[k] = ok ? pwr[i] : f4n{0, 0, 0, 0};
        wv[k] = ok ? wr[i] : f4n{0, 0, 0, 0};
    }
    if (ADD)
#pragma unroll
        for (int k = 0; k < NPT; ++k) rv[k] = branch_sum<NP>(rp[k]);
    float inv_r = 1.0f;
    if (POST) {
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < NPT; ++k) {
            const f4n v = rv[k];
            if (threadIdx.x + 256 * k < dv) ss += ((v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w));
        }
        ss = block_sum_256(ss, sh);
        inv_r = 1.0f / sqrtf(ss / (float)dim + eps);
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < NPT; ++k) {
        const uint32_t i = threadIdx.x + 256 * k;
        if (i >= dv) continue;
        f4n v = xv[k];
        if (ADD) {
            f4n b = rv[k];
            if (POST) b = (b * inv_r) * pv[k];
            v = (v + b) * scalar;
            xv[k] = v;
            xr[i] = v;
        }
        ss += ((v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w));
    }
    ss = block_sum_256(ss, sh);
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
#pragma unroll
    for (int k = 0; k < NPT; ++k) {
        const uint32_t i = threadIdx.x + 256 * k;
        if (i >= dv) continue;
        const f4n o = (xv[k] * inv) * wv[k];
        bf16x2 lo = {(__bf16)o.x, (__bf16)o.y}, hi = {(__bf16)o.z, (__bf16)o.w};
        *(bf16x2 *)(yb + off + 4 * (size_t)i) = lo;
        *(bf16x2 *)(yb + off + 4 * (size_t)i + 2) = hi;
        if (y) *(f4n *)(y + off + 4 * (size_t)i) = o;
    }
}

// The register form over several rows per workgroup (a grid of at most
// kChainGrid workgroups striding over the rows), the next row's x and r in
// flight while a row is reduced and stored, the norm weights loaded once.
// Loads are unconditional (a row past the end reloads the current one, from
// cache), so the compiler's waits leave the next row's loads outstanding.
// Per row, every sum and product is k_rmsnorm_chain_r's.
constexpr uint32_t kChainGrid = 256;
template <bool POST, bool ADD, int NP>
__global__ __launch_bounds__(256) void k_rmsnorm_chain_p(float *__restrict__ x, const float *__restrict__ r, size_t ps,
                                                         const float *__restrict__ pw, const float *__restrict__ w,
                                                         __bf16 *__restrict__ yb, float *__restrict__ y, uint32_t dim,
                                                         uint32_t rows, float eps, float scalar) {
    constexpr int NPT = 4;
    __shared__ float sh[4];
    const f4n *pwr = (const f4n *)pw;
    const f4n *wr = (const f4n *)w;
    const uint32_t dv = dim / 4;
    struct Row {
        f4n x[NPT], r[NPT][ADD ? NP : 1];
    };
    f4n pv[NPT], wv[NPT];
    uint32_t idx[NPT];
    uint32_t okm[NPT];
#pragma unroll
    for (int k = 0; k < NPT; ++k) {
        const uint32_t i = threadIdx.x + 256 * k;
        idx[k] = i < dv ? i : 0u;
        okm[k] = opaque_mask(i < dv);
    }
    auto mask4 = [](f4n v, uint32_t m) {
        return f4n{mask_f(v.x, m), mask_f(v.y, m), mask_f(v.z, m), mask_f(v.w, m)};
    };
    auto load = [&](uint32_t row, Row &d) {
        const f4n *xr = (const f4n *)(x + (size_t)row * dim);
#pragma unroll
        for (int k = 0; k < NPT; ++k) {
            d.x[k] = xr[idx[k]];
            if (ADD)
#pragma unroll
                for (int p = 0; p < NP; ++p) d.r[k][p] = ((const f4n *)(r + p * ps + (size_t)row * dim))[idx[k]];
        }
    };
    uint32_t row = blockIdx.x;
    Row A, B;
    load(row, A);
#pragma unroll
    for (int k = 0; k < NPT; ++k) {
        if (POST) pv[k] = pwr[idx[k]];
        wv[k] = wr[idx[k]];
    }
    auto process = [&](uint32_t row, Row &d) {
        const size_t off = (size_t)row * dim;
        f4n *xr = (f4n *)(x + off);
        f4n xv[NPT], rv[NPT];
#pragma unroll
        for (int k = 0; k < NPT; ++k) {
            xv[k] = mask4(d.x[k], okm[k]);
            if (ADD) {
                f4n v[NP];
#pragma unroll
                for (int p = 0; p < NP; ++p) v[p] = mask4(d.r[k][p], okm[k]);
                rv[k] = branch_sum<NP>(v);
            }
        }
        float inv_r = 1.0f;
        if (POST) {
            float ss = 0.0f;
#pragma unroll
            for (int k = 0; k < NPT; ++k) {
                const f4n v = rv[k];
                if (threadIdx.x + 256 * k < dv) ss += ((v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w));
            }
            ss = block_sum_256(ss, sh);
            inv_r = 1.0f / sqrtf(ss / (float)dim + eps);
        }
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < NPT; ++k) {
            const uint32_t i = threadIdx.x + 256 * k;
            if (i >= dv) continue;
            f4n v = xv[k];
            if (ADD) {
                f4n b = rv[k];
                if (POST) b = (b * inv_r) * pv[k];
                v = (v + b) * scalar;
                xv[k] = v;
                xr[i] = v;
            }
            ss += ((v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w));
        }
        ss = block_sum_256(ss, sh);
        const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
#pragma unroll
        for (int k = 0; k < NPT; ++k) {
            const uint32_t i = threadIdx.x + 256 * k;
            if (i >= dv) continue;
            const f4n o = (xv[k] * inv) * wv[k];
            bf16x2 lo = {(__bf16)o.x, (__bf16)o.y}, hi = {(__bf16)o.z, (__bf16)o.w};
            *(bf16x2 *)(yb + off + 4 * (size_t)i) = lo;
            *(bf16x2 *)(yb + off + 4 * (size_t)i + 2) = hi;
            if (y) *(f4n *)(y + off + 4 * (size_t)i) = o;
        }
    };
    const uint32_t G = gridDim.x;
    for (;;) {
        load(row + G < rows ? row + G : row, B);
        process(row, A);
        row += G;
        if (row >= rows) break;
        load(row + G < rows ? row + G : row, A);
        process(row, B);
        row += G;
        if (row >= rows) break;
    }
}

template <bool POST, bool ADD, int NP>
static void launch_chain_kind(hipStream_t s, float *x, const float *r, size_t ps, const float *post_w,
                              const float *w, __bf16 *yb, float *y, uint32_t dim, uint32_t rows, float eps,
                              float scalar) {
    if (dim <= 4096 && rows > kChainGrid)
        k_rmsnorm_chain_p<POST, ADD, NP><<<kChainGrid, 256, 0, s>>>(x, r, ps, post_w, w, yb, y, dim, rows, eps, scalar);
    else if (dim <= 4096)
        k_rmsnorm_chain_r<POST, ADD, NP><<<rows, 256, 0, s>>>(x, r, ps, post_w, w, yb, y, dim, eps, scalar);
    else k_rmsnorm_chain<POST, ADD, NP><<<rows, 256, 0, s>>>(x, r, ps, post_w, w, yb, y, dim, eps, scalar);
}

template <int NP>
static void launch_chain_np(hipStream_t s, float *x, const float *r, size_t ps, const float *post_w, const float *w,
                            __bf16 *yb, float *y, uint32_t dim, uint32_t rows, float eps, float scalar) {
    if (post_w) launch_chain_kind<true, true, NP>(s, x, r, ps, post_w, w, yb, y, dim, rows, eps, scalar);
    else launch_chain_kind<false, true, NP>(s, x, r, ps, post_w, w, yb, y, dim, rows, eps, scalar);
}

int launch_rmsnorm_chain(hipStream_t s, float *x, const float *r, const float *post_w, const float *w, __bf16 *yb,
                         float *y, uint32_t dim, uint32_t rows, float eps, float scalar, bool add, uint32_t nparts,
                         size_t pstride) {
    if (!add) launch_chain_kind<false, false, 1>(s, x, r, 0, post_w, w, yb, y, dim, rows, eps, scalar);
    else if (nparts == 4) launch_chain_np<4>(s, x, r, pstride, post_w, w, yb, y, dim, rows, eps, scalar);
    else if (nparts == 2) launch_chain_np<2>(s, x, r, pstride, post_w, w, yb, y, dim, rows, eps, scalar);
    else if (nparts == 1) launch_chain_np<1>(s, x, r, 0, post_w, w, yb, y, dim, rows, eps, scalar);
    else return CHN_E_UNSUPPORTED;
    return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
}

// Sum over the whole workgroup (blockDim.x a multiple of 64, <= 1024):
// wave sums, then the wave partials in index order.
__device__ __forceinline__ float block_sum_n(float v, float *sh) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) sh[wave] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; ++i) t += sh[i];
    __syncthreads();
    return t;
}

__device__ __forceinline__ void load8(const float *p, uint32_t t, bool ok, float (&v)[8]) {
    if (ok) {
        const f4n a = *(const f4n *)(p + 8 * (size_t)t), b = *(const f4n *)(p + 8 * (size_t)t + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.0f;
    }
}
__device__ __forceinline__ void store8(float *p, uint32_t t, const float (&v)[8]) {
    *(f4n *)(p + 8 * (size_t)t) = f4n{v[0], v[1], v[2], v[3]};
    *(f4n *)(p + 8 * (size_t)t + 4) = f4n{v[4], v[5], v[6], v[7]};
}

// The decode step's norms fused with the matvec input: with POST the
// residual branch is normalised first (post_attention / post_feedforward
// norm), with ADD it is added to x and scaled (add_rmsnorm), then
// y = rmsnorm(x) * w and the digit planes of y.  One workgroup of
// ceil(dim / 8) threads rounded up to whole waves, eight values per thread
// (four threads per 32-block, as the planes want them).  With rt.tab set
// (the step's first norm) the threads also write the step's RoPE table.
template <bool POST, bool ADD>
__global__ __launch_bounds__(1024) void k_norm_planes(float *__restrict__ x, const float *__restrict__ r,
                                                      const float *__restrict__ pw, const float *__restrict__ w,
                                                      float *__restrict__ y, uint32_t *__restrict__ xp, uint32_t dim,
                                                      float eps, float scalar, RopeTab rt,
                                                      const uint32_t *__restrict__ skip,
                                                      uint32_t *__restrict__ xb) {
    __shared__ float sh[16];
    const uint32_t t = threadIdx.x;
    if (rt.tab) rope_table(rt, t, blockDim.x);
    const bool ok = 8 * t < dim;
    if (skip && *skip) {
        // the last layer was quiescent: x keeps its value and y (the normed
        // row the reference's logits read) is whatever was last written
        if (xp || xb) {
            float yv[8];
            load8(y, t, ok, yv);
            if (xp) emit_planes8(yv, xp, dim / 32, t >> 2, t & 3, ok);
            if (xb) emit_bytes8(yv, xb, dim / 32, t >> 2, t & 3, ok);
        }
        return;
    }
    // every load is issued before the first reduction
    float xv[8], rv[8], pv[8], wv[8];
    load8(x, t, ok, xv);
    if (ADD) load8(r, t, ok, rv);
    if (POST) load8(pw, t, ok, pv);
    load8(w, t, ok, wv);
    if (ADD) {
        if (POST) {
            float ss = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) ss += rv[i] * rv[i];
            ss = block_sum_n(ss, sh);
            const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
#pragma unroll
            for (int i = 0; i < 8; ++i) rv[i] = (rv[i] * inv) * pv[i];
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[i] = (xv[i] + rv[i]) * scalar;
        if (ok) store8(x, t, xv);
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += xv[i] * xv[i];
    ss = block_sum_n(ss, sh);
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    float yv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) yv[i] = (xv[i] * inv) * wv[i];
    if (ok) store8(y, t, yv);
    if (xp) emit_planes8(yv, xp, dim / 32, t >> 2, t & 3, ok);
    if (xb) emit_bytes8(yv, xb, dim / 32, t >> 2, t & 3, ok);
}

int launch_norm_planes(hipStream_t s, float *x, const float *r, const float *post_w, const float *w, float *y,
                       uint32_t *xp, uint32_t dim, float eps, float scalar, bool add, const RopeTab *rope,
                       const uint32_t *skip, uint32_t *xb) {
    if (dim % 32 != 0 || dim > 8192) return CHN_E_UNSUPPORTED;
    if (rope && (rope->rot[0] > 2 * kRopePairs || rope->rot[1] > 2 * kRopePairs)) return CHN_E_UNSUPPORTED;
    const uint32_t nt = ((dim / 8 + 63) / 64) * 64;
    const RopeTab rt = rope ? *rope : RopeTab{nullptr, nullptr, {0.0f, 0.0f}, {0u, 0u}};
    if (!add) k_norm_planes<false, false><<<1, nt, 0, s>>>(x, r, post_w, w, y, xp, dim, eps, scalar, rt, skip, xb);
    else if (post_w) k_norm_planes<true, true><<<1, nt, 0, s>>>(x, r, post_w, w, y, xp, dim, eps, scalar, rt, skip, xb);
    else k_norm_planes<false, true><<<1, nt, 0, s>>>(x, r, post_w, w, y, xp, dim, eps, scalar, rt, skip, xb);
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
