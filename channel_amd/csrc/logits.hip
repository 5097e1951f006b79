// Logits and selection on gfx950:
//  * gemv_q8 (shaders/gemv_q8.wgsl) over the Q8_0 tied embedding,
//  * softcapped global top-64 (shaders/topk_pass1.wgsl, topk_pass2.wgsl),
//  * device restatements of the reference quantizers (src/quant.zig:21-98)
//    for weight ingest, and the embedding gather of forwardToken
//    (src/model/forward.zig:35-37).
//
// The Q8 matvec streams 36-byte blocks the way the Q4 matvec streams
// 20-byte ones (coalesced non-temporal 16-byte loads of row segments, LDS
// transpose to one lane per block).  Activations become three balanced
// base-256 digit planes of a 22-bit fixed-point value per 32-block, so a
// block is 24 v_dot4c_i32_i8 (signed weights x signed digits, exact), the
// three plane sums are combined in fp32 and scaled by f32 scale *
// 2^(e_b - 22).
#include "chn_internal.h"

namespace chn {

size_t xbytes_bytes(uint32_t nb) { return (size_t)nb * (XB_WORDS + 1) * 4; }

// Eight threads per 32-block, one per 4-element weight word.
__global__ __launch_bounds__(256) void k_xbytes(const float *__restrict__ x, uint32_t *__restrict__ xp, uint32_t nb) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t b = t >> 3, w = t & 7;
    const bool ok = b < nb;
    float4 v = ok ? *(const float4 *)(x + (size_t)b * 32 + w * 4) : make_float4(0, 0, 0, 0);
    float m = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    // NaN or Inf in the block: zero digits and a NaN scale (the products of
    // the reference's fp32 matvec would be non-finite)
    uint32_t bad = (uint32_t)!(fabsf(v.x) <= 3.4028235e38f) | (uint32_t)!(fabsf(v.y) <= 3.4028235e38f) |
                   (uint32_t)!(fabsf(v.z) <= 3.4028235e38f) | (uint32_t)!(fabsf(v.w) <= 3.4028235e38f);
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    m = fmaxf(m, __shfl_xor(m, 2, 64));
    m = fmaxf(m, __shfl_xor(m, 4, 64));
    bad |= __shfl_xor(bad, 1, 64);
    bad |= __shfl_xor(bad, 2, 64);
    bad |= __shfl_xor(bad, 4, 64);
    int e = 0;
    (void)frexpf(m, &e);
    float scale = 0.0f, inv = 0.0f;
    if (bad) {
        inv = __builtin_nanf("");
        v = make_float4(0, 0, 0, 0);
    } else if (m > 0.0f && e > -100) {
        scale = ldexpf(1.0f, XB_FRAC - e);
        inv = ldexpf(1.0f, e - XB_FRAC);
    }
    uint32_t u[4];
    u[0] = (uint32_t)((int)rintf(v.x * scale) + 0x808080);
    u[1] = (uint32_t)((int)rintf(v.y * scale) + 0x808080);
    u[2] = (uint32_t)((int)rintf(v.z * scale) + 0x808080);
    u[3] = (uint32_t)((int)rintf(v.w * scale) + 0x808080);
    if (!ok) return;
#pragma unroll
    for (int p = 0; p < XB_PLANES; ++p) {
        uint32_t word = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) word |= ((u[j] >> (8 * p)) & 0xffu) << (8 * j);
        xp[(size_t)(p * 8 + w) * nb + b] = word ^ 0x80808080u;
    }
    if (w == 0) ((float *)(xp + (size_t)XB_WORDS * nb))[b] = inv;
}

typedef uint32_t u32x4q __attribute__((ext_vector_type(4)));

constexpr int kQ8Seg = 128 * 9;   // LDS words per stream segment (128 blocks)

__device__ __forceinline__ void q8_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Whole rows per wave (K <= 4096), RPW rows per group, persistent grid.
template <int RPW>
__global__ __launch_bounds__(256) void k_q8mv(const uint32_t *__restrict__ W, const uint32_t *__restrict__ xp,
                                              float *__restrict__ y, uint32_t M, uint32_t nb) {
    constexpr int LV = RPW == 1 ? 0 : (RPW == 2 ? 1 : 2);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const size_t rw = (size_t)nb * 9;
    const uint32_t chunks = nb * 9 / 4;          // nb % 4 == 0
    __shared__ uint32_t seg[4][RPW * kQ8Seg];
    uint32_t *L = seg[wave];

    uint32_t P[2][XB_WORDS];
    float xs[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const uint32_t b = c * 64 + lane;
        const bool ok = b < nb;
#pragma unroll
        for (int i = 0; i < XB_WORDS; ++i) P[c][i] = ok ? xp[(size_t)i * nb + b] : 0u;
        xs[c] = ok ? ((const float *)(xp + (size_t)XB_WORDS * nb))[b] : 0.0f;
    }
    const uint32_t ngroups = (M + RPW - 1) / RPW;
    const uint32_t gstride = gridDim.x * 4;
    u32x4q pf[RPW][5];
    auto load = [&](uint32_t g) {
#pragma unroll
        for (int s = 0; s < RPW; ++s) {
            const uint32_t row = g * RPW + s;
            const u32x4q *base = (const u32x4q *)(W + (size_t)(row < M ? row : 0) * rw);
#pragma unroll
            for (int j = 0; j < 5; ++j) {
                const uint32_t c = lane + 64 * j;
                if (row < M && c < chunks) pf[s][j] = __builtin_nontemporal_load(base + c);
            }
        }
    };
    uint32_t g = blockIdx.x * 4 + wave;
    if (g < ngroups) load(g);
    for (; g < ngroups; g += gstride) {
#pragma unroll
        for (int s = 0; s < RPW; ++s)
#pragma unroll
            for (int j = 0; j < 5; ++j) {
                const uint32_t c = lane + 64 * j;
                if (c < chunks) *(u32x4q *)(L + s * kQ8Seg + 4 * c) = pf[s][j];
            }
        q8_lds_fence();
        if (g + gstride < ngroups) load(g + gstride);
        float acc[RPW];
#pragma unroll
        for (int s = 0; s < RPW; ++s) acc[s] = 0.0f;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const uint32_t b = c * 64 + lane;
            if (b < nb) {
#pragma unroll
                for (int s = 0; s < RPW; ++s) {
                    const uint32_t *p = L + s * kQ8Seg + 9 * b;
                    const float sw = __builtin_bit_cast(float, p[0]);
                    int pl[XB_PLANES];
#pragma unroll
                    for (int q = 0; q < XB_PLANES; ++q) {
                        int t = 0;
#pragma unroll
                        for (int w = 0; w < 8; ++w) t = __builtin_amdgcn_sdot4((int)p[1 + w], (int)P[c][q * 8 + w], t, false);
                        pl[q] = t;
                    }
                    const float T = fmaf((float)pl[2], 65536.0f, fmaf((float)pl[1], 256.0f, (float)pl[0]));
                    acc[s] = fmaf(T, sw * xs[c], acc[s]);
                }
            }
        }
        q8_lds_fence();
        const float sum = wave_reduce_v<RPW>(acc, lane);
        const int vi = lane >> (6 - LV);
        if ((lane & ((64 >> LV) - 1)) == 0 && g * RPW + vi < M) y[g * RPW + vi] = sum;
    }
}

// Q8R: the Q8_0 blocks repacked for coalesced streaming, codes first, then
// the f32 scales ([rows * nb]); 36 bytes per block as before.  The codes of
// a row are its blocks' first 16-byte halves in block order, then their
// second halves ([rows][2][nb] 16-byte words), so the lanes of a wave that
// take consecutive blocks read one contiguous run per half.
__global__ __launch_bounds__(256) void k_repack_q8(const uint32_t *__restrict__ src, u32x4q *__restrict__ D,
                                                   float *__restrict__ S, size_t nblk, uint32_t nb) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk) return;
    const uint32_t *p = src + i * 9;
    const size_t row = i / nb, h0 = row * 2 * nb + (i - row * nb);
    D[h0] = u32x4q{p[1], p[2], p[3], p[4]};
    D[h0 + nb] = u32x4q{p[5], p[6], p[7], p[8]};
    S[i] = __builtin_bit_cast(float, p[0]);
}

int launch_q8_repack(hipStream_t st, const uint32_t *W, uint32_t rows, uint32_t nb, void *dst) {
    const size_t nblk = (size_t)rows * nb;
    if (!nblk) return CHN_OK;
    k_repack_q8<<<(unsigned)((nblk + 255) / 256), 256, 0, st>>>(W, (u32x4q *)dst,
                                                               (float *)((unsigned char *)dst + nblk * 32), nblk, nb);
    return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
}

// The Q8 matvec over Q8R: lane l owns blocks l and l + 64 of each row (K <=
// 4096) and reads them straight from the stream (its two 16-byte codes words
// and the scale), no LDS; RPW rows per group, the next group in flight while
// one is reduced.  Every load is unconditional (indices clamped into the
// matrix; a lane past the row's blocks adds nothing, rows past M are not
// stored).  Per block and row the arithmetic, its order and the reduction
// are k_q8mv's, so the two give identical results.
template <int RPW>
__global__ __launch_bounds__(256) void k_q8rmv(const u32x4q *__restrict__ D, const float *__restrict__ S,
                                               const uint32_t *__restrict__ xp, float *__restrict__ y, uint32_t M,
                                               uint32_t nb) {
    constexpr int LV = RPW == 1 ? 0 : (RPW == 2 ? 1 : 2);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    uint32_t P[2][XB_WORDS];
    float xs[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const uint32_t b = c * 64 + lane, bc = min(b, nb - 1);
        const uint32_t keep = b < nb ? ~0u : 0u;
#pragma unroll
        for (int i = 0; i < XB_WORDS; ++i) P[c][i] = xp[(size_t)i * nb + bc] & keep;
        xs[c] = __builtin_bit_cast(float, xp[(size_t)XB_WORDS * nb + bc] & keep);
    }
    const uint32_t ngroups = (M + RPW - 1) / RPW;
    const uint32_t gstride = gridDim.x * 4;
    struct Grp {
        u32x4q d[RPW][2][2];
        float s[RPW][2];
    };
    auto load = [&](Grp &q, uint32_t g) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const uint32_t row = min(g * RPW + r, M - 1);
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const uint32_t b = min(c * 64 + lane, nb - 1);
                const size_t h0 = (size_t)row * 2 * nb + b;
                q.d[r][c][0] = __builtin_nontemporal_load(D + h0);
                q.d[r][c][1] = __builtin_nontemporal_load(D + h0 + nb);
                q.s[r][c] = __builtin_nontemporal_load(S + (size_t)row * nb + b);
            }
        }
    };
    uint32_t g = blockIdx.x * 4 + wave;
    Grp nx;
    load(nx, g < ngroups ? g : ngroups - 1);   // unconditional: a wave past the groups never uses it
    for (; g < ngroups; g += gstride) {
        const Grp cur = nx;
        if (g + gstride < ngroups) load(nx, g + gstride);
        float acc[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const uint32_t b = c * 64 + lane;
            if (b < nb) {
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    int pl[XB_PLANES];
#pragma unroll
                    for (int q = 0; q < XB_PLANES; ++q) {
                        int t = 0;
#pragma unroll
                        for (int w = 0; w < 8; ++w)
                            t = __builtin_amdgcn_sdot4((int)cur.d[r][c][w >> 2][w & 3], (int)P[c][q * 8 + w], t, false);
                        pl[q] = t;
                    }
                    const float T = fmaf((float)pl[2], 65536.0f, fmaf((float)pl[1], 256.0f, (float)pl[0]));
                    acc[r] = fmaf(T, cur.s[r][c] * xs[c], acc[r]);
                }
            }
        }
        const float sum = wave_reduce_v<RPW>(acc, lane);
        const int vi = lane >> (6 - LV);
        if ((lane & ((64 >> LV) - 1)) == 0 && g * RPW + vi < M) y[g * RPW + vi] = sum;
    }
}

int launch_gemv_q8r(hipStream_t st, const void *R, const float *x, float *y, uint32_t M, uint32_t nb,
                    uint32_t *xp_ws, bool planes_ready) {
    if (!planes_ready) k_xbytes<<<(8 * nb + 255) / 256, 256, 0, st>>>(x, xp_ws, nb);
    const uint32_t ngroups = (M + 3) / 4;
    uint32_t grid = (ngroups + 3) / 4;
    if (grid > 1024) grid = 1024;
    const u32x4q *D = (const u32x4q *)R;
    const float *S = (const float *)((const unsigned char *)R + (size_t)M * nb * 32);
    k_q8rmv<4><<<grid, 256, 0, st>>>(D, S, xp_ws, y, M, nb);
    return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
}

int launch_gemv_q8(hipStream_t st, const uint32_t *W, const float *x, float *y, uint32_t M, uint32_t nb,
                   uint32_t *xp_ws) {
    k_xbytes<<<(8 * nb + 255) / 256, 256, 0, st>>>(x, xp_ws, nb);
    const uint32_t ngroups = (M + 1) / 2;
    uint32_t grid = (ngroups + 3) / 4;
    if (grid > 1024) grid = 1024;
    k_q8mv<2><<<grid, 256, 0, st>>>(W, xp_ws, y, M, nb);
    return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
}

// ---------------------------------------------------------------------
// Softcapped top-64 on 64-bit keys orderable(value) << 32 | ~index (unique;
// descending key order = value descending, ties by ascending index).  Pass
// 1: a workgroup takes 1024 logits; each wave sorts four 64-key groups with
// shuffle bitonic networks and merges them to its top 64, and the four
// waves' lists merge through LDS.  Pass 2 merges the sorted tile lists
// (below).
// ---------------------------------------------------------------------
constexpr int kTopK = 64;
constexpr int kTile = 1024;

__device__ __forceinline__ uint64_t topk_key(float v, uint32_t idx) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)u << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}
__device__ __forceinline__ float key_value(uint64_t k) {
    uint32_t u = (uint32_t)(k >> 32);
    u = (u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u;
    return __builtin_bit_cast(float, u);
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, m, 64);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), m, 64);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
    const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)v, src, 64);
    const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(v >> 32), src, 64);
    return ((uint64_t)hi << 32) | lo;
}

// The wave's 64 keys (one per lane) sorted descending across lanes.
__device__ __forceinline__ uint64_t wave_sort64_desc(uint64_t key, int lane) {
#pragma unroll
    for (int k = 2; k <= 64; k <<= 1)
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const uint64_t o = shfl_xor_u64(key, j);
            const bool desc = (lane & k) == 0, lo = (lane & j) == 0;
            const uint64_t mx = key > o ? key : o, mn = key > o ? o : key;
            key = (lo == desc) ? mx : mn;
        }
    return key;
}

// Top 64 of two descending 64-key lists, descending: the elementwise max of
// a and reversed b is a bitonic sequence holding them; half-cleaners sort it.
__device__ __forceinline__ uint64_t wave_merge64_desc(uint64_t a, uint64_t b, int lane) {
    const uint64_t br = shfl_u64(b, 63 - lane);
    uint64_t key = a > br ? a : br;
#pragma unroll
    for (int j = 32; j > 0; j >>= 1) {
        const uint64_t o = shfl_xor_u64(key, j);
        const uint64_t mx = key > o ? key : o, mn = key > o ? o : key;
        key = (lane & j) == 0 ? mx : mn;
    }
    return key;
}

__global__ __launch_bounds__(256) void k_topk_tile(const float *__restrict__ logits, uint32_t V,
                                                   uint64_t *__restrict__ cand) {
    __shared__ uint64_t sh[4][kTopK];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t base = blockIdx.x * kTile + wave * 256;
    uint64_t k[4];
    float lv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) lv[u] = logits[min(base + 64 * u + lane, V - 1)];   // all in flight
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const uint32_t idx = base + 64 * u + lane;
        // padding keys (0) sort below every real key
        const uint64_t key = topk_key(30.0f * tanhf(lv[u] * (1.0f / 30.0f)), idx);
        k[u] = idx < V ? key : 0ull;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) k[u] = wave_sort64_desc(k[u], lane);
    sh[wave][lane] = wave_merge64_desc(wave_merge64_desc(k[0], k[1], lane), wave_merge64_desc(k[2], k[3], lane), lane);
    __syncthreads();
    if (wave == 0) {
        const uint64_t a = wave_merge64_desc(sh[0][lane], sh[1][lane], lane);
        const uint64_t b = wave_merge64_desc(sh[2][lane], sh[3][lane], lane);
        cand[(size_t)blockIdx.x * kTopK + lane] = wave_merge64_desc(a, b, lane);
    }
}

// Pass 2.  With at least 64 lists, the 64th largest list head T bounds the
// answer from below (the 64 heads at or above it are 64 distinct keys), so
// only keys >= T matter, and only the 64 lists whose heads are at or above T
// hold any: each contributes the prefix of its sorted list at or above T
// (with fewer lists, T = 0 and every key is a candidate).  When the
// candidates number at most kTopkFast (the usual case: a few keys per list)
// they are gathered into LDS and each finds its rank by counting the larger
// ones (keys are unique, so the ranks are exact and the gather order does
// not matter); otherwise 16 waves fold every list with the 64 + 64 -> 64
// merge and a four-level tree.  Heads are ranked the same way.
constexpr int kTopkFast = 1024;

__global__ __launch_bounds__(1024) void k_topk_merge(const uint64_t *__restrict__ cand, uint32_t nlist,
                                                     uint32_t *__restrict__ ids, float *__restrict__ vals,
                                                     GreedyTail tail) {
    constexpr int U = 8;                 // lists loaded per wave per batch (full fold)
    constexpr int kMaxLists = 262144 / kTile;
    __shared__ uint64_t sh[16][kTopK];
    __shared__ uint64_t heads[kMaxLists];
    __shared__ uint64_t cbuf[kTopkFast];
    __shared__ uint64_t outk[kTopK];
    __shared__ uint32_t sel[kTopK];
    __shared__ uint32_t ncand;
    __shared__ uint64_t thr;
    const uint32_t tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const uint32_t nsel = nlist < (uint32_t)kTopK ? nlist : (uint32_t)kTopK;
    if (tid == 0) {
        ncand = 0;
        thr = 0ull;
    }
    if (tid < (uint32_t)kTopK) outk[tid] = 0ull;
    if (tid < nlist) heads[tid] = cand[(size_t)tid * kTopK];
    __syncthreads();
    if (tid < nlist) {
        const uint64_t h = heads[tid];
        uint32_t r = 0;
        for (uint32_t j = 0; j < nlist; ++j) r += heads[j] > h ? 1u : 0u;
        if (r < (uint32_t)kTopK) sel[r] = tid;                   // the list with the r-th largest head
        if (nlist >= (uint32_t)kTopK && r == (uint32_t)kTopK - 1) thr = h;
    }
    __syncthreads();
    const uint64_t T = thr;
    // gather the prefixes at or above T: wave w takes selected lists w, w +
    // 16, ...; the four lists' loads go out together (a wave past nsel
    // reads list sel[0] and drops it)
    uint64_t keys[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t i = wave + 16 * q;
        keys[q] = cand[(size_t)sel[i < nsel ? i : 0u] * kTopK + lane];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t i = wave + 16 * q;
        if (i >= nsel) continue;                                    // uniform per wave
        const uint64_t key = keys[q];
        const uint64_t above = __ballot(key >= T);                   // a prefix: the list is sorted
        const uint32_t cnt = __popcll(above);
        uint32_t off = 0;
        if (lane == 0) off = atomicAdd(&ncand, cnt);
        off = __shfl(off, 0, 64);
        if ((uint32_t)lane < cnt && off + lane < (uint32_t)kTopkFast) cbuf[off + lane] = key;
    }
    __syncthreads();
    const uint32_t n = ncand;
    uint64_t res = 0ull;
    if (n <= (uint32_t)kTopkFast) {
        if (tid < n) {
            const uint64_t k = cbuf[tid];
            uint32_t r = 0;
            for (uint32_t j = 0; j < n; ++j) r += cbuf[j] > k ? 1u : 0u;
            if (r < (uint32_t)kTopK) outk[r] = k;               // padding keys (0) all land on one rank
        }
        __syncthreads();
        if (wave == 0) res = outk[lane];
    } else {
        uint64_t acc = 0ull;             // the empty list: below every real key
        for (uint32_t l0 = wave; l0 < nlist; l0 += 16 * U) {
            uint64_t c[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const uint32_t l = l0 + 16 * u;
                c[u] = l < nlist ? cand[(size_t)l * kTopK + lane] : 0ull;
            }
#pragma unroll
            for (int u = 0; u < U; ++u) acc = wave_merge64_desc(acc, c[u], lane);
        }
        sh[wave][lane] = acc;
        __syncthreads();
#pragma unroll
        for (int s = 8; s >= 1; s >>= 1) {
            if (wave < s) acc = wave_merge64_desc(sh[wave][lane], sh[wave + s][lane], lane);
            __syncthreads();
            if (wave < s) sh[wave][lane] = acc;
            __syncthreads();
        }
        res = acc;
    }
    if (wave == 0) {
        const uint32_t id = res ? 0xFFFFFFFFu - (uint32_t)res : 0u;
        ids[lane] = id;
        vals[lane] = res ? key_value(res) : -1e30f;
        if (tail.gen && lane == 0) {
            // a device-side greedy step: append the argmax, advance the clock
            const uint32_t count = tail.gen[1];
            if (count < tail.cap) tail.out[count] = id;
            tail.gen[1] = count + 1;
            tail.gen[0] = tail.gen[0] + 1;
        }
    }
}

size_t topk_ws_bytes(uint32_t V) { return (size_t)((V + kTile - 1) / kTile) * kTopK * 8; }

int launch_topk64(hipStream_t st, const float *logits, uint32_t V, uint32_t *ids, float *vals, uint64_t *ws,
                  const GreedyTail *tail) {
    const uint32_t tiles = (V + kTile - 1) / kTile;
    if (tiles) k_topk_tile<<<tiles, 256, 0, st>>>(logits, V, ws);
    k_topk_merge<<<1, 1024, 0, st>>>(ws, tiles, ids, vals, tail ? *tail : GreedyTail{nullptr, nullptr, 0});
    return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
}

// ---------------------------------------------------------------------
// Quantizers (bit-exact restatements of src/quant.zig:21-98) and the
// embedding gather x = bf16(embed[tok]) * sqrt(H).
// ---------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

__global__ void k_quantize_q4(const uint16_t *__restrict__ src, uint32_t *__restrict__ dst, uint64_t nblk) {
    // separate roundings of v * id and + 8, as the reference computes them
    // (HIP contracts a * b + c into one fma by default)
    #pragma clang fp contract(off)
    const uint64_t blk = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= nblk) return;
    const uint16_t *s = src + blk * 32;
    float v[32], amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        v[i] = bf16_bits_to_f32(s[i]);
        amax = fmaxf(amax, fabsf(v[i]));
    }
    const float d = amax / 8.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    // min = f16(-8 d): d >= 0, so it is f16(8 d) with the sign bit set
    // (written out so that d = 0 gives -0.0 as the reference's f16 cast does)
    const uint32_t sc = __builtin_bit_cast(unsigned short, (_Float16)d);
    const uint32_t mn = __builtin_bit_cast(unsigned short, (_Float16)(8.0f * d)) | 0x8000u;
    uint32_t *o = dst + blk * 5;
    o[0] = sc | (mn << 16);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t word = 0;
#pragma unroll
        for (int n = 0; n < 8; ++n) {
            const float t = v[8 * w + n] * id + 8.0f;
            int q = (int)roundf(t);
            q = q < 0 ? 0 : (q > 15 ? 15 : q);
            word |= (uint32_t)q << (4 * n);
        }
        o[1 + w] = word;
    }
}

__global__ void k_quantize_q8(const uint16_t *__restrict__ src, uint32_t *__restrict__ dst, uint64_t nblk) {
    #pragma clang fp contract(off)
    const uint64_t blk = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= nblk) return;
    const uint16_t *s = src + blk * 32;
    float v[32], amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
        v[i] = bf16_bits_to_f32(s[i]);
        amax = fmaxf(amax, fabsf(v[i]));
    }
    const float d = amax / 127.0f;
    const float id = amax > 0.0f ? 127.0f / amax : 0.0f;
    uint32_t *o = dst + blk * 9;
    o[0] = __builtin_bit_cast(uint32_t, d);
#pragma unroll
    for (int w = 0; w < 8; ++w) {
        uint32_t word = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            int q = (int)roundf(v[4 * w + j] * id);
            q = q < -128 ? -128 : (q > 127 ? 127 : q);
            word |= ((uint32_t)q & 0xffu) << (8 * j);
        }
        o[1 + w] = word;
    }
}

__global__ void k_embed(const uint16_t *__restrict__ table, const uint32_t *__restrict__ tokens, uint32_t n,
                        uint32_t H, float scale, float *__restrict__ x) {
    const uint32_t t = blockIdx.y;
    if (t >= n) return;
    const uint16_t *row = table + (size_t)tokens[t] * H;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < H; i += gridDim.x * blockDim.x)
        x[(size_t)t * H + i] = bf16_bits_to_f32(row[i]) * scale;
}

__global__ void k_to_bf16_bits(const float *__restrict__ src, uint16_t *__restrict__ dst, size_t n) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (; i < n; i += stride) {
        const uint32_t u = __builtin_bit_cast(uint32_t, src[i]);
        dst[i] = (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    }
}

int launch_embed(hipStream_t st, const uint16_t *table, const uint32_t *tokens, uint32_t n, uint32_t H, float scale,
                 float *x) {
    dim3 grid((H + 255) / 256, n);
    k_embed<<<grid, 256, 0, st>>>(table, tokens, n, H, scale, x);
    return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
}

int launch_quantize(hipStream_t st, int q8, const uint16_t *src, uint32_t *dst, uint64_t nblk) {
    if (!nblk) return CHN_OK;
    if (q8) k_quantize_q8<<<(unsigned)((nblk + 255) / 256), 256, 0, st>>>(src, dst, nblk);
    else k_quantize_q4<<<(unsigned)((nblk + 255) / 256), 256, 0, st>>>(src, dst, nblk);
    return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
}

}  // namespace chn

using namespace chn;

extern "C" int chn_gemv_q8(chn_ctx *ctx, const uint32_t *W, const float *x, float *y, uint32_t M, uint32_t K) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, W && x && y, "NULL argument");
    CHN_REQUIRE(ctx, K % 128 == 0 && K > 0 && K <= 4096, "K=%u: the Q8 matvec needs K %% 128 == 0, K <= 4096", K);
    CHN_REQUIRE(ctx, aligned(W, 16) && aligned(x, 16), "W and x must be 16-byte aligned");
    if (!M) return CHN_OK;
    int rc = ensure_workspace(ctx, xbytes_bytes(K / 32));
    if (rc) return rc;
    launch_gemv_q8(ctx->stream, W, x, y, M, K / 32, (uint32_t *)ctx->ws);
    CHN_LAUNCHED(ctx, "k_q8mv");
    return CHN_OK;
}

extern "C" int chn_q8_repack(chn_ctx *ctx, const uint32_t *W, uint32_t rows, uint32_t K, void *dst) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, W && dst, "NULL argument");
    CHN_REQUIRE(ctx, K % 32 == 0, "K=%u must be a multiple of 32", K);
    CHN_REQUIRE(ctx, aligned(dst, 16), "dst must be 16-byte aligned");
    if (launch_q8_repack(ctx->stream, W, rows, K / 32, dst)) return hip_fail(ctx, hipGetLastError(), "k_repack_q8");
    return CHN_OK;
}

extern "C" int chn_gemv_q8r(chn_ctx *ctx, const void *R, const float *x, float *y, uint32_t M, uint32_t K) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, R && x && y, "NULL argument");
    CHN_REQUIRE(ctx, K % 128 == 0 && K > 0 && K <= 4096, "K=%u: the Q8 matvec needs K %% 128 == 0, K <= 4096", K);
    CHN_REQUIRE(ctx, aligned(R, 16) && aligned(x, 16), "R and x must be 16-byte aligned");
    if (!M) return CHN_OK;
    int rc = ensure_workspace(ctx, xbytes_bytes(K / 32));
    if (rc) return rc;
    launch_gemv_q8r(ctx->stream, R, x, y, M, K / 32, (uint32_t *)ctx->ws);
    CHN_LAUNCHED(ctx, "k_q8rmv");
    return CHN_OK;
}

extern "C" int chn_topk64(chn_ctx *ctx, const float *logits, uint32_t V, uint32_t *ids, float *vals) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, logits && ids && vals, "NULL argument");
    CHN_REQUIRE(ctx, V > 0 && V <= 262144, "V=%u must be in 1..262144", V);
    int rc = ensure_workspace(ctx, topk_ws_bytes(V));
    if (rc) return rc;
    launch_topk64(ctx->stream, logits, V, ids, vals, (uint64_t *)ctx->ws);
    CHN_LAUNCHED(ctx, "k_topk");
    return CHN_OK;
}

extern "C" int chn_quantize_q4(chn_ctx *ctx, const uint16_t *src_bf16, uint32_t *dst, uint32_t rows, uint32_t cols) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, src_bf16 && dst, "NULL argument");
    CHN_REQUIRE(ctx, cols % 32 == 0, "cols=%u must be a multiple of 32", cols);
    const uint64_t nblk = (uint64_t)rows * (cols / 32);
    if (!nblk) return CHN_OK;
    k_quantize_q4<<<(unsigned)((nblk + 255) / 256), 256, 0, ctx->stream>>>(src_bf16, dst, nblk);
    CHN_LAUNCHED(ctx, "k_quantize_q4");
    return CHN_OK;
}

extern "C" int chn_quantize_q8(chn_ctx *ctx, const uint16_t *src_bf16, uint32_t *dst, uint32_t rows, uint32_t cols) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, src_bf16 && dst, "NULL argument");
    CHN_REQUIRE(ctx, cols % 32 == 0, "cols=%u must be a multiple of 32", cols);
    const uint64_t nblk = (uint64_t)rows * (cols / 32);
    if (!nblk) return CHN_OK;
    k_quantize_q8<<<(unsigned)((nblk + 255) / 256), 256, 0, ctx->stream>>>(src_bf16, dst, nblk);
    CHN_LAUNCHED(ctx, "k_quantize_q8");
    return CHN_OK;
}

extern "C" int chn_to_bf16_bits(chn_ctx *ctx, const float *src, uint16_t *dst, size_t n) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, (src && dst) || !n, "NULL argument");
    if (!n) return CHN_OK;
    size_t g = (n + 255) / 256;
    if (g > 65536) g = 65536;
    k_to_bf16_bits<<<(unsigned)g, 256, 0, ctx->stream>>>(src, dst, n);
    CHN_LAUNCHED(ctx, "k_to_bf16_bits");
    return CHN_OK;
}
