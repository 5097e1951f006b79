// Batch-1 decode matvecs over the reference's Q4 layout on gfx950:
// gemv_q4 (shaders/gemv_q4.wgsl), fused_qkv_q4 (shaders/fused_qkv_q4.wgsl)
// and fused_mlp_q4 (shaders/fused_mlp_q4.wgsl).
//
// The weight stream is HBM-bound; the design keeps the VALU cost per weight
// near one instruction so that the issue rate never caps the stream:
//
//  * Activations are turned once per call into "digit planes": per 32-block
//    b, X_i = rint(x_i * 2^(18-e_b)) with |x_i| < 2^e_b, written as five
//    balanced base-16 digits D_p in [-8, 7] (X = sum_p D_p 16^p), and each
//    digit plane packed as signed 4-bit lanes in the same nibble order as
//    the weights.  The quantisation error is <= 2^-18 of the block maximum,
//    the size of fp32's own rounding noise over a few thousand products.
//  * A Q4 word XOR 0x88888888 is exactly the eight signed 4-bit values
//    (q - 8), so sum_i (q_i - 8) X_i is an exact integer computed with
//    v_dot8c_i32_i4 (8 MACs per instruction), plane by plane in Horner
//    form; the block result is (float)T * scale_b * 2^(e_b - 18).
//  * Weights are streamed with coalesced non-temporal 16-byte loads of whole
//    row segments (prefetching the next row group into VGPRs while the
//    current one is computed), transposed through LDS to one lane per
//    20-byte block.  Waves are persistent and walk row groups with a
//    grid-wide stride, so the chip reads W as one contiguous front.
//  * WPR waves of a workgroup may split K; their partials meet in LDS in a
//    fixed order, so results are deterministic.
#include "chn_internal.h"

namespace chn {

// Four threads per 32-block, one per 8-element weight word.
__global__ __launch_bounds__(256) void k_xplanes(const float *__restrict__ x, uint32_t *__restrict__ xp,
                                                 uint32_t nb) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    const uint32_t b = t >> 2, w = t & 3;
    const bool ok = b < nb;
    float v[8];
    if (ok) {
        const float4 *xv = (const float4 *)(x + (size_t)b * 32 + w * 8);
        const float4 t0 = xv[0], t1 = xv[1];
        v[0] = t0.x; v[1] = t0.y; v[2] = t0.z; v[3] = t0.w;
        v[4] = t1.x; v[5] = t1.y; v[6] = t1.z; v[7] = t1.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.0f;
    }
    emit_planes8(v, xp, nb, b, w, ok);
}

int launch_xplanes(hipStream_t s, const float *x, uint32_t *xp, uint32_t nb) {
    k_xplanes<<<(4 * nb + 255) / 256, 256, 0, s>>>(x, xp, nb);
    return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
}

enum MatvecMode { MV_GEMV = 0, MV_QKV = 1, MV_MLP = 2 };

struct MatvecArgs {
    const uint32_t *W0, *W1, *W2;  // GEMV: W0. QKV: Wq, Wk, Wv. MLP: Wg, Wu.
    float *y0, *y1, *y2;           // GEMV: y0. QKV: q, k, v. MLP: act.
    const uint32_t *xp;            // activation digit planes
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

template <int MODE>
__device__ __forceinline__ void store_row(const MatvecArgs &a, uint32_t row, float v) {
    if (MODE == MV_QKV) {
        if (row < a.seg1) a.y0[row] = v;
        else if (row < a.seg2) a.y1[row - a.seg1] = v;
        else a.y2[row - a.seg2] = v;
    } else {
        a.y0[row] = v;
    }
}

// sum_i (q_i - 8) X_i for one block: q words XOR 8 per nibble, Horner over
// the digit planes (top plane first).
__device__ __forceinline__ int block_idot(const uint32_t *q, const uint32_t (&P)[XP_WORDS]) {
    uint32_t s[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) s[w] = q[w] ^ 0x88888888u;
    int acc = 0;
#pragma unroll
    for (int p = XP_PLANES - 1; p >= 0; --p) {
        if (p != XP_PLANES - 1) acc <<= 4;
#pragma unroll
        for (int w = 0; w < 4; ++w) acc = __builtin_amdgcn_sdot8((int)s[w], (int)P[p * 4 + w], acc, false);
    }
    return acc;
}

__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxBlocksPerWave = 128;          // two 64-block passes
constexpr int kSegWords = kMaxBlocksPerWave * 5; // LDS words per stream

// RPW rows (x NMAT matrices) per wave and row group; WPR waves split K.
// XIN (WPR == 1, K <= 4096): the workgroup converts x to digit planes in LDS
// itself (the same planes as k_xplanes), so the call is one launch; x's
// loads are issued before the first weights, the conversion runs while
// those are in flight.  A row segment is NJ 16-byte loads per lane
// (NJ = ceil(chunks / 64), chosen by the host), every one unconditional:
// indices past the segment or the matrix are clamped into it and their
// data is never used, so the compiler's waits for x leave the weights in
// flight.
template <int MODE, int RPW, int WPR, bool XIN, int NJ>
__global__ __launch_bounds__(256) void k_q4mv(MatvecArgs a, const float *__restrict__ x) {
    constexpr int NMAT = (MODE == MV_MLP) ? 2 : 1;
    constexpr int V = RPW * NMAT;
    constexpr int G = 4 / WPR;
    constexpr int LV = (V == 1) ? 0 : (V == 2) ? 1 : (V == 4) ? 2 : 3;
    static_assert(V == 1 || V == 2 || V == 4 || V == 8, "V must be a power of two <= 8");
    static_assert(NJ >= 1 && NJ <= 3, "a wave's segment is at most 128 blocks");

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int grp = wave / WPR, part = wave % WPR;
    const uint32_t nb = a.nb;

    // K range of this wave: blocks [kb0, kb0 + nblk), nblk % 4 == 0 (host
    // guarantees nb % 4 == 0 and per-wave ranges <= 128 blocks).
    const uint32_t per = (((nb + WPR - 1) / WPR) + 3) / 4 * 4;
    const uint32_t kb0 = part * per;
    const uint32_t kb1 = (kb0 + per < nb) ? kb0 + per : nb;
    const uint32_t nblk = kb1 > kb0 ? kb1 - kb0 : 0;
    const uint32_t chunks = nblk * 5 / 4;   // 16-byte chunks per stream segment

    __shared__ uint32_t seg[4][V * kSegWords];
    __shared__ float red[4][V];
    constexpr int kPl = XP_WORDS + 1;             // LDS words per block of planes
    __shared__ uint32_t lpl[XIN ? 128 * kPl : 1];
    uint32_t *L = seg[wave];

    // XIN: x's values, four threads per 32-block (eight values each), two passes
    // (loads clamped into x, values past it zeroed)
    float xv[XIN ? 2 : 1][8];
    if (XIN) {
#pragma unroll
        for (int ps = 0; ps < 2; ++ps) {
            const uint32_t b = ps * 64 + (threadIdx.x >> 2), w = threadIdx.x & 3;
            const uint32_t bc = min(b, nb - 1);
            const float4 t0 = *(const float4 *)(x + (size_t)bc * 32 + w * 8);
            const float4 t1 = *(const float4 *)(x + (size_t)bc * 32 + w * 8 + 4);
            const float z = b < nb ? 1.0f : 0.0f;
            xv[ps][0] = t0.x * z; xv[ps][1] = t0.y * z; xv[ps][2] = t0.z * z; xv[ps][3] = t0.w * z;
            xv[ps][4] = t1.x * z; xv[ps][5] = t1.y * z; xv[ps][6] = t1.z * z; xv[ps][7] = t1.w * z;
        }
    }

    const uint32_t ngroups = (a.M + RPW - 1) / RPW;
    const uint32_t gstride = gridDim.x * G;
    u32x4 pf[V][NJ];
    // clamps: the last chunk of the segment (a wave without blocks reads
    // the row's first chunk), the last row of the matrix
    const uint32_t c_last = chunks ? chunks - 1 : 0u;
    const uint32_t kb_ld = nblk ? kb0 : 0u;

    auto load = [&](uint32_t g) {
#pragma unroll
        for (int s = 0; s < V; ++s) {
            const uint32_t row = min(g * RPW + s / NMAT, a.M - 1);
            const uint32_t *base = row_base<MODE>(a, row, s % NMAT) + (size_t)kb_ld * 5;
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const uint32_t c = min(lane + 64 * j, c_last);
                pf[s][j] = __builtin_nontemporal_load((const u32x4 *)base + c);
            }
        }
    };

    uint32_t g = blockIdx.x * G + grp;
    load(g < ngroups ? g : ngroups - 1);    // unconditional: a wave past the groups never uses it

    // this lane's two blocks of activation planes
    uint32_t P[2][XP_WORDS];
    float xs[2];
    if (XIN) {
#pragma unroll
        for (int ps = 0; ps < 2; ++ps) {
            const uint32_t b = ps * 64 + (threadIdx.x >> 2);
            emit_planes8s(xv[ps], lpl, 1, kPl, b, threadIdx.x & 3, b < nb);
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const uint32_t bl = c * 64 + lane;
            const bool ok = bl < nblk;
            const uint32_t *src = lpl + (ok ? bl : 0u) * kPl;
#pragma unroll
            for (int i = 0; i < XP_WORDS; ++i) P[c][i] = ok ? src[i] : 0u;
            xs[c] = ok ? __builtin_bit_cast(float, src[XP_WORDS]) : 0.0f;
        }
    } else {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const uint32_t bl = c * 64 + lane;
            const bool ok = bl < nblk;
            const uint32_t b = kb0 + bl;
#pragma unroll
            for (int i = 0; i < XP_WORDS; ++i) P[c][i] = ok ? a.xp[(size_t)i * nb + b] : 0u;
            xs[c] = ok ? ((const float *)(a.xp + (size_t)XP_WORDS * nb))[b] : 0.0f;
        }
    }

    for (uint32_t gb = blockIdx.x * G; gb < ngroups; gb += gstride, g += gstride) {
        const bool gv = g < ngroups;
        if (gv) {
#pragma unroll
            for (int s = 0; s < V; ++s)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    const uint32_t c = lane + 64 * j;
                    if (c < chunks) *(u32x4 *)(L + s * kSegWords + 4 * c) = pf[s][j];
                }
        }
        wave_lds_fence();
        if (g + gstride < ngroups) load(g + gstride);

        float acc[V];
#pragma unroll
        for (int v = 0; v < V; ++v) acc[v] = 0.0f;
        if (gv) {
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const uint32_t bl = c * 64 + lane;
                if (bl < nblk) {
#pragma unroll
                    for (int s = 0; s < V; ++s) {
                        const uint32_t *p = L + s * kSegWords + 5 * bl;
                        const uint32_t w0 = p[0];
                        const uint32_t q[4] = {p[1], p[2], p[3], p[4]};
                        const int T = block_idot(q, P[c]);
                        acc[s] = fmaf((float)T, f16_lo_to_f32(w0) * xs[c], acc[s]);
                    }
                }
            }
        }
        wave_lds_fence();

        const float sum = wave_reduce_v<V>(acc, lane);
        const int vi = lane >> (6 - LV);
        const bool owner = (lane & ((64 >> LV) - 1)) == 0;
        if (WPR == 1) {
            if (gv) {
                if (NMAT == 1) {
                    const uint32_t row = g * RPW + vi;
                    if (owner && row < a.M) store_row<MODE>(a, row, sum);
                } else {
                    const float other = __shfl_xor(sum, 64 >> LV, 64);
                    const uint32_t row = g * RPW + (vi >> 1);
                    if (owner && (vi & 1) == 0 && row < a.M) a.y0[row] = gelu_tanh(sum) * other;
                }
            }
        } else {
            if (owner) red[wave][vi] = sum;
            __syncthreads();
            if (part == 0 && gv && lane < V) {
                float t = 0.0f;
#pragma unroll
                for (int w = 0; w < WPR; ++w) t += red[grp * WPR + w][lane];
                if (NMAT == 1) {
                    const uint32_t row = g * RPW + lane;
                    if (row < a.M) store_row<MODE>(a, row, t);
                } else {
                    const float other = __shfl_xor(t, 1, 64);
                    const uint32_t row = g * RPW + (lane >> 1);
                    if ((lane & 1) == 0 && row < a.M) a.y0[row] = gelu_tanh(t) * other;
                }
            }
            __syncthreads();
        }
    }
}

struct MvShape {
    int rpw, wpr;
    uint32_t grid;
};

// Launch shape (from a sweep on MI355X over the 12B decode shapes): the
// fewest waves splitting K such that each wave covers <= 128 blocks; two
// rows per wave (one gate/up row pair for the fused MLP, four for a plain
// GEMV without a K split); at most 1024 workgroups (4 per CU), persistent
// over row groups beyond that.
static MvShape pick_shape(int mode, uint32_t M, uint32_t nb) {
    MvShape s;
    s.wpr = nb <= 128 ? 1 : (nb <= 256 ? 2 : 4);
    // a plain GEMV whose rows fit one wave: four rows per wave, so each of
    // the fewer workgroups converts x once for twice the rows (8192 x 2048:
    // 6.15 us against 6.45 us at two rows)
    s.rpw = mode == MV_MLP ? 1 : (mode == MV_GEMV && s.wpr == 1 ? 4 : 2);
    const uint32_t G = 4 / s.wpr;
    const uint32_t ngroups = (M + s.rpw - 1) / s.rpw;
    const uint32_t grid = (ngroups + G - 1) / G;
    s.grid = grid < 1024 ? grid : 1024;
    return s;
}

template <int MODE, int WPR, bool XIN, int NJ>
static bool launch_nj(int rpw, const MatvecArgs &a, const float *x, uint32_t grid, hipStream_t st) {
    constexpr int NMAT = MODE == MV_MLP ? 2 : 1;
    switch (rpw) {
    case 1: k_q4mv<MODE, 1, WPR, XIN, NJ><<<grid, 256, 0, st>>>(a, x); return true;
    case 2: k_q4mv<MODE, 2, WPR, XIN, NJ><<<grid, 256, 0, st>>>(a, x); return true;
    case 4:
        if constexpr (4 * NMAT <= 8) { k_q4mv<MODE, 4, WPR, XIN, NJ><<<grid, 256, 0, st>>>(a, x); return true; }
        return false;
    }
    return false;
}

// NJ: 16-byte loads per lane for the widest wave segment (the kernel's
// per-wave block count, rounded as it rounds it)
template <int MODE, int WPR, bool XIN>
static bool launch_wpr(int rpw, const MatvecArgs &a, const float *x, uint32_t grid, hipStream_t st) {
    const uint32_t per = (((a.nb + WPR - 1) / WPR) + 3) / 4 * 4;
    const uint32_t chunks = (per < a.nb ? per : a.nb) * 5 / 4;
    const uint32_t nj = (chunks + 63) / 64;
    if (nj <= 1) return launch_nj<MODE, WPR, XIN, 1>(rpw, a, x, grid, st);
    if (nj == 2) return launch_nj<MODE, WPR, XIN, 2>(rpw, a, x, grid, st);
    if (nj == 3) return launch_nj<MODE, WPR, XIN, 3>(rpw, a, x, grid, st);
    return false;
}

// x != NULL: planes computed in the kernel (one wave per row: nb <= 128);
// otherwise a.xp holds them.
template <int MODE>
static bool launch_mode(const MvShape &s, const MatvecArgs &a, const float *x, hipStream_t st) {
    if (x) return s.wpr == 1 && launch_wpr<MODE, 1, true>(s.rpw, a, x, s.grid, st);
    switch (s.wpr) {
    case 1: return launch_wpr<MODE, 1, false>(s.rpw, a, nullptr, s.grid, st);
    case 2: return launch_wpr<MODE, 2, false>(s.rpw, a, nullptr, s.grid, st);
    case 4: return launch_wpr<MODE, 4, false>(s.rpw, a, nullptr, s.grid, st);
    }
    return false;
}


// ---------------------------------------------------------------------
// General-shape fallback (any K % 32 == 0, any 4-byte alignment): one lane
// per block, fp32 FMAs over v_cvt_f32_ubyteN, activations in registers
// reused over RPW rows, fixed-order LDS reduction.
// ---------------------------------------------------------------------
struct GenericArgs {
    const uint32_t *W0, *W1, *W2;
    float *y0, *y1, *y2;
    const float *x;
    uint32_t M, seg1, seg2, nb;
};

template <int MODE>
__device__ __forceinline__ const uint32_t *gen_row_base(const GenericArgs &a, uint32_t row, int mat) {
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
__global__ __launch_bounds__(256) void k_q4mv_generic(GenericArgs a) {
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
            rp[r * NMAT + m] = gen_row_base<MODE>(a, row < a.M ? row : 0, m);
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
static void gen_launch_one(const GenericArgs &a, uint32_t grid, hipStream_t s) {
    k_q4mv_generic<MODE, RPW, WPR><<<dim3(grid), dim3(256), 0, s>>>(a);
}

template <int MODE, int WPR>
static bool gen_launch_rpw(int rpw, const GenericArgs &a, uint32_t grid, hipStream_t s) {
    constexpr int NMAT = (MODE == MV_MLP) ? 2 : 1;
    constexpr int G = 4 / WPR;
    switch (rpw) {
    case 1:
        if constexpr (G * 1 * NMAT >= 4) { gen_launch_one<MODE, 1, WPR>(a, grid, s); return true; }
        return false;
    case 2:
        if constexpr (G * 2 * NMAT >= 4) { gen_launch_one<MODE, 2, WPR>(a, grid, s); return true; }
        return false;
    case 4:
        gen_launch_one<MODE, 4, WPR>(a, grid, s);
        return true;
    case 8:
        if constexpr (NMAT == 1) { gen_launch_one<MODE, 8, WPR>(a, grid, s); return true; }
        return false;
    }
    return false;
}

// Picks the launch shape: WPR waves split the column passes of a row group
// when a row has several 64-block passes; RPW (rows per wave) is the
// largest that still puts >= 3072 waves on the 1024 SIMDs.
static int launch_generic(chn_ctx *ctx, int mode, const GenericArgs &a) {
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
        ok = wpr == 1 ? gen_launch_rpw<MV_GEMV, 1>(rpw, a, grid, s)
           : wpr == 2 ? gen_launch_rpw<MV_GEMV, 2>(rpw, a, grid, s)
                      : gen_launch_rpw<MV_GEMV, 4>(rpw, a, grid, s);
        break;
    case MV_QKV:
        ok = wpr == 1 ? gen_launch_rpw<MV_QKV, 1>(rpw, a, grid, s)
           : wpr == 2 ? gen_launch_rpw<MV_QKV, 2>(rpw, a, grid, s)
                      : gen_launch_rpw<MV_QKV, 4>(rpw, a, grid, s);
        break;
    default:
        ok = wpr == 1 ? gen_launch_rpw<MV_MLP, 1>(rpw, a, grid, s)
           : wpr == 2 ? gen_launch_rpw<MV_MLP, 2>(rpw, a, grid, s)
                      : gen_launch_rpw<MV_MLP, 4>(rpw, a, grid, s);
        break;
    }
    if (!ok) return set_err(ctx, CHN_E_UNSUPPORTED, "no matvec tile for M=%u nb=%u", a.M, a.nb);
    CHN_LAUNCHED(ctx, "k_q4mv_generic");
    return CHN_OK;
}


// x (fp32, K) -> digit planes (in the matvec's own LDS for K <= 4096, else
// into xp_ws, xplanes_bytes(K/32), by a separate pass), then the matvec.
int launch_matvec(chn_ctx *ctx, int mode, MatvecArgs a, const float *x, uint32_t *xp_ws, bool planes_ready) {
    const uint32_t nb = a.nb;
    const bool fast = nb % 4 == 0 && nb <= 512 && aligned(a.W0, 16) && (!a.W1 || aligned(a.W1, 16)) &&
                      (!a.W2 || aligned(a.W2, 16));
    if (!fast) {
        GenericArgs g{a.W0, a.W1, a.W2, a.y0, a.y1, a.y2, x, a.M, a.seg1, a.seg2, nb};
        return launch_generic(ctx, mode, g);
    }
    const MvShape s = pick_shape(mode, a.M, nb);
    // one wave per row (K <= 4096): the kernel makes the planes itself
    const float *xin = (!planes_ready && s.wpr == 1) ? x : nullptr;
    uint32_t *xp = xp_ws;
    if (!planes_ready && !xin) {
        k_xplanes<<<(4 * nb + 255) / 256, 256, 0, ctx->stream>>>(x, xp, nb);
        CHN_LAUNCHED(ctx, "k_xplanes");
    }
    a.xp = xp;
    bool ok = mode == MV_GEMV ? launch_mode<MV_GEMV>(s, a, xin, ctx->stream)
            : mode == MV_QKV  ? launch_mode<MV_QKV>(s, a, xin, ctx->stream)
                              : launch_mode<MV_MLP>(s, a, xin, ctx->stream);
    if (!ok) return set_err(ctx, CHN_E_UNSUPPORTED, "no matvec tile for M=%u nb=%u", a.M, nb);
    CHN_LAUNCHED(ctx, "k_q4mv");
    return CHN_OK;
}

size_t mv_ws_bytes(uint32_t K) { return xplanes_bytes(K / 32); }

int mv_gemv(chn_ctx *ctx, const uint32_t *W, const float *x, float *y, uint32_t M, uint32_t K, uint32_t *ws,
            bool planes_ready) {
    MatvecArgs a{W, nullptr, nullptr, y, nullptr, nullptr, nullptr, M, M, M, K / 32};
    return launch_matvec(ctx, MV_GEMV, a, x, ws, planes_ready);
}
int mv_qkv(chn_ctx *ctx, const uint32_t *Wq, const uint32_t *Wk, const uint32_t *Wv, const float *x, float *q,
           float *k, float *v, uint32_t q_dim, uint32_t kv_dim, uint32_t K, uint32_t *ws, bool planes_ready) {
    MatvecArgs a{Wq, Wk, Wv, q, k, v, nullptr, q_dim + 2 * kv_dim, q_dim, q_dim + kv_dim, K / 32};
    return launch_matvec(ctx, MV_QKV, a, x, ws, planes_ready);
}
int mv_mlp(chn_ctx *ctx, const uint32_t *Wg, const uint32_t *Wu, const float *x, float *act, uint32_t M, uint32_t K,
           uint32_t *ws, bool planes_ready) {
    MatvecArgs a{Wg, Wu, nullptr, act, nullptr, nullptr, nullptr, M, M, M, K / 32};
    return launch_matvec(ctx, MV_MLP, a, x, ws, planes_ready);
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
    MatvecArgs a{W, nullptr, nullptr, y, nullptr, nullptr, nullptr, M, M, M, K / 32};
    rc = ensure_workspace(ctx, xplanes_bytes(K / 32));
    if (rc) return rc;
    return launch_matvec(ctx, MV_GEMV, a, x, (uint32_t *)ctx->ws, false);
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
    MatvecArgs a{Wq, Wk, Wv, q, k, v, nullptr, (uint32_t)M, q_dim, q_dim + kv_dim, K / 32};
    rc = ensure_workspace(ctx, xplanes_bytes(K / 32));
    if (rc) return rc;
    return launch_matvec(ctx, MV_QKV, a, x, (uint32_t *)ctx->ws, false);
}

extern "C" int chn_fused_mlp_q4(chn_ctx *ctx, const uint32_t *Wg, const uint32_t *Wu,
                                const float *x, float *act, uint32_t M, uint32_t K) {
    if (!ctx) return CHN_E_INVALID;
    int rc = check_common(ctx, x, K);
    if (rc) return rc;
    CHN_REQUIRE(ctx, Wg && Wu && act && aligned(Wg, 4) && aligned(Wu, 4), "NULL/misaligned argument");
    if (M == 0) return CHN_OK;
    MatvecArgs a{Wg, Wu, nullptr, act, nullptr, nullptr, nullptr, M, M, M, K / 32};
    rc = ensure_workspace(ctx, xplanes_bytes(K / 32));
    if (rc) return rc;
    return launch_matvec(ctx, MV_MLP, a, x, (uint32_t *)ctx->ws, false);
}
