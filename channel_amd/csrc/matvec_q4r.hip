// Batch-1 decode matvecs over repacked Q4 weights ("Q4R"), the layout the
// model keeps in HBM.  Same contractions as gemv_q4 / fused_qkv_q4 /
// fused_mlp_q4 (shaders/gemv_q4.wgsl, fused_qkv_q4.wgsl, fused_mlp_q4.wgsl):
//
//   y[r] = sum_b f16(s_rb) * sum_i (q_rbi - 8) * x[32 b + i]
//
// Q4R stores, per matrix, the 16 nibble bytes of every 32-block as one
// aligned 16-byte word ([rows][nb]) with each nibble XOR 8 -- exactly the
// signed value q - 8 in two's-complement 4-bit -- followed by the f16 scales
// ([rows][nb]).  The reference layout's f16 "min" half-word is never read
// by the dequantization (scale * (q - 8)) and is dropped: 18 bytes per 32
// weights instead of 20.  The repack is a pure bit permutation, so every
// product is the same as on the reference layout.
//
// Lane l of a wave owns blocks l and l + 64 of its K range: one aligned,
// fully coalesced 16-byte load (nibbles) and one 2-byte load (scale) per
// block, no LDS staging.  Activations arrive as digit planes (see
// chn_internal.h) held in registers; a block is 24 v_dot8c_i32_i4 in plane
// order, the exact integer sum is scaled once.  Waves are persistent over
// row groups; the next group's weights are in flight while the current one
// is reduced (DPP row sums + readlane).  Waves that split K (WPR > 1) meet
// in LDS in a fixed order.
#include "chn_internal.h"

namespace chn {

typedef uint32_t u32x4r __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void k_repack_q4(const uint32_t *__restrict__ src, u32x4r *__restrict__ N,
                                                   uint16_t *__restrict__ S, size_t nblk) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblk) return;
    const uint32_t *p = src + i * 5;
    N[i] = u32x4r{p[1] ^ 0x88888888u, p[2] ^ 0x88888888u, p[3] ^ 0x88888888u, p[4] ^ 0x88888888u};
    S[i] = (uint16_t)(p[0] & 0xffffu);
}

int launch_q4_repack(hipStream_t s, const uint32_t *W, uint32_t rows, uint32_t K, void *dst) {
    const size_t nblk = (size_t)rows * (K / 32);
    if (!nblk) return CHN_OK;
    u32x4r *N = (u32x4r *)dst;
    uint16_t *S = (uint16_t *)((unsigned char *)dst + nblk * 16);
    k_repack_q4<<<(unsigned)((nblk + 255) / 256), 256, 0, s>>>(W, N, S, nblk);
    return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
}

enum RMode { RV_GEMV = 0, RV_QKV = 1, RV_MLP = 2 };
constexpr uint32_t kRedIters = 8;   // row groups per workgroup at most, when waves split K

struct RMat {
    const u32x4r *N;
    const uint16_t *S;
};

struct RArgs {
    RMat m0, m1, m2;            // GEMV: m0. QKV: q, k, v. MLP: gate, up.
    float *y0, *y1, *y2;
    const uint32_t *xp;
    uint32_t M, seg1, seg2, nb;
    const uint32_t *skip;       // quiescence flag of the layer (NULL: never skipped)
};

// The wave's index in its workgroup, as a wave-uniform (scalar) value, so
// row pointers derived from it stay in SGPRs and loads take 32-bit lane
// offsets instead of per-lane 64-bit addresses.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// sum_i (q_i - 8) X_i of one block: the signed nibbles times each plane,
// in Horner order from the top plane (one accumulator: the dot's own add
// carries the running sum, so only the first needs a zero).  Exact: the
// partial sums stay below 2^30 in magnitude.
__device__ __forceinline__ int block_idot_r(const u32x4r s, const uint32_t (&P)[XP_WORDS]) {
    int acc = 0;
#pragma unroll
    for (int p = XP_PLANES - 1; p >= 0; --p) {
        if (p != XP_PLANES - 1) acc *= 16;
#pragma unroll
        for (int w = 0; w < 4; ++w) acc = __builtin_amdgcn_sdot8((int)s[w], (int)P[p * 4 + w], acc, false);
    }
    return acc;
}

// Whole-wave sums of V per-lane values; the V = 2 and V = 4 forms give
// each value the same summation tree (gate and up of one row match between
// the one-row and the two-row gate/up kernels bit for bit).
template <int V>
__device__ __forceinline__ void wave_sums(const float (&r)[V], float (&t)[V]) {
    if constexpr (V == 1) {
        t[0] = wave_sum64(r[0]);
    } else if constexpr (V % 4 == 0) {
#pragma unroll
        for (int i = 0; i < V; i += 4) {
            float q[4];
            wave_sum4(r[i], r[i + 1], r[i + 2], r[i + 3], q);
#pragma unroll
            for (int k = 0; k < 4; ++k) t[i + k] = q[k];
        }
    } else {
        static_assert(V % 2 == 0, "V must be 1 or even");
#pragma unroll
        for (int i = 0; i < V; i += 2) wave_sum2(r[i], r[i + 1], t[i], t[i + 1]);
    }
}

template <int MODE>
__device__ __forceinline__ void row_ptrs(const RArgs &a, uint32_t row, int mat, const u32x4r *&N,
                                         const uint16_t *&S) {
    const size_t nb = a.nb;
    if (MODE == RV_QKV) {
        if (row < a.seg1) {
            N = a.m0.N + row * nb;
            S = a.m0.S + row * nb;
        } else if (row < a.seg2) {
            N = a.m1.N + (row - a.seg1) * nb;
            S = a.m1.S + (row - a.seg1) * nb;
        } else {
            N = a.m2.N + (row - a.seg2) * nb;
            S = a.m2.S + (row - a.seg2) * nb;
        }
        return;
    }
    const RMat &m = (MODE == RV_MLP && mat == 1) ? a.m1 : a.m0;
    N = m.N + row * nb;
    S = m.S + row * nb;
}

template <int MODE>
__device__ __forceinline__ void store_r(const RArgs &a, uint32_t row, float v) {
    if (MODE == RV_QKV) {
        if (row < a.seg1) a.y0[row] = v;
        else if (row < a.seg2) a.y1[row - a.seg1] = v;
        else a.y2[row - a.seg2] = v;
    } else {
        a.y0[row] = v;
    }
}

template <int MODE, int RPW, int WPR>
__global__ __launch_bounds__(256) void k_q4rmv(RArgs a) {
    if (a.skip && *a.skip) return;            // a quiescent layer (uniform)
    constexpr int NMAT = (MODE == RV_MLP) ? 2 : 1;
    constexpr int V = RPW * NMAT;
    constexpr int G = 4 / WPR;
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const int grp = wave / WPR, part = wave % WPR;
    const uint32_t nb = a.nb;
    // K range of this wave: blocks [kb0, kb0 + nblk), nblk <= 128
    const uint32_t per = (nb + WPR - 1) / WPR;
    const uint32_t kb0 = part * per;
    const uint32_t kb1 = (kb0 + per < nb) ? kb0 + per : nb;
    const uint32_t nblk = kb1 > kb0 ? kb1 - kb0 : 0;
    const bool ok0 = (uint32_t)lane < nblk, ok1 = (uint32_t)(64 + lane) < nblk;
    // blocks without data read block 0 of the row (always valid) and are
    // zeroed through their planes
    const uint32_t b0 = ok0 ? kb0 + lane : 0u, b1 = ok1 ? kb0 + 64 + lane : 0u;
    // waves that split K park each row group's partial sums here and meet
    // once, after the loop (at most kRedIters row groups per workgroup)
    __shared__ float red[4][WPR > 1 ? kRedIters * V : 1];
    uint32_t it = 0;

    const uint32_t ngroups = (a.M + RPW - 1) / RPW;
    const uint32_t gstride = gridDim.x * G;
    u32x4r nq[V][2];
    uint16_t sq[V][2];
    auto load = [&](uint32_t g) {
#pragma unroll
        for (int s = 0; s < V; ++s) {
            uint32_t row = g * RPW + s / NMAT;
            row = row < a.M ? row : a.M - 1;
            const u32x4r *N;
            const uint16_t *S;
            row_ptrs<MODE>(a, row, s % NMAT, N, S);
            nq[s][0] = __builtin_nontemporal_load(N + b0);
            nq[s][1] = __builtin_nontemporal_load(N + b1);
            sq[s][0] = __builtin_nontemporal_load(S + b0);
            sq[s][1] = __builtin_nontemporal_load(S + b1);
        }
    };
    uint32_t g = blockIdx.x * G + grp;
    if (g < ngroups) load(g);

    // this lane's two blocks of activation planes (read from a valid block,
    // then masked, so no branches surround the loads)
    uint32_t P[2][XP_WORDS];
    float xs[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const bool ok = c ? ok1 : ok0;
        const uint32_t b = c ? b1 : b0;
#pragma unroll
        for (int i = 0; i < XP_WORDS; ++i) P[c][i] = a.xp[(size_t)i * nb + b];
        xs[c] = ((const float *)(a.xp + (size_t)XP_WORDS * nb))[b];
#pragma unroll
        for (int i = 0; i < XP_WORDS; ++i) P[c][i] = ok ? P[c][i] : 0u;
        xs[c] = ok ? xs[c] : 0.0f;
    }

    for (uint32_t gb = blockIdx.x * G; gb < ngroups; gb += gstride, g += gstride) {
        const bool gv = g < ngroups;
        u32x4r cq[V][2];
        uint16_t cs[V][2];
#pragma unroll
        for (int s = 0; s < V; ++s)
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                cq[s][c] = nq[s][c];
                cs[s][c] = sq[s][c];
            }
        if (g + gstride < ngroups) load(g + gstride);
        float part[V], tot[V];
#pragma unroll
        for (int s = 0; s < V; ++s) {
            float r = 0.0f;
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int T = block_idot_r(cq[s][c], P[c]);
                const float sf = (float)__builtin_bit_cast(_Float16, cs[s][c]);
                r = fmaf((float)T, sf * xs[c], r);
            }
            part[s] = r;
        }
        wave_sums<V>(part, tot);
        if (WPR == 1) {
            if (gv && lane == 0) {
#pragma unroll
                for (int r = 0; r < RPW; ++r) {
                    const uint32_t row = g * RPW + r;
                    if (row < a.M) {
                        if (NMAT == 1) store_r<MODE>(a, row, tot[r]);
                        else a.y0[row] = gelu_tanh(tot[2 * r]) * tot[2 * r + 1];
                    }
                }
            }
        } else {
            if (lane == 0) {
#pragma unroll
                for (int s = 0; s < V; ++s) red[wave][it * V + s] = tot[s];
            }
            ++it;
        }
    }
    if (WPR > 1) {
        // partial sums of the workgroup's row groups, parts in a fixed order
        __syncthreads();
        const uint32_t j = lane / RPW, r = lane % RPW;   // row group j, row r of it
        const uint32_t gj = blockIdx.x * G + grp + j * gstride;
        if (part == 0 && j < it && gj < ngroups) {
            float t0 = 0.0f, t1 = 0.0f;
#pragma unroll
            for (int w = 0; w < WPR; ++w) {
                t0 += red[grp * WPR + w][j * V + r * NMAT];
                if (NMAT == 2) t1 += red[grp * WPR + w][j * V + r * 2 + 1];
            }
            const uint32_t row = gj * RPW + r;
            if (row < a.M) {
                if (NMAT == 1) store_r<MODE>(a, row, t0);
                else a.y0[row] = gelu_tanh(t0) * t1;
            }
        }
    }
}

// ---- the decode step's norm as a matvec prologue ---------------------------

typedef float f32x4r __attribute__((ext_vector_type(4)));
// Eight values at 8t, or zeros when !ok.  The load itself is unconditional
// (chunk 0 when !ok): a branch around it would make the compiler's wait
// before the first use drain every load issued after it, the matvec's
// weights included.
__device__ __forceinline__ void ld8(const float *p, uint32_t t, bool ok, float (&v)[8]) {
    const size_t i = ok ? 8 * (size_t)t : 0;
    const f32x4r a = *(const f32x4r *)(p + i), b = *(const f32x4r *)(p + i + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    const uint32_t m = opaque_mask(ok);
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = mask_f(v[k], m);
}
__device__ __forceinline__ void st8(float *p, uint32_t t, const float (&v)[8]) {
    *(f32x4r *)(p + 8 * (size_t)t) = f32x4r{v[0], v[1], v[2], v[3]};
    *(f32x4r *)(p + 8 * (size_t)t + 4) = f32x4r{v[4], v[5], v[6], v[7]};
}
// Sum over the workgroup of C values per thread, in the order a workgroup of
// C x blockDim threads holding one value each would use: value c of thread
// t counts as thread t + c * blockDim ("virtual wave" w + c * waves).  DPP
// wave sums, then the virtual wave partials in index order.  One barrier:
// each call takes its own 16-float slice of LDS.
template <int C>
__device__ __forceinline__ float wg_sum_c(const float (&v)[C], float *sh) {
    const int nw = blockDim.x >> 6;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const float w = wave_sum64(v[c]);
        if ((threadIdx.x & 63) == 0) sh[(threadIdx.x >> 6) + c * nw] = w;
    }
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < C * nw; ++i) t += sh[i];
    return t;
}

// NormArgs' norm over dim values (dim % 32 == 0, dim <= 8 * C * blockDim):
// thread t holds the eight values 8 (t + c blockDim) .. + 7 of chunk c < C,
// four threads per 32-block.  The digit planes of y go to LDS block by block
// (kLdsBlk words per block: the plane words, then the scale; constant offsets
// from one base per block, and the odd stride keeps a wave's reads of
// consecutive blocks free of bank conflicts), workgroup 0 writes x_out and
// y.  The same arithmetic, in the same order, as the standalone norm kernel
// (eight values per thread, the wave partials in order).
constexpr int kLdsBlk = XP_WORDS + 1;
// Split in two so that the norm's inputs are requested before the matvec's
// first weights: loads complete in issue order, so the norm math then runs
// while the weights are still in flight.
//
// QG (quiescence gating) is 0 when the layer is not gated; 1 in the QKV
// kernel of a gated layer: the residual add is left out when the previous
// layer was skipped, the mean square of (stream - its value at the previous
// gated step) decides whether this layer runs (every workgroup computes the
// same value in the same order, so they agree), workgroup 0 publishes the
// decision, and y is written only where the reference writes it (by the
// previous layer's closing add_rmsnorm or by this layer's input norm); 2 in
// the gate/up kernel of a gated layer: workgroup 0 records the layer's input
// stream (x_in) as the next step's x_prev.
template <int C>
struct NormIn {
    float xv[C][8], rv[C][8], pv[C][8], wv[C][8], qv[C][8];
    uint32_t pskip;
};
template <int MODE, int C, int QG = 0>
__device__ __forceinline__ void norm_load(const NormArgs &n, uint32_t dim, NormIn<C> &v) {
    v.pskip = 0;
    if (QG == 1 && n.q.prev_skip) v.pskip = *n.q.prev_skip;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const uint32_t t = threadIdx.x + c * blockDim.x;
        const bool ok = 8 * t < dim;
        ld8(n.x_in, t, ok, v.xv[c]);
        if (MODE != NORM_PLAIN) ld8(n.r, t, ok, v.rv[c]);
        if (MODE == NORM_POST_ADD) ld8(n.pw, t, ok, v.pv[c]);
        ld8(n.w, t, ok, v.wv[c]);
        if (QG == 1) ld8(n.q.x_prev, t, ok, v.qv[c]);
    }
}
// Returns whether the layer runs (always true unless QG == 1).
template <int MODE, int C, int QG = 0>
__device__ __forceinline__ bool norm_to_lds(const NormArgs &n, uint32_t dim, NormIn<C> &v, uint32_t *lp,
                                            float *sh) {
    float ss[C];
    if (QG == 2 && blockIdx.x == 0) {
#pragma unroll
        for (int c = 0; c < C; ++c) {
            const uint32_t t = threadIdx.x + c * blockDim.x;
            if (8 * t < dim) st8(n.q.x_prev, t, v.xv[c]);
        }
    }
    const bool add_on = QG != 1 || v.pskip == 0;   // uniform
    if (MODE != NORM_PLAIN && add_on) {
        if (MODE == NORM_POST_ADD) {
#pragma unroll
            for (int c = 0; c < C; ++c) {
                ss[c] = 0.0f;
#pragma unroll
                for (int i = 0; i < 8; ++i) ss[c] += v.rv[c][i] * v.rv[c][i];
            }
            const float inv = 1.0f / sqrtf(wg_sum_c<C>(ss, sh + 16) / (float)dim + n.eps);
#pragma unroll
            for (int c = 0; c < C; ++c)
#pragma unroll
                for (int i = 0; i < 8; ++i) v.rv[c][i] = (v.rv[c][i] * inv) * v.pv[c][i];
        }
#pragma unroll
        for (int c = 0; c < C; ++c)
#pragma unroll
            for (int i = 0; i < 8; ++i) v.xv[c][i] = (v.xv[c][i] + v.rv[c][i]) * n.scalar;
    }
    bool active = true;
    if (QG == 1) {
        float dd[C];
#pragma unroll
        for (int c = 0; c < C; ++c) {
            dd[c] = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float d = v.xv[c][i] - v.qv[c][i];
                dd[c] += d * d;
            }
        }
        const float ms = wg_sum_c<C>(dd, sh + 32) / (float)dim;
        active = ms >= n.q.thresh || n.q.thresh <= 0.0f;
        if (blockIdx.x == 0 && threadIdx.x == 0) *n.q.skip = active ? 0u : 1u;
    }
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const uint32_t t = threadIdx.x + c * blockDim.x;
        if (blockIdx.x == 0 && 8 * t < dim) st8(n.x_out, t, v.xv[c]);
        ss[c] = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss[c] += v.xv[c][i] * v.xv[c][i];
    }
    const float inv = 1.0f / sqrtf(wg_sum_c<C>(ss, sh) / (float)dim + n.eps);
    const bool write_y = QG != 1 || (add_on && !n.q.first) || active;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const uint32_t t = threadIdx.x + c * blockDim.x;
        const bool ok = 8 * t < dim;
        float yv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) yv[i] = (v.xv[c][i] * inv) * v.wv[c][i];
        if (blockIdx.x == 0 && ok && n.y && write_y) st8(n.y, t, yv);
        emit_planes8s(yv, lp, 1, kLdsBlk, t >> 2, t & 3, ok);
    }
    return active;
}

// This lane's two blocks of planes from the LDS copy norm_to_lds wrote.
__device__ __forceinline__ void lane_planes_lds(const uint32_t *lp, uint32_t b0, uint32_t b1, bool ok0, bool ok1,
                                                uint32_t (&P)[2][XP_WORDS], float (&xs)[2]) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const uint32_t m = opaque_mask(c ? ok1 : ok0);
        const uint32_t *src = lp + (c ? b1 : b0) * kLdsBlk;
#pragma unroll
        for (int i = 0; i < XP_WORDS; ++i) P[c][i] = src[i] & m;
        xs[c] = __builtin_bit_cast(float, src[XP_WORDS] & m);
    }
}

// This lane's two blocks of activation planes from `src` (global or LDS,
// layout of chn_xplanes); blocks without data read block 0 and are zeroed.
__device__ __forceinline__ void lane_planes(const uint32_t *src, uint32_t nb, uint32_t b0, uint32_t b1, bool ok0,
                                            bool ok1, uint32_t (&P)[2][XP_WORDS], float (&xs)[2]) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const bool ok = c ? ok1 : ok0;
        const uint32_t b = c ? b1 : b0;
#pragma unroll
        for (int i = 0; i < XP_WORDS; ++i) P[c][i] = src[(size_t)i * nb + b];
        xs[c] = ((const float *)(src + (size_t)XP_WORDS * nb))[b];
#pragma unroll
        for (int i = 0; i < XP_WORDS; ++i) P[c][i] = ok ? P[c][i] : 0u;
        xs[c] = ok ? xs[c] : 0.0f;
    }
}

// QKV matvec with the step's norm as its prologue (K <= 4096): NW waves per
// workgroup, two rows per wave per group as k_q4rmv<RV_QKV, 2, 1>; the
// wave's first two groups' weights are in flight while the norm runs (the
// launch gives every wave two groups at the model's shapes).
template <int NORM, int NW = 8, int QG = 0>
__global__ __launch_bounds__(64 * NW) void k_q4rmv_qkv_nx(RArgs a, NormArgs n) {
    constexpr int RPW = 2;
    constexpr int NCH = (512 + 64 * NW - 1) / (64 * NW);   // norm chunks of eight values per thread: K <= 4096
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const uint32_t nb = a.nb;
    const bool ok0 = (uint32_t)lane < nb, ok1 = (uint32_t)(64 + lane) < nb;
    const uint32_t b0 = ok0 ? lane : 0u, b1 = ok1 ? 64 + lane : 0u;
    __shared__ uint32_t lp[128 * kLdsBlk];
    __shared__ float sh[48];

    const uint32_t ngroups = (a.M + RPW - 1) / RPW;
    const uint32_t gstride = gridDim.x * NW;
    struct Grp {   // this lane's two blocks of RPW rows
        u32x4r q[RPW][2];
        uint16_t s[RPW][2];
    };
    auto load = [&](Grp &d, uint32_t g) {
#pragma unroll
        for (int s = 0; s < RPW; ++s) {
            uint32_t row = g * RPW + s;
            row = row < a.M ? row : a.M - 1;
            const u32x4r *N;
            const uint16_t *S;
            row_ptrs<RV_QKV>(a, row, 0, N, S);
            d.q[s][0] = __builtin_nontemporal_load(N + b0);
            d.q[s][1] = __builtin_nontemporal_load(N + b1);
            d.s[s][0] = __builtin_nontemporal_load(S + b0);
            d.s[s][1] = __builtin_nontemporal_load(S + b1);
        }
    };
    uint32_t P[2][XP_WORDS];
    float xs[2];
    auto dot_store = [&](const Grp &c, uint32_t g) {
        float part[RPW], tot[RPW];
#pragma unroll
        for (int s = 0; s < RPW; ++s) {
            float r = 0.0f;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int T = block_idot_r(c.q[s][k], P[k]);
                const float sf = (float)__builtin_bit_cast(_Float16, c.s[s][k]);
                r = fmaf((float)T, sf * xs[k], r);
            }
            part[s] = r;
        }
        wave_sums<RPW>(part, tot);
#pragma unroll
        for (int s = 0; s < RPW; ++s) {
            const uint32_t row = g * RPW + s;
            if (lane == 0 && row < a.M) store_r<RV_QKV>(a, row, tot[s]);
        }
    };
    NormIn<NCH> nv;
    norm_load<NORM, NCH, QG>(n, nb * 32, nv);
    // The wave's first two row groups are requested before the norm runs,
    // unconditionally (the row index is clamped; a wave with one group loads
    // its own rows twice, from cache), so no branch makes the norm's waits
    // drain them.
    uint32_t g = blockIdx.x * NW + wave;
    const uint32_t g1 = g + gstride;
    const uint32_t ga = g < ngroups ? g : ngroups - 1;
    Grp A, B;
    load(A, ga);
    load(B, g1 < ngroups ? g1 : ga);
    if (n.rope.tab && blockIdx.x == 0) rope_table(n.rope, threadIdx.x, blockDim.x);
    const bool active = norm_to_lds<NORM, NCH, QG>(n, nb * 32, nv, lp, sh);
    if (QG && !active) return;                // a quiescent layer (the same decision in every workgroup)
    __syncthreads();
    lane_planes_lds(lp, b0, b1, ok0, ok1, P, xs);
    if (g < ngroups) dot_store(A, g);
    if (g1 < ngroups) dot_store(B, g1);

    // shapes with more than two groups per wave: one group in flight
    g = g1 + gstride;
    if (g < ngroups) {
        load(A, g);
        for (; g < ngroups; g += gstride) {
            const Grp c = A;
            if (g + gstride < ngroups) load(A, g + gstride);
            dot_store(c, g);
        }
    }
}

// Gate/up + GELU-tanh that also emits the digit planes of its output (the
// down projection's input), so no separate planes pass runs between the two.
// A workgroup of NW waves owns blocks of 32 consecutive rows; wave w takes
// rows w, w + NW, ... of a block, one gate/up pair at a time with the next
// pair (across blocks too) in flight, each row as k_q4rmv<RV_MLP, 1, 1>
// computes it.  The 32 results meet in LDS; four lanes then quantize the
// block.  Input planes come from a.xp (NORM < 0) or from the step's norm as
// the prologue (NORM = NormMode).  Needs K <= 4096 and M % 32 == 0.
template <int NW, int NORM, int QG = 0>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(4))) void k_q4rmv_mlp_xp(
    RArgs a, uint32_t *__restrict__ xo, NormArgs n) {
    constexpr int RW = 32 / NW;   // rows per wave per block
    if (QG && *n.q.skip) {
        // a quiescent layer: the stream passes unchanged; it is also the
        // layer's input at the next gated step
        if (blockIdx.x == 0)
            for (uint32_t i = threadIdx.x; 8 * i < a.nb * 32; i += blockDim.x) {
                float v[8];
                ld8(n.x_in, i, true, v);
                st8(n.x_out, i, v);
                st8(n.q.x_prev, i, v);
            }
        return;
    }
    const int wave = wave_id(), lane = threadIdx.x & 63;
    const uint32_t nb = a.nb;
    const bool ok0 = (uint32_t)lane < nb, ok1 = (uint32_t)(64 + lane) < nb;
    const uint32_t b0 = ok0 ? lane : 0u, b1 = ok1 ? 64 + lane : 0u;
    __shared__ float sact[32];
    __shared__ uint32_t lp[NORM >= 0 ? 128 * kLdsBlk : 1];
    __shared__ float sh[32];
    const uint32_t nrb = a.M / 32;

    struct RowPair {   // this lane's two blocks of one gate row and one up row
        u32x4r q[2][2];
        uint16_t s[2][2];
    };
    auto load = [&](RowPair &d, uint32_t row) {
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const u32x4r *N = (m ? a.m1.N : a.m0.N) + (size_t)row * nb;
            const uint16_t *S = (m ? a.m1.S : a.m0.S) + (size_t)row * nb;
            d.q[m][0] = __builtin_nontemporal_load(N + b0);
            d.q[m][1] = __builtin_nontemporal_load(N + b1);
            d.s[m][0] = __builtin_nontemporal_load(S + b0);
            d.s[m][1] = __builtin_nontemporal_load(S + b1);
        }
    };
    constexpr int NM = NORM < 0 ? 0 : NORM;
    constexpr int NCH = (NORM < 0) ? 1 : (512 + 64 * NW - 1) / (64 * NW);   // norm chunks: K <= 4096
    NormIn<NCH> nv;
    if (NORM >= 0) norm_load<NM, NCH, QG>(n, nb * 32, nv);
    uint32_t rb = blockIdx.x;
    RowPair nx;
    if (rb < nrb) load(nx, rb * 32 + wave);

    // this lane's two blocks of input planes, in registers
    uint32_t P[2][XP_WORDS];
    float xs[2];
    if (NORM >= 0) {
        norm_to_lds<NM, NCH, QG>(n, nb * 32, nv, lp, sh);
        __syncthreads();
        lane_planes_lds(lp, b0, b1, ok0, ok1, P, xs);
    } else {
        lane_planes(a.xp, nb, b0, b1, ok0, ok1, P, xs);
    }

    for (; rb < nrb; rb += gridDim.x) {
        const uint32_t nxt = rb + gridDim.x;
#pragma unroll 1
        for (int j = 0; j < RW; ++j) {
            const RowPair cur = nx;
            if (j + 1 < RW) load(nx, rb * 32 + wave + NW * (j + 1));
            else if (nxt < nrb) load(nx, nxt * 32 + wave);
            float r[2] = {0.0f, 0.0f};
#pragma unroll
            for (int m = 0; m < 2; ++m)
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    const int T = block_idot_r(cur.q[m][c], P[c]);
                    const float sf = (float)__builtin_bit_cast(_Float16, cur.s[m][c]);
                    r[m] = fmaf((float)T, sf * xs[c], r[m]);
                }
            float t[2];
            wave_sum2(r[0], r[1], t[0], t[1]);
            if (lane == 0) sact[wave + NW * j] = gelu_tanh(t[0]) * t[1];
        }
        __syncthreads();
        // an opaque copy of the thread index: otherwise the plane-store
        // addresses are hoisted out of the block loop and spilled
        uint32_t tx = threadIdx.x;
        __asm__ volatile("" : "+v"(tx));
        if (tx < 32) a.y0[rb * 32 + tx] = sact[tx];
        if (tx < 4) {
            float o[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = sact[8 * tx + i];
            emit_planes8(o, xo, nrb, rb, tx, true);
        }
        __syncthreads();   // sact is rewritten by the next block
    }
}

// Launch shape (from sweeps on MI355X at the 12B decode shapes with weights
// cold in HBM, graph replay): the fewest waves splitting K such that each
// covers <= 128 blocks; one gate/up row pair or two rows per wave.  Without
// a K split, one row group per wave up to 1024 workgroups (at 8192 x 3840 a
// 341-workgroup launch takes 10.5 us against 7.3 us at 1024), two per wave
// for small matrices (o_proj 3840 x 4096: 4.28 us at 240 against 4.41 at
// 480); with a K split, four row groups per workgroup.
template <int MODE, int WPR>
static void launch_rw(const RArgs &a, int rpw, uint32_t grid, hipStream_t s) {
    if (rpw == 1) k_q4rmv<MODE, 1, WPR><<<grid, 256, 0, s>>>(a);
    else k_q4rmv<MODE, 2, WPR><<<grid, 256, 0, s>>>(a);
}

static int launch_q4rmv(chn_ctx *ctx, int mode, RArgs a, const float *x, uint32_t *xp, bool planes_ready) {
    const uint32_t nb = a.nb;
    if (!planes_ready) {
        if (launch_xplanes(ctx->stream, x, xp, nb)) return hip_fail(ctx, hipGetLastError(), "k_xplanes");
    }
    a.xp = xp;
    const int wpr = nb <= 128 ? 1 : (nb <= 256 ? 2 : 4);
    const int rpw = mode == RV_MLP ? 1 : 2;
    const uint32_t G = 4 / wpr;
    const uint32_t ngroups = (a.M + rpw - 1) / rpw;
    const uint32_t need = (ngroups + G - 1) / G;      // workgroups at one row group per wave
    uint32_t grid;
    if (wpr == 1) {
        // one group per wave up to 1024 workgroups; small matrices two per wave
        grid = need <= 512 ? (need + 1) / 2 : (need < 1024 ? need : 1024);
    } else {
        // waves splitting K: four row groups per workgroup (down at 12B:
        // 9.4 us against 9.7 at 2.5 groups), never more than kRedIters
        grid = (need + 3) / 4;
        const uint32_t lo = (need + kRedIters - 1) / kRedIters;
        if (grid < lo) grid = lo;
    }
    if (!grid) grid = 1;
    hipStream_t s = ctx->stream;
    switch (mode) {
    case RV_GEMV:
        wpr == 1 ? launch_rw<RV_GEMV, 1>(a, rpw, grid, s)
                 : (wpr == 2 ? launch_rw<RV_GEMV, 2>(a, rpw, grid, s) : launch_rw<RV_GEMV, 4>(a, rpw, grid, s));
        break;
    case RV_QKV:
        wpr == 1 ? launch_rw<RV_QKV, 1>(a, rpw, grid, s)
                 : (wpr == 2 ? launch_rw<RV_QKV, 2>(a, rpw, grid, s) : launch_rw<RV_QKV, 4>(a, rpw, grid, s));
        break;
    default:
        wpr == 1 ? launch_rw<RV_MLP, 1>(a, rpw, grid, s)
                 : (wpr == 2 ? launch_rw<RV_MLP, 2>(a, rpw, grid, s) : launch_rw<RV_MLP, 4>(a, rpw, grid, s));
        break;
    }
    CHN_LAUNCHED(ctx, "k_q4rmv");
    return CHN_OK;
}

static RMat host_rmat(const void *W, uint32_t rows, uint32_t nb) {
    RMat m;
    m.N = (const u32x4r *)W;
    m.S = (const uint16_t *)((const unsigned char *)W + (size_t)rows * nb * 16);
    return m;
}

int mvr_gemv(chn_ctx *ctx, const void *W, const float *x, float *y, uint32_t M, uint32_t K, uint32_t *xp,
             bool planes_ready, const uint32_t *skip) {
    const uint32_t nb = K / 32;
    RArgs a{host_rmat(W, M, nb), {}, {}, y, nullptr, nullptr, nullptr, M, M, M, nb, skip};
    return launch_q4rmv(ctx, RV_GEMV, a, x, xp, planes_ready);
}
int mvr_qkv(chn_ctx *ctx, const void *Wq, const void *Wk, const void *Wv, const float *x, float *q, float *k,
            float *v, uint32_t q_dim, uint32_t kv_dim, uint32_t K, uint32_t *xp, bool planes_ready) {
    const uint32_t nb = K / 32;
    RArgs a{host_rmat(Wq, q_dim, nb), host_rmat(Wk, kv_dim, nb), host_rmat(Wv, kv_dim, nb), q, k, v, nullptr,
            q_dim + 2 * kv_dim, q_dim, q_dim + kv_dim, nb};
    return launch_q4rmv(ctx, RV_QKV, a, x, xp, planes_ready);
}
int mvr_mlp(chn_ctx *ctx, const void *Wg, const void *Wu, const float *x, float *act, uint32_t M, uint32_t K,
            uint32_t *xp, bool planes_ready) {
    const uint32_t nb = K / 32;
    RArgs a{host_rmat(Wg, M, nb), host_rmat(Wu, M, nb), {}, act, nullptr, nullptr, nullptr, M, M, M, nb};
    return launch_q4rmv(ctx, RV_MLP, a, x, xp, planes_ready);
}

// Gate/up launch shape (sweeps at 15360 x 3840 with weights cold in HBM):
// one 32-row block per workgroup, at most kMlpGrid workgroups (which then
// loop over blocks).  From planes: four waves on eight rows each (the next
// row pair in flight), 14.2 us against 14.6 us for eight waves on four.
constexpr uint32_t kMlpGrid = 2048;

int mvr_mlp_xp(chn_ctx *ctx, const void *Wg, const void *Wu, const uint32_t *xp_in, float *act,
               uint32_t *xp_out, uint32_t M, uint32_t K) {
    const uint32_t nb = K / 32;
    if (nb > 128 || M % 32 != 0) {
        const int rc = mvr_mlp(ctx, Wg, Wu, nullptr, act, M, K, (uint32_t *)xp_in, true);
        if (rc) return rc;
        if (launch_xplanes(ctx->stream, act, xp_out, M / 32)) return hip_fail(ctx, hipGetLastError(), "k_xplanes");
        return CHN_OK;
    }
    const RArgs a{host_rmat(Wg, M, nb), host_rmat(Wu, M, nb), {}, act, nullptr, nullptr, xp_in, M, M, M, nb};
    const uint32_t nrb = M / 32;
    if (!nrb) return CHN_OK;
    k_q4rmv_mlp_xp<4, -1><<<nrb < kMlpGrid ? nrb : kMlpGrid, 256, 0, ctx->stream>>>(a, xp_out, NormArgs{});
    CHN_LAUNCHED(ctx, "k_q4rmv_mlp_xp");
    return CHN_OK;
}

int mvr_mlp_nx(chn_ctx *ctx, const void *Wg, const void *Wu, float *act, uint32_t *xp_out, uint32_t M, uint32_t K,
               const NormArgs &n, int mode) {
    const uint32_t nb = K / 32;
    if (nb > 128 || M % 32 != 0 || nb == 0) return set_err(ctx, CHN_E_UNSUPPORTED, "fused norm gate/up: K=%u M=%u", K, M);
    const RArgs a{host_rmat(Wg, M, nb), host_rmat(Wu, M, nb), {}, act, nullptr, nullptr, nullptr, M, M, M, nb};
    const uint32_t nrb = M / 32;
    if (!nrb) return CHN_OK;
    // eight-wave workgroups here: the norm prologue, recomputed by every
    // workgroup, takes twice as long on four waves (16.3 us against 15.4 us
    // for the whole kernel)
    const uint32_t grid = nrb < kMlpGrid ? nrb : kMlpGrid;
    hipStream_t s = ctx->stream;
    if (n.q.skip) {
        if (mode == NORM_PLAIN) k_q4rmv_mlp_xp<8, NORM_PLAIN, 2><<<grid, 512, 0, s>>>(a, xp_out, n);
        else if (mode == NORM_ADD) k_q4rmv_mlp_xp<8, NORM_ADD, 2><<<grid, 512, 0, s>>>(a, xp_out, n);
        else k_q4rmv_mlp_xp<8, NORM_POST_ADD, 2><<<grid, 512, 0, s>>>(a, xp_out, n);
    } else if (mode == NORM_PLAIN) k_q4rmv_mlp_xp<8, NORM_PLAIN><<<grid, 512, 0, s>>>(a, xp_out, n);
    else if (mode == NORM_ADD) k_q4rmv_mlp_xp<8, NORM_ADD><<<grid, 512, 0, s>>>(a, xp_out, n);
    else k_q4rmv_mlp_xp<8, NORM_POST_ADD><<<grid, 512, 0, s>>>(a, xp_out, n);
    CHN_LAUNCHED(ctx, "k_q4rmv_mlp_xp");
    return CHN_OK;
}

int mvr_qkv_nx(chn_ctx *ctx, const void *Wq, const void *Wk, const void *Wv, float *q, float *k, float *v,
               uint32_t q_dim, uint32_t kv_dim, uint32_t K, const NormArgs &n, int mode) {
    const uint32_t nb = K / 32;
    if (nb > 128 || nb == 0) return set_err(ctx, CHN_E_UNSUPPORTED, "fused norm QKV: K=%u", K);
    const uint32_t M = q_dim + 2 * kv_dim;
    const RArgs a{host_rmat(Wq, q_dim, nb), host_rmat(Wk, kv_dim, nb), host_rmat(Wv, kv_dim, nb), q, k, v, nullptr,
                  M, q_dim, q_dim + kv_dim, nb};
    // eight-wave workgroups, two row groups per wave, at most one workgroup
    // per CU: every workgroup recomputes the norm, so fewer, longer-lived
    // workgroups win (8192 x 3840: 8.1 us against 8.7 us for 256 sixteen-wave
    // and 8.8 us for 512 eight-wave workgroups at one group per wave)
    const uint32_t need = ((M + 1) / 2 + 7) / 8;      // workgroups at one group per wave
    uint32_t grid = (need + 1) / 2;
    grid = grid < 1 ? 1 : (grid > 256 ? 256 : grid);
    hipStream_t s = ctx->stream;
    if (n.q.skip) {
        if (mode == NORM_PLAIN) k_q4rmv_qkv_nx<NORM_PLAIN, 8, 1><<<grid, 512, 0, s>>>(a, n);
        else if (mode == NORM_ADD) k_q4rmv_qkv_nx<NORM_ADD, 8, 1><<<grid, 512, 0, s>>>(a, n);
        else k_q4rmv_qkv_nx<NORM_POST_ADD, 8, 1><<<grid, 512, 0, s>>>(a, n);
    } else if (mode == NORM_PLAIN) k_q4rmv_qkv_nx<NORM_PLAIN, 8><<<grid, 512, 0, s>>>(a, n);
    else if (mode == NORM_ADD) k_q4rmv_qkv_nx<NORM_ADD, 8><<<grid, 512, 0, s>>>(a, n);
    else k_q4rmv_qkv_nx<NORM_POST_ADD, 8><<<grid, 512, 0, s>>>(a, n);
    CHN_LAUNCHED(ctx, "k_q4rmv_qkv_nx");
    return CHN_OK;
}

static int check_r(chn_ctx *ctx, const float *x, uint32_t K) {
    CHN_REQUIRE(ctx, K > 0 && K % 32 == 0 && K <= 16384, "K=%u must be a positive multiple of 32, <= 16384", K);
    CHN_REQUIRE(ctx, x && aligned(x, 16), "x must be non-NULL and 16-byte aligned");
    return CHN_OK;
}

}  // namespace chn

using namespace chn;

extern "C" int chn_q4_repack(chn_ctx *ctx, const uint32_t *W, uint32_t rows, uint32_t K, void *dst) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, W && dst, "NULL argument");
    CHN_REQUIRE(ctx, K % 32 == 0, "K=%u must be a multiple of 32", K);
    CHN_REQUIRE(ctx, aligned(dst, 16), "dst must be 16-byte aligned");
    if (launch_q4_repack(ctx->stream, W, rows, K, dst)) return hip_fail(ctx, hipGetLastError(), "k_repack_q4");
    return CHN_OK;
}

extern "C" int chn_gemv_q4r(chn_ctx *ctx, const void *W, const float *x, float *y, uint32_t M, uint32_t K) {
    if (!ctx) return CHN_E_INVALID;
    int rc = check_r(ctx, x, K);
    if (rc) return rc;
    CHN_REQUIRE(ctx, W && y && aligned(W, 16), "W/y must be non-NULL, W 16-byte aligned");
    if (!M) return CHN_OK;
    rc = ensure_workspace(ctx, xplanes_bytes(K / 32));
    if (rc) return rc;
    return mvr_gemv(ctx, W, x, y, M, K, (uint32_t *)ctx->ws, false);
}

extern "C" int chn_fused_qkv_q4r(chn_ctx *ctx, const void *Wq, const void *Wk, const void *Wv, const float *x,
                                 float *q, float *k, float *v, uint32_t q_dim, uint32_t kv_dim, uint32_t K) {
    if (!ctx) return CHN_E_INVALID;
    int rc = check_r(ctx, x, K);
    if (rc) return rc;
    CHN_REQUIRE(ctx, Wq && Wk && Wv && q && k && v, "NULL argument");
    CHN_REQUIRE(ctx, aligned(Wq, 16) && aligned(Wk, 16) && aligned(Wv, 16), "weights must be 16-byte aligned");
    if (!(q_dim + 2 * kv_dim)) return CHN_OK;
    rc = ensure_workspace(ctx, xplanes_bytes(K / 32));
    if (rc) return rc;
    return mvr_qkv(ctx, Wq, Wk, Wv, x, q, k, v, q_dim, kv_dim, K, (uint32_t *)ctx->ws, false);
}

extern "C" int chn_fused_mlp_q4r(chn_ctx *ctx, const void *Wg, const void *Wu, const float *x, float *act,
                                 uint32_t M, uint32_t K) {
    if (!ctx) return CHN_E_INVALID;
    int rc = check_r(ctx, x, K);
    if (rc) return rc;
    CHN_REQUIRE(ctx, Wg && Wu && act && aligned(Wg, 16) && aligned(Wu, 16), "NULL or misaligned argument");
    if (!M) return CHN_OK;
    rc = ensure_workspace(ctx, xplanes_bytes(K / 32));
    if (rc) return rc;
    return mvr_mlp(ctx, Wg, Wu, x, act, M, K, (uint32_t *)ctx->ws, false);
}

extern "C" int chn_xplanes(chn_ctx *ctx, const float *x, uint32_t K, uint32_t *planes) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, x && planes, "NULL argument");
    CHN_REQUIRE(ctx, K % 32 == 0, "K=%u must be a multiple of 32", K);
    CHN_REQUIRE(ctx, aligned(x, 16) && aligned(planes, 4), "x must be 16-byte and planes 4-byte aligned");
    if (!K) return CHN_OK;
    if (launch_xplanes(ctx->stream, x, planes, K / 32)) return hip_fail(ctx, hipGetLastError(), "k_xplanes");
    return CHN_OK;
}

static int check_xp(chn_ctx *ctx, const uint32_t *planes, uint32_t K) {
    CHN_REQUIRE(ctx, K > 0 && K % 32 == 0 && K <= 16384, "K=%u must be a positive multiple of 32, <= 16384", K);
    CHN_REQUIRE(ctx, planes && aligned(planes, 4), "planes must be non-NULL and 4-byte aligned");
    return CHN_OK;
}

extern "C" int chn_gemv_q4r_xp(chn_ctx *ctx, const void *W, const uint32_t *planes, float *y, uint32_t M,
                               uint32_t K) {
    if (!ctx) return CHN_E_INVALID;
    int rc = check_xp(ctx, planes, K);
    if (rc) return rc;
    CHN_REQUIRE(ctx, W && y && aligned(W, 16), "W/y must be non-NULL, W 16-byte aligned");
    if (!M) return CHN_OK;
    return mvr_gemv(ctx, W, nullptr, y, M, K, (uint32_t *)planes, true);
}

extern "C" int chn_fused_mlp_q4r_xp(chn_ctx *ctx, const void *Wg, const void *Wu, const uint32_t *planes,
                                    float *act, uint32_t *act_planes, uint32_t M, uint32_t K) {
    if (!ctx) return CHN_E_INVALID;
    int rc = check_xp(ctx, planes, K);
    if (rc) return rc;
    CHN_REQUIRE(ctx, Wg && Wu && act && aligned(Wg, 16) && aligned(Wu, 16), "NULL or misaligned argument");
    CHN_REQUIRE(ctx, !act_planes || (M % 32 == 0 && aligned(act_planes, 4)),
                "act_planes needs M %% 32 == 0 (M=%u) and 4-byte alignment", M);
    CHN_REQUIRE(ctx, !act_planes || act_planes != planes, "act_planes must not alias planes");
    if (!M) return CHN_OK;
    if (act_planes) return mvr_mlp_xp(ctx, Wg, Wu, planes, act, act_planes, M, K);
    return mvr_mlp(ctx, Wg, Wu, nullptr, act, M, K, (uint32_t *)planes, true);
}

// The decode step's pre-FFN block as the model launches it: the
// post-attention norm of r (post_w != NULL), the residual add, the pre-FFN
// norm, gate/up + GELU-tanh * up and the digit planes of act, one launch.
extern "C" int chn_ffn_gate_up_q4r(chn_ctx *ctx, const void *Wg, const void *Wu, const float *x_in, const float *r,
                                   const float *post_w, const float *pre_w, float *x_out, float *normed_out,
                                   float *act, uint32_t *act_planes, uint32_t M, uint32_t K, float eps) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, Wg && Wu && x_in && r && pre_w && x_out && act && act_planes, "NULL argument");
    CHN_REQUIRE(ctx, K > 0 && K % 32 == 0 && K <= 4096, "K=%u must be a positive multiple of 32, <= 4096", K);
    CHN_REQUIRE(ctx, M > 0 && M % 32 == 0, "M=%u must be a positive multiple of 32", M);
    CHN_REQUIRE(ctx, aligned(Wg, 16) && aligned(Wu, 16), "weights must be 16-byte aligned");
    CHN_REQUIRE(ctx, aligned(x_in, 16) && aligned(r, 16) && aligned(pre_w, 16) && aligned(x_out, 16) &&
                         (!post_w || aligned(post_w, 16)) && (!normed_out || aligned(normed_out, 16)),
                "vectors must be 16-byte aligned");
    CHN_REQUIRE(ctx, aligned(act_planes, 4), "act_planes must be 4-byte aligned");
    CHN_REQUIRE(ctx, x_out != x_in, "x_out must not alias x_in (other workgroups still read x_in)");
    const NormArgs n{x_in, r, post_w, pre_w, x_out, normed_out, eps, 1.0f, RopeTab{nullptr, nullptr, {0.0f, 0.0f}, {0u, 0u}}};
    return mvr_mlp_nx(ctx, Wg, Wu, act, act_planes, M, K, n, post_w ? NORM_POST_ADD : NORM_ADD);
}
