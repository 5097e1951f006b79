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

#include <type_traits>
#include <utility>

namespace chn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));

constexpr int GT = 128;          // tokens per workgroup tile
constexpr int GN = 128;          // features per workgroup tile

// Activations to bf16 (RNE); also zeroes z[0, nz) (the output of a split-K
// contraction, whose two halves add into it).
__global__ __launch_bounds__(256) void k_to_bf16(const float *__restrict__ x, __bf16 *__restrict__ y, size_t n,
                                                 float *__restrict__ z, size_t nz) {
    const size_t stride = (size_t)gridDim.x * blockDim.x * 4;
    for (size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4; i < n; i += stride) {
        if (i + 4 <= n) {
            const float4 v = *(const float4 *)(x + i);
            bf16x2 a = {(__bf16)v.x, (__bf16)v.y}, b = {(__bf16)v.z, (__bf16)v.w};
            *(bf16x2 *)(y + i) = a;
            *(bf16x2 *)(y + i + 2) = b;
        } else {
            for (size_t j = i; j < n; ++j) y[j] = (__bf16)x[j];
        }
    }
    for (size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 4; i < nz; i += stride) {
        if (i + 4 <= nz) *(float4 *)(z + i) = float4{0.f, 0.f, 0.f, 0.f};
        else
            for (size_t j = i; j < nz; ++j) z[j] = 0.f;
    }
}

constexpr int kGemmKB = 2;      // Q4 blocks per K step of the register-staged GEMM

struct GemmArgs {
    const __bf16 *X;       // [n_tok][K] bf16
    const uint32_t *W0, *W1; // Q4 [M][K/32][5], or Q4R (W1: up matrix for the fused MLP)
    float *Y;              // [n_tok][M]
    uint32_t n_tok, M, K;
    // Up to two more single-matrix segments sharing X (one launch for q, k
    // and v): segment g multiplies Wg[g] into Yg[g] ([n_tok][Mg[g]]).
    const uint32_t *Wg[2] = {nullptr, nullptr};
    float *Yg[2] = {nullptr, nullptr};
    uint32_t Mg[2] = {0, 0};
    // Register-staged kernel only: Yb != NULL writes the result as bf16 to
    // Yb ([n_tok][M]) instead of Y (the next contraction's input).
    __bf16 *Yb = nullptr;
    // Split K: with ypart, split p stores its partial sums to Y + p * ypart
    // ([n_tok][M] each, plain stores; the consumer adds them); without it
    // (the pipelined kernel's two halves) both add into Y, which starts at
    // zero.
    size_t ypart = 0;
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

// One nibble word (8 weights) to 8 bf16, given s and -8 s.  The empty asm
// hides the known-zero bits (so byte extraction lowers to
// v_cvt_f32_ubyte{0..3}) but lets unused results be removed.
__device__ __forceinline__ uint32_t opaque_nv(uint32_t v) {
    __asm__("" : "+v"(v));
    return v;
}
__device__ __forceinline__ u32x4v dequant_word_bf16(const uint32_t q, const float s, const float ms) {
    const uint32_t lo = opaque_nv(q & 0x0F0F0F0Fu);
    const uint32_t hi = opaque_nv((q >> 4) & 0x0F0F0F0Fu);
    u32x4v o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        bf16x2 p = {(__bf16)fmaf((float)((lo >> (8 * j)) & 0xffu), s, ms),
                    (__bf16)fmaf((float)((hi >> (8 * j)) & 0xffu), s, ms)};
        o[j] = __builtin_bit_cast(uint32_t, p);
    }
    return o;
}

// REP: weights in the repacked layout (16-byte nibble words, each nibble
// XOR 8, then f16 scales), un-XORed here so the dequantization is shared.
// KB Q4 blocks (32 K each) per step: the workgroup's chain of dependent
// load -> compute steps is K / (32 KB) long, and each step's loads return
// from L2 / HBM in about a microsecond, far longer than its MFMAs take.
template <int NMAT, bool REP, int KB>
__global__ __launch_bounds__(256, 2) void k_q4gemm(GemmArgs a) {
    constexpr int GK = 32 * KB;                  // K per step
    constexpr int LROW = GK * 2 + 16;            // LDS row stride in bytes (padded)
    constexpr int XC = GT * GK / 8 / 256;        // 16-byte X chunks per thread per step
    constexpr int WB = GN * KB / 256;            // weight blocks per thread per step (consecutive)
    __shared__ __attribute__((aligned(16))) unsigned char lx[GT * LROW];
    __shared__ __attribute__((aligned(16))) unsigned char lw[NMAT][GN * LROW];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wr = wave >> 1, wc = wave & 1;           // wave's 64x64 sub-tile
    const uint32_t n0 = blockIdx.x * GN, t0 = blockIdx.y * GT;
    const uint32_t nb = a.K / 32;
    const uint32_t steps = (a.K + GK - 1) / GK;

    // global -> register staging for one K step
    u32x4v xr[XC];                 // XC x 16 B of X per thread
    uint32_t ww0[NMAT][WB];
    u32x4v wq[NMAT][WB];
    const int w_row = tid / (KB / WB), w_blk = (tid % (KB / WB)) * WB;   // first weight block of this thread

    auto gload = [&](uint32_t ks) {
#pragma unroll
        for (int i = 0; i < XC; ++i) {
            const int c = tid + 256 * i;               // chunks of 16 B
            const int row = c / (GK / 8), col = c % (GK / 8);
            const uint32_t t = t0 + row;
            const uint32_t k = ks * GK + col * 8;
            xr[i] = (t < a.n_tok && k < a.K) ? *(const u32x4v *)(a.X + (size_t)t * a.K + k) : u32x4v{0, 0, 0, 0};
        }
        const uint32_t n = n0 + w_row;
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            const uint32_t *W = m == 0 ? a.W0 : a.W1;
#pragma unroll
            for (int j = 0; j < WB; ++j) {
                const uint32_t b = ks * KB + w_blk + j;
                if (n < a.M && b < nb) {
                    if (REP) {
                        const size_t i = (size_t)n * nb + b;
                        const u32x4g qv = ((const u32x4g *)W)[i];
                        wq[m][j] = u32x4v{qv[0] ^ 0x88888888u, qv[1] ^ 0x88888888u, qv[2] ^ 0x88888888u,
                                          qv[3] ^ 0x88888888u};
                        ww0[m][j] = ((const uint16_t *)((const unsigned char *)W + (size_t)a.M * nb * 16))[i];
                    } else {
                        const uint32_t *p = W + ((size_t)n * nb + b) * 5;
                        ww0[m][j] = p[0];
                        wq[m][j] = *(const u32x4_a4 *)(p + 1);
                    }
                } else {
                    ww0[m][j] = 0;
                    wq[m][j] = u32x4v{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
                }
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
        for (int i = 0; i < XC; ++i) {
            const int c = tid + 256 * i;
            *(u32x4v *)(lx + (c / (GK / 8)) * LROW + (c % (GK / 8)) * 16) = xr[i];
        }
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int j = 0; j < WB; ++j) {
                u32x4v d[4];
                dequant_block_bf16(ww0[m][j], wq[m][j], d);
                unsigned char *dst = lw[m] + w_row * LROW + (w_blk + j) * 64;
#pragma unroll
                for (int w = 0; w < 4; ++w) *(u32x4v *)(dst + 16 * w) = d[w];
            }
        __syncthreads();
        if (ks + 1 < steps) gload(ks + 1);

#pragma unroll
        for (int kk = 0; kk < KB; ++kk) {
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
                    if (a.Yb) a.Yb[(size_t)t * a.M + n] = (__bf16)v;
                    else a.Y[(size_t)t * a.M + n] = v;
                }
            }
        }
}

// f(std::integral_constant<int, i>) for i = 0 .. N-1 (compile-time indices,
// e.g. for the immediate offsets of asm LDS reads).
template <typename F, int... I>
__host__ __device__ __forceinline__ void static_for_(F &&f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__host__ __device__ __forceinline__ void static_for(F &&f) {
    static_for_(f, std::make_integer_sequence<int, N>{});
}

// ---------------------------------------------------------------------------
// The fused gate/up (two matrices, GELU-tanh * up epilogue) on 256-token x
// 128-feature tiles: eight waves (two per SIMD, one workgroup per CU), wave
// (wr, wc) a 64-token x 64-feature block of both matrices.  Every operand
// travels by DMA (global_load_lds) straight into LDS, so no register holds
// a load in flight and the waits are explicit vmcnt immediates:
//   X(j)      256 rows x 128 B of bf16 (16-byte chunks XOR-swizzled by
//             row), two slots: one step ahead (X is read from L2);
//   Wraw(j)   the raw Q4 bytes of both matrices (nibble words, scales),
//             two slots: fetched two steps before their tile is
//             multiplied (dequantized one step before).
// Each step the 512 threads dequantize the next step's Wraw (one 32-block
// each) into the other of two bf16 weight tiles while the current one is
// multiplied, so a step has one barrier; all LDS reads of the loop are asm
// and pinned after the waits.  K % 64 == 0.
// At 512 x 3840 -> 2 x 15360: 137.8 us against 162-164 us for the
// register-staged k_q4gemm<2> (128-token tiles, operands one step ahead),
// which still serves K % 64 != 0, and 159.6 us for this kernel with one
// tile, dequantized between two barriers per step.
template <bool REP>
struct Gemm2dCfg {
    static constexpr int BT = 256, GK = 64, SX = 2, SW = 2;
    static constexpr int LROW = GK * 2 + 16;               // weight tile row stride (padded)
    static constexpr int XSLOT = BT * GK * 2;              // 32 KB of X per step
    static constexpr int QSLOT = 2 * 128 * 2 * 16;         // nibble words per step, [m][blk][row]
    static constexpr int SWORDS = REP ? 2 * 128 : 2 * 128 * 2;   // scale words, REP [m][row] else [m][blk][row]
    static constexpr int SSLOT = SWORDS * 4;
    static constexpr int OFF_Q = SX * XSLOT, OFF_S = OFF_Q + SW * QSLOT, OFF_W = OFF_S + SW * SSLOT;
    static constexpr int WTILE = 2 * GN * LROW;             // bf16 tiles of both matrices
    static constexpr int LDS = OFF_W + 2 * WTILE;
    static constexpr int NS = SWORDS / 64;                 // scale instructions per step
};

template <bool REP>
__global__ __launch_bounds__(512) void k_q4gemm2d(GemmArgs a) {
    using C = Gemm2dCfg<REP>;
    constexpr int NMAT = 2;
    __shared__ __attribute__((aligned(16))) unsigned char sm[C::LDS];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave >> 1, wc = wave & 1;
    const uint32_t n0 = blockIdx.x * GN, t0 = blockIdx.y * C::BT;
    const uint32_t K = a.K, nb = K / 32, steps = K / C::GK;
    const uint32_t smb = lds_addr(sm);

    // ---- every DMA is issued by waves 4-7 (the second wave of each SIMD),
    // while waves 0-3 dequantize: X as 32 one-KB instructions per step, eight
    // per issuing wave; the raw weights as eight one-KB nibble instructions
    // (two per issuing wave) and NS scale instructions.  (Issuing them from
    // all eight waves stalled every wave on the CU's address rate right after
    // the barrier: 134-135 against 136-139 µs.)
    // (a dependent constant inside a DMA builtin's arguments makes the host
    // pass drop the kernel's launch stub: local copies)
    constexpr uint32_t GK = C::GK;
    const __bf16 *Xb = a.X;
    const int dw = (wave - 4) & 3;                             // issuing wave 0..3 (waves 4-7)
    uint32_t xe[8];                                            // element offsets (n_tok * K < 2^32)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int q = (i * 4 + dw) * 64 + lane;                // chunk position in the slot
        const int r = q >> 3, c = (q & 7) ^ ((r ^ (r >> 3)) & 7);
        xe[i] = (t0 + r < a.n_tok ? t0 + r : a.n_tok - 1) * K + c * 8;
    }
    auto issue_x = [&](uint32_t j) {                           // X(j) -> slot j % SX (j clamped)
        if (wave < 4) return;                                  // wave-uniform
        const uint32_t jj = j < steps ? j : steps - 1;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            __builtin_amdgcn_global_load_lds(Xb + (xe[i] + jj * GK),
                                             (lds_t *)(sm + (j % C::SX) * C::XSLOT + (i * 4 + dw) * 1024), 16, 0,
                                             0);
    };
    const unsigned char *wq_g[2], *ws_g[2];
    const uint32_t wq_step = REP ? 32 : 40, ws_step = REP ? 4 : 40;
    constexpr int NSW = (C::NS + 3) / 4;                       // scale instructions per issuing wave
    static_assert(NSW <= 2, "two scale instructions per issuing wave at most");
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int ch = (2 * dw + k) * 64 + lane;               // nibble chunk [m][blk][row]
        const int m = ch >> 8, blk = (ch >> 7) & 1, row = ch & 127;
        const uint32_t n = n0 + row < a.M ? n0 + row : a.M - 1;
        const unsigned char *W = (const unsigned char *)(m == 0 ? a.W0 : a.W1);
        wq_g[k] = REP ? W + ((size_t)n * nb + blk) * 16 : W + ((size_t)n * nb + blk) * 20 + 4;
    }
#pragma unroll
    for (int k = 0; k < NSW; ++k) {
        const int si = dw * NSW + k;                           // scale instruction
        const int sq = (si < C::NS ? si : 0) * 64 + lane;      // REP [m][row], else [m][blk][row]
        const int sm_ = REP ? sq >> 7 : sq >> 8, sblk = REP ? 0 : (sq >> 7) & 1, srow = sq & 127;
        const uint32_t ns = n0 + srow < a.M ? n0 + srow : a.M - 1;
        const unsigned char *Ws = (const unsigned char *)(sm_ == 0 ? a.W0 : a.W1);
        ws_g[k] = REP ? Ws + (size_t)a.M * nb * 16 + (size_t)ns * nb * 2 : Ws + ((size_t)ns * nb + sblk) * 20;
    }
    auto issue_w = [&](uint32_t j) {                           // Wraw(j) -> slot j % SW (j clamped)
        if (wave < 4) return;
        const uint32_t jj = j < steps ? j : steps - 1;
#pragma unroll
        for (int k = 0; k < 2; ++k)
            __builtin_amdgcn_global_load_lds(wq_g[k] + (size_t)jj * wq_step,
                                             (lds_t *)(sm + C::OFF_Q + (j % C::SW) * C::QSLOT + (2 * dw + k) * 1024),
                                             16, 0, 0);
#pragma unroll
        for (int k = 0; k < NSW; ++k)
            if (dw * NSW + k < C::NS)
                __builtin_amdgcn_global_load_lds(ws_g[k] + (size_t)jj * ws_step,
                                                 (lds_t *)(sm + C::OFF_S + (j % C::SW) * C::SSLOT + (dw * NSW + k) * 256),
                                                 4, 0, 0);
    };

    // ---- dequantization by waves 0-3, the first wave of each SIMD: thread
    // tid takes nibble chunks tid (gate) and tid + 256 (up), each a block of
    // one row ([m][blk][row]).  Those waves issue first and otherwise idle at
    // the next barrier while the SIMD's second wave finishes its MFMAs
    // (135.8 against 139.4 µs with every wave dequantizing one chunk).
    const int d_blk = (tid >> 7) & 1, d_row = tid & 127;       // the same for tid and tid + 256
    const uint32_t dq_q = smb + C::OFF_Q + tid * 16;
    const uint32_t dq_s = smb + C::OFF_S + (REP ? d_row : tid) * 4;
    const uint32_t dq_w = C::OFF_W + d_row * C::LROW + d_blk * 64;
    auto dequant = [&](auto slot_) {                           // Wraw slot SL -> bf16 tile SL
        constexpr int SL = decltype(slot_)::value;
        if (wave >= 4) return;                                 // wave-uniform
        u32x4v q0 = lds_read<u32x4v, SL * C::QSLOT>(dq_q);
        u32x4v q1 = lds_read<u32x4v, SL * C::QSLOT + 256 * 16>(dq_q);
        uint32_t s0 = lds_read<uint32_t, SL * C::SSLOT>(dq_s);
        uint32_t s1 = lds_read<uint32_t, SL * C::SSLOT + (REP ? 128 : 256) * 4>(dq_s);
        lds_wait();
        lds_pin(q0);
        lds_pin(q1);
        lds_pin(s0);
        lds_pin(s1);
        const float sc0 = f16_lo_to_f32(REP ? s0 >> (16 * d_blk) : s0), ms0 = -8.0f * sc0;
        const float sc1 = f16_lo_to_f32(REP ? s1 >> (16 * d_blk) : s1), ms1 = -8.0f * sc1;
        unsigned char *dst = sm + dq_w + SL * C::WTILE;
#pragma unroll
        for (int w = 0; w < 4; ++w)
            *(u32x4v *)(dst + 16 * w) = dequant_word_bf16(REP ? q0[w] ^ 0x88888888u : q0[w], sc0, ms0);
#pragma unroll
        for (int w = 0; w < 4; ++w)
            *(u32x4v *)(dst + GN * C::LROW + 16 * w) = dequant_word_bf16(REP ? q1[w] ^ 0x88888888u : q1[w], sc1, ms1);
    };

    // ---- fragment addresses: A (row r, chunk (4 kk + lane / 16) ^ sw(r)), B
    uint32_t xa[2][4];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const int r = wr * 64 + mt * 16 + (lane & 15);
            const int c = (4 * kk + (lane >> 4)) ^ ((r ^ (r >> 3)) & 7);
            xa[kk][mt] = smb + r * 128 + c * 16;
        }
    const uint32_t wa = smb + C::OFF_W + (wc * 64 + (lane & 15)) * C::LROW + (lane >> 4) * 16;

    f32x4 acc[NMAT][4][4];
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[m][i][j] = f32x4{0, 0, 0, 0};

    // Wraw(0) is dequantized into tile 0 first; then each step j waits for
    // X(j) and Wraw(j+1) (issued together at step j-1), passes one barrier,
    // issues X(j+1) and Wraw(j+2), dequantizes Wraw(j+1) into tile (j+1) % 2
    // and multiplies tile j % 2 with X slot j % 2: the dequantization of
    // the next step overlaps the other waves' MFMAs, with no second barrier.
    issue_w(0);
    wait_vm_lgkm0<0>();
    bare_barrier();                                            // every wave's share of Wraw(0)
    dequant(std::integral_constant<int, 0>{});
    issue_x(0);
    __asm__ volatile("" ::: "memory");
    issue_w(1);
    __asm__ volatile("" ::: "memory");

    auto step = [&](uint32_t j, auto xs_) {
        constexpr int XS = decltype(xs_)::value;               // == j % 2: X slot and tile of step j
        wait_vm_lgkm0<0>();                                    // X(j), Wraw(j+1); this wave's tile writes
        bare_barrier();                                        // ... every wave's; step j-1's reads done
        issue_x(j + 1);                                        // into the X slot step j-1 read
        __asm__ volatile("" ::: "memory");
        issue_w(j + 2);                                        // into the Wraw slot step j-1 dequantized
        __asm__ volatile("" ::: "memory");
        dequant(std::integral_constant<int, 1 - XS>{});        // Wraw(j+1) -> tile (j+1) % 2
        static_for<2>([&](auto kk_) {
            constexpr int KK = decltype(kk_)::value;
            bf16x8 af[4], bfm[NMAT][4];
            static_for<4>([&](auto mt_) {
                constexpr int MT = decltype(mt_)::value;
                af[MT] = lds_read<bf16x8, XS * C::XSLOT>(xa[KK][MT]);
            });
            static_for<NMAT * 4>([&](auto i_) {
                constexpr int I = decltype(i_)::value, M = I / 4, NT = I % 4;
                bfm[M][NT] = lds_read<bf16x8, XS * C::WTILE + M * GN * C::LROW + NT * 16 * C::LROW + KK * 64>(wa);
            });
            lds_wait();
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) lds_pin(af[mt]);
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) lds_pin(bfm[m][nt]);
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                    for (int nt = 0; nt < 4; ++nt)
                        acc[m][mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt], bfm[m][nt], acc[m][mt][nt],
                                                                                  0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);                 // one K half's fragments live at a time
        });
    };
    uint32_t j = 0;
    for (; j + 1 < steps; j += 2) {
        step(j, std::integral_constant<int, 0>{});
        step(j + 1, std::integral_constant<int, 1>{});
    }
    if (j < steps) step(j, std::integral_constant<int, 0>{});
    wait_vm_lgkm0<0>();                                        // no DMA may land after the workgroup ends

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
                    const float v = gelu_tanh(acc[0][mt][nt][i]) * acc[1][mt][nt][i];
                    if (a.Yb) a.Yb[(size_t)t * a.M + n] = (__bf16)v;
                    else a.Y[(size_t)t * a.M + n] = v;
                }
            }
        }
}

// ---------------------------------------------------------------------------
// Single-matrix contraction on 256-token x 128-feature tiles: the fused
// gate/up's pipeline with one matrix, eight waves (wr, wc) of 64 tokens x 64
// features, every operand by DMA (waves 4-7 issue, waves 0-3 dequantize),
// one barrier per K step of 64, each weight dequantized once per 256
// tokens.  K is split ksplit ways (work items), split ks storing its sums to
// Y + ks * ypart with plain stores; the consumer adds them.
template <bool REP>
struct Gemm2sCfg {
    static constexpr int BT = 256, GK = 64, SX = 2, SW = 2;
    static constexpr int LROW = GK * 2 + 16;
    static constexpr int XSLOT = BT * GK * 2;              // 32 KB of X per step
    static constexpr int QSLOT = GN * 2 * 16;              // nibble words per step, [blk][row]
    static constexpr int SWORDS = REP ? GN : 2 * GN;       // REP [row] (both blocks' f16 scales), else [blk][row]
    static constexpr int SSLOT = SWORDS * 4;
    static constexpr int OFF_Q = SX * XSLOT, OFF_S = OFF_Q + SW * QSLOT, OFF_W = OFF_S + SW * SSLOT;
    static constexpr int WTILE = GN * LROW;
    static constexpr int LDS = OFF_W + 2 * WTILE;
    static constexpr int NS = SWORDS / 64;                 // scale instructions per step
};

template <bool REP>
__global__ __launch_bounds__(512) void k_q4gemm2s(GemmArgs a, uint32_t n_ft, uint32_t n_tt, uint32_t ksplit) {
    using C = Gemm2sCfg<REP>;
    __shared__ __attribute__((aligned(16))) unsigned char sm[C::LDS];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = wave >> 1, wc = wave & 1;
    // work items (split, feature tile, token tile), token tile fastest; the
    // items are dealt to the XCDs in contiguous runs (workgroup i runs on
    // XCD i % 8), so the token tiles of a feature block share one L2
    const uint32_t nwork = n_ft * n_tt * ksplit, per = (nwork + 7) / 8;
    const uint32_t work = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (work >= nwork) return;                             // uniform, before any barrier
    const uint32_t tt = work % n_tt, ft = (work / n_tt) % n_ft, ks = work / (n_tt * n_ft);
    const uint32_t n0 = ft * GN, t0 = tt * C::BT;
    const uint32_t K = a.K, nb = K / 32, kper = K / ksplit, steps = kper / C::GK, kb0 = ks * kper / 32;
    const uint32_t smb = lds_addr(sm);

    constexpr uint32_t GK = C::GK;
    const __bf16 *Xb = a.X + ks * kper;
    const int dw = (wave - 4) & 3;                             // issuing wave 0..3 (waves 4-7)
    uint32_t xe[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int q = (i * 4 + dw) * 64 + lane;
        const int r = q >> 3, c = (q & 7) ^ ((r ^ (r >> 3)) & 7);
        xe[i] = (t0 + r < a.n_tok ? t0 + r : a.n_tok - 1) * K + c * 8;
    }
    auto issue_x = [&](uint32_t j) {
        if (wave < 4) return;
        const uint32_t jj = j < steps ? j : steps - 1;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            __builtin_amdgcn_global_load_lds(Xb + (xe[i] + jj * GK),
                                             (lds_t *)(sm + (j % C::SX) * C::XSLOT + (i * 4 + dw) * 1024), 16, 0,
                                             0);
    };
    const unsigned char *W = (const unsigned char *)a.W0;
    const unsigned char *wq_g, *ws_g;
    const uint32_t wq_step = REP ? 32 : 40, ws_step = REP ? 4 : 40;
    {
        const int ch = dw * 64 + lane;                         // nibble chunk [blk][row]
        const int blk = ch >> 7, row = ch & 127;
        const uint32_t n = n0 + row < a.M ? n0 + row : a.M - 1;
        wq_g = REP ? W + ((size_t)n * nb + kb0 + blk) * 16 : W + ((size_t)n * nb + kb0 + blk) * 20 + 4;
        const int sq = (dw < C::NS ? dw : 0) * 64 + lane;      // REP [row], else [blk][row]
        const int sblk = REP ? 0 : sq >> 7, srow = sq & 127;
        const uint32_t ns = n0 + srow < a.M ? n0 + srow : a.M - 1;
        ws_g = REP ? W + (size_t)a.M * nb * 16 + ((size_t)ns * nb + kb0) * 2 : W + ((size_t)ns * nb + kb0 + sblk) * 20;
    }
    auto issue_w = [&](uint32_t j) {
        if (wave < 4) return;
        const uint32_t jj = j < steps ? j : steps - 1;
        __builtin_amdgcn_global_load_lds(wq_g + (size_t)jj * wq_step,
                                         (lds_t *)(sm + C::OFF_Q + (j % C::SW) * C::QSLOT + dw * 1024), 16, 0, 0);
        if (dw < C::NS)
            __builtin_amdgcn_global_load_lds(ws_g + (size_t)jj * ws_step,
                                             (lds_t *)(sm + C::OFF_S + (j % C::SW) * C::SSLOT + dw * 256), 4, 0, 0);
    };

    const int d_blk = (tid >> 7) & 1, d_row = tid & 127;
    const uint32_t dq_q = smb + C::OFF_Q + (tid & 255) * 16;
    const uint32_t dq_s = smb + C::OFF_S + (REP ? d_row : (tid & 255)) * 4;
    const uint32_t dq_w = C::OFF_W + d_row * C::LROW + d_blk * 64;
    auto dequant = [&](auto slot_) {
        constexpr int SL = decltype(slot_)::value;
        if (wave >= 4) return;
        u32x4v q0 = lds_read<u32x4v, SL * C::QSLOT>(dq_q);
        uint32_t s0 = lds_read<uint32_t, SL * C::SSLOT>(dq_s);
        lds_wait();
        lds_pin(q0);
        lds_pin(s0);
        const float sc0 = f16_lo_to_f32(REP ? s0 >> (16 * d_blk) : s0), ms0 = -8.0f * sc0;
        unsigned char *dst = sm + dq_w + SL * C::WTILE;
#pragma unroll
        for (int w = 0; w < 4; ++w)
            *(u32x4v *)(dst + 16 * w) = dequant_word_bf16(REP ? q0[w] ^ 0x88888888u : q0[w], sc0, ms0);
    };

    uint32_t xa[2][4];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
            const int r = wr * 64 + mt * 16 + (lane & 15);
            const int c = (4 * kk + (lane >> 4)) ^ ((r ^ (r >> 3)) & 7);
            xa[kk][mt] = smb + r * 128 + c * 16;
        }
    const uint32_t wa = smb + C::OFF_W + (wc * 64 + (lane & 15)) * C::LROW + (lane >> 4) * 16;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0, 0, 0, 0};

    issue_w(0);
    wait_vm_lgkm0<0>();
    bare_barrier();
    dequant(std::integral_constant<int, 0>{});
    issue_x(0);
    __asm__ volatile("" ::: "memory");
    issue_w(1);
    __asm__ volatile("" ::: "memory");

    auto step = [&](uint32_t j, auto xs_) {
        constexpr int XS = decltype(xs_)::value;
        wait_vm_lgkm0<0>();
        bare_barrier();
        issue_x(j + 1);
        __asm__ volatile("" ::: "memory");
        issue_w(j + 2);
        __asm__ volatile("" ::: "memory");
        dequant(std::integral_constant<int, 1 - XS>{});
        static_for<2>([&](auto kk_) {
            constexpr int KK = decltype(kk_)::value;
            bf16x8 af[4], bfm[4];
            static_for<4>([&](auto mt_) {
                constexpr int MT = decltype(mt_)::value;
                af[MT] = lds_read<bf16x8, XS * C::XSLOT>(xa[KK][MT]);
            });
            static_for<4>([&](auto nt_) {
                constexpr int NT = decltype(nt_)::value;
                bfm[NT] = lds_read<bf16x8, XS * C::WTILE + NT * 16 * C::LROW + KK * 64>(wa);
            });
            lds_wait();
#pragma unroll
            for (int mt = 0; mt < 4; ++mt) lds_pin(af[mt]);
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) lds_pin(bfm[nt]);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int nt = 0; nt < 4; ++nt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mt], bfm[nt], acc[mt][nt], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        });
    };
    uint32_t j = 0;
    for (; j + 1 < steps; j += 2) {
        step(j, std::integral_constant<int, 0>{});
        step(j + 1, std::integral_constant<int, 1>{});
    }
    if (j < steps) step(j, std::integral_constant<int, 0>{});
    wait_vm_lgkm0<0>();

    float *Yp = a.Y + ks * a.ypart;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
            const uint32_t n = n0 + wc * 64 + nt * 16 + (lane & 15);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t t = t0 + wr * 64 + mt * 16 + (lane >> 4) * 4 + i;
                if (t < a.n_tok && n < a.M) Yp[(size_t)t * a.M + n] = acc[mt][nt][i];
            }
        }
}

// ---------------------------------------------------------------------------
// Pipelined contraction for K % 64 == 0 (every prefill shape of the model).
//
// A workgroup owns 128 tokens x BN features (per matrix) and walks K in steps
// of 64.  Step j's operands travel as one DMA group straight from global
// memory into LDS (global_load_lds_dwordx{4,1}: no registers, no ds_write):
//   X(j)      128 rows x 128 B of bf16, 16-byte chunk c of row r stored at
//             position c ^ sw(r), sw(r) = (r ^ r >> 3) & 7, so the 16 rows a
//             fragment read touches fall in distinct banks;
//   Wraw(j+1) the raw Q4 bytes of the next step: nibble words ([blk][row])
//             and scales.
// S groups are in flight in a ring; the wait for group j is an explicit
// vmcnt that leaves the younger groups outstanding, and the workgroup
// barrier carries no memory fence (a fenced barrier waits for every
// outstanding load).  While step j's MFMAs run, the waves dequantize
// Wraw(j+1) once into a double-buffered bf16 tile, so each weight is
// dequantized once per 128 tokens.
// The eight waves form two groups of four: group g multiplies K half g of
// every step (32 of the 64), each wave a 32-token x BN-feature block with
// v_mfma_f32_16x16x32_bf16, and the two groups' partial sums meet once, in
// LDS, at the end.  Two waves per SIMD let one wave's waits and dequant
// arithmetic overlap the other's MFMAs when the grid has one workgroup per
// CU.
// Tiles are dealt to the 8 XCDs in contiguous runs (workgroup i runs on XCD
// i % 8), with the 128-token tiles of one feature block adjacent, so a
// weight block's bytes are reused from one L2.
template <int NMAT, int BN, bool REP, int S>
struct PipeCfg {
    static constexpr int BT = 128, GK = 64, NTHR = 512;
    static constexpr int R = NMAT * BN;                    // weight rows per step (64 or 128)
    static constexpr int NW = R / 64;
    static constexpr int XSLOT = BT * GK * 2;              // 16 KB of X per step
    static constexpr int QSLOT = R * 2 * 16;               // nibble words per step, [m][blk][row]
    static constexpr int SWORDS = REP ? R : R * 2;         // scale words per step
    static constexpr int SSLOT = SWORDS * 4;
    static constexpr int WROW = GK * 2 + 16;               // padded bf16 weight row
    static constexpr int WBUF = R * WROW;
    static constexpr int OFF_Q = S * XSLOT, OFF_S = OFF_Q + S * QSLOT, OFF_W = OFF_S + S * SSLOT;
    static constexpr int OFF_D = OFF_W + 2 * WBUF;          // 256 B written by waves without a weight load
    static constexpr int LDS_MAIN = OFF_D + 256;
    static constexpr int LDS_RED = BT * R * 4;             // group-1 partial sums at the end
    static constexpr int LDS = LDS_MAIN > LDS_RED ? LDS_MAIN : LDS_RED;
    // Every DMA instruction runs with all 64 lanes, and every wave issues
    // PER = 3 per group, so one vmcnt fits all waves: 2 KB of X each, then
    // waves 0 .. NQ-1 1 KB of nibble words, waves NQ .. NQ+NS-1 256 B of
    // scales, and the rest 256 B into a dummy area.
    static constexpr int NQ = QSLOT / 1024, NS = SWORDS / 64, PER = 3;
    static_assert(NW == 1 || NW == 2, "64 or 128 weight rows per step");
    static_assert(NQ + NS <= 8, "one weight DMA instruction per wave");
};


template <int NMAT, int BN, bool REP, int S>
__global__ __launch_bounds__(512) void k_q4gemm_p(GemmArgs a, uint32_t n_ct, uint32_t n_tt, uint32_t ksplit) {
    using C = PipeCfg<NMAT, BN, REP, S>;
    constexpr int NTW = BN / 32;                           // 16-feature tiles per wave and matrix
    __shared__ __attribute__((aligned(16))) unsigned char sm[C::LDS];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // group grp multiplies K half grp of each step; within it, 2 x 2 waves of
    // 64 tokens (wr) x BN/2 features per matrix (wc)
    const int grp = wave >> 2, wr = (wave >> 1) & 1, wc = wave & 1;
    const uint32_t ntile = n_ct * n_tt, nwork = ntile * ksplit, per = (nwork + 7) / 8;
    const uint32_t work = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
    if (work >= nwork) return;
    const uint32_t ks = work / ntile, tile = work % ntile;
    // column tile -> segment (workgroup-uniform)
    uint32_t ct = tile / n_tt;
    const uint32_t *W0 = a.W0;
    float *Yp = a.Y;
    uint32_t Mloc = a.M;
    {
        const uint32_t c0 = (a.M + BN - 1) / BN, c1 = (a.Mg[0] + BN - 1) / BN;
        if (ct >= c0) {
            ct -= c0;
            const int g = ct >= c1 ? 1 : 0;
            if (g) ct -= c1;
            W0 = a.Wg[g];
            Yp = a.Yg[g];
            Mloc = a.Mg[g];
        }
    }
    const uint32_t n0 = ct * BN, t0 = (tile % n_tt) * C::BT;
    const uint32_t K = a.K, nb = K / 32, steps_all = K / 64;
    // K split between two workgroups: steps [0, h) and [h, steps_all)
    const uint32_t h = steps_all / 2, s_begin = ks ? h : 0;
    const uint32_t steps = ksplit == 1 ? steps_all : (ks ? steps_all - h : h);
    const uint32_t smb = lds_addr(sm);

    // ---- per-lane DMA sources (rows clamped in bounds; their results are not stored)
    const __bf16 *xg[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int q = (i * 8 + wave) * 64 + lane;          // chunk position in the X slot
        const int r = q >> 3, c = (q & 7) ^ ((r ^ (r >> 3)) & 7);
        const uint32_t t = min(t0 + r, a.n_tok - 1);
        xg[i] = a.X + (size_t)t * K + c * 8 + s_begin * 64;
    }
    // weight DMA of this wave: nibble instruction `wave` (role 0), scale
    // instruction `wave - NQ` (role 1) or the dummy load (role 2)
    const int role = wave < C::NQ ? 0 : (wave < C::NQ + C::NS ? 1 : 2);
    const unsigned char *wg;
    uint32_t w_lds, w_slot, w_step;
    {
        const int qi = role == 0 ? wave : 0, si = role == 1 ? wave - C::NQ : 0;
        const int q = qi * 64 + lane;                      // nibble chunk, [m][blk][row]
        const int qm = q / (BN * 2), qblk = (q % (BN * 2)) / BN, qrow = q % BN;
        const int sq = si * 64 + lane;                     // scale word, REP [m][row], else [m][blk][row]
        const int sm_ = REP ? sq / BN : sq / (BN * 2), sblk = REP ? 0 : (sq % (BN * 2)) / BN, srow = sq % BN;
        const int m = role == 0 ? qm : sm_, row = role == 0 ? qrow : srow;
        const uint32_t n = min(n0 + row, Mloc - 1);
        const unsigned char *W = (const unsigned char *)(m == 0 ? W0 : a.W1);
        if (role == 0) {
            wg = REP ? W + ((size_t)n * nb + qblk) * 16 : W + ((size_t)n * nb + qblk) * 20 + 4;
            w_lds = C::OFF_Q + qi * 1024;
            w_slot = C::QSLOT;
            w_step = REP ? 32 : 40;
        } else if (role == 1) {
            wg = REP ? W + (size_t)Mloc * nb * 16 + (size_t)n * nb * 2 : W + ((size_t)n * nb + sblk) * 20;
            w_lds = C::OFF_S + si * 256;
            w_slot = C::SSLOT;
            w_step = REP ? 4 : 40;
        } else {                                           // first 128 B of X (K >= 64)
            wg = (const unsigned char *)a.X + (lane * 4) % 128;
            w_lds = C::OFF_D;
            w_slot = 0;
            w_step = 0;
        }
        wg += (size_t)s_begin * w_step;
    }

    // Group j: X(j) -> X slot j % S and Wraw(j + 1) -> weight slot (j+1) % S.
    // Groups past the last step reload the last step's bytes (clamped) into
    // slots nobody reads again, so every wave issues the same count.
    auto issue_w = [&](uint32_t j) {
        const uint32_t jj = min(j, steps - 1);
        lds_t *dst = (lds_t *)(sm + w_lds + (j % S) * w_slot);
        if (role == 0) __builtin_amdgcn_global_load_lds(wg + (size_t)jj * w_step, dst, 16, 0, 0);
        else __builtin_amdgcn_global_load_lds(wg + (size_t)jj * w_step, dst, 4, 0, 0);
    };
    auto issue_group = [&](uint32_t j) {
        const uint32_t jj = min(j, steps - 1);
        const int xs = j % S;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            __builtin_amdgcn_global_load_lds(xg[i] + (size_t)jj * 64,
                                             (lds_t *)(sm + xs * C::XSLOT + (i * 8 + wave) * 1024), 16, 0, 0);
        issue_w(j + 1);
    };

    // ---- dequantization: thread -> weight row (consecutive lanes, distinct
    // banks) and NW consecutive nibble words of one block
    const int drow = tid % C::R, du = tid / C::R;
    const int dblk = C::NW == 1 ? du >> 2 : du >> 1;
    const int dword0 = C::NW == 1 ? du & 3 : (du & 1) * 2;
    const int dm = drow / BN, drw = drow % BN;
    const uint32_t dq_q = smb + C::OFF_Q + (((dm * 2 + dblk) * BN + drw) * 16 + dword0 * 4);
    const uint32_t dq_s = smb + C::OFF_S + (REP ? drow : (dm * 2 + dblk) * BN + drw) * 4;
    const uint32_t dq_w = C::OFF_W + drow * C::WROW + dblk * 64 + dword0 * 16;
    using RawW = typename std::conditional<C::NW == 1, uint32_t, u32x2v>::type;
    struct Raw {
        RawW w;
        uint32_t sw;
    };
    auto dq_load = [&](uint32_t j) {
        const uint32_t slot = j % S;
        Raw r;
        r.w = lds_read<RawW>(dq_q + slot * C::QSLOT);
        r.sw = lds_read<uint32_t>(dq_s + slot * C::SSLOT);
        return r;
    };
    auto dq_word = [&](const Raw &r, int w, float sc, float ms) {
        uint32_t q;
        if constexpr (C::NW == 1) q = r.w;
        else q = r.w[w];
        return dequant_word_bf16(REP ? q ^ 0x88888888u : q, sc, ms);
    };
    auto dq_scale = [&](const Raw &r, float &sc, float &ms) {
        sc = f16_lo_to_f32(REP ? r.sw >> (16 * dblk) : r.sw);
        ms = -8.0f * sc;
    };
    auto dq_store = [&](uint32_t j, u32x4v d0, u32x4v d1) {
        unsigned char *dst = sm + dq_w + (j & 1) * C::WBUF;
        *(u32x4v *)dst = d0;
        if (C::NW == 2) *(u32x4v *)(dst + 16) = d1;
    };
    auto dq_all = [&](uint32_t j, const Raw &r) {
        float sc, ms;
        dq_scale(r, sc, ms);
        dq_store(j, dq_word(r, 0, sc, ms), C::NW == 2 ? dq_word(r, 1, sc, ms) : u32x4v{0, 0, 0, 0});
    };

    // ---- fragments: this wave's 32 tokens and the BN features of its K half
    struct Frag {
        bf16x8 a[4], b[NMAT][NTW];
    };
    uint32_t xa[4], wa;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
        const int r = wr * 64 + mt * 16 + (lane & 15);
        const int c = (grp * 4 + (lane >> 4)) ^ ((r ^ (r >> 3)) & 7);
        xa[mt] = smb + r * 128 + c * 16;
    }
    wa = smb + C::OFF_W + (wc * (BN / 2) + (lane & 15)) * C::WROW + (grp * 32 + (lane >> 4) * 8) * 2;
    auto frag_load = [&](uint32_t j, Frag &f) {            // X slot j % S, bf16 tile j & 1
        const uint32_t xo = (j % S) * C::XSLOT, wo = (j & 1) * C::WBUF;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) f.a[mt] = lds_read<bf16x8>(xa[mt] + xo);
#pragma unroll
        for (int m = 0; m < NMAT; ++m) {
            const uint32_t wam = wa + wo + m * BN * C::WROW;
            f.b[m][0] = lds_read<bf16x8, 0 * 16 * C::WROW>(wam);
            f.b[m][1] = lds_read<bf16x8, 1 * 16 * C::WROW>(wam);
            if constexpr (NTW == 4) {
                f.b[m][2 % NTW] = lds_read<bf16x8, 2 * 16 * C::WROW>(wam);
                f.b[m][3 % NTW] = lds_read<bf16x8, 3 * 16 * C::WROW>(wam);
            }
        }
    };
    auto frag_pin = [&](Frag &f) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) lds_pin(f.a[mt]);
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt) lds_pin(f.b[m][nt]);
    };

    f32x4 acc[NMAT][4][NTW];
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < NTW; ++j) acc[m][i][j] = f32x4{0, 0, 0, 0};

    // ---- prologue: Wraw(0) and groups 0 .. S-2 in flight, Wraw(0) and
    // Wraw(1) dequantized, then group S-1 (its Wraw(S) reuses Wraw(0)'s slot).
    // The waits count DMA instructions in issue order, so the compiler may
    // not reorder these issues.
    issue_w(0);
#pragma unroll
    for (int g = 0; g < S - 1; ++g) {
        __asm__ volatile("" ::: "memory");
        issue_group(g);
    }
    __asm__ volatile("" ::: "memory");
    wait_vm_lgkm0<(S - 2) * C::PER>();                    // Wraw(0) and group 0 landed
    bare_barrier();                                        // ... for every wave's DMA
    {
        Raw r0 = dq_load(0), r1 = dq_load(1);
        lds_wait();
        lds_pin(r0.w);
        lds_pin(r0.sw);
        lds_pin(r1.w);
        lds_pin(r1.sw);
        dq_all(0, r0);
        dq_all(1, r1);
    }
    wait_vm_lgkm0<(S - 2) * C::PER>();
    bare_barrier();                                        // tiles 0, 1 written; Wraw(0)'s slot free
    issue_group(S - 1);
    __asm__ volatile("" ::: "memory");
    Frag fa, fb;
    frag_load(0, fa);
    lds_wait();
    frag_pin(fa);

    // ---- step s: multiply fragments `cur` (step s) while the fragments of
    // step s+1 load into `nxt` and Wraw(s+2) is dequantized into tile s & 1.
    // The LDS reads are spread between the MFMAs (a read after every second
    // MFMA) so that LDS traffic and matrix work overlap instead of running as
    // two bursts after each barrier.
    constexpr int NMF = NMAT * 4 * NTW;                    // MFMAs per step
    constexpr int NFR = 4 + NMAT * NTW;                    // fragment reads per step
    static_assert(NMF >= NFR, "at least one MFMA per fragment read");
    auto mfma = [&](int i, Frag &cur) {
        const int m = i / (4 * NTW), mt = (i / NTW) % 4, nt = i % NTW;
        acc[m][mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur.a[mt], cur.b[m][nt], acc[m][mt][nt], 0, 0, 0);
    };
    auto frag_read = [&](int i, uint32_t j, Frag &f) {     // read i of frag_load(j)
        const uint32_t xo = (j % S) * C::XSLOT, wo = (j & 1) * C::WBUF;
        if (i < 4) {
            f.a[i] = lds_read<bf16x8>(xa[i] + xo);
        } else {
            const int m = (i - 4) / NTW, nt = (i - 4) % NTW;
            f.b[m][nt] = lds_read<bf16x8>(wa + wo + m * BN * C::WROW + nt * 16 * C::WROW);
        }
    };
    auto step = [&](uint32_t s, Frag &cur, Frag &nxt) {
        wait_vm_lgkm0<(S - 2) * C::PER>();                // group s+1 landed
        bare_barrier();                                    // ... for every wave; tile s & 1 and X slot s % S free
        Raw raw = dq_load(s + 2);                          // first: LDS returns in issue order
        issue_group(s + S);
        // read r goes after MFMA (r * NMF) / NFR
#pragma unroll
        for (int i = 0; i < NMF; ++i) {
            mfma(i, cur);
#pragma unroll
            for (int r = 0; r < NFR; ++r)
                if ((r * NMF) / NFR == i) {
                    frag_read(r, s + 1, nxt);
                    if (r == NFR / 2) {
                        lds_wait_n<NFR / 2 + 1>();         // raw landed (the newest reads may fly)
                        lds_pin(raw.w);
                        lds_pin(raw.sw);
                    }
                }
            __builtin_amdgcn_sched_barrier(0);
        }
        dq_all(s + 2, raw);
        lds_wait();                                        // step s+1's fragments and the tile writes
        frag_pin(nxt);
    };
    uint32_t s = 0;
    for (; s + 1 < steps; s += 2) {
        step(s, fa, fb);
        step(s + 1, fb, fa);
    }
    if (s < steps) step(s, fa, fb);

    // ---- the K halves meet: group 1 parks its sums in LDS, group 0 adds and stores
    wait_vm_lgkm0<0>();
    bare_barrier();
    float *red = (float *)sm;                              // [wave & 3][m][mt][nt][64 lanes][4]
    const int rw = wave & 3;
    if (grp == 1) {
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int nt = 0; nt < NTW; ++nt)
                    *(f32x4 *)(red + ((((rw * NMAT + m) * 4 + mt) * NTW + nt) * 64 + lane) * 4) = acc[m][mt][nt];
    }
    __syncthreads();
    if (grp == 1) return;
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int nt = 0; nt < NTW; ++nt)
                acc[m][mt][nt] += *(const f32x4 *)(red + ((((rw * NMAT + m) * 4 + mt) * NTW + nt) * 64 + lane) * 4);

    // epilogue: lane holds tokens (lane>>4)*4 + i of each 16-row tile, feature
    // lane & 15.  Split K: the halves go to Y and Y + ypart, or add into Y,
    // which starts at zero (two addends from zero give the same sum in
    // either order, and the same as their sum formed by the consumer).
    float *Yo = Yp + (a.ypart ? ks * a.ypart : 0);
    const bool plain = ksplit == 1 || a.ypart;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < NTW; ++nt) {
            const uint32_t n = n0 + wc * (BN / 2) + nt * 16 + (lane & 15);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t t = t0 + wr * 64 + mt * 16 + (lane >> 4) * 4 + i;
                if (t < a.n_tok && n < Mloc) {
                    float v = acc[0][mt][nt][i];
                    if (NMAT == 2) v = gelu_tanh(v) * acc[NMAT - 1][mt][nt][i];
                    float *y = Yo + (size_t)t * Mloc + n;
                    if (plain) *y = v;
                    else unsafeAtomicAdd(y, v);
                }
            }
        }
}

// ksplit 2 (two workgroups per tile, each half of K) needs Y zeroed first,
// K >= 128, and NMAT == 1 (the fused epilogue is not additive).
template <int NMAT, int BN, bool REP, int S>
static void launch_gemm_p(hipStream_t st, const GemmArgs &a, uint32_t ksplit = 1) {
    const uint32_t n_ct = (a.M + BN - 1) / BN + (a.Mg[0] + BN - 1) / BN + (a.Mg[1] + BN - 1) / BN;
    const uint32_t n_tt = (a.n_tok + 127) / 128;
    const uint32_t per = (n_ct * n_tt * ksplit + 7) / 8;
    k_q4gemm_p<NMAT, BN, REP, S><<<8 * per, 512, 0, st>>>(a, n_ct, n_tt, ksplit);
}

static void launch_to_bf16(hipStream_t st, const float *X, __bf16 *xb, size_t n, float *z, size_t nz) {
    const size_t m = n > nz ? n : nz;
    unsigned g = (unsigned)((m / 4 + 255) / 256);
    if (g > 8192) g = 8192;
    if (g == 0) g = 1;
    k_to_bf16<<<g, 256, 0, st>>>(X, xb, n, z, nz);
}

// Launch shapes for one pipelined single-matrix contraction (K % 64 == 0),
// from sweeps at 512 tokens:
//  * 128 x 128 tiles when they alone give at least one workgroup per CU
//    (half the LDS fragment reads per MFMA of 128 x 64 tiles; 15360 x 3840:
//    97 us against 135 us, q/k/v 8192 x 3840: 54 against 69 us; 128 such
//    workgroups lose to 256 of 128 x 64);
//  * for long K 128 x 128 tiles with K split in two, whose larger per-step
//    work pays for itself over the longer loop: K >= 8192 when the halves
//    add into Y by atomics, K >= 4096 when they are stored to two buffers
//    (the atomic epilogue of two halves costs about as much as the plain
//    stores of four; at 512 tokens, 12B o_proj 4096 -> 3840 in 128 x 128
//    halves saves ~4 us a layer against 128 x 64 tiles over all of K);
//  * else 128-token x 64-feature tiles when they give at least ~200
//    workgroups, otherwise the same tiles with K split in two.
enum class PipeShape { BN64, BN64_K2, BN128, BN128_K2 };
static PipeShape pipe_shape(uint32_t n_tok, uint32_t M, uint32_t K, bool halves = false) {
    const uint32_t tt = (n_tok + 127) / 128;
    if (((M + 127) / 128) * tt >= 256) return PipeShape::BN128;
    if (K >= (halves ? 4096u : 8192u) && 2 * ((M + 127) / 128) * tt >= 192) return PipeShape::BN128_K2;
    if (((M + 63) / 64) * tt >= 192 || K < 128) return PipeShape::BN64;
    return PipeShape::BN64_K2;
}

template <bool REP>
static void launch_pipe(hipStream_t st, const GemmArgs &a, PipeShape ps) {
    if (ps == PipeShape::BN64) launch_gemm_p<1, 64, REP, 4>(st, a, 1);
    else if (ps == PipeShape::BN64_K2) launch_gemm_p<1, 64, REP, 4>(st, a, 2);
    else if (ps == PipeShape::BN128) launch_gemm_p<1, 128, REP, 4>(st, a, 1);
    else launch_gemm_p<1, 128, REP, 4>(st, a, 2);
}

// Four-way split of a long K on 256-token x 128-feature tiles (the
// single-matrix 256-token kernel) where its work items fill the CUs once and
// the caller takes four partial outputs: at 512 tokens the 12B down
// projection 15360 -> 3840, 81 against 89 us for 128 x 128 halves; the
// consumer's two extra partial reads cost ~3 us, so shorter K stays on the
// pipelined kernel (o_proj 4096 -> 3840: 29 against 31 us).
static bool split4_fits(uint32_t n_tok, uint32_t M, uint32_t K) {
    const uint32_t items = ((M + GN - 1) / GN) * ((n_tok + 255) / 256) * 4;
    return K >= 8192 && K % 256 == 0 && n_tok > 256 && items >= 192 && items <= 256;
}

int launch_q4gemm(chn_ctx *ctx, int nmat, const float *X, const uint32_t *W0, const uint32_t *W1, float *Y,
                  uint32_t n_tok, uint32_t M, uint32_t K, __bf16 *xb, bool repacked, __bf16 *Yb, PartialOut *po) {
    const size_t n = X ? (size_t)n_tok * K : 0;
    GemmArgs a{xb, W0, W1, Y, n_tok, M, K};
    if (po) po->parts = 1;
    if (nmat == 1 && K % 64 == 0 && po && po->max_parts >= 4 && split4_fits(n_tok, M, K)) {
        if (Yb) return set_err(ctx, CHN_E_UNSUPPORTED, "bf16 output needs the two-matrix contraction");
        if (n) {
            launch_to_bf16(ctx->stream, X, xb, n, nullptr, 0);
            CHN_LAUNCHED(ctx, "k_to_bf16");
        }
        a.ypart = po->stride;
        po->parts = 4;
        const uint32_t n_ft = (M + GN - 1) / GN, n_tt = (n_tok + 255) / 256, per = (n_ft * n_tt * 4 + 7) / 8;
        if (repacked) k_q4gemm2s<true><<<8 * per, 512, 0, ctx->stream>>>(a, n_ft, n_tt, 4);
        else k_q4gemm2s<false><<<8 * per, 512, 0, ctx->stream>>>(a, n_ft, n_tt, 4);
        CHN_LAUNCHED(ctx, "k_q4gemm2s");
        return CHN_OK;
    }
    if (nmat == 1 && K % 64 == 0) {
        if (Yb) return set_err(ctx, CHN_E_UNSUPPORTED, "bf16 output needs the two-matrix contraction");
        const bool halves_ok = po && po->max_parts >= 2;
        const PipeShape ps = pipe_shape(n_tok, M, K, halves_ok);
        const bool split = ps == PipeShape::BN64_K2 || ps == PipeShape::BN128_K2;
        if (split && halves_ok) {
            a.ypart = po->stride;
            po->parts = 2;
        }
        const bool zero = split && !a.ypart;
        if (n || zero) {
            launch_to_bf16(ctx->stream, X, xb, n, zero ? Y : nullptr, zero ? (size_t)n_tok * M : 0);
            CHN_LAUNCHED(ctx, "k_to_bf16");
        }
        if (repacked) launch_pipe<true>(ctx->stream, a, ps);
        else launch_pipe<false>(ctx->stream, a, ps);
        CHN_LAUNCHED(ctx, "k_q4gemm_p");
        return CHN_OK;
    }
    if (n) {
        launch_to_bf16(ctx->stream, X, xb, n, nullptr, 0);
        CHN_LAUNCHED(ctx, "k_to_bf16");
    }
    a.Yb = Yb;
    if (nmat == 2 && K % 64 == 0) {
        const dim3 g2((M + GN - 1) / GN, (n_tok + 255) / 256);
        if (repacked) k_q4gemm2d<true><<<g2, 512, 0, ctx->stream>>>(a);
        else k_q4gemm2d<false><<<g2, 512, 0, ctx->stream>>>(a);
        CHN_LAUNCHED(ctx, "k_q4gemm2d");
        return CHN_OK;
    }
    dim3 grid((M + GN - 1) / GN, (n_tok + GT - 1) / GT);
    if (repacked) {
        if (nmat == 1) k_q4gemm<1, true, kGemmKB><<<grid, 256, 0, ctx->stream>>>(a);
        else k_q4gemm<2, true, kGemmKB><<<grid, 256, 0, ctx->stream>>>(a);
    } else {
        if (nmat == 1) k_q4gemm<1, false, kGemmKB><<<grid, 256, 0, ctx->stream>>>(a);
        else k_q4gemm<2, false, kGemmKB><<<grid, 256, 0, ctx->stream>>>(a);
    }
    CHN_LAUNCHED(ctx, "k_q4gemm");
    return CHN_OK;
}

// q, k and v of one layer in one launch: three repacked matrices over the
// same activations (one bf16 conversion, none when X is NULL and xb already
// holds them).
int launch_q4gemm_qkv(chn_ctx *ctx, const float *X, const uint32_t *Wq, const uint32_t *Wk, const uint32_t *Wv,
                      float *Yq, float *Yk, float *Yv, uint32_t n_tok, uint32_t Mq, uint32_t Mkv, uint32_t K,
                      __bf16 *xb) {
    if (K % 64 != 0) {
        int rc = launch_q4gemm(ctx, 1, X, Wq, nullptr, Yq, n_tok, Mq, K, xb, true);
        if (!rc) rc = launch_q4gemm(ctx, 1, nullptr, Wk, nullptr, Yk, n_tok, Mkv, K, xb, true);
        if (!rc) rc = launch_q4gemm(ctx, 1, nullptr, Wv, nullptr, Yv, n_tok, Mkv, K, xb, true);
        return rc;
    }
    if (X) {
        launch_to_bf16(ctx->stream, X, xb, (size_t)n_tok * K, nullptr, 0);
        CHN_LAUNCHED(ctx, "k_to_bf16");
    }
    GemmArgs a{xb, Wq, nullptr, Yq, n_tok, Mq, K};
    a.Wg[0] = Wk;
    a.Yg[0] = Yk;
    a.Mg[0] = Mkv;
    a.Wg[1] = Wv;
    a.Yg[1] = Yv;
    a.Mg[1] = Mkv;
    // 128 x 128 tiles once they give a workgroup per CU, as pipe_shape
    const uint32_t ct128 = (Mq + 127) / 128 + 2 * ((Mkv + 127) / 128), tt = (n_tok + 127) / 128;
    if (ct128 * tt >= 256) launch_gemm_p<1, 128, true, 4>(ctx->stream, a, 1);
    else launch_gemm_p<1, 64, true, 4>(ctx->stream, a, 1);
    CHN_LAUNCHED(ctx, "k_q4gemm_p");
    return CHN_OK;
}

static int gemm_common(chn_ctx *ctx, int nmat, const uint32_t *W0, const uint32_t *W1, const float *X, float *Y,
                       uint32_t n_tok, uint32_t M, uint32_t K, bool repacked = false, __bf16 *Yb = nullptr) {
    CHN_REQUIRE(ctx, W0 && X && (Y || Yb) && (nmat == 1 || W1), "NULL argument");
    CHN_REQUIRE(ctx, K > 0 && K % 32 == 0, "K=%u must be a positive multiple of 32", K);
    CHN_REQUIRE(ctx, K % 8 == 0 && aligned(X, 16), "X must be 16-byte aligned");
    CHN_REQUIRE(ctx, aligned(W0, repacked ? 16 : 4) && (!W1 || aligned(W1, repacked ? 16 : 4)),
                "weights must be %d-byte aligned", repacked ? 16 : 4);
    if (!n_tok || !M) return CHN_OK;
    int rc = ensure_workspace(ctx, (size_t)n_tok * K * 2);
    if (rc) return rc;
    return launch_q4gemm(ctx, nmat, X, W0, W1, Y, n_tok, M, K, (__bf16 *)ctx->ws, repacked, Yb);
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

// The model's prefill contractions over repacked (Q4R) weights, as
// chn_prefill launches them.
extern "C" int chn_batch_gemm_q4r(chn_ctx *ctx, const void *W, const float *X, float *Y, uint32_t n_tok, uint32_t M,
                                  uint32_t K) {
    if (!ctx) return CHN_E_INVALID;
    return gemm_common(ctx, 1, (const uint32_t *)W, nullptr, X, Y, n_tok, M, K, true);
}

extern "C" int chn_batch_fused_mlp_q4r(chn_ctx *ctx, const void *Wg, const void *Wu, const float *X, float *Y,
                                       uint16_t *Y_bf16, uint32_t n_tok, uint32_t M, uint32_t K) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, (Y == nullptr) != (Y_bf16 == nullptr), "exactly one of Y and Y_bf16 must be given");
    return gemm_common(ctx, 2, (const uint32_t *)Wg, (const uint32_t *)Wu, X, Y, n_tok, M, K, true,
                       (__bf16 *)Y_bf16);
}

extern "C" int chn_batch_qkv_q4r(chn_ctx *ctx, const void *Wq, const void *Wk, const void *Wv, const float *X,
                                 float *Yq, float *Yk, float *Yv, uint32_t n_tok, uint32_t q_dim, uint32_t kv_dim,
                                 uint32_t K) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, Wq && Wk && Wv && X && Yq && Yk && Yv, "NULL argument");
    CHN_REQUIRE(ctx, K > 0 && K % 32 == 0, "K=%u must be a positive multiple of 32", K);
    CHN_REQUIRE(ctx, aligned(X, 16) && aligned(Wq, 16) && aligned(Wk, 16) && aligned(Wv, 16), "misaligned argument");
    if (!n_tok || !q_dim || !kv_dim) return CHN_OK;
    int rc = ensure_workspace(ctx, (size_t)n_tok * K * 2);
    if (rc) return rc;
    return launch_q4gemm_qkv(ctx, X, (const uint32_t *)Wq, (const uint32_t *)Wk, (const uint32_t *)Wv, Yq, Yk, Yv,
                             n_tok, q_dim, kv_dim, K, (__bf16 *)ctx->ws);
}
