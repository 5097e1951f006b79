// Internal definitions shared by the gfx950 kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/channel_hip.h"

struct chn_ctx {
    int device = 0;
    std::string name;           // the device's marketing name and gfx target
    hipStream_t stream = nullptr;
    hipEvent_t t0 = nullptr, t1 = nullptr;
    std::string err;
    // Workspace for kernels that need partials (split-K attention, ...).
    // Grown on demand outside graph capture; owned by the context.  ws_gen
    // counts reallocations: a recording made at another generation would
    // read a freed workspace and is refused.
    void *ws = nullptr;
    size_t ws_bytes = 0;
    uint64_t ws_gen = 0;
    bool recording = false;     // between chn_record_begin and chn_record_end
    std::vector<chn_recording *> recs;   // live recordings, released by chn_destroy
};

namespace chn {

int set_err(chn_ctx *ctx, int code, const char *fmt, ...);
int hip_fail(chn_ctx *ctx, hipError_t e, const char *what);
// Make sure ctx->ws holds at least `bytes`; returns a status code.
int ensure_workspace(chn_ctx *ctx, size_t bytes);
// Resolve, once per device (the context's device current), the address of
// the file-scope scratch chn_decode_attn_noalloc uses.
int noalloc_scratch_init(chn_ctx *ctx);

#define CHN_HIP(ctx, call)                                   \
    do {                                                     \
        hipError_t e_ = (call);                              \
        if (e_ != hipSuccess) return chn::hip_fail((ctx), e_, #call); \
    } while (0)

// Check the launch that was just enqueued.
#define CHN_LAUNCHED(ctx, what)                              \
    do {                                                     \
        hipError_t e_ = hipGetLastError();                   \
        if (e_ != hipSuccess) return chn::hip_fail((ctx), e_, what); \
    } while (0)

#define CHN_REQUIRE(ctx, cond, ...)                          \
    do {                                                     \
        if (!(cond)) return chn::set_err((ctx), CHN_E_INVALID, __VA_ARGS__); \
    } while (0)

inline bool aligned(const void *p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

// ---- activation digit planes (the matvec's input format)
// Per 32-block b of an activation vector: X_i = rint(x_i * 2^(18 - e_b))
// with |x_i| < 2^e_b, five balanced base-16 digits per X_i, each digit plane
// packed as signed 4-bit lanes in the weights' nibble order.  Stored SoA:
// u32 plane words at [(p * 4 + w) * nb + b] (p = plane, w = 8-element
// word), then nb float scales 2^(e_b - 18).  The rounding of x is at most
// 2^-18 of the block maximum (the size of fp32's own rounding noise over a
// few thousand accumulated products).
constexpr int XP_PLANES = 5;
constexpr int XP_FRAC = 18;
constexpr int XP_WORDS = XP_PLANES * 4;
// X + XP_BIAS has digit 8 + D_p in every hex position p < XP_PLANES
// (|X| < 2^XP_FRAC keeps every digit in [0, 15]).
constexpr uint32_t XP_BIAS = 0x88888u;
static_assert(XP_BIAS == (((1u << (4 * XP_PLANES)) - 1u) / 15u) * 8u, "XP_BIAS: 8 in each of XP_PLANES digits");
static_assert(4 * XP_PLANES - 1 >= XP_FRAC + 1, "digits must cover |X| < 2^XP_FRAC");
inline size_t xplanes_bytes(uint32_t nb) { return (size_t)nb * (XP_WORDS + 1) * 4; }

// ---- internal launchers (explicit workspaces; usable under graph capture)
// With planes_ready, `ws` already holds the digit planes of x (written by
// the producing kernel) and the fast matvec path reads them directly; x is
// still read by the general-shape path.
size_t mv_ws_bytes(uint32_t K);
int mv_gemv(chn_ctx *ctx, const uint32_t *W, const float *x, float *y, uint32_t M, uint32_t K, uint32_t *ws,
            bool planes_ready = false);
int mv_qkv(chn_ctx *ctx, const uint32_t *Wq, const uint32_t *Wk, const uint32_t *Wv, const float *x, float *q,
           float *k, float *v, uint32_t q_dim, uint32_t kv_dim, uint32_t K, uint32_t *ws, bool planes_ready = false);
int mv_mlp(chn_ctx *ctx, const uint32_t *Wg, const uint32_t *Wu, const float *x, float *act, uint32_t M, uint32_t K,
           uint32_t *ws, bool planes_ready = false);
int launch_rmsnorm(hipStream_t s, float *x, const float *r, const float *w, float *y, uint32_t dim, uint32_t rows,
                   float eps, float scalar, bool add);
// The prefill's norm chain per token row: the branch is the sum of the
// nparts (1, 2 or 4) partial outputs r + p * pstride of a split
// contraction, added in index order; with post_w, r' = rmsnorm(branch) *
// post_w (else r' = branch); with add, x = (x + r') * scalar (written
// back); y = rmsnorm(x) * w as bf16 into yb and, if y != NULL, as fp32.
// The same arithmetic, in the same order, as launch_rmsnorm's two passes.
int launch_rmsnorm_chain(hipStream_t s, float *x, const float *r, const float *post_w, const float *w, __bf16 *yb,
                         float *y, uint32_t dim, uint32_t rows, float eps, float scalar, bool add,
                         uint32_t nparts = 1, size_t pstride = 0);
// Digit planes of x (nb 32-blocks) into xp (xplanes_bytes(nb)).
int launch_xplanes(hipStream_t s, const float *x, uint32_t *xp, uint32_t nb);

// ---- repacked Q4 ("Q4R"): per matrix [rows][nb] 16-byte nibble words
// (each nibble XOR 8, i.e. two's-complement q - 8), then [rows][nb] f16
// scales.  18 bytes per 32 weights; the reference layout's unused f16 min
// is dropped.
inline size_t q4r_bytes(uint32_t rows, uint32_t K) { return (size_t)rows * (K / 32) * 18; }
int launch_q4_repack(hipStream_t s, const uint32_t *W, uint32_t rows, uint32_t K, void *dst);
// Matvecs over Q4R weights with activation planes already in xp (or, if
// !planes_ready, computed from x into xp first).  K % 32 == 0, K <= 16384.
// skip (or NULL): the layer's quiescence flag; when set the launch does nothing.
int mvr_gemv(chn_ctx *ctx, const void *W, const float *x, float *y, uint32_t M, uint32_t K, uint32_t *xp,
             bool planes_ready, const uint32_t *skip = nullptr);
int mvr_qkv(chn_ctx *ctx, const void *Wq, const void *Wk, const void *Wv, const float *x, float *q, float *k,
            float *v, uint32_t q_dim, uint32_t kv_dim, uint32_t K, uint32_t *xp, bool planes_ready);
int mvr_mlp(chn_ctx *ctx, const void *Wg, const void *Wu, const float *x, float *act, uint32_t M, uint32_t K,
            uint32_t *xp, bool planes_ready);
// gate/up that also writes the digit planes of act into xp_out (the down
// projection's input); xp_out must not alias xp_in
int mvr_mlp_xp(chn_ctx *ctx, const void *Wg, const void *Wu, const uint32_t *xp_in, float *act,
               uint32_t *xp_out, uint32_t M, uint32_t K);
// Decode-step norm with planes: r' = post ? rmsnorm(r) * post_w : r;
// x = add ? (x + r') * scalar : x; y = rmsnorm(x) * w; planes of y into xp
// (if non-NULL).  One row, dim % 8 == 0, dim <= 8192.
// Per-step RoPE table, written by the decode step's first norm kernel and
// read by every layer's attention: (cos, sin) of clock * theta^(-2d / rot)
// for d < rot / 2, kind 0 = sliding layers, kind 1 = full layers, each
// kRopePairs entries (rot <= 512).
constexpr uint32_t kRopePairs = 256;
struct RopeTab {
    const uint32_t *step;   // device {clock, ...}
    float2 *tab;            // [2][kRopePairs]
    float theta[2];
    uint32_t rot[2];
};
// skip (or NULL): the last layer's quiescence flag; when set, x keeps its
// value and the planes are made from y as it stands (the layer wrote none).
// xb (or NULL) receives the byte planes of y (the Q8 logits matvec's input,
// launch_gemv_q8r with planes_ready).
int launch_norm_planes(hipStream_t s, float *x, const float *r, const float *post_w, const float *w, float *y,
                       uint32_t *xp, uint32_t dim, float eps, float scalar, bool add,
                       const RopeTab *rope = nullptr, const uint32_t *skip = nullptr, uint32_t *xb = nullptr);

// The RoPE table entries i = t, t + nt, ... of rt (same arithmetic as the
// reference's per-element rotation: theta^(2d / rot) by powf, sincosf).
__device__ __forceinline__ void rope_table(const RopeTab &rt, uint32_t t, uint32_t nt) {
    const uint32_t clock = rt.step[0];
    for (uint32_t i = t; i < 2 * kRopePairs; i += nt) {
        // selects, not rt.rot[kind]: a runtime index into a by-value argument
        // would copy it to scratch
        const uint32_t kind = i / kRopePairs, d = i % kRopePairs, rot = kind ? rt.rot[1] : rt.rot[0];
        if (d < rot / 2) {
            const float fe = (2.0f * (float)d) / (float)rot;
            const float freq = 1.0f / powf(kind ? rt.theta[1] : rt.theta[0], fe);
            const float ang = (float)clock * freq;
            float sn, cs;
            sincosf(ang, &sn, &cs);
            rt.tab[i] = float2{cs, sn};
        }
    }
}

// The decode step's norm, as the fused matvecs recompute it in every
// workgroup: r' = post ? rmsnorm(r) * pw : r; xn = add ? (x_in + r') *
// scalar : x_in; y = rmsnorm(xn) * w, whose digit planes feed the matvec.
// Workgroup 0 writes xn to x_out (never x_in: the other workgroups still
// read it) and y (if non-NULL).
enum NormMode { NORM_PLAIN = 0, NORM_ADD = 1, NORM_POST_ADD = 2 };
// Quiescence gating of a decode layer (the reference's indirect dispatch,
// src/gpu/model_dispatch.zig:47-101, shaders/quiescence_gate.wgsl): a
// layer whose input stream moved by less than thresh (mean square) since
// the previous gated step runs none of its kernels.  NULL pointers: not
// gated.
struct Quiesce {
    const uint32_t *prev_skip;   // the previous layer's flag: its FFN residual was not produced
    uint32_t *skip;              // this layer's flag (written by the QKV kernel, read by the others)
    float *x_prev;               // this layer's input stream at the previous gated step
    float thresh;
    uint32_t first;              // layer 0: no previous layer wrote the normed row
};
struct NormArgs {
    const float *x_in, *r, *pw, *w;
    float *x_out, *y;
    float eps, scalar;
    RopeTab rope;          // tab != NULL: workgroup 0 also writes the step's RoPE table
    Quiesce q;             // zero: no gating
};
int mvr_qkv_nx(chn_ctx *ctx, const void *Wq, const void *Wk, const void *Wv, float *q, float *k, float *v,
               uint32_t q_dim, uint32_t kv_dim, uint32_t K, const NormArgs &n, int mode);
int mvr_mlp_nx(chn_ctx *ctx, const void *Wg, const void *Wu, float *act, uint32_t *xp_out, uint32_t M,
               uint32_t K, const NormArgs &n, int mode);
int launch_qkv_rope(hipStream_t st, const float *q_in, const float *k_in, const float *v_in, const float *qw,
                    const float *kw, float *q_out, float *kc, float *vc, const uint32_t *step, uint32_t num_q,
                    uint32_t num_kv, uint32_t D, uint32_t rot, int k_eq_v, float theta, float eps);
// tab (or NULL): the prompt's (cos, sin) table from launch_rope_tab_batch
// for this rot and theta.  frag (or NULL): launch_prefill_attn's fragment
// buffer for the same tokens, slot_offset previous keys and window; the
// launch then also writes the new keys' fragments (needs tab, D 256 and
// prefill_frags_fusable), and launch_prefill_attn is told so.
int launch_batch_qkv_rope(hipStream_t st, const float *q_in, const float *k_in, const float *v_in, const float *qw,
                          const float *kw, float *q_out, float *kc, float *vc, const uint32_t *slots,
                          uint32_t slot_offset, uint32_t start_clock, uint32_t n_tok, uint32_t num_q, uint32_t num_kv,
                          uint32_t D, uint32_t rot, int k_eq_v, float theta, float eps, const float2 *tab = nullptr,
                          unsigned char *frag = nullptr, size_t frag_bytes = 0, uint32_t window = 0);
int launch_rope_tab_batch(hipStream_t st, float2 *tab, uint32_t start_clock, uint32_t n_tok, uint32_t rot,
                          float theta);
size_t attn_ws_bytes(uint32_t num_q_heads, uint32_t head_dim, uint32_t max_slots);
// ws holds attn_ws_bytes(); xp (nullable) receives the digit planes of out
// (num_q_heads * head_dim / 32 blocks).
int launch_decode_attn(chn_ctx *ctx, const float *q, const float *kc, const float *vc, const uint32_t *slots,
                       const uint32_t *n_slots, uint32_t max_slots, uint32_t num_q_heads, uint32_t head_dim,
                       uint32_t kv_dim, uint32_t gqa, float scale, float *out, float *ws, uint32_t *xp);
// The decode step's qkv_rope fused into decode attention: q_in/k_in/v_in
// are the raw QKV matvec outputs, step = {clock, slot_idx, ...} on the
// device; the new token's K/V are written to the caches at slot_idx.
int launch_rope_decode_attn(chn_ctx *ctx, const float *q_in, const float *k_in, const float *v_in, const float *qw,
                            const float *kw, float *kc, float *vc, const uint32_t *step, const uint32_t *slots,
                            const uint32_t *n_slots, uint32_t max_slots, uint32_t num_q_heads, uint32_t head_dim,
                            uint32_t kv_dim, uint32_t gqa, uint32_t rot, int k_eq_v, const float2 *rope_tab,
                            float eps, float scale, float *out, float *ws, uint32_t *xp,
                            const uint32_t *skip = nullptr);
// out: [n_tok][num_q_heads * head_dim] fp32, or bf16 into outb when set.
// ws (prefill_attn_ws_bytes, or NULL): lets short prompts split each query
// tile's keys between two workgroups.  frag (prefill_frag_bytes for the
// KV heads and num_prev + n_tok keys): the keys' bf16 operand fragments,
// required at head_dim 256.
size_t prefill_attn_ws_bytes(uint32_t n_tok, uint32_t num_q_heads, uint32_t head_dim);
size_t prefill_frag_bytes(uint32_t num_kv_heads, uint32_t n_keys);
// new_frags_ready: the fragments of the new tokens' key chunks were written
// by launch_batch_qkv_rope; only the earlier keys' are built here.
bool prefill_frags_fusable(uint32_t num_prev, uint32_t head_dim, uint32_t gqa);
int launch_prefill_attn(hipStream_t st, const float *q, const float *kc, const float *vc, const uint32_t *slots,
                        uint32_t n_tok, uint32_t num_prev, uint32_t num_q_heads, uint32_t head_dim, uint32_t kv_dim,
                        uint32_t gqa, float scale, uint32_t window, float *out, __bf16 *outb, float *ws,
                        unsigned char *frag, size_t frag_bytes, bool new_frags_ready = false);
size_t xbytes_bytes(uint32_t nb);
int launch_gemv_q8(hipStream_t st, const uint32_t *W, const float *x, float *y, uint32_t M, uint32_t nb,
                   uint32_t *xp_ws);
// Q8R (Q8_0 repacked for coalesced streaming: [rows][2][nb] 16-byte code
// halves, then the [rows * nb] f32 scales) and the Q8 matvec over it
// (identical results to launch_gemv_q8 on the same weights).
int launch_q8_repack(hipStream_t st, const uint32_t *W, uint32_t rows, uint32_t nb, void *dst);
int launch_gemv_q8r(hipStream_t st, const void *R, const float *x, float *y, uint32_t M, uint32_t nb,
                    uint32_t *xp_ws, bool planes_ready = false);
size_t topk_ws_bytes(uint32_t V);
// Optional end of a device-side greedy step, done by the top-64 merge once
// ids[0] is known: out[gen[1]] = ids[0] (while gen[1] < cap), then gen[1] and
// the clock gen[0] advance by one.
struct GreedyTail {
    uint32_t *gen;
    uint32_t *out;
    uint32_t cap;
};
int launch_topk64(hipStream_t st, const float *logits, uint32_t V, uint32_t *ids, float *vals, uint64_t *ws,
                  const GreedyTail *tail = nullptr);
int launch_embed(hipStream_t st, const uint16_t *table, const uint32_t *tokens, uint32_t n, uint32_t H, float scale,
                 float *x);
int launch_quantize(hipStream_t st, int q8, const uint16_t *src, uint32_t *dst, uint64_t nblk);
// W0/W1 in the reference Q4 layout, or in Q4R with repacked.  X (fp32) is
// converted into xb; with X == NULL, xb already holds the bf16 activations.
// Yb (two-matrix form only): the result goes to Yb as bf16 instead of Y.
// po (single matrix): a shape that splits K may store its partial sums to
// Y + p * po->stride, p < po->max_parts (1, 2 or 4), with plain stores
// instead of clearing Y and adding into it; po->parts tells how many it
// wrote (their sum, in index order, is the result).
struct PartialOut {
    size_t stride = 0;         // elements between partial outputs
    uint32_t max_parts = 1;
    uint32_t parts = 1;        // set by the launch
};
int launch_q4gemm(chn_ctx *ctx, int nmat, const float *X, const uint32_t *W0, const uint32_t *W1, float *Y,
                  uint32_t n_tok, uint32_t M, uint32_t K, __bf16 *xb, bool repacked, __bf16 *Yb = nullptr,
                  PartialOut *po = nullptr);
// q, k, v (Q4R) over the same activations in one launch (X == NULL: xb
// already holds them).
int launch_q4gemm_qkv(chn_ctx *ctx, const float *X, const uint32_t *Wq, const uint32_t *Wk, const uint32_t *Wv,
                      float *Yq, float *Yk, float *Yv, uint32_t n_tok, uint32_t Mq, uint32_t Mkv, uint32_t K,
                      __bf16 *xb);

// ---------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------

// Hides known bits from the optimiser so that byte extraction from a
// masked nibble word lowers to v_cvt_f32_ubyte{0..3} (one op per weight)
// instead of a bitfield extract followed by a convert.
__device__ __forceinline__ uint32_t opaque_u32(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

__device__ __forceinline__ float f16_lo_to_f32(uint32_t w) {
    _Float16 h = __builtin_bit_cast(_Float16, (unsigned short)(w & 0xffffu));
    return (float)h;
}

// Dword-aligned 16-byte vector: global_load_dwordx4 accepts 4-byte
// alignment on gfx950, which lets one load take words 1..4 of a 20-byte
// Q4 block.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

// splitmix64 output function over a counter (same constants as the host
// restatement used to check generated inputs).
__device__ __forceinline__ uint64_t mix64(uint64_t seed, uint64_t idx) {
    uint64_t z = seed + (idx + 1ull) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__device__ __forceinline__ float gelu_tanh(float x) {
    float c = 0.044715f * x;
    c = c * x;
    c = c * x;
    float inner = 0.7978845608f * (x + c);
    return (0.5f * x) * (1.0f + tanhf(inner));
}

// Transposed butterfly: V values per lane (V a power of two <= 64) summed
// over the 64 lanes.  The sum for value index v ends up in every lane whose
// top log2(V) lane-index bits equal v, i.e. v = lane >> (6 - log2 V).
// All ones when ok, else zero, as a value the compiler cannot see through.
// Masking a loaded value with it (instead of `ok ? v : 0`) keeps the load
// unconditional: given a select, the compiler sinks the load into an
// `if (ok)` branch, and the wait after such a branch drains every load
// issued before it.
__device__ __forceinline__ uint32_t opaque_mask(bool ok) {
    uint32_t m = ok ? 0xffffffffu : 0u;
    __asm__ volatile("" : "+v"(m));
    return m;
}
__device__ __forceinline__ float mask_f(float v, uint32_t m) {
    return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, v) & m);
}

template <int V>
__device__ __forceinline__ float wave_reduce_v(const float (&acc)[V], int lane) {
    static_assert(V >= 1 && V <= 64 && (V & (V - 1)) == 0, "V must be a power of two <= 64");
    float cur[V];
#pragma unroll
    for (int i = 0; i < V; ++i) cur[i] = acc[i];
    int m = 32;
#pragma unroll
    for (int n = V; n > 1; n >>= 1, m >>= 1) {
        const int h = n / 2;
        const bool hi = (lane & m) != 0;
#pragma unroll
        for (int i = 0; i < V / 2; ++i)
            if (i < h) {
                const float send = hi ? cur[i] : cur[i + h];
                const float keep = hi ? cur[i + h] : cur[i];
                cur[i] = keep + __shfl_xor(send, m, 64);
            }
    }
    float s = cur[0];
    for (; m >= 1; m >>= 1) s += __shfl_xor(s, m, 64);
    return s;
}

template <int V>
constexpr int ilog2_c() { return V <= 1 ? 0 : 1 + ilog2_c<V / 2>(); }

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

// Exchanges across the four 16-lane rows of a wave on gfx950's lane-swap
// instructions (VALU, no LDS crossbar).  permlane16_swap(v, v) returns
// {rows (0,0,2,2), rows (1,1,3,3)} of v, permlane32_swap(v, v) returns
// {halves (0,0), halves (1,1)}: the partner value of lane ^ 16 (^ 32) is
// the element of the other row (half).
__device__ __forceinline__ float xor16_lane(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                    false, false);
    return __builtin_bit_cast(float, ((threadIdx.x >> 4) & 1) ? r[0] : r[1]);
}
__device__ __forceinline__ float xor32_lane(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v), __builtin_bit_cast(uint32_t, v),
                                                    false, false);
    return __builtin_bit_cast(float, ((threadIdx.x >> 5) & 1) ? r[0] : r[1]);
}
// Sum / max over lanes l, l ^ 16, l ^ 32, l ^ 48 (same position in the four
// rows), ((r0 op r1) op (r2 op r3)) in every lane.
__device__ __forceinline__ float rows4_sum(float v) {
    v += xor16_lane(v);
    return v + xor32_lane(v);
}
__device__ __forceinline__ float rows4_max(float v) {
    v = fmaxf(v, xor16_lane(v));
    return fmaxf(v, xor32_lane(v));
}

// Transposed pair sums on one lane swap: permlane32_swap(x, y) leaves
// {x_lo, y_lo} and {x_hi, y_hi}, so lane l of the low half gets
// x_l + x_{l+32} and lane l of the high half y_{l-32} + y_l (and likewise
// for rows 0/1 and 2/3 with permlane16_swap).  The two results pass through
// an empty asm as integers: this compiler otherwise folds "float of result 0
// + float of result 1" into result 0 + result 0.
__device__ __forceinline__ float add_swapped(uint32_t a, uint32_t b) {
    __asm__("" : "+v"(a), "+v"(b));
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float swap_add32(float x, float y) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, y),
                                                    false, false);
    return add_swapped(r[0], r[1]);
}
__device__ __forceinline__ float swap_add16(float x, float y) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, y),
                                                    false, false);
    return add_swapped(r[0], r[1]);
}
__device__ __forceinline__ float lane_f(float v, int l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
// Whole-wave sums of two / four values at once.  Every total is formed by
// the same tree, ((x_l + x_{l^32}) + (x_{l^16} + x_{l^48})) over the 16
// lanes of a DPP row, taken from the row's lane 0, so wave_sum2(a, b) and
// wave_sum4(a, b, ., .) give a and b the same bits.
__device__ __forceinline__ void wave_sum2(float a, float b, float &ta, float &tb) {
    float c = swap_add32(a, b);       // half 0: a, half 1: b
    c = row16_sum(swap_add16(c, c));
    ta = lane_f(c, 0);
    tb = lane_f(c, 32);
}
__device__ __forceinline__ void wave_sum4(float v0, float v1, float v2, float v3, float (&t)[4]) {
    const float a = swap_add32(v0, v2), b = swap_add32(v1, v3);   // half 0: v0, v1; half 1: v2, v3
    const float c = row16_sum(swap_add16(a, b));                   // rows 0..3: v0, v1, v2, v3
    t[0] = lane_f(c, 0);
    t[1] = lane_f(c, 16);
    t[2] = lane_f(c, 32);
    t[3] = lane_f(c, 48);
}

// Digit planes of one 32-block from the four lanes 4k..4k+3 of a wave that
// hold its words w = lane & 3 (eight consecutive values each).  All four
// lanes must call (with zeros where ok is false); only ok lanes store.
// Plane word (p, w) of block b goes to xp[(p * 4 + w) * ws + b * bs], the
// block's scale to xp[XP_WORDS * ws + b * bs].
// A block holding NaN or Inf gets zero digits and a NaN scale, so every
// product with it is NaN, as the fp32 products of the reference would be
// non-finite.  Blocks whose largest magnitude is below 2^-100 contribute
// zero (their products are below 2^-100 of the weights).
__device__ __forceinline__ void emit_planes8s(const float (&v)[8], uint32_t *__restrict__ xp, uint32_t ws,
                                              uint32_t bs, uint32_t b, uint32_t w, bool ok) {
    float m = 0.0f;
    uint32_t bad = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        m = fmaxf(m, fabsf(v[i]));
        bad |= !(fabsf(v[i]) <= 3.4028235e38f);     // NaN or Inf
    }
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    m = fmaxf(m, __shfl_xor(m, 2, 64));
    bad |= __shfl_xor(bad, 1, 64);
    bad |= __shfl_xor(bad, 2, 64);
    int e = 0;
    (void)frexpf(m, &e);           // m = f * 2^e, f in [0.5, 1): |x_i| < 2^e
    float scale = 0.0f, inv = 0.0f;
    if (bad) {
        inv = __builtin_nanf("");
    } else if (m > 0.0f && e > -100) {
        scale = ldexpf(1.0f, XP_FRAC - e);
        inv = ldexpf(1.0f, e - XP_FRAC);
    }
    uint32_t u[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) u[i] = (uint32_t)((int)rintf((bad ? 0.0f : v[i]) * scale) + (int)XP_BIAS);
    if (!ok) return;
#pragma unroll
    for (int p = 0; p < XP_PLANES; ++p) {
        uint32_t word = 0;
#pragma unroll
        for (int n = 0; n < 8; ++n) word |= ((u[n] >> (4 * p)) & 15u) << (4 * n);
        xp[(size_t)(p * 4 + w) * ws + (size_t)b * bs] = word ^ 0x88888888u;
    }
    if (w == 0) ((float *)xp)[(size_t)XP_WORDS * ws + (size_t)b * bs] = inv;
}

// Byte planes of the Q8 logits matvec's input: per 32-block, three balanced
// base-256 digits of a 22-bit fixed-point value, plane word (p, w) (four
// elements 4w .. 4w + 3) at xp[(p * 8 + w) * nb + b], the block's scale
// 2^(e_b - 22) at xp[XB_WORDS * nb + b] (as float).
constexpr int XB_PLANES = 3;
constexpr int XB_FRAC = 22;
constexpr int XB_WORDS = XB_PLANES * 8;   // 8 int8x4 words per plane per block

// The byte planes of one 32-block from the four lanes 4k..4k+3 of a wave
// that hold its values 8q .. 8q + 7 (q = lane & 3); all four lanes must
// call (with zeros where ok is false), only ok lanes store.  The same
// arithmetic per element as k_xbytes (eight lanes of four values): the
// block maximum is order-independent, so the planes are identical.
__device__ __forceinline__ void emit_bytes8(const float (&v)[8], uint32_t *__restrict__ xp, uint32_t nb,
                                            uint32_t b, uint32_t q, bool ok) {
    float m = 0.0f;
    uint32_t bad = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        m = fmaxf(m, fabsf(v[i]));
        bad |= !(fabsf(v[i]) <= 3.4028235e38f);     // NaN or Inf
    }
    m = fmaxf(m, __shfl_xor(m, 1, 64));
    m = fmaxf(m, __shfl_xor(m, 2, 64));
    bad |= __shfl_xor(bad, 1, 64);
    bad |= __shfl_xor(bad, 2, 64);
    int e = 0;
    (void)frexpf(m, &e);
    float scale = 0.0f, inv = 0.0f;
    if (bad) {
        inv = __builtin_nanf("");
    } else if (m > 0.0f && e > -100) {
        scale = ldexpf(1.0f, XB_FRAC - e);
        inv = ldexpf(1.0f, e - XB_FRAC);
    }
    uint32_t u[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) u[i] = (uint32_t)((int)rintf((bad ? 0.0f : v[i]) * scale) + 0x808080);
    if (!ok) return;
#pragma unroll
    for (int p = 0; p < XB_PLANES; ++p)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            uint32_t word = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) word |= ((u[4 * h + j] >> (8 * p)) & 0xffu) << (8 * j);
            xp[(size_t)(p * 8 + 2 * q + h) * nb + b] = word ^ 0x80808080u;
        }
    if (q == 0) ((float *)(xp + (size_t)XB_WORDS * nb))[b] = inv;
}

// Planes in the chn_xplanes layout: plane word (p, w) of block b at
// [(p * 4 + w) * nb + b], the scale at [XP_WORDS * nb + b].
__device__ __forceinline__ void emit_planes8(const float (&v)[8], uint32_t *__restrict__ xp, uint32_t nb,
                                             uint32_t b, uint32_t w, bool ok) {
    emit_planes8s(v, xp, nb, 1, b, w, ok);
}


// ---------------------------------------------------------------------
// DMA into LDS (global_load_lds) and the waits around it, shared by the
// pipelined prefill kernels.
// ---------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_t;

// vmcnt(n) and lgkmcnt(0) (gfx9 encoding: vmcnt[3:0] and [15:14],
// expcnt[6:4], lgkmcnt[11:8]).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    static_assert(N >= 0 && N < 64, "vmcnt immediate");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
}


// Workgroup barrier without a memory fence; the compiler may not move
// memory accesses across it.
__device__ __forceinline__ void bare_barrier() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
}

// LDS reads of DMA-filled memory.  The compiler cannot tell ring slots
// apart and would make every LDS read wait for the newest DMA group; reads
// issued as asm are ordered by the explicit waits instead.  Their results
// must stay in the registers the asm wrote until lds_wait() (a copy made
// earlier would copy a value not yet loaded): lds_pin() after the wait keeps
// every use below it.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
template <typename T, int OFF = 0>
__device__ __forceinline__ T lds_read(uint32_t addr) {
    static_assert(OFF >= 0 && OFF < 65536, "ds offset");
    T v;
    if constexpr (sizeof(T) == 16) __asm__ volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    else if constexpr (sizeof(T) == 8) __asm__ volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    else __asm__ volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
    return v;
}
__device__ __forceinline__ void lds_wait() { __asm__ volatile("s_waitcnt lgkmcnt(0)"); }
template <int N>                                           // all but the newest N LDS operations done
__device__ __forceinline__ void lds_wait_n() {
    static_assert(N >= 0 && N < 16, "lgkmcnt immediate");
    __asm__ volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N));
}
template <typename T>
__device__ __forceinline__ void lds_pin(T &v) {
    __asm__ volatile("" : "+v"(v));
}

}  // namespace chn
