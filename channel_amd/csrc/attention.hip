// Decode attention over the ring-buffer slot list (shaders/decode_attn.wgsl),
// prefill causal attention (shaders/batch_causal_attn.wgsl) and the
// per-head RMSNorm + RoPE + KV-cache write (shaders/qkv_rope.wgsl).
//
// Decode attention is split over the slot list ("flash-decoding").  The
// slot count S is read from device memory (so a captured graph replays with
// a new count).  The list is cut into 16-entry chunks dealt round-robin to
// at most 32 workgroups per KV head, so a 512-entry sliding window spreads
// over 256 workgroups and a full 4096-entry ring gives each eight chunks.
// A workgroup serves all of its KV head's GQA query heads from one pass over
// K and V: each 16-lane row of a wave owns one list entry per chunk (a 1 KB
// row, read as four 256-byte runs, 16 bytes per lane each: lane c holds
// dims 4c + 64f .. + 3), scores reduce inside the row with DPP, and each
// wave keeps its own online softmax state.  The four waves
// merge in LDS into one partial (m, l, sum p*V) per query head; a second
// kernel merges the partials (online, in a fixed order), writes the output
// and, optionally, its activation digit planes for the o_proj matvec.  The
// result equals the reference's two-pass softmax p_i = exp(s_i - max) /
// (sum exp(s_j - max) + 1e-9) up to rounding.
#include "chn_internal.h"

#include <mutex>
#include <type_traits>

namespace chn {

constexpr int kAttnChunk = 64;     // prefill: slots per online-softmax step
constexpr uint32_t kDecGrid = 32;  // decode: workgroups per KV head (at most)
constexpr int kMaxChunks = 8;      // decode: 16-entry chunks per split at most (4096 / 16 / kDecGrid)
static_assert(kMaxChunks * 16 * kDecGrid >= 4096, "a split's chunks of the largest list");
constexpr float kNegBig = -1e30f;

typedef float f4 __attribute__((ext_vector_type(4)));

// Decode splits per KV head: one per 16-entry chunk of max_slots, at most
// kDecGrid (a split then takes every kDecGrid-th chunk: 8 of 256 at 4096).
static uint32_t dec_splits(uint32_t max_slots) {
    const uint32_t n = (max_slots + 15) / 16;
    return n < kDecGrid ? n : kDecGrid;
}

// Decode workspace: partial sums [splits][num_q_heads][head_dim], then
// maxima and denominators [splits][num_q_heads].
size_t attn_ws_bytes(uint32_t num_q_heads, uint32_t head_dim, uint32_t max_slots) {
    return (size_t)dec_splits(max_slots) * num_q_heads * ((size_t)head_dim + 2) * 4;
}

// Prefill key split: a query tile's key chunks are cut into parts of about
// kPaPartChunks chunks, at most kPaParts parts (one workgroup each), so the
// causal tiles' walks come out about equally long; the workspace holds each
// part's sums [n_tok][heads][D] and (max, denominator) pairs.
constexpr uint32_t kPaParts = 4;
constexpr uint32_t kPaPartChunks = 4;
// Waves per prefill attention workgroup, 16 query rows each: eight waves
// (128 query rows) share every 64 KB chunk the workgroup copies into LDS.
constexpr int kPaWaves = 8;
size_t prefill_attn_ws_bytes(uint32_t n_tok, uint32_t num_q_heads, uint32_t head_dim) {
    return kPaParts * (size_t)n_tok * num_q_heads * ((size_t)head_dim + 2) * 4;
}

// Running softmax state of one lane: lane row r = lane / 16 holds slots
// r, r+4, r+8, r+12 of each wave's 16, column c = lane % 16 holds 16*DV
// consecutive dims, so one slot's row (1 KB at D = 256) is read by a
// 16-lane row as 64 contiguous bytes per lane and its score reduces inside
// the row with DPP.
template <int DV, int GQA>
struct AttnState {
    float M[GQA], l[GQA];
    f4 acc[GQA][4 * DV];
};

// One 64-slot chunk [c0, c0 + cnt) of the list for KV head kvh: scores,
// running max / sum update (rescaling the accumulators), p-weighted V.
template <int DV, int GQA>
__device__ __forceinline__ void attn_chunk(AttnState<DV, GQA> &st, const f4 (&q)[GQA][4 * DV],
                                           const float *__restrict__ Kc, const float *__restrict__ Vc,
                                           const uint32_t *__restrict__ slots, uint32_t c0, uint32_t cnt,
                                           uint32_t kv_dim, uint32_t kvh, float scale, float (&sc)[GQA][kAttnChunk]) {
    constexpr int D = DV * 256;
    constexpr int NF = 4 * DV;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane >> 4, c = lane & 15;
    const uint32_t base = c0 + wave * 16;
    const uint32_t nval = cnt > (uint32_t)(wave * 16) ? cnt - wave * 16 : 0;
    const uint32_t my_slot = (uint32_t)lane < nval && lane < 16 ? slots[base + lane] : 0u;
    const size_t dim0 = (size_t)kvh * D + (size_t)c * NF * 4;

    f4 kr[4][NF], vr[4][NF];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = r + 4 * u;
        const uint32_t ps = (uint32_t)__shfl(my_slot, i, 64);
        const bool ok = (uint32_t)i < nval;
        const float *kp = Kc + (size_t)ps * kv_dim + dim0;
#pragma unroll
        for (int f = 0; f < NF; ++f) kr[u][f] = ok ? *(const f4 *)(kp + 4 * f) : f4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = r + 4 * u;
        const uint32_t ps = (uint32_t)__shfl(my_slot, i, 64);
        const bool ok = (uint32_t)i < nval;
        const float *vp = Vc + (size_t)ps * kv_dim + dim0;
#pragma unroll
        for (int f = 0; f < NF; ++f) vr[u][f] = ok ? *(const f4 *)(vp + 4 * f) : f4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int h = 0; h < GQA; ++h) {
            float d = 0.0f;
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                d = fmaf(q[h][f].x, kr[u][f].x, d);
                d = fmaf(q[h][f].y, kr[u][f].y, d);
                d = fmaf(q[h][f].z, kr[u][f].z, d);
                d = fmaf(q[h][f].w, kr[u][f].w, d);
            }
            d = row16_sum(d);
            if (c == 0) sc[h][wave * 16 + r + 4 * u] = d * scale;
        }
    __syncthreads();
    float p[GQA];
#pragma unroll
    for (int h = 0; h < GQA; ++h) {
        const float sv = (uint32_t)lane < cnt ? sc[h][lane] : kNegBig;
        const float Mn = fmaxf(st.M[h], wave_max64(sv));
        const float e = (uint32_t)lane < cnt ? expf(sv - Mn) : 0.0f;
        const float rs = expf(st.M[h] - Mn);
        st.l[h] = st.l[h] * rs + wave_sum64(e);
#pragma unroll
        for (int f = 0; f < NF; ++f) st.acc[h][f] *= rs;
        st.M[h] = Mn;
        p[h] = e;
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int h = 0; h < GQA; ++h) sc[h][lane] = p[h];
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int i = r + 4 * u;
        if ((uint32_t)i < nval) {
#pragma unroll
            for (int h = 0; h < GQA; ++h) {
                const float pw = sc[h][wave * 16 + i];
#pragma unroll
                for (int f = 0; f < NF; ++f) st.acc[h][f] += pw * vr[u][f];
            }
        }
    }
    __syncthreads();   // sc is rewritten by the next chunk
}

// Sum the 16 (wave, row) partial accumulators of each head in a fixed order
// and hand each finished float4 column to `emit(head, column, value)`.
template <int DV, int GQA, typename Emit>
__device__ __forceinline__ void attn_reduce(const AttnState<DV, GQA> &st, f4 (*pacc)[GQA < 2 ? GQA : 2][64 * DV],
                                            Emit emit) {
    constexpr int NF = 4 * DV;
    constexpr int HC = GQA < 2 ? GQA : 2;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane >> 4, c = lane & 15;
#pragma unroll
    for (int h0 = 0; h0 < GQA; h0 += HC) {
#pragma unroll
        for (int hh = 0; hh < HC; ++hh)
#pragma unroll
            for (int f = 0; f < NF; ++f) pacc[wave * 4 + r][hh][c * NF + f] = st.acc[h0 + hh][f];
        __syncthreads();
        for (int idx = threadIdx.x; idx < HC * 16 * NF; idx += 256) {
            const int hh = idx / (16 * NF), col = idx % (16 * NF);
            f4 t = pacc[0][hh][col];
#pragma unroll
            for (int j = 1; j < 16; ++j) t += pacc[j][hh][col];
            emit(h0 + hh, col, t);
        }
        __syncthreads();
    }
}

template <int DV, int GQA>
__device__ __forceinline__ void load_q(f4 (&q)[GQA][4 * DV], const float *__restrict__ Q, uint32_t qh0) {
    constexpr int D = DV * 256;
    const int c = threadIdx.x & 15;
#pragma unroll
    for (int h = 0; h < GQA; ++h)
#pragma unroll
        for (int f = 0; f < 4 * DV; ++f) q[h][f] = *(const f4 *)(Q + (size_t)(qh0 + h) * D + c * 16 * DV + 4 * f);
}

// Inputs of the fused per-head RMSNorm + RoPE of the decode step
// (shaders/qkv_rope.wgsl): raw q/k/v from the QKV matvec, norm weights,
// device {clock, slot_idx}.
struct RopeArgs {
    const float *k_in, *v_in, *qw, *kw;
    const uint32_t *step;
    const float2 *tab;      // this layer kind's (cos, sin) for the step's clock
    uint32_t rot;
    float eps;
    int k_eq_v;
};

// One wave: RoPE over pairs (d, d + rot/2) of an LDS row in place; lane
// holds (cos, sin) of pairs d = lane + 64 k in cs[k].
template <int NP>
__device__ __forceinline__ void wave_rope_lds(float *row, uint32_t rot, const float2 (&cs)[NP], int lane) {
    const uint32_t half = rot / 2;
#pragma unroll
    for (int k = 0; k < NP; ++k) {
        const uint32_t d = lane + 64 * k;
        if (d < half) {
            const float v0 = row[d], v1 = row[d + half];
            row[d] = v0 * cs[k].x - v1 * cs[k].y;
            row[d + half] = v0 * cs[k].y + v1 * cs[k].x;
        }
    }
}

// Decode: grid (G, KV heads).  The slot list is taken in 16-entry chunks;
// workgroup `split` takes chunks split, split + G, split + 2 G, ..., two
// at a time, and row r of wave w holds entry
// 16 c + 4 w + r of chunk c.  The list entries of its first two chunks are
// read together with the slot count (the list holds max_slots entries; an
// entry is used only below the count), so the first K/V loads wait on one
// memory round trip; the next pair's entries are read while a pair is
// reduced, and each wave keeps a running softmax (max, sum, p-weighted V)
// over its chunks.  With ROPE, Q holds the raw q of the QKV matvec: every
// workgroup normalises and rotates its GQA query heads and the new token's
// K (and normalises its V) in LDS, uses them in place of the cache row of
// slot_idx, and split 0 writes them to the caches.
template <int DV, int GQA, bool ROPE>
__global__ __launch_bounds__(256) void k_attn_decode(const float *__restrict__ Q, float *Kc, float *Vc,
                                                     const uint32_t *__restrict__ slots,
                                                     const uint32_t *__restrict__ n_slots, uint32_t max_slots,
                                                     uint32_t num_q_heads, uint32_t kv_dim, float scale,
                                                     float *__restrict__ ws, RopeArgs ra,
                                                     const uint32_t *__restrict__ skip) {
    if (skip && *skip) return;          // a quiescent layer: no K/V write, no attention (uniform)
    constexpr int D = DV * 256;
    constexpr int NF = 4 * DV;          // float4 per lane per row
    const uint32_t split = blockIdx.x, kvh = blockIdx.y, G = gridDim.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r = lane >> 4, c = lane & 15;
    const uint32_t qh0 = kvh * GQA;

    __shared__ f4 sh_acc[4][GQA][D / 4];
    __shared__ float sh_m[4][GQA], sh_l[4][GQA];
    __shared__ float sh_q[ROPE ? GQA : 1][ROPE ? D : 4];
    __shared__ float sh_k[ROPE ? D : 4], sh_v[ROPE ? D : 4];

    // The prologue's inputs are loaded first (ROPE): the raw q / k / v of this
    // wave's items and their norm weights.  Loads complete in issue order, so
    // the norms below then run while the K/V rows are still in flight.
    constexpr int NIT = ROPE ? (GQA + 2 + 3) / 4 : 1;   // items per wave
    constexpr int DPL = D / 64;                          // values per lane
    float raw[NIT][DPL], nwt[NIT][DPL];
    float2 rcs[DPL / 2];                                 // (cos, sin) of pairs lane + 64 k
    if (ROPE) {
#pragma unroll
        for (int k = 0; k < DPL / 2; ++k) {
            const uint32_t d = lane + 64 * k;
            rcs[k] = d < ra.rot / 2 ? ra.tab[d] : float2{1.0f, 0.0f};
        }
        const float *vsrc = ra.k_eq_v ? ra.k_in : ra.v_in;
#pragma unroll
        for (int j = 0; j < NIT; ++j) {
            const int it = wave + 4 * j;
            const float *src = it < GQA ? Q + (size_t)(qh0 + it) * D
                                        : (it == GQA ? ra.k_in : vsrc) + (size_t)kvh * D;
            const float *wsrc = it < GQA ? ra.qw : ra.kw;
            const bool has = it < GQA + 2, hw = it < GQA + 1;
#pragma unroll
            for (int d = 0; d < DPL; ++d) {
                raw[j][d] = has ? src[lane + 64 * d] : 0.0f;
                nwt[j][d] = hw ? wsrc[lane + 64 * d] : 1.0f;
            }
        }
    }
    // splits without entries leave an empty partial (max -1e30, sum 0)
    auto write_empty = [&]() {
        float *wm = ws + (size_t)G * num_q_heads * D;
        float *wl = wm + (size_t)G * num_q_heads;
        if (threadIdx.x < (uint32_t)GQA) {
            wm[(size_t)split * num_q_heads + qh0 + threadIdx.x] = kNegBig;
            wl[(size_t)split * num_q_heads + qh0 + threadIdx.x] = 0.0f;
        }
    };

    const uint32_t row_ent = 4 * wave + r;
    const uint32_t ntmax = ((max_slots + 15) / 16 + G - 1 - split) / G;   // chunks this split could own
    auto entry = [&](uint32_t t) { return (split + G * t) * 16 + row_ent; };
    auto slot_at = [&](uint32_t t) {
        const uint32_t e = entry(t);
        const uint32_t v = slots[e < max_slots ? e : max_slots - 1];   // unconditional (exact waits)
        return t < ntmax ? v : 0u;
    };
    // Chunks go in pairs; NSET pairs are in flight: while one pair is reduced
    // the next one's K/V rows are loading.  Two sets where the registers
    // allow (D 256, GQA <= 2: 128 VGPRs of rows); they read every list entry
    // the split can own up front (at most kMaxChunks: 4096 entries in chunks
    // of 16 over min(256, kDecGrid) splits), one set reads a pair's entries
    // while the previous pair is reduced.  Either way the first entries are
    // read together with the count.
    constexpr int NSET = (DV == 1 && GQA <= 2) ? 2 : 1;
    constexpr int NSL = NSET == 2 ? kMaxChunks : 2;
    uint32_t sl[NSL];
#pragma unroll
    for (int t = 0; t < NSL; ++t) sl[t] = slot_at(t);
    uint32_t S = *n_slots;
    if (S > max_slots) S = max_slots;
    const uint32_t nch = (S + 15) / 16;
    const uint32_t iters = split < nch ? (nch - split + G - 1) / G : 0;
    // split 0 always runs when it has to write the new token's K/V
    if (!iters && !(ROPE && split == 0)) {
        write_empty();
        return;
    }
    const size_t dim0 = (size_t)kvh * D + (size_t)c * 4;

    bool ok[2 * NSET];                   // set s: buffers 2 s, 2 s + 1
    f4 kr[2 * NSET][NF], vr[2 * NSET][NF];
    // With two sets, rows past the count load cache row 0 instead: every
    // load is unconditional, so the waits count exactly the loads of the set
    // being reduced; their scores and V rows are masked in reduce.  One set
    // loads zeros for them.  The rows are read non-temporally: a step's K/V
    // over all layers outgrows the Infinity Cache, so allocating them there
    // only evicts other rows (4096 slots: 18.7-19.1 against 17.7-18.4 us per
    // step with the merge; decode +2 %).
    auto ldr = [](const float *p) { return __builtin_nontemporal_load((const f4 *)p); };
    auto issue = [&](int set, uint32_t t, uint32_t pa, uint32_t pb) {   // chunks t, t + 1 (t < iters)
        const int b0 = 2 * set, b1 = b0 + 1;
        ok[b0] = entry(t) < S;
        ok[b1] = t + 1 < iters && entry(t + 1) < S;
        const size_t ra = (size_t)(ok[b0] ? pa : 0u) * kv_dim + dim0;
        const size_t rb = (size_t)(ok[b1] ? pb : 0u) * kv_dim + dim0;
#pragma unroll
        for (int f = 0; f < NF; ++f) kr[b0][f] = NSET == 2 || ok[b0] ? ldr(Kc + ra + 64 * f) : f4{0, 0, 0, 0};
#pragma unroll
        for (int f = 0; f < NF; ++f) kr[b1][f] = NSET == 2 || ok[b1] ? ldr(Kc + rb + 64 * f) : f4{0, 0, 0, 0};
#pragma unroll
        for (int f = 0; f < NF; ++f) vr[b0][f] = NSET == 2 || ok[b0] ? ldr(Vc + ra + 64 * f) : f4{0, 0, 0, 0};
#pragma unroll
        for (int f = 0; f < NF; ++f) vr[b1][f] = NSET == 2 || ok[b1] ? ldr(Vc + rb + 64 * f) : f4{0, 0, 0, 0};
    };
    f4 q[GQA][NF];
    if (!ROPE) {                         // before the K/V rows: the first score needs q
#pragma unroll
        for (int h = 0; h < GQA; ++h)
#pragma unroll
            for (int f = 0; f < NF; ++f) q[h][f] = *(const f4 *)(Q + (size_t)(qh0 + h) * D + c * 4 + 64 * f);
    }
    // A split with a single chunk (every split of a list of at most 16 G
    // entries, e.g. a 512-entry sliding window) loads and reduces that chunk
    // only.  The rest of the kernel is instantiated once per form, so each
    // form's waits count its own loads.
    auto issue1 = [&](uint32_t pa) {    // chunk 0 alone, into buffer 0 (two-set shapes)
        ok[0] = entry(0) < S;
        const size_t ra = (size_t)(ok[0] ? pa : 0u) * kv_dim + dim0;
#pragma unroll
        for (int f = 0; f < NF; ++f) kr[0][f] = ldr(Kc + ra + 64 * f);
#pragma unroll
        for (int f = 0; f < NF; ++f) vr[0][f] = ldr(Vc + ra + 64 * f);
    };
    auto body = [&](auto single_) {
    constexpr bool SINGLE = decltype(single_)::value;
    if (SINGLE) issue1(sl[0]);
    else if (iters) issue(0, 0, sl[0], sl[1]);

        uint32_t new_slot = 0xFFFFFFFFu;
        if (ROPE) {
            new_slot = ra.step[1];
            // items: GQA query heads (RMSNorm * q_norm), the new K head
            // (* k_norm), the new V head (unit RMSNorm), into LDS
    #pragma unroll
            for (int j = 0; j < NIT; ++j) {
                const int it = wave + 4 * j;
                if (it < GQA + 2) {
                    float ss = 0.0f;
    #pragma unroll
                    for (int d = 0; d < DPL; ++d) ss += raw[j][d] * raw[j][d];
                    ss = wave_sum64(ss);
                    const float inv = 1.0f / sqrtf(ss / (float)D + ra.eps);
                    float *dst = it < GQA ? sh_q[it] : (it == GQA ? sh_k : sh_v);
    #pragma unroll
                    for (int d = 0; d < DPL; ++d) {
                        const float n = raw[j][d] * inv;
                        dst[lane + 64 * d] = it < GQA + 1 ? n * nwt[j][d] : n;
                    }
                }
            }
            __syncthreads();
            for (int it = wave; it < GQA + 1; it += 4)
                wave_rope_lds(it < GQA ? sh_q[it] : sh_k, ra.rot, rcs, lane);
            __syncthreads();
            if (split == 0) {
                float *kd = Kc + (size_t)new_slot * kv_dim + (size_t)kvh * D;
                float *vd = Vc + (size_t)new_slot * kv_dim + (size_t)kvh * D;
                for (int d = threadIdx.x; d < D; d += 256) {
                    kd[d] = sh_k[d];
                    vd[d] = sh_v[d];
                }
            }
            if (!iters) {
                write_empty();
                return;
            }
    #pragma unroll
            for (int h = 0; h < GQA; ++h)
    #pragma unroll
                for (int f = 0; f < NF; ++f) q[h][f] = *(const f4 *)&sh_q[h][c * 4 + 64 * f];
        }

        float M[GQA], L[GQA];
        f4 acc[GQA][NF];
    #pragma unroll
        for (int h = 0; h < GQA; ++h) {
            M[h] = kNegBig;
            L[h] = 0.0f;
    #pragma unroll
            for (int f = 0; f < NF; ++f) acc[h][f] = f4{0, 0, 0, 0};
        }
        // One chunk of buffer b into the running state (fresh: the new token's
        // row, in the rows that held it).  With two sets the rows that do not count (past the
        // slot count, or, with ROPE, the new token's row: its cache row may
        // predate split 0's write, so it is added from LDS after the loop) are
        // masked with bit operations, not selects: given a select the compiler
        // branches around the dot and copies the V rows into a second set of
        // registers at the join, which costs registers the two-set shapes do not have.
        // One set keeps the selects (its rows past the count hold zeros).
        bool has_new = false;
        auto reduce = [&](int b, uint32_t ps, bool fresh = false) {
            bool use = fresh ? has_new : ok[b];
            if constexpr (NSET == 2) {
                if (ROPE && !fresh) {
                    has_new = has_new || (use && ps == new_slot);
                    use = use && ps != new_slot;
                }
            } else if (ROPE && use && ps == new_slot) {
                // one set: the new token's row is replaced in place
    #pragma unroll
                for (int f = 0; f < NF; ++f) {
                    kr[b][f] = *(const f4 *)&sh_k[c * 4 + 64 * f];
                    vr[b][f] = *(const f4 *)&sh_v[c * 4 + 64 * f];
                }
            }
            uint32_t m = 0;
            if constexpr (NSET == 2) {
                m = opaque_mask(use);
    #pragma unroll
                for (int f = 0; f < NF; ++f)
                    vr[b][f] = f4{mask_f(vr[b][f].x, m), mask_f(vr[b][f].y, m), mask_f(vr[b][f].z, m),
                                  mask_f(vr[b][f].w, m)};
            }
    #pragma unroll
            for (int h = 0; h < GQA; ++h) {
                float d = 0.0f;
    #pragma unroll
                for (int f = 0; f < NF; ++f) {
                    d = fmaf(q[h][f].x, kr[b][f].x, d);
                    d = fmaf(q[h][f].y, kr[b][f].y, d);
                    d = fmaf(q[h][f].z, kr[b][f].z, d);
                    d = fmaf(q[h][f].w, kr[b][f].w, d);
                }
                float sc;
                if constexpr (NSET == 2)
                    sc = __builtin_bit_cast(float, (__builtin_bit_cast(uint32_t, row16_sum(d) * scale) & m) |
                                                       (__builtin_bit_cast(uint32_t, kNegBig) & ~m));
                else
                    sc = use ? row16_sum(d) * scale : kNegBig;
                const float mx = rows4_max(sc);
                const float Mn = fmaxf(M[h], mx);
                const float rs = expf(M[h] - Mn);
                const float p = NSET == 2 ? mask_f(expf(sc - Mn), m) : (use ? expf(sc - Mn) : 0.0f);
                const float psum = rows4_sum(p);
    #pragma unroll
                for (int f = 0; f < NF; ++f) acc[h][f] = acc[h][f] * rs + p * vr[b][f];
                L[h] = L[h] * rs + psum;
                M[h] = Mn;
            }
        };
        // Pair pr = chunks 2 pr, 2 pr + 1 goes to set pr % NSET; once reduced,
        // the set takes pair pr + NSET.  One straight-line body per pair count
        // (the count is uniform over the workgroup): no branch between a load
        // and its use, so each wait leaves the younger set in flight.  A chunk
        // past `iters` in the last pair is masked by ok[].
        if constexpr (NSET == 2 && SINGLE) {
            reduce(0, sl[0]);
        } else if constexpr (NSET == 2) {
            auto run = [&](auto np_) {
                constexpr int NP = decltype(np_)::value;
                if constexpr (NP > 1) issue(1, 2, sl[2 % NSL], sl[3 % NSL]);
    #pragma unroll
                for (int pr = 0; pr < NP; ++pr) {
                    const int set = pr % 2;
                    reduce(2 * set, sl[(2 * pr) % NSL]);
                    reduce(2 * set + 1, sl[(2 * pr + 1) % NSL]);
                    if (pr + 2 < NP) issue(set, 2 * (pr + 2), sl[(2 * pr + 4) % NSL], sl[(2 * pr + 5) % NSL]);
                }
            };
            const uint32_t np = (iters + 1) / 2;
            if constexpr (kMaxChunks == 4) {
                if (np <= 1) run(std::integral_constant<int, 1>{});
                else run(std::integral_constant<int, 2>{});
            } else {
                static_assert(kMaxChunks == 8, "one body per pair count");
                switch (np) {
                case 1: run(std::integral_constant<int, 1>{}); break;
                case 2: run(std::integral_constant<int, 2>{}); break;
                case 3: run(std::integral_constant<int, 3>{}); break;
                default: run(std::integral_constant<int, 4>{}); break;
                }
            }
        } else {
            uint32_t pa = sl[0], pb = sl[1];
    #pragma unroll 1
            for (uint32_t t = 0; t < iters; t += 2) {
                if (t > 0) issue(0, t, pa, pb);
                const uint32_t na = slot_at(t + 2), nb = slot_at(t + 3);
                reduce(0, pa);
                if (t + 1 < iters) reduce(1, pb);
                pa = na;
                pb = nb;
            }
        }
        // two sets: the new token's entry, from LDS, in the rows whose list
        // entry it is
        if (ROPE && NSET == 2 && __any(has_new)) {
    #pragma unroll
            for (int f = 0; f < NF; ++f) {
                kr[0][f] = *(const f4 *)&sh_k[c * 4 + 64 * f];
                vr[0][f] = *(const f4 *)&sh_v[c * 4 + 64 * f];
            }
            reduce(0, 0u, true);
        }
        // rows of the wave hold different entries of the same columns
    #pragma unroll
        for (int h = 0; h < GQA; ++h)
    #pragma unroll
            for (int f = 0; f < NF; ++f) {
                const f4 t = f4{rows4_sum(acc[h][f].x), rows4_sum(acc[h][f].y), rows4_sum(acc[h][f].z),
                                rows4_sum(acc[h][f].w)};
                if (r == 0) sh_acc[wave][h][c + 16 * f] = t;
            }
        if (lane < GQA) {
            sh_m[wave][lane] = M[lane];
            sh_l[wave][lane] = L[lane];
        }
        __syncthreads();

        // workgroup partial for this split: [G][nq][D] sums, then [G][nq] maxima
        // and [G][nq] denominators
        float *wacc = ws;
        float *wm = ws + (size_t)G * num_q_heads * D;
        float *wl = wm + (size_t)G * num_q_heads;
        for (int idx = threadIdx.x; idx < GQA * (D / 4); idx += 256) {
            const int h = idx / (D / 4), col = idx % (D / 4);
            float Mw = -1e9f;
    #pragma unroll
            for (int w = 0; w < 4; ++w) Mw = fmaxf(Mw, sh_m[w][h]);
            f4 t = f4{0, 0, 0, 0};
            float lw = 0.0f;
    #pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float e = expf(sh_m[w][h] - Mw);
                t += e * sh_acc[w][h][col];
                lw += e * sh_l[w][h];
            }
            *(f4 *)(wacc + ((size_t)split * num_q_heads + qh0 + h) * D + 4 * col) = t;
            if (col == 0) {
                wm[(size_t)split * num_q_heads + qh0 + h] = Mw;
                wl[(size_t)split * num_q_heads + qh0 + h] = lw;
            }
        }
    };
    if constexpr (NSET == 2) {
        if (iters == 1) body(std::true_type{});
        else body(std::false_type{});
    } else {
        body(std::false_type{});
    }
}

// Running softmax state (max, denominator, sum of p * V) and the merge of
// two states: rescale both to the larger max.
struct SoftState {
    float m, l;
    f4 t;
};
__device__ __forceinline__ SoftState soft_merge(const SoftState &x, const SoftState &y) {
    const float mn = fmaxf(x.m, y.m);
    const float a = expf(x.m - mn), b = expf(y.m - mn);
    return SoftState{mn, x.l * a + y.l * b, x.t * a + y.t * b};
}
template <int M>
__device__ __forceinline__ float xor_lane(float v) {
    return M == 16 ? xor16_lane(v) : xor32_lane(v);
}
template <int M>
__device__ __forceinline__ SoftState xor_state(const SoftState &x) {
    return SoftState{xor_lane<M>(x.m), xor_lane<M>(x.l),
                     f4{xor_lane<M>(x.t.x), xor_lane<M>(x.t.y), xor_lane<M>(x.t.z), xor_lane<M>(x.t.w)}};
}

// Merge of the split partials.  Every split leaves a partial, empty (sum 0)
// when it had no entries, so the merge needs no slot count.  Workgroup
// (column block, query head) owns 64 output values (16 float4 columns);
// thread (j, col), j = tid / 16, merges splits j, j + 16, ... online
// (running max, rescaled sums) with all of its loads issued at once (U per
// batch).  The 16 running states of a column then meet in a fixed tree:
// lanes 16 and 32 apart inside each wave by shuffles, then the four waves
// in LDS.  Writes the output and, for the o_proj matvec, its digit planes.
// S = 0 gives a zero row.
template <int DV, int U>
__global__ __launch_bounds__(256) void k_attn_merge(const float *__restrict__ ws, uint32_t nsplit,
                                                    uint32_t num_q_heads, float *__restrict__ out,
                                                    uint32_t *__restrict__ xp, uint32_t xp_nb,
                                                    const uint32_t *__restrict__ skip) {
    if (skip && *skip) return;          // a quiescent layer (uniform)
    constexpr int D = DV * 256;
    __shared__ f4 st_t[4][16];
    __shared__ float st_m[4][16], st_l[4][16];
    __shared__ float res[64];
    const uint32_t cb = blockIdx.x, qh = blockIdx.y;
    const int j0 = threadIdx.x >> 4, col = threadIdx.x & 15;
    const float *wacc = ws + (size_t)qh * D + cb * 64 + 4 * col;
    const float *wm = ws + (size_t)nsplit * num_q_heads * D + qh;
    const float *wl = wm + (size_t)nsplit * num_q_heads;
    const size_t stride = (size_t)num_q_heads * D;

    float m = kNegBig, l = 0.0f;
    f4 t = f4{0, 0, 0, 0};
    for (uint32_t jb = j0; jb < nsplit; jb += 16 * U) {
        float mj[U], lj[U];
        f4 aj[U];
        // every load unconditional (a split past nsplit reads split jb's
        // state again and is masked below), and each value given an opaque
        // use, so the compiler neither branches around a load nor sinks it
        // into its use: the U partials cost one memory round trip
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t j = jb + 16 * u < nsplit ? jb + 16 * u : jb;
            mj[u] = wm[(size_t)j * num_q_heads];
            lj[u] = wl[(size_t)j * num_q_heads];
            aj[u] = *(const f4 *)(wacc + j * stride);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) __asm__ volatile("" : "+v"(mj[u]), "+v"(lj[u]), "+v"(aj[u]));
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const bool v = jb + 16 * u < nsplit;
            mj[u] = v ? mj[u] : kNegBig;
            lj[u] = v ? lj[u] : 0.0f;
            aj[u] = v ? aj[u] : f4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            // an empty partial's sums were never written: select, not scale
            const f4 av = lj[u] > 0.0f ? aj[u] : f4{0, 0, 0, 0};
            const float mn = fmaxf(m, mj[u]);
            const float a = expf(m - mn), b = expf(mj[u] - mn);
            t = t * a + av * b;
            l = l * a + lj[u] * b;
            m = mn;
        }
    }
    SoftState st{m, l, t};
    st = soft_merge(st, xor_state<16>(st));
    st = soft_merge(st, xor_state<32>(st));
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) < 16) {
        st_t[wave][col] = st.t;
        st_m[wave][col] = st.m;
        st_l[wave][col] = st.l;
    }
    __syncthreads();
    if (threadIdx.x < 16) {
        const int cc = threadIdx.x;
        SoftState w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = SoftState{st_m[i][cc], st_l[i][cc], st_t[i][cc]};
        const SoftState f = soft_merge(soft_merge(w[0], w[1]), soft_merge(w[2], w[3]));
        const f4 T = f.t * (1.0f / (f.l + 1e-9f));
        *(f4 *)(out + (size_t)qh * D + cb * 64 + 4 * cc) = T;
        res[4 * cc + 0] = T.x; res[4 * cc + 1] = T.y; res[4 * cc + 2] = T.z; res[4 * cc + 3] = T.w;
    }
    if (!xp) return;
    __syncthreads();
    if (threadIdx.x < 8) {            // two 32-value blocks, four lanes each
        float o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = res[8 * threadIdx.x + i];
        emit_planes8(o, xp, xp_nb, qh * (D / 32) + cb * 2 + (threadIdx.x >> 2), threadIdx.x & 3, true);
    }
}

// Four consecutive output values at element offset o: fp32 into out, or
// bf16 into outb when it is set (the operand of the next contraction).
typedef __bf16 bf16x2a __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void store_out4(float *out, __bf16 *outb, size_t o, f4 v) {
    if (outb) {
        *(bf16x2a *)(outb + o) = bf16x2a{(__bf16)v.x, (__bf16)v.y};
        *(bf16x2a *)(outb + o + 2) = bf16x2a{(__bf16)v.z, (__bf16)v.w};
    } else {
        *(f4 *)(out + o) = v;
    }
}

// Prefill (shaders/batch_causal_attn.wgsl): one workgroup per (token, KV
// head) walks slots [start, prev + t + 1) of the list in 64-slot chunks with
// an online softmax; start = S - window for window > 0 and S > window.
template <int DV, int GQA>
__global__ __launch_bounds__(256) void k_prefill_attn(const float *__restrict__ Q, const float *__restrict__ Kc,
                                                      const float *__restrict__ Vc,
                                                      const uint32_t *__restrict__ slots, uint32_t num_prev,
                                                      uint32_t num_q_heads, uint32_t kv_dim, float scale,
                                                      uint32_t window, float *__restrict__ out,
                                                      __bf16 *__restrict__ outb) {
    constexpr int D = DV * 256;
    const uint32_t t = blockIdx.x, kvh = blockIdx.y;
    const uint32_t S = num_prev + t + 1;
    const uint32_t start = (window > 0 && S > window) ? S - window : 0;
    __shared__ float sc[GQA][kAttnChunk];
    __shared__ f4 pacc[16][GQA < 2 ? GQA : 2][64 * DV];
    const size_t q_row = (size_t)t * num_q_heads * D;
    f4 q[GQA][4 * DV];
    load_q<DV, GQA>(q, Q + q_row, kvh * GQA);
    AttnState<DV, GQA> st;
#pragma unroll
    for (int h = 0; h < GQA; ++h) {
        st.M[h] = -1e9f;
        st.l[h] = 0.0f;
#pragma unroll
        for (int f = 0; f < 4 * DV; ++f) st.acc[h][f] = f4{0, 0, 0, 0};
    }
    for (uint32_t c0 = start; c0 < S; c0 += kAttnChunk) {
        const uint32_t cnt = (S - c0 < (uint32_t)kAttnChunk) ? S - c0 : kAttnChunk;
        attn_chunk<DV, GQA>(st, q, Kc, Vc, slots, c0, cnt, kv_dim, kvh, scale, sc);
    }
    float inv[GQA];
#pragma unroll
    for (int h = 0; h < GQA; ++h) inv[h] = 1.0f / (st.l[h] + 1e-9f);
    attn_reduce<DV, GQA>(st, pacc, [&](int h, int col, f4 v) {
        const size_t o = q_row + (size_t)(kvh * GQA + h) * D + 4 * col;
        store_out4(out, outb, o, v * inv[h]);
    });
}

// ---------------------------------------------------------------------
// Prefill attention on the matrix cores, head_dim 256.
//
// Same result as k_prefill_attn (an online softmax over each query's causal
// window), computed per workgroup for 64 query rows (64 / GQA tokens x the
// GQA heads of one KV head) against 32-key chunks of the slot list:
//  * scores are formed transposed, S^T = K Q^T, with
//    v_mfma_f32_16x16x32_bf16; each fp32 operand is split into bf16 high
//    and low parts and a product is hi*hi + hi*lo + lo*hi (the dropped lo*lo
//    term is below 2^-16 of it), so the scores keep close to fp32 accuracy;
//  * the C layout of S^T puts keys 4g..4g+3 of each 16-key tile, for query
//    lane & 15, in lane group g = lane >> 4 - exactly the B-operand layout of
//    O^T = V^T P^T once the chunk's keys are permuted (positions 8g .. 8g+7
//    hold keys 4g..4g+3 and 16+4g..16+4g+3), so probabilities stay in
//    registers;
//  * a pre-pass (k_prefill_frags) splits the K and V rows of the keys into
//    bf16 high/low parts once per layer and stores them in the order the
//    MFMA operands are read: per 32-key chunk and KV head, 64 KB = K hi, K
//    lo, V^T hi, V^T lo, each 16 one-KB fragments in which lane l's 16 bytes
//    lie at 16 l.  The attention copies a chunk into LDS by DMA
//    (global_load_lds: no registers, no conversion) while the previous chunk
//    is multiplied, and every fragment read is one contiguous KB, free of
//    bank conflicts.
typedef __bf16 pbf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 pbf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t pu32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t pu32x2 __attribute__((ext_vector_type(2)));

// x -> (bf16 hi, bf16 lo) with hi + lo = x to within 2^-18 |x|, two lanes
// of x per 32-bit word.
struct HiLo {
    uint32_t hi, lo;
};
__device__ __forceinline__ HiLo split_bf16x2(float a, float b) {
    const pbf16x2 h = {(__bf16)a, (__bf16)b};
    const uint32_t hi = __builtin_bit_cast(uint32_t, h);
    const float ra = a - __builtin_bit_cast(float, hi << 16);
    const float rb = b - __builtin_bit_cast(float, hi & 0xffff0000u);
    const pbf16x2 l = {(__bf16)ra, (__bf16)rb};
    return HiLo{hi, __builtin_bit_cast(uint32_t, l)};
}
template <typename V>
__device__ __forceinline__ void put_hilo(V &h, V &l, int i, float a, float b) {
    const HiLo t = split_bf16x2(a, b);
    h[i] = t.hi;
    l[i] = t.lo;
}

constexpr int kPaNK = 32;                 // keys per chunk
constexpr int kPaFrag = 1024;             // one MFMA operand fragment: 64 lanes x 16 B
constexpr int kPaPlane = 16 * kPaFrag;    // one plane of a chunk: 16 fragments
constexpr int kPaChunkBytes = 4 * kPaPlane;   // K hi, K lo, V^T hi, V^T lo

// Plane fragments of a chunk.  K planes, fragment f = 8 tt + j: keys
// 16 tt + (lane & 15), dims 32 j + 8 (lane >> 4) .. +7.  V^T planes,
// fragment dt: dims 16 dt + (lane & 15), chunk positions 8 (lane >> 4) ..
// +7, where position 8 q + i holds key 4 q + i (i < 4) or 16 + 4 q + i - 4
// (the key order of the S^T accumulator layout).
__device__ __forceinline__ int vt_key(int pos) {
    const int q = pos >> 3, i = pos & 7;
    return i < 4 ? 4 * q + i : 16 + 4 * q + i - 4;
}

size_t prefill_frag_bytes(uint32_t num_kv_heads, uint32_t n_keys) {
    return (size_t)num_kv_heads * ((n_keys + kPaNK - 1) / kPaNK) * kPaChunkBytes;
}

// Pre-pass: grid (KV heads, chunks c_lo .. c_lo + gridDim.y - 1, 2): z = 0
// writes the chunk's K planes, z = 1 its V^T planes; chunk c_lo + blockIdx.y
// of KV head kvh = blockIdx.x goes to F + (kvh * nfch + blockIdx.y) *
// kPaChunkBytes (nfch chunks per head, of which the grid may cover the
// first ones only).  Keys at or past n_keys are zero.  The KV head is the
// fastest grid index here and in the attention (workgroup i runs on XCD
// i % 8), so with eight KV heads every workgroup of one head runs on one
// XCD and a head's fragments, read by all of its query tiles, stay in that
// XCD's L2.
__global__ __launch_bounds__(256) void k_prefill_frags(const float *__restrict__ Kc, const float *__restrict__ Vc,
                                                       const uint32_t *__restrict__ slots, uint32_t n_keys,
                                                       uint32_t c_lo, uint32_t nfch, uint32_t kv_dim,
                                                       unsigned char *__restrict__ F) {
    __shared__ f4 rows[kPaNK][64];                         // the chunk's K or V rows, 256 floats each
    const int tid = threadIdx.x;
    const uint32_t c = c_lo + blockIdx.y, kvh = blockIdx.x;
    const bool is_v = blockIdx.z != 0;
    {
        // every load unconditional (a key past n_keys reads the last key's
        // row and stores zeros), so the eight row loads fly together
        const int key = tid >> 3, part = tid & 7;           // 8 threads per row
        const uint32_t kp = c * kPaNK + key;
        const bool ok = kp < n_keys;
        const uint32_t slot = slots[min(kp, n_keys - 1)];
        const f4 *src = (const f4 *)((is_v ? Vc : Kc) + (size_t)slot * kv_dim + (size_t)kvh * 256);
        f4 r[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = src[part + 8 * i];
#pragma unroll
        for (int i = 0; i < 8; ++i) rows[key][part + 8 * i] = ok ? r[i] : f4{0, 0, 0, 0};
    }
    __syncthreads();
    unsigned char *Fc = F + ((size_t)kvh * nfch + blockIdx.y) * kPaChunkBytes + (is_v ? 2 * kPaPlane : 0);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int item = tid + 256 * u, f = item >> 6, l = item & 63;   // fragment f, lane l
        pu32x4 h, lo;
        if (!is_v) {
            const int key = 16 * (f >> 3) + (l & 15), d4 = 8 * (f & 7) + 2 * (l >> 4);
            const f4 x = rows[key][d4], y = rows[key][d4 + 1];
            put_hilo(h, lo, 0, x.x, x.y);
            put_hilo(h, lo, 1, x.z, x.w);
            put_hilo(h, lo, 2, y.x, y.y);
            put_hilo(h, lo, 3, y.z, y.w);
        } else {
            const int dim = 16 * f + (l & 15), g = l >> 4;
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = ((const float *)rows[vt_key(8 * g + i)])[dim];
            put_hilo(h, lo, 0, v[0], v[1]);
            put_hilo(h, lo, 1, v[2], v[3]);
            put_hilo(h, lo, 2, v[4], v[5]);
            put_hilo(h, lo, 3, v[6], v[7]);
        }
        *(pu32x4 *)(Fc + item * 16) = h;
        *(pu32x4 *)(Fc + kPaPlane + item * 16) = lo;
    }
}

// The key chunks [cf, ce) a query tile of TQ tokens walks (from its first
// token's window start to its last token's key) and the number of parts it
// is cut into (maxparts = 1: none).
struct PaGeom {
    uint32_t TQ, n_tok, num_prev, window, maxparts;
};
__host__ __device__ inline void pa_chunks(const PaGeom &g, uint32_t tile, uint32_t &cf, uint32_t &ce) {
    const uint32_t t_first = tile * g.TQ;
    const uint32_t t_last = t_first + g.TQ - 1 < g.n_tok - 1 ? t_first + g.TQ - 1 : g.n_tok - 1;
    const uint32_t S_first = g.num_prev + t_first + 1, S_end = g.num_prev + t_last + 1;
    const uint32_t k_first = (g.window > 0 && S_first > g.window) ? S_first - g.window : 0;
    cf = k_first / kPaNK;
    ce = (S_end + kPaNK - 1) / kPaNK;
}
__host__ __device__ inline uint32_t pa_parts(const PaGeom &g, uint32_t tile) {
    uint32_t cf, ce;
    pa_chunks(g, tile, cf, ce);
    const uint32_t np = (ce - cf + kPaPartChunks - 1) / kPaPartChunks;
    return np < 1 ? 1 : (np > g.maxparts ? g.maxparts : np);
}

// F: the pre-pass output for chunks c_lo .. c_lo + nfch - 1.  Grid (KV
// heads, work items): item `it` of a KV head is part `part` of query tile
// `tile`, the tiles' parts numbered in tile order; every wave finds its
// item's tile with a prefix sum of the tiles' part counts over the lanes.
template <int GQA>
__global__ __launch_bounds__(64 * kPaWaves) void k_prefill_attn_mf(const float *__restrict__ Q,
                                                         const unsigned char *__restrict__ F, uint32_t c_lo,
                                                         uint32_t nfch, uint32_t num_prev, uint32_t n_tok,
                                                         uint32_t num_q_heads, float scale, uint32_t window,
                                                         float *__restrict__ out, __bf16 *__restrict__ outb,
                                                         float *__restrict__ ws, uint32_t maxparts) {
    constexpr int D = 256, NK = kPaNK, TQ = 16 * kPaWaves / GQA;
    __shared__ __attribute__((aligned(16))) unsigned char ring[2][kPaChunkBytes];   // two chunks in flight

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, c = lane & 15;
    const uint32_t kvh = blockIdx.x;
    // the work item's query tile and key part
    const PaGeom geo{(uint32_t)TQ, n_tok, num_prev, window, maxparts};
    const uint32_t ntiles = (n_tok + TQ - 1) / TQ;
    uint32_t tile = 0, part = 0, nparts = 1;
    {
        const uint32_t it = blockIdx.y;
        uint32_t base = 0;
        for (uint32_t t0 = 0; t0 < ntiles; t0 += 64) {
            const uint32_t t = t0 + lane;
            const uint32_t np = t < ntiles ? pa_parts(geo, t) : 0u;
            uint32_t incl = np;                                    // inclusive prefix sum over the lanes
#pragma unroll
            for (int d = 1; d < 64; d *= 2) {
                const uint32_t v = (uint32_t)__shfl_up((int)incl, d, 64);
                incl += lane >= d ? v : 0u;
            }
            const uint32_t total = (uint32_t)__shfl((int)incl, 63, 64);
            if (it < base + total) {
                const uint32_t r = it - base;
                const uint64_t hit = __ballot(r < incl && r >= incl - np);
                const int L = __builtin_ctzll(hit);
                tile = t0 + L;
                nparts = (uint32_t)__shfl((int)np, L, 64);
                part = r - ((uint32_t)__shfl((int)incl, L, 64) - nparts);
                break;
            }
            base += total;
        }
        tile = __builtin_amdgcn_readfirstlane(tile);
        part = __builtin_amdgcn_readfirstlane(part);
        nparts = __builtin_amdgcn_readfirstlane(nparts);
    }
    // this lane's query: column c of the wave's 16 rows
    const int qi = wave * 16 + c;
    const uint32_t tq = tile * TQ + qi / GQA, head = kvh * GQA + qi % GQA;
    const uint32_t tqc = min(tq, n_tok - 1);
    const uint32_t Sq = num_prev + tqc + 1;                        // keys [startq, Sq)
    const uint32_t startq = (window > 0 && Sq > window) ? Sq - window : 0;
    // the tile's 32-key chunks [cf, ce) (from its first token's window start
    // to its last token), cut into nparts parts; the parts' partial states
    // meet in k_prefill_attn_merge
    uint32_t cf, ce;
    pa_chunks(geo, tile, cf, ce);
    const uint32_t per = (ce - cf + nparts - 1) / nparts;
    const uint32_t c_begin = min(ce, cf + part * per), c_stop = min(ce, c_begin + per);

    // chunk cc into ring stage st: wave w copies fragments NFR w .. NFR w + NFR - 1
    const unsigned char *Fk = F + (size_t)kvh * nfch * kPaChunkBytes + lane * 16;
    auto issue = [&](uint32_t cc, int st) {
        const unsigned char *src = Fk + (size_t)(cc - c_lo) * kPaChunkBytes;
        constexpr int NFR = 64 / kPaWaves;                     // fragments per wave
#pragma unroll
        for (int i = 0; i < NFR; ++i) {
            const int fr = wave * NFR + i;
            __builtin_amdgcn_global_load_lds(src + fr * kPaFrag, (lds_t *)(ring[st] + fr * kPaFrag), 16, 0, 0);
        }
    };

    // the first chunk's copy goes out before Q's loads, so the two overlap
    if (c_begin < c_stop) issue(c_begin, 0);

    // Q^T operand: lane holds query c, dims 32 j + 8 g .. +8, as hi / lo bf16
    pbf16x8 qh[8], ql[8];
    {
        const float *qrow = Q + ((size_t)tqc * num_q_heads + head) * D + 8 * g;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const f4 a = *(const f4 *)(qrow + 32 * j), b = *(const f4 *)(qrow + 32 * j + 4);
            pu32x4 h, l;
            put_hilo(h, l, 0, a.x, a.y);
            put_hilo(h, l, 1, a.z, a.w);
            put_hilo(h, l, 2, b.x, b.y);
            put_hilo(h, l, 3, b.z, b.w);
            qh[j] = __builtin_bit_cast(pbf16x8, h);
            ql[j] = __builtin_bit_cast(pbf16x8, l);
        }
    }

    f4 o[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = f4{0, 0, 0, 0};
    float m = -INFINITY, l = 0.0f;

    const uint32_t sm0 = lds_addr(ring[0]) + lane * 16;
    for (uint32_t cc = c_begin; cc < c_stop; ++cc) {
        const int st = (cc - c_begin) & 1;
        wait_vm_lgkm0<0>();                                        // this wave's share of chunk cc landed
        bare_barrier();                                            // ... every wave's; chunk cc-1's reads done
        if (cc + 1 < c_stop) issue(cc + 1, st ^ 1);
        __asm__ volatile("" ::: "memory");
        const uint32_t base = sm0 + st * kPaChunkBytes;
        const uint32_t c0 = cc * NK;

        // S^T tile tt: keys 16 tt + 4 g + i, query c.  Dims slice j's four
        // fragments (K hi / lo of both tiles) load while slice j-1 multiplies.
        f4 sacc[2] = {f4{0, 0, 0, 0}, f4{0, 0, 0, 0}};
        pbf16x8 kf[2][4];
        auto kread = [&](int j, pbf16x8 (&d)[4]) {
            d[0] = lds_read<pbf16x8>(base + (0 * 8 + j) * kPaFrag);
            d[1] = lds_read<pbf16x8>(base + kPaPlane + (0 * 8 + j) * kPaFrag);
            d[2] = lds_read<pbf16x8>(base + (1 * 8 + j) * kPaFrag);
            d[3] = lds_read<pbf16x8>(base + kPaPlane + (1 * 8 + j) * kPaFrag);
        };
        kread(0, kf[0]);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            pbf16x8 (&cur)[4] = kf[j & 1];
            if (j < 7) {
                kread(j + 1, kf[(j + 1) & 1]);
                lds_wait_n<4>();                                   // slice j landed (slice j+1 may fly)
            } else {
                lds_wait();
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) lds_pin(cur[k]);
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                sacc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur[2 * tt], qh[j], sacc[tt], 0, 0, 0);
                sacc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur[2 * tt], ql[j], sacc[tt], 0, 0, 0);
                sacc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur[2 * tt + 1], qh[j], sacc[tt], 0, 0, 0);
            }
        }
        // online softmax for query c over this chunk (lane groups g hold 8 keys each)
        float sv[8];
        float cmax = -INFINITY;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t kp = c0 + 16 * tt + 4 * g + i;
                const bool ok = kp >= startq && kp < Sq;
                const float v = ok ? sacc[tt][i] * scale : -INFINITY;
                sv[4 * tt + i] = v;
                cmax = fmaxf(cmax, v);
            }
        cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
        const float m_new = fmaxf(m, cmax);
        const float alpha = (m_new == -INFINITY) ? 1.0f : __expf(m - m_new);
        float psum = 0.0f, pv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            pv[i] = sv[i] == -INFINITY ? 0.0f : __expf(sv[i] - m_new);
            psum += pv[i];
        }
        psum += __shfl_xor(psum, 16, 64);
        psum += __shfl_xor(psum, 32, 64);
        l = l * alpha + psum;
        m = m_new;
        pu32x4 ph, pl;
#pragma unroll
        for (int i = 0; i < 4; ++i) put_hilo(ph, pl, i, pv[2 * i], pv[2 * i + 1]);
        const pbf16x8 bh = __builtin_bit_cast(pbf16x8, ph), bl = __builtin_bit_cast(pbf16x8, pl);
        // O^T tile dt: dims 16 dt + 4 g + i, query c; tile dt+1's V^T
        // fragments load while tile dt multiplies
        pbf16x8 vf[2][2];
        auto vread = [&](int dt, pbf16x8 (&d)[2]) {
            d[0] = lds_read<pbf16x8>(base + 2 * kPaPlane + dt * kPaFrag);
            d[1] = lds_read<pbf16x8>(base + 3 * kPaPlane + dt * kPaFrag);
        };
        vread(0, vf[0]);
#pragma unroll
        for (int dt = 0; dt < 16; ++dt) {
            pbf16x8 (&cur)[2] = vf[dt & 1];
            if (dt < 15) {
                vread(dt + 1, vf[(dt + 1) & 1]);
                lds_wait_n<2>();
            } else {
                lds_wait();
            }
            lds_pin(cur[0]);
            lds_pin(cur[1]);
            o[dt] *= alpha;
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur[0], bh, o[dt], 0, 0, 0);
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur[0], bl, o[dt], 0, 0, 0);
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(cur[1], bh, o[dt], 0, 0, 0);
        }
    }
    if (tq >= n_tok) return;
    const size_t orow = ((size_t)tq * num_q_heads + head) * D + 4 * g;
    if (nparts > 1) {
        // this part's unnormalised state: sums [part][token][head][D], then
        // (max, denominator) [part][token][head]
        const size_t nrow = (size_t)n_tok * num_q_heads;
#pragma unroll
        for (int dt = 0; dt < 16; ++dt) *(f4 *)(ws + part * nrow * D + orow + 16 * dt) = o[dt];
        if (g == 0) {
            float *ml = ws + maxparts * nrow * D + 2 * (part * nrow + (size_t)tq * num_q_heads + head);
            ml[0] = m;
            ml[1] = l;
        }
        return;
    }
    const float inv = 1.0f / (l + 1e-9f);
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) store_out4(out, outb, orow + 16 * dt, o[dt] * inv);
}

// The key-split parts' states of each (token, head) rescaled to their
// common maximum and normalised; four values per thread.  Rows of tiles
// that were not split were written by the attention itself.
__global__ __launch_bounds__(256) void k_prefill_attn_merge(const float *__restrict__ ws, PaGeom geo,
                                                            uint32_t num_q_heads, size_t nrow, uint32_t D,
                                                            float *__restrict__ out, __bf16 *__restrict__ outb) {
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4;   // element of [token][head][D]
    if (i >= nrow * D) return;
    const size_t row = i / D;
    const uint32_t nparts = pa_parts(geo, (uint32_t)(row / num_q_heads) / geo.TQ);
    if (nparts < 2) return;
    const uint32_t np_stride = geo.maxparts;   // the workspace holds maxparts parts
    const float *ml = ws + np_stride * nrow * D;
    // every part's state is requested at once (parts past nparts reload the
    // last one and are left out below), then combined in part order
    float mp[kPaParts], lp[kPaParts];
    f4 v[kPaParts];
#pragma unroll
    for (uint32_t p = 0; p < kPaParts; ++p) {
        const uint32_t pc = p < nparts ? p : nparts - 1;
        const float2 m2 = *(const float2 *)(ml + 2 * (pc * nrow + row));
        mp[p] = m2.x;
        lp[p] = m2.y;
        v[p] = *(const f4 *)(ws + pc * nrow * D + i);
    }
    // (an opaque use of every loaded value: otherwise the compiler sinks
    // the loads of the later parts into the branches that use them, and
    // each waits on its own round trip)
#pragma unroll
    for (uint32_t p = 0; p < kPaParts; ++p) __asm__ volatile("" : "+v"(mp[p]), "+v"(lp[p]), "+v"(v[p]));
    float mx = -INFINITY;
#pragma unroll
    for (uint32_t p = 0; p < kPaParts; ++p) mx = p < nparts ? fmaxf(mx, mp[p]) : mx;
    f4 t = f4{0, 0, 0, 0};
    float den = 0.0f;
#pragma unroll
    for (uint32_t p = 0; p < kPaParts; ++p) {
        if (p >= nparts) break;
        const float a = mp[p] == -INFINITY ? 0.0f : __expf(mp[p] - mx);
        t += v[p] * a;
        den += lp[p] * a;
    }
    store_out4(out, outb, i, t * (1.0f / (den + 1e-9f)));
}

static int launch_decode_impl(chn_ctx *ctx, const float *q, float *kc, float *vc, const uint32_t *slots,
                              const uint32_t *n_slots, uint32_t max_slots, uint32_t num_q_heads, uint32_t head_dim,
                              uint32_t kv_dim, uint32_t gqa, float scale, float *out, float *ws, uint32_t *xp,
                              const RopeArgs *ra, const uint32_t *skip = nullptr) {
    const uint32_t num_kv = num_q_heads / gqa;
    const uint32_t xp_nb = num_q_heads * head_dim / 32;
    const uint32_t nsplit = dec_splits(max_slots);
    dim3 grid(nsplit, num_kv);
    hipStream_t s = ctx->stream;
    const RopeArgs rz = ra ? *ra : RopeArgs{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 0, 0.0f, 0};
#define CHN_ATTN(DV, G)                                                                                           \
    do {                                                                                                          \
        if (ra)                                                                                                   \
            k_attn_decode<DV, G, true><<<grid, 256, 0, s>>>(q, kc, vc, slots, n_slots, max_slots,        \
                                                                     num_q_heads, kv_dim, scale, ws, rz, skip);   \
        else                                                                                                      \
            k_attn_decode<DV, G, false><<<grid, 256, 0, s>>>(q, kc, vc, slots, n_slots, max_slots,       \
                                                                      num_q_heads, kv_dim, scale, ws, rz, skip);  \
    } while (0)
    if (head_dim == 256) {
        switch (gqa) {
        case 1: CHN_ATTN(1, 1); break;
        case 2: CHN_ATTN(1, 2); break;
        case 4: CHN_ATTN(1, 4); break;
        case 8: CHN_ATTN(1, 8); break;
        default: return set_err(ctx, CHN_E_UNSUPPORTED, "gqa ratio %u unsupported", gqa);
        }
    } else if (head_dim == 512) {
        switch (gqa) {
        case 1: CHN_ATTN(2, 1); break;
        case 2: CHN_ATTN(2, 2); break;
        case 4: CHN_ATTN(2, 4); break;
        default: return set_err(ctx, CHN_E_UNSUPPORTED, "gqa ratio %u unsupported at head_dim 512", gqa);
        }
    } else {
        return set_err(ctx, CHN_E_UNSUPPORTED, "head_dim %u unsupported (256 or 512)", head_dim);
    }
#undef CHN_ATTN
    CHN_LAUNCHED(ctx, "k_attn_decode");
    const dim3 mgrid(head_dim / 64, num_q_heads);
    if (head_dim == 256)
        k_attn_merge<1, kDecGrid / 16><<<mgrid, 256, 0, s>>>(ws, nsplit, num_q_heads, out, xp, xp_nb, skip);
    else
        k_attn_merge<2, kDecGrid / 16><<<mgrid, 256, 0, s>>>(ws, nsplit, num_q_heads, out, xp, xp_nb, skip);
    CHN_LAUNCHED(ctx, "k_attn_merge");
    return CHN_OK;
}

int launch_decode_attn(chn_ctx *ctx, const float *q, const float *kc, const float *vc, const uint32_t *slots,
                       const uint32_t *n_slots, uint32_t max_slots, uint32_t num_q_heads, uint32_t head_dim,
                       uint32_t kv_dim, uint32_t gqa, float scale, float *out, float *ws, uint32_t *xp) {
    return launch_decode_impl(ctx, q, (float *)kc, (float *)vc, slots, n_slots, max_slots, num_q_heads, head_dim,
                              kv_dim, gqa, scale, out, ws, xp, nullptr);
}

int launch_rope_decode_attn(chn_ctx *ctx, const float *q_in, const float *k_in, const float *v_in, const float *qw,
                            const float *kw, float *kc, float *vc, const uint32_t *step, const uint32_t *slots,
                            const uint32_t *n_slots, uint32_t max_slots, uint32_t num_q_heads, uint32_t head_dim,
                            uint32_t kv_dim, uint32_t gqa, uint32_t rot, int k_eq_v, const float2 *rope_tab,
                            float eps, float scale, float *out, float *ws, uint32_t *xp, const uint32_t *skip) {
    if (rot > 2 * kRopePairs || rot > head_dim) return set_err(ctx, CHN_E_UNSUPPORTED, "rotary_dim %u", rot);
    const RopeArgs ra{k_in, v_in, qw, kw, step, rope_tab, rot, eps, k_eq_v};
    return launch_decode_impl(ctx, q_in, kc, vc, slots, n_slots, max_slots, num_q_heads, head_dim, kv_dim, gqa, scale,
                              out, ws, xp, &ra, skip);
}

// The key chunks [c_lo, c_hi) whose operand fragments a prefill's attention
// reads: from the first token's window start to the last key.
static void pa_frag_span(uint32_t n_tok, uint32_t num_prev, uint32_t window, uint32_t &c_lo, uint32_t &c_hi) {
    const uint32_t n_keys = num_prev + n_tok;
    const uint32_t k_lo = (window > 0 && num_prev + 1 > window) ? num_prev + 1 - window : 0;
    c_lo = k_lo / kPaNK;
    c_hi = (n_keys + kPaNK - 1) / kPaNK;
}

bool prefill_frags_fusable(uint32_t num_prev, uint32_t head_dim, uint32_t gqa) {
    return head_dim == 256 && (gqa == 1 || gqa == 2 || gqa == 4 || gqa == 8) && num_prev % kPaNK == 0;
}

int launch_prefill_attn(hipStream_t st, const float *q, const float *kc, const float *vc, const uint32_t *slots,
                        uint32_t n_tok, uint32_t num_prev, uint32_t num_q_heads, uint32_t head_dim, uint32_t kv_dim,
                        uint32_t gqa, float scale, uint32_t window, float *out, __bf16 *outb, float *ws,
                        unsigned char *frag, size_t frag_bytes, bool new_frags_ready) {
    if (head_dim == 256 && (gqa == 1 || gqa == 2 || gqa == 4 || gqa == 8)) {
        // the keys' operand fragments, chunks c_lo .. c_hi - 1; those of the
        // new tokens' chunks may be written already (by the rope kernel)
        const uint32_t num_kv = num_q_heads / gqa, n_keys = num_prev + n_tok;
        uint32_t c_lo, c_hi;
        pa_frag_span(n_tok, num_prev, window, c_lo, c_hi);
        const uint32_t nfch = c_hi - c_lo;
        if (!frag || frag_bytes < (size_t)num_kv * nfch * kPaChunkBytes) return CHN_E_UNSUPPORTED;
        if (new_frags_ready && !prefill_frags_fusable(num_prev, head_dim, gqa)) return CHN_E_UNSUPPORTED;
        const uint32_t c_pre = new_frags_ready ? num_prev / kPaNK : c_hi;   // pre-pass chunks [c_lo, c_pre)
        if (c_pre > c_lo)
            k_prefill_frags<<<dim3(num_kv, c_pre - c_lo, 2), 256, 0, st>>>(kc, vc, slots, n_keys, c_lo, nfch,
                                                                         kv_dim, frag);
        const uint32_t tq = 16 * kPaWaves / gqa;
        const uint32_t tiles = (n_tok + tq - 1) / tq;
        // Causal tiles differ in length (the last one walks every key): each
        // tile's chunks are cut into parts of about kPaPartChunks chunks (at
        // most kPaParts), so the longest walk is about that long and the
        // short tiles run whole (512 tokens: 16 tiles of 1..16 chunks -> 40
        // parts of at most 4 chunks per KV head).
        const PaGeom geo{tq, n_tok, num_prev, window, ws ? kPaParts : 1u};
        uint32_t items = 0, split_tiles = 0;
        for (uint32_t t = 0; t < tiles; ++t) {
            const uint32_t np = pa_parts(geo, t);
            items += np;
            split_tiles += np > 1 ? 1u : 0u;
        }
        const dim3 mgrid(num_q_heads / gqa, items);
#define CHN_PATTN_MF(G)                                                                                  \
    k_prefill_attn_mf<G><<<mgrid, 64 * kPaWaves, 0, st>>>(q, frag, c_lo, nfch, num_prev, n_tok, num_q_heads, scale, \
                                                         window, out, outb, ws, geo.maxparts)
        switch (gqa) {
        case 1: CHN_PATTN_MF(1); break;
        case 2: CHN_PATTN_MF(2); break;
        case 4: CHN_PATTN_MF(4); break;
        default: CHN_PATTN_MF(8); break;
        }
#undef CHN_PATTN_MF
        if (split_tiles) {
            const size_t nrow = (size_t)n_tok * num_q_heads, nq4 = nrow * head_dim / 4;
            k_prefill_attn_merge<<<(unsigned)((nq4 + 255) / 256), 256, 0, st>>>(ws, geo, num_q_heads, nrow, head_dim,
                                                                                  out, outb);
        }
        return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
    }
    dim3 grid(n_tok, num_q_heads / gqa);
#define CHN_PATTN(DV, G) \
    k_prefill_attn<DV, G><<<grid, 256, 0, st>>>(q, kc, vc, slots, num_prev, num_q_heads, kv_dim, scale, window, out, \
                                                outb)
    if (head_dim == 256) {
        switch (gqa) {
        case 1: CHN_PATTN(1, 1); break;
        case 2: CHN_PATTN(1, 2); break;
        case 4: CHN_PATTN(1, 4); break;
        case 8: CHN_PATTN(1, 8); break;
        default: return CHN_E_UNSUPPORTED;
        }
    } else if (head_dim == 512) {
        switch (gqa) {
        case 1: CHN_PATTN(2, 1); break;
        case 2: CHN_PATTN(2, 2); break;
        case 4: CHN_PATTN(2, 4); break;
        default: return CHN_E_UNSUPPORTED;
        }
    } else {
        return CHN_E_UNSUPPORTED;
    }
#undef CHN_PATTN
    return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
}

// ---------------------------------------------------------------------
// qkv_rope: one 64-lane workgroup per head.
// ---------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// RMSNorm * w, then RoPE on pairs (d, d + rot/2) at `clock`, suffix past
// rot copied (shaders/qkv_rope.wgsl:42-91).
__device__ void norm_rope_head(const float *__restrict__ in, const float *__restrict__ w, float *__restrict__ out,
                               uint32_t D, uint32_t rot, float theta, float eps, uint32_t clock, float *buf,
                               const float2 *__restrict__ cs_tab = nullptr) {
    const int lane = threadIdx.x;
    float ss = 0.0f;
    for (uint32_t d = lane; d < D; d += 64) ss += in[d] * in[d];
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)D + eps);
    for (uint32_t d = lane; d < D; d += 64) buf[d] = (in[d] * inv) * w[d];
    __syncthreads();
    const uint32_t half = rot / 2;
    for (uint32_t d = lane; d < half; d += 64) {
        const float v0 = buf[d], v1 = buf[d + half];
        float c, s;
        if (cs_tab) {
            const float2 t = cs_tab[d];
            c = t.x;
            s = t.y;
        } else {
            const float fe = (2.0f * (float)d) / (float)rot;
            const float freq = 1.0f / powf(theta, fe);
            const float ang = (float)clock * freq;
            c = cosf(ang);
            s = sinf(ang);
        }
        out[d] = v0 * c - v1 * s;
        out[d + half] = v0 * s + v1 * c;
    }
    for (uint32_t d = rot + lane; d < D; d += 64) out[d] = buf[d];
}

__global__ __launch_bounds__(64) void k_qkv_rope(const float *__restrict__ q_in, const float *__restrict__ k_in,
                                                 const float *__restrict__ v_in, const float *__restrict__ qw,
                                                 const float *__restrict__ kw, float *__restrict__ q_out,
                                                 float *__restrict__ k_cache, float *__restrict__ v_cache,
                                                 const uint32_t *__restrict__ step, uint32_t num_q,
                                                 uint32_t num_kv, uint32_t D, uint32_t rot, int k_eq_v,
                                                 float theta, float eps) {
    __shared__ float buf[512];
    const uint32_t head = blockIdx.x;
    const uint32_t clock = step[0], slot = step[1];
    if (head < num_q) {
        norm_rope_head(q_in + (size_t)head * D, qw, q_out + (size_t)head * D, D, rot, theta, eps, clock, buf);
        return;
    }
    const uint32_t h = head - num_q;
    if (h >= num_kv) return;
    const size_t kv_dim = (size_t)num_kv * D;
    const float *k = k_in + (size_t)h * D;
    const float *v = k_eq_v ? k : v_in + (size_t)h * D;
    norm_rope_head(k, kw, k_cache + (size_t)slot * kv_dim + (size_t)h * D, D, rot, theta, eps, clock, buf);
    // V: unit RMSNorm (no weight)
    const int lane = threadIdx.x;
    float ss = 0.0f;
    for (uint32_t d = lane; d < D; d += 64) ss += v[d] * v[d];
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)D + eps);
    float *vo = v_cache + (size_t)slot * kv_dim + (size_t)h * D;
    for (uint32_t d = lane; d < D; d += 64) vo[d] = v[d] * inv;
}

// batch_qkv_rope (shaders/batch_qkv_rope.wgsl): token t uses clock
// start_clock + t and writes its K/V at slot slots[slot_offset + t].
__global__ __launch_bounds__(64) void k_batch_qkv_rope(const float *__restrict__ q_in, const float *__restrict__ k_in,
                                                       const float *__restrict__ v_in, const float *__restrict__ qw,
                                                       const float *__restrict__ kw, float *__restrict__ q_out,
                                                       float *__restrict__ k_cache, float *__restrict__ v_cache,
                                                       const uint32_t *__restrict__ slots, uint32_t slot_offset,
                                                       uint32_t start_clock, uint32_t num_q, uint32_t num_kv,
                                                       uint32_t D, uint32_t rot, int k_eq_v, float theta, float eps,
                                                       const float2 *__restrict__ tab) {
    __shared__ float buf[512];
    const uint32_t head = blockIdx.x, t = blockIdx.y;
    const uint32_t clock = start_clock + t, slot = slots[slot_offset + t];
    const size_t q_dim = (size_t)num_q * D, kv_dim = (size_t)num_kv * D;
    const float2 *cs = tab ? tab + (size_t)t * (rot / 2) : nullptr;
    if (head < num_q) {
        norm_rope_head(q_in + t * q_dim + (size_t)head * D, qw, q_out + t * q_dim + (size_t)head * D, D, rot, theta,
                       eps, clock, buf, cs);
        return;
    }
    const uint32_t h = head - num_q;
    if (h >= num_kv) return;
    const float *k = k_in + t * kv_dim + (size_t)h * D;
    const float *v = k_eq_v ? k : v_in + t * kv_dim + (size_t)h * D;
    norm_rope_head(k, kw, k_cache + (size_t)slot * kv_dim + (size_t)h * D, D, rot, theta, eps, clock, buf, cs);
    const int lane = threadIdx.x;
    float ss = 0.0f;
    for (uint32_t d = lane; d < D; d += 64) ss += v[d] * v[d];
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)D + eps);
    float *vo = v_cache + (size_t)slot * kv_dim + (size_t)h * D;
    for (uint32_t d = lane; d < D; d += 64) vo[d] = v[d] * inv;
}

int launch_qkv_rope(hipStream_t st, const float *q_in, const float *k_in, const float *v_in, const float *qw,
                    const float *kw, float *q_out, float *kc, float *vc, const uint32_t *step, uint32_t num_q,
                    uint32_t num_kv, uint32_t D, uint32_t rot, int k_eq_v, float theta, float eps) {
    k_qkv_rope<<<num_q + num_kv, 64, 0, st>>>(q_in, k_in, v_in, qw, kw, q_out, kc, vc, step, num_q, num_kv, D, rot,
                                              k_eq_v, theta, eps);
    return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
}

// The same with four heads per workgroup, one per wave, for D a multiple of
// 256 and the angle table given: lane l holds dims 4 l + 256 j .. +3 (one
// 16-byte access each), the norm reduces across the wave, and each wave
// pairs (d, d + rot/2) through its own LDS row (a wave reads only what it
// wrote, so no workgroup barrier is needed).
template <int DV>
struct RopeRow {   // this lane's inputs of one head row: values, norm weights, angles
    f4 v[DV], wv[DV];
    float2 t[DV][4];
};
template <int DV>
__device__ __forceinline__ void rope_row_load(const float *__restrict__ in, const float *__restrict__ w,
                                              const float2 *__restrict__ cs, uint32_t rot, int lane, RopeRow<DV> &r) {
    const uint32_t half = rot / 2;
#pragma unroll
    for (int j = 0; j < DV; ++j) {
        r.v[j] = *(const f4 *)(in + 4 * lane + 256 * j);
        r.wv[j] = *(const f4 *)(w + 4 * lane + 256 * j);
    }
    // the angles too, with the inputs (after the LDS step of rope_row_math
    // the compiler may not move loads up past its memory clobber)
#pragma unroll
    for (int j = 0; j < DV; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t d = 4 * lane + 256 * j + e;
            const uint32_t p = d < half ? d : d - half;
            r.t[j][e] = cs[d < rot ? p : 0u];
        }
}
// RMSNorm (weights wv) and rotation of the row; o gets this lane's values.
template <int DV>
__device__ __forceinline__ void rope_row_math(const RopeRow<DV> &r, uint32_t rot, float eps, float *buf, int lane,
                                              f4 (&o)[DV]) {
    constexpr int D = 256 * DV;
    const uint32_t half = rot / 2;
    f4 v[DV];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < DV; ++j)
        ss += (r.v[j].x * r.v[j].x + r.v[j].y * r.v[j].y) + (r.v[j].z * r.v[j].z + r.v[j].w * r.v[j].w);
    ss = wave_sum64(ss);
    const float inv = 1.0f / sqrtf(ss / (float)D + eps);
#pragma unroll
    for (int j = 0; j < DV; ++j) {
        v[j] = (r.v[j] * inv) * r.wv[j];
        *(f4 *)(buf + 4 * lane + 256 * j) = v[j];
    }
    __builtin_amdgcn_wave_barrier();
    __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int j = 0; j < DV; ++j) {
        o[j] = v[j];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // branch-free (a branch would let the compiler sink the angle
            // load into it): past rot the pair indices stay inside the row
            // and the unrotated value is kept
            const uint32_t d = 4 * lane + 256 * j + e;
            const uint32_t p = d < half ? d : d - half;              // the pair's index
            const float v0 = buf[p], v1 = buf[p + half];
            const float rr = d < half ? v0 * r.t[j][e].x - v1 * r.t[j][e].y : v0 * r.t[j][e].y + v1 * r.t[j][e].x;
            o[j][e] = d < rot ? rr : o[j][e];
        }
    }
}
template <int DV>
__device__ __forceinline__ void norm_rope_head4(const float *__restrict__ in, const float *__restrict__ w,
                                                float *__restrict__ out, uint32_t rot, float eps, float *buf,
                                                const float2 *__restrict__ cs, int lane) {
    RopeRow<DV> r;
    rope_row_load<DV>(in, w, cs, rot, lane, r);
    f4 o[DV];
    rope_row_math<DV>(r, rot, eps, buf, lane, o);
#pragma unroll
    for (int j = 0; j < DV; ++j) *(f4 *)(out + 4 * lane + 256 * j) = o[j];
}

template <int DV>
__global__ __launch_bounds__(256) void k_batch_qkv_rope4(const float *__restrict__ q_in, const float *__restrict__ k_in,
                                                        const float *__restrict__ v_in, const float *__restrict__ qw,
                                                        const float *__restrict__ kw, float *__restrict__ q_out,
                                                        float *__restrict__ k_cache, float *__restrict__ v_cache,
                                                        const uint32_t *__restrict__ slots, uint32_t slot_offset,
                                                        uint32_t num_q, uint32_t num_kv, uint32_t rot, int k_eq_v,
                                                        float eps, const float2 *__restrict__ tab) {
    constexpr int D = 256 * DV;
    __shared__ __attribute__((aligned(16))) float buf[4][D];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t head = blockIdx.x * 4 + wave, t = blockIdx.y;
    if (head >= num_q + num_kv) return;                     // whole waves; no workgroup barrier follows
    const uint32_t slot = slots[slot_offset + t];
    const size_t q_dim = (size_t)num_q * D, kv_dim = (size_t)num_kv * D;
    const float2 *cs = tab + (size_t)t * (rot / 2);
    if (head < num_q) {
        norm_rope_head4<DV>(q_in + t * q_dim + (size_t)head * D, qw, q_out + t * q_dim + (size_t)head * D, rot, eps,
                            buf[wave], cs, lane);
        return;
    }
    const uint32_t h = head - num_q;
    const float *k = k_in + t * kv_dim + (size_t)h * D;
    const float *v = k_eq_v ? k : v_in + t * kv_dim + (size_t)h * D;
    // V's row is requested before K's norm and rotation run
    f4 vv[DV];
#pragma unroll
    for (int j = 0; j < DV; ++j) vv[j] = *(const f4 *)(v + 4 * lane + 256 * j);
    norm_rope_head4<DV>(k, kw, k_cache + (size_t)slot * kv_dim + (size_t)h * D, rot, eps, buf[wave], cs, lane);
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < DV; ++j)
        ss += (vv[j].x * vv[j].x + vv[j].y * vv[j].y) + (vv[j].z * vv[j].z + vv[j].w * vv[j].w);
    ss = wave_sum64(ss);
    const float inv = 1.0f / sqrtf(ss / (float)D + eps);
    float *vo = v_cache + (size_t)slot * kv_dim + (size_t)h * D;
#pragma unroll
    for (int j = 0; j < DV; ++j) *(f4 *)(vo + 4 * lane + 256 * j) = vv[j] * inv;
}

// k_batch_qkv_rope4<1> that also writes the new keys' attention operand
// fragments (the layout of k_prefill_frags), so that no pre-pass reads the
// new K/V rows back.  The new tokens' keys start a chunk (num_prev is a
// multiple of 32): chunk c0 + cc holds tokens 32 cc .. 32 cc + 31, keys
// past n_tok are zero.  Grid: nkw = 5 * num_kv * (new chunks) workgroups,
// one per (KV head, new chunk, part) with the KV head fastest, first (each
// is a longer chain than a query workgroup, so they start first), then
// n_tok * ceil(num_q / 4) workgroups of four query heads as
// k_batch_qkv_rope4.  Parts 0..3 are the K rows of the chunk's four 8-key
// quarters (two keys per wave), part 4 its V rows (eight per wave).
//  * K: RMSNorm + RoPE of each key's row; the even lane 2 m of the row,
//    given its odd neighbour's four values, holds dims 8 m .. 8 m + 7 - one
//    16-byte item of a K fragment - and stores its bf16 high and low parts;
//  * V: unit RMSNorm of each row; wave w takes the keys of V^T positions
//    8 w .. 8 w + 7, so each lane holds four V^T fragment items whole.
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8))) void k_batch_qkv_rope_frags(
    const float *__restrict__ q_in, const float *__restrict__ k_in, const float *__restrict__ v_in,
    const float *__restrict__ qw, const float *__restrict__ kw, float *__restrict__ q_out,
    float *__restrict__ k_cache, float *__restrict__ v_cache, const uint32_t *__restrict__ slots,
    uint32_t slot_offset, uint32_t n_tok, uint32_t num_q, uint32_t num_kv, uint32_t rot, int k_eq_v, float eps,
    const float2 *__restrict__ tab, unsigned char *__restrict__ F, uint32_t c0, uint32_t c_lo, uint32_t nfch,
    uint32_t nkw) {
    constexpr int D = 256;
    __shared__ __attribute__((aligned(16))) float buf[4][D];  // per-wave rotation rows (query and K paths)
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const size_t q_dim = (size_t)num_q * D, kv_dim = (size_t)num_kv * D;
    if (blockIdx.x >= nkw) {
        const uint32_t qb = (num_q + 3) / 4, wq = blockIdx.x - nkw;
        const uint32_t t = wq / qb, head = (wq % qb) * 4 + wave;
        if (head >= num_q) return;                          // whole waves; no workgroup barrier follows
        norm_rope_head4<1>(q_in + t * q_dim + (size_t)head * D, qw, q_out + t * q_dim + (size_t)head * D, rot,
                           eps, buf[wave], tab + (size_t)t * (rot / 2), lane);
        return;
    }
    const uint32_t j = blockIdx.x;
    const uint32_t h = j % num_kv, r = j / num_kv, cc = r / 5, part = r % 5;
    const bool is_v = part == 4;                             // uniform over the workgroup
    unsigned char *Fc = F + ((size_t)h * nfch + (c0 + cc - c_lo)) * kPaChunkBytes + (is_v ? 2 * kPaPlane : 0);
    // K: keys 8 part + 2 w, + 1 of the chunk in wave w (two keys: the query
    // workgroups share this kernel's register budget, and their occupancy
    // matters more); key k of this wave: its token (clamped into the
    // prompt) and whether it exists
    const uint32_t t0 = cc * kPaNK + 8 * part + 2 * wave;
    auto tok = [&](int k) { return t0 + k < n_tok ? t0 + k : n_tok - 1; };
    auto has = [&](int k) { return t0 + k < n_tok; };
    if (!is_v) {
        RopeRow<1> in[2];
#pragma unroll
        for (int k = 0; k < 2; ++k)
            rope_row_load<1>(k_in + tok(k) * kv_dim + (size_t)h * D, kw, tab + (size_t)tok(k) * (rot / 2), rot, lane,
                             in[k]);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            f4 o[1];
            rope_row_math<1>(in[k], rot, eps, buf[wave], lane, o);
            if (has(k)) {
                const uint32_t slot = slots[slot_offset + tok(k)];
                *(f4 *)(k_cache + (size_t)slot * kv_dim + (size_t)h * D + 4 * lane) = o[0];
            }
            // dims 8 m .. 8 m + 7 at the even lane 2 m
            const f4 x = has(k) ? o[0] : f4{0.0f, 0.0f, 0.0f, 0.0f};
            const f4 y = {__shfl_xor(x.x, 1, 64), __shfl_xor(x.y, 1, 64), __shfl_xor(x.z, 1, 64),
                          __shfl_xor(x.w, 1, 64)};
            if ((lane & 1) == 0) {
                const int key = 8 * part + 2 * wave + k, m = lane >> 1;
                const int f = 8 * (key >> 4) + (m >> 2), l = (key & 15) + 16 * (m & 3);
                pu32x4 hi, lo;
                put_hilo(hi, lo, 0, x.x, x.y);
                put_hilo(hi, lo, 1, x.z, x.w);
                put_hilo(hi, lo, 2, y.x, y.y);
                put_hilo(hi, lo, 3, y.z, y.w);
                *(pu32x4 *)(Fc + (f * 64 + l) * 16) = hi;
                *(pu32x4 *)(Fc + kPaPlane + (f * 64 + l) * 16) = lo;
            }
        }
        return;
    }
    // V: wave w takes the eight keys of chunk positions 8 w .. 8 w + 7 (the
    // key order of a V^T fragment item), so lane c, which holds dims
    // 4 c .. 4 c + 3 of every row, holds the four items of those dims whole
    const float *vsrc = (k_eq_v ? k_in : v_in) + (size_t)h * D + 4 * lane;
    const uint32_t tv0 = cc * kPaNK;
    auto vtok = [&](int i) {
        const uint32_t t = tv0 + vt_key(8 * wave + i);
        return t < n_tok ? t : n_tok - 1;
    };
    auto vhas = [&](int i) { return tv0 + vt_key(8 * wave + i) < n_tok; };
    f4 vn[8];   // the eight rows, normalised in place
#pragma unroll
    for (int i = 0; i < 8; ++i) vn[i] = *(const f4 *)(vsrc + vtok(i) * kv_dim);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float ss = (vn[i].x * vn[i].x + vn[i].y * vn[i].y) + (vn[i].z * vn[i].z + vn[i].w * vn[i].w);
        ss = wave_sum64(ss);
        const float inv = 1.0f / sqrtf(ss / (float)D + eps);
        vn[i] = vn[i] * inv;
        if (vhas(i)) {
            const uint32_t slot = slots[slot_offset + vtok(i)];
            *(f4 *)(v_cache + (size_t)slot * kv_dim + (size_t)h * D + 4 * lane) = vn[i];
        }
        vn[i] = vhas(i) ? vn[i] : f4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    // item (dt, l) of the V^T planes: dims 16 dt + (l & 15), positions 8 (l >> 4) .. + 7
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int d = 4 * lane + e, gi = (d >> 4) * 64 + (d & 15) + 16 * wave;
        pu32x4 hi, lo;
        put_hilo(hi, lo, 0, vn[0][e], vn[1][e]);
        put_hilo(hi, lo, 1, vn[2][e], vn[3][e]);
        put_hilo(hi, lo, 2, vn[4][e], vn[5][e]);
        put_hilo(hi, lo, 3, vn[6][e], vn[7][e]);
        *(pu32x4 *)(Fc + gi * 16) = hi;
        *(pu32x4 *)(Fc + kPaPlane + gi * 16) = lo;
    }
}

int launch_batch_qkv_rope(hipStream_t st, const float *q_in, const float *k_in, const float *v_in, const float *qw,
                          const float *kw, float *q_out, float *kc, float *vc, const uint32_t *slots,
                          uint32_t slot_offset, uint32_t start_clock, uint32_t n_tok, uint32_t num_q, uint32_t num_kv,
                          uint32_t D, uint32_t rot, int k_eq_v, float theta, float eps, const float2 *tab,
                          unsigned char *frag, size_t frag_bytes, uint32_t window) {
    if (frag) {
        // with the new keys' attention fragments (slot_offset = the number
        // of previous keys)
        const uint32_t num_prev = slot_offset;
        if (!tab || D != 256 || num_prev % kPaNK || !num_kv || num_q % num_kv) return CHN_E_UNSUPPORTED;
        uint32_t c_lo, c_hi;
        pa_frag_span(n_tok, num_prev, window, c_lo, c_hi);
        const uint32_t nfch = c_hi - c_lo, c0 = num_prev / kPaNK, nnew = c_hi - c0;
        if (frag_bytes < (size_t)num_kv * nfch * kPaChunkBytes) return CHN_E_UNSUPPORTED;
        const uint32_t nqw = n_tok * ((num_q + 3) / 4), nkw = 5 * num_kv * nnew;
        k_batch_qkv_rope_frags<<<nkw + nqw, 256, 0, st>>>(q_in, k_in, v_in, qw, kw, q_out, kc, vc, slots,
                                                         slot_offset, n_tok, num_q, num_kv, rot, k_eq_v, eps, tab,
                                                         frag, c0, c_lo, nfch, nkw);
        return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
    }
    if (tab && (D == 256 || D == 512)) {
        dim3 grid4((num_q + num_kv + 3) / 4, n_tok);
        if (D == 256)
            k_batch_qkv_rope4<1><<<grid4, 256, 0, st>>>(q_in, k_in, v_in, qw, kw, q_out, kc, vc, slots, slot_offset,
                                                        num_q, num_kv, rot, k_eq_v, eps, tab);
        else
            k_batch_qkv_rope4<2><<<grid4, 256, 0, st>>>(q_in, k_in, v_in, qw, kw, q_out, kc, vc, slots, slot_offset,
                                                        num_q, num_kv, rot, k_eq_v, eps, tab);
        return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
    }
    dim3 grid(num_q + num_kv, n_tok);
    k_batch_qkv_rope<<<grid, 64, 0, st>>>(q_in, k_in, v_in, qw, kw, q_out, kc, vc, slots, slot_offset, start_clock,
                                          num_q, num_kv, D, rot, k_eq_v, theta, eps, tab);
    return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
}

// (cos, sin) of (start_clock + t) * theta^(-2d / rot) for t < n_tok, d <
// rot / 2, at tab[t * rot / 2 + d]: the same expressions the batched
// rotation evaluates per element, once per prompt instead of per layer.
__global__ __launch_bounds__(256) void k_rope_tab_batch(float2 *__restrict__ tab, uint32_t start_clock,
                                                        uint32_t n_tok, uint32_t rot, float theta) {
    const uint32_t half = rot / 2;
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)n_tok * half) return;
    const uint32_t t = (uint32_t)(i / half), d = (uint32_t)(i % half);
    const float fe = (2.0f * (float)d) / (float)rot;
    const float freq = 1.0f / powf(theta, fe);
    const float ang = (float)(start_clock + t) * freq;
    tab[i] = float2{cosf(ang), sinf(ang)};
}

int launch_rope_tab_batch(hipStream_t st, float2 *tab, uint32_t start_clock, uint32_t n_tok, uint32_t rot,
                          float theta) {
    const size_t n = (size_t)n_tok * (rot / 2);
    if (!n) return CHN_OK;
    k_rope_tab_batch<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(tab, start_clock, n_tok, rot, theta);
    return hipGetLastError() == hipSuccess ? CHN_OK : CHN_E_HIP;
}

// ---- decode attention without allocation (chn_decode_attn_noalloc)
// The split partials live in a file-scope device array instead of the
// context workspace.  Each device holds its own copy until the process ends;
// host code never passes the array's name to a kernel, only the address
// hipGetSymbolAddress returns for the current device, taken once per device
// when a context is created on it (noalloc_scratch_init, from chn_init).
constexpr size_t kNoAllocBytes = (size_t)2 << 20;    // 2 MiB: num_q_heads * (head_dim + 2) <= 16384 at 32 splits
static __device__ __align__(256) float scratch[kNoAllocBytes / 4];
constexpr int kMaxDevices = 64;
static void *g_scratch[kMaxDevices];
static std::mutex g_scratch_mu;

int noalloc_scratch_init(chn_ctx *ctx) {
    if (ctx->device < 0 || ctx->device >= kMaxDevices) return CHN_OK;   // the entry point then refuses
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch[ctx->device]) return CHN_OK;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(ctx, e, "hipGetSymbolAddress(scratch)");
    if (!p) return set_err(ctx, CHN_E_HIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch[ctx->device] = p;
    return CHN_OK;
}

}  // namespace chn

using namespace chn;

static int check_decode_attn(chn_ctx *ctx, const float *q, const float *k_cache, const float *v_cache,
                             const uint32_t *slots, const uint32_t *n_slots, uint32_t max_slots,
                             uint32_t num_q_heads, uint32_t head_dim, uint32_t kv_dim, uint32_t gqa_ratio,
                             const float *out) {
    CHN_REQUIRE(ctx, q && k_cache && v_cache && slots && n_slots && out, "NULL argument");
    CHN_REQUIRE(ctx, gqa_ratio > 0 && num_q_heads % gqa_ratio == 0, "num_q_heads %u not a multiple of gqa %u",
                num_q_heads, gqa_ratio);
    CHN_REQUIRE(ctx, kv_dim >= (num_q_heads / gqa_ratio) * head_dim && kv_dim % 4 == 0,
                "kv_dim %u too small for %u kv heads of %u", kv_dim, num_q_heads / gqa_ratio, head_dim);
    CHN_REQUIRE(ctx, aligned(q, 16) && aligned(k_cache, 16) && aligned(v_cache, 16) && aligned(out, 16),
                "q, caches and out must be 16-byte aligned");
    CHN_REQUIRE(ctx, max_slots > 0 && max_slots <= 4096, "max_slots %u must be in 1..4096", max_slots);
    return CHN_OK;
}

extern "C" int chn_qkv_rope(chn_ctx *ctx, const float *q_in, const float *k_in, const float *v_in,
                            const float *q_norm_w, const float *k_norm_w, float *q_out, float *k_cache,
                            float *v_cache, const uint32_t *step_params, uint32_t num_q_heads,
                            uint32_t num_kv_heads, uint32_t head_dim, uint32_t rotary_dim, int k_eq_v,
                            float theta, float eps) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, q_in && k_in && (v_in || k_eq_v) && q_norm_w && k_norm_w && q_out && k_cache && v_cache &&
                    step_params, "NULL argument");
    CHN_REQUIRE(ctx, head_dim > 0 && head_dim <= 512, "head_dim %u must be in 1..512", head_dim);
    CHN_REQUIRE(ctx, rotary_dim <= head_dim && rotary_dim % 2 == 0, "rotary_dim %u must be even and <= head_dim",
                rotary_dim);
    const uint32_t nh = num_q_heads + num_kv_heads;
    if (!nh) return CHN_OK;
    launch_qkv_rope(ctx->stream, q_in, k_in, v_in, q_norm_w, k_norm_w, q_out, k_cache, v_cache, step_params,
                    num_q_heads, num_kv_heads, head_dim, rotary_dim, k_eq_v, theta, eps);
    CHN_LAUNCHED(ctx, "k_qkv_rope");
    return CHN_OK;
}

extern "C" int chn_decode_attn(chn_ctx *ctx, const float *q, const float *k_cache, const float *v_cache,
                               const uint32_t *slots, const uint32_t *n_slots, uint32_t max_slots,
                               uint32_t num_q_heads, uint32_t head_dim, uint32_t kv_dim, uint32_t gqa_ratio,
                               float scale, float *out) {
    if (!ctx) return CHN_E_INVALID;
    int rc = check_decode_attn(ctx, q, k_cache, v_cache, slots, n_slots, max_slots, num_q_heads, head_dim, kv_dim,
                               gqa_ratio, out);
    if (rc) return rc;
    if (!num_q_heads) return CHN_OK;
    rc = ensure_workspace(ctx, attn_ws_bytes(num_q_heads, head_dim, max_slots));
    if (rc) return rc;
    return launch_decode_attn(ctx, q, k_cache, v_cache, slots, n_slots, max_slots, num_q_heads, head_dim,
                              kv_dim, gqa_ratio, scale, out, (float *)ctx->ws, nullptr);
}

// chn_decode_attn with the partials in the device's file-scope scratch: no
// allocation, so it may run where hipMalloc may not (graph capture, serving
// loops).  Every call on one device shares the array; calls that overlap on
// one device race.  Every split writes its whole partial before the merge
// reads it (splits without list entries write an empty one), so nothing
// needs clearing between calls.
extern "C" int chn_decode_attn_noalloc(chn_ctx *ctx, const float *q, const float *k_cache, const float *v_cache,
                                       const uint32_t *slots, const uint32_t *n_slots, uint32_t max_slots,
                                       uint32_t num_q_heads, uint32_t head_dim, uint32_t kv_dim, uint32_t gqa_ratio,
                                       float scale, float *out) {
    if (!ctx) return CHN_E_INVALID;
    int rc = check_decode_attn(ctx, q, k_cache, v_cache, slots, n_slots, max_slots, num_q_heads, head_dim, kv_dim,
                               gqa_ratio, out);
    if (rc) return rc;
    if (!num_q_heads) return CHN_OK;
    const size_t need = attn_ws_bytes(num_q_heads, head_dim, max_slots);
    if (need > kNoAllocBytes)
        return set_err(ctx, CHN_E_UNSUPPORTED, "decode attention partials need %zu bytes; the allocation-free "
                       "scratch holds %zu", need, kNoAllocBytes);
    void *ws = ctx->device >= 0 && ctx->device < kMaxDevices ? g_scratch[ctx->device] : nullptr;
    if (!ws) return set_err(ctx, CHN_E_UNSUPPORTED, "no scratch address for device %d", ctx->device);
    return launch_decode_attn(ctx, q, k_cache, v_cache, slots, n_slots, max_slots, num_q_heads, head_dim,
                              kv_dim, gqa_ratio, scale, out, (float *)ws, nullptr);
}

extern "C" int chn_batch_qkv_rope(chn_ctx *ctx, const float *q_in, const float *k_in, const float *v_in,
                                  const float *q_norm_w, const float *k_norm_w, float *q_out, float *k_cache,
                                  float *v_cache, const uint32_t *slots, uint32_t slot_offset, uint32_t start_clock,
                                  uint32_t n_tok, uint32_t num_q_heads, uint32_t num_kv_heads, uint32_t head_dim,
                                  uint32_t rotary_dim, int k_eq_v, float theta, float eps) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, q_in && k_in && (v_in || k_eq_v) && q_norm_w && k_norm_w && q_out && k_cache && v_cache && slots,
                "NULL argument");
    CHN_REQUIRE(ctx, head_dim > 0 && head_dim <= 512, "head_dim %u must be in 1..512", head_dim);
    CHN_REQUIRE(ctx, rotary_dim <= head_dim && rotary_dim % 2 == 0, "rotary_dim %u must be even and <= head_dim",
                rotary_dim);
    if (!n_tok || !(num_q_heads + num_kv_heads)) return CHN_OK;
    launch_batch_qkv_rope(ctx->stream, q_in, k_in, v_in, q_norm_w, k_norm_w, q_out, k_cache, v_cache, slots,
                          slot_offset, start_clock, n_tok, num_q_heads, num_kv_heads, head_dim, rotary_dim, k_eq_v,
                          theta, eps);
    CHN_LAUNCHED(ctx, "k_batch_qkv_rope");
    return CHN_OK;
}

extern "C" int chn_batch_causal_attn(chn_ctx *ctx, const float *q, const float *k_cache, const float *v_cache,
                                     const uint32_t *slots, uint32_t n_tok, uint32_t num_prev_slots,
                                     uint32_t num_q_heads, uint32_t head_dim, uint32_t kv_dim, uint32_t gqa_ratio,
                                     float scale, uint32_t window, float *out) {
    if (!ctx) return CHN_E_INVALID;
    CHN_REQUIRE(ctx, q && k_cache && v_cache && slots && out, "NULL argument");
    CHN_REQUIRE(ctx, gqa_ratio > 0 && num_q_heads % gqa_ratio == 0, "num_q_heads %u not a multiple of gqa %u",
                num_q_heads, gqa_ratio);
    CHN_REQUIRE(ctx, kv_dim >= (num_q_heads / gqa_ratio) * head_dim && kv_dim % 4 == 0, "kv_dim %u too small", kv_dim);
    CHN_REQUIRE(ctx, aligned(q, 16) && aligned(k_cache, 16) && aligned(v_cache, 16) && aligned(out, 16),
                "q, caches and out must be 16-byte aligned");
    if (!n_tok || !num_q_heads) return CHN_OK;
    const size_t pws = prefill_attn_ws_bytes(n_tok, num_q_heads, head_dim);
    const size_t fb = prefill_frag_bytes(num_q_heads / gqa_ratio, num_prev_slots + n_tok);
    int rc = ensure_workspace(ctx, pws + fb);
    if (rc) return rc;
    rc = launch_prefill_attn(ctx->stream, q, k_cache, v_cache, slots, n_tok, num_prev_slots, num_q_heads, head_dim,
                             kv_dim, gqa_ratio, scale, window, out, nullptr, (float *)ctx->ws,
                             (unsigned char *)ctx->ws + pws, fb);
    if (rc == CHN_E_UNSUPPORTED)
        return set_err(ctx, rc, "head_dim %u / gqa %u unsupported", head_dim, gqa_ratio);
    CHN_LAUNCHED(ctx, "k_prefill_attn");
    return CHN_OK;
}
