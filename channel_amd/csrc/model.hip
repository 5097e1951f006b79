// Model-level host layer: the MI355X counterpart of GpuModelContext
// (src/gpu/model_gpu.zig:30-216), the decode graph (src/gpu/model_dispatch.zig:
// 10-153) and the batched prefill (src/gpu/batch_dispatch.zig:27-172).
//
// * Weights live in HBM as Q4 (attention and MLP matrices) and Q8 (tied
//   embedding for the logits); norms as fp32.  They are quantized on the
//   device from bf16 with bit-exact restatements of quantizeRowQ4_0 /
//   quantizeRowQ8_0, or generated in place for synthetic models.
// * One decode token is recorded once as a HIP graph (the counterpart of the
//   pre-recorded Vulkan command buffers) and replayed per token; the
//   per-token inputs (x, slot lists, {clock, slot_idx, S_global,
//   S_sliding}) are copied into fixed device buffers before each replay and
//   read by the kernels from device memory.
// * Prefill runs layer by layer on the stream, synchronizing every four
//   layers and calling the progress callback, as the reference does.
#include "chn_internal.h"

#include <cmath>
#include <cstring>
#include <vector>

struct chn_model {
    chn_ctx *ctx = nullptr;
    chn_model_config cfg{};
    struct Layer {
        uint32_t *Wq, *Wk, *Wv, *Wo, *Wg, *Wu, *Wd;
        float *in_norm, *q_norm, *k_norm, *post_attn, *pre_ffn, *post_ffn;
        float scalar;
        bool has_post_attn, has_post_ffn, full;
        float *kc, *vc;
        // head shape of this layer (full-attention layers may use the
        // global head_dim / KV head count, src/model/loader.zig:37-41)
        uint32_t D, nkv, qd, kvd, rot, gqa;
    };
    std::vector<Layer> L;
    uint32_t *embed_q8 = nullptr;      // tied embedding, Q8R (Q8_0 repacked for aligned streaming)
    uint16_t *embed_bf16 = nullptr;   // device copy of the tied embedding (input gather)
    float *final_norm = nullptr;
    // decode buffers
    float *x, *x2, *normed, *q, *k, *v, *attn, *mlp_out, *act, *logits;
    uint32_t *topk_ids;
    float *topk_vals;
    uint32_t *slots;   // [8192]: global list at 0, sliding list at 4096
    uint32_t *step;    // {clock, slot_idx, S_global, S_sliding}
    uint32_t *tok;     // one token id for chn_decode_token
    uint32_t *mv_ws;
    size_t mv_ws_words;
    float2 *rope_tab;    // [2][kRopePairs] (cos, sin) for the step's clock
    float *attn_ws;
    uint64_t *topk_ws;
    // prefill buffers
    uint32_t max_tok = 0;
    float *px, *pn, *pq, *pk, *pv, *pmlp, *pact, *pattn_ws;
    unsigned char *pfrag;   // prefill attention: the keys' bf16 operand fragments
    size_t pfrag_bytes;
    float2 *prope;       // prefill (cos, sin) per token: [2 kinds][T][rot / 2]
    __bf16 *pxb;
    uint32_t *pslots, *ptok;
    // pinned staging
    float *h_x = nullptr;
    uint32_t *h_slots = nullptr, *h_step = nullptr, *h_ids = nullptr;
    float *h_vals = nullptr;
    hipGraphExec_t exec[3] = {nullptr, nullptr, nullptr};   // without logits, with, greedy step
    bool use_graph = true;                                   // false: launch the kernels one by one
    // device-resident greedy decoding: {clock, count, start token}, tokens out
    uint32_t *gen = nullptr, *gen_tokens = nullptr;
    uint32_t *h_gen = nullptr;
    // prefill checkpoints: an event after every fourth layer, waited on in
    // order once the whole prefill is enqueued
    std::vector<hipEvent_t> pev;
    // ring state the greedy head reads: turn boundaries, recall clocks
    uint32_t *ring_bounds = nullptr, *ring_recall = nullptr;
    // quiescence: per layer a skip flag and the input stream at the previous
    // gated step ([num_layers][hidden], zero at creation)
    uint32_t *qflags = nullptr;
    float *qprev = nullptr;
    std::vector<void *> allocs;
};

namespace chn {

static constexpr uint32_t kSlotsMax = 4096;
static constexpr uint32_t kGreedyCap = 4096;   // most steps per chn_decode_greedy call

static int m_alloc(chn_model *m, size_t bytes, void **p) {
    hipError_t e = hipMalloc(p, bytes ? bytes : 256);
    if (e != hipSuccess) return hip_fail(m->ctx, e, "hipMalloc (model)");
    m->allocs.push_back(*p);
    return CHN_OK;
}
#define M_ALLOC(ptr, bytes)                                     \
    do {                                                        \
        void *p_;                                               \
        int rc_ = m_alloc(m, (bytes), &p_);                     \
        if (rc_) return rc_;                                    \
        ptr = (decltype(ptr))p_;                                \
    } while (0)

// Head shape of a layer kind: full-attention layers take global_head_dim and
// num_global_kv_heads when those are set (0 = same as the sliding layers),
// and rotate their whole head (loader.zig:37-41).
struct HeadShape {
    uint32_t D, nkv, rot;
};
static HeadShape head_shape(const chn_model_config &c, bool full) {
    HeadShape h{c.head_dim, c.num_kv_heads, c.rotary_dim};
    if (full && c.global_head_dim) {
        h.D = c.global_head_dim;
        h.rot = c.global_head_dim;
    }
    if (full && c.num_global_kv_heads) h.nkv = c.num_global_kv_heads;
    return h;
}
static void set_layer_shape(const chn_model_config &c, uint32_t i, chn_model::Layer &l) {
    l.full = c.layer_full[i] != 0;
    const HeadShape h = head_shape(c, l.full);
    l.D = h.D;
    l.nkv = h.nkv;
    l.rot = h.rot;
    l.qd = c.num_heads * h.D;
    l.kvd = h.nkv * h.D;
    l.gqa = c.num_heads / h.nkv;
}
struct MaxDims {
    uint32_t D, qd, kvd;
};
static MaxDims max_dims(const chn_model &m) {
    MaxDims d{0, 0, 0};
    for (const auto &l : m.L) {
        d.D = l.D > d.D ? l.D : d.D;
        d.qd = l.qd > d.qd ? l.qd : d.qd;
        d.kvd = l.kvd > d.kvd ? l.kvd : d.kvd;
    }
    return d;
}

static int validate_config(chn_ctx *ctx, const chn_model_config &c) {
    CHN_REQUIRE(ctx, c.num_layers >= 1 && c.num_layers <= 64, "num_layers %u must be 1..64", c.num_layers);
    CHN_REQUIRE(ctx, c.hidden_size % 128 == 0 && c.hidden_size <= 16384, "hidden_size %u must be a multiple of 128",
                c.hidden_size);
    CHN_REQUIRE(ctx, c.intermediate_size % 128 == 0 && c.intermediate_size <= 16384,
                "intermediate_size %u must be a multiple of 128", c.intermediate_size);
    for (int full = 0; full < 2; ++full) {
        const HeadShape h = head_shape(c, full != 0);
        CHN_REQUIRE(ctx, h.D == 256 || h.D == 512, "head_dim %u must be 256 or 512", h.D);
        CHN_REQUIRE(ctx, c.num_heads > 0 && h.nkv > 0 && c.num_heads % h.nkv == 0,
                    "num_heads %u must be a multiple of the KV head count %u", c.num_heads, h.nkv);
        const uint32_t gqa = c.num_heads / h.nkv;
        CHN_REQUIRE(ctx, gqa == 1 || gqa == 2 || gqa == 4 || (gqa == 8 && h.D == 256),
                    "GQA ratio %u unsupported at head_dim %u", gqa, h.D);
        CHN_REQUIRE(ctx, (c.num_heads * h.D) % 128 == 0, "q_dim must be a multiple of 128");
        CHN_REQUIRE(ctx, h.rot <= h.D && h.rot % 2 == 0, "rotary_dim %u invalid", h.rot);
    }
    CHN_REQUIRE(ctx, c.vocab_size >= 64 && c.vocab_size <= 262144, "vocab_size %u must be 64..262144", c.vocab_size);
    CHN_REQUIRE(ctx, c.hidden_size <= 4096, "hidden_size %u: the Q8 logits matvec needs K <= 4096", c.hidden_size);
    CHN_REQUIRE(ctx, c.max_prefill_tokens >= 1 && c.max_prefill_tokens <= 4096, "max_prefill_tokens %u invalid",
                c.max_prefill_tokens);
    CHN_REQUIRE(ctx, c.quiescence_thresh >= 0.0f && c.quiescence_thresh <= 3.0e38f, "quiescence_thresh must be >= 0");
    return CHN_OK;
}

// activation, KV and workspace buffers shared by both constructors
static int alloc_runtime(chn_model *m) {
    const chn_model_config &c = m->cfg;
    const uint32_t H = c.hidden_size, I = c.intermediate_size, V = c.vocab_size;
    const MaxDims md = max_dims(*m);
    const uint32_t qd = md.qd, kvd = md.kvd;
    for (auto &l : m->L) {
        M_ALLOC(l.kc, (size_t)kSlotsMax * l.kvd * 4);
        M_ALLOC(l.vc, (size_t)kSlotsMax * l.kvd * 4);
    }
    M_ALLOC(m->x, H * 4);
    M_ALLOC(m->x2, H * 4);
    M_ALLOC(m->normed, H * 4);
    M_ALLOC(m->q, qd * 4);
    M_ALLOC(m->k, kvd * 4);
    M_ALLOC(m->v, kvd * 4);
    M_ALLOC(m->attn, qd * 4);
    M_ALLOC(m->mlp_out, H * 4);
    M_ALLOC(m->act, I * 4);
    M_ALLOC(m->logits, (size_t)V * 4);
    M_ALLOC(m->topk_ids, 64 * 4);
    M_ALLOC(m->topk_vals, 64 * 4);
    M_ALLOC(m->slots, 2 * kSlotsMax * 4);
    M_ALLOC(m->step, 64);
    M_ALLOC(m->tok, 64);
    M_ALLOC(m->gen, 64);
    M_ALLOC(m->gen_tokens, (size_t)kGreedyCap * 4);
    M_ALLOC(m->ring_bounds, 1024 * 4);
    M_ALLOC(m->ring_recall, 128 * 4);
    M_ALLOC(m->qflags, (size_t)c.num_layers * 4);
    M_ALLOC(m->qprev, (size_t)c.num_layers * H * 4);
    const uint32_t kmax = H > I ? (H > qd ? H : qd) : (I > qd ? I : qd);
    size_t mvb = mv_ws_bytes(kmax);
    if (xbytes_bytes(H / 32) > mvb) mvb = xbytes_bytes(H / 32);
    m->mv_ws_words = mvb / 4;
    M_ALLOC(m->mv_ws, 2 * mvb);      // two plane sets: the gate/up input and its output
    M_ALLOC(m->attn_ws, attn_ws_bytes(c.num_heads, md.D, kSlotsMax));
    M_ALLOC(m->rope_tab, 2 * kRopePairs * sizeof(float2));
    M_ALLOC(m->topk_ws, topk_ws_bytes(V));
    const uint32_t T = c.max_prefill_tokens;
    m->max_tok = T;
    M_ALLOC(m->px, (size_t)T * H * 4);
    M_ALLOC(m->pn, (size_t)T * H * 4);
    M_ALLOC(m->pq, (size_t)T * qd * 4);
    M_ALLOC(m->pk, (size_t)T * kvd * 4);
    M_ALLOC(m->pv, (size_t)T * kvd * 4);
    M_ALLOC(m->pmlp, (size_t)4 * T * H * 4);          // up to four partial outputs of a split contraction
    M_ALLOC(m->pattn_ws, prefill_attn_ws_bytes(T, c.num_heads, md.D));
    // every key of a prefill (at most the ring plus the batch) for the KV
    // heads of the widest 256-dim layer
    m->pfrag_bytes = prefill_frag_bytes(md.kvd / 256 ? md.kvd / 256 : 1, kSlotsMax + T);
    M_ALLOC(m->pfrag, m->pfrag_bytes);
    M_ALLOC(m->prope, (size_t)2 * T * kRopePairs * sizeof(float2));
    M_ALLOC(m->pact, (size_t)T * I * 4);
    M_ALLOC(m->pxb, (size_t)T * (H > qd ? H : qd) * 2);   // bf16 operands of width H or qd; act goes to pact
    M_ALLOC(m->pslots, (size_t)(kSlotsMax + T) * 4);
    M_ALLOC(m->ptok, (size_t)T * 4);
    hipError_t e = hipHostMalloc((void **)&m->h_x, H * 4);
    if (e == hipSuccess) e = hipHostMalloc((void **)&m->h_slots, 2 * kSlotsMax * 4);
    if (e == hipSuccess) e = hipHostMalloc((void **)&m->h_step, 64);
    if (e == hipSuccess) e = hipHostMalloc((void **)&m->h_ids, 64 * 4);
    if (e == hipSuccess) e = hipHostMalloc((void **)&m->h_vals, 64 * 4);
    if (e == hipSuccess) e = hipHostMalloc((void **)&m->h_gen, (size_t)kGreedyCap * 4);
    if (e != hipSuccess) return hip_fail(m->ctx, e, "hipHostMalloc");
    m->pev.assign((c.num_layers + 3) / 4, nullptr);
    for (auto &ev : m->pev) {
        e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (e != hipSuccess) return hip_fail(m->ctx, e, "hipEventCreate");
    }
    // zero KV caches and slot buffers with a kernel (no memset nodes anywhere)
    for (auto &l : m->L) {
        int rc = chn_fill_u32(m->ctx, l.kc, 0, (size_t)kSlotsMax * l.kvd);
        if (!rc) rc = chn_fill_u32(m->ctx, l.vc, 0, (size_t)kSlotsMax * l.kvd);
        if (rc) return rc;
    }
    int rc = chn_fill_u32(m->ctx, m->slots, 0, 2 * kSlotsMax);
    if (!rc) rc = chn_fill_u32(m->ctx, m->step, 0, 16);
    if (!rc) rc = chn_fill_u32(m->ctx, m->topk_ids, 0, 64);
    if (!rc) rc = chn_fill_u32(m->ctx, m->gen, 0, 16);
    if (!rc) rc = chn_fill_u32(m->ctx, m->qflags, 0, c.num_layers);
    if (!rc) rc = chn_fill_u32(m->ctx, m->qprev, 0, (size_t)c.num_layers * H);
    // the state the reference's Server.init zeroes through its UMA slices
    // (src/server.zig:76-81: buf_logits, buf_x, the prefill's buf_x and
    // buf_normed_x) starts at zero here, so reads before the first step see
    // what they would see there
    if (!rc) rc = chn_fill_u32(m->ctx, m->x, 0, H);
    if (!rc) rc = chn_fill_u32(m->ctx, m->x2, 0, H);
    if (!rc) rc = chn_fill_u32(m->ctx, m->normed, 0, H);
    if (!rc) rc = chn_fill_u32(m->ctx, m->logits, 0, V);
    if (!rc) rc = chn_fill_u32(m->ctx, m->topk_vals, 0, 64);
    if (!rc) rc = chn_fill_u32(m->ctx, m->px, 0, (size_t)T * H);
    if (!rc) rc = chn_fill_u32(m->ctx, m->pn, 0, (size_t)T * H);
    return rc;
}

// ---- device-resident greedy steps
// The reference's ring (DynamicRingBuffer, src/ring_buffer.zig:17-355):
// anchors [0, A) keep clocks 0..A-1, the FIFO window [A, 3968) takes clock c
// at A + (c - A) mod (3968 - A), the recall tier [3968, 4096) holds
// retrieved entries.  gen = {clock, count, start token, A, n_boundaries,
// has_recall}.
static constexpr uint32_t kRecallStart = kSlotsMax - 128;
static constexpr uint32_t kMaxAnchors = kRecallStart - 64;    // setNumAnchors' cap
static constexpr uint32_t kMaxBoundaries = 1024;
static constexpr uint32_t kRecallNone = 0xFFFFFFFFu;

// Head of one greedy step: the step parameters {clock, slot_idx, S_global,
// S_sliding}, the chronological slot lists that getActiveSlotsLayer gives
// for a history in which every clock so far was written
// (src/ring_buffer.zig:291-333: anchors, the window from the snapped start
// (snapToBoundary, :92-100), then the recall slots whose clock has passed;
// the sliding list: the newest `window` clocks, anchors included, no
// recall), and the input token (the start token, then the previous step's
// argmax), and the step's input row x = bf16(embed[token]) * scale (the
// embedding gather, expandEmbeddings).
__global__ __launch_bounds__(256) void k_greedy_head(const uint32_t *__restrict__ gen,
                                                     const uint32_t *__restrict__ topk_ids,
                                                     const uint32_t *__restrict__ bounds,
                                                     const uint32_t *__restrict__ recall,
                                                     uint32_t *__restrict__ step, uint32_t *__restrict__ slots,
                                                     uint32_t *__restrict__ tok, uint32_t window,
                                                     const uint16_t *__restrict__ embed, uint32_t H, float scale,
                                                     float *__restrict__ x) {
    __shared__ uint32_t s_first, s_cnt[2];
    const uint32_t t = threadIdx.x, lane = t & 63, wave = t >> 6;
    if (t == 0) s_first = kRecallNone;
    __syncthreads();
    // The loads come in two rounds, each issued at once: the step state,
    // the last argmax and the recall ranks; then the input row (its address
    // needs the token) with the turn boundaries.
    const uint32_t clock = gen[0], count = gen[1], A = gen[3], nb = gen[4];
    const uint32_t tk0 = topk_ids[0];
    const uint32_t rec0 = t < 128 ? recall[t] : kRecallNone;   // read whether or not recall is on
    const uint32_t rec = gen[5] ? rec0 : kRecallNone;
    const uint32_t token = count == 0 ? gen[2] : tk0;
    const uint16_t *row = embed + (size_t)token * H;
    constexpr uint32_t kRowLoads = 4;   // 4 x 4 values per thread: H <= 4096
    const bool vec = H % 4 == 0 && H <= 4 * 256 * kRowLoads;
    uint2 rv[kRowLoads];
    if (vec) {
#pragma unroll
        for (uint32_t j = 0; j < kRowLoads; ++j) {
            const uint32_t i = t + 256 * j;
            rv[j] = i < H / 4 ? ((const uint2 *)row)[i] : make_uint2(0u, 0u);
        }
    }
    const uint32_t W = kRecallStart - A;
    // global window: raw start, snapped to the first boundary at or after it
    const uint32_t raw = clock >= W ? clock - W + 1 : 0;
    if (raw > A)
        for (uint32_t i = t; i < nb; i += 256)
            if (bounds[i] >= raw) atomicMin(&s_first, i);
    __syncthreads();
    const uint32_t gmin = s_first == kRecallNone ? raw : bounds[s_first];
    const uint32_t na = clock + 1 < A ? clock + 1 : A;
    const uint32_t gs = gmin > A ? gmin : A;
    const uint32_t nw = clock >= gs ? clock + 1 - gs : 0;
    for (uint32_t i = t; i < na; i += 256) slots[i] = i;
    for (uint32_t i = t; i < nw; i += 256) slots[na + i] = A + (gs + i - A) % W;
    // recall ranks whose clock has passed, in rank order (two waves, ballots)
    const bool f = rec != kRecallNone && rec <= clock;
    const uint64_t bal = __ballot(f);
    if (lane == 0 && wave < 2) s_cnt[wave] = (uint32_t)__popcll(bal);
    __syncthreads();
    const uint32_t pre = (uint32_t)__popcll(bal & ((1ull << lane) - 1ull)) + (wave == 1 ? s_cnt[0] : 0u);
    if (f) slots[na + nw + pre] = kRecallStart + t;
    // sliding list: the newest `window` clocks whose slot still holds them
    const uint32_t raws = clock >= window ? clock - window + 1 : 0;
    const uint32_t nas = na > raws ? na - raws : 0;
    uint32_t ss = raws > A ? raws : A;
    ss = raw > ss ? raw : ss;
    const uint32_t nsw = clock >= ss ? clock + 1 - ss : 0;
    uint32_t *sl = slots + kSlotsMax;
    for (uint32_t i = t; i < nas; i += 256) sl[i] = raws + i;
    for (uint32_t i = t; i < nsw; i += 256) sl[nas + i] = A + (ss + i - A) % W;
    if (t == 0) {
        step[0] = clock;
        step[1] = clock < A ? clock : A + (clock - A) % W;
        step[2] = na + nw + s_cnt[0] + s_cnt[1];
        step[3] = nas + nsw;
        tok[0] = token;
    }
    auto bf = [&](uint32_t b16) { return __builtin_bit_cast(float, b16 << 16) * scale; };
    if (vec) {
#pragma unroll
        for (uint32_t j = 0; j < kRowLoads; ++j) {
            const uint32_t i = t + 256 * j;
            if (i < H / 4)
                *(float4 *)(x + 4 * i) = make_float4(bf(rv[j].x & 0xffffu), bf(rv[j].x >> 16), bf(rv[j].y & 0xffffu),
                                                     bf(rv[j].y >> 16));
        }
    } else {
        for (uint32_t i = t; i < H; i += 256) x[i] = bf(row[i]);
    }
}

// ---- the decode sequence (recordLayerDirect / recordForwardGraph,
// src/gpu/model_dispatch.zig:10-45,103-126)
static int record_decode(chn_model *m, bool with_logits, const GreedyTail *tail = nullptr) {
    chn_ctx *ctx = m->ctx;
    hipStream_t s = ctx->stream;
    const chn_model_config &c = m->cfg;
    const uint32_t H = c.hidden_size, I = c.intermediate_size, nq = c.num_heads;
    const float eps = c.rms_norm_eps;
    int rc;
#define R_(call)                 \
    do {                         \
        rc = (call);             \
        if (rc) return rc;       \
    } while (0)
    // Six kernels per layer.  The step's norms run as the prologue of the
    // matvec that consumes them (every workgroup recomputes the norm into
    // LDS; workgroup 0 writes the new residual stream, alternating between
    // x and x2 so no workgroup reads a half-written one): QKV takes the
    // previous layer's FFN residual and this layer's input norm, gate/up
    // the attention residual and the pre-FFN norm.  Attention writes the
    // planes of its output for o_proj (mv_ws) and gate/up those of the
    // activations for down (the second plane set).
    uint32_t *xp = m->mv_ws, *xp_act = m->mv_ws + m->mv_ws_words;
    float *xa = m->x, *xb = m->x2;
    const RopeTab no_rope{nullptr, nullptr, {0.0f, 0.0f}, {0u, 0u}};
    // Quiescence gating (src/gpu/model_dispatch.zig:103-126): only in the
    // steps that return logits, for layers from num_layers / 3 on.
    const bool gate_on = with_logits && c.quiescence_thresh > 0.0f;
    const uint32_t dense_limit = c.num_layers / 3;
    auto gated = [&](uint32_t i) { return gate_on && i >= dense_limit; };
    for (uint32_t i = 0; i < c.num_layers; ++i) {
        const auto &l = m->L[i];
        uint32_t *skip = gated(i) ? m->qflags + i : nullptr;
        const Quiesce q{i > 0 && gated(i - 1) ? m->qflags + i - 1 : nullptr, skip,
                        skip ? m->qprev + (size_t)i * H : nullptr, c.quiescence_thresh, i == 0 ? 1u : 0u};
        NormArgs n1{xa, nullptr, nullptr, l.in_norm, xb, m->normed, eps, 1.0f, no_rope, skip ? q : Quiesce{}};
        int mode1 = NORM_PLAIN;
        if (i == 0) {
            // the step's first kernel also writes its RoPE table
            n1.rope = RopeTab{m->step, m->rope_tab, {c.rope_theta, c.rope_theta_full},
                              {head_shape(c, false).rot, head_shape(c, true).rot}};
        } else {
            const auto &p = m->L[i - 1];
            n1.r = m->mlp_out;
            n1.pw = p.has_post_ffn ? p.post_ffn : nullptr;
            n1.scalar = p.scalar;
            mode1 = p.has_post_ffn ? NORM_POST_ADD : NORM_ADD;
        }
        R_(mvr_qkv_nx(ctx, l.Wq, l.Wk, l.Wv, m->q, m->k, m->v, l.qd, l.kvd, H, n1, mode1));
        R_(launch_rope_decode_attn(ctx, m->q, m->k, m->v, l.q_norm, l.k_norm, l.kc, l.vc, m->step,
                                   m->slots + (l.full ? 0 : kSlotsMax), m->step + (l.full ? 2 : 3), kSlotsMax, nq, l.D,
                                   l.kvd, l.gqa, l.rot, (int)c.k_eq_v, m->rope_tab + (l.full ? kRopePairs : 0), eps,
                                   1.0f, m->attn, m->attn_ws, xp, skip));
        R_(mvr_gemv(ctx, l.Wo, m->attn, m->mlp_out, H, l.qd, xp, true, skip));
        const NormArgs n2{xb, m->mlp_out, l.has_post_attn ? l.post_attn : nullptr, l.pre_ffn, xa, m->normed,
                          eps, 1.0f, no_rope, skip ? Quiesce{nullptr, skip, q.x_prev, q.thresh, 0u} : Quiesce{}};
        R_(mvr_mlp_nx(ctx, l.Wg, l.Wu, m->act, xp_act, I, H, n2, l.has_post_attn ? NORM_POST_ADD : NORM_ADD));
        R_(mvr_gemv(ctx, l.Wd, m->act, m->mlp_out, H, I, xp_act, true, skip));
    }
    // the last layer's FFN residual (into x) and the final norm
    const auto &last = m->L[c.num_layers - 1];
    // (its byte planes are the logits matvec's input)
    R_(launch_norm_planes(s, xa, m->mlp_out, last.has_post_ffn ? last.post_ffn : nullptr, m->final_norm, m->normed,
                          nullptr, H, eps, last.scalar, true, nullptr,
                          gated(c.num_layers - 1) ? m->qflags + c.num_layers - 1 : nullptr,
                          with_logits ? m->mv_ws : nullptr));
    if (with_logits) {
        R_(launch_gemv_q8r(s, m->embed_q8, m->normed, m->logits, c.vocab_size, H / 32, m->mv_ws, true));
        R_(launch_topk64(s, m->logits, c.vocab_size, m->topk_ids, m->topk_vals, m->topk_ws, tail));
    }
#undef R_
    return CHN_OK;
}

static int record_greedy(chn_model *m) {
    hipStream_t s = m->ctx->stream;
    const uint32_t H = m->cfg.hidden_size;
    // the head also gathers the input row; the top-64 merge ends the step
    // (appends the argmax, advances the clock)
    k_greedy_head<<<1, 256, 0, s>>>(m->gen, m->topk_ids, m->ring_bounds, m->ring_recall, m->step, m->slots, m->tok,
                                    m->cfg.sliding_window, m->embed_bf16, H, sqrtf((float)H), m->x);
    if (hipGetLastError() != hipSuccess) return hip_fail(m->ctx, hipGetLastError(), "k_greedy_head");
    const GreedyTail tail{m->gen, m->gen_tokens, kGreedyCap};
    return record_decode(m, true, &tail);
}

static int build_graphs(chn_model *m) {
    hipStream_t s = m->ctx->stream;
    for (int wl = 0; wl < 3; ++wl) {
        CHN_HIP(m->ctx, hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
        int rc = wl == 2 ? record_greedy(m) : record_decode(m, wl == 1);
        hipGraph_t g = nullptr;
        hipError_t e = hipStreamEndCapture(s, &g);
        if (rc) {
            if (g) (void)hipGraphDestroy(g);
            return rc;
        }
        if (e != hipSuccess) return hip_fail(m->ctx, e, "hipStreamEndCapture");
        e = hipGraphInstantiate(&m->exec[wl], g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (e != hipSuccess) return hip_fail(m->ctx, e, "hipGraphInstantiate");
    }
    return CHN_OK;
}

static void free_model(chn_model *m) {
    if (!m) return;
    if (m->ctx) (void)hipStreamSynchronize(m->ctx->stream);
    for (int i = 0; i < 3; ++i)
        if (m->exec[i]) (void)hipGraphExecDestroy(m->exec[i]);
    for (void *p : m->allocs) (void)hipFree(p);
    if (m->h_x) (void)hipHostFree(m->h_x);
    if (m->h_slots) (void)hipHostFree(m->h_slots);
    if (m->h_step) (void)hipHostFree(m->h_step);
    if (m->h_ids) (void)hipHostFree(m->h_ids);
    if (m->h_vals) (void)hipHostFree(m->h_vals);
    if (m->h_gen) (void)hipHostFree(m->h_gen);
    for (hipEvent_t e : m->pev) (void)hipEventDestroy(e);
    delete m;
}

// bf16 (host) -> quantizeRowQ4_0 on the device into the reference layout
// (staging `tq`), then repacked into the model's Q4R matrix.  `tmp` holds
// at least rows*cols bf16, `tq` rows*cols/32 Q4 blocks.
static int ingest_q4r(chn_model *m, const uint16_t *src, uint32_t rows, uint32_t cols, uint32_t **dst,
                      uint16_t *tmp, uint32_t *tq) {
    const size_t nblk = (size_t)rows * (cols / 32);
    M_ALLOC(*dst, q4r_bytes(rows, cols));
    CHN_HIP(m->ctx, hipMemcpyAsync(tmp, src, (size_t)rows * cols * 2, hipMemcpyHostToDevice, m->ctx->stream));
    if (launch_quantize(m->ctx->stream, 0, tmp, tq, nblk)) return hip_fail(m->ctx, hipGetLastError(), "quantize");
    if (launch_q4_repack(m->ctx->stream, tq, rows, cols, *dst)) return hip_fail(m->ctx, hipGetLastError(), "repack");
    CHN_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    return CHN_OK;
}

// The tied embedding for the logits: quantizeRowQ8_0 of the device bf16
// copy into a staging buffer in the reference layout, then repacked into
// m->embed_q8 (Q8R, chn_q8_repack's layout).
static int quantize_embed_q8r(chn_model *m, uint32_t V, uint32_t H) {
    const size_t nblk = (size_t)V * (H / 32);
    uint32_t *tq = nullptr;
    CHN_HIP(m->ctx, hipMalloc((void **)&tq, nblk * 36));
    int rc = CHN_OK;
    if (launch_quantize(m->ctx->stream, 1, m->embed_bf16, tq, nblk))
        rc = hip_fail(m->ctx, hipGetLastError(), "quantize embedding");
    else if (launch_q8_repack(m->ctx->stream, tq, V, H / 32, m->embed_q8))
        rc = hip_fail(m->ctx, hipGetLastError(), "repack embedding");
    const hipError_t e = hipStreamSynchronize(m->ctx->stream);
    (void)hipFree(tq);
    if (!rc && e != hipSuccess) rc = hip_fail(m->ctx, e, "quantize embedding");
    return rc;
}

// bf16 norm weights -> fp32; missing norms -> 1.0 (createNormBuffer,
// src/gpu/model_gpu.zig:57-66)
static int ingest_norm(chn_model *m, const uint16_t *src, uint32_t n, float **dst) {
    M_ALLOC(*dst, n * 4);
    std::vector<float> h(n, 1.0f);
    if (src)
        for (uint32_t i = 0; i < n; ++i) {
            uint32_t u = (uint32_t)src[i] << 16;
            std::memcpy(&h[i], &u, 4);
        }
    CHN_HIP(m->ctx, hipMemcpy(*dst, h.data(), n * 4, hipMemcpyHostToDevice));
    return CHN_OK;
}

static int fill_ones(chn_model *m, uint32_t n, float **dst) {
    M_ALLOC(*dst, n * 4);
    return chn_fill_u32(m->ctx, *dst, 0x3F800000u, n);
}

}  // namespace chn

using namespace chn;

extern "C" int chn_model_create(chn_ctx *ctx, const chn_model_config *cfg, const chn_layer_weights *layers,
                                const uint16_t *embed_bf16, const uint16_t *final_norm_bf16, chn_model **out) {
    if (!ctx || !cfg || !layers || !embed_bf16 || !out) return ctx ? set_err(ctx, CHN_E_INVALID, "NULL argument") : CHN_E_INVALID;
    *out = nullptr;
    int rc = validate_config(ctx, *cfg);
    if (rc) return rc;
    chn_model *m = new chn_model();
    m->ctx = ctx;
    m->cfg = *cfg;
    const uint32_t H = cfg->hidden_size, I = cfg->intermediate_size;
    m->L.resize(cfg->num_layers);
    for (uint32_t i = 0; i < cfg->num_layers; ++i) set_layer_shape(*cfg, i, m->L[i]);
    const MaxDims md = max_dims(*m);
    const size_t tmp_elems = (size_t)I * H > (size_t)md.qd * H ? (size_t)I * H : (size_t)md.qd * H;
    uint16_t *tmp = nullptr;
    uint32_t *tq = nullptr;
    hipError_t e = hipMalloc(&tmp, tmp_elems * 2);
    if (e == hipSuccess) e = hipMalloc(&tq, tmp_elems / 32 * 20);
    if (e != hipSuccess) {
        (void)hipFree(tmp);
        free_model(m);
        return hip_fail(ctx, e, "hipMalloc (ingest staging)");
    }
#define C_(call)                 \
    do {                         \
        rc = (call);             \
        if (rc) goto fail;       \
    } while (0)
    for (uint32_t i = 0; i < cfg->num_layers; ++i) {
        const chn_layer_weights &w = layers[i];
        auto &l = m->L[i];
        const uint32_t D = l.D, qd = l.qd, kvd = l.kvd;
        if (!w.q_proj || !w.k_proj || !w.o_proj || !w.gate_proj || !w.up_proj || !w.down_proj) {
            rc = set_err(ctx, CHN_E_INVALID, "layer %u: missing projection weights", i);
            goto fail;
        }
        C_(ingest_q4r(m, w.q_proj, qd, H, &l.Wq, tmp, tq));
        C_(ingest_q4r(m, w.k_proj, kvd, H, &l.Wk, tmp, tq));
        // v_proj absent -> k_proj (src/gpu/model_gpu.zig:123)
        C_(ingest_q4r(m, w.v_proj ? w.v_proj : w.k_proj, kvd, H, &l.Wv, tmp, tq));
        C_(ingest_q4r(m, w.o_proj, H, qd, &l.Wo, tmp, tq));
        C_(ingest_q4r(m, w.gate_proj, I, H, &l.Wg, tmp, tq));
        C_(ingest_q4r(m, w.up_proj, I, H, &l.Wu, tmp, tq));
        C_(ingest_q4r(m, w.down_proj, H, I, &l.Wd, tmp, tq));
        C_(ingest_norm(m, w.input_layernorm, H, &l.in_norm));
        C_(ingest_norm(m, w.q_norm, D, &l.q_norm));
        C_(ingest_norm(m, w.k_norm, D, &l.k_norm));
        C_(ingest_norm(m, w.post_attention_layernorm, H, &l.post_attn));
        C_(ingest_norm(m, w.pre_feedforward_layernorm, H, &l.pre_ffn));
        C_(ingest_norm(m, w.post_feedforward_layernorm, H, &l.post_ffn));
        l.has_post_attn = w.post_attention_layernorm != nullptr;
        l.has_post_ffn = w.post_feedforward_layernorm != nullptr;
        l.scalar = w.has_layer_scalar ? w.layer_scalar : 1.0f;
    }
    // tied embedding: a device bf16 copy for the input gather, Q8 for the logits
    C_(m_alloc(m, (size_t)cfg->vocab_size * H * 2, (void **)&m->embed_bf16));
    C_(chn_upload(ctx, m->embed_bf16, embed_bf16, (size_t)cfg->vocab_size * H * 2));
    C_(m_alloc(m, (size_t)cfg->vocab_size * (H / 32) * 36, (void **)&m->embed_q8));
    C_(quantize_embed_q8r(m, cfg->vocab_size, H));
    C_(ingest_norm(m, final_norm_bf16, H, &m->final_norm));
    C_(alloc_runtime(m));
    C_(build_graphs(m));
#undef C_
    (void)hipFree(tmp);
    (void)hipFree(tq);
    *out = m;
    return CHN_OK;
fail:
    (void)hipFree(tmp);
    (void)hipFree(tq);
    free_model(m);
    return rc;
}

extern "C" int chn_model_create_synthetic(chn_ctx *ctx, const chn_model_config *cfg, uint64_t seed,
                                          chn_model **out) {
    if (!ctx || !cfg || !out) return ctx ? set_err(ctx, CHN_E_INVALID, "NULL argument") : CHN_E_INVALID;
    *out = nullptr;
    int rc = validate_config(ctx, *cfg);
    if (rc) return rc;
    chn_model *m = new chn_model();
    m->ctx = ctx;
    m->cfg = *cfg;
    const uint32_t H = cfg->hidden_size, I = cfg->intermediate_size, V = cfg->vocab_size;
    const float smin = 0.005f, smax = 0.02f;
    // staging for one matrix in the reference Q4 layout
    uint32_t *tq = nullptr;
    {
        size_t big = (size_t)I * H;
        for (uint32_t i = 0; i < cfg->num_layers; ++i) {
            const HeadShape h = head_shape(*cfg, cfg->layer_full[i] != 0);
            const size_t qh = (size_t)cfg->num_heads * h.D * H;
            if (qh > big) big = qh;
        }
        hipError_t e = hipMalloc(&tq, big / 32 * 20);
        if (e != hipSuccess) {
            delete m;
            return hip_fail(ctx, e, "hipMalloc (synthetic staging)");
        }
    }
#define C_(call)                 \
    do {                         \
        rc = (call);             \
        if (rc) goto fail;       \
    } while (0)
    m->L.resize(cfg->num_layers);
    for (uint32_t i = 0; i < cfg->num_layers; ++i) {
        auto &l = m->L[i];
        set_layer_shape(*cfg, i, l);
        const uint32_t D = l.D, qd = l.qd, kvd = l.kvd;
        const uint64_t ls = seed + 64ull * (i + 1);
        struct {
            uint32_t **w;
            uint32_t rows, cols;
        } mats[7] = {{&l.Wq, qd, H}, {&l.Wk, kvd, H}, {&l.Wv, kvd, H}, {&l.Wo, H, qd},
                     {&l.Wg, I, H},  {&l.Wu, I, H},   {&l.Wd, H, I}};
        for (int j = 0; j < 7; ++j) {
            // generated in the reference layout, kept repacked (Q4R)
            C_(m_alloc(m, q4r_bytes(mats[j].rows, mats[j].cols), (void **)mats[j].w));
            C_(chn_synth_q4(ctx, tq, mats[j].rows, mats[j].cols, ls + j, smin, smax));
            if (launch_q4_repack(ctx->stream, tq, mats[j].rows, mats[j].cols, *mats[j].w)) {
                rc = hip_fail(ctx, hipGetLastError(), "repack");
                goto fail;
            }
        }
        C_(fill_ones(m, H, &l.in_norm));
        C_(fill_ones(m, D, &l.q_norm));
        C_(fill_ones(m, D, &l.k_norm));
        C_(fill_ones(m, H, &l.post_attn));
        C_(fill_ones(m, H, &l.pre_ffn));
        C_(fill_ones(m, H, &l.post_ffn));
        l.has_post_attn = l.has_post_ffn = true;
        l.scalar = 1.0f;
    }
    // tied embedding: bf16 ~ N(0, 0.02) (kept on device for the input
    // gather), Q8-quantized for the logits exactly as quantizeRowQ8_0 would
    {
        const size_t n = (size_t)V * H;
        float *tmpf = nullptr;
        hipError_t e = hipMalloc(&tmpf, n * 4);
        if (e != hipSuccess) {
            rc = hip_fail(ctx, e, "hipMalloc (embedding staging)");
            goto fail;
        }
        rc = m_alloc(m, n * 2, (void **)&m->embed_bf16);
        if (rc) {
            (void)hipFree(tmpf);
            goto fail;
        }
        rc = chn_synth_normal(ctx, tmpf, n, seed + 7, 0.02f);
        if (!rc) rc = chn_to_bf16_bits(ctx, tmpf, m->embed_bf16, n);
        if (!rc) rc = chn_sync(ctx);
        (void)hipFree(tmpf);
        if (rc) goto fail;
        C_(m_alloc(m, (size_t)V * (H / 32) * 36, (void **)&m->embed_q8));
        C_(quantize_embed_q8r(m, V, H));
    }
    C_(fill_ones(m, H, &m->final_norm));
    C_(alloc_runtime(m));
    C_(chn_sync(ctx));
    C_(build_graphs(m));
#undef C_
    (void)hipFree(tq);
    *out = m;
    return CHN_OK;
fail:
    (void)hipFree(tq);
    free_model(m);
    return rc;
}

extern "C" void chn_model_destroy(chn_model *m) { free_model(m); }

extern "C" int chn_model_set_graph(chn_model *m, int enabled) {
    if (!m) return CHN_E_INVALID;
    CHN_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    m->use_graph = enabled != 0;
    return CHN_OK;
}

extern "C" int chn_model_embedding_bf16(chn_model *m, const uint16_t **table) {
    if (!m || !table) return CHN_E_INVALID;
    *table = m->embed_bf16;
    return CHN_OK;
}

extern "C" int chn_model_get_config(const chn_model *m, chn_model_config *cfg) {
    if (!m || !cfg) return CHN_E_INVALID;
    *cfg = m->cfg;
    return CHN_OK;
}

static int decode_run(chn_model *m, uint32_t clock, uint32_t slot_idx, const uint32_t *active, uint32_t n_active,
                      const uint32_t *sliding, uint32_t n_sliding, uint32_t *topk_ids, float *topk_vals,
                      uint32_t *token_out, bool x_ready) {
    chn_ctx *ctx = m->ctx;
    hipStream_t s = ctx->stream;
    CHN_REQUIRE(ctx, n_active <= kSlotsMax && n_sliding <= kSlotsMax, "slot lists longer than 4096");
    CHN_REQUIRE(ctx, slot_idx < kSlotsMax, "slot_idx %u out of range", slot_idx);
    CHN_REQUIRE(ctx, (active || !n_active) && (sliding || !n_sliding), "NULL slot list");
    for (uint32_t i = 0; i < n_active; ++i) CHN_REQUIRE(ctx, active[i] < kSlotsMax, "active slot out of range");
    for (uint32_t i = 0; i < n_sliding; ++i) CHN_REQUIRE(ctx, sliding[i] < kSlotsMax, "sliding slot out of range");
    std::memcpy(m->h_slots, active, n_active * 4);
    std::memcpy(m->h_slots + kSlotsMax, sliding, n_sliding * 4);
    m->h_step[0] = clock;
    m->h_step[1] = slot_idx;
    m->h_step[2] = n_active;
    m->h_step[3] = n_sliding;
    if (!x_ready) CHN_HIP(ctx, hipMemcpyAsync(m->x, m->h_x, m->cfg.hidden_size * 4, hipMemcpyHostToDevice, s));
    if (n_active) CHN_HIP(ctx, hipMemcpyAsync(m->slots, m->h_slots, n_active * 4, hipMemcpyHostToDevice, s));
    if (n_sliding)
        CHN_HIP(ctx, hipMemcpyAsync(m->slots + kSlotsMax, m->h_slots + kSlotsMax, n_sliding * 4,
                                    hipMemcpyHostToDevice, s));
    CHN_HIP(ctx, hipMemcpyAsync(m->step, m->h_step, 16, hipMemcpyHostToDevice, s));
    const bool wl = topk_ids != nullptr;
    if (m->use_graph) {
        CHN_HIP(ctx, hipGraphLaunch(m->exec[wl ? 1 : 0], s));
    } else {
        int rc = record_decode(m, wl);
        if (rc) return rc;
    }
    CHN_HIP(ctx, hipMemcpyAsync(m->h_ids, m->topk_ids, 64 * 4, hipMemcpyDeviceToHost, s));
    CHN_HIP(ctx, hipMemcpyAsync(m->h_vals, m->topk_vals, 64 * 4, hipMemcpyDeviceToHost, s));
    CHN_HIP(ctx, hipStreamSynchronize(s));
    if (wl) {
        std::memcpy(topk_ids, m->h_ids, 64 * 4);
        if (topk_vals) std::memcpy(topk_vals, m->h_vals, 64 * 4);
    }
    if (token_out) *token_out = m->h_ids[0];
    return CHN_OK;
}

extern "C" int chn_decode_step(chn_model *m, const float *x, uint32_t clock, uint32_t slot_idx,
                               const uint32_t *active, uint32_t n_active, const uint32_t *sliding,
                               uint32_t n_sliding, uint32_t *topk_ids, float *topk_vals, uint32_t *token_out) {
    if (!m || !x) return m ? set_err(m->ctx, CHN_E_INVALID, "x is NULL") : CHN_E_INVALID;
    std::memcpy(m->h_x, x, m->cfg.hidden_size * 4);
    return decode_run(m, clock, slot_idx, active, n_active, sliding, n_sliding, topk_ids, topk_vals, token_out, false);
}

extern "C" int chn_decode_token(chn_model *m, uint32_t token, uint32_t clock, uint32_t slot_idx,
                                const uint32_t *active, uint32_t n_active, const uint32_t *sliding,
                                uint32_t n_sliding, uint32_t *topk_ids, float *topk_vals, uint32_t *token_out) {
    if (!m) return CHN_E_INVALID;
    chn_ctx *ctx = m->ctx;
    CHN_REQUIRE(ctx, token < m->cfg.vocab_size, "token %u out of range", token);
    m->h_step[8] = token;
    CHN_HIP(ctx, hipMemcpyAsync(m->tok, m->h_step + 8, 4, hipMemcpyHostToDevice, ctx->stream));
    const uint32_t H = m->cfg.hidden_size;
    if (launch_embed(ctx->stream, m->embed_bf16, m->tok, 1, H, sqrtf((float)H), m->x))
        return hip_fail(ctx, hipGetLastError(), "k_embed");
    return decode_run(m, clock, slot_idx, active, n_active, sliding, n_sliding, topk_ids, topk_vals, token_out, true);
}

// n greedy steps on the device (see k_greedy_head): one host round trip
// for the whole run.
extern "C" int chn_decode_greedy(chn_model *m, uint32_t token, uint32_t clock, uint32_t n_steps,
                                 const chn_ring_state *ring, uint32_t *tokens_out) {
    if (!m) return CHN_E_INVALID;
    chn_ctx *ctx = m->ctx;
    hipStream_t s = ctx->stream;
    CHN_REQUIRE(ctx, token < m->cfg.vocab_size, "token %u out of range", token);
    CHN_REQUIRE(ctx, n_steps <= kGreedyCap, "n_steps %u exceeds %u", n_steps, kGreedyCap);
    CHN_REQUIRE(ctx, tokens_out || !n_steps, "NULL tokens_out");
    const chn_ring_state none{0, 0, nullptr, nullptr};
    const chn_ring_state &r = ring ? *ring : none;
    CHN_REQUIRE(ctx, r.num_anchors <= kMaxAnchors, "num_anchors %u exceeds %u", r.num_anchors, kMaxAnchors);
    CHN_REQUIRE(ctx, r.num_boundaries <= kMaxBoundaries, "%u turn boundaries (at most %u)", r.num_boundaries,
                kMaxBoundaries);
    CHN_REQUIRE(ctx, r.boundaries || !r.num_boundaries, "NULL boundaries");
    CHN_REQUIRE(ctx, (uint64_t)clock + n_steps <= 0xFFFFFFFEull, "clock %u + %u steps overflows", clock, n_steps);
    if (!n_steps) return CHN_OK;
    CHN_HIP(ctx, hipStreamSynchronize(s));
    // staging in the pinned buffer: gen at 0, boundaries at 16, recall at 16 + 1024
    uint32_t *hb = m->h_gen + 16, *hr = m->h_gen + 16 + kMaxBoundaries;
    m->h_gen[0] = clock;
    m->h_gen[1] = 0;
    m->h_gen[2] = token;
    m->h_gen[3] = r.num_anchors;
    m->h_gen[4] = r.num_boundaries;
    m->h_gen[5] = r.recall_clocks ? 1u : 0u;
    if (r.num_boundaries) std::memcpy(hb, r.boundaries, (size_t)r.num_boundaries * 4);
    if (r.recall_clocks) std::memcpy(hr, r.recall_clocks, 128 * 4);
    CHN_HIP(ctx, hipMemcpyAsync(m->gen, m->h_gen, 6 * 4, hipMemcpyHostToDevice, s));
    if (r.num_boundaries)
        CHN_HIP(ctx, hipMemcpyAsync(m->ring_bounds, hb, (size_t)r.num_boundaries * 4, hipMemcpyHostToDevice, s));
    if (r.recall_clocks) CHN_HIP(ctx, hipMemcpyAsync(m->ring_recall, hr, 128 * 4, hipMemcpyHostToDevice, s));
    for (uint32_t i = 0; i < n_steps; ++i) {
        if (m->use_graph) {
            CHN_HIP(ctx, hipGraphLaunch(m->exec[2], s));
        } else {
            int rc = record_greedy(m);
            if (rc) return rc;
        }
    }
    CHN_HIP(ctx, hipMemcpyAsync(m->h_gen, m->gen_tokens, (size_t)n_steps * 4, hipMemcpyDeviceToHost, s));
    CHN_HIP(ctx, hipStreamSynchronize(s));
    std::memcpy(tokens_out, m->h_gen, (size_t)n_steps * 4);
    return CHN_OK;
}

// gpuDispatchPrefillBatch (src/gpu/batch_dispatch.zig:27-172)
extern "C" int chn_prefill(chn_model *m, const uint32_t *tokens, uint32_t n, const uint16_t *embed_bf16,
                           const uint32_t *slots, uint32_t n_slots, uint32_t start_clock, uint32_t num_prev_slots,
                           float *logits_out, uint32_t *topk_ids, float *topk_vals, chn_progress_fn progress,
                           void *progress_ctx) {
    if (!m) return CHN_E_INVALID;
    chn_ctx *ctx = m->ctx;
    hipStream_t s = ctx->stream;
    const chn_model_config &c = m->cfg;
    if (n == 0 || n > m->max_tok) return set_err(ctx, CHN_E_BATCH_TOO_LARGE, "batch of %u tokens (max %u)", n, m->max_tok);
    CHN_REQUIRE(ctx, tokens && slots, "NULL tokens or slots");
    CHN_REQUIRE(ctx, n_slots >= num_prev_slots + n && n_slots <= kSlotsMax + m->max_tok,
                "slot list of %u entries must cover %u previous + %u new slots", n_slots, num_prev_slots, n);
    CHN_REQUIRE(ctx, embed_bf16 || m->embed_bf16, "no embedding table");
    for (uint32_t i = 0; i < n; ++i) CHN_REQUIRE(ctx, tokens[i] < c.vocab_size, "token %u out of range", tokens[i]);
    for (uint32_t i = 0; i < n_slots; ++i) CHN_REQUIRE(ctx, slots[i] < kSlotsMax, "slot out of range");
    const uint32_t H = c.hidden_size, I = c.intermediate_size, nq = c.num_heads;
    const float eps = c.rms_norm_eps;
    const float escale = sqrtf((float)H);

    // embeddings: x = bf16(embed[tok]) * sqrt(H) (expandEmbeddings, :14-23)
    if (embed_bf16) {
        std::vector<float> hx((size_t)n * H);
        for (uint32_t t = 0; t < n; ++t)
            for (uint32_t i = 0; i < H; ++i) {
                uint32_t u = (uint32_t)embed_bf16[(size_t)tokens[t] * H + i] << 16;
                float f;
                std::memcpy(&f, &u, 4);
                hx[(size_t)t * H + i] = f * escale;
            }
        CHN_HIP(ctx, hipMemcpyAsync(m->px, hx.data(), hx.size() * 4, hipMemcpyHostToDevice, s));
        CHN_HIP(ctx, hipStreamSynchronize(s));
    } else {
        // (a copy from pageable memory returns once the bytes are staged, so
        // the caller's array may change afterwards; no wait is needed here)
        CHN_HIP(ctx, hipMemcpyAsync(m->ptok, tokens, n * 4, hipMemcpyHostToDevice, s));
        if (launch_embed(s, m->embed_bf16, m->ptok, n, H, escale, m->px)) return hip_fail(ctx, hipGetLastError(), "k_embed");
    }
    CHN_HIP(ctx, hipMemcpyAsync(m->pslots, slots, (size_t)n_slots * 4, hipMemcpyHostToDevice, s));

    int rc;
#define P_(call)                 \
    do {                         \
        rc = (call);             \
        if (rc) return rc;       \
    } while (0)
    // Every contraction reads bf16 activations that their producer wrote
    // directly: the norm chains and the attention into pxb, gate/up into the
    // act buffer (as bf16).  Where o_proj and down split K, their partial
    // sums go to pmlp + p * max_tok * H and the next norm chain adds them.
    __bf16 *xb = m->pxb;
    __bf16 *actb = (__bf16 *)m->pact;
    // the prompt's rotation angles, once per kind (sliding / full layers)
    const HeadShape hs[2] = {head_shape(c, false), head_shape(c, true)};
    const float thetas[2] = {c.rope_theta, c.rope_theta_full};
    float2 *ptab[2] = {m->prope, m->prope + (size_t)m->max_tok * kRopePairs};
    for (int k = 0; k < 2; ++k) P_(launch_rope_tab_batch(s, ptab[k], start_clock, n, hs[k].rot, thetas[k]));
    for (uint32_t i = 0; i < c.num_layers; ++i) {
        const auto &l = m->L[i];
        const float theta = l.full ? c.rope_theta_full : c.rope_theta;
        if (i == 0)
            P_(launch_rmsnorm_chain(s, m->px, nullptr, nullptr, l.in_norm, xb, nullptr, H, n, eps, 1.0f, false));
        const uint32_t D = l.D, nkv = l.nkv, qd = l.qd, kvd = l.kvd, gqa = l.gqa;
        P_(launch_q4gemm_qkv(ctx, nullptr, l.Wq, l.Wk, l.Wv, m->pq, m->pk, m->pv, n, qd, kvd, H, xb));
        // sliding layers see the last 1024 slots (shaders/batch_causal_attn.wgsl:53)
        // unless the config sets another prefill window
        const uint32_t pwin = c.prefill_window ? c.prefill_window : 1024u, win = l.full ? 0u : pwin;
        // when the new keys start a 32-key chunk, the rope kernel also
        // writes their attention operand fragments
        const bool fuse = prefill_frags_fusable(num_prev_slots, D, gqa);
        P_(launch_batch_qkv_rope(s, m->pq, m->pk, m->pv, l.q_norm, l.k_norm, m->pq, l.kc, l.vc, m->pslots,
                                 num_prev_slots, start_clock, n, nq, nkv, D, l.rot, (int)c.k_eq_v, theta, eps,
                                 ptab[l.full ? 1 : 0], fuse ? m->pfrag : nullptr, m->pfrag_bytes, win));
        P_(launch_prefill_attn(s, m->pq, l.kc, l.vc, m->pslots, n, num_prev_slots, nq, D, kvd, gqa, 1.0f, win,
                               nullptr, xb, m->pattn_ws, m->pfrag, m->pfrag_bytes, fuse));
        const size_t pstride = (size_t)m->max_tok * H;
        PartialOut po_o{pstride, 2};
        P_(launch_q4gemm(ctx, 1, nullptr, l.Wo, nullptr, m->pmlp, n, H, qd, xb, true, nullptr, &po_o));
        P_(launch_rmsnorm_chain(s, m->px, m->pmlp, l.has_post_attn ? l.post_attn : nullptr, l.pre_ffn, xb, nullptr,
                                H, n, eps, 1.0f, true, po_o.parts, pstride));
        P_(launch_q4gemm(ctx, 2, nullptr, l.Wg, l.Wu, nullptr, n, I, H, xb, true, actb));
        PartialOut po_d{pstride, 4};
        P_(launch_q4gemm(ctx, 1, nullptr, l.Wd, nullptr, m->pmlp, n, H, I, actb, true, nullptr, &po_d));
        const bool last = i + 1 == c.num_layers;
        const float *next_norm = last ? m->final_norm : m->L[i + 1].in_norm;
        P_(launch_rmsnorm_chain(s, m->px, m->pmlp, l.has_post_ffn ? l.post_ffn : nullptr, next_norm, xb,
                                last ? m->pn : nullptr, H, n, eps, l.scalar, true, po_d.parts, pstride));
        if ((i + 1) % 4 == 0 || i + 1 == c.num_layers) {
            if (i + 1 == c.num_layers && (logits_out || topk_ids)) {
                CHN_HIP(ctx, hipMemcpyAsync(m->normed, m->pn + (size_t)(n - 1) * H, H * 4, hipMemcpyDeviceToDevice, s));
                P_(launch_gemv_q8r(s, m->embed_q8, m->normed, m->logits, c.vocab_size, H / 32, m->mv_ws));
                P_(launch_topk64(s, m->logits, c.vocab_size, m->topk_ids, m->topk_vals, m->topk_ws));
            }
            CHN_HIP(ctx, hipEventRecord(m->pev[i / 4], s));
        }
    }
#undef P_
    // the reference waits on its fence every four layers and reports
    // progress (src/gpu/batch_dispatch.zig:27-172); here the whole prefill is
    // already enqueued, so the device runs without gaps while the host waits
    // on each checkpoint in turn
    for (uint32_t k = 0; k < (c.num_layers + 3) / 4; ++k) {
        CHN_HIP(ctx, hipEventSynchronize(m->pev[k]));
        if (progress) progress(k * 4 + 4 < c.num_layers ? k * 4 + 4 : c.num_layers, c.num_layers, progress_ctx);
    }
    if (logits_out) CHN_HIP(ctx, hipMemcpy(logits_out, m->logits, (size_t)c.vocab_size * 4, hipMemcpyDeviceToHost));
    if (topk_ids) CHN_HIP(ctx, hipMemcpy(topk_ids, m->topk_ids, 64 * 4, hipMemcpyDeviceToHost));
    if (topk_vals) CHN_HIP(ctx, hipMemcpy(topk_vals, m->topk_vals, 64 * 4, hipMemcpyDeviceToHost));
    return CHN_OK;
}

// KV access for the callers that read or write the caches directly under
// UMA (snapshots, memory, hippocampus, memory_inject): slots
// [slot_begin, slot_begin + n) of layer `layer`, each row kv_dim floats.
extern "C" int chn_kv_read(chn_model *m, uint32_t layer, uint32_t slot_begin, uint32_t n, float *k_out,
                           float *v_out) {
    if (!m) return CHN_E_INVALID;
    CHN_REQUIRE(m->ctx, layer < m->cfg.num_layers && slot_begin + n <= kSlotsMax, "layer/slot range out of bounds");
    const auto &l = m->L[layer];
    const size_t row = l.kvd;
    CHN_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    if (k_out) CHN_HIP(m->ctx, hipMemcpy(k_out, l.kc + slot_begin * row, n * row * 4, hipMemcpyDeviceToHost));
    if (v_out) CHN_HIP(m->ctx, hipMemcpy(v_out, l.vc + slot_begin * row, n * row * 4, hipMemcpyDeviceToHost));
    return CHN_OK;
}

extern "C" int chn_kv_write(chn_model *m, uint32_t layer, uint32_t slot_begin, uint32_t n, const float *k_in,
                            const float *v_in) {
    if (!m) return CHN_E_INVALID;
    CHN_REQUIRE(m->ctx, layer < m->cfg.num_layers && slot_begin + n <= kSlotsMax, "layer/slot range out of bounds");
    const auto &l = m->L[layer];
    const size_t row = l.kvd;
    CHN_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    if (k_in) CHN_HIP(m->ctx, hipMemcpy(l.kc + slot_begin * row, k_in, n * row * 4, hipMemcpyHostToDevice));
    if (v_in) CHN_HIP(m->ctx, hipMemcpy(l.vc + slot_begin * row, v_in, n * row * 4, hipMemcpyHostToDevice));
    return CHN_OK;
}

// GpuEngine.submitPreRecorded(cmd_buf_decode) (src/gpu/kernels.zig:189-194,
// as src/model/bench.zig:12-15 calls it): one more run of the recorded decode
// step on the inputs already on the device -- the stream x, the slot lists
// and the step parameters the last decode call left there -- then a wait, as
// the reference waits on its fence.
extern "C" int chn_model_replay(chn_model *m, int with_logits, uint32_t *topk_ids, float *topk_vals) {
    if (!m) return CHN_E_INVALID;
    chn_ctx *ctx = m->ctx;
    hipStream_t s = ctx->stream;
    const bool wl = with_logits != 0;
    CHN_REQUIRE(ctx, wl || (!topk_ids && !topk_vals), "the step without logits has no top-64");
    if (m->use_graph) {
        CHN_HIP(ctx, hipGraphLaunch(m->exec[wl ? 1 : 0], s));
    } else {
        int rc = record_decode(m, wl);
        if (rc) return rc;
    }
    if (topk_ids) CHN_HIP(ctx, hipMemcpyAsync(m->h_ids, m->topk_ids, 64 * 4, hipMemcpyDeviceToHost, s));
    if (topk_vals) CHN_HIP(ctx, hipMemcpyAsync(m->h_vals, m->topk_vals, 64 * 4, hipMemcpyDeviceToHost, s));
    CHN_HIP(ctx, hipStreamSynchronize(s));
    if (topk_ids) std::memcpy(topk_ids, m->h_ids, 64 * 4);
    if (topk_vals) std::memcpy(topk_vals, m->h_vals, 64 * 4);
    return CHN_OK;
}

// Reads of buf_logits through asSlice (src/gpu/model_gpu.zig:30-216; zeroed
// by src/server.zig:77): the logits of the last step or prefill that
// computed them (vocab floats, fp32).
extern "C" int chn_model_read_logits(chn_model *m, float *logits_out) {
    if (!m || !logits_out) return m ? set_err(m->ctx, CHN_E_INVALID, "logits_out is NULL") : CHN_E_INVALID;
    CHN_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    CHN_HIP(m->ctx, hipMemcpy(logits_out, m->logits, (size_t)m->cfg.vocab_size * 4, hipMemcpyDeviceToHost));
    return CHN_OK;
}

// Device buffers the reference's host code reads through asSlice under UMA
// (src/server/decode.zig:13, src/server/prefill.zig:92-93): hidden state x
// and the last normed row.
extern "C" int chn_model_read_state(chn_model *m, float *x_out, float *normed_out) {
    if (!m) return CHN_E_INVALID;
    CHN_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
    if (x_out) CHN_HIP(m->ctx, hipMemcpy(x_out, m->x, m->cfg.hidden_size * 4, hipMemcpyDeviceToHost));
    if (normed_out) CHN_HIP(m->ctx, hipMemcpy(normed_out, m->normed, m->cfg.hidden_size * 4, hipMemcpyDeviceToHost));
    return CHN_OK;
}
