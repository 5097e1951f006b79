"""Model-level restatement of the reference's GPU decode and prefill
sequences, composed from the oracle primitives.  TEST INFRASTRUCTURE ONLY.

decode_step follows recordLayerDirect / recordForwardGraph
(src/gpu/model_dispatch.zig:10-45,103-126) and gpuDispatchForwardToken
(:128-153); prefill follows gpuDispatchPrefillBatch
(src/gpu/batch_dispatch.zig:27-172).  Weights are quantized from the same
bf16 tensors with the oracle's quantizers (src/quant.zig:21-98).
"""
import numpy as np

import oracle as O


def bf16_to_f32(b):
    return (np.asarray(b, np.uint32) << 16).view(np.float32)


def layer_shape(cfg, i):
    """(D, num_kv_heads, rotary_dim) of layer i: full-attention layers take
    global_head_dim / num_global_kv_heads when set and rotate the whole head
    (src/model/loader.zig:37-41)."""
    full = bool(cfg["layer_full"][i])
    D, nkv, rot = cfg["head_dim"], cfg["num_kv_heads"], cfg["rotary_dim"]
    if full and cfg.get("global_head_dim"):
        D = rot = cfg["global_head_dim"]
    if full and cfg.get("num_global_kv_heads"):
        nkv = cfg["num_global_kv_heads"]
    return D, nkv, rot


class Weights:
    """Quantized / fp32 copies of a model given as bf16 arrays (dict per layer
    with keys q_proj, k_proj, v_proj, o_proj, gate_proj, up_proj, down_proj,
    input_layernorm, q_norm, k_norm, post_attention_layernorm,
    pre_feedforward_layernorm, post_feedforward_layernorm, layer_scalar)."""

    def __init__(self, cfg, layers, embed_bf16, final_norm_bf16):
        self.cfg = cfg
        H = cfg["hidden_size"]
        self.layers = []
        for i, l in enumerate(layers):
            D, nkv, rot = layer_shape(cfg, i)

            def norm(key, n):
                v = l.get(key)
                return np.ones(n, np.float32) if v is None else bf16_to_f32(v).astype(np.float32)
            d = {
                "Wq": O.quantize_q4(l["q_proj"]), "Wk": O.quantize_q4(l["k_proj"]),
                "Wv": O.quantize_q4(l["v_proj"] if l.get("v_proj") is not None else l["k_proj"]),
                "Wo": O.quantize_q4(l["o_proj"]), "Wg": O.quantize_q4(l["gate_proj"]),
                "Wu": O.quantize_q4(l["up_proj"]), "Wd": O.quantize_q4(l["down_proj"]),
                "in_norm": norm("input_layernorm", H), "q_norm": norm("q_norm", D),
                "k_norm": norm("k_norm", D), "pre_ffn": norm("pre_feedforward_layernorm", H),
                "post_attn": None if l.get("post_attention_layernorm") is None
                else norm("post_attention_layernorm", H),
                "post_ffn": None if l.get("post_feedforward_layernorm") is None
                else norm("post_feedforward_layernorm", H),
                "scalar": np.float32(l.get("layer_scalar", 1.0)),
                "D": D, "nkv": nkv, "rot": rot,
            }
            self.layers.append(d)
        self.embed_bf16 = embed_bf16
        self.embed_q8 = O.quantize_q8(embed_bf16)
        self.final_norm = (np.ones(H, np.float32) if final_norm_bf16 is None
                           else bf16_to_f32(final_norm_bf16).astype(np.float32))

    @classmethod
    def synthetic(cls, cfg, seed, embed_bf16, nthreads=1):
        """The weights chn_model_create_synthetic generates from `seed`:
        layer i's matrices q, k, v, o, gate, up, down from orc_synth_q4 with
        seeds seed + 64 (i + 1) + 0..6 (codes uniform, f16 scales
        U(0.005, 0.02)), every norm 1.0 (post-attention and post-FFN norms
        present), layer scalar 1.0; the tied embedding is given (bf16 bits)
        and quantized to Q8 here."""
        self = cls.__new__(cls)
        self.cfg = cfg
        H, I = cfg["hidden_size"], cfg["intermediate_size"]
        self.layers = []
        for i in range(cfg["num_layers"]):
            D, nkv, rot = layer_shape(cfg, i)
            qd, kvd = cfg["num_heads"] * D, nkv * D
            ls = seed + 64 * (i + 1)
            shapes = [("Wq", qd, H), ("Wk", kvd, H), ("Wv", kvd, H), ("Wo", H, qd),
                      ("Wg", I, H), ("Wu", I, H), ("Wd", H, I)]
            d = {name: O.synth_q4(r, k, ls + j).reshape(r, -1) for j, (name, r, k) in enumerate(shapes)}
            ones_h = np.ones(H, np.float32)
            d.update({"in_norm": ones_h, "q_norm": np.ones(D, np.float32), "k_norm": np.ones(D, np.float32),
                      "pre_ffn": ones_h, "post_attn": ones_h, "post_ffn": ones_h, "scalar": np.float32(1.0),
                      "D": D, "nkv": nkv, "rot": rot})
            self.layers.append(d)
        self.embed_bf16 = np.asarray(embed_bf16, np.uint16).reshape(cfg["vocab_size"], H)
        self.embed_q8 = O.quantize_q8(self.embed_bf16, nthreads)
        self.final_norm = np.ones(H, np.float32)
        return self

    def embed(self, tokens):
        """x = bf16(embed[tok]) * sqrt(H) (src/model/forward.zig:35-37,
        src/gpu/batch_dispatch.zig:14-23)."""
        H = self.cfg["hidden_size"]
        s = np.sqrt(np.float32(H))
        return (bf16_to_f32(self.embed_bf16[np.asarray(tokens)]) * s).astype(np.float32)


def new_caches(cfg, nslot=4096):
    kvds = [layer_shape(cfg, i)[0] * layer_shape(cfg, i)[1] for i in range(cfg["num_layers"])]
    return ([np.zeros(nslot * k, np.float32) for k in kvds],
            [np.zeros(nslot * k, np.float32) for k in kvds])


class QuiescenceState:
    """What the reference's GPU model keeps across decode steps for
    quiescence gating (src/gpu/model_gpu.zig:131, model_dispatch.zig:47-126):
    per layer the input stream at the previous gated step (buf_x_prev,
    zero-initialised) and the normed row buf_normed_x, which a quiescent
    layer leaves as it was.  `log` collects per step the (layer, runs, mean
    square) of every gate."""

    def __init__(self, cfg, thresh):
        H = cfg["hidden_size"]
        self.thresh = float(thresh)
        self.x_prev = [np.zeros(H, np.float32) for _ in range(cfg["num_layers"])]
        self.normed = np.zeros(H, np.float32)
        self.log = []


def decode_step(W, kc, vc, x, clock, slot_idx, active, sliding, with_logits=True, nthreads=1, qstate=None):
    """One token through every layer; kc / vc (per-layer flat arrays) are
    updated in place.  Returns (x, normed, logits, ids, vals).  nthreads > 1
    uses the threaded matvecs (bit-identical results).  With a
    QuiescenceState whose threshold is positive, the steps with logits gate
    layers from num_layers / 3 on (recordLayerIndirect): the gate compares
    the stream with the layer's previous one, and a quiescent layer runs
    nothing (the stream, the normed row and its K/V slot keep their values);
    a running one starts from its own input norm."""
    c = W.cfg
    H, I = c["hidden_size"], c["intermediate_size"]
    nq, eps = c["num_heads"], c["rms_norm_eps"]
    x = np.array(x, np.float32)
    gate_on = with_logits and qstate is not None and qstate.thresh > 0.0
    dense = c["num_layers"] // 3
    normed = qstate.normed.copy() if qstate is not None else None
    gates = []
    for i, l in enumerate(W.layers):
        if gate_on and i >= dense:
            runs, ms = O.quiescence_gate(x, qstate.x_prev[i], qstate.thresh)
            gates.append((i, runs, ms))
            if not runs:
                continue
            normed = O.rmsnorm(x, l["in_norm"], eps)
        elif i == 0:
            normed = O.rmsnorm(x, l["in_norm"], eps)
        full = bool(c["layer_full"][i])
        theta = c["rope_theta_full"] if full else c["rope_theta"]
        D, nkv = l["D"], l["nkv"]
        qd, kvd = nq * D, nkv * D
        q, k, v = O.fused_qkv_q4(l["Wq"], l["Wk"], l["Wv"], normed, qd, kvd, H, nthreads)
        q = O.qkv_rope(q, k, v, l["q_norm"], l["k_norm"], kc[i], vc[i], nq, nkv, D, l["rot"],
                       c["k_eq_v"], theta, eps, clock, slot_idx)
        slots = np.asarray(active if full else sliding, np.uint32)
        attn = O.decode_attn(q, kc[i], vc[i], slots, nq, D, kvd, nq // nkv, 1.0)
        o = O.gemv_q4(l["Wo"], attn, H, qd, nthreads)
        if l["post_attn"] is not None:
            o = O.rmsnorm(o, l["post_attn"], eps)
        x, normed = O.add_rmsnorm(x, o, l["pre_ffn"], eps, 1.0)
        act = O.fused_mlp_q4(l["Wg"], l["Wu"], normed, I, H, nthreads)
        d = O.gemv_q4(l["Wd"], act, H, I, nthreads)
        if l["post_ffn"] is not None:
            d = O.rmsnorm(d, l["post_ffn"], eps)
        nxt = W.layers[i + 1]["in_norm"] if i + 1 < len(W.layers) else W.final_norm
        x, normed = O.add_rmsnorm(x, d, nxt, eps, float(l["scalar"]))
    if qstate is not None:
        qstate.normed = normed.copy()
        qstate.log.append(gates)
    logits = ids = vals = None
    if with_logits:
        logits = O.gemv_q8(W.embed_q8, normed, c["vocab_size"], H, nthreads)
        ids, vals = O.topk64(logits)
    return x, normed, logits, ids, vals


def _rows(fn, X, *args):
    return np.stack([fn(X[t], *args) for t in range(X.shape[0])]).astype(np.float32)


def prefill(W, kc, vc, tokens, slots, start_clock, num_prev, bf16_gemm=True, window=1024, nthreads=1):
    """gpuDispatchPrefillBatch; GEMMs use the bf16-operand model of the MFMA
    path when bf16_gemm (else fp32).  Returns (X, Xn, logits, ids, vals)."""
    c = W.cfg
    H, I = c["hidden_size"], c["intermediate_size"]
    nq, eps = c["num_heads"], c["rms_norm_eps"]
    n = len(tokens)
    if bf16_gemm:
        def gemm(Wm, X, nt, M, K):
            return O.batch_gemm_q4_bf16(Wm, X, nt, M, K, nthreads)
    else:
        gemm = O.batch_gemm_q4
    slots = np.asarray(slots, np.uint32)
    X = W.embed(tokens)
    Xn = _rows(O.rmsnorm, X, W.layers[0]["in_norm"], eps)
    for i, l in enumerate(W.layers):
        full = bool(c["layer_full"][i])
        theta = c["rope_theta_full"] if full else c["rope_theta"]
        D, nkv = l["D"], l["nkv"]
        qd, kvd = nq * D, nkv * D
        Q = gemm(l["Wq"], Xn, n, qd, H)
        K = gemm(l["Wk"], Xn, n, kvd, H)
        V = gemm(l["Wv"], Xn, n, kvd, H)
        Qr = np.zeros_like(Q)
        for t in range(n):
            Qr[t] = O.qkv_rope(Q[t], K[t], V[t], l["q_norm"], l["k_norm"], kc[i], vc[i], nq, nkv, D,
                               l["rot"], c["k_eq_v"], theta, eps, start_clock + t,
                               int(slots[num_prev + t]))
        A = O.batch_causal_attn(Qr, kc[i], vc[i], slots, n, num_prev, nq, D, kvd, nq // nkv, 1.0,
                                0 if full else window, nthreads).reshape(n, qd)
        Om = gemm(l["Wo"], A, n, H, qd)
        if l["post_attn"] is not None:
            Om = _rows(O.rmsnorm, Om, l["post_attn"], eps)
        Xs, Xn = zip(*[O.add_rmsnorm(X[t], Om[t], l["pre_ffn"], eps, 1.0) for t in range(n)])
        X, Xn = np.stack(Xs), np.stack(Xn)
        if bf16_gemm:
            G = gemm(l["Wg"], Xn, n, I, H)
            U = gemm(l["Wu"], Xn, n, I, H)
            Act = (O.gelu_tanh(G.ravel()).reshape(G.shape) * U).astype(np.float32)
        else:
            Act = O.batch_fused_mlp_q4(l["Wg"], l["Wu"], Xn, n, I, H)
        Dn = gemm(l["Wd"], Act, n, H, I)
        if l["post_ffn"] is not None:
            Dn = _rows(O.rmsnorm, Dn, l["post_ffn"], eps)
        nxt = W.layers[i + 1]["in_norm"] if i + 1 < len(W.layers) else W.final_norm
        Xs, Xn = zip(*[O.add_rmsnorm(X[t], Dn[t], nxt, eps, float(l["scalar"])) for t in range(n)])
        X, Xn = np.stack(Xs), np.stack(Xn)
    logits = O.gemv_q8(W.embed_q8, Xn[n - 1], c["vocab_size"], H, nthreads)
    ids, vals = O.topk64(logits)
    return X, Xn, logits, ids, vals


def random_bf16(shape, seed, std):
    """bf16 bits of N(0, std^2) values (nearest even)."""
    rng = np.random.default_rng(seed)
    return _bf16_round((rng.standard_normal(shape) * std).astype(np.float32))


def _bf16_round(v):
    u = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def random_model(cfg, seed):
    """Random bf16 weights: projections ~ N(0, 0.05^2), norms 1 + N(0, 0.1^2)
    (q/k norms a quarter of that, so that unit-scale q.k scores stay O(1)
    as trained q/k norms keep them), embedding ~ N(0, 0.02^2); even layers
    carry a post-FFN norm, odd layers a layer scalar of 0.75."""
    H, I = cfg["hidden_size"], cfg["intermediate_size"]

    def nrm(n, s, base=1.0):
        return _bf16_round((bf16_to_f32(random_bf16((n,), s, 0.1)) + np.float32(1.0)) * np.float32(base))

    layers = []
    for i in range(cfg["num_layers"]):
        s = seed + 100 * i
        D, nkv, _ = layer_shape(cfg, i)
        qd, kvd = cfg["num_heads"] * D, nkv * D
        layers.append({
            "q_proj": random_bf16((qd, H), s + 1, 0.05), "k_proj": random_bf16((kvd, H), s + 2, 0.05),
            "v_proj": random_bf16((kvd, H), s + 3, 0.05), "o_proj": random_bf16((H, qd), s + 4, 0.05),
            "gate_proj": random_bf16((I, H), s + 5, 0.05), "up_proj": random_bf16((I, H), s + 6, 0.05),
            "down_proj": random_bf16((H, I), s + 7, 0.05),
            "input_layernorm": nrm(H, s + 8), "q_norm": nrm(D, s + 9, 0.25), "k_norm": nrm(D, s + 10, 0.25),
            "post_attention_layernorm": nrm(H, s + 11), "pre_feedforward_layernorm": nrm(H, s + 12),
            "post_feedforward_layernorm": nrm(H, s + 13) if i % 2 == 0 else None,
            "layer_scalar": 1.0 if i % 2 == 0 else 0.75,
        })
    embed = random_bf16((cfg["vocab_size"], H), seed + 7, 0.02)
    return layers, embed, nrm(H, seed + 9)


def default_config(**kw):
    c = dict(hidden_size=3840, intermediate_size=15360, vocab_size=262144, num_layers=48,
             num_heads=16, num_kv_heads=8, head_dim=256, rotary_dim=256, global_head_dim=0,
             num_global_kv_heads=0, rms_norm_eps=1e-6,
             rope_theta=1e4, rope_theta_full=1e6, sliding_window=512, k_eq_v=0,
             max_prefill_tokens=1024)
    c.update(kw)
    if "layer_full" not in c:
        c["layer_full"] = [1 if (l + 1) % 5 == 0 else 0 for l in range(c["num_layers"])]
    return c


def slot_lists(clock, window):
    """Chronological slot lists with slot = clock (no wrap): the full list
    and the sliding window (the shape getActiveSlotsLayer gives for a
    context without anchors that has not wrapped, src/ring_buffer.zig:287-333)."""
    active = np.arange(clock + 1, dtype=np.uint32)
    sliding = active[max(0, clock + 1 - window):]
    return active, sliding

