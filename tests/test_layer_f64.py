"""An independent float64 restatement of the decode step, written from the
reference's CPU forward pass (src/model/forward.zig:19-167) and its kernels
(src/kernels.zig:7-10 geluTanh, :18-33 rmsNorm / unitRmsNorm, :101-119
applyRopePartial, :121-133 softmax), over the weights the GPU path holds:
the projections dequantized from Q4 (scale * (q - 8)) and the logits over
the Q8 embedding (shaders/gemv_q8.wgsl).  oracle/model.py's decode_step
composes the oracle's C kernels in the GPU dispatch order
(src/gpu/model_dispatch.zig:10-45); the two must agree to fp32 rounding
over several steps in x, the normed row, every K/V row written and the
logits.  This pins the layer composition (norm placement, the residual and
layer-scalar order, the partial RoPE pairing, the GQA head mapping, V's
unit norm, the sliding and full lists) with code that shares none of the
oracle's."""
import numpy as np

import oracle as O
from oracle import model as OM


def _rms(v, w, eps):
    return v / np.sqrt(np.mean(v * v) + eps) * w


def _rope(v, pos, D, rot, theta):
    """applyRopePartial on one head (pairs i, i + rot / 2 for i < rot / 2)."""
    out = v.copy()
    half = rot // 2
    i = np.arange(half, dtype=np.float64)
    ang = pos / np.power(theta, 2.0 * i / rot)
    c, s = np.cos(ang), np.sin(ang)
    out[:half] = v[:half] * c - v[half:rot] * s
    out[half:rot] = v[:half] * s + v[half:rot] * c
    return out


def _gelu(x):
    return 0.5 * x * (1.0 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))


def _step64(W, deq, kc, vc, x, clock, slot, active, sliding):
    c = W.cfg
    H, nq, eps = c["hidden_size"], c["num_heads"], c["rms_norm_eps"]
    for i, l in enumerate(W.layers):
        D, nkv, rot = l["D"], l["nkv"], l["rot"]
        full = bool(c["layer_full"][i])
        theta = c["rope_theta_full"] if full else c["rope_theta"]
        Wq, Wk, Wv, Wo, Wg, Wu, Wd = deq[i]
        xn = _rms(x, l["in_norm"], eps)
        q, k, v = Wq @ xn, Wk @ xn, Wv @ xn
        q = np.concatenate([_rope(_rms(q[h * D:(h + 1) * D], l["q_norm"], eps), clock, D, rot, theta)
                            for h in range(nq)])
        k = np.concatenate([_rope(_rms(k[h * D:(h + 1) * D], l["k_norm"], eps), clock, D, rot, theta)
                            for h in range(nkv)])
        v = np.concatenate([_rms(v[h * D:(h + 1) * D], 1.0, eps) for h in range(nkv)])
        kc[i][slot], vc[i][slot] = k, v
        lst = np.asarray(active if full else sliding)
        attn = np.zeros(nq * D)
        for h in range(nq):
            kvh = h // (nq // nkv)
            Ks, Vs = kc[i][lst, kvh * D:(kvh + 1) * D], vc[i][lst, kvh * D:(kvh + 1) * D]
            s = Ks @ q[h * D:(h + 1) * D]
            p = np.exp(s - s.max())
            attn[h * D:(h + 1) * D] = (p / p.sum()) @ Vs
        o = Wo @ attn
        if l["post_attn"] is not None:
            o = _rms(o, l["post_attn"], eps)
        x = x + o
        xn2 = _rms(x, l["pre_ffn"], eps)
        d = Wd @ (_gelu(Wg @ xn2) * (Wu @ xn2))
        if l["post_ffn"] is not None:
            d = _rms(d, l["post_ffn"], eps)
        x = (x + d) * float(l["scalar"])
    normed = _rms(x, W.final_norm, eps)
    return x, normed


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def test_decode_steps_match_float64_restatement():
    cfg = OM.default_config(hidden_size=128, intermediate_size=256, vocab_size=512, num_layers=3,
                            num_heads=4, num_kv_heads=2, head_dim=64, rotary_dim=32, layer_full=[0, 1, 0],
                            sliding_window=3, max_prefill_tokens=16)
    layers, embed, final = OM.random_model(cfg, 23)
    W = OM.Weights(cfg, layers, embed, final)
    H, I, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["vocab_size"]
    deq = []
    for l in W.layers:
        qd, kvd = cfg["num_heads"] * l["D"], l["nkv"] * l["D"]
        deq.append([O.dequant_q4(l["Wq"], qd, H).astype(np.float64), O.dequant_q4(l["Wk"], kvd, H).astype(np.float64),
                    O.dequant_q4(l["Wv"], kvd, H).astype(np.float64), O.dequant_q4(l["Wo"], H, qd).astype(np.float64),
                    O.dequant_q4(l["Wg"], I, H).astype(np.float64), O.dequant_q4(l["Wu"], I, H).astype(np.float64),
                    O.dequant_q4(l["Wd"], H, I).astype(np.float64)])
    E8 = O.dequant_q8(W.embed_q8, V, H).astype(np.float64)
    nslot = 16
    kc32, vc32 = OM.new_caches(cfg, nslot)
    kvds = [l["nkv"] * l["D"] for l in W.layers]
    kc64 = [np.zeros((nslot, d)) for d in kvds]
    vc64 = [np.zeros((nslot, d)) for d in kvds]
    toks = [5, 300, 17, 42, 511, 0, 99]
    for t, tok in enumerate(toks):
        active, sliding = OM.slot_lists(t, cfg["sliding_window"])
        x_in = W.embed([tok])[0]
        x32, n32, lg32, _, _ = OM.decode_step(W, kc32, vc32, x_in, t, t, active, sliding)
        x64, n64 = _step64(W, deq, kc64, vc64, x_in.astype(np.float64), t, t, active, sliding)
        assert _rel(x32, x64) < 2e-5, t
        assert _rel(n32, n64) < 2e-5, t
        assert _rel(lg32, E8 @ n64) < 2e-5, t
        for i, d in enumerate(kvds):
            assert _rel(kc32[i][t * d:(t + 1) * d], kc64[i][t]) < 2e-5, (t, i)
            assert _rel(vc32[i][t * d:(t + 1) * d], vc64[i][t]) < 2e-5, (t, i)
