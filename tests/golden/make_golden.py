"""Writes tests/golden/golden.npz: small input/output vectors for the hot
path, computed by an independent numpy restatement of the reference
semantics (float64 where the reference computes in fp32, float32 where the
reference's rounding steps are part of the result).

It does not import the oracle: the fixtures check the oracle (and, through
it, the GPU path) against a second, separately written computation.  The
reference ships no golden vectors for this path and its Zig implementation
cannot be built here; every formula below cites the reference line it
follows.

    python tests/golden/make_golden.py      # rewrites golden.npz
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "golden.npz")


# ---- scalar formats -------------------------------------------------------

def bf16_bits(v):
    """bf16.fromF32 (src/tensor.zig:7-13): round to nearest even on the bits."""
    u = np.asarray(v, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(b):
    return (np.asarray(b, np.uint32) << 16).view(np.float32)


def f16_bits(v):
    """@floatCast(f32 -> f16): IEEE round to nearest even."""
    return np.asarray(v, np.float32).astype(np.float16).view(np.uint16)


def round_away(t):
    """std.math.round: halves away from zero."""
    t = np.asarray(t, np.float64)
    return np.sign(t) * np.floor(np.abs(t) + 0.5)


# ---- quantizers (src/quant.zig:21-98) ---------------------------------------

def quant_q4(w_bf16):
    rows, cols = w_bf16.shape
    out = np.zeros((rows, cols // 32 * 5), np.uint32)
    for r in range(rows):
        for b in range(cols // 32):
            v = bf16_to_f32(w_bf16[r, 32 * b:32 * b + 32])
            amax = np.float32(np.max(np.abs(v)))
            d = np.float32(amax / np.float32(8.0))
            idv = np.float32(np.float32(1.0) / d) if d > 0 else np.float32(0.0)
            word0 = int(f16_bits(d)) | (int(f16_bits(np.float32(-8.0) * d)) << 16)
            t = (v * idv).astype(np.float32) + np.float32(8.0)
            q = np.clip(round_away(t.astype(np.float32)), 0, 15).astype(np.uint32)
            out[r, 5 * b] = word0
            for w in range(4):
                word = 0
                for n in range(8):
                    word |= int(q[8 * w + n]) << (4 * n)
                out[r, 5 * b + 1 + w] = word
    return out


def quant_q8(w_bf16):
    rows, cols = w_bf16.shape
    out = np.zeros((rows, cols // 32 * 9), np.uint32)
    for r in range(rows):
        for b in range(cols // 32):
            v = bf16_to_f32(w_bf16[r, 32 * b:32 * b + 32])
            amax = np.float32(np.max(np.abs(v)))
            d = np.float32(amax / np.float32(127.0))
            idv = np.float32(np.float32(127.0) / amax) if amax > 0 else np.float32(0.0)
            q = np.clip(round_away((v * idv).astype(np.float32)), -128, 127).astype(np.int64)
            out[r, 9 * b] = np.float32(d).view(np.uint32)
            by = (q & 0xFF).astype(np.uint32)
            for w in range(8):
                out[r, 9 * b + 1 + w] = (by[4 * w] | (by[4 * w + 1] << 8) | (by[4 * w + 2] << 16)
                                         | (by[4 * w + 3] << 24))
    return out


def deq_q4(W, rows, K):
    """(q - 8) * f16 scale, min half ignored (shaders/gemv_q4.wgsl:15-26)."""
    out = np.zeros((rows, K), np.float64)
    for r in range(rows):
        for b in range(K // 32):
            s = np.uint16(W[r, 5 * b] & 0xFFFF).view(np.float16).astype(np.float64)
            for w in range(4):
                word = int(W[r, 5 * b + 1 + w])
                for n in range(8):
                    out[r, 32 * b + 8 * w + n] = s * (((word >> (4 * n)) & 15) - 8)
    return out


def deq_q8(W, rows, K):
    out = np.zeros((rows, K), np.float64)
    for r in range(rows):
        for b in range(K // 32):
            s = np.uint32(W[r, 9 * b]).view(np.float32).astype(np.float64)
            for i in range(32):
                byte = (int(W[r, 9 * b + 1 + i // 4]) >> (8 * (i % 4))) & 0xFF
                out[r, 32 * b + i] = s * (byte - 256 if byte >= 128 else byte)
    return out


# ---- layer arithmetic in float64 ----------------------------------------------

def gelu_tanh(x):
    """src/kernels.zig:7-10 = shaders/fused_mlp_q4.wgsl:15-18."""
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + np.tanh(0.7978845608 * (x + 0.044715 * x ** 3)))


def rmsnorm(x, w, eps):
    """x * 1/sqrt(mean(x^2) + eps) * w (shaders/rmsnorm.wgsl)."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x) + eps) * np.asarray(w, np.float64)


def rope_angles(rot, theta, clock):
    """freq = 1/pow(theta, 2d/rot) and angle = f32(clock) * freq, both in
    fp32 as the shader computes them (shaders/qkv_rope.wgsl:74-78); pow is
    the correctly rounded fp32 result (computed in fp64, rounded once)."""
    d = np.arange(rot // 2, dtype=np.float32)
    fe = (np.float32(2.0) * d) / np.float32(rot)
    pw = np.power(np.float64(np.float32(theta)), fe.astype(np.float64)).astype(np.float32)
    freq = (np.float32(1.0) / pw).astype(np.float32)
    return (np.float32(clock) * freq).astype(np.float32).astype(np.float64)


def norm_rope(v, w, rot, theta, eps, clock):
    """Per-head RMSNorm * w, then rotation of pairs (d, d + rot/2)."""
    n = rmsnorm(v, w, eps)
    half = rot // 2
    a = rope_angles(rot, theta, clock)
    out = n.copy()
    out[:half] = n[:half] * np.cos(a) - n[half:rot] * np.sin(a)
    out[half:rot] = n[:half] * np.sin(a) + n[half:rot] * np.cos(a)
    return out


def attend(q, K, V):
    """p = exp(s - max) / (sum + 1e-9), out = sum p V (decode_attn.wgsl)."""
    s = K @ q
    m = max(np.max(s), -1e9)
    e = np.exp(s - m)
    return (e / (np.sum(e) + 1e-9)) @ V


def softcap(v):
    """30 * tanh(v / 30) (shaders/topk_pass1.wgsl:17-19)."""
    return 30.0 * np.tanh(np.asarray(v, np.float64) / 30.0)


# ---- fixtures -------------------------------------------------------------------

def main():
    rng = np.random.default_rng(20260101)
    g = {}

    # Q4 / Q8 pack of 4 x 64 with ties, zeros and a spike
    w = (rng.standard_normal((4, 64)) * 0.05).astype(np.float32)
    w[1, :32] = 0.0
    w[2, 32:] = np.linspace(-1.0, 1.0, 32, dtype=np.float32)
    w[3, 7] = 3.0
    wb = bf16_bits(w)
    g["pack_in_bf16"] = wb
    g["pack_q4"] = quant_q4(wb)
    g["pack_q8"] = quant_q8(wb)

    # GEMV 16 x 256
    wg = bf16_bits(rng.standard_normal((16, 256)) * 0.05)
    Wq = quant_q4(wg)
    x = rng.standard_normal(256).astype(np.float32)
    g["gemv_W"], g["gemv_x"] = Wq, x
    g["gemv_y"] = deq_q4(Wq, 16, 256) @ x.astype(np.float64)

    # fused MLP 32 x 128
    Wg = quant_q4(bf16_bits(rng.standard_normal((32, 128)) * 0.05))
    Wu = quant_q4(bf16_bits(rng.standard_normal((32, 128)) * 0.05))
    xm = rng.standard_normal(128).astype(np.float32)
    g["mlp_Wg"], g["mlp_Wu"], g["mlp_x"] = Wg, Wu, xm
    gg = deq_q4(Wg, 32, 128) @ xm.astype(np.float64)
    uu = deq_q4(Wu, 32, 128) @ xm.astype(np.float64)
    g["mlp_act"] = gelu_tanh(gg) * uu

    # Q8 logits 64 x 128
    E = quant_q8(bf16_bits(rng.standard_normal((64, 128)) * 0.02))
    xe = rng.standard_normal(128).astype(np.float32)
    g["q8_W"], g["q8_x"] = E, xe
    g["q8_y"] = deq_q8(E, 64, 128) @ xe.astype(np.float64)

    # decode attention: 4 query heads, 2 KV heads, D = 256, 64 of 80 slots
    nq, nkv, D, nslot = 4, 2, 256, 80
    kvd = nkv * D
    Kc = rng.standard_normal((nslot, kvd)).astype(np.float32)
    Vc = rng.standard_normal((nslot, kvd)).astype(np.float32)
    q = (rng.standard_normal(nq * D) * 0.1).astype(np.float32)
    slots = rng.permutation(nslot)[:64].astype(np.uint32)
    out = np.zeros(nq * D)
    for h in range(nq):
        kh = h // (nq // nkv)
        Ks = Kc[slots, kh * D:(kh + 1) * D].astype(np.float64)
        Vs = Vc[slots, kh * D:(kh + 1) * D].astype(np.float64)
        out[h * D:(h + 1) * D] = attend(q[h * D:(h + 1) * D].astype(np.float64), Ks, Vs)
    g["attn_q"], g["attn_K"], g["attn_V"], g["attn_slots"], g["attn_out"] = q, Kc, Vc, slots, out

    # qkv_rope at clock 4095, theta 1e6: 2 query heads, 1 KV head, D = 256
    qi = rng.standard_normal(2 * D).astype(np.float32)
    ki = rng.standard_normal(D).astype(np.float32)
    vi = rng.standard_normal(D).astype(np.float32)
    qw = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    kw = (1.0 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    g["rope_q"], g["rope_k"], g["rope_v"], g["rope_qw"], g["rope_kw"] = qi, ki, vi, qw, kw
    g["rope_q_out"] = np.concatenate([norm_rope(qi[h * D:(h + 1) * D], qw, D, 1e6, 1e-6, 4095)
                                      for h in range(2)])
    g["rope_k_out"] = norm_rope(ki, kw, D, 1e6, 1e-6, 4095)
    g["rope_v_out"] = rmsnorm(vi, np.ones(D), 1e-6)
    # partial rotary (rot 128) at clock 7, theta 1e4
    g["rope_q_out_rot128"] = np.concatenate([norm_rope(qi[h * D:(h + 1) * D], qw, 128, 1e4, 1e-6, 7)
                                             for h in range(2)])

    # top-64 of softcapped logits with ties (ties: lower index first)
    lg = (rng.standard_normal(8192) * 8).astype(np.float32)
    lg[[5, 4000, 8191]] = np.float32(40.0)
    lg[[17, 8000]] = np.float32(300.0)
    capped = softcap(lg)
    order = sorted(range(8192), key=lambda i: (-capped[i], i))[:64]
    g["topk_logits"], g["topk_ids"] = lg, np.array(order, np.uint32)
    g["topk_vals"] = capped[order]

    # norms: rmsnorm and add_rmsnorm with scalar 0.75 at 3840
    xn = rng.standard_normal(3840).astype(np.float32)
    rn = rng.standard_normal(3840).astype(np.float32)
    wn = (1.0 + 0.1 * rng.standard_normal(3840)).astype(np.float32)
    g["norm_x"], g["norm_r"], g["norm_w"] = xn, rn, wn
    g["norm_y"] = rmsnorm(xn, wn, 1e-6)
    xs = (xn.astype(np.float64) + rn) * 0.75
    g["addnorm_x"], g["addnorm_y"] = xs, rmsnorm(xs, wn, 1e-6)

    np.savez_compressed(OUT, **g)
    print(f"wrote {OUT}: {len(g)} arrays, {os.path.getsize(OUT)} bytes")


if __name__ == "__main__":
    main()
