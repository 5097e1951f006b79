"""Pins the CPU oracle before anything is compared against it.

Each test is chosen so that a plausible restatement mistake fails it: a wrong
rounding mode, a swapped nibble order, a dropped -8, a transposed operand, a
wrong RoPE pairing, a missing softmax max-shift.  Sources:
  * the reference's own known-answer data: src/gpu.zig:32-61 (Q4 GEMV on an
    all-1.0 matrix; the closed form y = 55.34375 is derived in the test) and
    src/tensor.zig:30-41 (bf16 round trip);
  * independent implementations: numpy's float16 conversion, float64
    brute-force contractions, complex-number rotation for RoPE;
  * mathematical invariants (zero codes, single non-zero, permutation and
    shift invariance of softmax attention, monotone softcap).
"""
import math

import numpy as np
import pytest

import oracle


def bf16_bits(a):
    """Nearest-even bf16 of float32 values, chosen by float64 distance."""
    a = np.asarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    lo = (u & 0xFFFF0000).astype(np.uint32)
    hi = (lo.astype(np.uint64) + 0x10000).astype(np.uint32)
    flo = lo.view(np.float32).astype(np.float64)
    fhi = hi.view(np.float32).astype(np.float64)
    x = a.astype(np.float64)
    dlo, dhi = np.abs(x - flo), np.abs(fhi - x)
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((lo >> 16) & 1 == 1))
    return np.where(pick_hi, hi >> 16, lo >> 16).astype(np.uint16)


def bf16_to_f32(b):
    return (np.asarray(b, np.uint32) << 16).view(np.float32)


def unpack_q4(W, rows, K):
    """Independent numpy unpack: f16 scale * (nibble - 8), float64."""
    blk = np.asarray(W, np.uint32).reshape(rows, K // 32, 5)
    scale = (blk[:, :, 0] & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float64)
    shifts = np.arange(8, dtype=np.uint32) * 4
    nib = (blk[:, :, 1:, None] >> shifts) & 0xF  # [rows, nb, 4 words, 8]
    q = nib.reshape(rows, K // 32, 32).astype(np.float64) - 8.0
    return (q * scale[:, :, None]).reshape(rows, K)


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-30))


# ---------------------------------------------------------------- scalars

def test_f16_matches_numpy_rne():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * 10,
        rng.uniform(-1e-5, 1e-5, 2000).astype(np.float32),      # f16 subnormals
        np.array([65504, 65520, 65519.99, 1e9, -1e9, 0.0, -0.0, 2**-24, 2**-25, 3 * 2**-26],
                 np.float32),
        # exact ties between two f16 neighbours
        (np.arange(1, 200, dtype=np.float32) * 2**-10 + 2**-12).astype(np.float32),
    ])
    got = oracle.f32_to_f16_bits(vals)
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_f16_to_f32_all_patterns():
    bits = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    finite = (bits & 0x7C00) != 0x7C00
    bits = bits[finite]
    got = oracle.f16_bits_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_bf16_reference_roundtrip_and_rne():
    # src/tensor.zig:30-41
    for v, tol in [(3.1415926, 0.02), (0.0, 0.0), (-42.5, 0.1)]:
        b = oracle.lib.orc_bf16_from_f32(v)
        assert abs(oracle.lib.orc_bf16_to_f32(b) - v) <= tol
    rng = np.random.default_rng(2)
    vals = np.concatenate([rng.standard_normal(5000).astype(np.float32),
                           bf16_to_f32(np.arange(0x3F80, 0x3FA0, dtype=np.uint16)) +
                           np.float32(2**-9)])  # includes exact ties
    assert np.array_equal(oracle.bf16_from_f32(vals), bf16_bits(vals))


# ---------------------------------------------------------------- Q4 format

def test_q4_kat_from_reference_gpu_test():
    """src/gpu.zig:38-60: 64x128 all-1.0 bf16 (0x3F80) quantized to Q4, x_i =
    (i mod 5)*0.25.  amax = 1 -> d = 0.125, every code = clamp(round(16)) =
    15, so w = 0.125*7 = 0.875 and y = 0.875 * sum(x) = 0.875 * 63.25 =
    55.34375 exactly for all 64 rows."""
    w = np.full((64, 128), 0x3F80, dtype=np.uint16)
    W = oracle.quantize_q4(w)
    blk = W.reshape(64, 4, 5)
    assert np.all(blk[:, :, 0] & 0xFFFF == 0x3000)          # f16(0.125)
    assert np.all(blk[:, :, 0] >> 16 == 0xBC00)             # f16(-1.0)
    assert np.all(blk[:, :, 1:] == 0xFFFFFFFF)              # all codes 15
    x = (np.arange(128) % 5).astype(np.float32) * 0.25
    y = oracle.gemv_q4(W, x, 64, 128)
    assert np.all(y == np.float32(55.34375))


def test_q4_nibble_position_probe():
    """One non-zero element per block: its code (15 or 0) must appear at word
    1 + j//8, nibble j%8; every other code is 8."""
    for j in range(32):
        for sign in (1.0, -1.0):
            row = np.zeros(32, np.float32)
            row[j] = sign * 3.0
            W = oracle.quantize_q4(bf16_bits(row)[None, :])[0]
            nibs = [(int(W[1 + i // 8]) >> (4 * (i % 8))) & 0xF for i in range(32)]
            want = [8] * 32
            want[j] = 15 if sign > 0 else 0
            assert nibs == want, (j, sign)


def test_q4_round_half_away_from_zero_and_clamp():
    """amax = 8 gives d = 1, id = 1: v*id + 8 hits exact .5 ties; Zig's
    std.math.round rounds them away from zero (RNE would differ at 10.5, 8.5)."""
    row = np.zeros(32, np.float32)
    row[:6] = [8.0, 2.5, 0.5, -2.5, -8.0, -0.5]
    W = oracle.quantize_q4(bf16_bits(row)[None, :])[0]
    nibs = [(int(W[1 + i // 8]) >> (4 * (i % 8))) & 0xF for i in range(32)]
    assert nibs[:6] == [15, 11, 9, 6, 0, 8]   # 16 clamps to 15; -0.5+8 = 7.5 -> 8
    assert W[0] & 0xFFFF == 0x3C00            # f16(1.0)


def test_q4_pack_unpack_roundtrip():
    rng = np.random.default_rng(3)
    vals = (rng.standard_normal((8, 256)) * 0.05).astype(np.float32)
    bits = bf16_bits(vals)
    v = bf16_to_f32(bits).astype(np.float64)
    W = oracle.quantize_q4(bits)
    deq = oracle.dequant_q4(W, 8, 256).astype(np.float64)
    assert np.allclose(deq, unpack_q4(W, 8, 256), rtol=0, atol=0)
    d = np.abs(v).reshape(8, 8, 32).max(axis=2) / 8.0
    err = np.abs(deq - v).reshape(8, 8, 32)
    # interior codes: |err| <= d/2, plus |q-8| <= 8 steps of the f16 scale's
    # rounding (8 * 2^-11 d).  Values above 7.5 d round to 16 and clamp to
    # 15 (error < d): the asymmetric top of the 0..15 code range.
    vb = v.reshape(8, 8, 32)
    dd = np.broadcast_to(d[:, :, None], err.shape)
    clamped = vb >= 7.5 * dd * (1 - 1e-6)
    assert np.all(err[~clamped] <= dd[~clamped] * (0.5 + 2**-7) + 1e-12)
    assert np.all(err[clamped] <= dd[clamped] * (1 + 2**-7))
    assert clamped.any()


def test_q8_pack_roundtrip_and_scale_word():
    rng = np.random.default_rng(4)
    vals = (rng.standard_normal((4, 128)) * 0.1).astype(np.float32)
    bits = bf16_bits(vals)
    v = bf16_to_f32(bits)
    W = oracle.quantize_q8(bits)
    blk = W.reshape(4, 4, 9)
    amax = np.abs(v).reshape(4, 4, 32).max(axis=2)
    assert np.array_equal(blk[:, :, 0].view(np.float32), (amax / np.float32(127.0)))
    deq = oracle.dequant_q8(W, 4, 128)
    d = (amax / 127.0)[:, :, None]
    assert np.all(np.abs(deq - v).reshape(4, 4, 32) <= d * 0.5 * (1 + 1e-6))


# ---------------------------------------------------------------- matvecs

def synth_q4(rows, K, seed):
    return oracle.synth_q4(rows, K, seed)


def test_gemv_q4_vs_float64():
    M, K = 96, 640   # 20 blocks: lanes 20..31 idle, exercises the tree
    W = synth_q4(M, K, 11)
    x = oracle.synth_normal(K, 12)
    y = oracle.gemv_q4(W, x, M, K)
    want = unpack_q4(W, M, K) @ x.astype(np.float64)
    assert rel_err(y, want) < 1e-5


def test_gemv_q4_invariants():
    M, K = 8, 256
    W = synth_q4(M, K, 13).reshape(M, K // 32, 5).copy()
    W[:, :, 1:] = 0x88888888                 # all codes 8 -> exactly zero
    x = oracle.synth_normal(K, 14)
    assert np.all(oracle.gemv_q4(W, x, M, K) == 0.0)
    W[3, 5, 2] = 0x88888F88                  # block 5, word 2 (elements 8..15), nibble 2
    s = np.uint16(W[3, 5, 0] & 0xFFFF).view(np.float16).astype(np.float32)
    y = oracle.gemv_q4(W, x, M, K)
    assert y[3] == np.float32(s * np.float32(7.0 * x[5 * 32 + 8 + 2]))
    assert np.all(np.delete(y, 3) == 0.0)


def test_fused_qkv_is_three_gemvs():
    K, qd, kvd = 256, 64, 32
    Wq, Wk, Wv = synth_q4(qd, K, 21), synth_q4(kvd, K, 22), synth_q4(kvd, K, 23)
    x = oracle.synth_normal(K, 24)
    q, k, v = oracle.fused_qkv_q4(Wq, Wk, Wv, x, qd, kvd, K)
    assert np.array_equal(q, oracle.gemv_q4(Wq, x, qd, K))
    assert np.array_equal(k, oracle.gemv_q4(Wk, x, kvd, K))
    assert np.array_equal(v, oracle.gemv_q4(Wv, x, kvd, K))


def test_gelu_tanh_constants():
    xs = np.linspace(-6, 6, 241).astype(np.float32)
    c = math.sqrt(2.0 / math.pi)
    want = [0.5 * v * (1 + math.tanh(c * (v + 0.044715 * v ** 3))) for v in xs.astype(float)]
    assert rel_err(oracle.gelu_tanh(xs), want) < 2e-6
    # the tanh form stays within 1e-3 of the exact erf GELU
    exact = [0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in xs.astype(float)]
    assert np.max(np.abs(oracle.gelu_tanh(xs) - np.array(exact))) < 1e-3


def test_fused_mlp_vs_float64():
    M, K = 32, 128
    Wg, Wu = synth_q4(M, K, 31), synth_q4(M, K, 32)
    x = oracle.synth_normal(K, 33)
    act = oracle.fused_mlp_q4(Wg, Wu, x, M, K)
    g = unpack_q4(Wg, M, K) @ x.astype(np.float64)
    u = unpack_q4(Wu, M, K) @ x.astype(np.float64)
    c = math.sqrt(2.0 / math.pi)
    want = 0.5 * g * (1 + np.tanh(c * (g + 0.044715 * g ** 3))) * u
    assert rel_err(act, want) < 1e-5


def test_mt_baseline_equals_single_thread():
    M, K = 300, 512
    W = synth_q4(M, K, 41)
    x = oracle.synth_normal(K, 42)
    assert np.array_equal(oracle.gemv_q4_mt(W, x, M, K, 3), oracle.gemv_q4(W, x, M, K))
    H, I = 64, 256
    Wg, Wu, Wd = synth_q4(I, H, 43), synth_q4(I, H, 44), synth_q4(H, I, 45)
    xh = oracle.synth_normal(H, 46)
    act, y = oracle.fused_mlp_step_mt(Wg, Wu, Wd, xh, H, I, 4)
    assert np.array_equal(act, oracle.fused_mlp_q4(Wg, Wu, xh, I, H))
    assert np.array_equal(y, oracle.gemv_q4(Wd, act, H, I))


def test_gemv_q8_vs_float64():
    M, K = 40, 256
    W = oracle.synth_q8(M, K, 51, 2e-4, 3.4e-4)
    x = oracle.synth_normal(K, 52)
    y = oracle.gemv_q8(W, x, M, K)
    want = oracle.dequant_q8(W, M, K).astype(np.float64) @ x.astype(np.float64)
    assert rel_err(y, want) < 1e-5


# ---------------------------------------------------------------- prefill

def test_batch_gemm_rows_are_gemvs():
    n, M, K = 5, 24, 256
    W = synth_q4(M, K, 61)
    X = oracle.synth_normal(n * K, 62).reshape(n, K)
    Y = oracle.batch_gemm_q4(W, X, n, M, K)
    want = X.astype(np.float64) @ unpack_q4(W, M, K).T
    assert Y.shape == (n, M) and rel_err(Y, want) < 1e-5


def test_batch_gemm_bf16_operand_model():
    n, M, K = 3, 16, 128
    W = synth_q4(M, K, 63)
    X = oracle.synth_normal(n * K, 64).reshape(n, K)
    Y = oracle.batch_gemm_q4_bf16(W, X, n, M, K)
    wq = bf16_to_f32(bf16_bits(unpack_q4(W, M, K).astype(np.float32))).astype(np.float64)
    xq = bf16_to_f32(bf16_bits(X)).astype(np.float64)
    assert rel_err(Y, xq @ wq.T) < 1e-5
    # and the bf16 model stays inside the 1e-2 prefill tolerance of fp32
    assert rel_err(Y, oracle.batch_gemm_q4(W, X, n, M, K)) < 1e-2


def test_batch_fused_mlp():
    n, M, K = 4, 16, 128
    Wg, Wu = synth_q4(M, K, 65), synth_q4(M, K, 66)
    X = oracle.synth_normal(n * K, 67).reshape(n, K)
    Y = oracle.batch_fused_mlp_q4(Wg, Wu, X, n, M, K)
    for t in range(n):
        assert rel_err(Y[t], oracle.fused_mlp_q4(Wg, Wu, X[t], M, K)) < 1e-6


# ---------------------------------------------------------------- attention

def attn64(Q, Kc, Vc, slots, H, D, kv_dim, gqa, scale=1.0):
    Q = Q.astype(np.float64).reshape(H, D)
    out = np.zeros((H, D))
    for h in range(H):
        kh = h // gqa
        Kr = np.stack([Kc[s * kv_dim + kh * D: s * kv_dim + (kh + 1) * D] for s in slots])
        Vr = np.stack([Vc[s * kv_dim + kh * D: s * kv_dim + (kh + 1) * D] for s in slots])
        sc = Kr.astype(np.float64) @ Q[h] * scale
        p = np.exp(sc - sc.max())
        p /= p.sum()
        out[h] = p @ Vr.astype(np.float64)
    return out.reshape(-1)


def test_decode_attn_vs_float64_and_invariants():
    H, KVH, D, nslot = 4, 2, 256, 64
    kv_dim = KVH * D
    Kc = oracle.synth_normal(nslot * kv_dim, 71)
    Vc = oracle.synth_normal(nslot * kv_dim, 72)
    Q = oracle.synth_normal(H * D, 73) * np.float32(0.1)
    rng = np.random.default_rng(5)
    slots = rng.permutation(nslot).astype(np.uint32)[:40]
    out = oracle.decode_attn(Q, Kc, Vc, slots, H, D, kv_dim, 2)
    assert rel_err(out, attn64(Q, Kc, Vc, slots, H, D, kv_dim, 2)) < 1e-5
    # permutation of the slot list changes nothing but rounding
    out2 = oracle.decode_attn(Q, Kc, Vc, slots[::-1].copy(), H, D, kv_dim, 2)
    assert rel_err(out2, out) < 1e-5
    # S = 1 -> V[slot] (times 1/(1+1e-9))
    one = oracle.decode_attn(Q, Kc, Vc, slots[:1], H, D, kv_dim, 2)
    s0 = int(slots[0])
    for h in range(H):
        kh = h // 2
        np.testing.assert_allclose(one[h * D:(h + 1) * D],
                                   Vc[s0 * kv_dim + kh * D: s0 * kv_dim + (kh + 1) * D],
                                   rtol=1e-6, atol=1e-7)
    # S = 0 -> zeros
    assert np.all(oracle.decode_attn(Q, Kc, Vc, slots[:0], H, D, kv_dim, 2) == 0)
    # identical keys -> uniform weights -> mean of V
    Kc2 = Kc.copy().reshape(nslot, kv_dim)
    Kc2[:] = Kc2[0]
    out3 = oracle.decode_attn(Q, Kc2.reshape(-1), Vc, slots, H, D, kv_dim, 2)
    mean = Vc.reshape(nslot, KVH, D)[slots].mean(axis=0)
    for h in range(H):
        np.testing.assert_allclose(out3[h * D:(h + 1) * D], mean[h // 2], rtol=1e-4, atol=1e-5)
    # a constant shift of every score (q -> q, K -> K + c*q_dir) is cancelled
    # by the max-subtraction: scale 1.0 vs large-magnitude scores stay finite
    big = oracle.decode_attn(Q * np.float32(50), Kc, Vc, slots, H, D, kv_dim, 2)
    assert np.all(np.isfinite(big))


def test_batch_causal_attn_matches_decode_per_token():
    H, KVH, D, prev, n = 2, 1, 256, 10, 6
    kv_dim = KVH * D
    total = prev + n
    Kc = oracle.synth_normal(total * kv_dim, 81)
    Vc = oracle.synth_normal(total * kv_dim, 82)
    Q = oracle.synth_normal(n * H * D, 83) * np.float32(0.1)
    slots = np.random.default_rng(6).permutation(total).astype(np.uint32)
    out = oracle.batch_causal_attn(Q, Kc, Vc, slots, n, prev, H, D, kv_dim, 2, 1.0, 0)
    win = oracle.batch_causal_attn(Q, Kc, Vc, slots, n, prev, H, D, kv_dim, 2, 1.0, 4)
    for t in range(n):
        S = prev + t + 1
        qt = Q[t * H * D:(t + 1) * H * D]
        assert np.array_equal(out[t * H * D:(t + 1) * H * D],
                              oracle.decode_attn(qt, Kc, Vc, slots[:S], H, D, kv_dim, 2))
        assert np.array_equal(win[t * H * D:(t + 1) * H * D],
                              oracle.decode_attn(qt, Kc, Vc, slots[S - 4:S], H, D, kv_dim, 2))


# ---------------------------------------------------------------- rope / norms

def test_qkv_rope_closed_forms():
    H, KVH, D = 2, 1, 256
    q = oracle.synth_normal(H * D, 91)
    k = oracle.synth_normal(KVH * D, 92)
    v = oracle.synth_normal(KVH * D, 93)
    qw = (1 + 0.1 * oracle.synth_normal(D, 94)).astype(np.float32)
    kw = (1 + 0.1 * oracle.synth_normal(D, 95)).astype(np.float32)
    nslot, slot = 8, 5
    kc = np.zeros(nslot * KVH * D, np.float32)
    vc = np.zeros(nslot * KVH * D, np.float32)

    def normed(a, w):
        a = a.astype(np.float64)
        return a / np.sqrt(np.mean(a * a) + 1e-6) * w

    # position 0: no rotation
    q0 = oracle.qkv_rope(q, k, v, qw, kw, kc, vc, H, KVH, D, D, False, 1e6, 1e-6, 0, slot)
    for h in range(H):
        np.testing.assert_allclose(q0[h * D:(h + 1) * D], normed(q[h * D:(h + 1) * D], qw),
                                   rtol=2e-6, atol=2e-6)
    # complex rotation of pairs (d, d + D/2) by pos * theta^(-2d/D).  At
    # position 4095 the reference's fp32 angle (f32(clock) * freq) carries up
    # to ~5e-4 rad of rounding, so that case gets atol 2e-3 (a wrong pairing,
    # sign or frequency is off by O(1)); position 7 is checked tightly.
    half = D // 2
    for pos, atol in ((7, 1e-5), (4095, 2e-3)):
        kc[:] = 0
        vc[:] = 0
        qr = oracle.qkv_rope(q, k, v, qw, kw, kc, vc, H, KVH, D, D, False, 1e6, 1e-6, pos, slot)
        rot = np.exp(1j * pos / (1e6 ** (2.0 * np.arange(half) / D)))
        for h in range(H):
            n = normed(q[h * D:(h + 1) * D], qw)
            z = (n[:half] + 1j * n[half:]) * rot
            np.testing.assert_allclose(qr[h * D:(h + 1) * D], np.concatenate([z.real, z.imag]),
                                       rtol=0, atol=atol)
        kz = normed(k, kw)
        z = (kz[:half] + 1j * kz[half:]) * rot
        kc2 = kc.reshape(nslot, KVH * D)
        np.testing.assert_allclose(kc2[slot], np.concatenate([z.real, z.imag]), atol=atol)
        np.testing.assert_allclose(vc.reshape(nslot, -1)[slot], normed(v, 1.0), rtol=2e-6,
                                   atol=2e-6)
        assert np.all(np.delete(kc2, slot, axis=0) == 0)
    # k_eq_v: V comes from raw K
    vc[:] = 0
    oracle.qkv_rope(q, k, v, qw, kw, kc, vc, H, KVH, D, D, True, 1e6, 1e-6, pos, slot)
    np.testing.assert_allclose(vc.reshape(nslot, -1)[slot], normed(k, 1.0), rtol=2e-6, atol=2e-6)


def test_rmsnorm_and_add_rmsnorm():
    dim = 3840
    c = np.full(dim, 3.0, np.float32)
    w = (1 + 0.1 * oracle.synth_normal(dim, 101)).astype(np.float32)
    y = oracle.rmsnorm(c, w, 1e-6)
    np.testing.assert_allclose(y, 3.0 / math.sqrt(9.0 + 1e-6) * w, rtol=1e-6)
    x = oracle.synth_normal(dim, 102)
    r = oracle.synth_normal(dim, 103)
    xn, y2 = oracle.add_rmsnorm(x, r, w, 1e-6, 0.5)
    s = (x.astype(np.float64) + r) * 0.5
    np.testing.assert_allclose(xn, s, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(y2, s / np.sqrt(np.mean(s * s) + 1e-6) * w, rtol=2e-6, atol=1e-6)


# ---------------------------------------------------------------- selection

def test_topk64_and_argmax():
    rng = np.random.default_rng(7)
    V = 8192
    logits = (rng.standard_normal(V) * 3).astype(np.float32)
    ids, vals = oracle.topk64(logits)
    capped = 30.0 * np.tanh(logits.astype(np.float64) / 30.0)
    order = np.argsort(-capped, kind="stable")[:64]
    assert np.array_equal(ids, order.astype(np.uint32))
    assert np.all(np.diff(vals) <= 0)
    np.testing.assert_allclose(vals, capped[order], rtol=1e-6)
    assert ids[0] == oracle.argmax(logits) == int(np.argmax(logits))
    assert oracle.argmax(np.array([1, 3, 3, 2], np.float32)) == 1   # first max
    # fewer than 64 logits: pad with -1e30
    ids2, vals2 = oracle.topk64(logits[:10])
    assert np.all(vals2[10:] == np.float32(-1e30))


# ---------------------------------------------------------------- generators

def splitmix64_stream(state, n):
    out = []
    for _ in range(n):
        state = (state + 0x9E3779B97F4A7C15) & (2**64 - 1)
        z = state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & (2**64 - 1)
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & (2**64 - 1)
        out.append(z ^ (z >> 31))
    return out


def test_mix64_is_splitmix64():
    # splitmix64 seeded with state 0 (Vigna's reference): first output
    assert oracle.mix64(0, 0) == 0xE220A8397B1DCDAF
    seed = 0xC4A77E1
    assert [oracle.mix64(seed, i) for i in range(5)] == splitmix64_stream(seed, 5)


def test_synth_distributions():
    rows, K = 64, 1024
    W = oracle.synth_q4(rows, K, 7).reshape(rows, K // 32, 5)
    s = (W[:, :, 0] & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float64)
    assert s.min() >= 0.005 * (1 - 2**-11) and s.max() <= 0.02 * (1 + 2**-11)
    codes = ((W[:, :, 1:, None] >> (np.arange(8, dtype=np.uint32) * 4)) & 0xF).ravel()
    counts = np.bincount(codes, minlength=16)
    assert counts.min() > 0.9 * codes.size / 16 and counts.max() < 1.1 * codes.size / 16
    z = oracle.synth_normal(200000, 9)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01


def test_threaded_forms_equal_serial():
    """The threaded checking forms split rows over threads and keep every
    row's arithmetic: results are bit-identical to the serial routines."""
    rng = np.random.default_rng(77)
    M, K, T = 96, 256, 5
    Wb = (rng.integers(0, 1 << 16, (M, K)) & 0xBFFF).astype(np.uint16)   # finite bf16
    assert np.array_equal(oracle.quantize_q4(Wb, 4), oracle.quantize_q4(Wb))
    assert np.array_equal(oracle.quantize_q8(Wb, 3), oracle.quantize_q8(Wb))
    W = oracle.synth_q4(M, K, 5)
    Wu = oracle.synth_q4(M, K, 6)
    x = rng.standard_normal(K).astype(np.float32)
    X = rng.standard_normal((T, K)).astype(np.float32)
    assert np.array_equal(oracle.gemv_q4(W, x, M, K, 4), oracle.gemv_q4(W, x, M, K))
    assert np.array_equal(oracle.fused_mlp_q4(W, Wu, x, M, K, 5), oracle.fused_mlp_q4(W, Wu, x, M, K))
    assert np.array_equal(oracle.batch_gemm_q4_bf16(W, X, T, M, K, 7), oracle.batch_gemm_q4_bf16(W, X, T, M, K))
    q, k, v = oracle.fused_qkv_q4(W, W, Wu, x, M, M, K, 3)
    q1, k1, v1 = oracle.fused_qkv_q4(W, W, Wu, x, M, M, K)
    assert np.array_equal(q, q1) and np.array_equal(k, k1) and np.array_equal(v, v1)
    E = oracle.quantize_q8(Wb)
    assert np.array_equal(oracle.gemv_q8(E, x, M, K, 4), oracle.gemv_q8(E, x, M, K))
    Kc = rng.standard_normal(64 * 512).astype(np.float32)
    Vc = rng.standard_normal(64 * 512).astype(np.float32)
    Q = rng.standard_normal(9 * 4 * 256).astype(np.float32)
    sl = rng.permutation(64).astype(np.uint32)
    for win in (0, 5):
        assert np.array_equal(oracle.batch_causal_attn(Q, Kc, Vc, sl, 9, 20, 4, 256, 512, 2, 1.0, win, 4),
                              oracle.batch_causal_attn(Q, Kc, Vc, sl, 9, 20, 4, 256, 512, 2, 1.0, win))
    # the array forms of the scalar routines
    xs = rng.standard_normal(300).astype(np.float32) * 20
    assert np.array_equal(oracle.gelu_tanh(xs), np.array([oracle.lib.orc_gelu_tanh(float(v)) for v in xs], np.float32))
    assert np.array_equal(oracle.softcap(xs), np.array([oracle.lib.orc_softcap(float(v)) for v in xs], np.float32))


def test_quiescence_gate_closed_form():
    """shaders/quiescence_gate.wgsl: the layer runs when mean((x - x_prev)^2)
    >= threshold (or the threshold is not positive); x_prev becomes x."""
    rng = np.random.default_rng(5)
    H = 3840
    x = rng.standard_normal(H).astype(np.float32)
    xp0 = (x + 0.01 * rng.standard_normal(H)).astype(np.float32)
    ms64 = float(np.mean((x.astype(np.float64) - xp0.astype(np.float64)) ** 2))
    for thresh, want in ((ms64 * 0.99, True), (ms64 * 1.01, False), (0.0, True), (-1.0, True)):
        xp = xp0.copy()
        runs, ms = oracle.quiescence_gate(x, xp, thresh)
        assert runs == want, thresh
        assert abs(ms - ms64) <= 1e-5 * ms64
        assert np.array_equal(xp, x)
    # an unchanged stream is quiescent for any positive threshold
    xp = x.copy()
    runs, ms = oracle.quiescence_gate(x, xp, 1e-30)
    assert not runs and ms == 0.0
