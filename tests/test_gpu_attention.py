"""GPU parity of decode attention, qkv_rope and the norms against the oracle,
plus the one-layer decode step at 12B dims (hidden 3840, 16 query / 8 KV
heads, head_dim 256, RoPE theta 1e6 at position 4095, full 4096-slot ring
with the write head at a random offset).  Tolerance: normwise relative
error <= 1e-3 (fp32)."""
import numpy as np
import pytest

import oracle
from gpu_util import f32_host, q4_host, rel_err, say, synth_normal_dev, synth_q4_dev

pytestmark = pytest.mark.gpu

TOL = 1e-3


def u32_dev(ctx, arr):
    return ctx.upload(np.ascontiguousarray(arr, dtype=np.uint32))


def ring_slots(head, n=4096):
    """Chronological slot list of a full ring whose newest entry is `head`."""
    return ((np.arange(n, dtype=np.int64) + head + 1) % n).astype(np.uint32)


@pytest.mark.parametrize("H,gqa,D,S,q_scale", [
    (16, 2, 256, 4096, 0.1),     # 12B full-attention layer, full ring
    (16, 2, 256, 4096, 1.0),     # unscaled q: peaked softmax
    (16, 2, 256, 512, 0.1),      # sliding window list
    (16, 2, 256, 65, 0.1),       # chunk boundary + 1
    (16, 2, 256, 64, 0.1),
    (16, 2, 256, 1, 0.1),
    (8, 1, 256, 300, 0.1),
    (8, 4, 256, 200, 0.1),
    (16, 8, 256, 130, 0.1),
    (8, 2, 512, 257, 0.05),      # head_dim 512 (global heads of larger configs)
])
def test_decode_attn_parity(ctx, H, gqa, D, S, q_scale):
    nslot = 4096
    kvh = H // gqa
    kv_dim = kvh * D
    seed = 7000 + H * 10 + gqa + S
    Kc = synth_normal_dev(ctx, nslot * kv_dim, seed)
    Vc = synth_normal_dev(ctx, nslot * kv_dim, seed + 1)
    Q = synth_normal_dev(ctx, H * D, seed + 2, q_scale)
    rng = np.random.default_rng(seed)
    perm = rng.permutation(nslot).astype(np.uint32)
    slots_h = perm[:S]
    slots = u32_dev(ctx, perm)      # the list has room for max_slots entries
    ns = u32_dev(ctx, [S])
    out = ctx.alloc(H * D * 4)
    say(f"decode_attn H={H} gqa={gqa} D={D} S={S}")
    ctx.call("chn_decode_attn", Q, Kc, Vc, slots, ns, nslot, H, D, kv_dim, gqa, 1.0, out)
    got = f32_host(ctx, out, H * D)
    want = oracle.decode_attn(f32_host(ctx, Q, H * D), f32_host(ctx, Kc, nslot * kv_dim),
                              f32_host(ctx, Vc, nslot * kv_dim), slots_h, H, D, kv_dim, gqa, 1.0)
    assert rel_err(got, want) < TOL


def test_decode_attn_zero_slots_and_count_from_device(ctx):
    """S = 0 gives zeros; the count is read from device memory at run time,
    so rewriting it changes the result without changing the call."""
    H, gqa, D = 4, 2, 256
    kv_dim = 2 * D
    Kc = synth_normal_dev(ctx, 128 * kv_dim, 1)
    Vc = synth_normal_dev(ctx, 128 * kv_dim, 2)
    Q = synth_normal_dev(ctx, H * D, 3, 0.1)
    slots_h = np.arange(128, dtype=np.uint32)
    slots = u32_dev(ctx, slots_h)
    ns = u32_dev(ctx, [0])
    out = ctx.alloc(H * D * 4)
    ctx.fill_u32(out, 0x7F800000, H * D)  # +inf sentinel
    say("decode_attn S=0")
    ctx.call("chn_decode_attn", Q, Kc, Vc, slots, ns, 128, H, D, kv_dim, gqa, 1.0, out)
    assert np.all(f32_host(ctx, out, H * D) == 0.0)
    ctx.upload(np.array([100], np.uint32), ns)
    ctx.call("chn_decode_attn", Q, Kc, Vc, slots, ns, 128, H, D, kv_dim, gqa, 1.0, out)
    want = oracle.decode_attn(f32_host(ctx, Q, H * D), f32_host(ctx, Kc, 128 * kv_dim),
                              f32_host(ctx, Vc, 128 * kv_dim), slots_h[:100], H, D, kv_dim, gqa)
    assert rel_err(f32_host(ctx, out, H * D), want) < TOL


@pytest.mark.parametrize("gqa,D,S", [(2, 256, 700), (2, 256, 4000), (4, 256, 300), (2, 512, 130)])
def test_decode_attn_ignores_unlisted_rows(ctx, gqa, D, S):
    """Cache rows that the first S list entries do not name hold NaN,
    slot 0 among them: rows past the count are loaded from slot 0 and
    masked, so the output is finite and equals the oracle's over the listed
    rows."""
    nslot, H = 4096, 8
    kv_dim = H // gqa * D
    rng = np.random.default_rng(S + gqa)
    K = rng.standard_normal((nslot, kv_dim)).astype(np.float32)
    V = rng.standard_normal((nslot, kv_dim)).astype(np.float32)
    perm = (rng.permutation(nslot - 1) + 1).astype(np.uint32)   # slot 0 never listed
    listed = perm[:S]
    unlisted = np.setdiff1d(np.arange(nslot), listed)
    K[unlisted] = np.nan
    V[unlisted] = np.nan
    q = (rng.standard_normal(H * D) * 0.1).astype(np.float32)
    Kc, Vc, Q = ctx.upload(K.ravel()), ctx.upload(V.ravel()), ctx.upload(q)
    slots, ns = u32_dev(ctx, np.concatenate([listed, np.zeros(nslot - S, np.uint32)])), u32_dev(ctx, [S])
    out = ctx.alloc(H * D * 4)
    say(f"decode_attn NaN outside the list: gqa={gqa} D={D} S={S}")
    ctx.call("chn_decode_attn", Q, Kc, Vc, slots, ns, nslot, H, D, kv_dim, gqa, 1.0, out)
    got = f32_host(ctx, out, H * D)
    assert np.all(np.isfinite(got))
    want = oracle.decode_attn(q, K.ravel(), V.ravel(), listed, H, D, kv_dim, gqa, 1.0)
    assert rel_err(got, want) < TOL


@pytest.mark.parametrize("nq,nkv,D,rot,k_eq_v,clock", [
    (16, 8, 256, 256, False, 4095),
    (8, 2, 256, 128, False, 77),     # partial rotary: suffix copied normed
    (4, 1, 512, 512, True, 1000),    # K = V (attention_k_eq_v)
])
def test_qkv_rope_parity(ctx, nq, nkv, D, rot, k_eq_v, clock):
    nslot = 64
    kv_dim = nkv * D
    seed = 8000 + nq + D + rot
    q = synth_normal_dev(ctx, nq * D, seed)
    k = synth_normal_dev(ctx, nkv * D, seed + 1)
    v = synth_normal_dev(ctx, nkv * D, seed + 2)
    qw_h = (1.0 + 0.1 * oracle.synth_normal(D, seed + 3)).astype(np.float32)
    kw_h = (1.0 + 0.1 * oracle.synth_normal(D, seed + 4)).astype(np.float32)
    qw, kw = ctx.upload(qw_h), ctx.upload(kw_h)
    kc = synth_normal_dev(ctx, nslot * kv_dim, seed + 5)
    vc = synth_normal_dev(ctx, nslot * kv_dim, seed + 6)
    kc_h = f32_host(ctx, kc, nslot * kv_dim)
    vc_h = f32_host(ctx, vc, nslot * kv_dim)
    slot = 37
    step = u32_dev(ctx, [clock, slot])
    qo = ctx.alloc(nq * D * 4)
    say(f"qkv_rope nq={nq} nkv={nkv} D={D} rot={rot}")
    ctx.call("chn_qkv_rope", q, k, v, qw, kw, qo, kc, vc, step, nq, nkv, D, rot, int(k_eq_v), 1e6, 1e-6)
    want_q = oracle.qkv_rope(f32_host(ctx, q, nq * D), f32_host(ctx, k, nkv * D),
                             f32_host(ctx, v, nkv * D), qw_h, kw_h, kc_h, vc_h, nq, nkv, D, rot,
                             k_eq_v, 1e6, 1e-6, clock, slot)
    assert rel_err(f32_host(ctx, qo, nq * D), want_q) < TOL
    kc_g = f32_host(ctx, kc, nslot * kv_dim).reshape(nslot, kv_dim)
    vc_g = f32_host(ctx, vc, nslot * kv_dim).reshape(nslot, kv_dim)
    assert rel_err(kc_g[slot], kc_h.reshape(nslot, kv_dim)[slot]) < TOL
    assert rel_err(vc_g[slot], vc_h.reshape(nslot, kv_dim)[slot]) < TOL
    others = np.arange(nslot) != slot
    assert np.array_equal(kc_g[others], kc_h.reshape(nslot, kv_dim)[others])
    assert np.array_equal(vc_g[others], vc_h.reshape(nslot, kv_dim)[others])


def test_norms_parity(ctx):
    dim, eps = 3840, 1e-6
    x = synth_normal_dev(ctx, dim, 1)
    r = synth_normal_dev(ctx, dim, 2)
    w_h = (1.0 + 0.1 * oracle.synth_normal(dim, 3)).astype(np.float32)
    w = ctx.upload(w_h)
    y = ctx.alloc(dim * 4)
    xh, rh = f32_host(ctx, x, dim), f32_host(ctx, r, dim)
    say("rmsnorm / add_rmsnorm 3840")
    ctx.call("chn_rmsnorm", x, w, y, dim, eps)
    assert rel_err(f32_host(ctx, y, dim), oracle.rmsnorm(xh, w_h, eps)) < 1e-5
    ctx.call("chn_add_rmsnorm", x, r, w, y, dim, eps, 0.5)
    xn, yn = oracle.add_rmsnorm(xh, rh, w_h, eps, 0.5)
    assert rel_err(f32_host(ctx, x, dim), xn) < 1e-6
    assert rel_err(f32_host(ctx, y, dim), yn) < 1e-5


def test_batch_norms_parity(ctx):
    n, dim, eps = 7, 3840, 1e-6
    X = synth_normal_dev(ctx, n * dim, 11)
    R = synth_normal_dev(ctx, n * dim, 12)
    w_h = (1.0 + 0.1 * oracle.synth_normal(dim, 13)).astype(np.float32)
    w = ctx.upload(w_h)
    Y = ctx.alloc(n * dim * 4)
    Xh = f32_host(ctx, X, n * dim).reshape(n, dim)
    Rh = f32_host(ctx, R, n * dim).reshape(n, dim)
    say("batch rmsnorm / add_rmsnorm 7x3840")
    ctx.call("chn_batch_rmsnorm", X, w, Y, n, dim, eps)
    Yg = f32_host(ctx, Y, n * dim).reshape(n, dim)
    for t in range(n):
        assert rel_err(Yg[t], oracle.rmsnorm(Xh[t], w_h, eps)) < 1e-5
    ctx.call("chn_batch_add_rmsnorm", X, R, w, Y, n, dim, eps, 1.0)
    Yg = f32_host(ctx, Y, n * dim).reshape(n, dim)
    Xg = f32_host(ctx, X, n * dim).reshape(n, dim)
    for t in range(n):
        xn, yn = oracle.add_rmsnorm(Xh[t], Rh[t], w_h, eps, 1.0)
        assert rel_err(Xg[t], xn) < 1e-6 and rel_err(Yg[t], yn) < 1e-5


def test_decoder_layer_step_12b(ctx):
    """Fused Q4 QKV (3840 -> 4096 | 2048 | 2048) + qkv_rope (theta 1e6,
    position 4095) + decode attention over the full 4096-slot ring (write
    head at a random slot) + o_proj (3840 x 4096 Q4) + RMSNorm; each stage is
    checked against the oracle fed the GPU's own inputs for that stage, and
    the end-to-end chain against the oracle's chain."""
    Hd, nq, nkv, D, nslot = 3840, 16, 8, 256, 4096
    q_dim, kv_dim = nq * D, nkv * D
    seed = 0xC4A77E1 + 3
    rng = np.random.default_rng(seed)
    head = int(rng.integers(0, nslot))
    x = synth_normal_dev(ctx, Hd, seed)
    Wq = synth_q4_dev(ctx, q_dim, Hd, seed + 1)
    Wk = synth_q4_dev(ctx, kv_dim, Hd, seed + 2)
    Wv = synth_q4_dev(ctx, kv_dim, Hd, seed + 3)
    Wo = synth_q4_dev(ctx, Hd, q_dim, seed + 4)
    kc = synth_normal_dev(ctx, nslot * kv_dim, seed + 5)
    vc = synth_normal_dev(ctx, nslot * kv_dim, seed + 6)
    ones_d = ctx.upload(np.ones(D, np.float32))
    ones_h = ctx.upload(np.ones(Hd, np.float32))
    kc0 = f32_host(ctx, kc, nslot * kv_dim)
    vc0 = f32_host(ctx, vc, nslot * kv_dim)
    q, k, v = ctx.alloc(q_dim * 4), ctx.alloc(kv_dim * 4), ctx.alloc(kv_dim * 4)
    qr = ctx.alloc(q_dim * 4)
    attn = ctx.alloc(q_dim * 4)
    o = ctx.alloc(Hd * 4)
    y = ctx.alloc(Hd * 4)
    slots_h = ring_slots(head, nslot)
    slots = u32_dev(ctx, slots_h)
    step = u32_dev(ctx, [4095, head, nslot, 0])
    say(f"layer step 12B, head slot {head}")
    ctx.call("chn_fused_qkv_q4", Wq, Wk, Wv, x, q, k, v, q_dim, kv_dim, Hd)
    ctx.call("chn_qkv_rope", q, k, v, ones_d, ones_d, qr, kc, vc, step, nq, nkv, D, D, 0, 1e6, 1e-6)
    ctx.call("chn_decode_attn", qr, kc, vc, slots, step.offset(8), nslot, nq, D, kv_dim, 2, 1.0, attn)
    ctx.call("chn_gemv_q4", Wo, attn, o, Hd, q_dim)
    ctx.call("chn_rmsnorm", o, ones_h, y, Hd, 1e-6)
    ctx.sync()

    xh = f32_host(ctx, x, Hd)
    Wqh, Wkh, Wvh = (q4_host(ctx, Wq, q_dim, Hd), q4_host(ctx, Wk, kv_dim, Hd),
                     q4_host(ctx, Wv, kv_dim, Hd))
    Woh = q4_host(ctx, Wo, Hd, q_dim)
    one_d = np.ones(D, np.float32)
    # stage by stage (oracle fed the GPU's stage inputs)
    rq, rk, rv = oracle.fused_qkv_q4(Wqh, Wkh, Wvh, xh, q_dim, kv_dim, Hd)
    qg, kg, vg = f32_host(ctx, q, q_dim), f32_host(ctx, k, kv_dim), f32_host(ctx, v, kv_dim)
    assert max(rel_err(qg, rq), rel_err(kg, rk), rel_err(vg, rv)) < TOL
    kc1, vc1 = kc0.copy(), vc0.copy()
    rqr = oracle.qkv_rope(qg, kg, vg, one_d, one_d, kc1, vc1, nq, nkv, D, D, False, 1e6, 1e-6,
                          4095, head)
    qrg = f32_host(ctx, qr, q_dim)
    kcg, vcg = f32_host(ctx, kc, nslot * kv_dim), f32_host(ctx, vc, nslot * kv_dim)
    assert rel_err(qrg, rqr) < TOL
    assert rel_err(kcg.reshape(nslot, -1)[head], kc1.reshape(nslot, -1)[head]) < TOL
    assert rel_err(vcg.reshape(nslot, -1)[head], vc1.reshape(nslot, -1)[head]) < TOL
    ra = oracle.decode_attn(qrg, kcg, vcg, slots_h, nq, D, kv_dim, 2, 1.0)
    ag = f32_host(ctx, attn, q_dim)
    assert rel_err(ag, ra) < TOL
    ro = oracle.gemv_q4(Woh, ag, Hd, q_dim)
    og = f32_host(ctx, o, Hd)
    assert rel_err(og, ro) < TOL
    assert rel_err(f32_host(ctx, y, Hd), oracle.rmsnorm(og, np.ones(Hd, np.float32), 1e-6)) < TOL
    # end-to-end oracle chain
    kc2, vc2 = kc0.copy(), vc0.copy()
    e_qr = oracle.qkv_rope(rq, rk, rv, one_d, one_d, kc2, vc2, nq, nkv, D, D, False, 1e6, 1e-6,
                           4095, head)
    e_a = oracle.decode_attn(e_qr, kc2, vc2, slots_h, nq, D, kv_dim, 2, 1.0)
    e_y = oracle.rmsnorm(oracle.gemv_q4(Woh, e_a, Hd, q_dim), np.ones(Hd, np.float32), 1e-6)
    assert rel_err(f32_host(ctx, y, Hd), e_y) < TOL
