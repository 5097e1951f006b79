"""GPU parity of the decode matvecs (gemv_q4, fused_qkv_q4, fused_mlp_q4)
against the oracle, through the C-ABI.  Inputs are generated on the device,
downloaded, and fed to the oracle, so both sides see identical bits.
Tolerance: normwise relative error <= 1e-3 (fp32 accumulation)."""
import numpy as np
import pytest

import channel_amd as ca
import oracle
from gpu_util import f32_host, q4_host, rel_err, say, synth_normal_dev, synth_q4_dev

pytestmark = pytest.mark.gpu

TOL = 1e-3


def test_synth_q4_matches_host_generator(ctx):
    say("synth_q4 64x1024")
    W = synth_q4_dev(ctx, 64, 1024, 0xC4A77E1)
    assert np.array_equal(q4_host(ctx, W, 64, 1024), oracle.synth_q4(64, 1024, 0xC4A77E1))


def test_gemv_q4_reference_kat(ctx):
    """src/gpu.zig:38-60 on the GPU: every row is exactly 55.34375."""
    import oracle as o
    w = np.full((64, 128), 0x3F80, dtype=np.uint16)
    W = ctx.upload(o.quantize_q4(w))
    x = ctx.upload((np.arange(128) % 5).astype(np.float32) * 0.25)
    y = ctx.alloc(64 * 4)
    say("gemv_q4 KAT 64x128")
    ctx.call("chn_gemv_q4", W, x, y, 64, 128)
    assert np.all(f32_host(ctx, y, 64) == np.float32(55.34375))


@pytest.mark.parametrize("M,K", [
    (8192, 2048),    # config: single Q4 matvec, N=8192 x K=2048
    (3840, 4096),    # o_proj at 12B dims
    (3840, 15360),   # down_proj at 12B dims
    (100, 640),      # 20 blocks: partial pass, rows not a tile multiple
    (33, 2080),      # 65 blocks: second pass has one live lane
    (7, 32),         # one block
    (1, 8192),
])
def test_gemv_q4_parity(ctx, M, K):
    seed = 1000 + M + K
    W = synth_q4_dev(ctx, M, K, seed)
    x = synth_normal_dev(ctx, K, seed + 1)
    y = ctx.alloc(M * 4)
    say(f"gemv_q4 M={M} K={K}")
    ctx.call("chn_gemv_q4", W, x, y, M, K)
    got = f32_host(ctx, y, M)
    want = oracle.gemv_q4(q4_host(ctx, W, M, K), f32_host(ctx, x, K), M, K)
    assert rel_err(got, want) < TOL


def test_gemv_q4_zero_codes_and_single_weight(ctx):
    """All codes 8 -> 0; one code 15 -> s * 7 * x[k].  The kernel sums
    q*x - 8*sum(x) per block (one VALU op per weight fewer than (q-8)*x), so
    these exact answers come back with cancellation rounding of a few ulp of
    8*sum|x|; the bounds below are 1e-5 of that scale, far below what any
    wrong nibble position or dropped -8 would produce."""
    M, K = 16, 256
    Wh = oracle.synth_q4(M, K, 5).reshape(M, K // 32, 5).copy()
    Wh[:, :, 1:] = 0x88888888
    Wh[9, 3, 4] = 0x8F888888          # block 3, word 4 (elements 24..31), nibble 6
    W = ctx.upload(Wh)
    xh = oracle.synth_normal(K, 6)
    x = ctx.upload(xh)
    y = ctx.alloc(M * 4)
    say("gemv_q4 zero/single")
    ctx.call("chn_gemv_q4", W, x, y, M, K)
    got = f32_host(ctx, y, M)
    scales = (Wh[:, :, 0] & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float64)
    bound = 1e-5 * 8 * scales.max() * np.abs(xh).sum()
    s = scales[9, 3]
    assert abs(got[9] - s * 7.0 * xh[3 * 32 + 24 + 6]) <= bound
    assert abs(got[9]) > 100 * bound
    assert np.all(np.abs(np.delete(got, 9)) <= bound)


@pytest.mark.parametrize("q_dim,kv_dim,K", [(4096, 2048, 3840), (96, 40, 256)])
def test_fused_qkv_q4_parity(ctx, q_dim, kv_dim, K):
    seed = 2000 + q_dim
    Wq = synth_q4_dev(ctx, q_dim, K, seed)
    Wk = synth_q4_dev(ctx, kv_dim, K, seed + 1)
    Wv = synth_q4_dev(ctx, kv_dim, K, seed + 2)
    x = synth_normal_dev(ctx, K, seed + 3)
    q, k, v = ctx.alloc(q_dim * 4), ctx.alloc(kv_dim * 4), ctx.alloc(kv_dim * 4)
    say(f"fused_qkv_q4 q={q_dim} kv={kv_dim} K={K}")
    ctx.call("chn_fused_qkv_q4", Wq, Wk, Wv, x, q, k, v, q_dim, kv_dim, K)
    rq, rk, rv = oracle.fused_qkv_q4(q4_host(ctx, Wq, q_dim, K), q4_host(ctx, Wk, kv_dim, K),
                                     q4_host(ctx, Wv, kv_dim, K), f32_host(ctx, x, K),
                                     q_dim, kv_dim, K)
    assert rel_err(f32_host(ctx, q, q_dim), rq) < TOL
    assert rel_err(f32_host(ctx, k, kv_dim), rk) < TOL
    assert rel_err(f32_host(ctx, v, kv_dim), rv) < TOL


@pytest.mark.parametrize("M,K", [(15360, 3840), (50, 96)])
def test_fused_mlp_q4_parity(ctx, M, K):
    seed = 3000 + M
    Wg = synth_q4_dev(ctx, M, K, seed)
    Wu = synth_q4_dev(ctx, M, K, seed + 1)
    x = synth_normal_dev(ctx, K, seed + 2)
    act = ctx.alloc(M * 4)
    say(f"fused_mlp_q4 M={M} K={K}")
    ctx.call("chn_fused_mlp_q4", Wg, Wu, x, act, M, K)
    want = oracle.fused_mlp_q4(q4_host(ctx, Wg, M, K), q4_host(ctx, Wu, M, K),
                               f32_host(ctx, x, K), M, K)
    assert rel_err(f32_host(ctx, act, M), want) < TOL


def test_rejects_bad_shapes(ctx):
    import channel_amd as ca
    W = synth_q4_dev(ctx, 4, 64, 1)
    x = synth_normal_dev(ctx, 64, 2)
    y = ctx.alloc(16)
    with pytest.raises(ca.ChannelError) as e:
        ctx.call("chn_gemv_q4", W, x, y, 4, 48)      # K % 32 != 0
    assert e.value.status == "Invalid"
    with pytest.raises(ca.ChannelError):
        ctx.call("chn_gemv_q4", W, x.ptr + 4, y, 4, 32)  # x not 16-byte aligned


# ---- repacked (Q4R) weights: the layout the model keeps in HBM ------------

def q4r_host(Wref, rows, K):
    """Host restatement of the repack: nibble words XOR 0x88888888, f16 scales."""
    W = Wref.reshape(rows, K // 32, 5)
    N = (W[:, :, 1:5] ^ np.uint32(0x88888888)).reshape(-1)
    S = (W[:, :, 0] & np.uint32(0xFFFF)).astype(np.uint16).reshape(-1)
    return np.concatenate([N.view(np.uint8), S.view(np.uint8)])


def repack_dev(ctx, W, rows, K):
    R = ctx.alloc(ca.q4r_bytes(rows, K))
    ctx.call("chn_q4_repack", W, rows, K, R)
    return R


@pytest.mark.parametrize("M,K", [(15360, 3840), (3840, 15360), (8192, 3840), (3840, 4096), (7, 32), (33, 2080),
                                 (100, 640), (1, 8192), (15, 16384)])
def test_q4r_gemv_parity(ctx, M, K):
    W = synth_q4_dev(ctx, M, K, 900 + M + K)
    x = synth_normal_dev(ctx, K, 901 + K)
    say(f"q4r gemv M={M} K={K}")
    R = repack_dev(ctx, W, M, K)
    Wh = q4_host(ctx, W, M, K)
    assert np.array_equal(ctx.download(R, np.uint8, ca.q4r_bytes(M, K)), q4r_host(Wh, M, K))
    y = ctx.alloc(M * 4)
    ctx.call("chn_gemv_q4r", R, x, y, M, K)
    got = f32_host(ctx, y, M)
    want = oracle.gemv_q4(Wh, f32_host(ctx, x, K), M, K)
    assert rel_err(got, want) < 1e-3
    y2 = ctx.alloc(M * 4)
    ctx.call("chn_gemv_q4", W, x, y2, M, K)
    assert rel_err(got, f32_host(ctx, y2, M)) < 1e-5


def test_q4r_fused_qkv_and_mlp(ctx):
    H, qd, kvd, I = 3840, 4096, 2048, 15360
    Wq, Wk, Wv = (synth_q4_dev(ctx, r, H, 950 + i) for i, r in enumerate((qd, kvd, kvd)))
    Rq, Rk, Rv = repack_dev(ctx, Wq, qd, H), repack_dev(ctx, Wk, kvd, H), repack_dev(ctx, Wv, kvd, H)
    x = synth_normal_dev(ctx, H, 960)
    q, k, v = ctx.alloc(qd * 4), ctx.alloc(kvd * 4), ctx.alloc(kvd * 4)
    say("q4r fused qkv 12B")
    ctx.call("chn_fused_qkv_q4r", Rq, Rk, Rv, x, q, k, v, qd, kvd, H)
    xh = f32_host(ctx, x, H)
    wq, wk, wv = oracle.fused_qkv_q4(q4_host(ctx, Wq, qd, H), q4_host(ctx, Wk, kvd, H), q4_host(ctx, Wv, kvd, H),
                                     xh, qd, kvd, H)
    assert rel_err(f32_host(ctx, q, qd), wq) < 1e-3
    assert rel_err(f32_host(ctx, k, kvd), wk) < 1e-3
    assert rel_err(f32_host(ctx, v, kvd), wv) < 1e-3
    Wg, Wu = synth_q4_dev(ctx, I, H, 970), synth_q4_dev(ctx, I, H, 971)
    Rg, Ru = repack_dev(ctx, Wg, I, H), repack_dev(ctx, Wu, I, H)
    act = ctx.alloc(I * 4)
    say("q4r fused mlp 12B")
    ctx.call("chn_fused_mlp_q4r", Rg, Ru, x, act, I, H)
    want = oracle.fused_mlp_q4(q4_host(ctx, Wg, I, H), q4_host(ctx, Wu, I, H), xh, I, H)
    assert rel_err(f32_host(ctx, act, I), want) < 1e-3


def test_q4r_bad_shapes(ctx):
    W = ctx.alloc(1 << 20)
    x = ctx.alloc(1 << 16)
    for K in (0, 48, 16416):
        with pytest.raises(ca.ChannelError):
            ctx.call("chn_gemv_q4r", W, x, x, 4, K)


# ---- activation digit planes and the plane-input entries ------------------

def decode_planes(P, K):
    """Host decoding of chn_xplanes output: integers X and block scales."""
    nb = K // 32
    words = P[:20 * nb].reshape(5, 4, nb)                       # [plane][group][block]
    inv = P[20 * nb:].view(np.float32)
    sh = np.arange(8, dtype=np.uint32) * 4
    dig = (((words[..., None] ^ np.uint32(0x88888888)) >> sh) & 15).astype(np.int64) - 8   # [p][w][b][n]
    X = sum(dig[p] * (16 ** p) for p in range(5))               # [w][b][n]
    return X.transpose(1, 0, 2).reshape(nb, 32), inv


def test_xplanes_reconstruct_exactly(ctx):
    K = 3840
    rng = np.random.default_rng(41)
    xh = rng.standard_normal(K).astype(np.float32)
    xh[0:32] = 0.0                                   # zero block
    xh[32:64] *= 1e-30                               # tiny block
    xh[64:96] = 0.0
    xh[64 + 5] = 4.0                                 # max exactly a power of two
    xh[96:128] = -xh[96:128] * 1e3                   # large block
    x = ctx.upload(xh)
    P = ctx.alloc(ca.xplanes_bytes(K))
    say("xplanes 3840")
    ctx.call("chn_xplanes", x, K, P)
    X, inv = decode_planes(ctx.download(P, np.uint32, ca.xplanes_bytes(K) // 4), K)
    xb = xh.reshape(-1, 32).astype(np.float64)
    for b in range(K // 32):
        m = np.abs(xb[b]).max()
        if m == 0.0 or m < 2.0 ** -100:
            assert inv[b] == 0.0 and np.all(X[b] == 0), b
            continue
        e = int(np.log2(inv[b])) + 18                  # inv = 2^(e - 18)
        assert inv[b] == np.float32(2.0 ** (e - 18)), b
        assert 2.0 ** (e - 1) <= m < 2.0 ** e, b       # frexp exponent of the block max
        assert np.array_equal(X[b], np.rint(xb[b] * 2.0 ** (18 - e)).astype(np.int64)), b
        assert np.abs(X[b] * float(inv[b]) - xb[b]).max() <= 0.5 * float(inv[b])


@pytest.mark.parametrize("M,K", [(15360, 3840), (64, 256), (64, 8192), (96, 640)])
def test_q4r_plane_entries_match(ctx, M, K):
    """chn_gemv_q4r_xp / chn_fused_mlp_q4r_xp on chn_xplanes(x) give the
    same bits as the x-input entries; the fused act planes equal
    chn_xplanes(act) (K = 8192 takes the separate-pass path)."""
    Wg, Wu = synth_q4_dev(ctx, M, K, 1200 + M), synth_q4_dev(ctx, M, K, 1201 + M)
    Rg, Ru = repack_dev(ctx, Wg, M, K), repack_dev(ctx, Wu, M, K)
    x = synth_normal_dev(ctx, K, 1202 + K)
    P = ctx.alloc(ca.xplanes_bytes(K))
    say(f"q4r plane entries M={M} K={K}")
    ctx.call("chn_xplanes", x, K, P)
    y1, y2 = ctx.alloc(M * 4), ctx.alloc(M * 4)
    ctx.call("chn_gemv_q4r", Rg, x, y1, M, K)
    ctx.call("chn_gemv_q4r_xp", Rg, P, y2, M, K)
    assert np.array_equal(f32_host(ctx, y1, M), f32_host(ctx, y2, M))
    a1, a2, a3 = ctx.alloc(M * 4), ctx.alloc(M * 4), ctx.alloc(M * 4)
    ctx.call("chn_fused_mlp_q4r", Rg, Ru, x, a1, M, K)
    ctx.call("chn_fused_mlp_q4r_xp", Rg, Ru, P, a2, None, M, K)
    AP = ctx.alloc(ca.xplanes_bytes(M))
    ctx.call("chn_fused_mlp_q4r_xp", Rg, Ru, P, a3, AP, M, K)
    h1 = f32_host(ctx, a1, M)
    assert np.array_equal(h1, f32_host(ctx, a2, M))
    assert np.array_equal(h1, f32_host(ctx, a3, M))
    AQ = ctx.alloc(ca.xplanes_bytes(M))
    ctx.call("chn_xplanes", a1, M, AQ)
    n = ca.xplanes_bytes(M) // 4
    assert np.array_equal(ctx.download(AP, np.uint32, n), ctx.download(AQ, np.uint32, n))
    want = oracle.fused_mlp_q4(q4_host(ctx, Wg, M, K), q4_host(ctx, Wu, M, K), f32_host(ctx, x, K), M, K)
    assert rel_err(h1, want) < 1e-3


def test_q4r_plane_entries_reject(ctx):
    W = ctx.alloc(1 << 16)
    P = ctx.alloc(ca.xplanes_bytes(256))
    a = ctx.alloc(64 * 4)
    with pytest.raises(ca.ChannelError):
        ctx.call("chn_fused_mlp_q4r_xp", W, W, P, a, P, 64, 256)        # act planes alias the input planes
    with pytest.raises(ca.ChannelError):
        ctx.call("chn_fused_mlp_q4r_xp", W, W, P, a, a, 50, 256)        # M % 32 != 0 with act planes
    with pytest.raises(ca.ChannelError):
        ctx.call("chn_xplanes", a, 48, P)                                # K % 32 != 0


@pytest.mark.parametrize("post", [True, False])
def test_ffn_gate_up_fused_norm_12b(ctx, post):
    """chn_ffn_gate_up_q4r, the decode step's pre-FFN launch, at 12B dims
    (hidden 3840, FFN 15360): post-attention norm, residual add and pre-FFN
    norm as the prologue of gate/up (src/gpu/model_dispatch.zig:33-40)."""
    H, I, eps = 3840, 15360, 1e-6
    rng = np.random.default_rng(8 + post)
    Wg, Wu = synth_q4_dev(ctx, I, H, 1300), synth_q4_dev(ctx, I, H, 1301)
    Rg, Ru = repack_dev(ctx, Wg, I, H), repack_dev(ctx, Wu, I, H)
    xh = (rng.standard_normal(H) * 3).astype(np.float32)
    rh = rng.standard_normal(H).astype(np.float32)
    pw = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    fw = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    x, r = ctx.upload(xh), ctx.upload(rh)
    pwd, fwd = ctx.upload(pw), ctx.upload(fw)
    xo, nx, act = ctx.alloc(H * 4), ctx.alloc(H * 4), ctx.alloc(I * 4)
    AP = ctx.alloc(ca.xplanes_bytes(I))
    say(f"ffn_gate_up fused norm 15360x3840 post={post}")
    ctx.call("chn_ffn_gate_up_q4r", Rg, Ru, x, r, pwd if post else None, fwd, xo, nx, act, AP, I, H, eps)
    rr = oracle.rmsnorm(rh, pw, eps) if post else rh
    x_o, n_o = oracle.add_rmsnorm(xh, rr, fw, eps, 1.0)
    assert rel_err(f32_host(ctx, xo, H), x_o) < 1e-5
    assert rel_err(f32_host(ctx, nx, H), n_o) < 1e-5
    got = f32_host(ctx, act, I)
    want = oracle.fused_mlp_q4(q4_host(ctx, Wg, I, H), q4_host(ctx, Wu, I, H), n_o, I, H, oracle.NTHREADS)
    assert rel_err(got, want) < 1e-3
    AQ = ctx.alloc(ca.xplanes_bytes(I))
    ctx.call("chn_xplanes", act, I, AQ)
    n = ca.xplanes_bytes(I) // 4
    assert np.array_equal(ctx.download(AP, np.uint32, n), ctx.download(AQ, np.uint32, n))
    with pytest.raises(ca.ChannelError):
        ctx.call("chn_ffn_gate_up_q4r", Rg, Ru, x, r, None, fwd, x, nx, act, AP, I, H, eps)   # x_out aliases x_in
