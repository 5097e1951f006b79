"""GPU parity of the logits path and the ingest kernels against the oracle:
Q8_0 logits matvec (fp32 bar 1e-3 normwise; the 12B shape 262144 x 3840),
softcapped top-64 (ids and values identical to the oracle on the same
logits, ties to the lower index), the bf16 -> Q4 / Q8_0 quantizers and the
fp32 -> bf16 rounding (bit-exact), and the prefill RoPE / causal attention
kernels (fp32 bar)."""
import numpy as np
import pytest

import channel_amd as ca
import oracle
from gpu_util import f32_host, rel_err, say, synth_normal_dev

pytestmark = pytest.mark.gpu

TOL = 1e-3


def synth_q8_dev(ctx, rows, K, seed, smin=0.0005, smax=0.002):
    buf = ctx.alloc(ca.q8_bytes(rows, K))
    ctx.call("chn_synth_q8", buf, rows, K, seed, smin, smax)
    return buf


@pytest.mark.parametrize("M,K", [(262144, 3840), (4096, 256), (64, 128), (1000, 4096), (7, 640)])
def test_gemv_q8(ctx, M, K):
    W = synth_q8_dev(ctx, M, K, 100 + M % 97)
    x = synth_normal_dev(ctx, K, 200 + K)
    y = ctx.alloc(M * 4)
    say(f"gemv_q8 M={M} K={K}")
    ctx.call("chn_gemv_q8", W, x, y, M, K)
    Wh = ctx.download(W, np.uint32, M * (K // 32) * 9)
    want = oracle.gemv_q8(Wh, f32_host(ctx, x, K), M, K)
    got = f32_host(ctx, y, M)
    assert rel_err(got, want) < TOL
    # elementwise as well: the first rows within 1e-5 of their magnitude scale
    r = min(8, M)
    scale = np.abs(oracle.dequant_q8(Wh[: r * (K // 32) * 9], r, K)).max() * np.abs(f32_host(ctx, x, K)).sum()
    assert np.max(np.abs(got[:r] - want[:r])) <= 1e-5 * scale


@pytest.mark.parametrize("M,K", [(262144, 3840), (1001, 128), (7, 4096)])
def test_gemv_q8r_matches_q8(ctx, M, K):
    """The model's logits run on Q8R (the Q8_0 blocks repacked: per row the
    blocks' first 16 codes, then their last 16, then all f32 scales).  The
    repack keeps every byte, and the Q8R matvec gives the reference-layout
    matvec's results bit for bit."""
    nb = K // 32
    W = synth_q8_dev(ctx, M, K, 300 + M % 89)
    R = ctx.alloc(ca.q8_bytes(M, K))
    ctx.call("chn_q8_repack", W, M, K, R)
    x = synth_normal_dev(ctx, K, 301 + K)
    y1, y2 = ctx.alloc(M * 4), ctx.alloc(M * 4)
    say(f"gemv_q8r M={M} K={K}")
    ctx.call("chn_gemv_q8", W, x, y1, M, K)
    ctx.call("chn_gemv_q8r", R, x, y2, M, K)
    assert np.array_equal(ctx.download(y1, np.uint32, M), ctx.download(y2, np.uint32, M))
    Wh = ctx.download(W, np.uint32, M * nb * 9).reshape(M * nb, 9)
    Rh = ctx.download(R, np.uint32, M * nb * 9)
    codes = Rh[: M * nb * 8].reshape(M, 2, nb, 4).transpose(0, 2, 1, 3).reshape(M * nb, 8)
    assert np.array_equal(codes, Wh[:, 1:])
    assert np.array_equal(Rh[M * nb * 8:], Wh[:, 0])
    if M <= 4096:
        want = oracle.gemv_q8(Wh.ravel(), f32_host(ctx, x, K), M, K)
        assert rel_err(f32_host(ctx, y2, M), want) < TOL


def test_gemv_q8_shapes_rejected(ctx):
    buf = ctx.alloc(1 << 16)
    for K in (96, 4224, 0):
        with pytest.raises(ca.ChannelError):
            ctx.call("chn_gemv_q8", buf, buf, buf, 4, K)


@pytest.mark.parametrize("V", [262144, 4096, 2048, 100, 64, 3000])
def test_topk64_exact(ctx, V):
    rng = np.random.default_rng(V)
    lg = (rng.standard_normal(V) * 8).astype(np.float32)
    if V >= 200:
        # planted ties across tiles and a cap-saturated run
        lg[V - 1] = lg[5] = lg[V // 2] = np.float32(40.0)
        lg[17] = lg[V - 3] = np.float32(300.0)
        lg[100:110] = np.float32(25.0)
    d = ctx.upload(lg)
    ids = ctx.alloc(256)
    vals = ctx.alloc(256)
    say(f"topk64 V={V}")
    ctx.call("chn_topk64", d, V, ids, vals)
    gi = ctx.download(ids, np.uint32, 64)
    gv = ctx.download(vals, np.float32, 64)
    wi, wv = oracle.topk64(lg)
    k = min(64, V)
    assert np.array_equal(gi[:k], wi[:k])
    assert np.allclose(gv[:k], wv[:k], rtol=1e-6, atol=0)
    assert np.all(np.diff(gv[:k].astype(np.float64)) <= 0)


@pytest.mark.parametrize("V", [5000, 1025])
def test_topk64_all_ties(ctx, V):
    """Every logit saturates the cap to the same value: the answer is the 64
    lowest indices, in order, whichever tiles they sit in."""
    lg = np.full(V, 1000.0, np.float32)
    d = ctx.upload(lg)
    ids = ctx.alloc(256)
    vals = ctx.alloc(256)
    say(f"topk64 all ties V={V}")
    ctx.call("chn_topk64", d, V, ids, vals)
    gi = ctx.download(ids, np.uint32, 64)
    wi, wv = oracle.topk64(lg)
    assert np.array_equal(gi, np.arange(64, dtype=np.uint32))
    assert np.array_equal(gi, wi)
    assert np.array_equal(ctx.download(vals, np.float32, 64), wv)


@pytest.mark.parametrize("case", ["clustered", "ramp"])
def test_topk64_concentrated(ctx, case):
    """The merge takes its threshold from the tiles' maxima: 'clustered'
    puts 40 of the top values in each of two tiles (a few lists contribute
    long prefixes), 'ramp' puts every top value in the last tiles (more
    candidates than the gathered path holds, so every list is folded)."""
    V = 262144
    rng = np.random.default_rng(11)
    if case == "clustered":
        lg = (rng.standard_normal(V) * 0.5).astype(np.float32)
        lg[3 * 1024 + 7: 3 * 1024 + 47] = np.linspace(20.0, 21.0, 40, dtype=np.float32)
        lg[200 * 1024 + 500: 200 * 1024 + 540] = np.linspace(20.5, 21.5, 40, dtype=np.float32)
    else:
        lg = np.linspace(-5.0, 5.0, V, dtype=np.float32)
    d = ctx.upload(lg)
    ids = ctx.alloc(256)
    vals = ctx.alloc(256)
    say(f"topk64 {case}")
    ctx.call("chn_topk64", d, V, ids, vals)
    wi, wv = oracle.topk64(lg)
    assert np.array_equal(ctx.download(ids, np.uint32, 64), wi)
    assert np.allclose(ctx.download(vals, np.float32, 64), wv, rtol=1e-6, atol=0)


def test_topk64_small_vocab_padding(ctx):
    """Fewer than 64 logits: the tail is padded (ids 0, value -1e30)."""
    lg = np.array([3.0, -1.0, 7.0, 7.0, 0.5], np.float32)
    d = ctx.upload(lg)
    ids = ctx.alloc(256)
    vals = ctx.alloc(256)
    ctx.call("chn_topk64", d, 5, ids, vals)
    gi = ctx.download(ids, np.uint32, 64)
    gv = ctx.download(vals, np.float32, 64)
    assert list(gi[:5]) == [2, 3, 0, 4, 1]
    assert np.all(gv[5:] == np.float32(-1e30))


def _bf16_test_matrix(rows, cols, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, cols)) * rng.choice([1e-3, 0.05, 3.0, 200.0], size=(rows, 1)))
    w = w.astype(np.float32)
    w[0] = 0.0                       # all-zero block -> scale 0
    w[1, :32] = 1e-30                # subnormal-scale f16 (flushes)
    w[2, 5] = 7.0                    # single spike
    w[3, :32] = np.linspace(-1, 1, 32)  # exact ties at .5 after scaling
    b = oracle.bf16_from_f32(w).reshape(rows, cols)
    return b


@pytest.mark.parametrize("rows,cols", [(64, 256), (1000, 3840), (5, 32)])
def test_quantize_bit_exact(ctx, rows, cols):
    b = _bf16_test_matrix(rows, cols, rows + cols)
    src = ctx.upload(b)
    d4 = ctx.alloc(ca.q4_bytes(rows, cols))
    d8 = ctx.alloc(ca.q8_bytes(rows, cols))
    say(f"quantize rows={rows} cols={cols}")
    ctx.call("chn_quantize_q4", src, d4, rows, cols)
    ctx.call("chn_quantize_q8", src, d8, rows, cols)
    g4 = ctx.download(d4, np.uint32, rows * cols // 32 * 5).reshape(rows, -1)
    g8 = ctx.download(d8, np.uint32, rows * cols // 32 * 9).reshape(rows, -1)
    for got, want in ((g4, oracle.quantize_q4(b)), (g8, oracle.quantize_q8(b))):
        bad = np.argwhere(got != want)
        assert bad.size == 0, (f"{len(bad)} words differ, first at {tuple(bad[0])}: "
                               f"{got[tuple(bad[0])]:#010x} vs {want[tuple(bad[0])]:#010x}")


def test_to_bf16_bits_exact(ctx):
    rng = np.random.default_rng(1)
    v = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 1e3,
                        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, 3.4e38, 1.00390625, 1.01171875],
                                 np.float32)])
    src = ctx.upload(v)
    dst = ctx.alloc(v.size * 2)
    say("to_bf16_bits")
    ctx.call("chn_to_bf16_bits", src, dst, v.size)
    assert np.array_equal(ctx.download(dst, np.uint16, v.size), oracle.bf16_from_f32(v))


@pytest.mark.parametrize("nq,nkv,D,rot,keqv,n,off", [
    (16, 8, 256, 256, 0, 37, 5),
    (4, 2, 256, 128, 0, 9, 0),
    (8, 1, 512, 512, 1, 3, 2),
])
def test_batch_qkv_rope(ctx, nq, nkv, D, rot, keqv, n, off):
    qd, kvd = nq * D, nkv * D
    nslot = 256
    rng = np.random.default_rng(nq + n)
    q = rng.standard_normal((n, qd)).astype(np.float32)
    k = rng.standard_normal((n, kvd)).astype(np.float32)
    v = rng.standard_normal((n, kvd)).astype(np.float32)
    qn = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    kn = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    slots = rng.permutation(nslot)[: off + n].astype(np.uint32)
    start_clock = 4000
    dq, dk, dv = ctx.upload(q), ctx.upload(k), ctx.upload(v)
    dqn, dkn = ctx.upload(qn), ctx.upload(kn)
    qo = ctx.alloc(q.nbytes)
    kc = ctx.zeros(nslot * kvd * 4)
    vc = ctx.zeros(nslot * kvd * 4)
    ds = ctx.upload(slots)
    say(f"batch_qkv_rope nq={nq} nkv={nkv} D={D} n={n}")
    ctx.call("chn_batch_qkv_rope", dq, dk, dv, dqn, dkn, qo, kc, vc, ds, off, start_clock, n, nq, nkv, D, rot,
             keqv, 1e6, 1e-6)
    kc_o = np.zeros(nslot * kvd, np.float32)
    vc_o = np.zeros(nslot * kvd, np.float32)
    qo_o = np.stack([oracle.qkv_rope(q[t], k[t], v[t], qn, kn, kc_o, vc_o, nq, nkv, D, rot, keqv, 1e6, 1e-6,
                                     start_clock + t, int(slots[off + t])) for t in range(n)])
    assert rel_err(f32_host(ctx, qo, n * qd), qo_o.ravel()) < TOL
    assert rel_err(f32_host(ctx, kc, nslot * kvd), kc_o) < TOL
    assert rel_err(f32_host(ctx, vc, nslot * kvd), vc_o) < TOL


@pytest.mark.parametrize("nq,gqa,D,n,prev,window", [
    (16, 2, 256, 70, 0, 0),       # 12B full layer, one chunk of 70 tokens
    (16, 2, 256, 70, 100, 64),    # sliding window narrower than the list
    (8, 4, 256, 5, 300, 0),
    (4, 1, 512, 33, 17, 20),
    (16, 2, 256, 1, 0, 0),
    (16, 2, 256, 512, 0, 1024),   # 12B 512-token prefill (matrix-core path)
    (8, 8, 256, 20, 40, 0),       # GQA 8: 8 tokens per tile
    (4, 1, 256, 45, 10, 30),      # GQA 1, window inside the list
    (16, 2, 256, 100, 37, 50),    # window start and list end off the 32-key chunk grid
    (16, 2, 256, 130, 300, 100),  # long earlier context, window of 100
])
def test_batch_causal_attn(ctx, nq, gqa, D, n, prev, window):
    kvh = nq // gqa
    kvd = kvh * D
    nslot = 512
    rng = np.random.default_rng(n + prev + window)
    Kc = synth_normal_dev(ctx, nslot * kvd, 40 + n)
    Vc = synth_normal_dev(ctx, nslot * kvd, 41 + n)
    Q = synth_normal_dev(ctx, n * nq * D, 42 + n, 0.1)
    slots = rng.permutation(nslot)[: prev + n].astype(np.uint32)
    ds = ctx.upload(slots)
    out = ctx.alloc(n * nq * D * 4)
    say(f"batch_causal_attn nq={nq} gqa={gqa} D={D} n={n} prev={prev} window={window}")
    ctx.call("chn_batch_causal_attn", Q, Kc, Vc, ds, n, prev, nq, D, kvd, gqa, 1.0, window, out)
    want = oracle.batch_causal_attn(f32_host(ctx, Q, n * nq * D), f32_host(ctx, Kc, nslot * kvd),
                                    f32_host(ctx, Vc, nslot * kvd), slots, n, prev, nq, D, kvd, gqa, 1.0,
                                    window)
    assert rel_err(f32_host(ctx, out, n * nq * D), want) < TOL
