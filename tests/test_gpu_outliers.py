"""The decode matvecs on activations that are hard for their input format.

Every Q4 matvec reads x as 18-bit block fixed point (per 32-block, values
rounded to 2^-18 of the block's power-of-two bound, exact integer block
dots, fp32 across blocks); the Q8 logits read 22-bit planes.  N(0, 1)
inputs are the easy case.  Here x has, at the 12B shapes:

* spike blocks: one channel 1e3..1e4 times its neighbours (the outlier
  channels of real residual streams), which coarsen the rounding of the
  other 31 values of the block;
* blocks scaled by 1e-30, all-zero blocks and blocks mixing +-1e3 with
  +-1e-3 values;

The bar is the fp32 one (normwise 1e-3 against the oracle); the largest
elementwise error is printed.  Non-finite inputs must come out non-finite
(the reference's fp32 products are NaN or +-Inf).
"""
import numpy as np
import pytest

import channel_amd as ca
import oracle
from gpu_util import f32_host, q4_host, rel_err, say, synth_q4_dev

pytestmark = pytest.mark.gpu


def outlier_x(K, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(K).astype(np.float64)
    nb = K // 32
    for b in range(nb):
        blk = slice(32 * b, 32 * b + 32)
        kind = b % 8
        if kind in (0, 3):                                    # one spike channel
            c = 32 * b + rng.integers(0, 32)
            x[c] = rng.choice([-1, 1]) * 10.0 ** rng.uniform(3, 4) * max(1.0, abs(x[c]))
        elif kind == 5:
            x[blk] *= 1e-30
        elif kind == 6 and b % 16 == 6:
            x[blk] = 0.0
        elif kind == 7:                                       # +-1e3 next to +-1e-3
            x[blk] = np.where(np.arange(32) % 2 == 0, 1e3, 1e-3) * rng.choice([-1, 1], 32)
    return x.astype(np.float32)


def elem_err(got, want):
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    big = np.abs(w) >= 1e-3 * np.max(np.abs(w))
    return float(np.max(np.abs(g[big] - w[big]) / np.abs(w[big])))


def check(name, got, want):
    e, ee = rel_err(got, want), elem_err(got, want)
    say(f"  {name}: normwise {e:.2e}, elementwise {ee:.2e}")
    assert e < 1e-3, name


def repacked(ctx, W, rows, K):
    R = ctx.alloc(ca.q4r_bytes(rows, K))
    ctx.call("chn_q4_repack", W, rows, K, R)
    return R


@pytest.mark.parametrize("M,K", [(8192, 2048), (3840, 4096), (3840, 15360)])
def test_gemv_outliers(ctx, M, K):
    """Config 1's GEMV (reference layout), o_proj and down (repacked, the
    model's layout)."""
    W = synth_q4_dev(ctx, M, K, 7000 + K)
    xh = outlier_x(K, K)
    x = ctx.upload(xh)
    y1, y2 = ctx.alloc(M * 4), ctx.alloc(M * 4)
    say(f"gemv outliers M={M} K={K}")
    ctx.call("chn_gemv_q4", W, x, y1, M, K)
    ctx.call("chn_gemv_q4r", repacked(ctx, W, M, K), x, y2, M, K)
    want = oracle.gemv_q4(q4_host(ctx, W, M, K), xh, M, K, oracle.NTHREADS)
    check("gemv_q4", f32_host(ctx, y1, M), want)
    check("gemv_q4r", f32_host(ctx, y2, M), want)


def test_qkv_and_gate_up_outliers(ctx):
    H, qd, kvd, I = 3840, 4096, 2048, 15360
    xh = outlier_x(H, 99)
    x = ctx.upload(xh)
    Wq, Wk, Wv = (synth_q4_dev(ctx, r, H, 7100 + i) for i, r in enumerate((qd, kvd, kvd)))
    q, k, v = ctx.alloc(qd * 4), ctx.alloc(kvd * 4), ctx.alloc(kvd * 4)
    say("fused qkv outliers 3840 -> 4096 | 2048 | 2048")
    ctx.call("chn_fused_qkv_q4r", repacked(ctx, Wq, qd, H), repacked(ctx, Wk, kvd, H), repacked(ctx, Wv, kvd, H),
             x, q, k, v, qd, kvd, H)
    wq, wk, wv = oracle.fused_qkv_q4(q4_host(ctx, Wq, qd, H), q4_host(ctx, Wk, kvd, H), q4_host(ctx, Wv, kvd, H),
                                     xh, qd, kvd, H, oracle.NTHREADS)
    check("q", f32_host(ctx, q, qd), wq)
    check("k", f32_host(ctx, k, kvd), wk)
    check("v", f32_host(ctx, v, kvd), wv)
    Wg, Wu = synth_q4_dev(ctx, I, H, 7200), synth_q4_dev(ctx, I, H, 7201)
    act = ctx.alloc(I * 4)
    say("fused gate/up outliers 3840 -> 15360")
    ctx.call("chn_fused_mlp_q4r", repacked(ctx, Wg, I, H), repacked(ctx, Wu, I, H), x, act, I, H)
    want = oracle.fused_mlp_q4(q4_host(ctx, Wg, I, H), q4_host(ctx, Wu, I, H), xh, I, H, oracle.NTHREADS)
    check("gate/up", f32_host(ctx, act, I), want)


def test_q8_logits_outliers(ctx):
    """The tied-embedding logits at full vocabulary, 262144 x 3840."""
    V, H = 262144, 3840
    W = ctx.alloc(ca.q8_bytes(V, H))
    ctx.call("chn_synth_q8", W, V, H, 7300, 0.0001, 0.0005)
    xh = outlier_x(H, 7301)
    x = ctx.upload(xh)
    y = ctx.alloc(V * 4)
    say("gemv_q8 outliers 262144 x 3840")
    ctx.call("chn_gemv_q8", W, x, y, V, H)
    Wh = ctx.download(W, np.uint32, ca.q8_bytes(V, H) // 4)
    check("q8 logits", f32_host(ctx, y, V), oracle.gemv_q8(Wh, xh, V, H, oracle.NTHREADS))


@pytest.mark.parametrize("bad", [np.nan, np.inf, -np.inf])
def test_non_finite_activations_propagate(ctx, bad):
    """One non-finite entry of x makes every output non-finite, as in the
    reference's fp32 matvecs (NaN here where the reference may give +-Inf)."""
    M, K = 256, 1024
    W = synth_q4_dev(ctx, M, K, 7400)
    Wu = synth_q4_dev(ctx, M, K, 7401)
    xh = np.random.default_rng(3).standard_normal(K).astype(np.float32)
    xh[517] = bad
    x = ctx.upload(xh)
    R, Ru = repacked(ctx, W, M, K), repacked(ctx, Wu, M, K)
    Wh = q4_host(ctx, W, M, K)
    want = oracle.gemv_q4(Wh, xh, M, K)
    assert not np.any(np.isfinite(want))
    say(f"non-finite x ({bad})")
    outs = {}
    for fn, args in (("chn_gemv_q4", (W, x)), ("chn_gemv_q4r", (R, x))):
        y = ctx.alloc(M * 4)
        ctx.call(fn, *args, y, M, K)
        outs[fn] = f32_host(ctx, y, M)
    act = ctx.alloc(M * 4)
    ctx.call("chn_fused_mlp_q4r", R, Ru, x, act, M, K)
    outs["chn_fused_mlp_q4r"] = f32_host(ctx, act, M)
    W8 = ctx.alloc(ca.q8_bytes(M, K))
    ctx.call("chn_synth_q8", W8, M, K, 7402, 0.001, 0.005)
    y8 = ctx.alloc(M * 4)
    ctx.call("chn_gemv_q8", W8, x, y8, M, K)
    outs["chn_gemv_q8"] = f32_host(ctx, y8, M)
    for fn, y in outs.items():
        assert not np.any(np.isfinite(y)), fn
    # finite blocks elsewhere still give finite results when the bad value is gone
    xh[517] = 0.5
    ctx.upload(xh, x)
    y = ctx.alloc(M * 4)
    ctx.call("chn_gemv_q4r", R, x, y, M, K)
    assert rel_err(f32_host(ctx, y, M), oracle.gemv_q4(Wh, xh, M, K)) < 1e-3
