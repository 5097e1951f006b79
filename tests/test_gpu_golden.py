"""The HIP kernels against the committed golden vectors (tests/golden):
bit-exact quantizers and top-64 ids, fp32 bar (1e-3 normwise; observed
~1e-7) for matvecs, attention, RoPE and norms."""
import os

import numpy as np
import pytest

import channel_amd as ca
from gpu_util import f32_host, rel_err, say

pytestmark = pytest.mark.gpu

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"), allow_pickle=False)
TOL = 1e-3


def test_golden_quantizers(ctx):
    b = G["pack_in_bf16"]
    src = ctx.upload(b)
    d4 = ctx.alloc(ca.q4_bytes(4, 64))
    d8 = ctx.alloc(ca.q8_bytes(4, 64))
    say("golden quantizers")
    ctx.call("chn_quantize_q4", src, d4, 4, 64)
    ctx.call("chn_quantize_q8", src, d8, 4, 64)
    assert np.array_equal(ctx.download(d4, np.uint32, 40).reshape(4, 10), G["pack_q4"])
    assert np.array_equal(ctx.download(d8, np.uint32, 72).reshape(4, 18), G["pack_q8"])


def test_golden_matvecs(ctx):
    W, x = ctx.upload(G["gemv_W"]), ctx.upload(G["gemv_x"])
    y = ctx.alloc(16 * 4)
    say("golden gemv_q4 16x256")
    ctx.call("chn_gemv_q4", W, x, y, 16, 256)
    assert rel_err(f32_host(ctx, y, 16), G["gemv_y"]) < TOL
    Wg, Wu, xm = ctx.upload(G["mlp_Wg"]), ctx.upload(G["mlp_Wu"]), ctx.upload(G["mlp_x"])
    act = ctx.alloc(32 * 4)
    say("golden fused_mlp_q4 32x128")
    ctx.call("chn_fused_mlp_q4", Wg, Wu, xm, act, 32, 128)
    assert rel_err(f32_host(ctx, act, 32), G["mlp_act"]) < TOL
    E, xe = ctx.upload(G["q8_W"]), ctx.upload(G["q8_x"])
    ye = ctx.alloc(64 * 4)
    say("golden gemv_q8 64x128")
    ctx.call("chn_gemv_q8", E, xe, ye, 64, 128)
    assert rel_err(f32_host(ctx, ye, 64), G["q8_y"]) < TOL


def test_golden_attention(ctx):
    q, K, V = ctx.upload(G["attn_q"]), ctx.upload(G["attn_K"]), ctx.upload(G["attn_V"])
    slots = ctx.upload(np.concatenate([G["attn_slots"], np.zeros(16, np.uint32)]))   # room for max_slots = 80
    ns = ctx.upload(np.array([64], np.uint32))
    out = ctx.alloc(4 * 256 * 4)
    say("golden decode_attn")
    ctx.call("chn_decode_attn", q, K, V, slots, ns, 80, 4, 256, 512, 2, 1.0, out)
    assert rel_err(f32_host(ctx, out, 1024), G["attn_out"]) < TOL


@pytest.mark.parametrize("rot,theta,clock,key", [(256, 1e6, 4095, "rope_q_out"), (128, 1e4, 7, "rope_q_out_rot128")])
def test_golden_rope(ctx, rot, theta, clock, key):
    dq, dk, dv = ctx.upload(G["rope_q"]), ctx.upload(G["rope_k"]), ctx.upload(G["rope_v"])
    qw, kw = ctx.upload(G["rope_qw"]), ctx.upload(G["rope_kw"])
    qo = ctx.alloc(512 * 4)
    kc = ctx.zeros(4 * 256 * 4)
    vc = ctx.zeros(4 * 256 * 4)
    step = ctx.upload(np.array([clock, 2], np.uint32))
    say(f"golden qkv_rope rot={rot} clock={clock}")
    ctx.call("chn_qkv_rope", dq, dk, dv, qw, kw, qo, kc, vc, step, 2, 1, 256, rot, 0, theta, 1e-6)
    assert rel_err(f32_host(ctx, qo, 512), G[key]) < TOL
    if rot == 256:
        assert rel_err(f32_host(ctx, kc, 256, 512 * 4), G["rope_k_out"]) < TOL
        assert rel_err(f32_host(ctx, vc, 256, 512 * 4), G["rope_v_out"]) < TOL


def test_golden_topk_and_norms(ctx):
    lg = ctx.upload(G["topk_logits"])
    ids, vals = ctx.alloc(256), ctx.alloc(256)
    say("golden topk64")
    ctx.call("chn_topk64", lg, 8192, ids, vals)
    assert np.array_equal(ctx.download(ids, np.uint32, 64), G["topk_ids"])
    assert rel_err(ctx.download(vals, np.float32, 64), G["topk_vals"]) < 1e-6
    x, r, w = ctx.upload(G["norm_x"]), ctx.upload(G["norm_r"]), ctx.upload(G["norm_w"])
    y = ctx.alloc(3840 * 4)
    say("golden norms")
    ctx.call("chn_rmsnorm", x, w, y, 3840, 1e-6)
    assert rel_err(f32_host(ctx, y, 3840), G["norm_y"]) < TOL
    ctx.call("chn_add_rmsnorm", x, r, w, y, 3840, 1e-6, 0.75)
    assert rel_err(f32_host(ctx, x, 3840), G["addnorm_x"]) < TOL
    assert rel_err(f32_host(ctx, y, 3840), G["addnorm_y"]) < TOL
