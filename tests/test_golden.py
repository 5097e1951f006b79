"""The oracle against the committed golden vectors (tests/golden/golden.npz,
written by tests/golden/make_golden.py from an independent numpy
restatement).  Bars: bit-exact for the quantizers and the top-64 ids;
normwise 1e-6 for the fp32 matvecs, norms and RoPE (float64 fixtures);
1e-5 for attention."""
import os

import numpy as np
import pytest

import oracle as O

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden.npz"), allow_pickle=False)


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def test_pack_q4_q8_bit_exact():
    assert np.array_equal(O.quantize_q4(G["pack_in_bf16"]), G["pack_q4"])
    assert np.array_equal(O.quantize_q8(G["pack_in_bf16"]), G["pack_q8"])


def test_gemv_q4():
    assert rel(O.gemv_q4(G["gemv_W"], G["gemv_x"], 16, 256), G["gemv_y"]) < 1e-6


def test_fused_mlp_q4():
    assert rel(O.fused_mlp_q4(G["mlp_Wg"], G["mlp_Wu"], G["mlp_x"], 32, 128), G["mlp_act"]) < 1e-6


def test_gemv_q8():
    assert rel(O.gemv_q8(G["q8_W"], G["q8_x"], 64, 128), G["q8_y"]) < 1e-6


def test_decode_attn():
    out = O.decode_attn(G["attn_q"], G["attn_K"].ravel(), G["attn_V"].ravel(), G["attn_slots"], 4, 256, 512, 2)
    assert rel(out, G["attn_out"]) < 1e-5


@pytest.mark.parametrize("rot,theta,clock,key", [(256, 1e6, 4095, "rope_q_out"), (128, 1e4, 7, "rope_q_out_rot128")])
def test_qkv_rope(rot, theta, clock, key):
    kc = np.zeros(4 * 256, np.float32)
    vc = np.zeros(4 * 256, np.float32)
    q = O.qkv_rope(G["rope_q"], G["rope_k"], G["rope_v"], G["rope_qw"], G["rope_kw"], kc, vc, 2, 1, 256, rot, 0,
                   theta, 1e-6, clock, 2)
    assert rel(q, G[key]) < 1e-6
    if rot == 256:
        assert rel(kc[512:768], G["rope_k_out"]) < 1e-6
        assert rel(vc[512:768], G["rope_v_out"]) < 1e-6


def test_topk64():
    ids, vals = O.topk64(G["topk_logits"])
    assert np.array_equal(ids, G["topk_ids"])
    assert rel(vals, G["topk_vals"]) < 1e-6


def test_norms():
    assert rel(O.rmsnorm(G["norm_x"], G["norm_w"], 1e-6), G["norm_y"]) < 1e-6
    x2, y2 = O.add_rmsnorm(G["norm_x"], G["norm_r"], G["norm_w"], 1e-6, 0.75)
    assert rel(x2, G["addnorm_x"]) < 1e-6
    assert rel(y2, G["addnorm_y"]) < 1e-6


def test_planted_mistakes_fail():
    """A dropped term, a wrong index and a transposed operand in a copy of
    the oracle's inputs all move the result far outside the bars."""
    W = G["gemv_W"].copy()
    W[3, 7] ^= 0x1      # one nibble changed
    assert rel(O.gemv_q4(W, G["gemv_x"], 16, 256), G["gemv_y"]) > 1e-4
    x = G["gemv_x"].copy()
    x[[0, 1]] = x[[1, 0]]   # swapped operands
    assert rel(O.gemv_q4(G["gemv_W"], x, 16, 256), G["gemv_y"]) > 1e-4
    sl = G["attn_slots"].copy()
    sl[0] = (sl[0] + 1) % 80  # wrong slot
    out = O.decode_attn(G["attn_q"], G["attn_K"].ravel(), G["attn_V"].ravel(), sl, 4, 256, 512, 2)
    assert rel(out, G["attn_out"]) > 1e-4
