"""CPU checks of the model-level oracle (oracle/model.py).

The decode sequence (src/gpu/model_dispatch.zig:10-45) and the batched
prefill (src/gpu/batch_dispatch.zig:27-172) are two separately written
compositions of the same layer; run over the same prompt token by token and
as one batch they must agree (fp32 GEMMs, so only summation order differs).
The sliding window is exercised by giving the decode steps a short sliding
list and the prefill the same window.
"""
import numpy as np
import pytest

import oracle as O
from oracle import model as OM


def _cfg():
    return OM.default_config(hidden_size=128, intermediate_size=256, vocab_size=512, num_layers=3,
                             num_heads=2, num_kv_heads=1, head_dim=256, rotary_dim=128,
                             layer_full=[0, 1, 0], max_prefill_tokens=16)


@pytest.fixture(scope="module")
def weights():
    cfg = _cfg()
    layers, embed, final = OM.random_model(cfg, 11)
    return OM.Weights(cfg, layers, embed, final)


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


@pytest.mark.parametrize("window", [1024, 5])
def test_prefill_equals_token_by_token_decode(weights, window):
    cfg = weights.cfg
    toks = [3, 17, 255, 4, 99, 100, 7, 300, 42, 1]
    kc1, vc1 = OM.new_caches(cfg, 64)
    kc2, vc2 = OM.new_caches(cfg, 64)
    X, Xn, logits_p, ids_p, _ = OM.prefill(weights, kc1, vc1, toks, np.arange(len(toks)), 0, 0,
                                           bf16_gemm=False, window=window)
    for t, tok in enumerate(toks):
        active, sliding = OM.slot_lists(t, window)
        x, normed, logits_d, ids_d, _ = OM.decode_step(weights, kc2, vc2, weights.embed([tok])[0], t, t,
                                                       active, sliding)
        assert _rel(X[t], x) < 1e-4
        assert _rel(Xn[t], normed) < 1e-4
    for i in range(cfg["num_layers"]):
        assert _rel(kc1[i][: len(toks) * 256], kc2[i][: len(toks) * 256]) < 1e-4
        assert _rel(vc1[i][: len(toks) * 256], vc2[i][: len(toks) * 256]) < 1e-4
    assert _rel(logits_p, logits_d) < 1e-4
    assert ids_p[0] == ids_d[0]


def test_window_changes_sliding_layers_only(weights):
    """A window shorter than the prompt changes the output (the sliding
    layers see fewer slots); the full layer's K/V rows, computed before any
    attention of that layer, depend only on earlier layers."""
    cfg = weights.cfg
    toks = [5, 6, 7, 8, 9, 10, 11, 12]
    out = []
    for w in (1024, 3):
        kc, vc = OM.new_caches(cfg, 64)
        X, *_ = OM.prefill(weights, kc, vc, toks, np.arange(8), 0, 0, bf16_gemm=False, window=w)
        out.append((X, kc, vc))
    # layer 0 K/V are written before its attention: identical
    assert np.array_equal(out[0][1][0], out[1][1][0])
    # the last rows differ once the window cuts slots
    assert _rel(out[0][0][7], out[1][0][7]) > 1e-3
    # the first 3 tokens see at most 3 slots either way
    assert _rel(out[0][0][:3], out[1][0][:3]) < 1e-6


def test_bf16_prefill_close_to_fp32(weights):
    """The bf16-operand GEMM model stays within the bf16 bar of the fp32 path."""
    cfg = weights.cfg
    toks = [1, 2, 3, 4, 5, 6]
    r = []
    for bf in (False, True):
        kc, vc = OM.new_caches(cfg, 64)
        r.append(OM.prefill(weights, kc, vc, toks, np.arange(6), 0, 0, bf16_gemm=bf))
    assert _rel(r[1][2], r[0][2]) < 1e-2


def test_embed_scale_and_missing_norms():
    """x = bf16(embed) * sqrt(H) (src/model/forward.zig:35-37); absent norms
    read as 1.0 and absent post norms are skipped."""
    cfg = _cfg()
    layers, embed, _ = OM.random_model(cfg, 5)
    for l in layers:
        l["post_attention_layernorm"] = None
        l["q_norm"] = None
    W = OM.Weights(cfg, layers, embed, None)
    assert np.all(W.final_norm == 1.0) and np.all(W.layers[0]["q_norm"] == 1.0)
    assert W.layers[0]["post_attn"] is None
    e = W.embed([7])[0]
    want = OM.bf16_to_f32(embed[7]) * np.float32(np.sqrt(np.float32(128)))
    assert np.array_equal(e, want.astype(np.float32))
    assert abs(float(e[0]) - float(OM.bf16_to_f32(embed[7][0])) * 128 ** 0.5) < 1e-4


def test_topk_of_decode_matches_logits(weights):
    cfg = weights.cfg
    kc, vc = OM.new_caches(cfg, 16)
    a, s = OM.slot_lists(0, 1024)
    _, _, logits, ids, vals = OM.decode_step(weights, kc, vc, weights.embed([9])[0], 0, 0, a, s)
    capped = O.softcap(logits)
    order = np.argsort(-capped.astype(np.float64), kind="stable")[:64]
    assert np.array_equal(ids, order.astype(np.uint32))
    assert np.array_equal(vals, capped[order])


def test_global_head_shape_layers():
    """Full-attention layers with their own head_dim / KV head count
    (global_head_dim 512, one global KV head, whole-head rotation) run
    through both compositions consistently."""
    cfg = OM.default_config(hidden_size=128, intermediate_size=256, vocab_size=512, num_layers=3,
                            num_heads=2, num_kv_heads=1, head_dim=256, rotary_dim=128, global_head_dim=512,
                            num_global_kv_heads=1, layer_full=[0, 1, 0], max_prefill_tokens=16)
    layers, embed, final = OM.random_model(cfg, 3)
    assert layers[1]["q_proj"].shape == (2 * 512, 128) and layers[0]["q_proj"].shape == (2 * 256, 128)
    W = OM.Weights(cfg, layers, embed, final)
    toks = [1, 5, 9, 13, 17, 21]
    kc1, vc1 = OM.new_caches(cfg, 32)
    kc2, vc2 = OM.new_caches(cfg, 32)
    assert kc1[1].size == 32 * 512 and kc1[0].size == 32 * 256
    X, *_ = OM.prefill(W, kc1, vc1, toks, np.arange(6), 0, 0, bf16_gemm=False)
    for t, tok in enumerate(toks):
        a, s = OM.slot_lists(t, 1024)
        x, *_ = OM.decode_step(W, kc2, vc2, W.embed([tok])[0], t, t, a, s)
        assert _rel(X[t], x) < 1e-4


def _unit_norm_model(seed, num_layers=6):
    cfg = OM.default_config(hidden_size=256, intermediate_size=512, vocab_size=1024, num_layers=num_layers,
                            num_heads=4, num_kv_heads=2, head_dim=256, rotary_dim=128, max_prefill_tokens=16,
                            sliding_window=8, layer_full=[i % 3 == 2 for i in range(num_layers)])
    layers, embed, _ = OM.random_model(cfg, seed)
    for l in layers:       # every norm 1.0 (absent post norms are skipped)
        for k in ("input_layernorm", "q_norm", "k_norm", "pre_feedforward_layernorm"):
            l[k] = None
        l["post_attention_layernorm"] = l["post_feedforward_layernorm"] = None
        l["layer_scalar"] = 1.0
    return cfg, layers, embed


def test_quiescence_composition():
    """The gated decode step (recordLayerIndirect data flow): threshold 0 or
    a step without logits changes nothing; an unreachable threshold skips
    every gated layer, which leaves exactly the model of the first
    num_layers / 3 layers (all norms 1, so the stale normed row equals the
    final norm's) and leaves the gated layers' K/V slots untouched."""
    cfg, layers, embed = _unit_norm_model(3)
    W = OM.Weights(cfg, layers, embed, None)
    dense = cfg["num_layers"] // 3
    x = W.embed([17])[0]
    act, sl = OM.slot_lists(0, 8)
    kc0, vc0 = OM.new_caches(cfg, 64)
    ref = OM.decode_step(W, kc0, vc0, x, 0, 0, act, sl)
    for thresh, logits in ((0.0, True), (1e30, False)):
        kc, vc = OM.new_caches(cfg, 64)
        got = OM.decode_step(W, kc, vc, x, 0, 0, act, sl, with_logits=logits, qstate=OM.QuiescenceState(cfg, thresh))
        assert np.array_equal(got[0], ref[0]) and np.array_equal(got[1], ref[1])
    kc, vc = OM.new_caches(cfg, 64)
    qs = OM.QuiescenceState(cfg, 1e30)
    got = OM.decode_step(W, kc, vc, x, 0, 0, act, sl, qstate=qs)
    assert [g[0] for g in qs.log[0]] == list(range(dense, cfg["num_layers"]))
    assert not any(g[1] for g in qs.log[0])
    cfg_t = dict(cfg, num_layers=dense, layer_full=cfg["layer_full"][:dense])
    Wt = OM.Weights(cfg_t, layers[:dense], embed, None)
    kt, vt = OM.new_caches(cfg_t, 64)
    want = OM.decode_step(Wt, kt, vt, x, 0, 0, act, sl)
    for a, b in zip(got, want):
        assert np.array_equal(a, b)
    for i in range(dense, cfg["num_layers"]):
        assert not kc[i].any() and not vc[i].any()
