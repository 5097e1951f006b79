"""GPU parity of the model level: a small random model ingested from bf16
through chn_model_create (device Q4/Q8 quantization), batched prefill, then
graph-replayed decode steps, all against the model oracle (oracle/model.py,
following src/gpu/model_dispatch.zig and src/gpu/batch_dispatch.zig).

Bars: prefill runs on bf16 MFMA operands (normwise 1e-2 on logits and KV
rows); decode is fp32 (1e-3), with its caches taken from the GPU after the
prefill so that the bf16 prefill error does not enter the decode check.
Top-64 lists must be a valid top-64 of the oracle's logits (identical up to
the order of near-ties).
"""
import numpy as np
import pytest

import channel_amd as ca
from channel_amd.model import Model
from gpu_util import assert_topk_valid, rel_err, say
import oracle
from oracle import model as OM
from oracle import ring as OR

pytestmark = pytest.mark.gpu

CFG = OM.default_config(hidden_size=256, intermediate_size=512, vocab_size=4096, num_layers=3,
                        num_heads=4, num_kv_heads=2, head_dim=256, rotary_dim=128,
                        layer_full=[0, 1, 0], max_prefill_tokens=64, sliding_window=16)
WINDOW = 16


@pytest.fixture(scope="module")
def pair(ctx):
    layers, embed, final = OM.random_model(CFG, 21)
    W = OM.Weights(CFG, layers, embed, final)
    say("model_create small random model")
    m = Model.create(ctx, CFG, layers, embed, final)
    yield W, m
    m.close()


def _kv_all(m, n):
    return [m.kv_read(i, 0, n) for i in range(CFG["num_layers"])]


def test_prefill_then_decode(pair):
    W, m = pair
    kvd = CFG["num_kv_heads"] * CFG["head_dim"]
    toks = [int(t) for t in np.random.default_rng(3).integers(0, CFG["vocab_size"], 40)]
    n = len(toks)
    calls = []
    say("prefill 40 tokens")
    lg, ids, vals = m.prefill_batch(toks, np.arange(n), 0, 0, embed_bf16=W.embed_bf16,
                                    progress=lambda i, t: calls.append((i, t)))
    assert calls == [(3, 3)]
    kc, vc = OM.new_caches(CFG, 4096)
    _, Xn, lg_o, ids_o, vals_o = OM.prefill(W, kc, vc, toks, np.arange(n), 0, 0, bf16_gemm=True,
                                            window=1024)
    assert rel_err(lg, lg_o) < 1e-2
    assert_topk_valid(ids, vals, lg_o, 1e-2, "prefill 40 tokens")
    kv = _kv_all(m, n)
    for i in range(CFG["num_layers"]):
        assert rel_err(kv[i][0], kc[i][: n * kvd].reshape(n, kvd)) < 1e-2
        assert rel_err(kv[i][1], vc[i][: n * kvd].reshape(n, kvd)) < 1e-2
    # the decode state holds the last normed row
    _, normed = m.read_state()
    assert rel_err(normed, Xn[n - 1]) < 1e-2

    # continue with greedy decode from the GPU's caches
    for i in range(CFG["num_layers"]):
        kc[i][: n * kvd] = kv[i][0].ravel()
        vc[i][: n * kvd] = kv[i][1].ravel()
    tok = int(ids[0])
    for clock in range(n, n + 4):
        active, sliding = OM.slot_lists(clock, WINDOW)
        x_in = W.embed([tok])[0]
        say(f"decode clock={clock} tok={tok}")
        t_gpu, ids_g, vals_g = m.forward_token(x_in, clock, clock, active, sliding)
        x_o, nx_o, lg_o, ids_o, vals_o = OM.decode_step(W, kc, vc, x_in, clock, clock, active, sliding)
        assert t_gpu == ids_g[0]
        assert_topk_valid(ids_g, vals_g, lg_o, 1e-3, f"decode clock {clock}")
        x_g, nx_g = m.read_state()
        assert rel_err(x_g, x_o) < 1e-3
        assert rel_err(nx_g, nx_o) < 1e-3
        for i in range(CFG["num_layers"]):
            k_g, v_g = m.kv_read(i, clock, 1)
            assert rel_err(k_g[0], kc[i][clock * kvd:(clock + 1) * kvd]) < 1e-3
            assert rel_err(v_g[0], vc[i][clock * kvd:(clock + 1) * kvd]) < 1e-3
        tok = int(ids_g[0])


def test_decode_without_logits_and_ring_slots(pair):
    """The no-logits graph updates state and caches only; slot lists in ring
    order (the write head mid-ring) and a slot index different from clock."""
    W, m = pair
    kvd = CFG["num_kv_heads"] * CFG["head_dim"]
    rng = np.random.default_rng(9)
    # fill 200 ring slots with random K/V, identical on both sides
    kc, vc = OM.new_caches(CFG, 4096)
    for i in range(CFG["num_layers"]):
        k = rng.standard_normal((200, kvd)).astype(np.float32)
        v = rng.standard_normal((200, kvd)).astype(np.float32)
        m.kv_write(i, 3000, k, v)
        kc[i][3000 * kvd:3200 * kvd] = k.ravel()
        vc[i][3000 * kvd:3200 * kvd] = v.ravel()
        k_back, v_back = m.kv_read(i, 3000, 200)
        assert np.array_equal(k_back, k) and np.array_equal(v_back, v)
    clock, slot = 5000, 3199
    active = np.arange(3000, 3200, dtype=np.uint32)
    sliding = active[-WINDOW:]
    x_in = W.embed([77])[0]
    say("decode without logits")
    m.forward_token(x_in, clock, slot, active, sliding, topk=False)
    x_o, nx_o, *_ = OM.decode_step(W, kc, vc, x_in, clock, slot, active, sliding, with_logits=False)
    x_g, nx_g = m.read_state()
    assert rel_err(x_g, x_o) < 1e-3
    assert rel_err(nx_g, nx_o) < 1e-3
    for i in range(CFG["num_layers"]):
        k_g, _ = m.kv_read(i, slot, 1)
        assert rel_err(k_g[0], kc[i][slot * kvd:(slot + 1) * kvd]) < 1e-3


def test_prefill_after_previous_slots(pair):
    """A second prefill chunk attends over num_prev_slots earlier slots."""
    W, m = pair
    kvd = CFG["num_kv_heads"] * CFG["head_dim"]
    rng = np.random.default_rng(5)
    kc, vc = OM.new_caches(CFG, 4096)
    prev = np.arange(100, 130, dtype=np.uint32)
    for i in range(CFG["num_layers"]):
        k = (rng.standard_normal((30, kvd)) * 0.5).astype(np.float32)
        v = rng.standard_normal((30, kvd)).astype(np.float32)
        m.kv_write(i, 100, k, v)
        kc[i][100 * kvd:130 * kvd] = k.ravel()
        vc[i][100 * kvd:130 * kvd] = v.ravel()
    toks = [5, 900, 31, 4000, 2, 2, 17, 64]
    new = np.arange(130, 138, dtype=np.uint32)
    slots = np.concatenate([prev, new])
    say("prefill with 30 previous slots")
    lg, ids, vals = m.prefill_batch(toks, slots, 30, 30, embed_bf16=W.embed_bf16)
    _, _, lg_o, _, _ = OM.prefill(W, kc, vc, toks, slots, 30, 30, bf16_gemm=True)
    assert rel_err(lg, lg_o) < 1e-2
    assert_topk_valid(ids, vals, lg_o, 1e-2, "prefill after 30 previous slots")


def test_model_errors(pair):
    W, m = pair
    with pytest.raises(ca.ChannelError) as e:
        m.prefill_batch(list(range(65)), np.arange(65), 0, 0, embed_bf16=W.embed_bf16)
    assert e.value.status == "BatchTooLarge"
    with pytest.raises(ca.ChannelError) as e:
        m.prefill_batch([], [], 0, 0, embed_bf16=W.embed_bf16)
    assert e.value.status == "BatchTooLarge"
    with pytest.raises(ca.ChannelError):
        m.prefill_batch([1, 2], [0, 4096], 0, 0, embed_bf16=W.embed_bf16)
    with pytest.raises(ca.ChannelError):
        m.prefill_batch([1, 5000], [0, 1], 0, 0, embed_bf16=W.embed_bf16)
    with pytest.raises(ca.ChannelError):
        m.forward_token(np.zeros(256, np.float32), 0, 4096, [0], [0])
    with pytest.raises(ca.ChannelError):
        m.forward_token(np.zeros(256, np.float32), 0, 0, np.arange(4097), [0])
    with pytest.raises(ca.ChannelError):
        m.forward_token_id(CFG["vocab_size"], 0, 0, [0], [0])
    with pytest.raises(ca.ChannelError):
        m.decode_greedy(1, 0, 4097)
    with pytest.raises(ca.ChannelError):
        m.decode_greedy(CFG["vocab_size"], 0, 1)
    with pytest.raises(ca.ChannelError):
        m.kv_read(3, 0, 1)
    with pytest.raises(ca.ChannelError):
        m.kv_read(0, 4090, 7)


def test_synthetic_model_token_path(ctx):
    """chn_decode_token gathers bf16(embed[tok]) * sqrt(H) on the device; it
    must match chn_decode_step fed with the same row from the host."""
    cfg = dict(CFG, num_layers=2, layer_full=[1, 0])
    say("model_create_synthetic")
    with Model.synthetic(ctx, cfg, 1234) as m1, Model.synthetic(ctx, cfg, 1234) as m2:
        import ctypes
        p = ctypes.c_void_p()
        assert ca.lib.chn_model_embedding_bf16(m1.handle, ctypes.byref(p)) == 0 and p.value
        H = cfg["hidden_size"]
        tok = 1001
        row = ctx.download(p.value + tok * H * 2, np.uint16, H)
        x_in = OM.bf16_to_f32(row) * np.float32(np.sqrt(np.float32(H)))
        for clock in range(3):
            active, sliding = OM.slot_lists(clock, WINDOW)
            t1, ids1, vals1 = m1.forward_token_id(tok, clock, clock, active, sliding)
            t2, ids2, vals2 = m2.forward_token(x_in, clock, clock, active, sliding)
            assert np.array_equal(ids1, ids2) and np.array_equal(vals1, vals2)
            assert np.all(np.diff(vals1) <= 0) and np.all(ids1 < cfg["vocab_size"])
            tok = int(t1)
            row = ctx.download(p.value + tok * H * 2, np.uint16, H)
            x_in = OM.bf16_to_f32(row) * np.float32(np.sqrt(np.float32(H)))


def test_decode_logits_equal_standalone_q8(ctx):
    """The decode step's final norm writes the byte planes of the normed row
    that the Q8 logits matvec reads (no separate planes pass).  The step's
    top-64 must equal, bit for bit, chn_gemv_q8r + chn_topk64 run on the
    same normed row, which make their planes with the standalone pass."""
    import ctypes
    cfg = dict(CFG, num_layers=2, layer_full=[1, 0])
    H, V = cfg["hidden_size"], cfg["vocab_size"]
    with Model.synthetic(ctx, cfg, 4321) as m:
        p = ctypes.c_void_p()
        assert ca.lib.chn_model_embedding_bf16(m.handle, ctypes.byref(p)) == 0 and p.value
        emb = ctx.download(p.value, np.uint16, V * H).reshape(V, H)
        E8 = ctx.upload(oracle.quantize_q8(emb).ravel())
        R = ctx.alloc(ca.q8_bytes(V, H))
        ctx.call("chn_q8_repack", E8, V, H, R)
        y, ids_d, vals_d = ctx.alloc(V * 4), ctx.alloc(256), ctx.alloc(256)
        tok = 77
        for clock in range(3):
            active, sliding = OM.slot_lists(clock, WINDOW)
            say(f"decode step clock={clock}, logits of the normed row")
            t, ids, vals = m.forward_token_id(tok, clock, clock, active, sliding)
            _, normed = m.read_state()
            ctx.call("chn_gemv_q8r", R, ctx.upload(normed), y, V, H)
            ctx.call("chn_topk64", y, V, ids_d, vals_d)
            assert np.array_equal(ids, ctx.download(ids_d, np.uint32, 64))
            assert np.array_equal(vals.view(np.uint32), ctx.download(vals_d, np.uint32, 64))
            tok = int(t)


def test_eager_launches_match_graph(ctx):
    """chn_model_set_graph(0) launches the decode kernels one by one; the
    results are bit-identical to the graph replay."""
    cfg = dict(CFG, num_layers=2, layer_full=[0, 1])
    say("eager vs graph decode")
    with Model.synthetic(ctx, cfg, 77) as mg, Model.synthetic(ctx, cfg, 77) as me:
        me.set_graph(False)
        tok_g = tok_e = 5
        for clock in range(4):
            active, sliding = OM.slot_lists(clock, WINDOW)
            tok_g, ids_g, vals_g = mg.forward_token_id(tok_g, clock, clock, active, sliding)
            tok_e, ids_e, vals_e = me.forward_token_id(tok_e, clock, clock, active, sliding)
            assert np.array_equal(ids_g, ids_e) and np.array_equal(vals_g, vals_e)
            xg, ng = mg.read_state()
            xe, ne = me.read_state()
            assert np.array_equal(xg, xe) and np.array_equal(ng, ne)


@pytest.mark.parametrize("graph", [True, False])
def test_replay_equals_decode_step(ctx, graph):
    """chn_model_replay (submitPreRecorded(cmd_buf_decode), as
    src/model/bench.zig:12-15 calls it) runs the recorded step again on the
    inputs the last call left on the device.  It must equal, bit for bit,
    chn_decode_step fed with the device's stream x and the same lists:
    top-64, state, logits and the K/V row written; likewise the step without
    logits.  Also: the device state starts at zero, as src/server.zig:76-81
    leaves it, and the context reports a device name (src/gpu.zig:24-30)."""
    cfg = dict(CFG, num_layers=2, layer_full=[0, 1])
    kvd = CFG["num_kv_heads"] * CFG["head_dim"]
    assert ctx.device_name
    say(f"replay vs decode_step, graph={graph} on {ctx.device_name}")
    with Model.synthetic(ctx, cfg, 61) as ma, Model.synthetic(ctx, cfg, 61) as mb:
        ma.set_graph(graph)
        mb.set_graph(graph)
        x0, n0 = ma.read_state()
        assert not x0.any() and not n0.any() and not ma.read_logits().any()
        clock = 37
        active, sliding = OM.slot_lists(clock, WINDOW)
        x_in = np.random.default_rng(61).standard_normal(cfg["hidden_size"]).astype(np.float32)
        ta, ida, va = ma.forward_token(x_in, clock, clock, active, sliding)
        tb, idb, vb = mb.forward_token(x_in, clock, clock, active, sliding)
        assert np.array_equal(ida, idb) and np.array_equal(va, vb)
        for with_logits in (True, False, True):
            x_dev, _ = mb.read_state()
            out = ma.replay(with_logits)
            _, idb, vb = mb.forward_token(x_dev, clock, clock, active, sliding, topk=with_logits)
            if with_logits:
                assert np.array_equal(out[0], idb) and np.array_equal(out[1].view(np.uint32), vb.view(np.uint32))
                assert np.array_equal(ma.read_logits().view(np.uint32), mb.read_logits().view(np.uint32))
            xa, na = ma.read_state()
            xb, nb = mb.read_state()
            assert np.array_equal(xa, xb) and np.array_equal(na, nb)
            assert not np.array_equal(xa, x_dev)        # the step ran on the device's stream
            for layer in range(2):
                ka, va_ = ma.kv_read(layer, clock, 1)
                kb, vb_ = mb.kv_read(layer, clock, 1)
                assert np.array_equal(ka, kb) and np.array_equal(va_, vb_)
                assert ka.shape == (1, kvd)
        with pytest.raises(ca.ChannelError):
            lib = ca.lib
            import ctypes
            ids = np.zeros(64, np.uint32)
            ma._check("chn_model_replay", lib.chn_model_replay(ma.handle, 0, ids.ctypes.data_as(ctypes.c_void_p), None))


def ring_lists(clock, window):
    """Slot lists of the reference's ring without anchors (slot = clock mod
    3968), from the ring restatement oracle/ring.py."""
    from oracle.ring import Ring
    ring = Ring(1, 0)
    for c in range(max(0, clock - 3968), clock):
        ring.activate_slot(0, c)
    _, active, sliding = OR.decode_lists(ring, clock, window)
    return np.asarray(active, np.uint32), np.asarray(sliding, np.uint32)


GREEDY_CASES = [
    # (clock0, anchors, boundaries, recall {rank: clock})
    (0, 0, (), None),
    (3965, 0, (), None),                                    # the window wraps at 3968
    (3966, 512, (100, 600, 3971), {0: 50, 5: 3968, 9: 9000}),  # snap past the anchors, recall joins
]


@pytest.mark.parametrize("clock0,anchors,bounds,recall", GREEDY_CASES)
def test_decode_greedy_matches_token_loop(ctx, clock0, anchors, bounds, recall):
    """chn_decode_greedy (device-resident steps, slot lists generated on the
    device) equals the same steps driven from the host with the lists of
    the ring restatement (oracle/ring.py: getSlotIndexLayer /
    getActiveSlotsLayer after activateSlot, src/model/forward.zig:41-47),
    bit for bit: tokens, state and the K/V rows written."""
    from oracle.ring import Ring
    cfg = dict(CFG, num_layers=2, layer_full=[0, 1])
    n = 6
    say(f"decode_greedy clock0={clock0} anchors={anchors}")
    rc = None
    ring = Ring(1, anchors)
    for b in bounds:
        ring.mark_boundary(b)
    if recall is not None:
        rc = np.full(128, 0xFFFFFFFF, np.uint32)
        for rank, clk in recall.items():
            rc[rank] = clk
            ring.write_recall_kv(0, rank, clk)
    for c in range(clock0):
        ring.activate_slot(0, c)
    with Model.synthetic(ctx, cfg, 99) as mg, Model.synthetic(ctx, cfg, 99) as mh:
        toks = mg.decode_greedy(17, clock0, n, num_anchors=anchors, boundaries=bounds, recall_clocks=rc)
        tok = 17
        want, slots = [], []
        for i in range(n):
            clock = clock0 + i
            slot, active, sliding = OR.decode_lists(ring, clock, WINDOW)
            assert len(active) <= 4096 and max(active) < 4096
            tok, _, _ = mh.forward_token_id(tok, clock, slot, active, sliding)
            want.append(tok)
            slots.append(slot)
        assert list(toks) == want
        xg, ng = mg.read_state()
        xh, nh = mh.read_state()
        assert np.array_equal(xg, xh) and np.array_equal(ng, nh)
        for layer in range(2):
            for slot in slots:
                kg, vg = mg.kv_read(layer, slot, 1)
                kh, vh = mh.kv_read(layer, slot, 1)
                assert np.array_equal(kg, kh) and np.array_equal(vg, vh)
    if clock0 == 3965:
        assert slots[3] == 0            # clock 3968 takes slot 0, not 3968


def test_created_model_token_path_matches_step(pair):
    """Models ingested from bf16 keep a device copy of the embedding: the
    device gather equals bf16(embed[tok]) * sqrt(H) fed from the host."""
    W, m = pair
    x_in = W.embed([123])[0]
    active, sliding = ring_lists(900, WINDOW)
    t1, ids1, vals1 = m.forward_token_id(123, 900, 900, active, sliding)
    x1, n1 = m.read_state()
    t2, ids2, vals2 = m.forward_token(x_in, 900, 900, active, sliding)
    x2, n2 = m.read_state()
    assert np.array_equal(ids1, ids2) and np.array_equal(vals1, vals2)
    assert np.array_equal(x1, x2) and np.array_equal(n1, n2)


CFG_G = OM.default_config(hidden_size=256, intermediate_size=512, vocab_size=4096, num_layers=3,
                          num_heads=4, num_kv_heads=2, head_dim=256, rotary_dim=128, global_head_dim=512,
                          num_global_kv_heads=1, layer_full=[0, 1, 0], max_prefill_tokens=64,
                          sliding_window=16)


def test_global_head_shape_model(ctx):
    """Full-attention layers with global_head_dim 512 and one KV head (GQA 4)
    next to sliding layers with head_dim 256 (GQA 2): prefill and decode
    against the oracle."""
    layers, embed, final = OM.random_model(CFG_G, 31)
    W = OM.Weights(CFG_G, layers, embed, final)
    say("model_create global head shapes")
    with Model.create(ctx, CFG_G, layers, embed, final) as m:
        toks = [int(t) for t in np.random.default_rng(8).integers(0, 4096, 20)]
        n = len(toks)
        lg, ids, vals = m.prefill_batch(toks, np.arange(n), 0, 0, embed_bf16=W.embed_bf16)
        kc, vc = OM.new_caches(CFG_G, 4096)
        _, _, lg_o, _, _ = OM.prefill(W, kc, vc, toks, np.arange(n), 0, 0, bf16_gemm=True)
        assert rel_err(lg, lg_o) < 1e-2
        for i in range(3):
            k, v = m.kv_read(i, 0, n)
            kvd = k.shape[1]
            assert kvd == 512   # one 512-wide global KV head, or two 256-wide sliding ones
            assert rel_err(k, kc[i][: n * kvd].reshape(n, kvd)) < 1e-2
            kc[i][: n * kvd] = k.ravel()
            vc[i][: n * kvd] = v.ravel()
        tok = int(ids[0])
        for clock in range(n, n + 3):
            active, sliding = OM.slot_lists(clock, WINDOW)
            x_in = W.embed([tok])[0]
            say(f"global-shape decode clock={clock}")
            t_gpu, ids_g, vals_g = m.forward_token(x_in, clock, clock, active, sliding)
            x_o, nx_o, lg_o, _, _ = OM.decode_step(W, kc, vc, x_in, clock, clock, active, sliding)
            assert_topk_valid(ids_g, vals_g, lg_o, 1e-3, f"global-shape decode clock {clock}")
            x_g, _ = m.read_state()
            assert rel_err(x_g, x_o) < 1e-3
            tok = int(ids_g[0])


@pytest.mark.parametrize("anchors", [0, 32])
def test_prefill_chunked_as_the_server_calls_it(pair, anchors):
    """The server's batched prefill (src/server/prefill.zig:61-97): the
    prompt in chunks of max_tokens; per chunk the previous slots from
    getPrefillPrevSlots, then getSlotIndex of each new clock, every layer's
    slot activated; logits and the top-64 only for the last chunk.  Against
    the oracle run through the same chunks (ring restatement oracle/ring.py)."""
    from oracle.ring import Ring
    W, m = pair
    max_tok = CFG["max_prefill_tokens"]
    toks = [int(t) for t in np.random.default_rng(70 + anchors).integers(0, CFG["vocab_size"], 150)]
    ring = Ring(CFG["num_layers"], 0)
    ring.set_num_anchors(anchors)
    kc, vc = OM.new_caches(CFG, 4096)
    clock, off = 0, 0
    while off < len(toks):
        chunk = toks[off:off + max_tok]
        last = off + len(chunk) == len(toks)
        prev = ring.prefill_prev_slots(0, clock, len(chunk))
        c_slots = list(prev)
        for i in range(len(chunk)):
            c_slots.append(ring.slot_index(0, clock + i))
            for layer in range(CFG["num_layers"]):
                ring.activate_slot(layer, clock + i)
        say(f"chunked prefill clock={clock} n={len(chunk)} prev={len(prev)} anchors={anchors}")
        lg, ids, vals = m.prefill_batch(chunk, c_slots, clock, len(prev), embed_bf16=W.embed_bf16,
                                        logits=last, topk=last)
        _, _, lg_o, _, _ = OM.prefill(W, kc, vc, chunk, c_slots, clock, len(prev), bf16_gemm=True)
        clock += len(chunk)
        off += len(chunk)
    assert rel_err(lg, lg_o) < 1e-2
    assert_topk_valid(ids, vals, lg_o, 1e-2, f"chunked prefill, anchors {anchors}")


CFG_Q = OM.default_config(hidden_size=256, intermediate_size=512, vocab_size=4096, num_layers=6,
                          num_heads=4, num_kv_heads=2, head_dim=256, rotary_dim=128,
                          layer_full=[0, 0, 1, 0, 0, 1], max_prefill_tokens=16, sliding_window=16)
# (token, clock, with logits): repeated clocks rewrite a slot with the same
# values, so the stream entering the first gated layer does not move
STEPS_Q = [(5, 0, True), (5, 0, True), (9, 1, True), (9, 1, False), (9, 1, True), (9, 1, True),
           (3, 2, True), (4, 3, True), (4, 3, True)]


def _quiescence_oracle(W, thresh):
    """The steps through the oracle; per step its outputs and the K/V rows of
    slots 0..3 of every layer after it."""
    qs = OM.QuiescenceState(CFG_Q, thresh)
    kc, vc = OM.new_caches(CFG_Q, 4096)
    kvd = CFG_Q["num_kv_heads"] * CFG_Q["head_dim"]
    outs, kv = [], []
    for tok, clock, logits in STEPS_Q:
        act, sl = OM.slot_lists(clock, 16)
        outs.append(OM.decode_step(W, kc, vc, W.embed([tok])[0], clock, clock, act, sl, with_logits=logits,
                                   qstate=qs))
        kv.append([(k[: 4 * kvd].reshape(4, kvd).copy(), v[: 4 * kvd].reshape(4, kvd).copy()) for k, v in zip(kc, vc)])
    return qs, outs, kv


def test_quiescence_gating_matches_oracle(ctx):
    """Quiescence-gated decode (src/gpu/model_dispatch.zig:47-126,
    shaders/quiescence_gate.wgsl) against the oracle's gated composition:
    the stream, the normed row, the top-64 and every K/V row after each step
    (quiescent layers write no K/V).  The threshold is chosen from the
    oracle's own gate values, at least 1% away from every one of them, with
    both outcomes present and some layers quiescent although their stream
    moved, so rounding cannot flip a decision."""
    layers, embed, final = OM.random_model(CFG_Q, 41)
    W = OM.Weights(CFG_Q, layers, embed, final)
    chosen = None
    for thresh in np.geomspace(1e-5, 10.0, 61):
        qs, outs, kv = _quiescence_oracle(W, thresh)
        gates = [g for step in qs.log for g in step]
        margin = min((abs(np.log(g[2] / thresh)) for g in gates if g[2] > 0), default=np.inf)
        moved_skips = sum(1 for g in gates if not g[1] and g[2] > 0)
        if margin > 0.01 and any(g[1] for g in gates) and moved_skips >= 2:
            chosen = (float(thresh), qs, outs, kv)
            break
    assert chosen is not None
    thresh, qs, outs, kv_o = chosen
    say(f"quiescence threshold {thresh:.3g}; quiescent layers per step: "
        f"{[[g[0] for g in step if not g[1]] for step in qs.log]}")
    with Model.create(ctx, dict(CFG_Q, quiescence_thresh=thresh), layers, embed, final) as m:
        for s, (tok, clock, logits) in enumerate(STEPS_Q):
            act, sl = OM.slot_lists(clock, 16)
            say(f"gated decode step {s}: token {tok} clock {clock} logits {logits}")
            _, ids, vals = m.forward_token(W.embed([tok])[0], clock, clock, act, sl, topk=logits)
            x_o, n_o, lg_o, _, _ = outs[s]
            x_g, n_g = m.read_state()
            assert rel_err(x_g, x_o) < 1e-3 and rel_err(n_g, n_o) < 1e-3
            if logits:
                assert_topk_valid(ids, vals, lg_o, 1e-3, f"gated step {s}")
            for i in range(CFG_Q["num_layers"]):
                k, v = m.kv_read(i, 0, 4)
                k_o, v_o = kv_o[s][i]
                assert np.array_equal(k == 0, k_o == 0), (s, i)      # the same rows written
                assert rel_err(k, k_o) < 1e-3 and rel_err(v, v_o) < 1e-3, (s, i)


def _gated_greedy_oracle(W, thresh, tok0, n):
    """n greedy steps from clock 0 through the oracle's gated composition:
    its tokens, per step its outputs and the relative top-2 margin."""
    qs = OM.QuiescenceState(CFG_Q, thresh)
    kc, vc = OM.new_caches(CFG_Q, 4096)
    toks, outs, margins = [], [], []
    tok = tok0
    for clock in range(n):
        act, sl = OM.slot_lists(clock, 16)
        out = OM.decode_step(W, kc, vc, W.embed([tok])[0], clock, clock, act, sl, with_logits=True, qstate=qs)
        vals = out[4].astype(np.float64)
        margins.append((vals[0] - vals[1]) / np.max(np.abs(vals)))
        tok = int(out[3][0])
        toks.append(tok)
        outs.append(out)
    return qs, toks, outs, margins, kc, vc


def test_gated_greedy_matches_token_loop_and_oracle(ctx):
    """chn_decode_greedy with quiescence gating on (every greedy step
    computes logits, so layers from num_layers / 3 on are gated): its tokens,
    state and K/V rows equal the gated token loop (chn_decode_token with the
    same lists) bit for bit, and both follow the oracle's gated greedy run:
    the same tokens, the stream and normed row within 1e-3 at every step,
    and the same layers quiescent (a quiescent layer writes no K/V row).
    The threshold is chosen from the oracle's own gate values along the
    greedy run: at least 5% away from every one of them, with both outcomes
    present, and every step's argmax ahead of the runner-up by at least 2e-3
    of the largest value, so rounding can flip neither a gate nor a token."""
    layers, embed, final = OM.random_model(CFG_Q, 41)
    W = OM.Weights(CFG_Q, layers, embed, final)
    n, tok0 = 8, 17
    best = None
    for thresh in np.geomspace(1e-3, 10.0, 41):
        qs, toks, outs, margins, kc, vc = _gated_greedy_oracle(W, thresh, tok0, n)
        gates = [g for step in qs.log for g in step]
        gm = min((abs(np.log(g[2] / thresh)) for g in gates if g[2] > 0), default=np.inf)
        skips = sum(1 for g in gates if not g[1])
        runs = len(gates) - skips
        if gm > 0.05 and min(margins) >= 2e-3 and skips >= 2 and runs >= 2:
            if best is None or min(skips, runs) > best[0]:
                best = (min(skips, runs), float(thresh), qs, toks, outs, kc, vc)
    assert best is not None
    _, thresh, qs, toks_o, outs, kc_o, vc_o = best
    kvd = CFG_Q["num_kv_heads"] * CFG_Q["head_dim"]
    say(f"gated greedy: threshold {thresh:.3g}; quiescent layers per step: "
        f"{[[g[0] for g in step if not g[1]] for step in qs.log]}")
    cfg = dict(CFG_Q, quiescence_thresh=thresh)
    with Model.create(ctx, cfg, layers, embed, final) as mg, Model.create(ctx, cfg, layers, embed, final) as mh:
        say("decode_greedy 8 gated steps")
        toks_g = mg.decode_greedy(tok0, 0, n)
        tok, want = tok0, []
        for clock in range(n):
            act, sl = OM.slot_lists(clock, 16)
            say(f"gated token loop clock={clock} tok={tok}")
            tok, ids, vals = mh.forward_token_id(tok, clock, clock, act, sl)
            want.append(tok)
            x_o, n_o, lg_o, _, _ = outs[clock]
            x_h, n_h = mh.read_state()
            assert rel_err(x_h, x_o) < 1e-3 and rel_err(n_h, n_o) < 1e-3, clock
            assert_topk_valid(ids, vals, lg_o, 1e-3, f"gated greedy step {clock}")
        assert list(toks_g) == want == toks_o
        xg, ng = mg.read_state()
        xh, nh = mh.read_state()
        assert np.array_equal(xg, xh) and np.array_equal(ng, nh)
        for i in range(CFG_Q["num_layers"]):
            kg, vg = mg.kv_read(i, 0, n)
            kh, vh = mh.kv_read(i, 0, n)
            assert np.array_equal(kg, kh) and np.array_equal(vg, vh), i
            k_o = kc_o[i][: n * kvd].reshape(n, kvd)
            v_o = vc_o[i][: n * kvd].reshape(n, kvd)
            assert np.array_equal(np.all(kg == 0, axis=1), np.all(k_o == 0, axis=1)), i   # same rows written
            assert rel_err(kg, k_o) < 1e-3 and rel_err(vg, v_o) < 1e-3, i


def test_prefill_window_option(ctx):
    """prefill_window = sliding_window makes the prefill's sliding layers
    use the decode window instead of the reference's fixed 1024."""
    cfg = dict(CFG, prefill_window=WINDOW, num_layers=2, layer_full=[0, 1])
    layers, embed, final = OM.random_model(cfg, 55)
    W = OM.Weights(cfg, layers, embed, final)
    toks = [int(t) for t in np.random.default_rng(55).integers(0, cfg["vocab_size"], 40)]
    say("prefill with prefill_window 16")
    with Model.create(ctx, cfg, layers, embed, final) as m:
        lg, ids, vals = m.prefill_batch(toks, np.arange(40), 0, 0, embed_bf16=W.embed_bf16)
    kc, vc = OM.new_caches(cfg, 4096)
    _, _, lg16, _, _ = OM.prefill(W, kc, vc, toks, np.arange(40), 0, 0, bf16_gemm=True, window=WINDOW)
    kc, vc = OM.new_caches(cfg, 4096)
    _, _, lg1024, _, _ = OM.prefill(W, kc, vc, toks, np.arange(40), 0, 0, bf16_gemm=True, window=1024)
    assert rel_err(lg, lg16) < 1e-2
    assert rel_err(lg16, lg1024) > 1e-2          # the window matters at 40 tokens


def test_prefill_window_second_chunk(ctx):
    """A second prefill chunk after 64 previous keys (whole 32-key chunks)
    under prefill_window 16: the attention's first key chunk is an earlier
    one (its operand fragments built from the caches) and the new keys'
    fragments come with their RMSNorm + RoPE.  Logits, top-64 and the new
    K/V rows against the oracle run through the same two chunks."""
    cfg = dict(CFG, prefill_window=WINDOW, num_layers=2, layer_full=[0, 1])
    layers, embed, final = OM.random_model(cfg, 56)
    W = OM.Weights(cfg, layers, embed, final)
    kvd = cfg["num_kv_heads"] * cfg["head_dim"]
    toks = [int(t) for t in np.random.default_rng(56).integers(0, cfg["vocab_size"], 104)]
    slots = np.arange(104, dtype=np.uint32)
    kc, vc = OM.new_caches(cfg, 4096)
    with Model.create(ctx, cfg, layers, embed, final) as m:
        say("prefill chunk 1: 64 tokens, prefill_window 16")
        m.prefill_batch(toks[:64], slots[:64], 0, 0, embed_bf16=W.embed_bf16, logits=False, topk=False)
        OM.prefill(W, kc, vc, toks[:64], slots[:64], 0, 0, bf16_gemm=True, window=WINDOW)
        say("prefill chunk 2: 40 tokens over 64 previous slots")
        lg, ids, vals = m.prefill_batch(toks[64:], slots, 64, 64, embed_bf16=W.embed_bf16)
        _, _, lg_o, _, _ = OM.prefill(W, kc, vc, toks[64:], slots, 64, 64, bf16_gemm=True, window=WINDOW)
        kv = [m.kv_read(i, 64, 40) for i in range(cfg["num_layers"])]
    assert rel_err(lg, lg_o) < 1e-2
    assert_topk_valid(ids, vals, lg_o, 1e-2, "second prefill chunk, window 16")
    for i, (k_g, v_g) in enumerate(kv):
        ek = rel_err(k_g.ravel(), kc[i][64 * kvd:104 * kvd])
        ev = rel_err(v_g.ravel(), vc[i][64 * kvd:104 * kvd])
        say(f"  layer {i}: new K rows {ek:.2e}, V rows {ev:.2e}")
        assert ek < 1e-2 and ev < 1e-2


def test_k_eq_v_model_prefill_then_decode(ctx):
    """attention_k_eq_v with v_proj absent (src/gpu/model_gpu.zig:123): V's
    projection is k_proj's and V is the raw K row under a unit RMSNorm, in
    the prefill's RoPE + fragment kernel and in the decode step's fused
    attention.  Prefill logits, every K/V row, then two decode steps from
    the GPU's caches, against the oracle."""
    cfg = dict(CFG, k_eq_v=1, num_layers=2, layer_full=[0, 1])
    layers, embed, final = OM.random_model(cfg, 57)
    for l in layers:
        l["v_proj"] = None
    W = OM.Weights(cfg, layers, embed, final)
    kvd = cfg["num_kv_heads"] * cfg["head_dim"]
    toks = [int(t) for t in np.random.default_rng(57).integers(0, cfg["vocab_size"], 40)]
    n = len(toks)
    kc, vc = OM.new_caches(cfg, 4096)
    with Model.create(ctx, cfg, layers, embed, final) as m:
        say("k_eq_v model: prefill 40 tokens")
        lg, ids, vals = m.prefill_batch(toks, np.arange(n), 0, 0, embed_bf16=W.embed_bf16)
        _, _, lg_o, _, _ = OM.prefill(W, kc, vc, toks, np.arange(n), 0, 0, bf16_gemm=True, window=1024)
        assert rel_err(lg, lg_o) < 1e-2
        assert_topk_valid(ids, vals, lg_o, 1e-2, "k_eq_v prefill")
        for i in range(cfg["num_layers"]):
            k_g, v_g = m.kv_read(i, 0, n)
            assert rel_err(k_g, kc[i][: n * kvd].reshape(n, kvd)) < 1e-2
            assert rel_err(v_g, vc[i][: n * kvd].reshape(n, kvd)) < 1e-2
            kc[i][: n * kvd] = k_g.ravel()
            vc[i][: n * kvd] = v_g.ravel()
        tok = int(ids[0])
        for clock in range(n, n + 2):
            active, sliding = OM.slot_lists(clock, WINDOW)
            x_in = W.embed([tok])[0]
            say(f"k_eq_v model: decode clock={clock}")
            _, ids_g, vals_g = m.forward_token(x_in, clock, clock, active, sliding)
            x_o, nx_o, lg_o, _, _ = OM.decode_step(W, kc, vc, x_in, clock, clock, active, sliding)
            assert_topk_valid(ids_g, vals_g, lg_o, 1e-3, f"k_eq_v decode clock {clock}")
            x_g, _ = m.read_state()
            assert rel_err(x_g, x_o) < 1e-3
            for i in range(cfg["num_layers"]):
                k_g, v_g = m.kv_read(i, clock, 1)
                assert rel_err(k_g[0], kc[i][clock * kvd:(clock + 1) * kvd]) < 1e-3
                assert rel_err(v_g[0], vc[i][clock * kvd:(clock + 1) * kvd]) < 1e-3
            tok = int(ids_g[0])
