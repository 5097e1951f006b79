"""GPU parity of the model at the 12B-class shapes the benchmark runs:
hidden 3840, FFN 15360, 16 query / 8 KV heads, head_dim 256, vocab 262144,
sliding window 512, theta 1e4 (sliding) / 1e6 (full).

* Two layers (one sliding, one full) of the seeded synthetic model: a
  512-token prefill (the benchmark's prompt, so the prefill GEMMs take the
  same tile shapes: q/k/v in one launch on 128 x 128 tiles, down split in
  K, gate/up writing bf16) against the oracle's bf16-operand model
  (normwise 1e-2 on logits, every K/V row and the last normed row), then
  four decode steps through chn_decode_token against the oracle in fp32
  (1e-3), starting from the GPU's caches.  The decode steps run the fused
  norm prologues at K = 3840, down at K = 15360 and the attention with
  fused RoPE for 16 heads.
* Two layers over full 4096-slot rings, decoding across the ring's wrap at
  clock 3968 with ~3968-entry global lists, against the oracle in fp32.
* All 48 layers after the benchmark's 512-token prompt: chn_decode_greedy
  against the same steps driven token by token (bit for bit), and every
  step's top-64 against the oracle's Q8 logits of the downloaded final
  normed row.

The synthetic weights are regenerated on the host by the oracle's
restatement of the generator (bit-exact, tests/test_gpu_golden.py); the
bf16 embedding is downloaded and quantized to Q8 by the oracle.
"""
import ctypes

import numpy as np
import pytest

import channel_amd as ca
import oracle as O
from channel_amd import ring
from channel_amd.model import Model
from gpu_util import assert_topk_valid, rel_err, say
from oracle import model as OM

pytestmark = pytest.mark.gpu

SEED = 0xC4A77E1 + 4
CFG2 = OM.default_config(num_layers=2, layer_full=[0, 1], max_prefill_tokens=512)
NT = O.NTHREADS


def elem_err(got, want):
    """Largest elementwise relative error over entries at least 1e-3 of the
    largest magnitude (smaller entries are compared normwise only)."""
    g = np.asarray(got, np.float64).ravel()
    w = np.asarray(want, np.float64).ravel()
    big = np.abs(w) >= 1e-3 * np.max(np.abs(w))
    return float(np.max(np.abs(g[big] - w[big]) / np.abs(w[big])))


def embedding(ctx, m):
    p = ctypes.c_void_p()
    assert ca.lib.chn_model_embedding_bf16(m.handle, ctypes.byref(p)) == 0 and p.value
    c = m.config
    return ctx.download(p.value, np.uint16, c.vocab_size * c.hidden_size).reshape(c.vocab_size, c.hidden_size)


@pytest.fixture(scope="module")
def two_layers(ctx):
    say("model_create_synthetic: 2 layers at 12B dims")
    m = Model.synthetic(ctx, CFG2, SEED)
    say("regenerate weights on the host, Q8 embedding")
    W = OM.Weights.synthetic(CFG2, SEED, embedding(ctx, m), NT)
    yield W, m
    m.close()


def test_12b_layers_prefill_512_then_decode(two_layers):
    W, m = two_layers
    n = 512
    kvd = CFG2["num_kv_heads"] * CFG2["head_dim"]
    toks = np.random.default_rng(12).integers(0, CFG2["vocab_size"], n).astype(np.uint32)
    slots = np.arange(n, dtype=np.uint32)
    say("prefill 512 tokens at 12B dims")
    lg, ids, vals = m.prefill_batch(toks, slots, 0, 0)
    say("oracle prefill (bf16 operands)")
    kc, vc = OM.new_caches(CFG2)
    _, Xn, lg_o, _, _ = OM.prefill(W, kc, vc, toks, slots, 0, 0, bf16_gemm=True, window=1024, nthreads=NT)
    e = rel_err(lg, lg_o)
    say(f"  prefill logits: normwise {e:.2e}, elementwise {elem_err(lg, lg_o):.2e}")
    assert e < 1e-2
    assert_topk_valid(ids, vals, lg_o, 1e-2, "prefill")
    for i in range(2):
        k, v = m.kv_read(i, 0, n)
        ek = rel_err(k, kc[i][: n * kvd].reshape(n, kvd))
        ev = rel_err(v, vc[i][: n * kvd].reshape(n, kvd))
        say(f"  layer {i} K/V rows: {ek:.2e} / {ev:.2e}")
        assert ek < 1e-2 and ev < 1e-2
        kc[i][: n * kvd] = k.ravel()          # decode continues from the GPU's caches
        vc[i][: n * kvd] = v.ravel()
    _, normed = m.read_state()
    assert rel_err(normed, Xn[n - 1]) < 1e-2

    tok = int(ids[0])
    for clock in range(n, n + 4):
        slot, active, sliding = ring.decode_lists(clock, CFG2["sliding_window"])
        say(f"decode clock={clock} tok={tok}")
        t_gpu, ids_g, vals_g = m.forward_token_id(tok, clock, slot, active, sliding)
        x_in = W.embed([tok])[0]
        x_o, nx_o, lg_o, _, _ = OM.decode_step(W, kc, vc, x_in, clock, slot, active, sliding, nthreads=NT)
        x_g, nx_g = m.read_state()
        ex, en = rel_err(x_g, x_o), rel_err(nx_g, nx_o)
        say(f"  x {ex:.2e} (elementwise {elem_err(x_g, x_o):.2e}), normed {en:.2e}")
        assert ex < 1e-3 and en < 1e-3
        assert t_gpu == ids_g[0]
        assert_topk_valid(ids_g, vals_g, lg_o, 1e-3, f"decode {clock}")
        for i in range(2):
            k_g, v_g = m.kv_read(i, slot, 1)
            assert rel_err(k_g[0], kc[i][slot * kvd:(slot + 1) * kvd]) < 1e-3
            assert rel_err(v_g[0], vc[i][slot * kvd:(slot + 1) * kvd]) < 1e-3
        tok = int(ids_g[0])


def test_12b_layers_prefill_ragged_tiles(two_layers):
    """A 300-token prefill at the 12B layer dims: every contraction's last
    token tile is ragged (300 = 256 + 44 for the 256-token tiles of gate/up
    and of down, whose K is split four ways; 2 x 128 + 44 for q/k/v and o)
    and the attention's last query tile holds 44 of its 64 tokens; then a
    second chunk of 212 tokens over those 300 slots.  Against the oracle's
    bf16-operand model as the 512-token test: logits, every K/V row of both
    layers and the last normed row; then a third chunk of 100 tokens after
    the 512 slots (the new keys start a 32-key chunk)."""
    W, m = two_layers
    n = 300
    kvd = CFG2["num_kv_heads"] * CFG2["head_dim"]
    toks = np.random.default_rng(300).integers(0, CFG2["vocab_size"], n).astype(np.uint32)
    slots = np.arange(n, dtype=np.uint32)
    say("prefill 300 tokens at 12B dims")
    lg, ids, vals = m.prefill_batch(toks, slots, 0, 0)
    kc, vc = OM.new_caches(CFG2)
    _, Xn, lg_o, _, _ = OM.prefill(W, kc, vc, toks, slots, 0, 0, bf16_gemm=True, window=1024, nthreads=NT)
    e = rel_err(lg, lg_o)
    say(f"  prefill logits: normwise {e:.2e}, elementwise {elem_err(lg, lg_o):.2e}")
    assert e < 1e-2
    assert_topk_valid(ids, vals, lg_o, 1e-2, "prefill 300")
    for i in range(2):
        k, v = m.kv_read(i, 0, n)
        ek = rel_err(k, kc[i][: n * kvd].reshape(n, kvd))
        ev = rel_err(v, vc[i][: n * kvd].reshape(n, kvd))
        tail = rel_err(k[256:], kc[i][256 * kvd: n * kvd].reshape(n - 256, kvd))
        say(f"  layer {i} K/V rows: {ek:.2e} / {ev:.2e}; K rows 256..299 {tail:.2e}")
        assert ek < 1e-2 and ev < 1e-2 and tail < 1e-2
        kc[i][: n * kvd] = k.ravel()          # the second chunk starts from the GPU's caches
        vc[i][: n * kvd] = v.ravel()
    _, normed = m.read_state()
    assert rel_err(normed, Xn[n - 1]) < 1e-2

    # a second chunk of 212 tokens over the 300 previous slots: the key list's
    # 32-key chunk 9 holds 12 previous and 20 new keys, and every contraction
    # runs one ragged token tile (212 < 256)
    n2 = 212
    toks2 = np.random.default_rng(212).integers(0, CFG2["vocab_size"], n2).astype(np.uint32)
    slots2 = np.arange(n + n2, dtype=np.uint32)
    say("prefill 212 more tokens after 300 previous slots")
    lg2, ids2, vals2 = m.prefill_batch(toks2, slots2, n, n)
    _, Xn2, lg2_o, _, _ = OM.prefill(W, kc, vc, toks2, slots2, n, n, bf16_gemm=True, window=1024, nthreads=NT)
    e2 = rel_err(lg2, lg2_o)
    say(f"  second chunk logits: normwise {e2:.2e}")
    assert e2 < 1e-2
    assert_topk_valid(ids2, vals2, lg2_o, 1e-2, "prefill 212 after 300")
    for i in range(2):
        k, v = m.kv_read(i, n, n2)
        ek = rel_err(k, kc[i][n * kvd:(n + n2) * kvd].reshape(n2, kvd))
        ev = rel_err(v, vc[i][n * kvd:(n + n2) * kvd].reshape(n2, kvd))
        say(f"  layer {i} new K/V rows: {ek:.2e} / {ev:.2e}")
        assert ek < 1e-2 and ev < 1e-2
        kc[i][n * kvd:(n + n2) * kvd] = k.ravel()
        vc[i][n * kvd:(n + n2) * kvd] = v.ravel()
    _, normed = m.read_state()
    assert rel_err(normed, Xn2[n2 - 1]) < 1e-2

    # a third chunk of 100 tokens after 512 previous slots (whole 32-key
    # chunks): the new keys' operand fragments come with their RoPE, the 16
    # earlier chunks' from the caches
    n0, n3 = n + n2, 100
    toks3 = np.random.default_rng(100).integers(0, CFG2["vocab_size"], n3).astype(np.uint32)
    slots3 = np.arange(n0 + n3, dtype=np.uint32)
    say("prefill 100 more tokens after 512 previous slots")
    lg3, ids3, vals3 = m.prefill_batch(toks3, slots3, n0, n0)
    _, Xn3, lg3_o, _, _ = OM.prefill(W, kc, vc, toks3, slots3, n0, n0, bf16_gemm=True, window=1024, nthreads=NT)
    e3 = rel_err(lg3, lg3_o)
    say(f"  third chunk logits: normwise {e3:.2e}")
    assert e3 < 1e-2
    assert_topk_valid(ids3, vals3, lg3_o, 1e-2, "prefill 100 after 512")
    for i in range(2):
        k, v = m.kv_read(i, n0, n3)
        ek = rel_err(k, kc[i][n0 * kvd:(n0 + n3) * kvd].reshape(n3, kvd))
        ev = rel_err(v, vc[i][n0 * kvd:(n0 + n3) * kvd].reshape(n3, kvd))
        say(f"  layer {i} new K/V rows: {ek:.2e} / {ev:.2e}")
        assert ek < 1e-2 and ev < 1e-2
    _, normed = m.read_state()
    assert rel_err(normed, Xn3[n3 - 1]) < 1e-2


def test_12b_layers_decode_full_ring_across_wrap(two_layers):
    """Decode at the 12B layer dims over full rings: every one of the 4096
    slots of both layers holds K/V rows (the same random rows on both
    sides), then four steps at clocks 3966..3969 through chn_decode_token
    with the lists of the ring restatement (oracle/ring.py, no anchors):
    3967 and 3968 entries in the global list, the window wrapping at 3968
    (clocks 3968 and 3969 take slots 0 and 1, and the list runs 2..3967,
    0, 1), the sliding list the newest 512.  Against the oracle in fp32:
    x, the normed row and the K/V rows written within 1e-3, the top-64
    valid.  This is the model's attention with fused RoPE on ~3968-entry
    lists, which the chunked greedy tests compare only with other HIP paths."""
    from oracle.ring import Ring
    from oracle import ring as OR
    W, m = two_layers
    kvd = CFG2["num_kv_heads"] * CFG2["head_dim"]
    rng = np.random.default_rng(3968)
    kc, vc = OM.new_caches(CFG2)
    for i in range(2):
        k = (rng.standard_normal((4096, kvd)) * 0.05).astype(np.float32)
        v = rng.standard_normal((4096, kvd)).astype(np.float32)
        say(f"fill all 4096 slots of layer {i}")
        m.kv_write(i, 0, k, v)
        kc[i][:] = k.ravel()
        vc[i][:] = v.ravel()
    ring = Ring(1, 0)
    clock0 = 3966
    for c in range(clock0):
        ring.activate_slot(0, c)
    tok = 4242
    for clock in range(clock0, clock0 + 4):
        slot, active, sliding = OR.decode_lists(ring, clock, CFG2["sliding_window"])
        active = np.asarray(active, np.uint32)
        sliding = np.asarray(sliding, np.uint32)
        assert len(active) >= 3967 and len(sliding) == 512
        say(f"decode clock={clock} slot={slot} global {len(active)} entries (first {active[0]}, last "
            f"{active[-1]}), sliding {len(sliding)}")
        t_gpu, ids_g, vals_g = m.forward_token_id(tok, clock, slot, active, sliding)
        x_o, nx_o, lg_o, _, _ = OM.decode_step(W, kc, vc, W.embed([tok])[0], clock, slot, active, sliding,
                                               nthreads=NT)
        x_g, nx_g = m.read_state()
        ex, en = rel_err(x_g, x_o), rel_err(nx_g, nx_o)
        say(f"  x {ex:.2e} (elementwise {elem_err(x_g, x_o):.2e}), normed {en:.2e}")
        assert ex < 1e-3 and en < 1e-3
        assert t_gpu == ids_g[0]
        assert_topk_valid(ids_g, vals_g, lg_o, 1e-3, f"full-ring decode {clock}")
        for i in range(2):
            k_g, v_g = m.kv_read(i, slot, 1)
            ek = rel_err(k_g[0], kc[i][slot * kvd:(slot + 1) * kvd])
            ev = rel_err(v_g[0], vc[i][slot * kvd:(slot + 1) * kvd])
            assert ek < 1e-3 and ev < 1e-3, (i, ek, ev)
        if clock >= 3968:
            assert slot == clock - 3968 and active[-1] == slot and active[0] == clock - 3967
        tok = int(ids_g[0])


def test_12b_48_layers_greedy(ctx):
    """The full 48-layer model: device-resident greedy steps equal the
    token-by-token steps bit for bit, and every step's top-64 is the top-64
    of the oracle's Q8 logits of that step's final normed row."""
    cfg = OM.default_config(max_prefill_tokens=512)
    say("model_create_synthetic x2: 48 layers at 12B dims")
    with Model.synthetic(ctx, cfg, SEED) as mg, Model.synthetic(ctx, cfg, SEED) as mh:
        emb = embedding(ctx, mg)
        E8 = O.quantize_q8(emb, NT)
        del emb
        n_prompt = 512                     # the benchmark's prompt
        prompt = np.random.default_rng(48).integers(0, cfg["vocab_size"], n_prompt).astype(np.uint32)
        slots = np.arange(n_prompt, dtype=np.uint32)
        say("prefill 512 tokens on both")
        _, ids_g, vals_g = mg.prefill_batch(prompt, slots, 0, 0, logits=False)
        _, ids_h, vals_h = mh.prefill_batch(prompt, slots, 0, 0, logits=False)
        assert np.array_equal(ids_g, ids_h) and np.array_equal(vals_g, vals_h)
        n = 5
        say("decode_greedy 5 steps")
        toks = mg.decode_greedy(int(ids_g[0]), n_prompt, n)
        tok, want = int(ids_h[0]), []
        for i in range(n):
            clock = n_prompt + i
            slot, active, sliding = ring.decode_lists(clock, cfg["sliding_window"])
            say(f"token loop clock={clock}")
            tok, ids, vals = mh.forward_token_id(tok, clock, slot, active, sliding)
            _, normed = mh.read_state()
            lg = O.gemv_q8(E8, normed, cfg["vocab_size"], cfg["hidden_size"], NT)
            assert_topk_valid(ids, vals, lg, 1e-3, f"48-layer step {clock}")
            want.append(tok)
        assert list(toks) == want
        xg, ng = mg.read_state()
        xh, nh = mh.read_state()
        assert np.array_equal(xg, xh) and np.array_equal(ng, nh)
