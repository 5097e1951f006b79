"""Recordings (chn_record_begin / chn_record_end / chn_submit, the reference's
pre-recorded command buffers, src/gpu/kernels.zig:89-194): a recorded
sequence replays bit for bit like the same calls run one by one, on every
submission, with the program's own eager work and synchronizations between
submissions; and the misuse cases are refused on the host."""
import numpy as np
import pytest

import channel_amd as ca
from channel_amd import Context
from gpu_util import f32_host, say, synth_normal_dev, synth_q4_dev

pytestmark = pytest.mark.gpu


def _u32(ctx, arr):
    return ctx.upload(np.ascontiguousarray(arr, dtype=np.uint32))


def test_recording_replays_like_eager_calls(ctx):
    H, gqa, D, nslot, S = 16, 2, 256, 4096, 600
    kv_dim = H // gqa * D
    copies = 3
    K = [synth_normal_dev(ctx, nslot * kv_dim, 900 + c) for c in range(copies)]
    V = [synth_normal_dev(ctx, nslot * kv_dim, 910 + c) for c in range(copies)]
    q = synth_normal_dev(ctx, H * D, 920, 0.1)
    rng = np.random.default_rng(921)
    slots = _u32(ctx, rng.permutation(nslot))
    ns = _u32(ctx, [S])
    M, Kd = 3840, 4096
    W = synth_q4_dev(ctx, M, Kd, 922)
    x = synth_normal_dev(ctx, Kd, 923)
    out_e = [ctx.alloc(H * D * 4) for _ in range(copies)]
    out_r = [ctx.alloc(H * D * 4) for _ in range(copies)]
    y_e, y_r = ctx.alloc(M * 4), ctx.alloc(M * 4)

    say("record: eager reference calls")
    for c in range(copies):
        ctx.call("chn_decode_attn", q, K[c], V[c], slots, ns, nslot, H, D, kv_dim, gqa, 1.0, out_e[c])
    ctx.call("chn_gemv_q4", W, x, y_e, M, Kd)
    want = [f32_host(ctx, o, H * D) for o in out_e]
    want_y = f32_host(ctx, y_e, M)

    ctx.record_begin()
    for c in range(copies):
        ctx.call("chn_decode_attn", q, K[c], V[c], slots, ns, nslot, H, D, kv_dim, gqa, 1.0, out_r[c])
    ctx.call("chn_gemv_q4", W, x, y_r, M, Kd)
    rec = ctx.record_end()
    try:
        for rep in range(3):
            say(f"record: submission {rep}")
            # eager work between submissions: poison the outputs
            for o in out_r:
                ctx.fill_u32(o, 0x7FC00000 + rep, H * D)
            ctx.fill_u32(y_r, 0x7FC00000 + rep, M)
            ctx.sync()
            rec.submit()
            ctx.sync()
            for c in range(copies):
                got = f32_host(ctx, out_r[c], H * D)
                assert np.array_equal(got.view(np.uint32), want[c].view(np.uint32)), (rep, c)
            assert np.array_equal(f32_host(ctx, y_r, M).view(np.uint32), want_y.view(np.uint32)), rep
    finally:
        rec.free()


def test_recording_misuse_is_refused():
    with Context(0) as c2:
        x = synth_normal_dev(c2, 256, 930)
        W = synth_q4_dev(c2, 64, 256, 931)
        y = c2.alloc(64 * 4)
        c2.call("chn_gemv_q4", W, x, y, 64, 256)           # workspace sized for K = 256
        c2.record_begin()
        with pytest.raises(ca.ChannelError):
            c2.record_begin()                                # already recording
        c2.call("chn_gemv_q4", W, x, y, 64, 256)
        rec = c2.record_end()
        rec.submit()
        c2.sync()
        with pytest.raises(ca.ChannelError):
            c2.record_end()                                  # not recording
        # a call that would grow the workspace (here to the 4 MB of bf16
        # activations of a 512 x 4096 contraction) is refused while recording
        n_tok, Kb = 512, 4096
        Wb = synth_q4_dev(c2, 64, Kb, 932)
        Xb = synth_normal_dev(c2, n_tok * Kb, 933)
        Yb = c2.alloc(n_tok * 64 * 4)
        c2.record_begin()
        with pytest.raises(ca.ChannelError) as ei:
            c2.call("chn_batch_gemm_q4", Wb, Xb, Yb, n_tok, 64, Kb)
        assert "workspace" in str(ei.value)
        c2.record_end().free()
        # once the workspace has moved, the old recording is refused
        c2.call("chn_batch_gemm_q4", Wb, Xb, Yb, n_tok, 64, Kb)
        c2.sync()
        with pytest.raises(ca.ChannelError) as ei:
            rec.submit()
        assert "reallocated" in str(ei.value)
        rec.free()
        # a recording still live when its context is destroyed is released
        # by chn_destroy
        c2.record_begin()
        c2.call("chn_gemv_q4", W, x, y, 64, 256)
        live = c2.record_end()
        live.submit()
        c2._recs.remove(live)
