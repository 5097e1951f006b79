"""chn_decode_attn_noalloc, the allocation-free decode attention: the split
partials live in a file-scope device array, not in the context workspace.
Through the C-ABI, its output must equal chn_decode_attn's bit for bit (the
same kernels on another buffer), on consecutive calls in which a later call
is smaller than an earlier one (the array keeps the previous call's
contents), and the oracle's within the fp32 bar.  Shapes beyond the array
are refused."""
import numpy as np
import pytest

import channel_amd as ca
import oracle
from gpu_util import f32_host, rel_err, say, synth_normal_dev

pytestmark = pytest.mark.gpu


def _case(ctx, H, gqa, D, S, max_slots, seed):
    kvh = H // gqa
    kv_dim = kvh * D
    nslot = 4096
    Kc = synth_normal_dev(ctx, nslot * kv_dim, seed)
    Vc = synth_normal_dev(ctx, nslot * kv_dim, seed + 1)
    Q = synth_normal_dev(ctx, H * D, seed + 2, 0.1)
    perm = np.random.default_rng(seed).permutation(nslot).astype(np.uint32)[:max_slots]
    slots = ctx.upload(perm)
    ns = ctx.upload(np.array([S], np.uint32))
    a, b = ctx.alloc(H * D * 4), ctx.alloc(H * D * 4)
    say(f"decode_attn_noalloc H={H} gqa={gqa} D={D} S={S} max_slots={max_slots}")
    ctx.call("chn_decode_attn_noalloc", Q, Kc, Vc, slots, ns, max_slots, H, D, kv_dim, gqa, 1.0, a)
    ctx.call("chn_decode_attn", Q, Kc, Vc, slots, ns, max_slots, H, D, kv_dim, gqa, 1.0, b)
    got, ref = f32_host(ctx, a, H * D), f32_host(ctx, b, H * D)
    assert np.array_equal(got, ref)
    want = oracle.decode_attn(f32_host(ctx, Q, H * D), f32_host(ctx, Kc, nslot * kv_dim),
                              f32_host(ctx, Vc, nslot * kv_dim), perm[:S], H, D, kv_dim, gqa, 1.0)
    assert rel_err(got, want) < 1e-3


def test_decode_attn_noalloc_matches_decode_attn(ctx):
    # the 12B full-attention layer over the whole ring, then smaller calls
    # that leave stale partials of the first one in the array
    _case(ctx, 16, 2, 256, 4096, 4096, 8100)
    _case(ctx, 4, 1, 256, 37, 64, 8200)
    _case(ctx, 8, 2, 512, 300, 512, 8300)
    _case(ctx, 16, 2, 256, 0, 512, 8400)       # empty list: zeros


def test_decode_attn_noalloc_refuses_oversize(ctx):
    H, D = 32, 512                              # 32 * 514 * 32 splits * 4 B > 2 MiB
    buf = ctx.zeros(4096 * H * D * 4)
    slots = ctx.upload(np.arange(4096, dtype=np.uint32))
    ns = ctx.upload(np.array([10], np.uint32))
    with pytest.raises(ca.ChannelError) as e:
        ctx.call("chn_decode_attn_noalloc", buf, buf, buf, slots, ns, 4096, H, D, H * D, 1, 1.0, buf)
    assert e.value.status == "Unsupported"
    # the same shape over a short list fits (fewer splits)
    out = ctx.alloc(H * D * 4)
    ctx.call("chn_decode_attn_noalloc", buf, buf, buf, slots, ns, 256, 8, D, 8 * D, 1, 1.0, out)
