"""Helpers shared by the GPU parity tests."""
import sys

import numpy as np

import channel_amd as ca


def rel_err(got, want):
    """Normwise relative error max|got - want| / max|want| (fp64)."""
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    return float(np.max(np.abs(g - w)) / max(np.max(np.abs(w)), 1e-30))


def say(*a):
    """Print and flush before a GPU step so a crash still names the case."""
    print(*a, flush=True)
    sys.stdout.flush()


def synth_q4_dev(ctx, rows, K, seed, smin=0.005, smax=0.02):
    buf = ctx.alloc(ca.q4_bytes(rows, K))
    ctx.call("chn_synth_q4", buf, rows, K, seed, smin, smax)
    return buf


def synth_normal_dev(ctx, n, seed, stddev=1.0):
    buf = ctx.alloc(n * 4)
    ctx.call("chn_synth_normal", buf, n, seed, stddev)
    return buf


def q4_host(ctx, buf, rows, K):
    return ctx.download(buf, np.uint32, rows * (K // 32) * 5)


def f32_host(ctx, buf, n, byte_offset=0):
    return ctx.download(buf, np.float32, n, byte_offset)


def assert_topk_valid(ids, vals, logits_want, tol):
    """ids/vals are a valid top-64 of softcap(logits_want) under tolerance:
    values match the exact top-64 within tol * max|value|, ids are distinct,
    and each id's exact capped value is within 2 * that of the value at its
    position (so only near-ties may be ordered differently)."""
    import oracle
    capped = oracle.softcap(logits_want)
    want_ids, want_vals = oracle.topk64(logits_want)
    atol = tol * float(np.max(np.abs(want_vals)))
    assert len(set(int(i) for i in ids)) == 64
    assert np.all(np.abs(np.asarray(vals, np.float64) - want_vals) <= atol)
    assert np.all(np.abs(capped[np.asarray(ids, np.int64)].astype(np.float64) - want_vals) <= 2 * atol)
    return int(np.sum(np.asarray(ids) == want_ids))
