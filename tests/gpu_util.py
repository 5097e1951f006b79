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
