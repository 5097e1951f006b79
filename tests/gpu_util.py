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


def assert_topk_valid(ids, vals, logits_want, tol, label=""):
    """ids/vals must be the top-64 of softcap(logits_want) up to the error
    bound atol = tol * max|value|:

    * ids are distinct and every value is within atol of the exact value at
      its rank;
    * where the id at a rank differs from the oracle's, the GPU's id must be
      a near-tie: its exact capped value lies within 2 * atol of the exact
      value at that rank (each such rank is reported with its margin);
    * the argmax (rank 0, the greedy token) must equal the oracle's unless
      the oracle's own top-2 margin is below 2 * atol (reported).

    Returns (number of ranks whose id matches, list of reported ranks)."""
    import oracle
    ids = np.asarray(ids, np.int64)
    capped = oracle.softcap(logits_want).astype(np.float64)
    want_ids, want_vals = oracle.topk64(logits_want)
    want_vals = want_vals.astype(np.float64)
    atol = tol * float(np.max(np.abs(want_vals)))
    assert len(set(int(i) for i in ids)) == 64, f"{label}: repeated ids"
    dv = np.abs(np.asarray(vals, np.float64) - want_vals)
    assert np.all(dv <= atol), f"{label}: value error {dv.max():.3g} > {atol:.3g}"
    flagged = []
    for k in np.nonzero(ids != want_ids.astype(np.int64))[0]:
        margin = abs(capped[ids[k]] - want_vals[k])
        flagged.append((int(k), int(ids[k]), int(want_ids[k]), margin))
        say(f"  {label} near-tie at rank {k}: id {ids[k]} for {want_ids[k]}, "
            f"exact values differ by {margin:.3g} (bound {2 * atol:.3g})")
        assert margin <= 2 * atol, f"{label}: rank {k} reordered by {margin:.3g} > {2 * atol:.3g}"
    if ids[0] != want_ids[0]:
        top2 = want_vals[0] - want_vals[1]
        assert top2 <= 2 * atol, f"{label}: argmax {ids[0]} != {want_ids[0]} with oracle top-2 margin {top2:.3g}"
    n_match = 64 - len(flagged)
    say(f"  {label} top-64: {n_match}/64 ranks identical")
    return n_match, flagged
