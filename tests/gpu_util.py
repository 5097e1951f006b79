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
    """ids/vals must be the top-64 of softcap(logits_want), exactly up to the
    error the GPU's values actually carry.

    * The measured error delta = max |vals[k] - softcap(logits_want)[ids[k]]|
      over the 64 candidates (the GPU's value of each id it returned against
      that id's exact value) must be within the stated tolerance
      atol = tol * max|value|, and so must the value at every rank against
      the exact value at that rank.
    * A rank whose id differs from the oracle's is accepted only as a
      near-tie that this error explains: its exact value lies within
      bound = min(2 * delta + 4 ulp, 2 * atol) of the exact value at that
      rank.  (Sorting moves no value by more than the error, so a reordering
      by rounding alone never exceeds 2 * delta.)
    * The argmax (rank 0, the greedy token) must equal the oracle's unless
      the oracle's own top-2 margin is within the same bound.

    Prints, under `label`, the number of identical ranks, delta and the
    bound; every flagged rank is printed with its margin.
    Returns (number of ranks whose id matches, list of flagged ranks)."""
    import oracle
    ids = np.asarray(ids, np.int64)
    got = np.asarray(vals, np.float64)
    capped = oracle.softcap(logits_want).astype(np.float64)
    want_ids, want_vals = oracle.topk64(logits_want)
    want_vals = want_vals.astype(np.float64)
    vmax = float(np.max(np.abs(want_vals)))
    atol = tol * vmax
    assert len(set(int(i) for i in ids)) == 64, f"{label}: repeated ids"
    assert np.all((ids >= 0) & (ids < capped.size)), f"{label}: id out of range"
    delta = float(np.max(np.abs(got - capped[ids])))
    assert delta <= atol, f"{label}: value error {delta:.3g} at the returned ids > {atol:.3g}"
    dv = np.abs(got - want_vals)
    assert np.all(dv <= atol), f"{label}: value error {dv.max():.3g} at a rank > {atol:.3g}"
    ulp = float(np.spacing(np.float32(vmax)))
    bound = min(2.0 * delta + 4.0 * ulp, 2.0 * atol)
    flagged = []
    for k in np.nonzero(ids != want_ids.astype(np.int64))[0]:
        margin = abs(capped[ids[k]] - want_vals[k])
        flagged.append((int(k), int(ids[k]), int(want_ids[k]), margin))
        say(f"  {label} near-tie at rank {k}: id {ids[k]} for {want_ids[k]}, "
            f"exact values differ by {margin:.3g} (bound {bound:.3g})")
        assert margin <= bound, f"{label}: rank {k} reordered by {margin:.3g} > bound {bound:.3g}"
    if ids[0] != want_ids[0]:
        top2 = want_vals[0] - want_vals[1]
        assert top2 <= bound, f"{label}: argmax {ids[0]} != {want_ids[0]} with oracle top-2 margin {top2:.3g}"
    n_match = 64 - len(flagged)
    say(f"  {label} top-64: {n_match}/64 ranks identical, {len(flagged)} flagged; "
        f"measured error {delta:.3g}, reorder bound {bound:.3g} (tol {atol:.3g})")
    return n_match, flagged
