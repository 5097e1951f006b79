"""The top-64 parity check (gpu_util.assert_topk_valid) on the CPU: it must
accept what rounding can do and reject what it cannot.  The mistakes are
planted in the candidate lists handed to the check, which stand in for a
GPU's output; the oracle's top-64 is the reference."""
import numpy as np
import pytest

import oracle
from gpu_util import assert_topk_valid


def _logits(seed, V=8192):
    return (np.random.default_rng(seed).standard_normal(V) * 6.0).astype(np.float32)


def test_exact_and_rounded_lists_pass():
    lg = _logits(1)
    ids, vals = oracle.topk64(lg)
    assert assert_topk_valid(ids, vals, lg, 1e-3, "exact")[0] == 64
    # a perturbation of the size fp32 reordering leaves: the list of the
    # perturbed logits, with their values
    noisy = (lg * (1.0 + 1e-6 * np.random.default_rng(2).standard_normal(lg.size))).astype(np.float32)
    ids_n, vals_n = oracle.topk64(noisy)
    assert_topk_valid(ids_n, vals_n, lg, 1e-3, "rounded")


def test_near_tie_within_the_measured_error_passes():
    lg = _logits(3)
    ids, vals = oracle.topk64(lg)
    # ranks 10 and 11 a hair apart; a GPU whose values carry that much error
    # may return them swapped, with values consistent with its order
    lg[ids[11]] = np.nextafter(lg[ids[10]], np.float32(-np.inf))
    ids, vals = oracle.topk64(lg)
    got_ids, got_vals = ids.copy(), vals.copy()
    got_ids[10], got_ids[11] = ids[11], ids[10]
    n_match, flagged = assert_topk_valid(got_ids, got_vals, lg, 1e-3, "near-tie")
    assert n_match == 62 and [f[0] for f in flagged] == [10, 11]


def test_reordering_beyond_the_measured_error_fails():
    """Rank 63 replaced by the 65th value, 1e-3 of the maximum below it: the
    values are exact, so no rounding explains it.  The stated tolerance
    (1e-2) alone would accept it."""
    lg = _logits(4)
    ids, vals = oracle.topk64(lg)
    capped = oracle.softcap(lg)
    order = np.argsort(-capped.astype(np.float64), kind="stable")
    c65 = order[64]
    # place the 65th just 1e-3 * max below the 64th
    target = np.float64(vals[63]) - 1e-3 * np.max(np.abs(vals))
    lg[c65] = np.float32(30.0 * np.arctanh(target / 30.0))
    ids, vals = oracle.topk64(lg)
    capped = oracle.softcap(lg)
    got_ids, got_vals = ids.copy(), vals.copy()
    got_ids[63], got_vals[63] = c65, capped[c65]
    with pytest.raises(AssertionError, match="reordered"):
        assert_topk_valid(got_ids, got_vals, lg, 1e-2, "planted reorder")


def test_changed_argmax_fails_unless_a_tie():
    lg = _logits(5)
    ids, vals = oracle.topk64(lg)
    got_ids, got_vals = ids.copy(), vals.copy()
    got_ids[0], got_ids[1] = ids[1], ids[0]
    got_vals[0], got_vals[1] = vals[1], vals[0]
    with pytest.raises(AssertionError):
        assert_topk_valid(got_ids, got_vals, lg, 1e-2, "planted argmax")


def test_value_error_beyond_tolerance_fails():
    lg = _logits(6)
    ids, vals = oracle.topk64(lg)
    bad = vals.copy()
    bad[5] += 0.01 * np.max(np.abs(vals))
    with pytest.raises(AssertionError, match="value error"):
        assert_topk_valid(ids, bad, lg, 1e-3, "planted value")
