"""The ring geometry: oracle/ring.py (restatement of DynamicRingBuffer,
src/ring_buffer.zig) pinned by the reference's own ring tests and by what
the geometry fixes in closed form, and channel_amd/ring.py (the closed-form
lists chn_decode_greedy generates on the device) checked against it."""
import numpy as np
import pytest

from channel_amd import ring as R
from oracle.ring import Ring, decode_lists


# ---- the reference's own tests, transcribed (src/ring_buffer.zig:393-597)

def test_ref_tiers_and_window():
    """'ring buffer tiers and window eviction' (src/ring_buffer.zig:393-410)."""
    ring = Ring(2, 4)
    assert ring.total_slots == 4096
    for c in range(20):
        ring.write_kv(0, c)
    s = ring.active_slots(0, 19)
    assert len(s) == 20 and s[0] == 0 and s[3] == 3


def test_ref_recall_slots():
    """'recall slots are written, cleared, and included in active set'
    (src/ring_buffer.zig:412-431)."""
    ring = Ring(32, 2)
    ring.write_recall_kv(16, 0, 100)
    ring.write_recall_kv(16, 1, 50)
    assert len(ring.active_slots(16, 101)) == 2
    ring.clear_recall()
    assert len(ring.active_slots(16, 101)) == 0


def test_ref_prefill_prev_slots_bounds():
    """'prefill slot calculation strictly respects physical ring buffer
    bounds' (src/ring_buffer.zig:433-468)."""
    ring = Ring(2, 512)
    for c in range(5000):
        ring.activate_slot(0, c)
        ring.write_kv(0, c)
    chunk_len = 226
    prev = ring.prefill_prev_slots(0, 5000, chunk_len)
    assert len(prev) + chunk_len <= ring.total_slots
    assert len(prev) >= 512
    clocks = [ring.clocks[0][s] for s in prev]
    assert all(b > a for a, b in zip(clocks, clocks[1:]))


def test_ref_rollback():
    """'ring buffer rollbackClock cleanly deactivates transient probe slots'
    (src/ring_buffer.zig:575-597)."""
    ring = Ring(2, 4)
    for c in range(10):
        for layer in range(2):
            ring.activate_slot(layer, c)
    assert ring.total_ingested == 10
    for c in range(10, 13):
        for layer in range(2):
            ring.activate_slot(layer, c)
    assert ring.total_ingested == 13
    s11 = ring.slot_index(0, 11)
    assert ring.active[0][s11]
    ring.rollback_clock(10)
    assert ring.total_ingested == 10 and not ring.active[0][s11]


# ---- what the geometry fixes

@pytest.mark.parametrize("A", [0, 4, 512, 3904])
def test_slot_index_closed_form(A):
    ring = Ring(1, A)
    W = 4096 - 128 - A
    assert ring.window_size() == W and ring.recall_start() == 3968
    for c in list(range(0, 40)) + list(range(3900, 4100)) + [A + k * W + d for k in range(3) for d in (-1, 0, 1)]:
        if c < 0:
            continue
        s = ring.slot_index(0, c)
        assert s == (c if c < A else A + (c - A) % W)
        assert s < 3968                          # never in the recall tier
    # W consecutive window clocks fill [A, 3968) exactly once
    first = A + 7
    assert sorted(ring.slot_index(0, c) for c in range(first, first + W)) == list(range(A, 3968))
    # no anchors: the window wraps at clock 3968 (not 4096)
    if A == 0:
        assert ring.slot_index(0, 3967) == 3967 and ring.slot_index(0, 3968) == 0


@pytest.mark.parametrize("A,sw", [(0, 512), (4, 16), (512, 512), (512, 1024), (3904, 512)])
def test_contiguous_history_lists(A, sw):
    """Every clock written once, in order: the global list is the anchors
    plus the newest W clocks (at most 3968 entries), the sliding list the
    newest sw clocks, chronological, without repeats."""
    ring = Ring(1, A)
    W = 3968 - A
    checks = sorted({0, 1, A, A + 1, 600, 3967, 3968, 3969, 4095, 4096, 4100, 3968 + W - 1, 3968 + W, 9000})
    c_done = -1
    for c in checks:
        for cc in range(c_done + 1, c + 1):
            ring.write_kv(0, cc)
        c_done = c
        g = ring.active_slots_layer(0, c, False, sw)
        s = ring.active_slots_layer(0, c, True, sw)
        want_clocks = list(range(min(c + 1, A))) + list(range(max(A, c - W + 1), c + 1))
        assert [ring.clocks[0][x] if x >= A else x for x in g] == want_clocks
        assert len(g) == min(c + 1, 3968) and len(set(g)) == len(g)
        # the sliding list: the newest sw clocks, less window clocks whose
        # slot a newer clock has taken (only when sw > W)
        raw_s = max(0, c - sw + 1)
        want_s = [x for x in range(min(c + 1, A)) if x >= raw_s] + list(range(max(raw_s, A, c - W + 1), c + 1))
        assert [ring.clocks[0][x] if x >= A else x for x in s] == want_s
        assert len(s) == (min(c + 1, sw) if sw <= W else len(want_s))


def test_boundary_snap_and_recall():
    """snapToBoundary moves the global window's start to the first
    boundary at or after its raw start (only once the raw start passes the
    anchors); recall ranks join the global list once their clock has
    passed; the sliding list ignores both."""
    A, sw = 512, 512
    ring = Ring(1, A)
    for b in (100, 600, 4000):
        ring.mark_boundary(b)
    ring.mark_boundary(4000)                      # a repeat is not added
    assert ring.boundary_list() == [100, 600, 4000]
    for c in range(3968):
        ring.write_kv(0, c)
    ring.write_recall_kv(0, 0, 50)
    ring.write_recall_kv(0, 5, 3969)
    g = ring.active_slots_layer(0, 3967, False, sw)
    # raw start 3967 - 3456 + 1 = 512 <= A: no snap, window from clock 512
    assert g[:A] == list(range(A)) and len(g) == A + 3456 + 1
    assert g[-1] == 3968                          # recall rank 0 (clock 50)
    ring.write_kv(0, 3968)
    ring.write_kv(0, 3969)
    g = ring.active_slots_layer(0, 3969, False, sw)
    # raw start 514 > A: snapped to the boundary at 600
    assert [ring.clocks[0][x] for x in g[A:A + 2]] == [600, 601]
    assert g[-2:] == [3968, 3973]                 # rank 5 joins at clock 3969
    s = ring.active_slots_layer(0, 3969, True, sw)
    assert len(s) == sw and all(x < 3968 for x in s)


# ---- the closed form the device implements, against the restatement

@pytest.mark.parametrize("A,bounds,recall", [
    (0, [], None),
    (4, [], None),
    (512, [100, 600, 4000], {0: 50, 5: 3969, 127: 10}),
    (0, [3000, 3970, 3975], {1: 0}),
    (3904, [], None),
])
def test_closed_form_matches_restatement(A, bounds, recall):
    sw = 512
    ring = Ring(1, A)
    for b in bounds:
        ring.mark_boundary(b)
    rc = np.full(128, R.RECALL_NONE, np.uint32)
    for rank, clk in (recall or {}).items():
        ring.write_recall_kv(0, rank, clk)
        rc[rank] = clk
    checks = {0, 1, 5, A, 511, 512, 513, 3966, 3967, 3968, 3969, 3971, 3975, 4095, 4096, 7423, 7424, 7999}
    for c in range(0, 8000):
        if c not in checks:
            ring.activate_slot(0, c)
            continue
        slot, g, s = decode_lists(ring, c, sw)
        slot2, g2, s2 = R.decode_lists(c, sw, A, bounds, rc if recall else None)
        assert slot2 == slot
        assert list(g2) == g, c
        assert list(s2) == s, c


def test_closed_form_rejects_too_many_anchors():
    with pytest.raises(ValueError):
        R.decode_lists(10, 512, num_anchors=3905)
