"""Slot lists of the reference's 4096-slot KV ring for a contiguous history,
in closed form.

The reference's host computes, per decode token, the physical slot of the
new K/V and the chronological slot lists that the global and the sliding
attention layers read (getSlotIndexLayer / getActiveSlotsLayer,
src/ring_buffer.zig:117-122,291-333, called from src/model/forward.zig:41-47).
The ring has three tiers: anchors [0, A) hold clocks 0..A-1 for good, the
FIFO window [A, 3968) holds clock c at A + (c - A) mod (3968 - A), and the
recall tier [3968, 4096) holds retrieved entries.  For a history in which
every clock up to the current one was written and nothing was evicted, the
lists have the closed form below; ``chn_decode_greedy`` generates the same
lists on the device.
"""
import numpy as np

TOTAL_SLOTS = 4096
RECALL_SLOTS = 128
RECALL_START = TOTAL_SLOTS - RECALL_SLOTS      # 3968
MAX_ANCHORS = RECALL_START - 64                # setNumAnchors' cap (src/ring_buffer.zig:101-103)
MAX_BOUNDARIES = 1024
RECALL_NONE = 0xFFFFFFFF                       # an inactive recall slot


def window_size(num_anchors):
    return RECALL_START - num_anchors if RECALL_START > num_anchors else 1


def slot_index(clock, num_anchors=0):
    """Physical slot of `clock` (getSlotIndexLayer)."""
    if clock < num_anchors:
        return clock
    return num_anchors + (clock - num_anchors) % window_size(num_anchors)


def _snap(raw_min, num_anchors, boundaries):
    if raw_min <= num_anchors or len(boundaries) == 0:
        return raw_min
    for b in boundaries:
        if b >= raw_min:
            return int(b)
    return raw_min


def decode_lists(clock, sliding_window, num_anchors=0, boundaries=(), recall_clocks=None):
    """(slot_idx, global list, sliding list) for decode step `clock`.

    boundaries: turn-boundary clocks, oldest first (at most 1024), which
    move the start of the global window forward (snapToBoundary);
    recall_clocks: per recall rank r (slot 3968 + r) the clock stored there,
    or RECALL_NONE; a rank joins the global list once its clock <= `clock`.
    """
    A = int(num_anchors)
    if A > MAX_ANCHORS:
        raise ValueError(f"num_anchors {A} exceeds {MAX_ANCHORS}")
    W = window_size(A)
    c = int(clock)
    anchors = np.arange(min(c + 1, A), dtype=np.int64)

    def window(first):
        cl = np.arange(first, c + 1, dtype=np.int64)
        return np.where(cl < A, cl, A + (cl - A) % W)

    raw = c - W + 1 if c >= W else 0
    g = [anchors, window(max(_snap(raw, A, list(boundaries)), A))]
    if recall_clocks is not None:
        rc = np.asarray(recall_clocks, np.int64)
        g.append(RECALL_START + np.nonzero((rc != RECALL_NONE) & (rc <= c))[0])
    sw = int(sliding_window)
    raw_s = c - sw + 1 if c >= sw else 0
    # window clocks older than the newest W have been overwritten in place
    s = [anchors[anchors >= raw_s], window(max(raw_s, A, raw))]
    return (slot_index(c, A), np.concatenate(g).astype(np.uint32), np.concatenate(s).astype(np.uint32))
