"""Restatement of the reference's KV ring geometry (DynamicRingBuffer,
src/ring_buffer.zig:17-355): which physical slot a clock's K/V lands in and
which slots, in which order, a decode step or a prefill chunk attends over.
TEST INFRASTRUCTURE ONLY (imported by tests/ to check the device's lists).

Only the slot bookkeeping is restated (clocks, active flags, turn
boundaries); the K/V payload is not, since the GPU caches hold it.  Plain
Python: the arithmetic is integer and the cases are small.
"""

TOTAL_SLOTS = 4096          # src/ring_buffer.zig:3
UPPER_RECALL_SLOTS = 128    # src/ring_buffer.zig:4
MAX_BOUNDARIES = 1024       # src/ring_buffer.zig:21


class Ring:
    """DynamicRingBuffer without the K/V payload.  Method names follow the
    reference (snake_case)."""

    def __init__(self, num_layers, num_anchors):
        # init (src/ring_buffer.zig:35-59): window_size / num_recall ignored
        self.num_layers = num_layers
        self.num_anchors = num_anchors
        self.total_slots = TOTAL_SLOTS
        self.clocks = [[0] * TOTAL_SLOTS for _ in range(num_layers)]
        self.active = [[False] * TOTAL_SLOTS for _ in range(num_layers)]
        self.total_ingested = 0
        self.boundaries = [0] * MAX_BOUNDARIES
        self.num_turn_boundaries = 0

    # markBoundary (src/ring_buffer.zig:79-90): a repeated clock replaces the
    # last entry's type; the list is a ring of MAX_BOUNDARIES
    def mark_boundary(self, clock):
        n = self.num_turn_boundaries
        if n > 0 and self.boundaries[(n - 1) % MAX_BOUNDARIES] == clock:
            return
        self.boundaries[n % MAX_BOUNDARIES] = clock
        self.num_turn_boundaries = n + 1

    def boundary_list(self):
        """The boundaries snapToBoundary scans, oldest first."""
        n = self.num_turn_boundaries
        start = n - MAX_BOUNDARIES if n > MAX_BOUNDARIES else 0
        return [self.boundaries[i % MAX_BOUNDARIES] for i in range(start, n)]

    # snapToBoundary (src/ring_buffer.zig:92-100)
    def snap_to_boundary(self, raw_min_clock):
        if raw_min_clock <= self.num_anchors or self.num_turn_boundaries == 0:
            return raw_min_clock
        for b in self.boundary_list():
            if b >= raw_min_clock:
                return b
        return raw_min_clock

    # setNumAnchors (src/ring_buffer.zig:101-103)
    def set_num_anchors(self, n):
        self.num_anchors = min(n, self.total_slots - UPPER_RECALL_SLOTS - 64)

    # recallSlots / recallStart / windowSize (src/ring_buffer.zig:104-115)
    def recall_slots(self, layer=0):
        return 0 if self.total_slots < UPPER_RECALL_SLOTS * 2 else UPPER_RECALL_SLOTS

    def recall_start(self, layer=0):
        return self.total_slots - self.recall_slots(layer)

    def window_size(self, layer=0):
        start = self.recall_start(layer)
        return start - self.num_anchors if start > self.num_anchors else 1

    # getSlotIndexLayer (src/ring_buffer.zig:117-122)
    def slot_index(self, layer, clock):
        if clock < self.num_anchors:
            return clock
        return self.num_anchors + (clock - self.num_anchors) % self.window_size(layer)

    # activateSlot (src/ring_buffer.zig:124-132)
    def activate_slot(self, layer, clock):
        slot = self.slot_index(layer, clock)
        self.clocks[layer][slot] = clock
        self.active[layer][slot] = True
        if layer == 0 and clock >= self.total_ingested:
            self.total_ingested = clock + 1
        return slot

    # deactivateSlot (src/ring_buffer.zig:134-141)
    def deactivate_slot(self, layer, clock):
        slot = self.slot_index(layer, clock)
        if self.clocks[layer][slot] == clock:
            self.active[layer][slot] = False
            self.clocks[layer][slot] = 0

    # rollbackClock (src/ring_buffer.zig:143-151)
    def rollback_clock(self, target_clock):
        if target_clock >= self.total_ingested:
            return
        for c in range(target_clock, self.total_ingested):
            for layer in range(self.num_layers):
                self.deactivate_slot(layer, c)
        self.total_ingested = target_clock

    # writeKV (src/ring_buffer.zig:257-268), bookkeeping only
    def write_kv(self, layer, clock):
        slot = self.slot_index(layer, clock)
        self.clocks[layer][slot] = clock
        self.active[layer][slot] = True
        if layer == 0 and clock >= self.total_ingested:
            self.total_ingested = clock + 1
        return slot

    # clearRecall (src/ring_buffer.zig:270-275)
    def clear_recall(self):
        for layer in range(self.num_layers):
            for s in range(self.recall_start(layer), self.total_slots):
                self.active[layer][s] = False

    # writeRecallKV (src/ring_buffer.zig:277-285), bookkeeping only
    def write_recall_kv(self, layer, rank, clock):
        slot = self.recall_start(layer) + rank
        if slot >= self.total_slots:
            return
        self.clocks[layer][slot] = clock
        self.active[layer][slot] = True

    # getActiveSlotsLayer (src/ring_buffer.zig:291-333)
    def active_slots_layer(self, layer, curr_clock, is_sliding, sliding_window):
        out = []
        act, clk = self.active[layer], self.clocks[layer]
        eff = sliding_window if is_sliding else self.window_size(layer)
        raw_min = curr_clock - eff + 1 if curr_clock >= eff else 0
        min_valid = raw_min if is_sliding else self.snap_to_boundary(raw_min)
        # 1. anchors (slot = clock)
        for s in range(min(curr_clock + 1, self.num_anchors)):
            if act[s] and (not is_sliding or s >= min_valid):
                out.append(s)
        # 2. the window in chronological order
        dyn_start = max(min_valid, self.num_anchors)
        if curr_clock >= dyn_start:
            for c in range(dyn_start, curr_clock + 1):
                slot = self.slot_index(layer, c)
                if act[slot] and clk[slot] == c:
                    out.append(slot)
        # 3. recall slots (full-attention lists only)
        if not is_sliding:
            for s in range(self.recall_start(layer), self.total_slots):
                if act[s] and clk[s] <= curr_clock:
                    out.append(s)
        return out

    # getActiveSlots (src/ring_buffer.zig:287-289)
    def active_slots(self, layer, curr_clock):
        return self.active_slots_layer(layer, curr_clock, False, 1024)

    # getPrefillPrevSlots (src/ring_buffer.zig:335-378)
    def prefill_prev_slots(self, layer, start_clock, chunk_len):
        out = []
        if start_clock == 0 or chunk_len == 0:
            return out
        act, clk = self.active[layer], self.clocks[layer]
        end_clock = start_clock + chunk_len - 1
        w = self.window_size(layer)
        raw_min = end_clock - w + 1 if end_clock >= w else 0
        min_valid = self.snap_to_boundary(raw_min)
        for s in range(min(start_clock, self.num_anchors)):
            if act[s]:
                out.append(s)
        dyn_start = max(min_valid, self.num_anchors)
        if start_clock > dyn_start:
            for c in range(dyn_start, start_clock):
                slot = self.slot_index(layer, c)
                if act[slot] and clk[slot] == c:
                    out.append(slot)
        for s in range(self.recall_start(layer), self.total_slots):
            if act[s] and clk[s] < start_clock:
                out.append(s)
        return out


def decode_lists(ring, clock, sliding_window):
    """What forwardToken's GPU branch hands gpuDispatchForwardToken for one
    token (src/model/forward.zig:41-47): activate the clock on layer 0, then
    its slot and the global and sliding lists of layer 0."""
    ring.activate_slot(0, clock)
    slot = ring.slot_index(0, clock)
    active = ring.active_slots_layer(0, clock, False, sliding_window)
    sliding = ring.active_slots_layer(0, clock, True, sliding_window)
    return slot, active, sliding
