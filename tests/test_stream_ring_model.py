"""CPU model of the search kernel's candidate-run ring (search_kernel.hip:
append_runs / consume / gather), checked for bounds under both tile orders.

The kernel appends up to 64 runs of sorted points per traversal batch (one per
lane, in lane order) to a 128-entry LDS ring and consumes the resulting virtual
stream in tiles of 32 positions.  Each lane maps its stream position to a
point position through the ring entry whose end exceeds it (r_vend) and the
previous entry's end (the run's first stream position).  Tiles are gathered
either one ahead of the current tile's hit handling (rows of up to 32 floats)
or after the retirement of the fully consumed runs (wider rows).

This model replays the same index arithmetic on random run streams (many empty
and single-point runs, which fill the ring fastest) and asserts, for both
orders: every lookup stays within the live entries [ring_tail, ring_head), the
entry before it has not been overwritten, every gathered position equals the
stream's true point position and lies in [0, N), and an append never writes a
slot that is still live.
"""
import numpy as np
import pytest

K_RING = 128
TILE = 32
LANES = 64


class RingModel:
    def __init__(self, n_points):
        self.N = n_points
        self.r_start = [0] * K_RING
        self.r_vend = [0] * K_RING      # entry K_RING - 1 starts at 0 (the first run's begin)
        self.ring_head = 0
        self.ring_tail = 0
        self.v_total = 0
        self.v_done = 0
        self.jr = [0] * TILE            # per-lane current run (lanes n and n + 32 agree)
        self.truth = []                 # the stream's point positions, in order
        self.gathered = []

    def append_runs(self, runs):
        assert len(runs) <= LANES
        incl = 0
        k = 0
        live_lo = self.ring_tail - 1    # the entry before the tail is still read
        for start, length in runs:
            if length <= 0:
                continue
            incl += length
            slot_abs = self.ring_head + k
            # the slot must not hold a live entry (or the one before the tail)
            assert slot_abs - live_lo < K_RING, "append overwrites a live ring entry"
            slot = slot_abs & (K_RING - 1)
            self.r_start[slot] = start
            self.r_vend[slot] = self.v_total + incl
            self.truth.extend(range(start, start + length))
            k += 1
        self.ring_head += k
        self.v_total += incl

    def gather(self, v0, count):
        pos = []
        for n in range(count):
            v = v0 + n
            jr = max(self.jr[n], self.ring_tail)
            while True:
                assert self.ring_tail <= jr < self.ring_head, "lookup outside the live entries"
                if self.r_vend[jr & (K_RING - 1)] > v:
                    break
                jr += 1
            self.jr[n] = jr
            j = jr & (K_RING - 1)
            p = self.r_start[j] + (v - self.r_vend[(jr - 1) & (K_RING - 1)])
            assert 0 <= p < self.N, "gathered position out of range"
            assert p == self.truth[v], "gathered position differs from the stream"
            pos.append(p)
        return pos

    def consume(self, final_pass, prefetch):
        avail = self.v_total - self.v_done
        if not (avail >= TILE or (final_pass and avail > 0)):
            return
        cur = (self.v_done, min(TILE, avail), self.gather(self.v_done, min(TILE, avail)))
        while True:
            vn = self.v_done + cur[1]
            an = self.v_total - vn
            has_next = an >= TILE or (final_pass and an > 0)
            nxt = None
            if prefetch and has_next:
                nxt = (vn, min(TILE, an), self.gather(vn, min(TILE, an)))
            self.gathered.extend(cur[2])
            self.v_done = vn
            while self.ring_tail < self.ring_head and self.r_vend[self.ring_tail & (K_RING - 1)] <= self.v_done:
                self.ring_tail += 1
            if not has_next:
                break
            cur = nxt if prefetch else (vn, min(TILE, an), self.gather(vn, min(TILE, an)))


def random_batch(rs, n_points, style):
    runs = []
    for _ in range(LANES):
        if style == "singles":
            length = int(rs.choice([0, 1], p=[0.2, 0.8]))
        elif style == "mixed":
            length = int(rs.choice([0, 1, 2, 3, rs.randint(4, 200)], p=[0.3, 0.3, 0.1, 0.1, 0.2]))
        else:                           # long runs (dense cells)
            length = int(rs.randint(0, 2000))
        length = min(length, n_points)
        start = int(rs.randint(0, n_points - length + 1))
        runs.append((start, length))
    return runs


@pytest.mark.parametrize("prefetch", [True, False])
@pytest.mark.parametrize("style", ["singles", "mixed", "long"])
def test_ring_indexing_stays_in_bounds(prefetch, style):
    rs = np.random.RandomState(7 + prefetch + 3 * len(style))
    for trial in range(6):
        n_points = int(rs.choice([1, 37, 5000, 10 ** 6]))
        m = RingModel(n_points)
        batches = int(rs.randint(1, 60))
        for b in range(batches):
            m.append_runs(random_batch(rs, n_points, style))
            m.consume(final_pass=(b == batches - 1), prefetch=prefetch)
        # the final pass drains the stream: every position was gathered once, in order
        assert m.v_done == m.v_total
        assert m.gathered == m.truth


def test_ring_holds_the_worst_case_backlog():
    # after a non-final consume at most 31 positions remain, i.e. at most 32
    # live runs (31 single-point runs plus a partly consumed one); 64 more
    # runs leave the slot before the tail untouched
    for prefetch in (True, False):
        m = RingModel(10 ** 6)
        m.append_runs([(i, 1) for i in range(LANES)])        # 64 single-point runs
        m.append_runs([])
        m.consume(final_pass=False, prefetch=prefetch)       # two tiles consumed, 0 left
        m.append_runs([(1000, 40)] + [(2000 + i, 1) for i in range(63)])
        m.consume(final_pass=False, prefetch=prefetch)       # 103 positions: 96 consumed
        assert m.v_total - m.v_done < TILE
        assert m.ring_head - m.ring_tail <= TILE
        m.append_runs([(5000 + i, 1) for i in range(LANES)])
        m.consume(final_pass=True, prefetch=prefetch)
        assert m.gathered == m.truth
