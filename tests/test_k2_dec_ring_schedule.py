"""Host-side replay of the decode GEMM's LDS buffer schedule (``k2_dec`` in
nano-vllm-int4_amd/csrc/w4a4_gemm.hip).

The kernel's main loop is replayed as a sequence of phases separated by
workgroup barriers, with the LDS buffers each phase writes or reads: the
activation slice ``a_l[2]``, the group dots ``dots[2]`` and the round's scales
``sal[2]`` / ``swl[2]``, each double-buffered on the round's parity.  A round
is 8 K groups (8 waves, ring depth 4) or 16 (16 waves, ring depth 2); the
schedule is the same, only the round count changes.  Threads
of a workgroup run the phases of one barrier interval in any interleaving, so
the schedule is race-free iff no buffer copy is written in an interval in
which it is also read (every read in this kernel is of data other threads
wrote), and every read finds the copy last written with its own round; within a
thread, every use of a register-ring slot must find the slot holding its
round.  The
replay follows the loop structure of the source (D-round register ring,
steady state over whole ring turns, tail of at most D rounds) for the K of
every projection, and the planted mistakes show the check rejects a
single-buffered copy, a missing barrier and a refill into a live slot.
"""
import pytest

class Replay:
    def __init__(self):
        self.interval = 0
        self.events = []          # (interval, buffer, copy, kind, round)
        self.copies = 2

    def access(self, buf, r, kind):
        self.events.append((self.interval, buf, r % self.copies, kind, r))

    # phases of k2_dec
    def mma(self, r):             # reads slice r, writes round r's dots and scales
        self.access("a_l", r, "R")
        for b in ("dots", "sal", "swl"):
            self.access(b, r, "W")

    def stage_a(self, r):         # writes slice r
        self.access("a_l", r, "W")

    def epilogue(self, r):        # reads round r's dots and scales
        for b in ("dots", "sal", "swl"):
            self.access(b, r, "R")

    def barrier(self):
        self.interval += 1


class Ring:
    """The per-thread register ring: slot u holds the weight fragment, the
    activation chunks and the scales of one round (rw[u], ra[u], rs[u])."""
    def __init__(self, D):
        self.D = D
        self.slot = {}              # (array, slot) -> round

    def issue(self, r, u):
        for arr in ("rw", "ra", "rs"):
            self.slot[(arr, u)] = r

    def use(self, arr, u, r):
        assert self.slot.get((arr, u)) == r, f"{arr}[{u}] holds round {self.slot.get((arr, u))}, not {r}"


def shipped(R, D, rp=None, ring=None):
    """The loop of k2_dec as built, with the register slots each phase uses."""
    rp = rp or Replay()
    ring = ring or Ring(D)
    for u in range(D):
        ring.issue(u, u)
    ring.use("ra", 0, 0)
    rp.stage_a(0)
    rp.barrier()
    r0 = 0
    while r0 + D < R:
        for u in range(D):
            un = (u + 1) % D
            ring.use("rw", u, r0 + u), ring.use("rs", u, r0 + u)
            rp.mma(r0 + u)
            ring.use("ra", un, r0 + u + 1)
            rp.stage_a(r0 + u + 1)
            ring.issue(r0 + u + D, u)
            rp.barrier()
            rp.epilogue(r0 + u)
        r0 += D
    for u in range(D):
        un = (u + 1) % D
        if r0 + u < R:
            ring.use("rw", u, r0 + u), ring.use("rs", u, r0 + u)
            rp.mma(r0 + u)
            if r0 + u + 1 < R:
                ring.use("ra", un, r0 + u + 1)
                rp.stage_a(r0 + u + 1)
            rp.barrier()
            rp.epilogue(r0 + u)
    return rp


def overlapped(R, D, rp=None):
    """Round r + 1's MFMAs issued before round r's epilogue in one barrier
    interval (the measured-slower variant's schedule as described)."""
    rp = rp or Replay()
    rp.stage_a(0)
    rp.barrier()
    rp.mma(0)
    if R > 1:
        rp.stage_a(1)
    rp.barrier()
    for r in range(R):
        if r + 1 < R:
            rp.mma(r + 1)
            if r + 2 < R:
                rp.stage_a(r + 2)
        rp.epilogue(r)
        rp.barrier()
    return rp


def hazards(rp):
    """Write/read pairs on one buffer copy inside one barrier interval, and
    reads that do not find their own round in the copy."""
    found = []
    by_slot = {}
    for iv, buf, copy, kind, r in rp.events:
        by_slot.setdefault((iv, buf, copy), []).append((kind, r))
    for (iv, buf, copy), acc in by_slot.items():
        kinds = {k for k, _ in acc}
        if "W" in kinds and "R" in kinds:
            found.append(("same-interval write and read", iv, buf, copy))
    state = {}
    for iv in range(rp.interval + 1):
        evs = [e for e in rp.events if e[0] == iv]
        for _, buf, copy, kind, r in evs:
            if kind == "R":
                w = state.get((buf, copy))
                if w != r:
                    found.append(("stale read", iv, buf, copy, r, w))
        for _, buf, copy, kind, r in evs:
            if kind == "W":
                state[(buf, copy)] = r
    return found


def overlapped_with_ring(R, D, rp=None, ring=None):
    """The overlapped order with its register ring: a prologue that forms
    round 0's products and stages round 1, then per interval the products of
    round r + 1, the epilogue of round r, the staging of round r + 2 and the
    refill of round r + 1's slot with round r + 1 + D."""
    rp = rp or Replay()
    ring = ring or Ring(D)
    for u in range(D):
        ring.issue(u, u)
    ring.use("ra", 0, 0)
    rp.stage_a(0)
    rp.barrier()
    ring.use("rw", 0, 0), ring.use("rs", 0, 0)
    rp.mma(0)
    if R > 1:
        ring.use("ra", 1 % D, 1)
        rp.stage_a(1)
    ring.issue(D, 0)
    rp.barrier()

    def interval(r, steady):
        if steady or r + 1 < R:
            ring.use("rw", (r + 1) % D, r + 1), ring.use("rs", (r + 1) % D, r + 1)
            rp.mma(r + 1)
        rp.epilogue(r)
        if steady or r + 2 < R:
            ring.use("ra", (r + 2) % D, r + 2)
            rp.stage_a(r + 2)
        if steady:
            ring.issue(r + 1 + D, (r + 1) % D)
    r0 = 0
    while r0 + D + 1 < R:
        for u in range(D):
            interval(r0 + u, True)
            rp.barrier()
        r0 += D
    for u in range(D + 1):
        if r0 + u < R:
            interval(r0 + u, False)
            if r0 + u + 1 < R:
                rp.barrier()
    return rp


# K of the four Qwen3-8B projections, the test shapes and K with a partial
# last round; G = K/128 groups, GR groups per round (8 or 16 waves), R =
# ceil(G/GR) rounds; the launcher's ring depths (4 with 8 waves, 2 with 16)
# and others.
KS = (256, 512, 1024, 2048, 2176, 3200, 4096, 6272, 8192, 12160, 12288)
CASES = [(K, GR, D) for K in KS for GR in (8, 16) for D in (2, 3, 4, 6) if GR == 8 or K >= 2048]


@pytest.mark.parametrize("K,GR,D", CASES)
def test_shipped_schedule_is_race_free(K, GR, D):
    R = (K // 128 + GR - 1) // GR
    rp = shipped(R, D)
    assert hazards(rp) == []
    epilogues = [e[4] for e in rp.events if e[1] == "dots" and e[3] == "R"]
    assert epilogues == list(range(R))           # every round's epilogue once, in order
    assert rp.interval == R + 1                  # the prologue's barrier, then one per round


@pytest.mark.parametrize("K,GR,D", CASES)
def test_overlapped_schedule_is_race_free(K, GR, D):
    R = (K // 128 + GR - 1) // GR
    assert hazards(overlapped(R, D)) == []
    rp = overlapped_with_ring(R, D)
    assert hazards(rp) == []
    assert [e[4] for e in rp.events if e[1] == "dots" and e[3] == "R"] == list(range(R))


def test_single_buffered_dots_is_rejected():
    rp = Replay()
    orig = rp.access

    def access(buf, r, kind):
        if buf == "dots":
            rp.events.append((rp.interval, buf, 0, kind, r))
        else:
            orig(buf, r, kind)
    rp.access = access
    assert any(h[2] == "dots" for h in hazards(overlapped(12, 4, rp)))


def test_ring_refill_into_a_live_slot_is_rejected():
    class Early(Ring):       # refill the slot of round r + 1 instead of round r's
        def issue(self, r, u):
            super().issue(r, u if r < self.D else (u + 1) % self.D)
    with pytest.raises(AssertionError):
        shipped(12, 4, ring=Early(4))
    with pytest.raises(AssertionError):
        overlapped_with_ring(12, 4, ring=Early(4))


def test_missing_barrier_is_rejected():
    rp = Replay()
    rp.stage_a(0)
    rp.mma(0)              # reads slice 0 in the interval that writes it
    assert hazards(rp)
