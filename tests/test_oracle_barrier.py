"""Pins the oracle of the epoch / arrival barrier (k3_collectives.cu:21-35,
k3_rs_arrive_v2.cu:41-76) by playing the ranks with host threads: every rank
passes a slot only after every peer has arrived on it in the same call (checked
through a per-rank payload written before each arrival), across calls with
different grids; a rank that never arrives is given up on at the deadline and
reported; a late rank's stale counter holds the others back; a slot skipped in
one call can never be passed again (why every call must arrive on every slot)."""
import threading
import time

import numpy as np

import oracle as O

SLOTS = 372  # the manifest's coll_flags
SLOT_LIST = [1, 2, 95]
SPIN = 2_000_000_000  # ns, the reference's bail-out


class Ranks:
    def __init__(self, n):
        self.n = n
        self.flags = [np.zeros(SLOTS, np.uint64) for _ in range(n)]
        self.peer = np.array([f.ctypes.data for f in self.flags], np.uint64)
        for f in self.flags:
            O.flags_init(f)


def _threads(n, fn):
    errors = []

    def body(r):
        try:
            fn(r)
        except BaseException as e:  # surfaced in the main thread below
            errors.append((r, e))

    ts = [threading.Thread(target=body, args=(r,)) for r in range(n)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(30)
    assert not any(t.is_alive() for t in ts), "a rank thread did not finish"
    if errors:
        raise errors[0][1]


def test_every_rank_passes_only_after_every_peer():
    R = Ranks(4)
    calls = [896, 1, 7, 896]  # units per call: the collective grid at 16384, 4 and other token counts
    payload = np.full((4, SLOTS), -1, np.int64)
    masks = []

    def rank(r):
        g = np.random.default_rng(r)
        for c, units in enumerate(calls):
            O.epoch_bump(R.flags[r], units)
            for s in SLOT_LIST:
                time.sleep(float(g.uniform(0, 0.002)))
                payload[r, s] = c  # this rank's slice of the collective on slot s
                m = O.rs_arrive(R.flags[r], R.peer, units, s, 4, SPIN)
                masks.append(m)
                assert (payload[:, s] >= c).all(), (r, c, s, payload[:, s])

    _threads(4, rank)
    assert masks == [0] * (4 * len(calls) * len(SLOT_LIST))
    for f in R.flags:
        assert int(f[0]) == sum(calls)
        for s in SLOT_LIST:
            assert int(f[s]) == sum(calls)


def test_missing_rank_is_given_up_and_reported():
    R = Ranks(4)
    spin = 20_000_000
    out = {}

    def rank(r):
        O.epoch_bump(R.flags[r], 896)
        if r == 3:  # dead peer: bumps its epoch, never arrives
            return
        t0 = time.perf_counter()
        out[r] = (O.rs_arrive(R.flags[r], R.peer, 896, 1, 4, spin), time.perf_counter() - t0)

    _threads(4, rank)
    for r in range(3):
        m, dt = out[r]
        assert m == 1 << 3
        assert 0.019 <= dt < 5.0
    # the arrivals of the live ranks still count: rank 3 arriving late finds them there
    assert O.rs_arrive(R.flags[3], R.peer, 896, 1, 4, spin) == 0


def test_late_rank_holds_the_others_back():
    """After one full call every counter sits at the call's total; in the next
    call rank 3's counter is stale (below the new epoch) until it arrives, and no
    rank passes before then."""
    R = Ranks(4)

    def first(r):
        O.epoch_bump(R.flags[r], 896)
        assert O.rs_arrive(R.flags[r], R.peer, 896, 1, 4, SPIN) == 0

    _threads(4, first)
    t_arrive = {}
    t_pass = {}

    def second(r):
        O.epoch_bump(R.flags[r], 3)
        if r == 3:
            time.sleep(0.1)
        t_arrive[r] = time.perf_counter()
        assert O.rs_arrive(R.flags[r], R.peer, 3, 1, 4, SPIN) == 0
        t_pass[r] = time.perf_counter()

    _threads(4, second)
    for r in range(3):
        assert t_pass[r] >= t_arrive[3]
    assert all(int(f[1]) == 899 for f in R.flags)


def test_skipped_slot_never_passes_again():
    """Every call raises the epoch for every slot: a call that skips slot 2
    leaves it one call behind for good, so later waits on it give up."""
    R = Ranks(2)
    for f in R.flags:
        O.epoch_bump(f, 5)

    def call1(r):  # slot 1 only
        assert O.rs_arrive(R.flags[r], R.peer, 5, 1, 2, SPIN) == 0

    _threads(2, call1)
    for f in R.flags:
        O.epoch_bump(f, 5)
    res = {}

    def call2(r):
        res[r] = O.rs_arrive(R.flags[r], R.peer, 5, 2, 2, 20_000_000)

    _threads(2, call2)
    assert res == {0: 0b11, 1: 0b11}  # 5 arrivals against an epoch of 10


def test_single_rank_passes_on_its_own_arrival():
    R = Ranks(1)
    O.epoch_bump(R.flags[0], 896)
    assert O.rs_arrive(R.flags[0], R.peer, 896, 7, 1, 1000) == 0
    assert int(R.flags[0][7]) == 896


def test_comparison_is_on_the_low_word():
    """The wait compares the low 32 bits of the counters (k3_rs_arrive1.cu:56-58):
    a counter past 2^32 compares by its low word."""
    R = Ranks(2)
    R.flags[0][0] = (1 << 32) + 5          # epoch: low word 5
    R.flags[1][4] = 7                       # peer: low word 7 >= 5, the u64 far below the epoch
    assert O.rs_arrive(R.flags[0], R.peer, 5, 4, 2, 1_000_000) == 0  # own counter 5
    R.flags[1][5] = (1 << 32) + 3           # peer: low word 3 < 5, the u64 above 5
    assert O.rs_arrive(R.flags[0], R.peer, 5, 5, 2, 1_000_000) == 0b10
