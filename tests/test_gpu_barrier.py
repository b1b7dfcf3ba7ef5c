"""GPU: the epoch / arrival barrier of the push family (module k3_barrier.hip,
keys k3_collectives and k3_rs_arrive_v2) on one GPU.  The ranks' counter arrays
are local buffers whose addresses go into flags_peer; the peers' arrivals are
played by the host, either before the launch (their counters raised on the
stream) or while the wait runs (a counter array in coherent pinned host memory
written by the host).  Every wait is bounded: the missing-rank cases use a build
that gives up after 20 ms, the others finish as soon as the counters reach the
epoch, and a wait that gave up shows as a non-zero mask, never as a hang."""
import ctypes
import json
import os
import time

import numpy as np
import pytest
import torch

import k3h
import oracle as O
from k3data import H, from_dev, normal_bf16, rng, to_dev

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SLOTS = 372
SHORT = "k3_rs_arrive_v2+K3_SPIN_US=20000"
MASK_SPEC = {"params": ["out buffer<u64>", "in buffer<u64>", "i32", "i32", "i32", "out buffer<u32>"]}
ARRIVE_SPEC = {"params": ["in buffer<bf16>", "out buffer<bf16>", "in buffer<u64>", "out buffer<u64>",
                          "in buffer<u64>", "i64", "i32", "i32", "i32", "i32", "i32"]}


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _op(ctx, module, entry, spec):
    s = dict(spec, impl={"launches": [{"module": module, "entry": entry, "block": [64, 1, 1],
                                        "grid": [1, 1, 1]}]})
    return k3h.ManifestOp(ctx, f"{module}:{entry}", s)


class GpuRanks:
    def __init__(self, ctx, n):
        self.flags = [torch.full((SLOTS,), -1, dtype=torch.int64, device="cuda") for _ in range(n)]
        for f in self.flags:
            ctx.flags_init(f, SLOTS)
        self.peer = torch.tensor([f.data_ptr() for f in self.flags], dtype=torch.int64, device="cuda")

    def arrive_peers(self, me, units, slot):
        for q, f in enumerate(self.flags):
            if q != me:
                f[slot] += units


def _timed(fn):
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e)  # ms


def test_flags_init_and_epoch_bump(ctx):
    _case("flags_init / epoch_bump")
    f = torch.full((SLOTS + 4,), 77, dtype=torch.int64, device="cuda")
    ctx.flags_init(f, SLOTS)
    got = f.cpu().numpy()
    assert (got[:SLOTS] == 0).all() and (got[SLOTS:] == 77).all()
    for units in (896, 1, 7):
        ctx.epoch_bump(f, units)
    assert int(f[0]) == 904 and (f[1:SLOTS].cpu().numpy() == 0).all()


def test_arrive_after_every_peer(ctx):
    """Calls with different grids, three slots each: rank 2 passes every slot with
    no rank missing, and its counters follow the epoch."""
    R, me = GpuRanks(ctx, 4), 2
    missing = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    own = torch.tensor([R.flags[me].data_ptr()], dtype=torch.int64, device="cuda")
    total = 0
    for units in (896, 1, 7, 896):
        _case(f"arrive units {units}")
        total += units
        for f in R.flags:
            ctx.epoch_bump(f, units)
        for s in (1, 2, 95):
            R.arrive_peers(me, units, s)
            ms = _timed(lambda: ctx.rs_arrive(R.flags[me], R.peer, units, s, 4, missing))
            assert int(missing[0]) == 0
            assert ms < 200.0, ms  # the wait ends when the counters reach the epoch (give-up: 2 s)
        # the manifest entry (no mask), a slot only this rank uses, nranks 1
        ms = _timed(lambda: ctx.rs_arrive(R.flags[me], own, units, 200, 1))
        assert ms < 200.0, ms
        assert int(R.flags[me][200]) == total
        assert int(R.flags[me][0]) == total
        for s in (1, 2, 95):
            assert int(R.flags[me][s]) == total


@pytest.mark.parametrize("late", [0, 3])
def test_arrive_gives_up_on_a_missing_rank(ctx, late):
    """Call 1: every rank arrives on slot 5.  Call 2: rank `late` does not, so its
    counter stays at call 1's total (stale, below the new epoch): the 20 ms build
    gives up on it alone and reports it; this rank's own arrival is still counted."""
    R, me = GpuRanks(ctx, 4), 1
    missing = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    arrive = _op(ctx, SHORT, "k3h_rs_arrive_mask", MASK_SPEC)
    _case(f"give-up late={late}: call 1 passes")
    for f in R.flags:
        ctx.epoch_bump(f, 896)
    R.arrive_peers(me, 896, 5)
    arrive([R.flags[me], R.peer, 896, 5, 4, missing], {})
    torch.cuda.synchronize()
    assert int(missing[0]) == 0 and int(R.flags[me][5]) == 896
    _case(f"give-up late={late}: call 2 gives up on rank {late}")
    for f in R.flags:
        ctx.epoch_bump(f, 3)
    for q, f in enumerate(R.flags):
        if q not in (me, late):
            f[5] += 3
    ms = _timed(lambda: arrive([R.flags[me], R.peer, 3, 5, 4, missing], {}))
    assert int(missing[0]) == 1 << late
    assert 19.0 <= ms < 1000.0, ms
    assert int(R.flags[me][5]) == 899
    _case(f"give-up late={late}: manifest entry of the short build, slot nobody else reached")
    ms = _timed(lambda: _op(ctx, SHORT, "kern_k3_rs_arrive1", ARRIVE_SPEC)(
        [None, None, None, R.flags[me], R.peer, 0, 1, 6, 6, me, 4], {}))
    assert 19.0 <= ms < 1000.0, ms
    assert int(R.flags[me][6]) == 1


def _hip():
    L = ctypes.CDLL("libamdhip64.so")
    L.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_uint]
    L.hipHostFree.argtypes = [ctypes.c_void_p]
    L.hipHostGetDevicePointer.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_void_p,
                                          ctypes.c_uint]
    return L


def test_arrive_sees_a_peer_arriving_during_the_wait(ctx):
    """Rank 1's counters live in coherent pinned host memory; the host raises them
    50 ms after the launch, while rank 0 polls.  The wait must end then, well
    before its 2 s give-up."""
    L = _hip()
    hp = ctypes.c_void_p()
    assert L.hipHostMalloc(ctypes.byref(hp), SLOTS * 8, 0x40000000) == 0  # hipHostMallocCoherent
    try:
        dp = ctypes.c_void_p()
        assert L.hipHostGetDevicePointer(ctypes.byref(dp), hp, 0) == 0
        host = np.ctypeslib.as_array((ctypes.c_uint64 * SLOTS).from_address(hp.value))
        host[:] = 0
        own = torch.zeros(SLOTS, dtype=torch.int64, device="cuda")
        peer = torch.tensor([own.data_ptr(), dp.value], dtype=torch.int64, device="cuda")
        missing = torch.full((1,), -1, dtype=torch.int32, device="cuda")
        ctx.epoch_bump(own, 896)
        torch.cuda.synchronize()
        _case("live peer: launch, then arrive from the host after 50 ms")
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        ctx.rs_arrive(own, peer, 896, 9, 2, missing)
        e.record()
        time.sleep(0.05)
        assert not e.query(), "the wait ended before the peer arrived"
        host[9] = 896
        torch.cuda.synchronize()
        ms = s.elapsed_time(e)
        assert int(missing[0]) == 0
        assert 40.0 <= ms < 1500.0, ms
        assert int(own[9]) == 896
    finally:
        torch.cuda.synchronize()
        L.hipHostFree(hp)


def test_manifest_push_then_normed_sync(ctx):
    """The default manifest's res_in sequence on rank 2 of 4: k3_flags_init (load
    program), k3_epoch_bump (coll_epoch, grid from the tokens), the residual push,
    then k3_allgather_push (normed_sync: the arrival barrier on slot 1), all from
    the manifest's own op descriptions; the peers' pushes and arrivals are played
    by the host."""
    ops = json.load(open(os.path.join(GOLDEN, "manifest_hot_ops.json")))
    tokens, B, rank = 4 * 24, 24, 2
    env = {"tokens": tokens, "rank_tp": rank}
    units = -(-(-(-tokens // 4) * 7168) // 32768)  # the manifest's grid expression: 6 here
    R = GpuRanks(ctx, 4)
    _case("manifest k3_flags_init / k3_epoch_bump")
    for f in R.flags:
        k3h.ManifestOp(ctx, "k3_flags_init", ops["k3_flags_init"])([f, SLOTS], env)
        k3h.ManifestOp(ctx, "k3_epoch_bump", ops["k3_epoch_bump"])([f], env)
    torch.cuda.synchronize()
    assert all(int(f[0]) == units for f in R.flags)
    _case("manifest attnres_rms_push_first_v3 + k3_allgather_push")
    g = rng(611)
    prefix, blocks = normal_bf16(g, (B, H)), normal_bf16(g, (B, 8, H), 0.0, 2.0)
    sw = g.standard_normal(H, dtype=np.float32) * np.float32(0.05)
    gamma = normal_bf16(g, (H,), 1.0, 0.1)
    normed = [torch.zeros((4 * B, H), dtype=torch.bfloat16, device="cuda") for _ in range(4)]
    npeer = torch.tensor([t.data_ptr() for t in normed], dtype=torch.int64, device="cuda")
    k3h.ManifestOp(ctx, "attnres_rms_push_first_v3", ops["attnres_rms_push_first_v3"])(
        [to_dev(prefix), to_dev(blocks), to_dev(sw), to_dev(gamma), normed[rank], npeer, B], env)
    R.arrive_peers(rank, units, 1)
    ms = _timed(lambda: k3h.ManifestOp(ctx, "k3_allgather_push", ops["k3_allgather_push"])(
        [normed[rank], normed[rank], npeer, R.flags[rank], R.peer, units, 1], env))
    assert ms < 200.0, ms
    assert int(R.flags[rank][1]) == units
    _, wn = O.attnres_rms(prefix, blocks, sw, gamma, 0, 1, B)
    for q in range(4):
        got = from_dev(normed[q])[rank * B:(rank + 1) * B]
        assert (got == wn).all(), f"normed_all[{q}]"


def test_arrive_compares_the_low_word(ctx):
    """As the reference (k3_rs_arrive1.cu:56-58) and the oracle: the wait compares
    the low 32 bits, so a peer counter past 2^32 compares by its low word."""
    _case("low-word comparison")
    own = torch.zeros(SLOTS, dtype=torch.int64, device="cuda")
    peer = torch.zeros(SLOTS, dtype=torch.int64, device="cuda")
    fpeer = torch.tensor([own.data_ptr(), peer.data_ptr()], dtype=torch.int64, device="cuda")
    missing = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    arrive = _op(ctx, SHORT, "k3h_rs_arrive_mask", MASK_SPEC)
    own[0] = (1 << 32) + 5   # epoch: low word 5
    peer[4] = 7              # low word 7 >= 5 (the u64 far below the epoch)
    arrive([own, fpeer, 5, 4, 2, missing], {})
    torch.cuda.synchronize()
    assert int(missing[0]) == 0
    peer[5] = (1 << 32) + 3  # low word 3 < 5 (the u64 above 5): given up on after 20 ms
    arrive([own, fpeer, 5, 5, 2, missing], {})
    torch.cuda.synchronize()
    assert int(missing[0]) == 0b10
