"""GPU parity: the residual push family (res_in storing normed into every rank's
normed_all, its statistics hand-off to res_mlp, the land_add2 fold) and res_mlp's
statistics-consuming nb entries, against the C oracle through the k3h C-ABI.
Bar: bit-exact for every output.  On one GPU the four "ranks'" normed_all
buffers are four local allocations whose addresses go into dst_peer."""
import json
import os

import numpy as np
import pytest
import torch

import k3h
import oracle as O
from k3data import H, from_dev, normal_bf16, rng, to_dev

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
SENTINEL = 0x7fbf  # a NaN pattern no kernel produces from these inputs


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _eq(name, got, want):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (name, got.shape, want.shape)
    bad = np.flatnonzero(got.ravel() != want.ravel())
    assert bad.size == 0, f"{name}: {bad.size} of {got.size} differ, first at {bad[:5]}"


def _inputs(seed, B):
    g = rng(seed)
    prefix = normal_bf16(g, (B, H))
    partial = normal_bf16(g, (B, H))
    blocks = normal_bf16(g, (B, 8, H), 0.0, 2.0)
    sw = g.standard_normal(H, dtype=np.float32) * np.float32(0.05)
    sw_mlp = g.standard_normal(H, dtype=np.float32) * np.float32(0.05)
    gamma = normal_bf16(g, (H,), 1.0, 0.1)
    return g, prefix, partial, blocks, sw, sw_mlp, gamma


class Ranks:
    """nranks normed_all buffers [nranks * B, H] on this GPU, filled with a sentinel."""

    def __init__(self, nranks, B):
        self.bufs = [torch.full((nranks * B, H), 0, dtype=torch.int16, device="cuda").fill_(SENTINEL)
                     .view(torch.bfloat16) for _ in range(nranks)]
        self.peer = torch.tensor([b.data_ptr() for b in self.bufs], dtype=torch.int64, device="cuda")
        self.B = B

    def check(self, rank, want):
        B = self.B
        for q, buf in enumerate(self.bufs):
            got = from_dev(buf)
            _eq(f"normed_all[{q}] slice of rank {rank}", got[rank * B:(rank + 1) * B], want)
            rest = np.concatenate([got[:rank * B], got[(rank + 1) * B:]])
            assert (rest == SENTINEL).all(), f"normed_all[{q}]: rows outside rank {rank}'s slice written"


@pytest.mark.parametrize("version", [1, 3])
@pytest.mark.parametrize("nb,snapshot,B,rank,nranks", [
    (0, 1, 37, 1, 4),     # the manifest's first-layer call (nb 0, snapshot 1): the 896-thread entry
    (0, 0, 5, 0, 1),      # nb 0, one rank, no snapshot
    (0, 1, 19, 7, 8),     # nb 0, eight ranks (the most), last rank
    (3, 0, 16, 0, 4),
    (8, 1, 9, 3, 4),      # nb = 8: no snapshot slot left
    (2, 1, 5, 0, 1),      # one rank: no peers read
    (1, 1, 11, 2, 4),     # nb 1..8 run the 256-thread split entries
    (4, 0, 6, 5, 8),
    (5, 1, 13, 1, 4),
    (6, 1, 7, 2, 4),
    (7, 0, 10, 0, 8),
])
def test_attnres_rms_push(ctx, version, nb, snapshot, B, rank, nranks):
    _case(f"push v{version} nb={nb} snapshot={snapshot} B={B} rank={rank}/{nranks}")
    _, prefix, _, blocks, sw, _, gamma = _inputs(400 + nb + B, B)
    R = Ranks(nranks, B)
    blk = to_dev(blocks)
    ctx.attnres_rms_push(to_dev(prefix), blk, to_dev(sw), to_dev(gamma), R.bufs[rank], R.peer, nb,
                         snapshot, B, rank, nranks, version=version)
    torch.cuda.synchronize()
    wblk, wn = O.attnres_rms(prefix, blocks, sw, gamma, nb, snapshot, B)
    R.check(rank, wn)
    _eq("blocks", from_dev(blk), wblk)


@pytest.mark.parametrize("nb,B", [(0, 8), (1, 33), (2, 12), (3, 10), (4, 9), (5, 16), (6, 5), (7, 11),
                                  (8, 7)])
def test_attnres_rms_push_stats(ctx, nb, B):
    _case(f"push_stats nb={nb} B={B}")
    _, prefix, _, blocks, sw, sw_mlp, gamma = _inputs(420 + nb, B)
    R = Ranks(4, B)
    stats = torch.full((B, 8, 2), -1.0, dtype=torch.float32, device="cuda")
    blk = to_dev(blocks)
    ctx.attnres_rms_push_stats(to_dev(prefix), blk, to_dev(sw), to_dev(gamma), R.bufs[2], R.peer,
                               nb, 1, B, 2, 4, to_dev(sw_mlp), stats)
    torch.cuda.synchronize()
    wblk, wn, wst = O.attnres_rms_stats(prefix, blocks, sw, gamma, nb, 1, B, sw_mlp=sw_mlp)
    R.check(2, wn)
    _eq("blocks", from_dev(blk), wblk)
    got = from_dev(stats)
    _eq("stats", got[:, :nb].view(np.uint32), wst[:, :nb].view(np.uint32))
    assert (got[:, nb:] == -1.0).all(), "stats past nb written"


@pytest.mark.parametrize("nb,two,B", [(0, 1, 12), (1, 1, 9), (2, 0, 10), (3, 1, 6), (4, 0, 21),
                                      (4, 1, 7), (5, 1, 5), (6, 0, 9), (7, 1, 8), (8, 1, 6)])
def test_attnres_rms_push_add2(ctx, nb, two, B):
    _case(f"push_add2 nb={nb} two={two} B={B}")
    g, _, _, blocks, sw, sw_mlp, gamma = _inputs(440 + nb, B)
    p1, p2, prefix2 = (normal_bf16(g, (B, H)) for _ in range(3))
    R = Ranks(4, B)
    stats = torch.zeros((B, 8, 2), dtype=torch.float32, device="cuda")
    hidden = torch.empty((B, H), dtype=torch.bfloat16, device="cuda")
    blk = to_dev(blocks)
    ctx.attnres_rms_push_add2(blk, to_dev(sw), to_dev(gamma), R.bufs[0], R.peer, nb, 1, B, 0, 4,
                              to_dev(sw_mlp), stats, to_dev(p1), to_dev(p2), to_dev(prefix2),
                              hidden, two)
    torch.cuda.synchronize()
    wh = O.land_add2_bf16(p1, p2, prefix2, two, B)
    _eq("hidden", from_dev(hidden), wh)
    wblk, wn, wst = O.attnres_rms_stats(wh, blocks, sw, gamma, nb, 1, B, sw_mlp=sw_mlp)
    R.check(0, wn)
    _eq("blocks", from_dev(blk), wblk)
    _eq("stats", from_dev(stats)[:, :nb].view(np.uint32), wst[:, :nb].view(np.uint32))


@pytest.mark.parametrize("nb", range(1, 9))
def test_nb_stats_consumer(ctx, nb):
    """res_mlp's nb entries with res_in's statistics: bit-exact with the oracle for
    every nb_stats, and -- given statistics computed with sw_mlp = res_mlp's sw --
    bit-identical to the plain nb entry (k3_residual_nb), the hand-off's contract."""
    B = 19
    _, prefix, partial, blocks, sw_in, sw_mlp, gamma = _inputs(460 + nb, B)
    R = Ranks(1, B)
    stats = torch.zeros((B, 8, 2), dtype=torch.float32, device="cuda")
    d = {k: to_dev(v) for k, v in (("prefix", prefix), ("partial", partial), ("blocks", blocks),
                                    ("sw_in", sw_in), ("sw_mlp", sw_mlp), ("gamma", gamma))}
    # res_in on the GPU produces the statistics (candidates c < nb)
    ctx.attnres_rms_push_stats(d["prefix"], d["blocks"], d["sw_in"], d["gamma"], R.bufs[0], R.peer,
                               nb, 0, B, 0, 1, d["sw_mlp"], stats)
    p2a = torch.empty((B, H), dtype=torch.bfloat16, device="cuda")
    na = torch.empty_like(p2a)
    ctx.land_add_attnres_rms_nb(d["partial"], d["prefix"], d["blocks"], d["sw_mlp"], d["gamma"],
                                p2a, na, nb, 0, B)
    torch.cuda.synchronize()
    plain = (from_dev(p2a), from_dev(na))
    st = from_dev(stats)
    for ns in sorted({0, 1, nb // 2, nb}):
        _case(f"nb_stats consumer nb={nb} nb_stats={ns}")
        p2 = torch.empty((B, H), dtype=torch.bfloat16, device="cuda")
        nrm = torch.empty_like(p2)
        ctx.land_add_attnres_rms_nb_stats(d["partial"], d["prefix"], d["blocks"], d["sw_mlp"],
                                          d["gamma"], p2, nrm, nb, 0, B, stats, ns)
        torch.cuda.synchronize()
        wp2, wn = O.land_add_attnres_rms_stats(partial, prefix, blocks, sw_mlp, gamma, nb, 0, B, st, ns)
        _eq("prefix2", from_dev(p2), wp2)
        _eq("normed", from_dev(nrm), wn)
        _eq("normed == plain nb entry", from_dev(nrm), plain[1])


@pytest.mark.parametrize("two,B", [(0, 3), (1, 40)])
def test_land_add2_bf16(ctx, two, B):
    _case(f"land_add2_bf16 two={two} B={B}")
    g = rng(480 + B)
    p1, p2, prefix2 = (normal_bf16(g, (B, H)) for _ in range(3))
    hidden = torch.empty((B, H), dtype=torch.bfloat16, device="cuda")
    ctx.land_add2_bf16(to_dev(p1), to_dev(p2), to_dev(prefix2), hidden, two, B)
    torch.cuda.synchronize()
    _eq("hidden", from_dev(hidden), O.land_add2_bf16(p1, p2, prefix2, two, B))


def test_push_full_rank_share(ctx):
    """One rank's share at the 16k prefill: B = 4096 rows, nb = 0, snapshot."""
    B = 4096
    _case(f"push v3 at B={B}")
    g = rng(490)
    prefix = normal_bf16(g, (B, H))
    gamma = normal_bf16(g, (H,), 1.0, 0.1)
    blocks = torch.zeros((B, 8, H), dtype=torch.bfloat16, device="cuda")
    R = Ranks(4, B)
    ctx.attnres_rms_push(to_dev(prefix), blocks, None, to_dev(gamma), R.bufs[1], R.peer, 0, 1, B,
                         1, 4, version=3)
    torch.cuda.synchronize()
    _, wn = O.attnres_rms(prefix, None, None, gamma, 0, 0, B)
    R.check(1, wn)
    _eq("blocks[:, 0]", from_dev(blocks)[:, 0], prefix)


@pytest.mark.parametrize("nb", [0, 4, 8])
def test_push_add2_full_rank_share(ctx, nb):
    """push_add2 at one rank's share of the 16k prefill (B = 4096 rows, the
    benchmarked shape), every row bit-exact: hidden, every rank's normed copy,
    the snapshot slot and the statistics."""
    B = 4096
    _case(f"push_add2 nb={nb} at B={B}")
    g, _, _, blocks, sw, sw_mlp, gamma = _inputs(470 + nb, B)
    p1, p2, prefix2 = (normal_bf16(g, (B, H)) for _ in range(3))
    R = Ranks(4, B)
    stats = torch.zeros((B, 8, 2), dtype=torch.float32, device="cuda")
    hidden = torch.empty((B, H), dtype=torch.bfloat16, device="cuda")
    blk = to_dev(blocks)
    ctx.attnres_rms_push_add2(blk, to_dev(sw), to_dev(gamma), R.bufs[3], R.peer, nb, 1, B, 3, 4,
                              to_dev(sw_mlp), stats, to_dev(p1), to_dev(p2), to_dev(prefix2),
                              hidden, 1)
    torch.cuda.synchronize()
    wh = O.land_add2_bf16(p1, p2, prefix2, 1, B)
    _eq("hidden", from_dev(hidden), wh)
    wblk, wn, wst = O.attnres_rms_stats(wh, blocks, sw, gamma, nb, 1, B, sw_mlp=sw_mlp)
    R.check(3, wn)
    _eq("blocks", from_dev(blk), wblk)
    _eq("stats", from_dev(stats)[:, :nb].view(np.uint32), wst[:, :nb].view(np.uint32))


def test_manifest_push_ops(ctx):
    """attnres_rms_push_first_v3, attnres_rms_push_add2 and the nb4 / nb8 stats
    entries run from the manifests' own op descriptions (rank from the env)."""
    ops = json.load(open(os.path.join(GOLDEN, "manifest_hot_ops.json")))
    tokens, B, rank = 4 * 24, 24, 2
    env = {"tokens": tokens, "rank_tp": rank}
    g, prefix, partial, blocks, sw, sw_mlp, gamma = _inputs(495, B)
    _case("manifest attnres_rms_push_first_v3")
    R = Ranks(4, B)
    blk = to_dev(blocks)
    k3h.ManifestOp(ctx, "attnres_rms_push_first_v3", ops["attnres_rms_push_first_v3"])(
        [to_dev(prefix), blk, to_dev(sw), to_dev(gamma), R.bufs[rank], R.peer, B], env)
    torch.cuda.synchronize()
    wblk, wn = O.attnres_rms(prefix, blocks, sw, gamma, 0, 1, B)
    R.check(rank, wn)
    _eq("blocks", from_dev(blk), wblk)

    _case("manifest attnres_rms_push_add2")
    nb = 3
    p1, p2, prefix2 = (normal_bf16(g, (B, H)) for _ in range(3))
    R = Ranks(4, B)
    blk = to_dev(blocks)
    stats = torch.zeros((B, 8, 2), dtype=torch.float32, device="cuda")
    hidden = torch.empty((B, H), dtype=torch.bfloat16, device="cuda")
    k3h.ManifestOp(ctx, "attnres_rms_push_add2", ops["attnres_rms_push_add2"])(
        [blk, to_dev(sw), to_dev(gamma), R.bufs[rank], R.peer, nb, 1, B, to_dev(sw_mlp), stats,
         to_dev(p1), to_dev(p2), to_dev(prefix2), hidden, 1], env)
    torch.cuda.synchronize()
    wh = O.land_add2_bf16(p1, p2, prefix2, 1, B)
    _eq("hidden", from_dev(hidden), wh)
    wblk, wn, wst = O.attnres_rms_stats(wh, blocks, sw, gamma, nb, 1, B, sw_mlp=sw_mlp)
    R.check(rank, wn)
    _eq("stats", from_dev(stats)[:, :nb].view(np.uint32), wst[:, :nb].view(np.uint32))

    for op, k in (("land_add_attnres_rms_bf16_v2_nb4", 4), ("land_add_attnres_rms_bf16_v2_nb8", 8)):
        _case(f"manifest {op}")
        st = np.asarray(g.standard_normal((B, 8, 2)) * 100, np.float32)
        st[..., 0] = np.abs(st[..., 0]) + 1.0
        p2t = torch.empty((B, H), dtype=torch.bfloat16, device="cuda")
        nrm = torch.empty_like(p2t)
        k3h.ManifestOp(ctx, op, ops[op])(
            [to_dev(partial), to_dev(prefix), to_dev(blocks), to_dev(sw), to_dev(gamma), p2t, nrm, k,
             0, B, to_dev(st), k - 1], env)
        torch.cuda.synchronize()
        wp2, wn = O.land_add_attnres_rms_stats(partial, prefix, blocks, sw, gamma, k, 0, B, st, k - 1)
        _eq(f"{op} prefix2", from_dev(p2t), wp2)
        _eq(f"{op} normed", from_dev(nrm), wn)
