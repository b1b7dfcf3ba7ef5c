"""GPU parity: router top-k, argmax, EP routing tables, MXFP8 permute, weighted
finalize and the weight layouts against the C oracle -- bit-exact for indices,
weights, every routing table, permuted bytes and the finalize output (both
sides use the same fma order)."""
import json
import os

import numpy as np
import pytest
import torch

import k3h
import oracle as O
from k3data import from_dev, normal_bf16, rng, to_bf16, to_dev

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
E, RANK = 56, 0
_MOE_V4 = "k3_moe_prefill_v4+EP_RANKS=4+EP_STRIDED=1+TILE_SHIFT=7+SCATTER_WARPS=16"


def _case(m):
    print(f"[case] {m}", flush=True)


def _eq(name, got, want):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (name, got.shape, want.shape)
    bad = np.flatnonzero(got.ravel() != want.ravel())
    assert bad.size == 0, f"{name}: {bad.size} of {got.size} differ, first at {bad[:5]}"


def _router_inputs(T, seed):
    g = rng(seed)
    S = g.standard_normal((T, 224), dtype=np.float32)
    S[0, 10:20] = S[0, 5]
    bias = (g.standard_normal(224) * 0.01).astype(np.float32)
    bias[10:20] = bias[5]
    rs = to_bf16(np.array([2.5], np.float32))
    return S, bias, rs


def _run_router(ctx, S, bias, rs, T, topk):
    idx = torch.empty((T, topk), dtype=torch.int32, device="cuda")
    wts = torch.empty((T, topk), dtype=torch.float32, device="cuda")
    ctx.router_topk(to_dev(S), to_dev(bias), to_dev(rs), idx, wts, T, topk=topk)
    torch.cuda.synchronize()
    return from_dev(idx), from_dev(wts)


@pytest.mark.parametrize("T,topk", [(16384, 8), (4096, 16), (1, 16), (5, 8)])
def test_router_topk(ctx, T, topk):
    _case(f"router_topk T={T} topk={topk}")
    S, bias, rs = _router_inputs(T, 1300 + T)
    want_i, want_w = O.router_topk(S, bias, rs[0], T, topk)
    idx, wts = _run_router(ctx, S, bias, rs, T, topk)
    _eq("idx", idx, want_i)
    _eq("wts", wts.view(np.uint32), want_w.view(np.uint32))


@pytest.mark.parametrize("topk", [8, 16])
def test_router_topk_ties(ctx, topk):
    """Equal keys: rows of one repeated logit (every key equal), rows whose logits
    repeat with period 32 or 64 (equal keys in different slots of one lane and in
    different lanes), and odd row counts; ties must go to the smallest expert id."""
    _case(f"router_topk ties topk={topk}")
    T = 9
    S = np.zeros((T, 224), np.float32)
    S[1] = 0.5
    S[2] = np.tile(np.linspace(-1, 1, 32, dtype=np.float32), 7)
    S[3] = np.tile(np.linspace(1, -1, 64, dtype=np.float32), 4)[:224]
    S[4] = np.repeat(np.float32([0.25, -0.25, 1.0, 0.0, 2.0, -2.0, 0.75]), 32)
    S[5:] = np.random.default_rng(77).integers(-2, 3, (T - 5, 224)).astype(np.float32)
    bias = np.zeros(224, np.float32)
    rs = np.array([0x4020], np.uint16)  # bf16 2.5
    want_i, want_w = O.router_topk(S, bias, rs[0], T, topk)
    assert (want_i[0] == np.arange(topk)).all()  # all keys equal: experts 0 .. topk - 1
    idx, wts = _run_router(ctx, S, bias, rs, T, topk)
    _eq("idx", idx, want_i)
    _eq("wts", wts.view(np.uint32), want_w.view(np.uint32))


@pytest.mark.parametrize("topk", [8, 16])
def test_router_topk_near_ties(ctx, topk):
    """Rows whose largest logits lie a few ulps apart (and rows with an infinite
    logit): the keys near the top-k boundary differ in their last bits, and the
    exact keys must decide the picks and their order (a kernel that ranked by an
    approximate logistic first would be caught here)."""
    _case(f"router_topk near ties topk={topk}")
    T = 95
    g = rng(1770 + topk)
    S = g.standard_normal((T, 224), dtype=np.float32)
    for t in range(T - 3):
        top = g.choice(224, size=topk + 4, replace=False)
        base = np.float32(2.0 + g.random())
        steps = g.integers(0, 4, topk + 4).astype(np.int32)  # 0-3 ulps apart, shuffled
        S[t, top] = (base.view(np.int32) + steps).view(np.float32)
    S[T - 3, 200] = np.inf
    S[T - 2, 17] = -np.inf
    bias = (g.standard_normal(224) * 1e-7).astype(np.float32)  # perturbations of a few ulps
    rs = to_bf16(np.array([2.5], np.float32))
    want_i, want_w = O.router_topk(S, bias, rs[0], T, topk)
    idx, wts = _run_router(ctx, S, bias, rs, T, topk)
    _eq("idx", idx, want_i)
    _eq("wts", wts.view(np.uint32), want_w.view(np.uint32))


@pytest.mark.parametrize("topk", [8, 16])
def test_router_topk_candidate_edges(ctx, topk):
    """Rows at the edges of the key order: 40 experts within a few ulps of each
    other at the top of a row (in one lane-half and spread over slots), every
    logistic 0 or 1 (keys equal to the biases, or the biases plus one),
    infinite logits, -inf and +inf biases (infinite keys tie and go to the
    smallest ids), and a second bias vector finite for five experts only, so
    that the top-k reaches into the -inf keys."""
    _case(f"router_topk candidate edges topk={topk}")
    T = 12
    g = rng(1990 + topk)
    S = g.standard_normal((T, 224), dtype=np.float32)
    close = (np.float32(3.0).view(np.int32) + g.integers(0, 3, 40)).astype(np.int32)
    S[1, :40] = close.view(np.float32)
    S[2, :] = S[1, :]
    S[3, 100:140] = close.view(np.float32)
    S[5, :] = np.float32(-200.0)  # every logistic 0: keys are the biases
    S[6, ::7] = np.inf
    S[7, :] = np.float32(40.0)  # every logistic 1
    rs = to_bf16(np.array([2.5], np.float32))
    b1 = (g.standard_normal(224) * 0.01).astype(np.float32)
    b1[30:224:3] = -np.inf
    b1[[3, 77, 150]] = np.inf
    b2 = (g.standard_normal(224) * 0.01).astype(np.float32)
    b2[5:] = -np.inf
    for bias in (b1, b2):
        want_i, want_w = O.router_topk(S, bias, rs[0], T, topk)
        idx, wts = _run_router(ctx, S, bias, rs, T, topk)
        _eq("idx", idx, want_i)
        _eq("wts", wts.view(np.uint32), want_w.view(np.uint32))


def test_argmax_f32(ctx):
    _case("argmax")
    g = rng(1400)
    B, n, parts = 16, 163840, 64
    x = g.standard_normal((B, n), dtype=np.float32)
    x[1, 100] = x[1, 150000] = 9.0
    x[2, :] = -np.inf
    x[3, 77] = np.inf
    pm, pi = O.argmax_partial(x, B, n, parts)
    out = O.argmax_final(pm, pi, B, parts)
    d_pm = torch.empty(B * parts, dtype=torch.float32, device="cuda")
    d_pi = torch.empty(B * parts, dtype=torch.int32, device="cuda")
    d_out = torch.empty(B, dtype=torch.int64, device="cuda")
    ctx.argmax_f32(to_dev(x), d_pm, d_pi, d_out, B, n, parts)
    torch.cuda.synchronize()
    _eq("pmax", from_dev(d_pm).view(np.uint32), pm.view(np.uint32))
    _eq("pidx", from_dev(d_pi), pi)
    _eq("out", from_dev(d_out), out)


def _gpu_route(ctx, ids, T, topk):
    nblk = (T + 255) // 256
    cap = T * topk + E * 128
    d_ids = to_dev(ids)
    bc = torch.empty(nblk * E, dtype=torch.int32, device="cuda")
    bo = torch.empty(nblk * E, dtype=torch.int32, device="cuda")
    cb = torch.full((cap // 128 + 1,), -1, dtype=torch.int32, device="cuda")
    cl = torch.full((cap // 128 + 1,), -1, dtype=torch.int32, device="cuda")
    nne = torch.zeros(1, dtype=torch.int32, device="cuda")
    tp = torch.zeros(1, dtype=torch.int32, device="cuda")
    rmap = torch.full((cap,), -1, dtype=torch.int32, device="cuda")
    e2p = torch.empty(T * topk, dtype=torch.int32, device="cuda")
    ctx.moe_route_count(d_ids, T, RANK, E, bc, topk=topk)
    ctx.moe_route_tables(bc, nblk, E, 128, bo, cb, cl, nne, tp, rmap, T=T, topk=topk)
    ctx.moe_route_scatter(d_ids, bo, T, RANK, E, rmap, e2p, topk=topk)
    torch.cuda.synchronize()
    return dict(bc=bc, bo=bo, cb=cb, cl=cl, nne=nne, tp=tp, rmap=rmap, e2p=e2p)


# T = 40000: 157 blocks x 56 experts exceed the 8192 counts route_tables stages in LDS
@pytest.mark.parametrize("T,topk", [(16384, 8), (16384, 16), (300, 16), (257, 8), (40000, 8)])
def test_ep_routing_tables(ctx, T, topk):
    _case(f"routing T={T} topk={topk}")
    S, bias, rs = _router_inputs(T, 1500 + T + topk)
    ids, _ = O.router_topk(S, bias, rs[0], T, topk)
    nblk = (T + 255) // 256
    bc = O.route_count(ids, T, topk, RANK, E)
    tab = O.route_tables(bc, nblk, E, 128, T * topk + E * 128)
    rmap, e2p = O.route_scatter(ids, tab["blockoff"], T, topk, RANK, E, tab["route_map"])
    d = _gpu_route(ctx, ids, T, topk)
    _eq("blockcount", from_dev(d["bc"]), bc)
    _eq("blockoff", from_dev(d["bo"]), tab["blockoff"])
    nne, tp = tab["num_non_exiting"], tab["total_padded"]
    assert from_dev(d["nne"])[0] == nne and from_dev(d["tp"])[0] == tp
    _eq("cta_batch", from_dev(d["cb"])[:nne], tab["cta_batch"][:nne])
    _eq("cta_limit", from_dev(d["cl"])[:nne], tab["cta_limit"][:nne])
    _eq("route_map", from_dev(d["rmap"])[:tp], rmap[:tp])
    _eq("exp2perm", from_dev(d["e2p"]), e2p)


# one launch of k3h_moe_route against the oracle's chain; each case runs twice on
# one `sync` (the barrier words must come back zero); T = 1 and T = 65536 are the
# smallest and largest grids of the one-launch path
@pytest.mark.parametrize("T,topk", [(16384, 8), (16384, 16), (300, 16), (257, 8), (40000, 8),
                                    (1, 8), (65536, 8)])
def test_route_one_launch(ctx, T, topk):
    _case(f"one-launch routing T={T} topk={topk}")
    S, bias, rs = _router_inputs(T, 1700 + T + topk)
    ids, _ = O.router_topk(S, bias, rs[0], T, topk)
    nblk = (T + 255) // 256
    bc = O.route_count(ids, T, topk, RANK, E)
    cap = T * topk + E * 128
    tab = O.route_tables(bc, nblk, E, 128, cap)
    rmap, e2p = O.route_scatter(ids, tab["blockoff"], T, topk, RANK, E, tab["route_map"])
    nne, tp = tab["num_non_exiting"], tab["total_padded"]
    d_ids = to_dev(ids)
    sync = torch.zeros(2, dtype=torch.int32, device="cuda")
    for rep in range(2):
        o = dict(bc=torch.full((nblk * E,), -7, dtype=torch.int32, device="cuda"),
                 bo=torch.full((nblk * E,), -7, dtype=torch.int32, device="cuda"),
                 cb=torch.full((cap // 128 + 1,), -7, dtype=torch.int32, device="cuda"),
                 cl=torch.full((cap // 128 + 1,), -7, dtype=torch.int32, device="cuda"),
                 nne=torch.full((1,), -7, dtype=torch.int32, device="cuda"),
                 tp=torch.full((1,), -7, dtype=torch.int32, device="cuda"),
                 rmap=torch.full((cap,), -7, dtype=torch.int32, device="cuda"),
                 e2p=torch.full((T * topk,), -7, dtype=torch.int32, device="cuda"))
        ctx.moe_route(d_ids, T, RANK, E, o["bc"], o["bo"], o["cb"], o["cl"], o["nne"], o["tp"],
                      o["rmap"], o["e2p"], sync, topk=topk)
        torch.cuda.synchronize()
        assert from_dev(sync).tolist() == [0, 0], "barrier words not reset"
        _eq("blockcount", from_dev(o["bc"]), bc)
        _eq("blockoff", from_dev(o["bo"]), tab["blockoff"])
        assert from_dev(o["nne"])[0] == nne and from_dev(o["tp"])[0] == tp
        _eq("cta_batch", from_dev(o["cb"])[:nne], tab["cta_batch"][:nne])
        _eq("cta_limit", from_dev(o["cl"])[:nne], tab["cta_limit"][:nne])
        _eq("route_map", from_dev(o["rmap"])[:tp], rmap[:tp])
        assert (from_dev(o["rmap"])[tp:] == -7).all(), "rows past total_padded written"
        _eq("exp2perm", from_dev(o["e2p"]), e2p)


def _route_expect(T, topk, seed):
    S, bias, rs = _router_inputs(T, seed)
    ids, _ = O.router_topk(S, bias, rs[0], T, topk)
    nblk = (T + 255) // 256
    cap = T * topk + E * 128
    bc = O.route_count(ids, T, topk, RANK, E)
    tab = O.route_tables(bc, nblk, E, 128, cap)
    rmap, e2p = O.route_scatter(ids, tab["blockoff"], T, topk, RANK, E, tab["route_map"])
    return ids, nblk, cap, bc, tab, rmap, e2p


def _route_outputs(T, topk, nblk, cap):
    def fill(n):
        return torch.full((n,), -7, dtype=torch.int32, device="cuda")
    return dict(bc=fill(nblk * E), bo=fill(nblk * E), cb=fill(cap // 128 + 1), cl=fill(cap // 128 + 1),
                nne=fill(1), tp=fill(1), rmap=fill(cap), e2p=fill(T * topk))


# The barrier's give-up path, forced from the host so that every workgroup still
# exits normally: sync[0] preset to -1 makes the arrivals stop one short of the
# grid size, so every workgroup's bounded wait expires and the first to give up
# poisons the count; preset to a poisoned value, every workgroup gives up at its
# first poll.  The outputs must say "nothing routed" (num_non_exiting 0,
# total_padded -1, every exp2perm entry -1, the other tables untouched), `sync`
# must come back zero, and the same `sync` must then serve a normal call.
@pytest.mark.parametrize("T,preset", [(1, -1), (300, -1), (16384, -1), (16384, -(1 << 20))])
def test_route_one_launch_gives_up(ctx, T, preset):
    topk = 8
    _case(f"one-launch routing give-up T={T} sync[0]={preset}")
    ids, nblk, cap, bc, tab, rmap, e2p = _route_expect(T, topk, 1900 + T)
    d_ids = to_dev(ids)
    sync = torch.tensor([preset, 0], dtype=torch.int32, device="cuda")
    o = _route_outputs(T, topk, nblk, cap)
    ctx.moe_route(d_ids, T, RANK, E, o["bc"], o["bo"], o["cb"], o["cl"], o["nne"], o["tp"],
                  o["rmap"], o["e2p"], sync, topk=topk)
    torch.cuda.synchronize()
    assert from_dev(sync).tolist() == [0, 0], "barrier words not reset after giving up"
    assert from_dev(o["nne"])[0] == 0 and from_dev(o["tp"])[0] == -1
    assert (from_dev(o["e2p"]) == -1).all(), "exp2perm not cleared on give-up"
    _eq("blockcount", from_dev(o["bc"]), bc)  # phase 1 precedes the barrier
    for k in ("bo", "cb", "cl", "rmap"):
        assert (from_dev(o[k]) == -7).all(), f"{k} written although the barrier failed"
    o = _route_outputs(T, topk, nblk, cap)
    ctx.moe_route(d_ids, T, RANK, E, o["bc"], o["bo"], o["cb"], o["cl"], o["nne"], o["tp"],
                  o["rmap"], o["e2p"], sync, topk=topk)
    torch.cuda.synchronize()
    assert from_dev(sync).tolist() == [0, 0]
    nne, tp = tab["num_non_exiting"], tab["total_padded"]
    assert from_dev(o["nne"])[0] == nne and from_dev(o["tp"])[0] == tp
    _eq("blockoff", from_dev(o["bo"]), tab["blockoff"])
    _eq("route_map", from_dev(o["rmap"])[:tp], rmap[:tp])
    _eq("exp2perm", from_dev(o["e2p"]), e2p)


def test_route_one_launch_empty_and_limits(ctx):
    z = torch.zeros(64, dtype=torch.int32, device="cuda")
    nne = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    tp = torch.full((1,), -7, dtype=torch.int32, device="cuda")
    ctx.moe_route(z, 0, RANK, E, z, z, z, z, nne, tp, z, z, z[:2], topk=8)
    torch.cuda.synchronize()
    assert nne.item() == 0 and tp.item() == 0
    with pytest.raises(ValueError):
        ctx.moe_route(z, 65537, RANK, E, z, z, z, z, nne, tp, z, z, z[:2], topk=8)


def test_permute_and_finalize_config5(ctx):
    """Config 5: 16384 tokens, top-8 of 224, EP rank 0 of 4 (56 local experts):
    router -> tables -> MXFP8 permute of the quantised activations -> finalize of
    bf16 expert outputs over the permuted rows."""
    T, topk, H = 16384, 8, 7168
    _case("config5 permute + finalize")
    S, bias, rs = _router_inputs(T, 1600)
    ids, wts = O.router_topk(S, bias, rs[0], T, topk)
    d = _gpu_route(ctx, ids, T, topk)
    tp = int(from_dev(d["tp"])[0])
    rmap = from_dev(d["rmap"])[:tp]
    g = rng(1601)
    x = normal_bf16(g, (T, H), outlier_p=0.001)
    q, sf = O.moe_quant(x, T, H)
    pq = torch.empty((tp, H), dtype=torch.uint8, device="cuda")
    psf = torch.empty((tp, H // 32), dtype=torch.uint8, device="cuda")
    ctx.moe_permute_mx(to_dev(q), to_dev(sf), d["rmap"], d["tp"], H, pq, psf)
    torch.cuda.synchronize()
    wpq, wpsf = O.moe_permute_mx(q, sf, rmap, tp, H)
    _eq("pq", from_dev(pq), wpq)
    _eq("psf", from_dev(psf), wpsf)
    del pq, psf
    fc2 = normal_bf16(g, (tp, H))
    out = torch.empty((T, H), dtype=torch.bfloat16, device="cuda")
    ctx.moe_finalize(to_dev(fc2), d["e2p"], to_dev(wts), out, T, H, topk=topk)
    torch.cuda.synchronize()
    want = O.moe_finalize(fc2, from_dev(d["e2p"]), wts, T, topk, H)
    _eq("finalize", from_dev(out), want)


# 70000 rows: past the 16384-workgroup grid cap, so waves stride over rows;
# 16384 columns: the widest row (16 vectors per lane)
@pytest.mark.parametrize("rows,tp,cols", [(70000, 69001, 1024), (300, 257, 16384)])
def test_permute_rows_and_widths(ctx, rows, tp, cols):
    _case(f"permute rows={rows} tp={tp} cols={cols}")
    g = rng(1650 + cols)
    T = 1000
    q = g.integers(0, 256, (T, cols), dtype=np.uint8)
    sf = g.integers(0, 256, (T, cols // 32), dtype=np.uint8)
    rmap = g.integers(0, T, rows, dtype=np.int32)
    pq = torch.zeros((rows, cols), dtype=torch.uint8, device="cuda")
    psf = torch.zeros((rows, cols // 32), dtype=torch.uint8, device="cuda")
    d_tp = torch.tensor([tp], dtype=torch.int32, device="cuda")
    ctx.moe_permute_mx(to_dev(q), to_dev(sf), to_dev(rmap), d_tp, cols, pq, psf)
    torch.cuda.synchronize()
    wpq, wpsf = O.moe_permute_mx(q, sf, rmap, tp, cols)
    _eq("pq", from_dev(pq)[:tp], wpq)
    _eq("psf", from_dev(psf)[:tp], wpsf)
    assert not from_dev(pq)[tp:].any() and not from_dev(psf)[tp:].any()  # rows past tp untouched


@pytest.mark.parametrize("cols", [3584, 7168, 8])
def test_finalize_cols(ctx, cols):
    T, topk = 1000, 16
    _case(f"finalize cols={cols}")
    S, bias, rs = _router_inputs(T, 1700 + cols)
    ids, wts = O.router_topk(S, bias, rs[0], T, topk)
    d = _gpu_route(ctx, ids, T, topk)
    tp = int(from_dev(d["tp"])[0])
    fc2 = normal_bf16(rng(1701), (tp, cols))
    out = torch.empty((T, cols), dtype=torch.bfloat16, device="cuda")
    ctx.moe_finalize(to_dev(fc2), d["e2p"], to_dev(wts), out, T, cols, topk=topk)
    torch.cuda.synchronize()
    _eq("finalize", from_dev(out), O.moe_finalize(fc2, from_dev(d["e2p"]), wts, T, topk, cols))


@pytest.mark.parametrize("topk,cols", [(8, 7168), (16, 7168), (8, 1032), (16, 8)])
def test_finalize_every_slot_count(ctx, topk, cols):
    """Token t has exactly t % (topk + 1) local slots, at random slot positions and
    rows: every per-count path of the finalize kernel (0 .. topk live slots), and
    for cols = 1032 a last step that covers only part of the row."""
    _case(f"finalize slot counts topk={topk} cols={cols}")
    g = rng(1750 + topk + cols)
    T, rows = 4 * (topk + 1) + 3, 97
    e2p = np.full((T, topk), -1, dtype=np.int32)
    for t in range(T):
        live = g.choice(topk, size=t % (topk + 1), replace=False)
        e2p[t, live] = g.integers(0, rows, size=live.size)
    wts = g.random((T, topk), dtype=np.float32) * 2 - 0.5
    fc2 = normal_bf16(g, (rows, cols))
    out = torch.empty((T, cols), dtype=torch.bfloat16, device="cuda")
    d_fc2, d_e2p, d_wts = to_dev(fc2), to_dev(e2p.reshape(-1)), to_dev(wts)
    ctx.moe_finalize(d_fc2, d_e2p, d_wts, out, T, cols, topk=topk)
    torch.cuda.synchronize()
    want = O.moe_finalize(fc2, e2p.reshape(-1), wts, T, topk, cols)
    _eq("finalize", from_dev(out), want)
    # the manifest entry (one wave per token, grid ceil(T/2) x 128), which the typed
    # call does not launch, on the same inputs
    key = _MOE_V4 + ("+TOPK=8" if topk == 8 else "")
    spec = {"params": ["in buffer<bf16>", "in buffer<i32>", "in buffer<f32>", "out buffer<bf16>",
                       "i32", "i32"],
            "impl": {"launches": [{"module": key, "entry": "kern_k3_moe_finalize",
                                   "grid": [{"ceil_div": ["tokens", 2]}, 1, 1], "block": [128, 1, 1]}]}}
    out2 = torch.empty((T, cols), dtype=torch.bfloat16, device="cuda")
    k3h.ManifestOp(ctx, "moe_finalize", spec)([d_fc2, d_e2p, d_wts, out2, T, cols], {"tokens": T})
    torch.cuda.synchronize()
    _eq("finalize (manifest entry)", from_dev(out2), want)


def test_weight_layouts(ctx):
    _case("w_shuffle / sf_shuffle")
    g = rng(1800)
    experts, n, rb, kg = 3, 256, 64, 8
    src = g.integers(0, 256, (experts * n * rb,), dtype=np.uint8)
    s2 = g.integers(0, 256, (experts * n * kg,), dtype=np.uint8)
    for gated in (0, 1):
        dst = torch.empty_like(to_dev(src))
        ctx.moe_w_shuffle(to_dev(src), dst, experts, n, rb, gated)
        d2 = torch.empty_like(to_dev(s2))
        ctx.moe_sf_shuffle(to_dev(s2), d2, experts, n, kg, gated)
        torch.cuda.synchronize()
        _eq("w_shuffle", from_dev(dst), O.moe_w_shuffle(src, experts, n, rb, gated))
        _eq("sf_shuffle", from_dev(d2), O.moe_sf_shuffle(s2, experts, n, kg, gated))


def test_manifest_router_and_routing_ops(ctx):
    """ops router_topk, moe_route_count (v3 module), moe_route_tables and
    moe_route_scatter (v4 module) and moe_finalize (v3) of the default manifest."""
    ops = json.load(open(os.path.join(GOLDEN, "manifest_hot_ops.json")))
    tokens = 4096
    B = tokens // 4  # router rows: ceil(tokens / 4)
    env = {"tokens": tokens}
    S, bias, rs = _router_inputs(B, 1900)
    idx = torch.empty((B, 16), dtype=torch.int32, device="cuda")
    wts = torch.empty((B, 16), dtype=torch.float32, device="cuda")
    _case("manifest router_topk")
    k3h.ManifestOp(ctx, "router_topk", ops["router_topk"])(
        [to_dev(S), to_dev(bias), to_dev(rs), idx, wts, B], env)
    torch.cuda.synchronize()
    wi, ww = O.router_topk(S, bias, rs[0], B, 16)
    _eq("idx", from_dev(idx), wi)
    _eq("wts", from_dev(wts).view(np.uint32), ww.view(np.uint32))
    # routing over all gathered tokens (the manifest routes `tokens` ids rows)
    S2, b2, _ = _router_inputs(tokens, 1901)
    ids, w16 = O.router_topk(S2, b2, rs[0], tokens, 16)
    nblk = tokens // 256
    cap = tokens * 16 + E * 128
    bc = torch.empty(nblk * E, dtype=torch.int32, device="cuda")
    bo = torch.empty_like(bc)
    cb = torch.empty(cap // 128 + 1, dtype=torch.int32, device="cuda")
    cl = torch.empty_like(cb)
    nne = torch.zeros(1, dtype=torch.int32, device="cuda")
    tp = torch.zeros(1, dtype=torch.int32, device="cuda")
    rmap = torch.full((cap,), -1, dtype=torch.int32, device="cuda")
    e2p = torch.empty(tokens * 16, dtype=torch.int32, device="cuda")
    d_ids = to_dev(ids)
    _case("manifest moe_route_*")
    k3h.ManifestOp(ctx, "moe_route_count", ops["moe_route_count"])([d_ids, tokens, RANK, bc], env)
    k3h.ManifestOp(ctx, "moe_route_tables", ops["moe_route_tables"])(
        [bc, nblk, bo, cb, cl, nne, tp, rmap], env)
    k3h.ManifestOp(ctx, "moe_route_scatter", ops["moe_route_scatter"])(
        [d_ids, bo, tokens, RANK, rmap, e2p], env)
    torch.cuda.synchronize()
    obc = O.route_count(ids, tokens, 16, RANK, E)
    tab = O.route_tables(obc, nblk, E, 128, cap)
    wr, we = O.route_scatter(ids, tab["blockoff"], tokens, 16, RANK, E, tab["route_map"])
    t = tab["total_padded"]
    assert from_dev(tp)[0] == t
    _eq("route_map", from_dev(rmap)[:t], wr[:t])
    _eq("exp2perm", from_dev(e2p), we)
    # finalize at the manifest's cols = 3584
    _case("manifest moe_finalize")
    fc2 = normal_bf16(rng(1902), (t, 3584))
    out = torch.empty((tokens, 3584), dtype=torch.bfloat16, device="cuda")
    k3h.ManifestOp(ctx, "moe_finalize", ops["moe_finalize"])(
        [to_dev(fc2), e2p, to_dev(w16), out, tokens], env)
    torch.cuda.synchronize()
    _eq("finalize", from_dev(out), O.moe_finalize(fc2, we, w16, tokens, 16, 3584))


def test_finalize_special_values(ctx):
    """NaN (either sign), +-inf, +-max finite, a subnormal and -0 in the expert
    output rows and NaN / +-inf in the routing weights: each token's weighted sum
    carries them as the oracle's fixed-order sum (inf - inf and 0 x inf give NaN,
    sums past the largest finite round to inf); both the typed call and the
    manifest entry."""
    specials = np.array([0x7FC0, 0xFFC1, 0x7F80, 0xFF80, 0x7F7F, 0xFF7F, 0x0001, 0x8000], np.uint16)
    topk, cols = 8, 1032
    _case("finalize special values")
    g = rng(1790)
    T, rows = 60, 97
    e2p = np.full((T, topk), -1, dtype=np.int32)
    for t in range(T):
        live = g.choice(topk, size=t % (topk + 1), replace=False)
        e2p[t, live] = g.integers(0, rows, size=live.size)
    wts = g.random((T, topk), dtype=np.float32) * 2 - 0.5
    wts.reshape(-1)[g.choice(T * topk, 6, replace=False)] = [np.nan, np.inf, -np.inf, 0.0, 3e38, -0.0]
    fc2 = normal_bf16(g, (rows, cols))
    flat = fc2.reshape(-1)
    flat[g.choice(flat.size, 200, replace=False)] = specials[np.arange(200) % specials.size]
    want = O.moe_finalize(fc2, e2p.reshape(-1), wts, T, topk, cols)
    d_fc2, d_e2p, d_wts = to_dev(fc2), to_dev(e2p.reshape(-1)), to_dev(wts)
    out = torch.empty((T, cols), dtype=torch.bfloat16, device="cuda")
    ctx.moe_finalize(d_fc2, d_e2p, d_wts, out, T, cols, topk=topk)
    spec = {"params": ["in buffer<bf16>", "in buffer<i32>", "in buffer<f32>", "out buffer<bf16>",
                       "i32", "i32"],
            "impl": {"launches": [{"module": _MOE_V4 + "+TOPK=8", "entry": "kern_k3_moe_finalize",
                                   "grid": [{"ceil_div": ["tokens", 2]}, 1, 1], "block": [128, 1, 1]}]}}
    out2 = torch.empty((T, cols), dtype=torch.bfloat16, device="cuda")
    k3h.ManifestOp(ctx, "moe_finalize", spec)([d_fc2, d_e2p, d_wts, out2, T, cols], {"tokens": T})
    torch.cuda.synchronize()
    for name, got in (("finalize", from_dev(out)), ("finalize (manifest entry)", from_dev(out2))):
        gn, wn = (got & 0x7FFF) > 0x7F80, (want & 0x7FFF) > 0x7F80
        assert np.array_equal(gn, wn), f"{name}: NaN positions differ ({gn.sum()} vs {wn.sum()})"
        print(f"  {name}: {gn.sum()} NaN, {((got & 0x7FFF) == 0x7F80).sum()} inf", flush=True)
        assert np.array_equal(got[~gn], want[~wn]), f"{name}: non-NaN values differ"
