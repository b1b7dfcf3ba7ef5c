"""Pins the router / argmax / EP-routing / finalize oracles with independent
methods: top-k by a full stable sort, argmax by numpy, routing tables by their
invariants (bijection, stable per-expert order, tile padding), finalize
against float64 sums."""
import numpy as np
import pytest

import oracle as O
from k3data import bf16_to_f32, normal_bf16, rng, to_bf16


def _ord(f32):
    b = f32.astype(np.float32).view(np.uint32)
    return np.where(b & 0x80000000, ~b, b | 0x80000000).astype(np.uint64)


@pytest.mark.parametrize("topk", [8, 16])
def test_router_topk_equals_full_stable_sort(topk):
    g = rng(70 + topk)
    B = 256
    S = g.standard_normal((B, 224), dtype=np.float32)
    S[0, 10:20] = S[0, 5]            # ties: equal sig and bias -> smallest e first
    bias = (g.standard_normal(224) * 0.01).astype(np.float32)
    bias[10:20] = bias[5]
    rs = to_bf16(np.array([2.5], np.float32))[0]
    idx, wts = O.router_topk(S, bias, rs, B, topk)
    sig = O.sigmoid(S)
    key = _ord((sig + bias).astype(np.float32))
    for b in range(B):
        order = np.lexsort((np.arange(224), -key[b].astype(np.int64)))  # key desc, then e asc
        assert np.array_equal(idx[b], order[:topk]), b
    # weights: renormalised selected sigmoids times rs (float64 reference, 2 f32 ulp)
    ps = np.take_along_axis(sig, idx, 1).astype(np.float64)
    want = ps / ps.sum(1, keepdims=True) * 2.5
    assert np.all(np.abs(wts - want) <= 2 * np.spacing(np.abs(want).astype(np.float32)))


def test_sigmoid_close_to_float64():
    x = np.linspace(-30, 30, 200001, dtype=np.float32)
    got = O.sigmoid(x).astype(np.float64)
    want = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.all(np.abs(got - want) <= 3 * np.spacing(want.astype(np.float32)))


def test_argmax_two_stage_matches_numpy():
    g = rng(80)
    B, n, parts = 8, 5000, 64
    x = g.standard_normal((B, n), dtype=np.float32)
    x[1, 100] = x[1, 4000] = 9.0     # tie: smallest index wins
    x[2, :] = -np.inf                 # all -inf: index 0
    pmax, pidx = O.argmax_partial(x, B, n, parts)
    out = O.argmax_final(pmax, pidx, B, parts)
    assert np.array_equal(out, np.argmax(x, axis=1))
    # empty chunks of a short row carry the neutral element
    pm2, pi2 = O.argmax_partial(x[:, :10], B, 10, parts)
    assert np.all(pi2.reshape(B, parts)[:, 10:] == 0x7fffffff)


def _route(T, topk, E=56, rank=0, seed=90):
    g = rng(seed)
    S = g.standard_normal((T, 224), dtype=np.float32)
    bias = (g.standard_normal(224) * 0.01).astype(np.float32)
    ids, _ = O.router_topk(S, bias, to_bf16(np.array([2.5], np.float32))[0], T, topk)
    nblk = (T + 255) // 256
    bc = O.route_count(ids, T, topk, rank, E)
    cap = T * topk + E * 128
    tab = O.route_tables(bc, nblk, E, 128, cap)
    rmap, e2p = O.route_scatter(ids, tab["blockoff"], T, topk, rank, E, tab["route_map"])
    return ids, bc, tab, rmap, e2p


@pytest.mark.parametrize("T,topk", [(1000, 8), (4096, 16), (300, 16)])
def test_routing_invariants(T, topk):
    E, rank = 56, 0
    ids, bc, tab, rmap, e2p = _route(T, topk, E, rank)
    loc = np.where(ids % 4 == rank, ids // 4, -1)
    loc[loc >= E] = -1
    count = np.bincount(loc[loc >= 0], minlength=E)
    # counts per 256-token block
    for b in range((T + 255) // 256):
        blk = loc[256 * b:256 * (b + 1)]
        assert np.array_equal(bc[b * E:(b + 1) * E], np.bincount(blk[blk >= 0], minlength=E))
    ctas = -(-count // 128)
    off = np.concatenate([[0], np.cumsum(ctas)])
    assert tab["num_non_exiting"] == off[-1] and tab["total_padded"] == 128 * off[-1]
    tp = tab["total_padded"]
    e2p = e2p.reshape(T, topk)
    # exp2perm: -1 exactly for non-local slots, a bijection onto the real rows
    assert np.array_equal(e2p < 0, loc < 0)
    rows = e2p[e2p >= 0]
    assert len(np.unique(rows)) == rows.size == count.sum()
    real = np.zeros(tp, bool)
    real[rows] = True
    for e in range(E):
        lo = 128 * off[e]
        seg = np.arange(lo, lo + count[e])
        assert real[seg].all() and not real[lo + count[e]:128 * off[e + 1]].any()
        # stable: rows of expert e in ascending expanded-index order
        te = np.argwhere(loc == e)
        want_rows = lo + np.arange(len(te))
        assert np.array_equal(e2p[te[:, 0], te[:, 1]], want_rows)
    # route_map: the token of every real row, token 0 on padding rows
    tt = np.nonzero(e2p >= 0)[0]
    assert np.array_equal(rmap[e2p[e2p >= 0]], tt)
    assert np.all(rmap[:tp][~real] == 0)
    # CTA tables
    nne = tab["num_non_exiting"]
    for i in range(nne):
        j = int(np.searchsorted(off, i, side="right") - 1)
        assert tab["cta_batch"][i] == j
        assert tab["cta_limit"][i] == min(128 * (i + 1), 128 * off[j] + count[j])


def test_finalize_against_float64():
    T, topk, cols = 512, 8, 7168
    ids, bc, tab, rmap, e2p = _route(T, topk, seed=91)
    g = rng(92)
    wts = g.random((T, topk), dtype=np.float32)
    fc2 = normal_bf16(g, (tab["total_padded"], cols))
    out = O.moe_finalize(fc2, e2p, wts, T, topk, cols)
    e2p = e2p.reshape(T, topk)
    f = bf16_to_f32(fc2).astype(np.float64)
    want = np.zeros((T, cols))
    mag = np.zeros((T, cols))
    for k in range(topk):
        m = e2p[:, k] >= 0
        want[m] += wts[m, k, None].astype(np.float64) * f[e2p[m, k]]
        mag[m] += np.abs(wts[m, k, None].astype(np.float64) * f[e2p[m, k]])
    got = bf16_to_f32(out).astype(np.float64)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 1e-38))) - 7)
    # one bf16 rounding of the result plus the f32 rounding of <= topk fma terms
    assert np.all(np.abs(got - want) <= ulp + topk * 2.0**-23 * mag)
    assert not out[(e2p < 0).all(1)].any()  # tokens with no local slot: zeros


def test_permute_and_shuffles():
    T, topk, cols = 700, 8, 7168
    ids, bc, tab, rmap, e2p = _route(T, topk, seed=93)
    g = rng(94)
    q = g.integers(0, 256, (T, cols), dtype=np.uint8)
    sf = g.integers(0, 256, (T, cols // 32), dtype=np.uint8)
    tp = tab["total_padded"]
    pq, psf = O.moe_permute_mx(q, sf, rmap[:tp], tp, cols)
    assert np.array_equal(pq, q[rmap[:tp]]) and np.array_equal(psf, sf[rmap[:tp]])
    # weight shuffle: a permutation of the rows inside every 32-row group
    n, rb = 256, 32
    src = np.repeat(np.arange(2 * n, dtype=np.uint16), rb // 2).view(np.uint8).reshape(2 * n, rb)
    for gated in (0, 1):
        dst = O.moe_w_shuffle(np.ascontiguousarray(src), 2, n, rb, gated)
        taken = dst.view(np.uint16)[:, 0].reshape(2, n) - np.arange(2)[:, None] * n
        assert sorted(taken[0].tolist()) == list(range(n))
        if not gated:
            assert taken[0, 1] == 4 and taken[0, 8] == 1 and taken[0, 32 + 9] == 32 + 5
        else:
            # r=1 -> u=4 (even) -> 2;  r=8 -> u=1 (odd) -> n/2 + 0
            assert taken[0, 1] == 2 and taken[0, 8] == n // 2 and taken[0, 0] == 0
    kg = 8
    s2 = g.integers(0, 256, (2 * n * kg,), dtype=np.uint8)
    d2 = O.moe_sf_shuffle(s2, 2, n, kg, 0)
    assert sorted(d2.tolist()) == sorted(s2.tolist())


@pytest.mark.parametrize("gated", [0, 1])
def test_sf_shuffle_byte_placement(gated):
    """kern_k3_moe_sf_shuffle's destination layout (k3_moe_prefill_v4.cu:320-327),
    restated by reshapes instead of the oracle's index formula: the scale rows
    first take the weight shuffle's row order (read off the separately pinned
    moe_w_shuffle), then every 128-row block x 4-column group forms one 512-byte
    unit ordered [row % 32][(row % 128) / 32][column % 4]."""
    E, n, kg = 2, 256, 12
    g = rng(77 + gated)
    src = g.integers(0, 256, (E, n, kg), dtype=np.uint8)
    # the row each destination row reads, from moe_w_shuffle over tagged rows
    tags = np.repeat(np.arange(E * n, dtype=np.uint16), 8).view(np.uint8).reshape(E * n, 16)
    perm = O.moe_w_shuffle(np.ascontiguousarray(tags), E, n, 16, gated).view(np.uint16)[:, 0]
    perm = perm.reshape(E, n) - (np.arange(E) * n)[:, None]
    rows = np.take_along_axis(src, perm[:, :, None].astype(np.int64), axis=1)   # [E, n, kg]
    want = rows.reshape(E, n // 128, 4, 32, kg // 4, 4).transpose(0, 1, 4, 3, 2, 5).reshape(E, -1)
    got = O.moe_sf_shuffle(np.ascontiguousarray(src.reshape(-1)), E, n, kg, gated).reshape(E, -1)
    assert np.array_equal(got, want)
