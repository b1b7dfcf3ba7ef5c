"""GPU: the MoE block end to end on the routing kernels' own tables -- router
top-8, route count / tables / scatter (EP rank 0 of 4, strided experts), MX
quantisation of the latent rows, fc1 gathering its rows through route_map with
the SiTU-GLU + MXFP8 epilogue, fc2 with bf16 output, weighted finalize.

Every stage is checked against the oracle fed with the GPU's output of the
stage before it, so that a difference is attributed to the stage that made it:
the routing tables and the finalize bit-exact, the GEMM accumulators within
2^-11 of sum |a w| of the float64 product, fc1's codes / scales equal to the
oracle epilogue of the kernel's own accumulators, fc2's bf16 the RNE of its
accumulators."""
import numpy as np
import pytest
import torch

import oracle as O
from k3data import from_dev, normal_bf16, rng, to_bf16, to_dev

pytestmark = pytest.mark.gpu

T, TOPK, E, RANK = 384, 8, 56, 0
KL, INTER, COLS = 512, 256, 512


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _tile_row(T_, j, n):  # gated tile order: up, gate, up, gate, ...
    return (n // 2 if T_ & 1 else 0) + 32 * (T_ >> 1) + j


def test_moe_chain(ctx):
    _case(f"MoE chain T={T} top-{TOPK} E={E} K={KL} inter={INTER} cols={COLS}")
    g = rng(7700)
    S = g.standard_normal((T, 224), dtype=np.float32)
    bias = (g.standard_normal(224) * 0.01).astype(np.float32)
    rs = to_bf16(np.array([2.5], np.float32))
    idx = torch.empty((T, TOPK), dtype=torch.int32, device="cuda")
    wts = torch.empty((T, TOPK), dtype=torch.float32, device="cuda")
    ctx.router_topk(to_dev(S), to_dev(bias), to_dev(rs), idx, wts, T, topk=TOPK)

    nblk, cap = (T + 255) // 256, T * TOPK + E * 128
    max_tiles = cap // 128
    bc = torch.empty(nblk * E, dtype=torch.int32, device="cuda")
    bo = torch.empty_like(bc)
    cb = torch.full((max_tiles + 1,), -1, dtype=torch.int32, device="cuda")
    cl = torch.full_like(cb, -1)
    nne = torch.zeros(1, dtype=torch.int32, device="cuda")
    tp = torch.zeros(1, dtype=torch.int32, device="cuda")
    rmap = torch.full((cap,), -1, dtype=torch.int32, device="cuda")
    e2p = torch.empty(T * TOPK, dtype=torch.int32, device="cuda")
    ctx.moe_route_count(idx, T, RANK, E, bc, topk=TOPK)
    ctx.moe_route_tables(bc, nblk, E, 128, bo, cb, cl, nne, tp, rmap, T=T, topk=TOPK)
    ctx.moe_route_scatter(idx, bo, T, RANK, E, rmap, e2p, topk=TOPK)
    torch.cuda.synchronize()
    ids = from_dev(idx)
    tab = O.route_tables(O.route_count(ids, T, TOPK, RANK, E), nblk, E, 128, cap)
    want_rmap, want_e2p = O.route_scatter(ids, tab["blockoff"], T, TOPK, RANK, E, tab["route_map"])
    nt, tpad = int(nne[0]), int(tp[0])
    assert (nt, tpad) == (tab["num_non_exiting"], tab["total_padded"])
    assert np.array_equal(from_dev(rmap)[:tpad], want_rmap[:tpad])
    assert np.array_equal(from_dev(e2p), want_e2p)
    cta = from_dev(cb)
    assert np.array_equal(cta[:nt], tab["cta_batch"][:nt])
    print(f"  {nt} route tiles, {tpad} padded rows", flush=True)

    # latent rows -> MXFP8 on the GPU
    x = normal_bf16(g, (T, KL), outlier_p=0.01)
    aq = torch.empty((T, KL), dtype=torch.uint8, device="cuda")
    asf = torch.empty((T, KL // 32), dtype=torch.uint8, device="cuda")
    ctx.moe_quant(to_dev(x), aq, asf, T, KL)

    # expert weights, row-major e2m1 + E8M0, tiled on the GPU
    w13 = g.integers(0, 256, (E, 2 * INTER, KL // 2), dtype=np.uint8)
    s13 = g.integers(121, 126, (E, 2 * INTER, KL // 32)).astype(np.uint8)
    w2 = g.integers(0, 256, (E, COLS, INTER // 2), dtype=np.uint8)
    s2 = g.integers(121, 126, (E, COLS, INTER // 32)).astype(np.uint8)

    def tiled(w, s, n, k, gated):
        wt = torch.empty(w.size, dtype=torch.uint8, device="cuda")
        st = torch.empty(s.size, dtype=torch.uint8, device="cuda")
        ctx.moe_w_tile(to_dev(w), wt, E, n, k, gated)
        ctx.moe_sf_tile(to_dev(s), st, E, n, k, gated)
        return wt, st
    w13t, s13t = tiled(w13, s13, 2 * INTER, KL, 1)
    w2t, s2t = tiled(w2, s2, COLS, INTER, 0)
    alpha = torch.full((E,), 4.0, device="cuda")
    beta = torch.full((E,), 25.0, device="cuda")
    rows = max_tiles * 128

    # fc1: accumulators, then the fused SiTU-GLU + MXFP8 epilogue
    acc1 = torch.full((rows, 2 * INTER), float("nan"), device="cuda")
    ctx.moe_gemm_mx(ctx.GEMM_F32, aq, asf, rmap, w13t, s13t, nne, cb, max_tiles, E, 2 * INTER, KL,
                    acc1)
    q1 = torch.empty((rows, INTER), dtype=torch.uint8, device="cuda")
    sf1 = torch.empty((rows, INTER // 32), dtype=torch.uint8, device="cuda")
    ctx.moe_gemm_mx(ctx.GEMM_SITU_MX, aq, asf, rmap, w13t, s13t, nne, cb, max_tiles, E, 2 * INTER,
                    KL, q1, sf1, alpha, beta)
    torch.cuda.synchronize()
    live = nt * 128
    a1 = from_dev(acc1)[:live]
    raw = np.empty_like(a1)
    for Tt in range(2 * INTER // 32):
        r0 = _tile_row(Tt, 0, 2 * INTER)
        raw[:, r0:r0 + 32] = a1[:, 32 * Tt:32 * Tt + 32]
    rm = from_dev(rmap)
    ref = O.moe_gemm_mx(from_dev(aq), from_dev(asf), rm, w13, s13, nt, cta[:nt], E, 2 * INTER, KL)
    mag = O.moe_gemm_mx(from_dev(aq), from_dev(asf), rm, w13, s13, nt, cta[:nt], E, 2 * INTER, KL,
                        magnitude=True)
    assert (np.abs(raw.astype(np.float64) - ref) <= 2.0 ** -11 * mag).all(), "fc1 accumulators"
    eq, esf = O.moe_fc1_epilogue(raw, np.full(live, 4.0), np.full(live, 25.0))
    gq, gsf = from_dev(q1)[:live], from_dev(sf1)[:live]
    sf_bad = gsf != esf  # the SiTU's one-ulp tolerance may move a block max across a power of 2
    assert sf_bad.mean() < 1e-3 and (np.abs(gsf.astype(int) - esf.astype(int)) <= 1).all()
    order = lambda c: np.where(c & 0x80, -(c.astype(np.int32) & 0x7f), c.astype(np.int32) & 0x7f)
    d = np.abs(order(gq) - order(eq))[np.repeat(~sf_bad, 32, axis=1)]
    print(f"  fc1: scales differing {sf_bad.mean():.2e}, codes differing {(d > 0).mean():.2e}", flush=True)
    assert d.max() <= 1 and (d > 0).mean() < 1e-3, "fc1 e4m3 codes"

    # fc2 on fc1's output rows
    acc2 = torch.full((rows, COLS), float("nan"), device="cuda")
    ctx.moe_gemm_mx(ctx.GEMM_F32, q1, sf1, None, w2t, s2t, nne, cb, max_tiles, E, COLS, INTER, acc2)
    o2 = torch.empty((rows, COLS), dtype=torch.bfloat16, device="cuda")
    ctx.moe_gemm_mx(ctx.GEMM_BF16, q1, sf1, None, w2t, s2t, nne, cb, max_tiles, E, COLS, INTER, o2)
    torch.cuda.synchronize()
    a2 = from_dev(acc2)[:live]
    ref2 = O.moe_gemm_mx(from_dev(q1), from_dev(sf1), None, w2, s2, nt, cta[:nt], E, COLS, INTER)
    mag2 = O.moe_gemm_mx(from_dev(q1), from_dev(sf1), None, w2, s2, nt, cta[:nt], E, COLS, INTER,
                         magnitude=True)
    assert (np.abs(a2.astype(np.float64) - ref2) <= 2.0 ** -11 * mag2).all(), "fc2 accumulators"
    b2 = from_dev(o2)[:live]
    want_b2 = torch.from_numpy(a2).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(b2, want_b2), "fc2 bf16"

    # weighted finalize of the local experts' rows
    out = torch.empty((T, COLS), dtype=torch.bfloat16, device="cuda")
    ctx.moe_finalize(o2, e2p, wts, out, T, COLS, topk=TOPK)
    torch.cuda.synchronize()
    want = O.moe_finalize(from_dev(o2)[:tpad], from_dev(e2p), from_dev(wts), T, TOPK, COLS)
    assert np.array_equal(from_dev(out), want), "finalize"
