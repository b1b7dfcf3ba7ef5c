"""GPU parity: the MoE expert GEMMs on the MX-scaled matrix cores (module
k3h_moe_gemm) against the C oracle, through the k3h C-ABI.

* Weight layouts (k3h_moe_w_tile / k3h_moe_sf_tile): bit-exact against a numpy
  restatement of the tiled layouts.
* Accumulators (GEMM_F32): |C_gpu - C| <= 2^-11 * sum_k |a_k w_k| per element
  against the float64 product.  The matrix cores do not round every partial sum
  to f32: the error of one 64-deep MFMA measured up to 2^-12.4 of its sum of
  magnitudes, so the bound covers one such step per element with margin, while a
  wrong scale, operand lane or K order costs O(1) of it.
* bf16 output (GEMM_BF16, fc2): bit-exact RNE of the same kernel's f32
  accumulators, and within the accumulator bound plus one bf16 rounding of C.
* fc1 (GEMM_SITU_MX): the oracle's epilogue (bf16 landing of up / gate, exact
  SiTU with the expert's alpha / beta, MX quantisation) applied to the kernel's
  own f32 accumulators: E8M0 scales and e4m3 codes identical except where the
  activation's one-ulp SiTU tolerance moves a value across a rounding boundary
  (fewer than 1e-3 of codes, by one code; fewer than 1e-3 of scales, by one).
Tiles past the live count, and tiles whose expert is out of range, are not
written."""
import numpy as np
import pytest
import torch

import oracle as O
from k3data import from_dev, normal_bf16, rng, to_dev

pytestmark = pytest.mark.gpu


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _tile_row(T, j, n, gated):
    if not gated:
        return 32 * T + j
    return (n // 2 if T & 1 else 0) + 32 * (T >> 1) + j


def _w_tile_np(w, n, k, gated):
    E = w.shape[0]
    NT, KT = n // 32, k // 64
    out = np.empty((E, NT, KT, 64, 16), np.uint8)
    l = np.arange(64)
    for T in range(NT):
        r = np.array([_tile_row(T, j, n, gated) for j in l % 32])
        for kt in range(KT):
            off = 32 * kt + 16 * (l // 32)
            idx = off[:, None] + np.arange(16)[None, :]
            out[:, T, kt] = w[:, r[:, None], idx]
    return out


def _sf_tile_np(wsf, n, k, gated):
    """[E][n/128][k/128][64 lanes][4 tiles][2]: tile T = 4 G + u, byte s = block 4 ks + 2 s + h."""
    E = wsf.shape[0]
    NG, KS = n // 128, k // 128
    out = np.empty((E, NG, KS, 64, 4, 2), np.uint8)
    l = np.arange(64)
    for G in range(NG):
        for u in range(4):
            r = np.array([_tile_row(4 * G + u, j, n, gated) for j in l % 32])
            for ks in range(KS):
                for s in range(2):
                    out[:, G, ks, :, u, s] = wsf[:, r, 4 * ks + 2 * s + l // 32]
    return out


def _inputs(seed, rows_src, E, N, K, wsf_range=(118, 134)):
    g = rng(seed)
    x = normal_bf16(g, (rows_src, K), outlier_p=0.01)
    q, sf = O.moe_quant(x, rows_src, K)
    w = g.integers(0, 256, (E, N, K // 2), dtype=np.uint8)
    wsf = g.integers(wsf_range[0], wsf_range[1], (E, N, K // 32)).astype(np.uint8)
    return g, q, sf, w, wsf


def _tiled(ctx, w, wsf, E, N, K, gated):
    dw, dsf = to_dev(w), to_dev(wsf)
    wt = torch.empty(w.size, dtype=torch.uint8, device="cuda")
    st = torch.empty(wsf.size, dtype=torch.uint8, device="cuda")
    ctx.moe_w_tile(dw, wt, E, N, K, gated)
    ctx.moe_sf_tile(dsf, st, E, N, K, gated)
    return wt, st


@pytest.mark.parametrize("gated", [0, 1])
def test_weight_tiles(ctx, gated):
    _case(f"w_tile / sf_tile gated={gated}")
    E, N, K = 3, 256, 512
    _, _, _, w, wsf = _inputs(7100 + gated, 8, E, N, K)
    wt, st = _tiled(ctx, w, wsf, E, N, K, gated)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(wt).reshape(-1), _w_tile_np(w, N, K, gated).reshape(-1))
    assert np.array_equal(from_dev(st).reshape(-1), _sf_tile_np(wsf, N, K, gated).reshape(-1))


def _run_f32(ctx, q, sf, rows, wt, st, cta, nt, max_tiles, E, N, K):
    out = torch.full((max_tiles * 128, N), float("nan"), dtype=torch.float32, device="cuda")
    d_rows = None if rows is None else to_dev(rows)
    ctx.moe_gemm_mx(ctx.GEMM_F32, to_dev(q), to_dev(sf), d_rows, wt, st,
                    to_dev(np.array([nt], np.int32)), to_dev(cta), max_tiles, E, N, K, out)
    torch.cuda.synchronize()
    return from_dev(out)


def _check_acc(got, q, sf, rows, w, wsf, cta, nt, E, N, K):
    ref = O.moe_gemm_mx(q, sf, rows, w, wsf, nt, cta, E, N, K)
    mag = O.moe_gemm_mx(q, sf, rows, w, wsf, nt, cta, E, N, K, magnitude=True)
    live = ~np.isnan(ref[:, 0])
    assert np.isnan(got[~np.concatenate([live, np.zeros(got.shape[0] - live.size, bool)])]).all()
    g, r, m = got[:live.size][live].astype(np.float64), ref[live], mag[live]
    ratio = np.abs(g - r) / np.maximum(m, 1e-300)
    print(f"  max |err| / sum|aw| = {ratio.max():.3g} (2^{np.log2(ratio.max() + 1e-300):.1f}), "
          f"median {np.median(ratio):.3g}", flush=True)
    assert ratio.max() <= 2.0 ** -11
    return ref, mag, live


# N % 512 == 0 and 256 <= K <= 3584 run the persistent 512-column 8-wave entry
# kern_k3h_moe_gemm2_f32 (one entry for every K, its step loop runs K / 128 steps
# with the stage index held at run time: K 256 / 384 / 512 start the next item in
# each of the three stage rotations, 3072 and 3584 are the fc2 / fc1 depths); the
# others the 256-column entries (K > 3584: the _w entries).
@pytest.mark.parametrize("E,N,K,gather", [(4, 512, 1024, True), (3, 256, 3584, False),
                                          (2, 768, 256, True), (2, 256, 7168, True),
                                          (2, 512, 3584, True), (3, 1024, 3072, False),
                                          (2, 512, 256, True), (2, 512, 384, False),
                                          (2, 1536, 512, True)])
def test_gemm_f32_accumulators(ctx, E, N, K, gather):
    _case(f"gemm f32 E={E} N={N} K={K} gather={gather}")
    rows_src = 700
    g, q, sf, w, wsf = _inputs(7200 + N + K, rows_src, E, N, K)
    cta = np.array([0, E - 1, 1 % E, E, 0, 0], np.int32)  # tile 3: expert out of range
    nt, max_tiles = 5, 6                                   # tile 5: past the live count
    if gather:
        rows = g.integers(0, rows_src, max_tiles * 128).astype(np.int32)
        qa, sfa = q, sf
    else:
        rows = None
        src = g.integers(0, rows_src, max_tiles * 128)
        qa, sfa = np.ascontiguousarray(q[src]), np.ascontiguousarray(sf[src])
    wt, st = _tiled(ctx, w, wsf, E, N, K, 0)
    got = _run_f32(ctx, qa, sfa, rows, wt, st, cta, nt, max_tiles, E, N, K)
    _check_acc(got, qa, sfa, rows, w, wsf, cta, nt, E, N, K)


@pytest.mark.parametrize("E,N,K", [(3, 512, 1024), (3, 1024, 3072), (3, 256, 1024)])
def test_gemm_bf16(ctx, E, N, K):
    _case(f"gemm bf16 (fc2 form) E={E} N={N} K={K}")
    g, q, sf, w, wsf = _inputs(7300 + N + K, 512, E, N, K)
    cta = np.array([2, 0, 1, 1], np.int32)
    nt = max_tiles = 4
    wt, st = _tiled(ctx, w, wsf, E, N, K, 0)
    acc = _run_f32(ctx, q, sf, None, wt, st, cta, nt, max_tiles, E, N, K)
    out = torch.zeros((max_tiles * 128, N), dtype=torch.bfloat16, device="cuda")
    ctx.moe_gemm_mx(ctx.GEMM_BF16, to_dev(q), to_dev(sf), None, wt, st,
                    to_dev(np.array([nt], np.int32)), to_dev(cta), max_tiles, E, N, K, out)
    torch.cuda.synchronize()
    got = from_dev(out)
    want = torch.from_numpy(acc).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    ref, mag, _ = _check_acc(acc, q, sf, None, w, wsf, cta, nt, E, N, K)
    gf = (got.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    assert (np.abs(gf - ref) <= 2.0 ** -11 * mag + 2.0 ** -8 * np.abs(ref)).all()


def _logical_to_raw(c, N):
    """Columns of a gated tiling (up, gate, up, gate, ... 32-wide tiles) -> [up | gate]."""
    out = np.empty_like(c)
    for T in range(N // 32):
        r = _tile_row(T, 0, N, 1)
        out[:, r:r + 32] = c[:, 32 * T:32 * T + 32]
    return out


@pytest.mark.parametrize("E,inter,K,ab", [(4, 256, 1024, (4.0, 25.0)), (2, 128, 3584, (4.0, 25.0)),
                                          (3, 384, 512, (3.0, 20.0)), (2, 256, 3584, (4.0, 25.0)),
                                          (2, 512, 384, (3.0, 20.0))])
def test_gemm_situ_mx(ctx, E, inter, K, ab):
    _case(f"gemm situ_mx (fc1 form) E={E} inter={inter} K={K} alpha,beta={ab}")
    N = 2 * inter
    rows_src = 600
    # weight scales near 2^-4 keep |C| in the range where SiTU is not saturated
    g, q, sf, w, wsf = _inputs(7400 + inter + K, rows_src, E, N, K, wsf_range=(121, 126))
    cta = np.array([1, 0, E - 1, 1], np.int32)
    nt, max_tiles = 3, 4
    rows = g.integers(0, rows_src, max_tiles * 128).astype(np.int32)
    wt, st = _tiled(ctx, w, wsf, E, N, K, 1)
    acc_logical = _run_f32(ctx, q, sf, rows, wt, st, cta, nt, max_tiles, E, N, K)
    alpha = np.full(E, ab[0], np.float32)
    beta = np.full(E, ab[1], np.float32)
    oq = torch.full((max_tiles * 128, inter), 0x5a, dtype=torch.uint8, device="cuda")
    osf = torch.full((max_tiles * 128, inter // 32), 0x5a, dtype=torch.uint8, device="cuda")
    ctx.moe_gemm_mx(ctx.GEMM_SITU_MX, to_dev(q), to_dev(sf), to_dev(rows), wt, st,
                    to_dev(np.array([nt], np.int32)), to_dev(cta), max_tiles, E, N, K, oq, osf,
                    to_dev(alpha), to_dev(beta))
    torch.cuda.synchronize()
    gq, gsf = from_dev(oq), from_dev(osf)
    live = nt * 128
    assert (gq[live:] == 0x5a).all() and (gsf[live:] == 0x5a).all()
    acc = _logical_to_raw(acc_logical[:live], N)
    # the accumulators themselves against the float64 product (weight-row order)
    ref = O.moe_gemm_mx(q, sf, rows, w, wsf, nt, cta, E, N, K)
    mag = O.moe_gemm_mx(q, sf, rows, w, wsf, nt, cta, E, N, K, magnitude=True)
    assert (np.abs(acc.astype(np.float64) - ref) <= 2.0 ** -11 * mag).all()
    e_rows = np.repeat(cta[:nt], 128)
    wq, wsf_ = O.moe_fc1_epilogue(acc, alpha[e_rows], beta[e_rows])
    sf_bad = gsf[:live] != wsf_
    print(f"  scales differing: {sf_bad.mean():.2e}", flush=True)
    assert sf_bad.mean() < 1e-3 and (np.abs(gsf[:live].astype(int) - wsf_.astype(int)) <= 1).all()
    same = np.repeat(~sf_bad, 32, axis=1)
    def order(c):  # e4m3 code -> monotone integer
        c = c.astype(np.int32)
        return np.where(c & 0x80, -(c & 0x7f), c & 0x7f)
    d = np.abs(order(gq[:live]) - order(wq))[same]
    print(f"  codes differing: {(d > 0).mean():.2e}, max {d.max()}", flush=True)
    assert d.max() <= 1 and (d > 0).mean() < 1e-3


def test_gemm_rejects_bad_shapes(ctx):
    z = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    i = torch.zeros(8, dtype=torch.int32, device="cuda")
    f = torch.zeros(1 << 16, dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError):  # N not a multiple of 256
        ctx.moe_gemm_mx(ctx.GEMM_F32, z, z, None, z, z, i, i, 1, 1, 128, 128, f)
    with pytest.raises(ValueError):  # K not a multiple of 128
        ctx.moe_gemm_mx(ctx.GEMM_F32, z, z, None, z, z, i, i, 1, 1, 256, 64, f)
    big = torch.zeros(1 << 21, dtype=torch.uint8, device="cuda")
    with pytest.raises(ValueError):  # K above the scale table's 7168
        ctx.moe_gemm_mx(ctx.GEMM_F32, big, big, None, big, big, i, i, 1, 1, 256, 7296, f)


def _grid_rows(max_tiles, nc):
    """Rows of the 4-wave kernels' grid (k3h_moe_gemm_mx's split coverage)."""
    need = max(8 * -(-max_tiles // (8 // xc)) * -(-nc // xc) for xc in (1, 2, 4, 8))
    return -(-need // nc)


@pytest.mark.parametrize("K", [256, 384, 1536, 3072, 3584])
def test_wide_items_match_4wave(ctx, K):
    """The persistent 512-column entries (kern_k3h_moe_gemm2_f32 / _bf16, which the
    typed calls take for N % 512 == 0 and K <= 3584) against the 4-wave entries
    launched directly and against the fc1 kernel's tiling (GEMM_F32_SITU_TILING),
    bit for bit, at K up to fc1's 3584, at a size where every workgroup runs several
    items back to back (the step pipeline crossing items) and some tiles have an
    out-of-range expert or lie past the live count.  The 4-wave entries are pinned
    against the oracle by the tests above."""
    import ctypes
    import k3h
    E, N, live, max_tiles = 6, 1024, 1100, 1120
    _case(f"wide vs 4-wave E={E} N={N} K={K} tiles={live}")
    g = rng(7700 + K)
    rows_src = 4096
    q = g.integers(0, 256, (rows_src, K), dtype=np.uint8)
    q[(q & 0x7f) == 0x7f] = 0x3c  # no NaN codes
    sf = g.integers(120, 130, (rows_src, K // 32)).astype(np.uint8)
    w = g.integers(0, 256, (E, N, K // 2), dtype=np.uint8)
    wsf = g.integers(118, 134, (E, N, K // 32)).astype(np.uint8)
    cta = np.sort(g.integers(0, E, max_tiles)).astype(np.int32)
    cta[g.integers(0, live, 40)] = E  # out-of-range experts (skipped items)
    rows = g.integers(-1, rows_src, max_tiles * 128).astype(np.int32)  # -1: padding rows
    wt, st = _tiled(ctx, w, wsf, E, N, K, 0)
    dq, dsf, dr, dcta = to_dev(q), to_dev(sf), to_dev(rows), to_dev(cta)
    nt = to_dev(np.array([live], np.int32))
    for ep, dt, fill, entry in ((ctx.GEMM_F32, torch.float32, float("nan"), "kern_k3h_moe_gemm_f32"),
                                (ctx.GEMM_BF16, torch.bfloat16, 0.0, "kern_k3h_moe_gemm_bf16")):
        got = torch.full((max_tiles * 128, N), fill, dtype=dt, device="cuda")
        ctx.moe_gemm_mx(ep, dq, dsf, dr, wt, st, nt, dcta, max_tiles, E, N, K, got)
        ref = torch.full_like(got, fill)
        args = k3h.pack_args(["buffer"] * 7 + ["i32"] * 4 + ["buffer"],
                             [dq, dsf, dr, wt, st, nt, dcta, E, N, K, max_tiles, ref])
        fn = ctx.function("k3h_moe_gemm", entry)
        grid = (ctypes.c_uint32 * 3)(N // 256, _grid_rows(max_tiles, N // 256), 1)
        block = (ctypes.c_uint32 * 3)(256, 1, 1)
        cbuf = ctypes.create_string_buffer(args, len(args))
        k3h._check(ctx.L.k3h_launch(fn, grid, block, 0, None, ctypes.cast(cbuf, ctypes.c_void_p),
                                    len(args)), entry)
        torch.cuda.synchronize()
        same = torch.equal(got.view(torch.uint8), ref.view(torch.uint8))
        print(f"  {entry}: identical = {same}", flush=True)
        assert same
        if ep == ctx.GEMM_F32:
            # the fc1 kernel's tiling (256-column items, swapped operand roles)
            fc1t = torch.full_like(got, fill)
            ctx.moe_gemm_mx(ctx.GEMM_F32_SITU_TILING, dq, dsf, dr, wt, st, nt, dcta, max_tiles, E, N,
                            K, fc1t)
            torch.cuda.synchronize()
            same = torch.equal(got.view(torch.uint8), fc1t.view(torch.uint8))
            print(f"  kern_k3h_moe_gemm_situ_acc: identical = {same}", flush=True)
            assert same
