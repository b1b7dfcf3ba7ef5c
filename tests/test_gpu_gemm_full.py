"""GPU parity of the MoE expert GEMMs at the shape they are benchmarked at: the
reference's moe_fc1 / moe_fc2 (manifest ops 405185 / 405419; kernels.toml:1-9)
with 56 local experts, latent K 3584, intermediate 3072, output columns 3584,
over the top-8 routing of 16,384 tokens for EP rank 0 of 4 (about 279 route
tiles, 35k padded rows).  At this size the kernel's per-XCD split of (tile,
column block) items covers every XCD and the weights span 616 MB, which the
small-shape tests do not reach.

The GPU runs every tile.  Checked:

* on every live row: the shipped fc1 kernel's own tiling (256-column items,
  swapped operand roles, its per-XCD item split; GEMM_F32_SITU_TILING) gives
  accumulators bit-identical to the persistent 512-column f32 kernel;
* on every live row: fc1's e4m3 codes and E8M0 scales (GEMM_SITU_MX) equal the
  oracle's epilogue applied to those accumulators, up to the SiTU's one-ulp
  tolerance (fewer than 1e-3 of codes / scales off, by one);
* on a fixed sample of 16 whole route tiles (2048 padded rows, padding rows
  included) spread evenly over the live tiles -- so over all tile quarters of
  the per-XCD split -- and every column of those rows: fc1 and fc2 accumulators
  (GEMM_F32) within 2^-11 * sum_k |a_k w_k| of the float64 product (the bound of
  tests/test_gpu_gemm.py: one 64-deep MFMA step measured up to 2^-12.4 of its
  sum of magnitudes);
* on every live row: fc2's bf16 output equal to the RNE of the same kernel's f32
  accumulators (compared on the GPU: torch's f32 -> bf16 cast is RNE).

Routing comes from the oracle's router and tables on the host (the GPU routing
kernels have their own bit-exact tests); fc2 reads fc1's GPU output in place,
as in the bench."""
import numpy as np
import pytest
import torch

import oracle as O
from k3data import from_dev, rng, to_bf16, to_dev

pytestmark = pytest.mark.gpu

T, TOPK, E, RANK = 16384, 8, 56, 0
KL, INTER, COLS = 3584, 3072, 3584
SAMPLE = 16


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _tile_row(t, j, n):  # gated tile order: up, gate, up, gate, ...
    return (n // 2 if t & 1 else 0) + 32 * (t >> 1) + j


def _logical_to_raw(c, n):
    out = np.empty_like(c)
    for t in range(n // 32):
        r = _tile_row(t, 0, n)
        out[:, r:r + 32] = c[:, 32 * t:32 * t + 32]
    return out


def _acc_ok(name, got, ref, mag):
    ratio = np.abs(got.astype(np.float64) - ref) / np.maximum(mag, 1e-300)
    print(f"  {name}: max |err| / sum|aw| = 2^{np.log2(ratio.max() + 1e-300):.1f}, "
          f"median {np.median(ratio):.3g}", flush=True)
    assert ratio.max() <= 2.0 ** -11, name


def _bytes(g, n):
    """n uniform random bytes (the generator's raw 64-bit outputs)."""
    return g.bit_generator.random_raw(-(-n // 8)).view(np.uint8)[:n]


def _weights(g, n, k, sf_lo, sf_hi):
    """Uniform e2m1 byte pairs; E8M0 scales uniform over [sf_lo, sf_hi)."""
    w = _bytes(g, E * n * k // 2).reshape(E, n, k // 2)
    r = _bytes(g, E * n * k // 32).reshape(E, n, k // 32)
    wsf = (sf_lo + r % (sf_hi - sf_lo)).astype(np.uint8)
    return w, wsf


def _tiled(ctx, w, wsf, n, k, gated):
    wt = torch.empty(w.size, dtype=torch.uint8, device="cuda")
    st = torch.empty(wsf.size, dtype=torch.uint8, device="cuda")
    ctx.moe_w_tile(to_dev(w), wt, E, n, k, gated)
    ctx.moe_sf_tile(to_dev(wsf), st, E, n, k, gated)
    return wt, st


def test_moe_gemm_bench_shape(ctx):
    _case(f"MoE fc1/fc2 at T={T} top-{TOPK} E={E} K={KL} inter={INTER} cols={COLS}")
    g = rng(7900)
    S = g.standard_normal((T, 224), dtype=np.float32)
    bias = (g.standard_normal(224) * 0.01).astype(np.float32)
    rs = int(to_bf16(np.array([2.5], np.float32))[0])
    ids, _ = O.router_topk(S, bias, rs, T, TOPK)
    nblk, cap = (T + 255) // 256, T * TOPK + E * 128
    tab = O.route_tables(O.route_count(ids, T, TOPK, RANK, E), nblk, E, 128, cap)
    rmap, _ = O.route_scatter(ids, tab["blockoff"], T, TOPK, RANK, E, tab["route_map"])
    nt, max_tiles = tab["num_non_exiting"], cap // 128
    cta = tab["cta_batch"][:max_tiles].copy()
    print(f"  live tiles {nt}, padded rows {tab['total_padded']}", flush=True)
    assert 250 < nt <= max_tiles and (rmap[:nt * 128] >= 0).all()
    sel = np.unique(np.linspace(0, nt - 1, SAMPLE).round().astype(np.int64))
    assert sel.size == SAMPLE
    rows_sel = np.concatenate([np.arange(128 * t, 128 * t + 128) for t in sel])
    cta_sel = np.ascontiguousarray(cta[sel])
    d_rmap, d_cta = to_dev(rmap[:max_tiles * 128]), to_dev(cta)
    d_nt = to_dev(np.array([nt], np.int32))
    d_sel = torch.from_numpy(rows_sel).cuda()

    # latent rows ~N(0,1) quantised on the GPU (moe_quant has its own bit-exact
    # tests); the oracle's product takes the same codes and scales
    tg = torch.Generator(device="cuda")
    tg.manual_seed(7901)
    lat = torch.randn((T, KL), generator=tg, device="cuda").to(torch.bfloat16)
    d_aq = torch.empty((T, KL), dtype=torch.uint8, device="cuda")
    d_asf = torch.empty((T, KL // 32), dtype=torch.uint8, device="cuda")
    ctx.moe_quant(lat, d_aq, d_asf, T, KL)
    del lat
    aq, asf = from_dev(d_aq), from_dev(d_asf)
    # weight scales near 2^-4 keep fc1's outputs where the SiTU is not saturated
    w13, s13 = _weights(g, 2 * INTER, KL, 121, 126)
    w2, s2 = _weights(g, COLS, INTER, 118, 134)
    w13t, s13t = _tiled(ctx, w13, s13, 2 * INTER, KL, 1)
    w2t, s2t = _tiled(ctx, w2, s2, COLS, INTER, 0)

    # ---- fc1: accumulators, then the SiTU-GLU + MXFP8 epilogue
    live = nt * 128
    _case("fc1 accumulators (GEMM_F32, rows through route_map)")
    acc1 = torch.empty((max_tiles * 128, 2 * INTER), dtype=torch.float32, device="cuda")
    ctx.moe_gemm_mx(ctx.GEMM_F32, d_aq, d_asf, d_rmap, w13t, s13t, d_nt, d_cta, max_tiles, E,
                    2 * INTER, KL, acc1)
    _case("fc1 accumulators of the fc1 kernel's own tiling (GEMM_F32_SITU_TILING), every live row")
    acc1t = torch.empty((max_tiles * 128, 2 * INTER), dtype=torch.float32, device="cuda")
    ctx.moe_gemm_mx(ctx.GEMM_F32_SITU_TILING, d_aq, d_asf, d_rmap, w13t, s13t, d_nt, d_cta,
                    max_tiles, E, 2 * INTER, KL, acc1t)
    torch.cuda.synchronize()
    n_diff = int((acc1[:live].view(torch.int32) != acc1t[:live].view(torch.int32)).sum().item())
    print(f"  fc1 tiling vs persistent f32 kernel: {n_diff} of {live * 2 * INTER} differ", flush=True)
    assert n_diff == 0
    acc1_s = _logical_to_raw(from_dev(acc1[d_sel]), 2 * INTER)
    del acc1
    src1 = np.ascontiguousarray(rmap[rows_sel])
    ref1 = O.moe_gemm_mx(aq, asf, src1, w13, s13, SAMPLE, cta_sel, E, 2 * INTER, KL)
    mag1 = O.moe_gemm_mx(aq, asf, src1, w13, s13, SAMPLE, cta_sel, E, 2 * INTER, KL, magnitude=True)
    _acc_ok("fc1", acc1_s, ref1, mag1)
    del ref1, mag1, acc1_s

    _case("fc1 epilogue (GEMM_SITU_MX), every live row")
    alpha = torch.full((E,), 4.0, device="cuda")
    beta = torch.full((E,), 25.0, device="cuda")
    o1 = torch.empty((max_tiles * 128, INTER), dtype=torch.uint8, device="cuda")
    o1sf = torch.empty((max_tiles * 128, INTER // 32), dtype=torch.uint8, device="cuda")
    ctx.moe_gemm_mx(ctx.GEMM_SITU_MX, d_aq, d_asf, d_rmap, w13t, s13t, d_nt, d_cta, max_tiles, E,
                    2 * INTER, KL, o1, o1sf, alpha, beta)
    torch.cuda.synchronize()
    del w13t, s13t

    def order(c):  # e4m3 code -> monotone integer
        c = c.astype(np.int32)
        return np.where(c & 0x80, -(c & 0x7f), c & 0x7f)
    # the oracle's epilogue of the fc1 kernel's own accumulators, in row chunks
    n_sf = n_code = n_sf_bad = n_code_bad = 0
    for r0 in range(0, live, 8192):
        r1 = min(live, r0 + 8192)
        acc = _logical_to_raw(from_dev(acc1t[r0:r1]), 2 * INTER)
        wq, wsf_ = O.moe_fc1_epilogue(acc, np.full(r1 - r0, 4.0, np.float32),
                                      np.full(r1 - r0, 25.0, np.float32))
        gq, gsf = from_dev(o1[r0:r1]), from_dev(o1sf[r0:r1])
        sf_bad = gsf != wsf_
        assert (np.abs(gsf.astype(int) - wsf_.astype(int)) <= 1).all()
        same = np.repeat(~sf_bad, 32, axis=1)
        d = np.abs(order(gq) - order(wq))[same]
        assert d.size == 0 or d.max() <= 1
        n_sf, n_sf_bad = n_sf + sf_bad.size, n_sf_bad + int(sf_bad.sum())
        n_code, n_code_bad = n_code + d.size, n_code_bad + int((d > 0).sum())
    del acc1t
    print(f"  fc1 over {live} rows: scales differing {n_sf_bad / n_sf:.2e}, "
          f"codes differing {n_code_bad / max(n_code, 1):.2e}", flush=True)
    assert n_sf_bad / n_sf < 1e-3 and n_code_bad / max(n_code, 1) < 1e-3

    # ---- fc2 over fc1's GPU output, read in place
    _case("fc2 accumulators (GEMM_F32, fc1 output in place)")
    acc2 = torch.empty((max_tiles * 128, COLS), dtype=torch.float32, device="cuda")
    ctx.moe_gemm_mx(ctx.GEMM_F32, o1, o1sf, None, w2t, s2t, d_nt, d_cta, max_tiles, E, COLS, INTER,
                    acc2)
    _case("fc2 bf16 output (GEMM_BF16)")
    out2 = torch.empty((max_tiles * 128, COLS), dtype=torch.bfloat16, device="cuda")
    ctx.moe_gemm_mx(ctx.GEMM_BF16, o1, o1sf, None, w2t, s2t, d_nt, d_cta, max_tiles, E, COLS, INTER,
                    out2)
    torch.cuda.synchronize()
    live = nt * 128
    rne = acc2[:live].to(torch.bfloat16).view(torch.int16)
    n_diff = int((rne != out2[:live].view(torch.int16)).sum().item())
    print(f"  fc2 bf16 vs RNE of its accumulators: {n_diff} of {live * COLS} differ", flush=True)
    assert n_diff == 0
    acc2_s = from_dev(acc2[d_sel])
    del acc2, out2
    a2 = from_dev(o1[d_sel])
    a2sf = from_dev(o1sf[d_sel])
    ref2 = O.moe_gemm_mx(a2, a2sf, None, w2, s2, SAMPLE, cta_sel, E, COLS, INTER)
    mag2 = O.moe_gemm_mx(a2, a2sf, None, w2, s2, SAMPLE, cta_sel, E, COLS, INTER, magnitude=True)
    _acc_ok("fc2", acc2_s, ref2, mag2)
