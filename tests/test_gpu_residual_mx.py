"""GPU parity: K1 residual family, MXFP8 quant and the fused residual + RMSNorm
+ MXFP8 op against the C oracle, through the k3h C-ABI.  Bar: bit-exact for
every output (prefix2/hidden/blocks by construction; normed because kernel and
oracle share the reduction order and a correctly rounded 1/sqrt; q/sf because
the MX rule is exact)."""
import json
import os

import numpy as np
import pytest
import torch

import k3h
import oracle as O
from k3data import H, bf16_to_f32, from_dev, normal_bf16, rng, to_bf16, to_dev

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _eq(name, got, want):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (name, got.shape, want.shape)
    bad = np.flatnonzero(got.ravel() != want.ravel())
    assert bad.size == 0, f"{name}: {bad.size} of {got.size} differ, first at {bad[:5]}"


def _k1_inputs(seed, B, land="bf16"):
    g = rng(seed)
    prefix = normal_bf16(g, (B, H))
    partial = normal_bf16(g, (B, H)) if land == "bf16" else g.standard_normal((B, H), dtype=np.float32)
    blocks = normal_bf16(g, (B, 8, H), 0.0, 2.0)
    sw = g.standard_normal(H, dtype=np.float32) * np.float32(0.05)
    gamma = normal_bf16(g, (H,), 1.0, 0.1)
    return prefix, partial, blocks, sw, gamma


@pytest.mark.parametrize("eps", [1e-6, 1e-5])
def test_k1b_config1_nb0(ctx, eps):
    """Config 1: tokens 1024, hidden 7168, plain residual add + RMSNorm."""
    B = 1024
    _case(f"k1b nb0 B={B} eps={eps}")
    prefix, partial, blocks, sw, gamma = _k1_inputs(100, B)
    want_p2, want_n = O.land_add_attnres_rms(partial, prefix, None, None, gamma, 0, 0, B, eps)
    d = {k: to_dev(v) for k, v in dict(prefix=prefix, partial=partial, blocks=blocks, gamma=gamma).items()}
    sw_d = to_dev(sw)
    p2 = torch.empty((B, H), dtype=torch.bfloat16, device="cuda")
    nrm = torch.empty_like(p2)
    ctx.land_add_attnres_rms(d["partial"], d["prefix"], d["blocks"], sw_d, d["gamma"], p2, nrm, 0, 0, B, eps)
    torch.cuda.synchronize()
    _eq("prefix2", from_dev(p2), want_p2)
    _eq("normed", from_dev(nrm), want_n)


@pytest.mark.parametrize("land", ["bf16", "f32"])
@pytest.mark.parametrize("nb,snapshot", [(0, 1), (1, 0), (2, 0), (3, 1), (5, 0), (8, 0), (8, 1)])
def test_k1b_mixing(ctx, land, nb, snapshot):
    B = 24
    _case(f"k1b land={land} nb={nb} snapshot={snapshot}")
    prefix, partial, blocks, sw, gamma = _k1_inputs(200 + nb, B, land)
    want_p2, want_n = O.land_add_attnres_rms(partial, prefix, blocks, sw, gamma, nb, snapshot, B)
    p2 = torch.empty((B, H), dtype=torch.bfloat16, device="cuda")
    nrm = torch.empty_like(p2)
    ctx.land_add_attnres_rms(to_dev(partial), to_dev(prefix), to_dev(blocks), to_dev(sw),
                             to_dev(gamma), p2, nrm, nb, snapshot, B)
    torch.cuda.synchronize()
    _eq("prefix2", from_dev(p2), want_p2)
    _eq("normed", from_dev(nrm), want_n)


@pytest.mark.parametrize("nb", range(1, 9))
@pytest.mark.parametrize("snapshot", [0, 1])
def test_k1b_per_nb_entries(ctx, nb, snapshot):
    """The typed nb entries (vector-split body) against the oracle; with snapshot
    the prefix row is not read and prefix2 is the landed partial."""
    B = 12
    _case(f"k1b_nb{nb} snapshot={snapshot}")
    prefix, partial, blocks, sw, gamma = _k1_inputs(300 + nb, B)
    want_p2, want_n = O.land_add_attnres_rms(partial, prefix, blocks, sw, gamma, nb, snapshot, B)
    p2 = torch.empty((B, H), dtype=torch.bfloat16, device="cuda")
    nrm = torch.empty_like(p2)
    ctx.land_add_attnres_rms_nb(to_dev(partial), to_dev(prefix), to_dev(blocks), to_dev(sw),
                                to_dev(gamma), p2, nrm, nb, snapshot, B)
    torch.cuda.synchronize()
    _eq("prefix2", from_dev(p2), want_p2)
    _eq("normed", from_dev(nrm), want_n)


@pytest.mark.parametrize("nb", [4, 8])
def test_k1b_per_nb_full_rank_share(ctx, nb):
    """The typed nb entry at the benchmarked shape (B = 4096 rows of one rank's
    16k-prefill share), every row bit-exact."""
    B = 4096
    _case(f"k1b_nb{nb} at B={B}")
    prefix, partial, blocks, sw, gamma = _k1_inputs(320 + nb, B)
    want_p2, want_n = O.land_add_attnres_rms(partial, prefix, blocks, sw, gamma, nb, 0, B)
    p2 = torch.empty((B, H), dtype=torch.bfloat16, device="cuda")
    nrm = torch.empty_like(p2)
    ctx.land_add_attnres_rms_nb(to_dev(partial), to_dev(prefix), to_dev(blocks), to_dev(sw),
                                to_dev(gamma), p2, nrm, nb, 0, B)
    torch.cuda.synchronize()
    _eq("prefix2", from_dev(p2), want_p2)
    _eq("normed", from_dev(nrm), want_n)


@pytest.mark.parametrize("nb,snapshot", [(0, 0), (0, 1), (3, 1), (7, 1), (8, 1), (4, 0)])
def test_k1a_attnres_rms(ctx, nb, snapshot):
    B = 10
    _case(f"k1a nb={nb} snapshot={snapshot}")
    prefix, _, blocks, sw, gamma = _k1_inputs(400 + nb, B)
    want_blk, want_n = O.attnres_rms(prefix, blocks, sw, gamma, nb, snapshot, B)
    blk_d = to_dev(blocks)
    nrm = torch.empty((B, H), dtype=torch.bfloat16, device="cuda")
    ctx.attnres_rms(to_dev(prefix), blk_d, to_dev(sw), to_dev(gamma), nrm, nb, snapshot, B)
    torch.cuda.synchronize()
    _eq("blocks", from_dev(blk_d), want_blk)
    _eq("normed", from_dev(nrm), want_n)


@pytest.mark.parametrize("two", [0, 1])
def test_k1c_land_add2(ctx, two):
    B = 33
    _case(f"k1c two={two}")
    g = rng(500 + two)
    p1 = g.standard_normal((B, H), dtype=np.float32) * np.float32(3)
    p2 = g.standard_normal((B, H), dtype=np.float32)
    prefix2 = normal_bf16(g, (B, H))
    want = O.land_add2(p1, p2, prefix2, two, B)
    hid = torch.empty((B, H), dtype=torch.bfloat16, device="cuda")
    ctx.land_add2(to_dev(p1), to_dev(p2), to_dev(prefix2), hid, two, B)
    torch.cuda.synchronize()
    _eq("hidden", from_dev(hid), want)


def _run_moe_quant(ctx, x, rows, cols):
    q = torch.empty(rows * cols, dtype=torch.uint8, device="cuda")
    sf = torch.empty(rows * cols // 32, dtype=torch.uint8, device="cuda")
    ctx.moe_quant(to_dev(x), q, sf, rows, cols)
    torch.cuda.synchronize()
    return from_dev(q), from_dev(sf)


@pytest.mark.parametrize("rows,cols", [(64, 3584), (1024, 7168), (3, 7168), (1, 32), (7, 96)])
def test_moe_quant(ctx, rows, cols):
    _case(f"moe_quant {rows}x{cols}")
    g = rng(600 + rows)
    x = normal_bf16(g, (rows, cols), outlier_p=0.001)
    x.reshape(-1)[:32] = 0
    wq, wsf = O.moe_quant(x, rows, cols)
    q, sf = _run_moe_quant(ctx, x, rows, cols)
    _eq("sf", sf, wsf.reshape(-1))
    _eq("q", q, wq.reshape(-1))


def test_moe_quant_every_bf16_pattern(ctx):
    """All 65536 bf16 patterns, NaN included, in shuffled 32-value blocks (so
    blocks also hold +-inf and NaN): exercises the hardware e4m3 conversion over
    every input and many block scales; NaN inputs give the canonical 0x7f of the
    saturating conversion and are ignored by the block amax."""
    _case("moe_quant all bf16 patterns")
    g = rng(700)
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    reps = []
    for k in range(4):
        reps.append(h[g.permutation(h.size)])
    h = np.concatenate(reps)
    h = h[: (h.size // 32) * 32]
    rows = h.size // 32
    wq, wsf = O.moe_quant(h, rows, 32)
    q, sf = _run_moe_quant(ctx, h, rows, 32)
    _eq("sf", sf, wsf.reshape(-1))
    _eq("q", q, wq.reshape(-1))


def _fused(ctx, x, res, gamma, B, eps, want_normed=True):
    xd, rd, gd = to_dev(x), to_dev(res), to_dev(gamma)
    ro = torch.empty((B, H), dtype=torch.bfloat16, device="cuda")
    q = torch.empty((B, H), dtype=torch.uint8, device="cuda")
    sf = torch.empty((B, H // 32), dtype=torch.uint8, device="cuda")
    nrm = torch.empty((B, H), dtype=torch.bfloat16, device="cuda") if want_normed else None
    ctx.residual_rms_mxfp8(xd, rd, gd, ro, q, sf, nrm, eps=eps, B=B)
    torch.cuda.synchronize()
    return from_dev(ro), from_dev(q), from_dev(sf), (from_dev(nrm) if want_normed else None)


def test_fused_residual_rms_mxfp8_nan(ctx):
    """NaN in a row (either input, either sign): its residual_out holds the NaN,
    its whole normed row is NaN, every payload byte the canonical 0x7f and every
    block scale 127 (the block amax ignores NaN); the other rows are unaffected."""
    _case("fused residual+rms+mxfp8 NaN rows")
    B = 4
    g = rng(850)
    x = normal_bf16(g, (B, H), outlier_p=0.001)
    res = normal_bf16(g, (B, H))
    gamma = normal_bf16(g, (H,), 1.0, 0.1)
    x[1, 100] = 0x7FC0
    res[2, 7000] = 0xFFC1
    x[3, 31] = 0xFF81
    wro, wq, wsf, wn = O.residual_rms_mxfp8(x, res, gamma, B, 1e-6)
    ro, q, sf, nrm = _fused(ctx, x, res, gamma, B, 1e-6)
    _eq("q", q, wq)
    _eq("sf", sf, wsf)
    for name, got, want in (("residual_out", ro, wro), ("normed", nrm, wn)):
        gn, wn_ = np.isnan(bf16_to_f32(got)), np.isnan(bf16_to_f32(want))
        assert np.array_equal(gn, wn_), f"{name}: NaN positions differ"
        _eq(name, got[~gn], want[~wn_])
    assert (q[1:] == 0x7F).all() and (sf[1:] == 127).all() and (q[0] != 0x7F).all()


@pytest.mark.parametrize("B", [1024, 16384])
def test_fused_residual_rms_mxfp8(ctx, B):
    """Config 2 (16384 x 7168, 0.1% outliers x50) and a 1024-row slice."""
    _case(f"fused residual+rms+mxfp8 B={B}")
    g = rng(800 + B)
    x = normal_bf16(g, (B, H), outlier_p=0.001)
    res = normal_bf16(g, (B, H))
    gamma = normal_bf16(g, (H,), 1.0, 0.1)
    wro, wq, wsf, wn = O.residual_rms_mxfp8(x, res, gamma, B, 1e-6)
    ro, q, sf, nrm = _fused(ctx, x, res, gamma, B, 1e-6)
    _eq("residual_out", ro, wro)
    _eq("normed", nrm, wn)
    _eq("sf", sf, wsf)
    _eq("q", q, wq)
    # q / sf are the MX rule applied to the kernel's own normed row
    q2, sf2 = O.moe_quant(nrm, B, H)
    _eq("q(normed)", q, q2)
    _eq("sf(normed)", sf, sf2)
    # without the optional normed output the other outputs are unchanged
    ro3, q3, sf3, _ = _fused(ctx, x, res, gamma, B, 1e-6, want_normed=False)
    _eq("residual_out (no normed)", ro3, wro)
    _eq("q (no normed)", q3, wq)
    _eq("sf (no normed)", sf3, wsf)


@pytest.mark.parametrize("B", [1, 3, 7])
def test_fused_ragged_rows_and_eps(ctx, B):
    _case(f"fused ragged B={B}")
    g = rng(900 + B)
    x = normal_bf16(g, (B, H), outlier_p=0.01)
    res = normal_bf16(g, (B, H))
    gamma = normal_bf16(g, (H,), 1.0, 0.1)
    for eps in (1e-6, 1e-5, 0.5):
        wro, wq, wsf, wn = O.residual_rms_mxfp8(x, res, gamma, B, eps)
        ro, q, sf, nrm = _fused(ctx, x, res, gamma, B, eps)
        _eq("residual_out", ro, wro)
        _eq("normed", nrm, wn)
        _eq("q", q, wq)
        _eq("sf", sf, wsf)


def test_zero_rows_launch_nothing(ctx):
    _case("B=0")
    t = torch.zeros(16, dtype=torch.bfloat16, device="cuda")
    u = torch.zeros(16, dtype=torch.uint8, device="cuda")
    g = torch.zeros(H, dtype=torch.bfloat16, device="cuda")
    ctx.residual_rms_mxfp8(t, t, g, t, u, u, None, eps=1e-6, B=0)
    torch.cuda.synchronize()


def test_manifest_ops_through_module_launch(ctx):
    """The manifests' own op descriptions (parameter kinds, argument maps, grid
    expressions) run unchanged through k3h_launch on the gfx950 code objects."""
    ops = json.load(open(os.path.join(GOLDEN, "manifest_hot_ops.json")))
    tokens = 4 * 40  # B = ceil(tokens / 4) = 40 rows
    B = 40
    env = {"tokens": tokens}
    # moe_quant: cols is fixed at 3584 by the op's argument map
    _case("manifest moe_quant")
    g = rng(1000)
    x = normal_bf16(g, (B, 3584), outlier_p=0.001)
    q = torch.empty(B * 3584, dtype=torch.uint8, device="cuda")
    sf = torch.empty(B * 112, dtype=torch.uint8, device="cuda")
    k3h.ManifestOp(ctx, "moe_quant", ops["moe_quant"])([to_dev(x), q, sf, B], env)
    torch.cuda.synchronize()
    wq, wsf = O.moe_quant(x, B, 3584)
    _eq("q", from_dev(q), wq.reshape(-1))
    _eq("sf", from_dev(sf), wsf.reshape(-1))
    # K1b (l0-bf16 land_add_attnres_rms_bf16_v2) and the nb1 entry of the default manifest
    prefix, partial, blocks, sw, gamma = _k1_inputs(1001, B)
    for op, nb in (("land_add_attnres_rms_bf16_v2", 2), ("land_add_attnres_rms_bf16_v2_nb1", 1)):
        _case(f"manifest {op}")
        p2 = torch.empty((B, H), dtype=torch.bfloat16, device="cuda")
        nrm = torch.empty_like(p2)
        args = [to_dev(partial), to_dev(prefix), to_dev(blocks), to_dev(sw), to_dev(gamma), p2, nrm,
                nb, 0, B]
        k3h.ManifestOp(ctx, op, ops[op])(args, env)
        torch.cuda.synchronize()
        wp2, wn = O.land_add_attnres_rms(partial, prefix, blocks, sw, gamma, nb, 0, B)
        _eq(f"{op} prefix2", from_dev(p2), wp2)
        _eq(f"{op} normed", from_dev(nrm), wn)
    # an nb entry called with another candidate count writes nothing
    _case("manifest nb1 entry with nb_in=2")
    p2 = torch.zeros((B, H), dtype=torch.bfloat16, device="cuda")
    nrm = torch.zeros_like(p2)
    args = [to_dev(partial), to_dev(prefix), to_dev(blocks), to_dev(sw), to_dev(gamma), p2, nrm, 2, 0, B]
    k3h.ManifestOp(ctx, "land_add_attnres_rms_bf16_v2_nb1", ops["land_add_attnres_rms_bf16_v2_nb1"])(args, env)
    torch.cuda.synchronize()
    assert not from_dev(p2).any() and not from_dev(nrm).any()


@pytest.mark.parametrize("nb", [0, 1, 4])
def test_k1b_special_values(ctx, nb):
    """Specials (NaN of either sign, +-inf, +-max finite, the smallest subnormal,
    -0) planted in partial, prefix and the block candidates of some rows: landing,
    AttnRes scores (NaN / inf scores through the softmax's exp) and the norm
    propagate them exactly as the oracle, through the 128-thread entry and the
    typed nb entry (vector-split body)."""
    specials = np.array([0x7FC0, 0xFFC1, 0x7F80, 0xFF80, 0x7F7F, 0xFF7F, 0x0001, 0x8000], np.uint16)
    B = 16
    _case(f"k1b special values nb={nb}")
    prefix, partial, blocks, sw, gamma = _k1_inputs(400 + nb, B)
    g = rng(401 + nb)
    # one special per row in rows 0..11 (rows 12..15 clean), in partial, prefix or a
    # block candidate in turn, so that finite specials take their own paths (a
    # largest-finite value overflows the sum of squares, a subnormal or -0 does not)
    for r in range(12):
        sv = specials[r % specials.size]
        c = int(g.integers(0, H))
        tgt = r % 3
        if tgt == 0:
            partial[r, c] = sv
        elif tgt == 1:
            prefix[r, c] = sv
        else:
            blocks[r, int(g.integers(0, max(nb, 1))), c] = sv
    want_p2, want_n = O.land_add_attnres_rms(partial, prefix, blocks, sw, gamma, nb, 0, B)

    def check(name, got, want):
        gn, wn = (got & 0x7FFF) > 0x7F80, (want & 0x7FFF) > 0x7F80
        assert np.array_equal(gn, wn), f"{name}: NaN positions differ ({gn.sum()} vs {wn.sum()})"
        assert np.array_equal(got[~gn], want[~wn]), f"{name}: non-NaN values differ"

    entries = [("128-thread entry", ctx.land_add_attnres_rms)]
    if nb > 0:
        entries.append(("typed nb entry", ctx.land_add_attnres_rms_nb))
    for label, fn in entries:
        p2 = torch.empty((B, H), dtype=torch.bfloat16, device="cuda")
        nrm = torch.empty_like(p2)
        fn(to_dev(partial), to_dev(prefix), to_dev(blocks), to_dev(sw), to_dev(gamma), p2, nrm, nb, 0, B)
        torch.cuda.synchronize()
        got_n = from_dev(nrm)
        print(f"  {label}: normed NaN rows {int(((got_n & 0x7FFF) > 0x7F80).any(axis=1).sum())} of {B}",
              flush=True)
        check(f"{label} prefix2", from_dev(p2), want_p2)
        check(f"{label} normed", got_n, want_n)
