"""GPU parity: landing kernels of the shared-expert MLP and the MoE latent norm
(kern_k3_rms, kern_k3_land, the SiTU landings and the fused SiTU + rms) against
the C oracle through the k3h C-ABI.  Bar: bit-exact for rms (shared reduction
order, correctly rounded 1/sqrt) and land (one RNE); the SiTU activation within
one bf16 ulp of the exact value, with fewer than 1e-3 of the outputs off by one."""
import json
import os

import numpy as np
import pytest
import torch

import k3h
import oracle as O
from k3data import bf16_to_f32, from_dev, normal_bf16, rng, to_bf16, to_dev, ulp_diff_bf16

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _eq(name, got, want):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (name, got.shape, want.shape)
    bad = np.flatnonzero(got.ravel() != want.ravel())
    assert bad.size == 0, f"{name}: {bad.size} of {got.size} differ, first at {bad[:5]}"


def _close1(name, got, want, frac=1e-3):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape
    nan_g, nan_w = (bf16_to_f32(got) != bf16_to_f32(got)), (bf16_to_f32(want) != bf16_to_f32(want))
    assert np.array_equal(nan_g, nan_w), f"{name}: NaN positions differ"
    d = ulp_diff_bf16(got[~nan_g], want[~nan_w])
    print(f"  {name}: max ulp {d.max() if d.size else 0}, differing {(d > 0).mean() if d.size else 0:.2e}",
          flush=True)
    assert d.size == 0 or (d.max() <= 1 and (d > 0).mean() < frac), name


@pytest.mark.parametrize("h,B", [(3584, 4096), (3584, 37), (7168, 20), (1024, 3), (12, 5),
                                  (1000, 4), (16384, 3), (40000, 2)])
def test_rms(ctx, h, B):
    _case(f"rms h={h} B={B}")
    g = rng(500 + h + B)
    x = normal_bf16(g, (B, h), outlier_p=0.001)
    gamma = normal_bf16(g, (h,), 1.0, 0.1)
    o = torch.full((B, h), 0, dtype=torch.bfloat16, device="cuda")
    ctx.rms(to_dev(x), to_dev(gamma), o, h, B)
    torch.cuda.synchronize()
    _eq("o", from_dev(o), O.rms(x, gamma, h, B))


@pytest.mark.parametrize("n,off,ldc,B", [(3584, 0, 3584, 4096), (3584, 0, 3584, 13),
                                          (1000, 24, 2048, 7), (1001, 3, 1010, 5)])
def test_land(ctx, n, off, ldc, B):
    _case(f"land n={n} off={off} ldc={ldc} B={B}")
    g = rng(520 + n + B)
    p = g.standard_normal((B, ldc), dtype=np.float32) * np.float32(3.0)
    o = torch.zeros((B, n), dtype=torch.bfloat16, device="cuda")
    ctx.land(to_dev(p), o, n, off, ldc, B)
    torch.cuda.synchronize()
    _eq("o", from_dev(o), O.land(p, n, off, ldc, B))


@pytest.mark.parametrize("kind,n,B", [("f32", 33792, 64), ("f32", 6144, 97), ("land_bf16", 6144, 33),
                                       ("situ_bf16", 33792, 16), ("f32", 24, 3), ("situ_bf16", 13, 4),
                                       ("f32", 13, 3)])
def test_land_situ(ctx, kind, n, B):
    _case(f"land_situ {kind} n={n} B={B}")
    g = rng(540 + n + B)
    if kind == "f32":
        p = (g.standard_normal((B, 2 * n)) * 3.0).astype(np.float32)
        pd = to_dev(p)
    else:
        p = normal_bf16(g, (B, 2 * n), std=3.0)
        pd = to_dev(p)
    act = torch.zeros((B, n), dtype=torch.bfloat16, device="cuda")
    ctx.land_situ(pd, act, n, B, variant=None if kind != "situ_bf16" else "situ_bf16")
    torch.cuda.synchronize()
    _close1("act", from_dev(act), O.land_situ(p, n, B))


@pytest.mark.parametrize("pad", [0, 4])
def test_situ_special_values(ctx, pad):
    """0, +-inf, NaN, huge and tiny gate / up operands; n = 484 takes the
    per-element path, n = 488 the 8-wide one."""
    vals = np.array([0.0, -0.0, 1e-30, -1e-30, 1e-3, -1e-3, 0.25, 0.9999, 1.0, 4.0, -4.0, 20.0, -20.0,
                     87.0, -87.0, 90.0, -90.0, 1e30, -1e30, np.inf, -np.inf, np.nan], np.float32)
    gg, uu = np.meshgrid(vals, vals, indexing="ij")
    gg = np.concatenate([gg.ravel(), np.ones(pad, np.float32)])
    uu = np.concatenate([uu.ravel(), np.ones(pad, np.float32)])
    n = gg.size
    _case(f"situ special values n={n}")
    p = to_bf16(np.concatenate([gg, uu])[None, :])
    act = torch.zeros((1, n), dtype=torch.bfloat16, device="cuda")
    ctx.land_situ(to_dev(p), act, n, 1)
    torch.cuda.synchronize()
    got, want = from_dev(act), O.land_situ(p, n, 1)
    fg, fw = bf16_to_f32(got), bf16_to_f32(want)
    # denormal-range results (|x| < 2^-126) may flush to zero on the GPU
    tiny = np.abs(fw) < np.float32(2.0 ** -126)
    assert (np.abs(fg[tiny]) < np.float32(2.0 ** -126)).all()
    _close1("special", got[~tiny], want[~tiny], frac=0.05)


@pytest.mark.parametrize("tokens", [16384, 100, 16])
def test_situ_rms(ctx, tokens):
    n, h = 6144, 3584
    B = L = -(-tokens // 4)
    _case(f"situ_rms tokens={tokens} B=L={B}")
    g = rng(560 + tokens)
    sp = normal_bf16(g, (B, 2 * n), std=2.0)
    lat = normal_bf16(g, (L, h))
    gam = normal_bf16(g, (h,), 1.0, 0.1)
    act = torch.zeros((B, n), dtype=torch.bfloat16, device="cuda")
    ln = torch.zeros((L, h), dtype=torch.bfloat16, device="cuda")
    ctx.situ_rms(to_dev(sp), act, to_dev(lat), to_dev(gam), ln, n, B, h, L, tokens)
    torch.cuda.synchronize()
    wa, wl = O.situ_rms(sp, lat, gam, n, B, h, L, tokens)
    _eq("ln", from_dev(ln), wl)
    _close1("act", from_dev(act), wa)


def test_manifest_land_ops(ctx):
    """The manifests' landing ops run from their own op descriptions."""
    ops = json.load(open(os.path.join(GOLDEN, "manifest_hot_ops.json")))
    tokens = 4 * 24
    B = 24
    env = {"tokens": tokens}
    g = rng(580)
    _case("manifest land_situ_n33792 (f32)")
    p = (g.standard_normal((B, 2 * 33792)) * 3.0).astype(np.float32)
    act = torch.zeros((B, 33792), dtype=torch.bfloat16, device="cuda")
    k3h.ManifestOp(ctx, "land_situ_n33792", ops["land_situ_n33792"])([to_dev(p), act, B], env)
    torch.cuda.synchronize()
    _close1("land_situ_n33792", from_dev(act), O.land_situ(p, 33792, B))
    del p
    _case("manifest l0 land_situ_n33792 (bf16)")
    pb = normal_bf16(g, (B, 2 * 33792), std=3.0)
    act = torch.zeros((B, 33792), dtype=torch.bfloat16, device="cuda")
    k3h.ManifestOp(ctx, "l0_land_situ_n33792", ops["l0_land_situ_n33792"])([to_dev(pb), act, B], env)
    torch.cuda.synchronize()
    _close1("l0_land_situ_n33792", from_dev(act), O.land_situ(pb, 33792, B))
    _case("manifest l0 land_situ_n6144")
    p = (g.standard_normal((B, 2 * 6144)) * 3.0).astype(np.float32)
    act = torch.zeros((B, 6144), dtype=torch.bfloat16, device="cuda")
    k3h.ManifestOp(ctx, "land_situ_n6144", ops["land_situ_n6144"])([to_dev(p), act, B], env)
    torch.cuda.synchronize()
    _close1("land_situ_n6144", from_dev(act), O.land_situ(p, 6144, B))
    _case("manifest l0 rms and land_n3584")
    x = normal_bf16(g, (B, 3584))
    gm = normal_bf16(g, (3584,), 1.0, 0.1)
    o = torch.zeros((B, 3584), dtype=torch.bfloat16, device="cuda")
    k3h.ManifestOp(ctx, "rms", ops["rms"])([to_dev(x), to_dev(gm), o, B], env)
    pf = g.standard_normal((B, 3584), dtype=np.float32)
    o2 = torch.zeros((B, 3584), dtype=torch.bfloat16, device="cuda")
    k3h.ManifestOp(ctx, "land_n3584", ops["land_n3584"])([to_dev(pf), o2, B], env)
    torch.cuda.synchronize()
    _eq("rms", from_dev(o), O.rms(x, gm, 3584, B))
    _eq("land_n3584", from_dev(o2), O.land(pf, 3584, 0, 3584, B))
    _case("manifest land_situ_rms")
    sp = normal_bf16(g, (B, 2 * 6144), std=2.0)
    lat = normal_bf16(g, (B, 3584))
    act = torch.zeros((B, 6144), dtype=torch.bfloat16, device="cuda")
    ln = torch.zeros((B, 3584), dtype=torch.bfloat16, device="cuda")
    k3h.ManifestOp(ctx, "land_situ_rms", ops["land_situ_rms"])(
        [to_dev(sp), act, to_dev(lat), to_dev(gm), ln, B, B], env)
    torch.cuda.synchronize()
    wa, wl = O.situ_rms(sp, lat, gm, 6144, B, 3584, B, tokens)
    _eq("land_situ_rms ln", from_dev(ln), wl)
    _close1("land_situ_rms act", from_dev(act), wa)
