"""GPU parity: MLA prep (f32 and bf16 partial modules; q_norm, paged latent
rows, gate landing) and the latent-norm + RoPE + q packing op against the C
oracle, bit-exact."""
import json
import os

import numpy as np
import pytest
import torch

import k3h
import oracle as O
from k3data import from_dev, normal_bf16, rng, to_dev

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _case(m):
    print(f"[case] {m}", flush=True)


def _eq(name, got, want):
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape, (name, got.shape, want.shape)
    bad = np.flatnonzero(got.ravel() != want.ravel())
    assert bad.size == 0, f"{name}: {bad.size} of {got.size} differ, first at {bad[:5]}"


def _prep_inputs(B, bf16, seed, ps, lo, npages):
    g = rng(seed)
    pf = g.standard_normal((B, 5184), dtype=np.float32)
    partial = normal_bf16(g, (B, 5184)) if bf16 else pf
    gq = normal_bf16(g, (1536,), 1.0, 0.1)
    gk = normal_bf16(g, (512,), 1.0, 0.1)
    slots = g.permutation(npages * 64)[:B].astype(np.int64)
    slots[::7] = -1
    slab0 = g.integers(0, 65535, npages * ps, dtype=np.uint16)
    return partial, gq, gk, slots, slab0


@pytest.mark.parametrize("bf16", [True, False])
@pytest.mark.parametrize("B,ps,lo", [(16384, 2 * 64 * 576, 64 * 576), (13, 884736, 5 * 64 * 576)])
def test_mla_prep(ctx, bf16, B, ps, lo):
    _case(f"mla_prep B={B} bf16={bf16} page_stride={ps}")
    npages = (B + 63) // 64 + 1
    partial, gq, gk, slots, slab0 = _prep_inputs(B, bf16, 3000 + B, ps, lo, npages)
    want_slab, want_q, want_g = O.mla_prep(partial, gq, gk, slots, slab0, lo, ps, B)
    d_slab = to_dev(slab0)
    qn = torch.empty((B, 1536), dtype=torch.bfloat16, device="cuda")
    gate = torch.empty((B, 3072), dtype=torch.bfloat16, device="cuda")
    ctx.mla_prep(to_dev(partial), to_dev(gq), to_dev(gk), to_dev(slots), d_slab, lo, qn, gate, B,
                 page_stride=ps)
    torch.cuda.synchronize()
    _eq("q_norm", from_dev(qn), want_q)
    _eq("mla_gate", from_dev(gate), want_g)
    _eq("slab", from_dev(d_slab), want_slab)


@pytest.mark.parametrize("T,H", [(16384, 16), (7, 24), (1, 16)])
def test_mla_rope_pack(ctx, T, H):
    _case(f"mla_rope_pack T={T} H={H}")
    g = rng(3100 + T)
    lat = normal_bf16(g, (T, 512))
    kr = normal_bf16(g, (T, 64))
    q = normal_bf16(g, (T, H, 192))
    gk = normal_bf16(g, (512,), 1.0, 0.1)
    pos = np.arange(T, dtype=np.int64) if T > 8 else g.integers(0, 16384, T).astype(np.int64)
    wl, wq = O.mla_rope_pack(lat, kr, q, gk, pos, T, H, 50000.0, 1e-6)
    lo = torch.empty((T, 576), dtype=torch.bfloat16, device="cuda")
    qo = torch.empty((T, H, 192), dtype=torch.bfloat16, device="cuda")
    ctx.mla_rope_pack(to_dev(lat), to_dev(kr), to_dev(q), to_dev(gk), to_dev(pos), lo, qo, T, H)
    torch.cuda.synchronize()
    _eq("latent_out", from_dev(lo), wl)
    _eq("q_out", from_dev(qo), wq)


def test_manifest_mla_prep(ctx):
    ops = json.load(open(os.path.join(GOLDEN, "manifest_hot_ops.json")))
    tokens = 256
    B = tokens // 4
    _case("manifest mla_prep")
    ps, lo = 884736, 2 * 64 * 576
    partial, gq, gk, slots, slab0 = _prep_inputs(B, True, 3200, ps, lo, 3)
    d_slab = to_dev(slab0)
    qn = torch.empty((B, 1536), dtype=torch.bfloat16, device="cuda")
    gate = torch.empty((B, 3072), dtype=torch.bfloat16, device="cuda")
    k3h.ManifestOp(ctx, "mla_prep", ops["mla_prep"])(
        [to_dev(partial), to_dev(gq), to_dev(gk), to_dev(slots), d_slab, lo, qn, gate, B],
        {"tokens": tokens})
    torch.cuda.synchronize()
    ws, wq, wg = O.mla_prep(partial, gq, gk, slots, slab0, lo, ps, B)
    _eq("q_norm", from_dev(qn), wq)
    _eq("mla_gate", from_dev(gate), wg)
    _eq("slab", from_dev(d_slab), ws)


SPECIALS16 = np.array([0x7FC0, 0xFFC1, 0x7F80, 0xFF80, 0x7F7F, 0xFF7F, 0x0001, 0x8000], np.uint16)
SPECIALS32 = np.array([np.nan, -np.nan, np.inf, -np.inf, 3.4e38, -3.4e38, 1e-45, -0.0], np.float32)


def _eq_special(name, got, want):
    """bf16 outputs: NaN at the same positions (any NaN pattern), every other
    value bit-exact (infinities included)."""
    got, want = np.asarray(got), np.asarray(want)
    gn, wn = (got & 0x7FFF) > 0x7F80, (want & 0x7FFF) > 0x7F80
    assert np.array_equal(gn, wn), f"{name}: NaN positions differ ({gn.sum()} vs {wn.sum()})"
    bad = np.flatnonzero(got[~gn] != want[~wn])
    print(f"  {name}: {gn.sum()} NaN, {((got & 0x7FFF) == 0x7F80).sum()} inf", flush=True)
    assert bad.size == 0, f"{name}: {bad.size} non-NaN values differ"


def _plant(a, specials, n, g):
    flat = a.reshape(-1)
    flat[g.choice(flat.size, n, replace=False)] = specials[np.arange(n) % specials.size]


@pytest.mark.parametrize("bf16", [True, False])
def test_mla_prep_special_values(ctx, bf16):
    """NaN (either sign), +-inf, +-max finite, the smallest subnormal and -0 in the
    fused partial rows: the head norms, the latent landing and the gate landing
    carry them exactly as the oracle (a NaN or infinity in a normed group makes
    the group's sum of squares NaN / inf)."""
    B, ps, lo = 40, 884736, 5 * 64 * 576
    _case(f"mla_prep special values bf16={bf16}")
    partial, gq, gk, slots, slab0 = _prep_inputs(B, bf16, 3300, ps, lo, 2)
    g = rng(3301)
    _plant(partial, SPECIALS16 if bf16 else SPECIALS32, 96, g)
    want_slab, want_q, want_g = O.mla_prep(partial, gq, gk, slots, slab0, lo, ps, B)
    d_slab = to_dev(slab0)
    qn = torch.empty((B, 1536), dtype=torch.bfloat16, device="cuda")
    gate = torch.empty((B, 3072), dtype=torch.bfloat16, device="cuda")
    ctx.mla_prep(to_dev(partial), to_dev(gq), to_dev(gk), to_dev(slots), d_slab, lo, qn, gate, B,
                 page_stride=ps)
    torch.cuda.synchronize()
    _eq_special("q_norm", from_dev(qn), want_q)
    _eq_special("mla_gate", from_dev(gate), want_g)
    _eq_special("slab", from_dev(d_slab), want_slab)


def test_mla_rope_pack_special_values(ctx):
    """Specials in the latent rows, k_rope and q (nope and rope dims): a NaN or
    infinity in a latent row makes its norm NaN / 0-scaled, rotated pairs mix
    their two inputs, copied dims pass unchanged; all as the oracle."""
    T, H = 20, 16
    _case("mla_rope_pack special values")
    g = rng(3400)
    lat, kr, q = normal_bf16(g, (T, 512)), normal_bf16(g, (T, 64)), normal_bf16(g, (T, H, 192))
    gk = normal_bf16(g, (512,), 1.0, 0.1)
    for a, n in ((lat, 24), (kr, 16), (q, 96)):
        _plant(a, SPECIALS16, n, g)
    pos = g.integers(0, 16384, T).astype(np.int64)
    wl, wq = O.mla_rope_pack(lat, kr, q, gk, pos, T, H, 50000.0, 1e-6)
    lo = torch.empty((T, 576), dtype=torch.bfloat16, device="cuda")
    qo = torch.empty((T, H, 192), dtype=torch.bfloat16, device="cuda")
    ctx.mla_rope_pack(to_dev(lat), to_dev(kr), to_dev(q), to_dev(gk), to_dev(pos), lo, qo, T, H)
    torch.cuda.synchronize()
    _eq_special("latent_out", from_dev(lo), wl)
    _eq_special("q_out", from_dev(qo), wq)
