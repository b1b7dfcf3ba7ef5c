"""Pins the MLA oracles: RMSNorms against float64, landing copies against
torch's bf16 cast, slab addressing, and the RoPE rotation against the double
closed form (position 0 is the identity)."""
import numpy as np
import torch

import oracle as O
from k3data import bf16_to_f32, normal_bf16, rng, to_bf16, ulp_diff_bf16


def _rms_ref(x_bf16, gamma_bf16, eps):
    x = bf16_to_f32(x_bf16).astype(np.float64)
    r = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    y = to_bf16((x * r).astype(np.float32))
    return to_bf16(bf16_to_f32(y) * bf16_to_f32(gamma_bf16))


def test_mla_prep_against_float64_and_landing():
    g = rng(300)
    B, ps, lo = 9, 3 * 64 * 576, 64 * 576
    pf = g.standard_normal((B, 5184), dtype=np.float32)
    gq = normal_bf16(g, (1536,), 1.0, 0.1)
    gk = normal_bf16(g, (512,), 1.0, 0.1)
    slots = np.array([0, 63, 64, 130, -1, 5, 191, 70, 1], np.int64)
    slab0 = g.integers(0, 65535, 3 * ps, dtype=np.uint16)
    slab, qn, gate = O.mla_prep(pf, gq, gk, slots, slab0, lo, ps, B)
    pb = to_bf16(pf)
    assert np.array_equal(gate, pb[:, 2112:])
    d = ulp_diff_bf16(qn, _rms_ref(pb[:, :1536], gq, 1e-5))
    assert d.max() <= 1 and (d > 0).mean() < 2e-3
    kvn = _rms_ref(pb[:, 1536:2048], gk, 1e-5)
    touched = np.zeros(slab.size, bool)
    for b, s in enumerate(slots):
        if s < 0:
            continue
        at = (s // 64) * ps + lo + (s % 64) * 576
        touched[at:at + 576] = True
        assert ulp_diff_bf16(slab[at:at + 512], kvn[b]).max() <= 1
        assert np.array_equal(slab[at + 512:at + 576], pb[b, 2048:2112])
    assert np.array_equal(slab[~touched], slab0[~touched])
    # the bf16-partial module computes the same from the landed values
    slab2, qn2, gate2 = O.mla_prep(pb, gq, gk, slots, slab0, lo, ps, B)
    assert np.array_equal(slab2, slab) and np.array_equal(qn2, qn) and np.array_equal(gate2, gate)


def test_rope_pack_against_closed_form():
    g = rng(310)
    T, H = 64, 16
    lat = normal_bf16(g, (T, 512))
    kr = normal_bf16(g, (T, 64))
    q = normal_bf16(g, (T, H, 192))
    gk = normal_bf16(g, (512,), 1.0, 0.1)
    pos = np.concatenate([[0, 1, 16383], g.integers(0, 16384, T - 3)]).astype(np.int64)
    lo, qo = O.mla_rope_pack(lat, kr, q, gk, pos, T, H, 50000.0, 1e-6)
    assert np.array_equal(qo[:, :, :128], q[:, :, :128])
    d = ulp_diff_bf16(lo[:, :512], _rms_ref(lat, gk, 1e-6))
    assert d.max() <= 1 and (d > 0).mean() < 2e-3
    j = np.arange(32)
    ang = pos[:, None].astype(np.float64) * 50000.0 ** (-(2.0 * j) / 64.0)
    c, s = np.cos(ang), np.sin(ang)

    def rot(x):  # x [..., 64] bf16 -> closed form in double
        x = bf16_to_f32(x).astype(np.float64)
        x0, x1 = x[..., 0::2], x[..., 1::2]
        cc = c.reshape(c.shape[:1] + (1,) * (x0.ndim - 2) + (32,))
        ss = s.reshape(cc.shape)
        y = np.empty_like(x)
        y[..., 0::2] = x0 * cc - x1 * ss
        y[..., 1::2] = x0 * ss + x1 * cc
        return to_bf16(y.astype(np.float32))

    for got, want in ((lo[:, 512:], rot(kr)), (qo[:, :, 128:], rot(q[:, :, 128:]))):
        d = ulp_diff_bf16(got, want)
        assert d.max() <= 1 and (d > 0).mean() < 2e-3
    # position 0 rotates by zero: the rope dims come through unchanged
    assert np.array_equal(lo[0, 512:], kr[0]) and np.array_equal(qo[0, :, 128:], q[0, :, 128:])
