"""Pins the K1 residual, MXFP8 and per-tensor fp8 oracles against independent
implementations: torch's bf16 arithmetic, float64 RMSNorm / softmax mixing,
and torch's float8_e4m3fn cast."""
import numpy as np
import pytest
import torch

import oracle as O
from k3data import H, bf16_to_f32, normal_bf16, rng, to_bf16, ulp_diff_bf16


def _tbf(h):
    return torch.from_numpy(h.view(np.int16)).view(torch.bfloat16)


def _bf(t):
    return t.view(torch.int16).numpy().view(np.uint16)


def _normed_f64(mixed_bf16, gamma_bf16, eps):
    """bf16(bf16(mixed * r) * gamma) with r from a float64 mean of squares."""
    m = bf16_to_f32(mixed_bf16).astype(np.float64)
    r = 1.0 / np.sqrt((m * m).mean(axis=-1, keepdims=True) + eps)
    y = to_bf16((m * r).astype(np.float32))
    return to_bf16(bf16_to_f32(y) * bf16_to_f32(gamma_bf16))


@pytest.mark.parametrize("land", ["bf16", "f32"])
@pytest.mark.parametrize("eps", [1e-5, 1e-6])
def test_k1b_nb0_against_torch_and_float64(land, eps):
    g = rng(10)
    B = 24
    prefix = normal_bf16(g, (B, H))
    gamma = normal_bf16(g, (H,), 1.0, 0.1)
    if land == "bf16":
        partial = normal_bf16(g, (B, H))
        pf = _tbf(partial).float()
    else:
        partial = g.standard_normal((B, H), dtype=np.float32)
        pf = torch.from_numpy(partial).bfloat16().float()
    p2, normed = O.land_add_attnres_rms(partial, prefix, None, None, gamma, 0, 0, B, eps)
    want_p2 = _bf((_tbf(prefix).float() + pf).bfloat16())
    assert np.array_equal(p2, want_p2)
    d = ulp_diff_bf16(normed, _normed_f64(p2, gamma, eps))
    assert d.max() <= 1 and (d > 0).mean() < 1e-3


def test_k1b_snapshot_lands_partial():
    g = rng(11)
    B = 4
    partial = g.standard_normal((B, H), dtype=np.float32)
    gamma = normal_bf16(g, (H,), 1.0, 0.1)
    p2, _ = O.land_add_attnres_rms(partial, None, None, None, gamma, 0, 1, B)
    assert np.array_equal(p2, to_bf16(partial))


@pytest.mark.parametrize("nb", [1, 3, 8])
def test_k1b_attnres_mixing_against_float64(nb):
    g = rng(20 + nb)
    B = 8
    prefix = normal_bf16(g, (B, H))
    partial = normal_bf16(g, (B, H))
    blocks = normal_bf16(g, (B, 8, H), 0.0, 2.0)
    sw = (g.standard_normal(H, dtype=np.float32) * np.float32(0.05))
    gamma = normal_bf16(g, (H,), 1.0, 0.1)
    eps = 1e-5
    p2, normed = O.land_add_attnres_rms(partial, prefix, blocks, sw, gamma, nb, 0, B, eps)
    # float64 restatement: scores, softmax over [blocks 0..nb-1, prefix2], mix
    cands = np.concatenate([bf16_to_f32(blocks[:, :nb]), bf16_to_f32(p2)[:, None]], axis=1)
    c64 = cands.astype(np.float64)
    sq = (c64 * c64).sum(-1)
    dp = (c64 * sw.astype(np.float64)).sum(-1)
    sc = dp / np.sqrt(sq / H + eps)
    p = np.exp(sc - sc.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    m64 = (p[:, :, None] * c64).sum(1)
    ref = _normed_f64(to_bf16(m64.astype(np.float32)), gamma, eps)
    d = ulp_diff_bf16(normed, ref)
    # where the mix cancels (|mixed| << the candidates) f32 and f64 sums differ
    # by more than a bf16 ulp of the small result: bound those absolutely.
    mag = np.abs(c64).max(1)
    clean = np.abs(m64) > 0.05 * mag
    # a one-ulp flip of the f32-vs-f64 mixed value can become two after gamma
    assert d[clean].max() <= 2 and (d[clean] > 0).mean() < 1e-3
    r = 1.0 / np.sqrt((bf16_to_f32(ref).astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-30)
    err = np.abs(bf16_to_f32(normed).astype(np.float64) - bf16_to_f32(ref))
    refv = np.abs(bf16_to_f32(ref).astype(np.float64))
    ulp = np.exp2(np.floor(np.log2(np.maximum(refv, 1e-30))) - 7)
    bound = 2 * ulp + 4e-7 * mag * r * 1.5  # f32 rounding of the mix, carried through r, gamma
    assert np.all(err[~clean] <= bound[~clean])


def test_k1a_snapshot_and_k1c():
    g = rng(30)
    B = 6
    prefix = normal_bf16(g, (B, H))
    blocks = normal_bf16(g, (B, 8, H))
    sw = g.standard_normal(H, dtype=np.float32) * np.float32(0.05)
    gamma = normal_bf16(g, (H,), 1.0, 0.1)
    blk2, normed = O.attnres_rms(prefix, blocks, sw, gamma, 2, 1, B)
    assert np.array_equal(blk2[:, 2], prefix)
    assert np.array_equal(np.delete(blk2, 2, axis=1), np.delete(blocks, 2, axis=1))
    # nb = 0 without snapshot: plain RMSNorm of the prefix
    _, n0 = O.attnres_rms(prefix, blocks, sw, gamma, 0, 0, B)
    assert ulp_diff_bf16(n0, _normed_f64(prefix, gamma, 1e-5)).max() <= 1
    p1 = g.standard_normal((B, H), dtype=np.float32)
    p2 = g.standard_normal((B, H), dtype=np.float32)
    for two in (0, 1):
        hid = O.land_add2(p1, p2, prefix, two, B)
        s = _tbf(prefix).float() + torch.from_numpy(p1).bfloat16().float()
        if two:
            s = s + torch.from_numpy(p2).bfloat16().float()
        assert np.array_equal(hid, _bf(s.bfloat16()))


def _mx_numpy(x_bf16):
    """Independent MXFP8: numpy amax, ceil(log2) in float64, torch e4m3 cast."""
    v = bf16_to_f32(x_bf16).reshape(-1, 32)
    amax = np.abs(v).max(-1)
    with np.errstate(divide="ignore"):
        e = np.where(amax > 0, np.ceil(np.log2((amax / np.float32(448)).astype(np.float64))), 0)
    e = np.clip(e, -127, 127).astype(np.int64)
    s = np.ldexp(np.float32(1.0), -e).astype(np.float32)
    y = (v * s[:, None]).astype(np.float32)
    q = torch.from_numpy(np.clip(y, -448, 448)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return q.reshape(-1), (e + 127).astype(np.uint8)


def test_moe_quant_against_numpy_torch():
    g = rng(40)
    rows, cols = 64, 3584
    x = normal_bf16(g, (rows, cols), outlier_p=0.001)
    x[3, :32] = 0                       # an all-zero block
    x[5, 32:64] = to_bf16(np.full(32, 1e-40, np.float32))  # subnormal block
    x[7, :32] = to_bf16(np.linspace(-448 * 4, 448 * 4, 32).astype(np.float32))
    q, sf = O.moe_quant(x, rows, cols)
    wq, wsf = _mx_numpy(x)
    assert np.array_equal(sf.reshape(-1), wsf)
    assert np.array_equal(q.reshape(-1), wq)


def test_moe_quant_all_bf16_patterns():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = bf16_to_f32(h)
    h = h[np.isfinite(f)]
    h = h[: (h.size // 32) * 32]
    rows = h.size // 32
    q, sf = O.moe_quant(np.ascontiguousarray(h), rows, 32)
    wq, wsf = _mx_numpy(h)
    assert np.array_equal(sf.reshape(-1), wsf)
    assert np.array_equal(q.reshape(-1), wq)


def test_moe_quant_nan_ignored_by_amax():
    """A NaN of any kind (quiet or signalling bf16 pattern, either sign, first,
    middle or last in its block) is ignored by the block amax and quantises to
    the canonical 0x7f: the block equals the same block with its NaNs replaced
    by zero everywhere else.  (glibc's fmaxf would turn a signalling NaN into a
    quiet NaN amax, so a NaN last in its block would reset the scale.)"""
    g = rng(41)
    rows, cols = 8, 256
    x = normal_bf16(g, (rows, cols), outlier_p=0.01)
    nan_pats = [0x7F81, 0xFF86, 0x7FC0, 0xFFC1, 0x7FFF, 0xFFBF]
    pos = []
    for k, pat in enumerate(nan_pats):
        for j in (0, 17, 31):
            r, c = (k + j) % rows, 32 * ((k * 3 + j) % (cols // 32)) + j
            x[r, c] = pat
            pos.append((r, c))
    x[7, 64:96] = 0x7F81  # a block of NaN only: amax 0, scale 127
    z = x.copy()
    isn = np.isnan(bf16_to_f32(x))
    z[isn] = 0
    q, sf = O.moe_quant(x, rows, cols)
    wq, wsf = _mx_numpy(z)
    assert np.array_equal(sf.reshape(-1), wsf)
    assert (q[isn] == 0x7F).all()
    assert np.array_equal(q[~isn], wq.reshape(rows, cols)[~isn])
    assert sf[7, 2] == 127
    # per-tensor v1 partials ignore every NaN as well
    p = O.quant_fp8_amax(x.reshape(-1), rows * cols, 4, v2=False)
    pz = O.quant_fp8_amax(z.reshape(-1), rows * cols, 4, v2=False)
    assert np.array_equal(p, pz)


def test_fused_is_k1b_then_moe_quant():
    g = rng(50)
    B = 16
    x = normal_bf16(g, (B, H), outlier_p=0.001)
    res = normal_bf16(g, (B, H))
    gamma = normal_bf16(g, (H,), 1.0, 0.1)
    ro, q, sf, normed = O.residual_rms_mxfp8(x, res, gamma, B, 1e-6)
    p2, n2 = O.land_add_attnres_rms(x, res, None, None, gamma, 0, 0, B, 1e-6)
    assert np.array_equal(ro, p2) and np.array_equal(normed, n2)
    q2, sf2 = O.moe_quant(n2, B, H)
    assert np.array_equal(q, q2) and np.array_equal(sf, sf2)
    # dequantised payload stays within one e4m3 step of the normed value
    deq = O.e4m3_decode(q[:2]).astype(np.float64) * np.ldexp(1.0, sf[:2].astype(np.int64) - 127).repeat(32, -1)
    ref = bf16_to_f32(normed[:2]).astype(np.float64)
    scale = np.ldexp(1.0, sf[:2].astype(np.int64) - 127).repeat(32, -1)
    assert np.all(np.abs(deq - ref) <= np.maximum(np.abs(ref) * 2.0**-4, scale * 2.0**-9) + 1e-30)


@pytest.mark.parametrize("v2", [0, 1])
def test_quant_fp8_pair_against_numpy(v2):
    g = rng(60 + v2)
    n = 7168 * 40 + 5  # ragged tail
    x = normal_bf16(g, (n,), outlier_p=0.001)
    partials = O.quant_fp8_amax(x, n, 64, v2=bool(v2))
    assert partials.max() == np.abs(bf16_to_f32(x)).max()
    y, scale = O.quant_fp8_apply(x, n, partials, 64)
    amax = np.float32(np.abs(bf16_to_f32(x)).max())
    s = np.float32(amax / np.float32(448))
    assert scale[0] == s
    inv = np.float32(np.float32(1) / s)
    want = torch.from_numpy(np.clip(bf16_to_f32(x) * inv, -448, 448).astype(np.float32)).to(
        torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(y, want)


@pytest.mark.parametrize("v2,n,nb", [(0, 7168 * 40 + 5, 64), (1, 7168 * 40 + 5, 64), (1, 8 * 256 * 3 + 3, 2),
                                     (0, 1000, 3)])
def test_quant_fp8_amax_partials_per_block(v2, n, nb):
    """Every amax partial, not only their maximum: block b's slice of the grid
    stride (kern_quant_fp8_amax: elements (i // 256) % nb == b; _v2: 8-element
    vectors (i // 8 // 256) % nb == b, the n % 8 tail in block 0), restated by
    reshapes over a zero-padded |x|."""
    g = rng(90 + v2 + n % 7)
    x = normal_bf16(g, (n,), outlier_p=0.01)
    a = np.abs(bf16_to_f32(x))
    got = O.quant_fp8_amax(x, n, nb, v2=bool(v2))
    if not v2:
        stride = nb * 256
        pad = np.zeros(-(-n // stride) * stride, np.float32)
        pad[:n] = a
        want = pad.reshape(-1, nb, 256).max(axis=(0, 2))
    else:
        nv = n // 8
        stride = nb * 256
        pad = np.zeros(-(-nv // stride) * stride * 8, np.float32)
        pad[:nv * 8] = a[:nv * 8]
        want = pad.reshape(-1, nb, 256 * 8).max(axis=(0, 2))
        if n % 8:
            want[0] = max(want[0], a[nv * 8:].max())
    assert np.array_equal(got, want.astype(np.float32))
    # a planted change of one element moves exactly its own block's partial
    i = n // 3
    y = x.copy()
    y[i] = 0x7f00  # bf16 1.7e38, larger than every other |x|
    b = (i // 256) % nb if not v2 else ((i // 8) // 256) % nb if i < (n // 8) * 8 else 0
    got2 = O.quant_fp8_amax(y, n, nb, v2=bool(v2))
    changed = np.nonzero(got2 != got)[0].tolist()
    assert changed == [b]
