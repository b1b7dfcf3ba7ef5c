"""Pins the oracle of the residual push family (statistics hand-off res_in ->
res_mlp, land_add2 with bf16 partials) and of the landing kernels (rms, land,
SiTU, the fused SiTU + rms) against independent implementations: float64
sums, numpy/torch bf16 arithmetic, and the closed form of the activation."""
import numpy as np
import pytest
import torch

import oracle as O
from k3data import H, bf16_to_f32, normal_bf16, rng, to_bf16, ulp_diff_bf16


def _k1(seed, B, nb_blocks=8):
    g = rng(seed)
    prefix = normal_bf16(g, (B, H))
    partial = normal_bf16(g, (B, H))
    blocks = normal_bf16(g, (B, 8, H))
    sw = (g.standard_normal(H).astype(np.float32) * np.float32(0.05))
    sw_mlp = (g.standard_normal(H).astype(np.float32) * np.float32(0.05))
    gamma = normal_bf16(g, (H,), 1.0, 0.1)
    return prefix, partial, blocks, sw, sw_mlp, gamma


# ---------------------------------------------------------------- push / stats
@pytest.mark.parametrize("nb", [1, 4, 8])
def test_push_stats_are_float64_sums(nb):
    """stats[b, c] = (sum x^2, sum x * sw_mlp) over block candidate c, in f32."""
    B = 3
    prefix, _, blocks, sw, sw_mlp, gamma = _k1(300 + nb, B)
    _, normed, stats = O.attnres_rms_stats(prefix, blocks, sw, gamma, nb, 0, B, sw_mlp=sw_mlp)
    x = bf16_to_f32(blocks[:, :nb]).astype(np.float64)
    sq = (x * x).sum(-1)
    dm = (x * sw_mlp.astype(np.float64)).sum(-1)
    assert np.allclose(stats[:, :nb, 0], sq, rtol=1e-5)
    assert np.allclose(stats[:, :nb, 1], dm, rtol=1e-4, atol=1e-3)
    assert not stats[:, nb:].any()  # candidates past nb are not written
    # the statistics ride along: normed is K1a's
    _, want = O.attnres_rms(prefix, blocks, sw, gamma, nb, 0, B)
    assert np.array_equal(normed, want)


@pytest.mark.parametrize("nb", [1, 3, 8])
def test_stats_handoff_is_bit_identical(nb):
    """res_mlp fed res_in's statistics (sw_mlp = res_mlp's own sw) computes the
    same bits as res_mlp without them, for every nb_stats <= nb.  With sw_mlp
    different from res_in's sw, a hand-off that passed dp (x . sw) instead of
    x . sw_mlp would fail here."""
    B = 4
    prefix, partial, blocks, sw_in, sw_mlp, gamma = _k1(310 + nb, B)
    _, _, stats = O.attnres_rms_stats(prefix, blocks, sw_in, gamma, nb, 0, B, sw_mlp=sw_mlp)
    want = O.land_add_attnres_rms(partial, prefix, blocks, sw_mlp, gamma, nb, 0, B)
    for ns in sorted({0, 1, nb - 1, nb}):
        got = O.land_add_attnres_rms_stats(partial, prefix, blocks, sw_mlp, gamma, nb, 0, B, stats, ns)
        assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1]), ns


def test_stats_in_are_used():
    """A perturbed statistic changes the mix (the consumer does read them)."""
    B, nb = 2, 4
    prefix, partial, blocks, sw, sw_mlp, gamma = _k1(320, B)
    _, _, stats = O.attnres_rms_stats(prefix, blocks, sw, gamma, nb, 0, B, sw_mlp=sw)
    base = O.land_add_attnres_rms_stats(partial, prefix, blocks, sw, gamma, nb, 0, B, stats, nb)[1]
    bad = stats.copy()
    bad[:, 0, 1] += np.float32(5.0)
    got = O.land_add_attnres_rms_stats(partial, prefix, blocks, sw, gamma, nb, 0, B, bad, nb)[1]
    assert not np.array_equal(got, base)
    # nb_stats above nb is clamped to nb
    got = O.land_add_attnres_rms_stats(partial, prefix, blocks, sw, gamma, nb, 0, B, stats, nb + 3)[1]
    assert np.array_equal(got, base)


@pytest.mark.parametrize("two", [0, 1])
def test_land_add2_bf16_against_torch(two):
    g = rng(330 + two)
    B = 5
    p1, p2, pr = (normal_bf16(g, (B, H)) for _ in range(3))
    t = lambda h: torch.from_numpy(h.view(np.int16)).view(torch.bfloat16).float()
    x = t(pr) + t(p1)
    if two:
        x = x + t(p2)
    want = x.bfloat16().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.land_add2_bf16(p1, p2, pr, two, B), want)
    # equals K1c with f32 partials holding the same (bf16-exact) values
    f1, f2 = bf16_to_f32(p1), bf16_to_f32(p2)
    assert np.array_equal(O.land_add2(f1, f2, pr, two, B), want)


# ---------------------------------------------------------------- rms / land
def _rms_f64(x, gamma, eps=1e-5):
    m = bf16_to_f32(x).astype(np.float64)
    r = 1.0 / np.sqrt((m * m).mean(axis=-1, keepdims=True) + eps)
    y = to_bf16((m * r).astype(np.float32))
    return to_bf16(bf16_to_f32(y) * bf16_to_f32(gamma))


@pytest.mark.parametrize("h", [3584, 7168, 12, 1000, 16392, 40000])
def test_rms_against_float64(h):
    g = rng(340 + h)
    B = 6
    x = normal_bf16(g, (B, h))
    gamma = normal_bf16(g, (h,), 1.0, 0.1)
    d = ulp_diff_bf16(O.rms(x, gamma, h, B), _rms_f64(x, gamma))
    assert d.max() <= 1 and (d > 0).mean() < 2e-3


def test_rms_outlier_row_and_zero_row():
    h, B = 3584, 2
    g = rng(349)
    x = normal_bf16(g, (B, h))
    x[1] = 0
    x[0, 17] = to_bf16(np.array([3000.0], np.float32))[0]
    gamma = normal_bf16(g, (h,), 1.0, 0.1)
    got = O.rms(x, gamma, h, B)
    assert not got[1].any()  # 0 * r = 0
    d = ulp_diff_bf16(got, _rms_f64(x, gamma))
    assert d.max() <= 1


@pytest.mark.parametrize("n,off,ldc", [(3584, 0, 3584), (1000, 24, 2048), (1001, 3, 1010)])
def test_land_against_torch(n, off, ldc):
    g = rng(350 + n)
    B = 4
    p = g.standard_normal((B, ldc), dtype=np.float32) * np.float32(3.0)
    want = to_bf16(p[:, off:off + n])
    assert np.array_equal(O.land(p, n, off, ldc, B), want)


# ---------------------------------------------------------------- SiTU
def _situ_f64(g, u):
    g = g.astype(np.float64)
    uy = (u.astype(np.float32) * np.float32(0.04)).astype(np.float64)
    with np.errstate(over="ignore"):
        gate = 4.0 * np.tanh(g / 4.0) / (1.0 + np.exp(-g))
    return (gate * 25.0 * np.tanh(uy)).astype(np.float32)


def test_situ_closed_form():
    g = rng(360)
    a = (g.standard_normal(200000) * 4.0).astype(np.float32)
    b = (g.standard_normal(200000) * 40.0).astype(np.float32)
    got = O.situ(a, b)
    want = _situ_f64(a, b)
    assert np.allclose(got, want, rtol=2e-7, atol=1e-30)
    # special values: odd in u, zero at g = 0 or u = 0, limits at g -> +-inf
    assert np.array_equal(O.situ(a, -b), -got)
    assert not O.situ(np.zeros(8, np.float32), b[:8]).any()
    assert not O.situ(a[:8], np.zeros(8, np.float32)).any()
    inf = np.float32(np.inf)
    lim = O.situ(np.array([inf, -inf], np.float32), np.array([1e6, 1e6], np.float32))
    assert lim[0] == np.float32(100.0) and lim[1] == 0.0
    assert np.isnan(O.situ(np.array([np.nan], np.float32), np.array([1.0], np.float32)))[0]


@pytest.mark.parametrize("kind", ["f32", "bf16"])
def test_land_situ_lands_operands_first(kind):
    g = rng(370)
    B, n = 3, 1024
    if kind == "f32":
        p = (g.standard_normal((B, 2 * n)) * 3.0).astype(np.float32)
        ops = bf16_to_f32(to_bf16(p))
    else:
        p = normal_bf16(g, (B, 2 * n), std=3.0)
        ops = bf16_to_f32(p)
    want = to_bf16(_situ_f64(ops[:, :n], ops[:, n:]))
    got = O.land_situ(p, n, B)
    d = ulp_diff_bf16(got, want)
    assert d.max() <= 1 and (d > 0).mean() < 1e-3


def test_situ_rms_is_land_situ_plus_rms():
    """The fused job layout computes the bf16 SiTU landing and kern_k3_rms: at
    h = 3584 (448 vectors) the 512-thread rms job's reduction equals the
    1024-thread one bit for bit (the extra warps add zeros)."""
    g = rng(380)
    tokens, n, h = 64, 6144, 3584
    B = L = tokens // 4
    sp = normal_bf16(g, (B, 2 * n), std=2.0)
    lat = normal_bf16(g, (L, h))
    gam = normal_bf16(g, (h,), 1.0, 0.1)
    act, ln = O.situ_rms(sp, lat, gam, n, B, h, L, tokens)
    assert np.array_equal(act, O.land_situ(sp, n, B))
    assert np.array_equal(ln, O.rms(lat, gam, h, L))
    # rows past the grid's cover are untouched; h % 8 != 0 stores no rms rows
    act2, ln2 = O.situ_rms(sp, lat, gam, n, B, h, L, 16)
    assert np.array_equal(act2[:4], act[:4]) and not act2[4:].any() and not ln2[4:].any()
    _, ln3 = O.situ_rms(sp[:, :24], lat[:, :12], gam[:12], 12, B, 12, L, tokens)
    assert not ln3.any()
