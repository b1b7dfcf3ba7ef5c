"""Pins the oracle's numeric primitives against independent implementations:
torch's bf16 / float8_e4m3fn casts, a brute-force nearest-value search, the
float64 exponential, and the exact ceil(log2(.)) definition of the E8M0 scale."""
import math

import numpy as np
import pytest
import torch

import oracle as O
from k3data import bf16_to_f32, rng


def _f32(bits):
    return np.asarray(bits, np.uint32).view(np.float32)


def test_bf16_rne_matches_torch_random_and_ties():
    g = rng(1)
    bits = g.integers(0, 2**32, 200000, dtype=np.uint64).astype(np.uint32)
    # exact ties (low half 0x8000) with even and odd kept halves, and near-ties
    ties = (g.integers(0, 2**16, 20000, dtype=np.uint32) << 16) | 0x8000
    near = (g.integers(0, 2**16, 20000, dtype=np.uint32) << 16) | 0x7fff
    bits = np.concatenate([bits, ties, near, ties + 1])
    x = _f32(bits)
    x = x[np.isfinite(x)]
    got = O.f32_to_bf16(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def test_bf16_to_f32_is_exact_widening():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = bf16_to_f32(h)
    fin = np.isfinite(f)
    assert np.array_equal(O.f32_to_bf16(f[fin]), h[fin])


def _torch_e4m3(x: np.ndarray) -> np.ndarray:
    """torch float8_e4m3fn cast (RNE) after saturating to +-448."""
    t = torch.from_numpy(np.clip(x, -448.0, 448.0).astype(np.float32))
    return t.to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_matches_torch_over_all_bf16_and_scales():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    base = bf16_to_f32(h)
    base = base[~np.isnan(base)]
    for s in [1.0, 2.0**-8, 2.0**-4, 2.0**4, 2.0**8, 2.0**-120, 2.0**100, 0.7]:
        x = (base * np.float32(s)).astype(np.float32)
        got = O.e4m3(x)
        want = _torch_e4m3(x)
        # torch keeps the sign of +-0 like the OCP encoder; inf saturates after clip
        assert np.array_equal(got, want), f"scale {s}"


def _e4m3_table():
    vals = []
    for c in range(256):
        e, m = (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            continue
        v = math.ldexp(m, -9) if e == 0 else math.ldexp(8 + m, e - 10)
        vals.append((-v if c & 0x80 else v, c))
    return vals


def test_e4m3_bruteforce_nearest_even():
    table = _e4m3_table()
    pos = sorted((v, c) for v, c in table if c < 0x80)
    g = rng(2)
    xs = np.concatenate([
        g.uniform(-460, 460, 4000), g.uniform(-1, 1, 4000) * 2.0**-6,
        np.array([v for v, _ in pos]) * 1.0,                       # exact codes
        np.array([(a[0] + b[0]) / 2 for a, b in zip(pos, pos[1:])]),  # exact midpoints
    ]).astype(np.float32)
    got = O.e4m3(xs)
    for x, c in zip(xs.tolist(), got.tolist()):
        a = abs(x)
        if a >= 448.0:
            want = 0x7e
        else:
            best = min(pos, key=lambda vc: (abs(vc[0] - a), vc[1] & 1))
            want = best[1]
        if math.copysign(1.0, x) < 0:
            want |= 0x80
        assert c == want, (x, hex(c), hex(want))


def test_e4m3_decode_encode_roundtrip_and_nan():
    codes = np.array([c for c in range(256) if (c & 0x7f) != 0x7f], np.uint8)
    vals = O.e4m3_decode(codes)
    assert np.array_equal(O.e4m3(vals), codes)
    assert O.e4m3(np.array([np.nan], np.float32))[0] & 0x7f == 0x7f
    assert O.e4m3(np.array([np.inf, -np.inf, 1e30, -1e30], np.float32)).tolist() == [0x7e, 0xfe, 0x7e, 0xfe]


def test_expf_within_two_ulp_of_float64():
    x = np.concatenate([np.linspace(-87.0, 88.7, 400001, dtype=np.float32),
                        rng(3).uniform(-20, 20, 100000).astype(np.float32)])
    got = O.expf(x).astype(np.float64)
    want = np.exp(x.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    err = np.abs(got - want) / ulp
    assert err.max() <= 2.0, err.max()
    assert O.expf(np.zeros(1, np.float32))[0] == 1.0


def test_mx_exponent_closed_form_all_bf16():
    """ceil(log2(amax/448)) (the reference's formula) equals E - 8 + (M > 1.75)
    clamped to [-127, 127] for every positive finite bf16 -- the integer form the
    GPU kernels use."""
    h = np.arange(1, 0x7f80, dtype=np.uint32)
    amax = bf16_to_f32(h.astype(np.uint16))
    got = np.array([O.mx_exp(float(a)) for a in amax])
    E = (h >> 7).astype(np.int64) - 127
    closed = np.clip(E - 8 + ((h & 0x7f) > 0x60), -127, 127)
    assert np.array_equal(got, closed)
    # and the float formula evaluated by numpy in f32 / f64
    q = (amax / np.float32(448.0)).astype(np.float32)
    ref = np.clip(np.ceil(np.log2(q.astype(np.float64))), -127, 127).astype(np.int64)
    assert np.array_equal(got, ref)
    assert O.mx_exp(0.0) == 0 and O.mx_exp(float("inf")) == 127


@pytest.mark.parametrize("x", [0.0, 1.0, -1.0, 10.0, -10.0, 80.0, -80.0, -88.0, -88.8, -100.0, 100.0])
def test_sigmoid_matches_f32_definition(x):
    """1 / (1 + e^-x) evaluated with an f32 e^-x (inf once it overflows f32)."""
    L = O.lib()
    got = L.k3o_sigmoid(x)
    e = np.float32(math.exp(-x)) if -x < 89 else np.float32(np.inf)
    want = float(np.float32(1.0) / (np.float32(1.0) + e))
    assert abs(got - want) <= 2 * float(np.spacing(np.float32(want))), (got, want)
