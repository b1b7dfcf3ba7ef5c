"""CPU checks of the benchmark input generator (k3h_synth_normal): bit for bit
against a pure-Python restatement of splitmix64 -> xoshiro256** -> Box-Muller ->
f32 -> bf16 (small n, with outliers), the published xoshiro256** output for a
fixed state, and the sample statistics of a large draw."""
import math
import struct

import numpy as np
import torch

import k3h

MASK = (1 << 64) - 1


def _fnv1a64(s):
    h = 0xcbf29ce484222325
    for ch in s.encode():
        h = ((h ^ ch) * 0x100000001b3) & MASK
    return h


class _Xo:
    def __init__(self, seed):
        self.s = []
        x = seed
        for _ in range(4):
            x = (x + 0x9e3779b97f4a7c15) & MASK
            z = x
            z = ((z ^ (z >> 30)) * 0xbf58476d1ce4e5b9) & MASK
            z = ((z ^ (z >> 27)) * 0x94d049bb133111eb) & MASK
            self.s.append(z ^ (z >> 31))

    @staticmethod
    def _rotl(x, k):
        return ((x << k) | (x >> (64 - k))) & MASK

    def next(self):
        s = self.s
        r = (self._rotl((s[1] * 5) & MASK, 7) * 9) & MASK
        t = (s[1] << 17) & MASK
        s[2] ^= s[0]
        s[3] ^= s[1]
        s[1] ^= s[2]
        s[0] ^= s[3]
        s[2] ^= t
        s[3] = self._rotl(s[3], 45)
        return r

    def uniform(self):
        return (self.next() >> 11) * 2.0 ** -53


class _Normal:
    def __init__(self, seed):
        self.x, self.spare = _Xo(seed), None

    def next(self):
        if self.spare is not None:
            v, self.spare = self.spare, None
            return v
        u1, u2 = self.x.uniform(), self.x.uniform()
        r = math.sqrt(-2.0 * math.log(1.0 - u1))
        a = 6.283185307179586476925 * u2
        self.spare = r * math.sin(a)
        return r * math.cos(a)


def _bf16(f32):
    u = struct.unpack("<I", struct.pack("<f", f32))[0]
    u = (u + 0x7fff + ((u >> 16) & 1)) & 0xffffffff
    return u >> 16


def _reference(name, n, mean, std, p, big):
    seed = lambda suf: 24301 ^ _fnv1a64(name + suf)
    g, pick, out_n = _Normal(seed("")), _Xo(seed("#bernoulli")), _Normal(seed("#outlier"))
    out = []
    for _ in range(n):
        v = mean + std * g.next()
        if p > 0 and pick.uniform() < p:
            v = big * out_n.next()
        out.append(_bf16(struct.unpack("<f", struct.pack("<f", v))[0]))
    return np.array(out, np.uint16)


def test_xoshiro_published_output():
    x = _Xo(0)
    x.s = [1, 2, 3, 4]
    assert x.next() == 11520          # rotl(2 * 5, 7) * 9
    assert x.next() == 0
    assert x.next() == 1509978240


def test_generator_matches_restatement():
    for name, n, mean, std, p in (("2/x", 2000, 0.0, 1.0, 0.05), ("2/gamma", 700, 1.0, 0.1, 0.0)):
        got = k3h.synth_normal(name, (n,), mean, std, p, 50.0).view(torch.int16).numpy().view(np.uint16)
        want = _reference(name, n, mean, std, p, 50.0)
        assert np.array_equal(got, want), name


def test_generator_statistics_and_f32():
    x = k3h.synth_normal("2/residual", (1 << 20,)).float().numpy().astype(np.float64)
    assert abs(x.mean()) < 5e-3 and abs(x.std() - 1.0) < 5e-3
    y = k3h.synth_normal("2/x", (1 << 20,), outlier_p=0.001).float().numpy()
    frac = (np.abs(y) > 6.0).mean()
    assert 0.0006 < frac < 0.0012     # about 0.1% x 50 outliers (|50 z| > 6 nearly always)
    b = k3h.synth_normal("5/bias", (4096,), std=0.01, dtype=torch.float32).numpy()
    assert b.dtype == np.float32 and abs(b.std() - 0.01) < 1e-3
    assert k3h.synth_normal("5/bias", (8,), std=0.01, dtype=torch.float32).tolist() == b[:8].tolist()
