"""Seeded synthetic inputs for the tests (numpy; bf16 as uint16 bit patterns).

bf16 rounding of the generated f32 values goes through torch's CPU cast, which
is independent of the oracle's encoder."""
import numpy as np
import torch

H = 7168


def rng(seed: int) -> np.random.Generator:
    return np.random.default_rng(seed)


def to_bf16(x: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16).copy()


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)


def normal_bf16(g: np.random.Generator, shape, mean=0.0, std=1.0, outlier_p=0.0, outlier_x=50.0):
    x = g.standard_normal(shape, dtype=np.float32) * np.float32(std) + np.float32(mean)
    if outlier_p > 0:
        m = g.random(shape) < outlier_p
        x[m] = g.standard_normal(int(m.sum()), dtype=np.float32) * np.float32(outlier_x)
    return to_bf16(x)


def to_dev(a: np.ndarray, dtype=None):
    """numpy -> torch GPU tensor; uint16 arrays become bfloat16."""
    t = torch.from_numpy(np.ascontiguousarray(a))
    if a.dtype == np.uint16:
        t = t.view(torch.int16).view(torch.bfloat16)
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def from_dev(t) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy()
    return t.numpy()


def ulp_diff_bf16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in bf16 ulps between bit patterns (monotone integer map)."""
    def key(h):
        h = h.astype(np.int32)
        return np.where(h & 0x8000, -(h & 0x7fff), h & 0x7fff)
    return np.abs(key(a) - key(b))
