"""GPU parity: per-tensor fp8 pair (v1 and v2 modules) against the C oracle,
bit-exact for the partials, the scale and every e4m3 byte."""
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


@pytest.mark.parametrize("v2", [True, False])
@pytest.mark.parametrize("n,nb", [(16384 * 7168, 2048), (7168 * 40 + 5, 64), (13, 4), (4096, 2048)])
def test_quant_fp8_tensor(ctx, v2, n, nb):
    print(f"[case] quant_fp8_tensor v2={v2} n={n} nb={nb}", flush=True)
    g = rng(1100 + n % 97)
    x = normal_bf16(g, (n,), outlier_p=0.001)
    want_p = O.quant_fp8_amax(x, n, nb, v2=v2)
    want_y, want_s = O.quant_fp8_apply(x, n, want_p, nb)
    xd = to_dev(x)
    y = torch.empty(n + 8, dtype=torch.uint8, device="cuda")
    s = torch.empty(1, dtype=torch.float32, device="cuda")
    p = torch.empty(nb, dtype=torch.float32, device="cuda")
    ctx.quant_fp8_tensor(xd, y, s, p, n, v2=v2)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(p), want_p)
    assert from_dev(s)[0] == want_s[0]
    assert np.array_equal(from_dev(y)[:n], want_y)


@pytest.mark.parametrize("v2", [True, False])
def test_quant_fp8_tensor_nan(ctx, v2):
    """NaN inputs of either sign: v1 partials ignore them, v2 partials take the
    |bf16| pattern maximum (a NaN partial, compared as bits), the scale comes
    from the non-NaN partials, and each NaN gives the canonical e4m3 NaN 0x7f."""
    n, nb = 7168 * 8 + 3, 64
    print(f"[case] quant_fp8_tensor NaN v2={v2}", flush=True)
    g = rng(1150)
    x = normal_bf16(g, (n,), outlier_p=0.001)
    nan_at = [5, 1000, 30000, n - 1]
    x[nan_at] = [0x7FC0, 0xFFC1, 0x7F81, 0xFFFF]
    want_p = O.quant_fp8_amax(x, n, nb, v2=v2)
    want_y, want_s = O.quant_fp8_apply(x, n, want_p, nb)
    y = torch.empty(n + 8, dtype=torch.uint8, device="cuda")
    s = torch.empty(1, dtype=torch.float32, device="cuda")
    p = torch.empty(nb, dtype=torch.float32, device="cuda")
    ctx.quant_fp8_tensor(to_dev(x), y, s, p, n, v2=v2)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(p).view(np.uint32), want_p.view(np.uint32))
    assert from_dev(s).view(np.uint32)[0] == want_s.view(np.uint32)[0]
    got_y = from_dev(y)[:n]
    assert np.array_equal(got_y, want_y)
    assert (got_y[nan_at] == 0x7F).all()


def test_quant_fp8_zero_tensor_scale_one(ctx):
    n = 4096
    x = np.zeros(n, np.uint16)
    y = torch.full((n,), 0x55, dtype=torch.uint8, device="cuda")
    s = torch.empty(1, dtype=torch.float32, device="cuda")
    p = torch.empty(16, dtype=torch.float32, device="cuda")
    ctx.quant_fp8_tensor(to_dev(x), y, s, p, n)
    torch.cuda.synchronize()
    assert from_dev(s)[0] == 1.0 and not from_dev(y).any()


def test_quant_fp8_manifest_op(ctx):
    """ops.quant_fp8_tensor of the default manifest (two launches, grid 2048)."""
    ops = json.load(open(os.path.join(GOLDEN, "manifest_hot_ops.json")))
    n = 4096 * 7168
    g = rng(1200)
    x = normal_bf16(g, (n,), outlier_p=0.001)
    y = torch.empty(n, dtype=torch.uint8, device="cuda")
    s = torch.empty(1, dtype=torch.float32, device="cuda")
    p = torch.empty(2048, dtype=torch.float32, device="cuda")
    k3h.ManifestOp(ctx, "quant_fp8_tensor", ops["quant_fp8_tensor"])([to_dev(x), y, s, p, n], {"tokens": 16384})
    torch.cuda.synchronize()
    want_p = O.quant_fp8_amax(x, n, 2048, v2=True)
    want_y, want_s = O.quant_fp8_apply(x, n, want_p, 2048)
    assert np.array_equal(from_dev(p), want_p)
    assert from_dev(s)[0] == want_s[0]
    assert np.array_equal(from_dev(y), want_y)
