"""CPU pins of the MoE expert GEMM oracle (oracle/k3_oracle_gemm.c).

The reference's moe_fc1 / moe_fc2 are prebuilt binaries that cannot run here,
so the oracle restates the mathematics of an MX block-scaled product; these
tests pin it against independent statements of the same mathematics:
* e2m1 decoding against the OCP FP4 value table;
* the product against a float64 numpy matmul whose e4m3 operands are decoded by
  torch's float8_e4m3fn (not the oracle's decoder) and whose scales are applied
  as powers of two;
* the route_map gather against the product of explicitly gathered rows;
* the general-alpha/beta activation against the K3 landing's SiTU (alpha 4,
  beta 25) bit for bit and against a float64 numpy formula otherwise;
* the fc1 epilogue against the composition of the pinned landing SiTU
  (gate | up operand order) and the pinned MX quantiser."""
import numpy as np
import pytest
import torch

import oracle as O
from k3data import normal_bf16, rng

FP4 = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6, -0.0, -0.5, -1, -1.5, -2, -3, -4, -6])


def test_e2m1_table():
    assert np.array_equal(O.e2m1_decode(np.arange(16)), FP4.astype(np.float32))


def _mx_inputs(g, rows, E, N, K):
    x = normal_bf16(g, (rows, K), outlier_p=0.01)
    q, sf = O.moe_quant(x, rows, K)
    w = g.integers(0, 256, (E, N, K // 2), dtype=np.uint8)
    wsf = g.integers(118, 134, (E, N, K // 32)).astype(np.uint8)
    return q, sf, w, wsf


def _dequant_np(q, sf, w, wsf):
    a = torch.from_numpy(q.copy()).view(torch.float8_e4m3fn).double().numpy()
    a = a * np.exp2(np.repeat(sf.astype(np.float64) - 127, 32, axis=1))
    lo, hi = w & 15, w >> 4
    nib = np.stack([lo, hi], -1).reshape(w.shape[0], w.shape[1], -1)
    wd = FP4[nib] * np.exp2(np.repeat(wsf.astype(np.float64) - 127, 32, axis=2))
    return a, wd


def test_gemm_matches_numpy_float64():
    g = rng(7001)
    E, N, K = 3, 64, 256
    q, sf, w, wsf = _mx_inputs(g, 256, E, N, K)
    cta = np.array([2, 0], np.int32)
    got = O.moe_gemm_mx(q, sf, None, w, wsf, 2, cta, E, N, K)
    a, wd = _dequant_np(q, sf, w, wsf)
    want = np.concatenate([a[:128] @ wd[2].T, a[128:] @ wd[0].T])
    assert np.allclose(got, want, rtol=1e-12, atol=0)
    mag = O.moe_gemm_mx(q, sf, None, w, wsf, 2, cta, E, N, K, magnitude=True)
    assert np.allclose(mag, np.concatenate([np.abs(a[:128]) @ np.abs(wd[2]).T,
                                            np.abs(a[128:]) @ np.abs(wd[0]).T]), rtol=1e-12)


def test_gemm_gather_and_skipped_tiles():
    g = rng(7002)
    E, N, K = 2, 32, 128
    q, sf, w, wsf = _mx_inputs(g, 300, E, N, K)
    rows = g.integers(0, 300, 3 * 128).astype(np.int32)
    rows[5] = -1  # treated as token 0
    cta = np.array([1, 5, 0], np.int32)  # tile 1 has no such expert: left untouched
    got = O.moe_gemm_mx(q, sf, rows, w, wsf, 3, cta, E, N, K)
    src = np.where(rows < 0, 0, rows)
    plain = O.moe_gemm_mx(np.ascontiguousarray(q[src]), np.ascontiguousarray(sf[src]), None, w, wsf,
                          3, np.array([1, 1, 0], np.int32), E, N, K)
    assert np.array_equal(got[:128], plain[:128]) and np.array_equal(got[256:], plain[256:])
    assert np.isnan(got[128:256]).all()


@pytest.mark.parametrize("alpha,beta", [(4.0, 25.0), (3.0, 20.0), (1.702, 7.0)])
def test_situ_ab(alpha, beta):
    g = rng(7003)
    gv = (g.standard_normal(4096) * 6).astype(np.float32)
    uv = (g.standard_normal(4096) * 40).astype(np.float32)
    got = O.situ_ab(gv, uv, alpha, beta)
    if alpha == 4.0 and beta == 25.0:
        assert np.array_equal(got.view(np.uint32), O.situ(gv, uv).view(np.uint32))
    uy = (uv * np.float32(np.float32(1.0) / np.float32(beta))).astype(np.float64)
    want = (alpha * np.tanh(gv.astype(np.float64) / alpha) / (1 + np.exp(-gv.astype(np.float64)))
            * beta * np.tanh(uy))
    assert np.allclose(got, want.astype(np.float32), rtol=2e-7, atol=1e-30)


def test_fc1_epilogue_is_landing_situ_then_mx_quant():
    g = rng(7004)
    rows, half = 64, 96
    c = (g.standard_normal((rows, 2 * half)) * 8).astype(np.float32)
    q, sf = O.moe_fc1_epilogue(c, np.full(rows, 4.0), np.full(rows, 25.0))
    gate_up = np.ascontiguousarray(np.concatenate([c[:, half:], c[:, :half]], 1))
    act = O.land_situ(gate_up, half, rows)
    q2, sf2 = O.moe_quant(act, rows, half)
    assert np.array_equal(q, q2) and np.array_equal(sf, sf2)
