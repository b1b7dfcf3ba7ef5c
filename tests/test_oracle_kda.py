"""Pins the KDA span-gather and output-gate oracles: float64 conv / RMS / SiLU
restatements (within one bf16 ulp), exact landing copies, and the window
protocol's defining property -- a span of n rows equals n spans of one row."""
import numpy as np
import pytest
import torch

import oracle as O
from k3data import bf16_to_f32, normal_bf16, rng, to_bf16, ulp_diff_bf16

HEADS, INNER = 24, 3072


def _inputs(rows, seed):
    g = rng(seed)
    partial = normal_bf16(g, (rows, 4 * INNER))
    cw = bf16_to_f32(normal_bf16(g, (3, 4, INNER), 0.0, 0.5))  # bf16-representable taps
    win = normal_bf16(g, (3, 3, INNER))
    wsm = g.standard_normal((rows, 256), dtype=np.float32)
    return partial, cw, win, wsm


def test_span_gather_against_float64_definition():
    rows, at, span = 40, 5, 30
    partial, cw, win, wsm = _inputs(rows, 200)
    q, k, v, beta, flow, nw = O.span_gather(partial, cw, win, wsm, at, span)
    for s, out in enumerate((q, k, v)):
        x = np.concatenate([bf16_to_f32(win[s]), bf16_to_f32(partial[at:at + span, s * INNER:(s + 1) * INNER])]).astype(np.float64)
        y = sum(x[t:t + span] * cw[s, t].astype(np.float64) for t in range(4))
        sb = bf16_to_f32(to_bf16(y.astype(np.float32))).astype(np.float64)
        want = to_bf16((sb / (1.0 + np.exp(-sb))).astype(np.float32))
        d = ulp_diff_bf16(out, want)
        assert d.max() <= 1 and (d > 0).mean() < 2e-3, (s, d.max(), (d > 0).mean())
        # the window leaves holding the span's last three inputs
        assert np.array_equal(nw[s], partial[at + span - 3:at + span, s * INNER:(s + 1) * INNER])
    tb = lambda a: torch.from_numpy(a).bfloat16().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(beta.reshape(HEADS, span), tb(np.ascontiguousarray(wsm[at:at + span, :HEADS].T)))
    assert np.array_equal(flow, tb(np.ascontiguousarray(wsm[at:at + span, 96:224])))


def test_span_gather_span_of_n_equals_n_steps():
    rows, at, span = 24, 2, 19
    partial, cw, win, wsm = _inputs(rows, 201)
    q, k, v, _, _, nw = O.span_gather(partial, cw, win, wsm, at, span)
    w = win.copy()
    for i in range(span):
        qi, ki, vi, _, _, w = O.span_gather(partial, cw, w, wsm, at + i, 1)
        assert np.array_equal(qi[0], q[i]) and np.array_equal(ki[0], k[i]) and np.array_equal(vi[0], v[i])
    assert np.array_equal(w, nw)
    # a span shorter than the window keeps old window rows
    _, _, _, _, _, w2 = O.span_gather(partial, cw, win, wsm, at, 2)
    assert np.array_equal(w2[:, 0], win[:, 2])


@pytest.mark.parametrize("eps", [1e-5, 1e-6])
def test_kda_out_gate_against_float64(eps):
    """Against the float64 definition at both compiled eps values; a third of the
    heads have amplitude 1e-3 (mean square ~1e-6), where the eps term sets the
    norm, so a wrong eps fails."""
    rows, at, span = 20, 3, 12
    g = rng(210)
    attn = normal_bf16(g, (span, INNER))
    a32 = bf16_to_f32(attn).reshape(span, HEADS, 128)
    a32[:, ::3] *= np.float32(1e-3)
    attn = to_bf16(a32.reshape(span, INNER))
    gate = normal_bf16(g, (rows, 4 * INNER))
    gamma_o = (1.0 + 0.1 * g.standard_normal(128)).astype(np.float32)
    gated = O.kda_out_gate(attn, gate, gamma_o, np.zeros((rows, INNER), np.uint16), at, span, eps=eps)
    a = bf16_to_f32(attn).astype(np.float64).reshape(span, HEADS, 128)
    gg = bf16_to_f32(gate[at:at + span, 3 * INNER:]).astype(np.float64).reshape(span, HEADS, 128)
    gt = bf16_to_f32(to_bf16((1.0 / (1.0 + np.exp(-gg))).astype(np.float32))).astype(np.float64)

    def ref(e):
        r = 1.0 / np.sqrt((a * a).mean(-1, keepdims=True) + e)
        o = bf16_to_f32(to_bf16((a * r * gamma_o).astype(np.float32))).astype(np.float64)
        return to_bf16((o * gt).reshape(span, INNER).astype(np.float32))

    d = ulp_diff_bf16(gated[at:at + span], ref(eps))
    assert d.max() <= 1 and (d > 0).mean() < 2e-3
    other = ulp_diff_bf16(gated[at:at + span], ref(1e-5 if eps == 1e-6 else 1e-6))
    assert (other > 1).mean() > 0.1, "eps does not reach the result"
    assert not gated[:at].any() and not gated[at + span:].any()
