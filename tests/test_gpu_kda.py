"""GPU parity: KDA span gather (conv + SiLU, beta/flow landing, window update)
and output gate (per-head RMS x gamma_o x sigmoid gate) against the C oracle.
Bar: landing copies and the window bit-exact; conv/SiLU and gate outputs within
one bf16 ulp (the kernels use the hardware 2^x / reciprocal logistic, the
checker the exact one), with the differing fraction reported and bounded."""
import json
import os

import numpy as np
import pytest
import torch

import k3h
import oracle as O
from k3data import bf16_to_f32, from_dev, normal_bf16, rng, to_bf16, to_dev, ulp_diff_bf16

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
HEADS, INNER = 24, 3072
LINE_BYTES = 1628160
REC_BYTES = HEADS * 128 * 128 * 4
WIN_BYTES = 3 * INNER * 2


def _case(m):
    print(f"[case] {m}", flush=True)


def _close1(name, got, want, frac=2e-3):
    d = ulp_diff_bf16(np.asarray(got), np.asarray(want))
    print(f"  {name}: max ulp {d.max()}, differing {(d > 0).mean():.2e}", flush=True)
    assert d.max() <= 1 and (d > 0).mean() < frac, name


class Span:
    """Device buffers of one span_gather call over `rows` batch rows; the KDA
    state holds 3 lines and the span's windows live in line `line`."""

    def __init__(self, rows, seed, line=1):
        g = rng(seed)
        self.partial = normal_bf16(g, (rows, 4 * INNER))
        self.cw = bf16_to_f32(normal_bf16(g, (3, 4, INNER), 0.0, 0.5))
        self.win = normal_bf16(g, (3, 3, INNER))
        self.wsm = g.standard_normal((rows, 256), dtype=np.float32)
        self.line = line
        state = g.integers(0, 256, 3 * LINE_BYTES, dtype=np.uint8)
        off = line * LINE_BYTES + REC_BYTES
        state[off:off + 3 * WIN_BYTES] = self.win.reshape(-1).view(np.uint8)
        self.state0 = state
        self.d_state = to_dev(state)
        self.d_partial, self.d_cw, self.d_wsm = to_dev(self.partial), to_dev(self.cw), to_dev(self.wsm)
        self.d_line = to_dev(np.full(rows, line, np.int32))

    def window(self):
        st = from_dev(self.d_state)
        off = self.line * LINE_BYTES + REC_BYTES
        return st[off:off + 3 * WIN_BYTES].view(np.uint16).reshape(3, 3, INNER), st

    def run(self, ctx, at, span):
        outs = [torch.empty((span, INNER), dtype=torch.bfloat16, device="cuda") for _ in range(3)]
        beta = torch.empty(HEADS * span, dtype=torch.bfloat16, device="cuda")
        flow = torch.empty((span, 128), dtype=torch.bfloat16, device="cuda")
        ctx.span_gather(self.d_partial, self.d_cw, self.d_state, self.d_line, LINE_BYTES, self.d_wsm,
                        *outs, beta, flow, to_dev(np.array([at], np.int32)), span)
        torch.cuda.synchronize()
        return [from_dev(o) for o in outs] + [from_dev(beta), from_dev(flow)]


# spans cover the typed call's tile pairs: whole pairs (32, 16384), a pair whose
# second tile is partial (17, 45) or past the span (65), and spans under 3 rows
@pytest.mark.parametrize("rows,at,span", [(16384, 0, 16384), (100, 7, 45), (10, 4, 2), (40, 0, 17),
                                          (40, 3, 32), (80, 5, 65), (8, 6, 1)])
def test_span_gather(ctx, rows, at, span):
    _case(f"span_gather rows={rows} at={at} span={span}")
    sp = Span(rows, 2000 + span)
    q, k, v, beta, flow, nw = O.span_gather(sp.partial, sp.cw, sp.win, sp.wsm, at, span)
    got = sp.run(ctx, at, span)
    for nm, gq, wq in zip("qkv", got[:3], (q, k, v)):
        _close1(f"span_{nm}", gq, wq)
    assert np.array_equal(got[3], beta) and np.array_equal(got[4], flow)
    win, st = sp.window()
    assert np.array_equal(win, nw)
    off = sp.line * LINE_BYTES + REC_BYTES
    rest = np.ones(st.size, bool)
    rest[off:off + 3 * WIN_BYTES] = False
    assert np.array_equal(st[rest], sp.state0[rest]), "span_gather wrote outside the window"


def test_span_gather_split_spans_match_one_span(ctx):
    """Window protocol on the GPU: spans 16 + 1 + 23 continue exactly as one span of 40."""
    _case("span_gather split spans")
    a = Span(48, 2100)
    one = a.run(ctx, 3, 40)
    w_one, _ = a.window()
    b = Span(48, 2100)
    parts, at = [], 3
    for n in (16, 1, 23):
        parts.append(b.run(ctx, at, n))
        at += n
    w_split, _ = b.window()
    for j in range(3):
        assert np.array_equal(np.concatenate([p[j] for p in parts]), one[j])
    assert np.array_equal(w_split, w_one)


@pytest.mark.parametrize("rows,at,span,eps,tiny", [
    (16384, 0, 16384, 1e-6, False),   # config 3b as stated: eps 1e-6, attn ~N(0,1)
    (16384, 0, 16384, 1e-5, False),
    (50, 9, 33, 1e-6, True),          # heads of amplitude 1e-3: the norm's eps sets the result
    (50, 9, 33, 1e-5, True),
])
def test_kda_out_gate(ctx, rows, at, span, eps, tiny):
    _case(f"kda_out_gate rows={rows} at={at} span={span} eps={eps} tiny={tiny}")
    g = rng(2200 + span)
    attn = normal_bf16(g, (span, INNER))
    if tiny:
        a = bf16_to_f32(attn).reshape(span, HEADS, 128)
        a[:, ::3] *= np.float32(1e-3)
        attn = to_bf16(a.reshape(span, INNER))
    gate = normal_bf16(g, (rows, 4 * INNER))
    gamma_o = (1.0 + 0.1 * g.standard_normal(128)).astype(np.float32)
    want = O.kda_out_gate(attn, gate, gamma_o, np.zeros((rows, INNER), np.uint16), at, span, eps=eps)
    gated = torch.zeros((rows, INNER), dtype=torch.bfloat16, device="cuda")
    ctx.kda_out_gate(to_dev(attn), to_dev(gate), to_dev(gamma_o), gated,
                     to_dev(np.array([at], np.int32)), span, eps=eps)
    torch.cuda.synchronize()
    got = from_dev(gated)
    _close1("gated", got[at:at + span], want[at:at + span])
    assert not got[:at].any() and not got[at + span:].any()
    if tiny:
        other = O.kda_out_gate(attn, gate, gamma_o, np.zeros((rows, INNER), np.uint16), at, span,
                               eps=1e-5 if eps == 1e-6 else 1e-6)
        assert (ulp_diff_bf16(got[at:at + span], other[at:at + span]) > 1).mean() > 0.1, \
            "the other eps's module would have passed: eps not exercised"


def test_kda_out_gate_rejects_other_eps(ctx):
    with pytest.raises(ValueError, match="invalid argument"):
        z = torch.zeros(4 * INNER, dtype=torch.bfloat16, device="cuda")
        ctx.kda_out_gate(z, z, torch.ones(128, device="cuda"), z, to_dev(np.array([0], np.int32)),
                         1, eps=1e-4)


@pytest.mark.parametrize("span", [1000, 2048])
def test_span_gather_manifest_geometry_matches_typed(ctx, span):
    """The entry under the manifest's (INNER/512, 4, ceil(span/16)) x 128 grid (one
    16-row tile per workgroup) and under the typed call's 256-thread workgroups
    (two tiles, taps handed over in LDS) produce the same bits."""
    ops = json.load(open(os.path.join(GOLDEN, "manifest_hot_ops.json")))
    _case(f"span_gather manifest vs typed geometry span={span}")
    a, b = Span(span + 2, 2400 + span), Span(span + 2, 2400 + span)
    typed = a.run(ctx, 2, span)
    outs = [torch.empty((span, INNER), dtype=torch.bfloat16, device="cuda") for _ in range(3)]
    beta = torch.empty(HEADS * span, dtype=torch.bfloat16, device="cuda")
    flow = torch.empty((span, 128), dtype=torch.bfloat16, device="cuda")
    k3h.ManifestOp(ctx, "span_gather_v2", ops["span_gather_v2"])(
        [b.d_partial, b.d_cw, b.d_state, b.d_line, b.d_wsm, *outs, beta, flow,
         to_dev(np.array([2], np.int32)), span], {"tokens": span})
    torch.cuda.synchronize()
    man = [from_dev(o) for o in outs] + [from_dev(beta), from_dev(flow)]
    for j in range(5):
        assert np.array_equal(typed[j], man[j]), j
    assert np.array_equal(a.window()[1], b.window()[1])


def test_manifest_kda_ops(ctx):
    ops = json.load(open(os.path.join(GOLDEN, "manifest_hot_ops.json")))
    tokens = 64
    env = {"tokens": tokens}
    _case("manifest span_gather_v2")
    sp = Span(tokens, 2300)
    outs = [torch.empty((tokens, INNER), dtype=torch.bfloat16, device="cuda") for _ in range(3)]
    beta = torch.empty(HEADS * tokens, dtype=torch.bfloat16, device="cuda")
    flow = torch.empty((tokens, 128), dtype=torch.bfloat16, device="cuda")
    at_d = to_dev(np.array([0], np.int32))
    k3h.ManifestOp(ctx, "span_gather_v2", ops["span_gather_v2"])(
        [sp.d_partial, sp.d_cw, sp.d_state, sp.d_line, sp.d_wsm, *outs, beta, flow, at_d, tokens], env)
    torch.cuda.synchronize()
    q, k, v, wb, wf, nw = O.span_gather(sp.partial, sp.cw, sp.win, sp.wsm, 0, tokens)
    for nm, o, w in zip("qkv", outs, (q, k, v)):
        _close1(f"span_{nm}", from_dev(o), w)
    assert np.array_equal(from_dev(beta), wb) and np.array_equal(from_dev(flow), wf)
    assert np.array_equal(sp.window()[0], nw)
    _case("manifest kda_out_gate_v2")
    g = rng(2301)
    attn = normal_bf16(g, (tokens, INNER))
    gamma_o = (1.0 + 0.1 * g.standard_normal(128)).astype(np.float32)
    gated = torch.zeros((tokens, INNER), dtype=torch.bfloat16, device="cuda")
    k3h.ManifestOp(ctx, "kda_out_gate_v2", ops["kda_out_gate_v2"])(
        [to_dev(attn), sp.d_partial, to_dev(gamma_o), gated, at_d, tokens], env)
    torch.cuda.synchronize()
    want = O.kda_out_gate(attn, sp.partial, gamma_o, np.zeros((tokens, INNER), np.uint16), 0, tokens)
    _close1("gated", from_dev(gated), want)


def _special_match(name, got, want):
    """NaN positions and infinities (with sign) identical; finite values within one ulp."""
    gf, wf = bf16_to_f32(np.asarray(got)), bf16_to_f32(np.asarray(want))
    gn, wn = np.isnan(gf), np.isnan(wf)
    assert np.array_equal(gn, wn), f"{name}: NaN positions differ ({gn.sum()} vs {wn.sum()})"
    gi, wi = np.isinf(gf), np.isinf(wf)
    assert np.array_equal(gi, wi) and np.array_equal(np.sign(gf[gi]), np.sign(wf[wi])), \
        f"{name}: infinities differ"
    fin = ~(gn | gi)
    d = ulp_diff_bf16(np.asarray(got)[fin], np.asarray(want)[fin])
    print(f"  {name}: {gn.sum()} NaN, {gi.sum()} inf, finite max ulp {d.max() if d.size else 0}",
          flush=True)
    assert d.size == 0 or d.max() <= 1, name


SPECIALS = np.array([0x7FC0, 0xFFC1, 0x7F80, 0xFF80, 0x7F7F, 0xFF7F, 0x0001, 0x8000], np.uint16)


def test_span_gather_special_values(ctx):
    """NaN (either sign), +-inf, +-max finite, a subnormal and -0 in the q/k/v bands
    and in the carried window: the conv and SiLU propagate them as the oracle does
    (SiLU(-inf) and inf - inf give NaN, SiLU(+inf) = +inf), within one ulp elsewhere;
    the landing copies and the window stay bit-exact."""
    _case("span_gather special values")
    sp = Span(40, 2500)
    g = rng(2501)
    flat = sp.partial.reshape(-1)
    pos = g.choice(flat.size, 64, replace=False)
    flat[pos] = SPECIALS[np.arange(64) % SPECIALS.size]
    w = sp.win.reshape(-1)
    wpos = g.choice(w.size, 16, replace=False)
    w[wpos] = SPECIALS[np.arange(16) % SPECIALS.size]
    off = sp.line * LINE_BYTES + REC_BYTES
    sp.state0[off:off + 3 * WIN_BYTES] = sp.win.reshape(-1).view(np.uint8)
    sp.d_state = to_dev(sp.state0)
    sp.d_partial = to_dev(sp.partial)
    q, k, v, beta, flow, nw = O.span_gather(sp.partial, sp.cw, sp.win, sp.wsm, 2, 33)
    got = sp.run(ctx, 2, 33)
    for nm, gq, wq in zip("qkv", got[:3], (q, k, v)):
        _special_match(f"span_{nm}", gq, wq)
    assert np.array_equal(got[3], beta) and np.array_equal(got[4], flow)
    win, _ = sp.window()
    assert np.array_equal(win, nw)


def test_kda_out_gate_special_values(ctx):
    """NaN and +-inf in attention rows (a NaN or an infinity makes its head's
    sum of squares NaN / inf, so r is NaN / 0) and in the gate (sigmoid(+-inf) =
    1 / 0, NaN stays NaN): positions and values as the oracle's."""
    _case("kda_out_gate special values")
    rows, at, span = 40, 3, 30
    g = rng(2600)
    attn = normal_bf16(g, (span, INNER))
    gate = normal_bf16(g, (rows, 4 * INNER))
    a = attn.reshape(-1)
    a[g.choice(a.size, 24, replace=False)] = SPECIALS[np.arange(24) % SPECIALS.size]
    gb = gate[:, 3 * INNER:].copy().reshape(-1)
    gb[g.choice(gb.size, 24, replace=False)] = SPECIALS[np.arange(24) % SPECIALS.size]
    gate[:, 3 * INNER:] = gb.reshape(rows, INNER)
    gamma_o = (1.0 + 0.1 * g.standard_normal(128)).astype(np.float32)
    want = O.kda_out_gate(attn, gate, gamma_o, np.zeros((rows, INNER), np.uint16), at, span, eps=1e-6)
    gated = torch.zeros((rows, INNER), dtype=torch.bfloat16, device="cuda")
    ctx.kda_out_gate(to_dev(attn), to_dev(gate), to_dev(gamma_o), gated,
                     to_dev(np.array([at], np.int32)), span, eps=1e-6)
    torch.cuda.synchronize()
    got = from_dev(gated)
    _special_match("gated", got[at:at + span], want[at:at + span])
