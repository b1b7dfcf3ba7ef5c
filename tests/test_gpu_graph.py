"""GPU: the k3h launches captured into a HIP graph replay to the eager results.

One prefill-shaped chain (fused residual + RMSNorm + MXFP8, per-tensor fp8 pair,
router top-k, EP routing count / tables / scatter, MXFP8 permute, K1 with
candidate blocks, res_in push to the local and a second "peer" buffer, SiTU
landing on the compact grid) is captured once on torch's capture stream.  Each
replay gets new inputs copied into the graph's static buffers, the same chain is
run eagerly into a second set of outputs, and every output of the replay must
equal the eager one bit for bit.  Outputs are refilled with a sentinel (a torch
fill kernel, outside the graph) before every replay and eager run, so a launch
that the graph dropped shows up as sentinel bytes.  The library issues no
memset or allocation, so nothing but kernel nodes is recorded.  A second graph
holds the arrival barrier that follows the push (epoch bump, a peer's arrival
played by a torch add, the one-wave wait), replayed between eager runs."""
import numpy as np
import pytest
import torch

from k3data import H, normal_bf16, rng, to_bf16

pytestmark = pytest.mark.gpu

T = 512          # tokens
TOPK = 16
E = 56           # local experts of one EP4 rank
RANK = 1
NB = 4           # K1 candidate blocks
N_SITU = 6144
NBLK = (T + 255) // 256
CAP = T * TOPK + E * 128


def _case(msg):
    print(f"[case] {msg}", flush=True)


def _inputs(seed):
    g = rng(seed)
    S = g.standard_normal((T, 224), dtype=np.float32)
    return dict(
        x=normal_bf16(g, (T, H), outlier_p=0.001),
        res=normal_bf16(g, (T, H)),
        gamma=normal_bf16(g, (H,), 1.0, 0.1),
        S=S,
        bias=(g.standard_normal(224) * 0.01).astype(np.float32),
        rs=to_bf16(np.array([2.5], np.float32)),
        partial=normal_bf16(g, (T, H)),
        prefix=normal_bf16(g, (T, H)),
        blocks=normal_bf16(g, (T, 8, H)),
        sw=(g.standard_normal(H) * 0.05).astype(np.float32),
        sp=(g.standard_normal((T, 2 * N_SITU)) * 3.0).astype(np.float32),
    )


def _static_inputs(first):
    out = {}
    for k, a in first.items():
        t = torch.from_numpy(np.ascontiguousarray(a))
        if a.dtype == np.uint16:
            t = t.view(torch.int16).view(torch.bfloat16)
        out[k] = t.cuda()
    return out


def _load(static, host):
    for k, a in host.items():
        t = torch.from_numpy(np.ascontiguousarray(a))
        if a.dtype == np.uint16:
            t = t.view(torch.int16).view(torch.bfloat16)
        static[k].copy_(t)


def _outputs():
    d = "cuda"
    o = dict(
        res_out=torch.empty((T, H), dtype=torch.bfloat16, device=d),
        q=torch.empty(T * H, dtype=torch.uint8, device=d),
        sf=torch.empty(T * H // 32, dtype=torch.uint8, device=d),
        normed=torch.empty((T, H), dtype=torch.bfloat16, device=d),
        y8=torch.empty(T * H + 8, dtype=torch.uint8, device=d),
        scale=torch.empty(1, dtype=torch.float32, device=d),
        parts=torch.empty(64, dtype=torch.float32, device=d),
        idx=torch.empty((T, TOPK), dtype=torch.int32, device=d),
        wts=torch.empty((T, TOPK), dtype=torch.float32, device=d),
        bc=torch.empty(NBLK * E, dtype=torch.int32, device=d),
        bo=torch.empty(NBLK * E, dtype=torch.int32, device=d),
        cb=torch.empty(CAP // 128 + 1, dtype=torch.int32, device=d),
        cl=torch.empty(CAP // 128 + 1, dtype=torch.int32, device=d),
        nne=torch.empty(1, dtype=torch.int32, device=d),
        tp=torch.empty(1, dtype=torch.int32, device=d),
        rmap=torch.empty(CAP, dtype=torch.int32, device=d),
        e2p=torch.empty(T * TOPK, dtype=torch.int32, device=d),
        pq=torch.empty(CAP * H, dtype=torch.uint8, device=d),
        psf=torch.empty(CAP * H // 32, dtype=torch.uint8, device=d),
        prefix2=torch.empty((T, H), dtype=torch.bfloat16, device=d),
        k1n=torch.empty((T, H), dtype=torch.bfloat16, device=d),
        push_blocks=torch.empty((T, 8, H), dtype=torch.bfloat16, device=d),
        normed_all=torch.empty((2 * T, H), dtype=torch.bfloat16, device=d),
        peer_all=torch.empty((2 * T, H), dtype=torch.bfloat16, device=d),
        act=torch.empty((T, N_SITU), dtype=torch.bfloat16, device=d),
    )
    o["dst_peer"] = torch.tensor([o["peer_all"].data_ptr(), o["normed_all"].data_ptr()],
                                 dtype=torch.int64, device=d)
    return o


def _clear(o):
    """Sentinel fill of every output (torch fill kernels)."""
    for k, t in o.items():
        if k == "dst_peer":
            continue
        if t.dtype == torch.bfloat16:
            t.view(torch.int16).fill_(0x7f5a)
        elif t.dtype == torch.float32:
            t.view(torch.int32).fill_(0x5a5a5a5a)
        elif t.dtype == torch.int32:
            t.fill_(-7)
        else:
            t.fill_(0x5a)


def _chain(ctx, i, o):
    ctx.residual_rms_mxfp8(i["x"], i["res"], i["gamma"], o["res_out"], o["q"], o["sf"],
                           normed=o["normed"], eps=1e-6, B=T)
    ctx.quant_fp8_tensor(o["normed"], o["y8"], o["scale"], o["parts"], T * H)
    ctx.router_topk(i["S"], i["bias"], i["rs"], o["idx"], o["wts"], T, topk=TOPK)
    ctx.moe_route_count(o["idx"], T, RANK, E, o["bc"], topk=TOPK)
    ctx.moe_route_tables(o["bc"], NBLK, E, 128, o["bo"], o["cb"], o["cl"], o["nne"], o["tp"],
                         o["rmap"], T=T, topk=TOPK)
    ctx.moe_route_scatter(o["idx"], o["bo"], T, RANK, E, o["rmap"], o["e2p"], topk=TOPK)
    ctx.moe_permute_mx(o["q"], o["sf"], o["rmap"], o["tp"], H, o["pq"], o["psf"])
    ctx.land_add_attnres_rms_nb(i["partial"], i["prefix"], i["blocks"], i["sw"], i["gamma"],
                                o["prefix2"], o["k1n"], NB, 0, T)
    ctx.stream_copy(i["blocks"], o["push_blocks"])
    ctx.attnres_rms_push(o["prefix2"], o["push_blocks"], i["sw"], i["gamma"], o["normed_all"],
                         o["dst_peer"], NB, 1, T, 1, 2, version=3)
    ctx.land_situ(i["sp"], o["act"], N_SITU, T)


def _bits(t):
    if t.dtype in (torch.bfloat16,):
        return t.view(torch.int16)
    if t.dtype == torch.float32:
        return t.view(torch.int32)
    return t


def test_graph_replays_match_eager(ctx):
    _case(f"graph capture of the prefill chain T={T}")
    static = _static_inputs(_inputs(9000))
    g_out, e_out = _outputs(), _outputs()
    # eager pass first: loads every code object the chain uses before capture
    _clear(g_out)
    _chain(ctx, static, g_out)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _chain(ctx, static, g_out)
    torch.cuda.synchronize()

    for r in range(4):
        _case(f"replay {r}")
        _load(static, _inputs(9001 + r))
        _clear(e_out)
        _chain(ctx, static, e_out)
        torch.cuda.synchronize()
        _clear(g_out)
        graph.replay()
        torch.cuda.synchronize()
        for k in e_out:
            if k == "dst_peer":
                continue
            a, b = _bits(g_out[k]), _bits(e_out[k])
            bad = int((a != b).sum())
            assert bad == 0, f"replay {r}: {k}: {bad} of {a.numel()} differ"
        # the push reached both buffers and the routing produced rows
        assert int(e_out["tp"][0]) > 0
        assert torch.equal(_bits(e_out["normed_all"][T:]), _bits(e_out["peer_all"][T:]))
    graph.reset()


def test_graph_replays_the_arrival_barrier(ctx):
    """The res_in sequence's barrier part captured: the epoch bump, the peer's
    arrival (played by a torch add on its counter, a kernel node) and the one-wave
    arrival wait.  Replays and eager runs alternate; every one must leave the
    counters at the protocol's totals and report no rank given up on (a wait that
    gave up would also take 2 s)."""
    _case("graph capture of epoch bump + peer arrival + arrive")
    own = torch.zeros(372, dtype=torch.int64, device="cuda")
    peer = torch.zeros(372, dtype=torch.int64, device="cuda")
    fpeer = torch.tensor([own.data_ptr(), peer.data_ptr()], dtype=torch.int64, device="cuda")
    missing = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    units, slot = 896, 3

    def seq():
        ctx.epoch_bump(own, units)
        peer[slot] += units
        ctx.rs_arrive(own, fpeer, units, slot, 2, missing)

    seq()  # loads the code objects before capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        seq()
    torch.cuda.synchronize()
    calls = 1
    for r in range(4):
        _case(f"barrier replay {r}")
        missing.fill_(-1)
        graph.replay()
        calls += 1
        torch.cuda.synchronize()
        assert int(missing[0]) == 0, f"replay {r}: ranks given up on {int(missing[0])}"
        missing.fill_(-1)
        seq()  # eager between replays
        calls += 1
        torch.cuda.synchronize()
        assert int(missing[0]) == 0
        total = calls * units
        assert int(own[0]) == total and int(own[slot]) == total and int(peer[slot]) == total
    graph.reset()
