"""Headline benchmark: fused residual add + RMSNorm + MXFP8 at 16384 x 7168 on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--ops]

A step is one launch of ``k3h_residual_rms_mxfp8`` over the whole [16384, 7168]
chunk with inputs resident in HBM.  Timing: W untimed
warm-up steps, then K steps between two HIP events on the launch stream, with a
device synchronisation on both sides.  ``value`` is the effective HBM bandwidth
(algorithmic bytes per step / mean step time).  Algorithmic bytes: x and the
residual read once, gamma once, residual_out + e4m3 payload + E8M0 scales
written once = 825,767,936 B.

``roofline`` gives the achieved rate against MI355X's 8 TB/s HBM peak and, when
``profiles/traffic.json`` holds rocprofv3 FETCH_SIZE/WRITE_SIZE counts for the
kernel, the measured HBM bytes per launch.  ``cpu_baseline`` times the C oracle
(OpenMP over the host cores) on the same inputs -- the checker run as a
reported baseline, never the measured path.  One JSON line goes to stdout;
progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "kern-k3_amd"))

METRIC = "effective HBM GB/s (% of peak) for residual+RMSNorm+MXFP8 at 16384x7168"
H = 7168
T = 16384
PEAK_GBS = 8000.0


def algo_bytes(rows: int) -> int:
    n = rows * H
    return 2 * n * 2 + H * 2 + n * 2 + n + n // 32


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def make_inputs(rows: int, seed: int = 24301):
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    x = torch.randn((rows, H), generator=g, device="cuda", dtype=torch.float32)
    out = torch.rand((rows, H), generator=g, device="cuda") < 0.001
    x = torch.where(out, torch.randn((rows, H), generator=g, device="cuda") * 50.0, x)
    x = x.to(torch.bfloat16)
    res = torch.randn((rows, H), generator=g, device="cuda", dtype=torch.float32).to(torch.bfloat16)
    gamma = (1.0 + 0.1 * torch.randn(H, generator=g, device="cuda")).to(torch.bfloat16)
    return x, res, gamma


def cpu_baseline(x, res, gamma, gpu_out, budget_s: float = 10.0) -> dict:
    """Times the C oracle (the checker) on the same inputs, bounded to ~budget_s."""
    import numpy as np
    import torch
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O

    def h(t):
        return t.cpu().view(torch.int16).numpy().view(np.uint16)

    xh, rh, gh = h(x), h(res), h(gamma)
    rows = xh.shape[0]
    times = []
    t_start = time.perf_counter()
    out = None
    while not times or (time.perf_counter() - t_start < budget_s and len(times) < 5):
        t0 = time.perf_counter()
        out = O.residual_rms_mxfp8(xh, rh, gh, rows, 1e-6, want_normed=False)
        times.append(time.perf_counter() - t0)
    best = sorted(times)[len(times) // 2]
    ro, q, sf = (t.cpu().numpy() if t.dtype != torch.bfloat16 else h(t) for t in gpu_out)
    match = bool((out[0] == ro).all() and (out[1] == q).all() and (out[2] == sf).all())
    return {
        "value": round(algo_bytes(rows) / best / 1e9, 2),
        "unit": "GB/s",
        "cores": O.num_threads(),
        "kind": "port",
        "sample": f"full {rows}x{H} workload, median of {len(times)} oracle passes "
                  f"({best * 1e3:.0f} ms each); bit-exact vs GPU: {match}",
    }


def copy_ceiling(ctx, rows: int, reps: int) -> float:
    """Rate of the plain 16-byte streaming copy over one [rows, 7168] bf16 tensor."""
    import torch
    src = torch.empty(rows * H, dtype=torch.bfloat16, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    s = torch.cuda.current_stream()
    for _ in range(3):
        ctx.stream_copy(src, dst, stream=s)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(reps):
        ctx.stream_copy(src, dst, stream=s)
    e1.record(s)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    gbs = 2 * src.numel() * 2 / (us * 1e-6) / 1e9
    log(f"copy ceiling: {us:.1f} us per {2 * src.numel() * 2 / 1e6:.0f} MB -> {gbs:.0f} GB/s")
    del src, dst
    return gbs


def load_traffic(kernel: str, workload: str):
    p = os.path.join(REPO, "profiles", "traffic.json")
    try:
        d = json.load(open(p))
        return d[kernel][workload]["hbm_bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--rows", type=int, default=T)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--op", choices=["fused", "copy"], default="fused",
                    help="copy: only the 16-byte streaming copy (counter calibration)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {a.gpus}); the op family shards "
              "by rows / heads / experts with no exchange on the measured path.", file=sys.stderr)
        return 2

    import torch
    import k3h

    ctx = k3h.Ctx()
    rows = a.rows
    copy_gbs = copy_ceiling(ctx, rows, a.steps if a.op == "copy" else 20)
    if a.op == "copy":
        print(json.dumps({"op": "k3h_stream_copy", "bytes_per_launch": 2 * rows * H * 2,
                          "gbs": round(copy_gbs, 1)}), flush=True)
        return 0
    log(f"inputs {rows}x{H} bf16 on {torch.cuda.get_device_name(0)}")
    x, res, gamma = make_inputs(rows)
    ro = torch.empty_like(x)
    q = torch.empty((rows, H), dtype=torch.uint8, device="cuda")
    sf = torch.empty((rows, H // 32), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()

    def step():
        ctx.residual_rms_mxfp8(x, res, gamma, ro, q, sf, None, eps=1e-6, B=rows, stream=stream)

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(a.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / a.steps
    nbytes = algo_bytes(rows)
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"{ms * 1e3:.1f} us/step, {gbs:.0f} GB/s ({100 * gbs / PEAK_GBS:.1f}% of 8 TB/s)")

    traffic = load_traffic("k3h_residual_rms_mxfp8", f"{rows}x{H}")
    roof = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / PEAK_GBS, 4), "traffic": traffic,
            "kernel": "k3h_residual_rms_mxfp8", "algorithmic_bytes": nbytes,
            "avg_launch_us": round(ms * 1e3, 2), "copy_ceiling_gbs": round(copy_gbs, 1)}
    cpu = None
    if not a.no_cpu:
        log("CPU baseline: C oracle on the same inputs")
        cpu = cpu_baseline(x, res, gamma, (ro, q, sf), a.cpu_budget)
        log(f"CPU {cpu['value']} GB/s on {cpu['cores']} threads; {cpu['sample']}")
    line = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (torch randn from seed 24301; 0.1% outliers x50)",
        "config": {"workload": "fused residual add + RMSNorm + MXFP8 (BASELINE config 2)",
                   "tokens": rows, "hidden": H, "eps": 1e-6, "block": 32,
                   "payload": "e4m3 (OCP)", "scale": "E8M0"},
        "pct_of_peak": round(100 * gbs / PEAK_GBS, 2),
        "roofline": roof, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
