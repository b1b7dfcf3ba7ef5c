"""Build the gfx950 code objects, the k3h host library and the CPU oracle.

Code objects follow the reference's module naming (kernels.toml keys): a module
key is ``<base>[+DEFINE=value]...``; ``<base>`` selects the HIP source and each
``+DEFINE=value`` becomes ``-DDEFINE=value``.  One ``<key>.hsaco`` per key is
written to ``kern-k3_amd/build/``, next to ``libk3h.so`` (the C-ABI of
``include/k3h.h``).  ``build/modules.lock.json`` records the sha256 of every code
object, mirroring the reference's pinned-module check (scripts/check.py:19-50).

Usage: ``python kern-k3_amd/build.py [--jobs N] [--only KEY ...]``.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import hashlib
import json
import os
import shutil
import subprocess
import sys
import time

PKG = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
OUT = os.path.join(PKG, "build")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# base name -> HIP source (relative to csrc/kernels)
SOURCES = {
    "k3_residual_v2": "k3_residual_v2.hip",
    "k3_residual_nb": "k3_residual_nb.hip",
    "k3_residual_nb_stats": "k3_residual_nb.hip",
    "k3_residual_push": "k3_residual_push.hip",
    "k3_residual_push_v3": "k3_residual_push.hip",
    "k3_residual_push_stats": "k3_residual_push.hip",
    "k3_residual_push_add2": "k3_residual_push.hip",
    "k3h_fused": "k3h_fused.hip",
    "k3_moe_prefill_v3": "k3_moe_prefill.hip",
    "k3_moe_prefill_v4": "k3_moe_prefill.hip",
    "k3_quant_fp8_pair": "k3_quant_fp8_pair.hip",
    "k3_quant_fp8_pair_v2": "k3_quant_fp8_pair.hip",
    "k3_router_argmax": "k3_router_argmax.hip",
    "k3_span_gather_v3": "k3_span_gather.hip",
    "k3_kda_out_gate_v3": "k3_kda_out_gate.hip",
    "k3_mla_prep_v2": "k3_mla_prep.hip",
    "k3_mla_prep_bf16": "k3_mla_prep.hip",
    "k3h_mla_rope": "k3h_mla_rope.hip",
    "k3_land": "k3_land.hip",
    "k3_land_bf16": "k3_land.hip",
    "k3_situ_bf16": "k3_land.hip",
    "k3_land_fused": "k3_land.hip",
    "k3h_moe_gemm": "k3h_moe_gemm.hip",
    "k3h_probe": "k3h_probe.hip",
    "k3_collectives": "k3_barrier.hip",
    "k3_rs_arrive1": "k3_barrier.hip",
    "k3_rs_arrive_v2": "k3_barrier.hip",
}

# defines implied by a base name that shares its source with another base
IMPLIED = {
    "k3_land": ["-DK3_LAND_MODULE=1"],
    "k3_land_bf16": ["-DK3_LAND_MODULE=2"],
    "k3_situ_bf16": ["-DK3_LAND_MODULE=3"],
    "k3_land_fused": ["-DK3_LAND_MODULE=4"],
    "k3_residual_nb_stats": ["-DK3_NB_STATS=1", "-DLAND_BF16=1"],  # kernels.toml: defines { LAND_BF16 = 1 }
    "k3_residual_push": ["-DK3_PUSH=1"],
    "k3_residual_push_v3": ["-DK3_PUSH=1"],
    "k3_residual_push_stats": ["-DK3_PUSH=2"],
    "k3_residual_push_add2": ["-DK3_PUSH=3"],
    "k3_quant_fp8_pair_v2": ["-DK3_QUANT_V2=1"],
    "k3_mla_prep_bf16": ["-DK3_MLA_BF16=1"],
}

# Every module key the host library or the manifests may load.
MODULES = [
    "k3_residual_v2",
    "k3_residual_v2+LAND_BF16=1",
    "k3_residual_v2+K3_EPS=1e-6f",
    "k3_residual_v2+LAND_BF16=1+K3_EPS=1e-6f",
    "k3_residual_nb+LAND_BF16=1",
    "k3_residual_nb_stats",
    "k3_residual_push",
    "k3_residual_push_v3",
    "k3_residual_push_stats",
    "k3_residual_push_add2",
    "k3h_fused",
    "k3_moe_prefill_v3+EP_STRIDED=1",
    "k3_moe_prefill_v4+EP_RANKS=4+EP_STRIDED=1+TILE_SHIFT=7+SCATTER_WARPS=16",
    "k3_moe_prefill_v4+EP_RANKS=4+EP_STRIDED=1+TILE_SHIFT=7+SCATTER_WARPS=16+TOPK=8",
    "k3_quant_fp8_pair",
    "k3_quant_fp8_pair_v2",
    "k3_router_argmax",
    "k3_router_argmax+TOPK=8",
    "k3_span_gather_v3+HEADS=24",
    "k3_kda_out_gate_v3+HEADS=24",
    "k3_kda_out_gate_v3+HEADS=24+K11_RMS_EPS=1e-6f",
    "k3_mla_prep_v2+INNER=3072+MLA_FUSED=5184",
    "k3_mla_prep_bf16+INNER=3072+MLA_FUSED=5184",
    "k3h_mla_rope",
    "k3_land",
    "k3_land_bf16",
    "k3_situ_bf16",
    "k3_land_fused",
    "k3h_moe_gemm",
    "k3h_probe",
    "k3_collectives",
    "k3_rs_arrive1",
    "k3_rs_arrive_v2",
    "k3_rs_arrive_v2+K3_SPIN_US=20000",  # 20 ms give-up: the missing-rank tests
]

DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "--genco", "-std=c++17",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-mcode-object-version=5",
    # packed-fp32 instructions are kept out of every code object
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

HOST_SOURCES = ["k3h_module.cpp", "k3h_ops_residual.cpp", "k3h_ops_push.cpp", "k3h_ops_land.cpp", "k3h_ops_gemm.cpp", "k3h_ops_quant.cpp", "k3h_ops_moe.cpp", "k3h_ops_kda.cpp", "k3h_ops_mla.cpp", "k3h_synth.cpp"]
# host sources that carry device data (compiled as HIP for gfx950 into the library)
HOST_HIP_SOURCES = ["k3h_noalloc.hip"]


def module_defines(key: str) -> tuple[str, list[str]]:
    parts = key.split("+")
    base = parts[0]
    if base not in SOURCES:
        raise KeyError(f"unknown module base {base!r} in {key!r}")
    defs = list(IMPLIED.get(base, []))
    for p in parts[1:]:
        if "=" not in p:
            raise ValueError(f"bad define {p!r} in module key {key!r}")
        defs.append("-D" + p)
    return SOURCES[base], defs


def _run(cmd: list[str], what: str) -> None:
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines()
                    if "packed-fp32-ops" not in l and "--hip-link" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build of {what} failed ({r.returncode}):\n{' '.join(cmd)}\n{out}")


def build_module(key: str) -> str:
    src, defs = module_defines(key)
    dst = os.path.join(OUT, key + ".hsaco")
    tmp = dst + ".tmp"
    cmd = [HIPCC, *DEVICE_FLAGS, *defs, "-I", CSRC, "-o", tmp,
           os.path.join(CSRC, "kernels", src)]
    _run(cmd, key)
    os.replace(tmp, dst)
    return dst


def build_host() -> str:
    dst = os.path.join(OUT, "libk3h.so")
    tmp = dst + ".tmp"
    srcs = [os.path.join(CSRC, "host", s) for s in HOST_SOURCES]
    hip_srcs = [os.path.join(CSRC, "host", s) for s in HOST_HIP_SOURCES]
    cmd = [HIPCC, "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
           f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-Wall", "-Wextra", "-I", os.path.join(REPO, "include"), "-I", os.path.join(CSRC, "host"),
           "-o", tmp, *srcs, *hip_srcs]
    _run(cmd, "libk3h.so")
    os.replace(tmp, dst)
    return dst


def build_oracle() -> str | None:
    odir = os.path.join(REPO, "oracle")
    if not os.path.exists(os.path.join(odir, "Makefile")):
        return None
    subprocess.run(["make", "-s", "-C", odir, "-B"], check=True)
    return os.path.join(odir, "libk3oracle.so")


def write_lock() -> None:
    lock = {}
    for key in MODULES:
        with open(os.path.join(OUT, key + ".hsaco"), "rb") as f:
            lock[key] = hashlib.sha256(f.read()).hexdigest()
    with open(os.path.join(OUT, "modules.lock.json"), "w") as f:
        json.dump({"arch": ARCH, "modules": lock}, f, indent=1, sort_keys=True)


def build(jobs: int | None = None, only: list[str] | None = None, oracle: bool = True) -> None:
    if not shutil.which(HIPCC) and not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(OUT, exist_ok=True)
    keys = only or MODULES
    t0 = time.time()
    jobs = jobs or min(8, os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(build_module, k) for k in keys]
        futs.append(ex.submit(build_host))
        if oracle:
            futs.append(ex.submit(build_oracle))
        for f in futs:
            f.result()
    if not only:
        write_lock()
    print(f"[k3 build] {len(keys)} code objects + libk3h.so in {time.time() - t0:.1f}s -> {OUT}",
          flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--only", nargs="*", default=None)
    ap.add_argument("--no-oracle", action="store_true")
    a = ap.parse_args()
    build(a.jobs, a.only, oracle=not a.no_oracle)
    return 0


if __name__ == "__main__":
    sys.exit(main())
