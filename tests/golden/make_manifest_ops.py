"""Extracts the hot-path op descriptions from the reference manifests into
manifest_hot_ops.json (run in the build container, where /root/reference exists;
the tests read only the committed JSON).

The extracted data is the ABI contract: parameter kinds and order, the launch
list (module key, entry, block, grid expression, argument mapping)."""
import json
import os

REF = "/root/reference/manifests"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "manifest_hot_ops.json")

HOT = {
    "k3-tp4-prefill-16k.json": [
        "land_add_attnres_rms_bf16_v2_nb1", "quant_fp8_tensor", "moe_quant", "moe_route_count",
        "moe_route_tables", "moe_route_scatter", "moe_finalize", "router_topk", "mla_prep",
        "span_gather_v2", "kda_out_gate_v2",
        # residual push family and landing kernels
        "attnres_rms_push_first_v3", "attnres_rms_push_add2", "land_add_attnres_rms_bf16_v2_nb4",
        "land_add_attnres_rms_bf16_v2_nb8", "land_situ_n33792", "land_situ_rms",
        # epoch / arrival barrier (normed_sync after the push; coll_epoch; the load program's init)
        "k3_allgather_push", "k3_epoch_bump", "k3_flags_init",
    ],
    "k3-tp4-prefill-16k-l0-bf16.json": [
        "attnres_rms_v2", "land_add_attnres_rms_bf16_v2", "land_add2_v2",
        "rms", "land_n3584", "land_situ_n6144", ("land_situ_n33792", "l0_land_situ_n33792"),
    ],
}


def main():
    out = {}
    for fn, ops in HOT.items():
        with open(os.path.join(REF, fn)) as f:
            m = json.load(f)
        for op in ops:
            name, key = op if isinstance(op, tuple) else (op, op)
            out[key] = {"manifest": fn, **m["ops"][name]}
        out.setdefault("_vars", m["vars"])
    with open(OUT, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
    print(f"wrote {len(out) - 1} ops to {OUT}")


if __name__ == "__main__":
    main()
