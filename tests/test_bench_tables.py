"""CPU checks of bench.py's measurement tables on synthetic inputs: the rocprofv3
counter CSV reader, the copy-calibrated HBM byte table and the per-op markdown
table.  No GPU: the CSVs and the ops JSON are written here."""
import csv
import json
import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, REPO)
import bench  # noqa: E402

COPY_BYTES = 1 << 20  # the synthetic copy moves 1 MiB in and 1 MiB out


def _pmc_csv(path, counter, per_kernel):
    """rocprofv3-style counter_collection.csv: one row per dispatch, in the order given."""
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"])
        w.writeheader()
        did = 0
        for name, values in per_kernel:
            for v in values:
                did += 1
                w.writerow({"Dispatch_Id": did, "Kernel_Name": name + "(int, float*)",
                            "Counter_Name": counter, "Counter_Value": v})


def _ops_json(path):
    rows = [
        {"op": "stream copy (ceiling)", "kernel": "k3h_stream_copy", "shape": "s", "bytes": 2 * COPY_BYTES,
         "launches": 3, "us": 2.0, "us_p10": 1.9, "us_p90": 2.1, "gbs": 1048.6, "pct_peak": 13.1,
         "us_dirty": 2.0, "gbs_dirty": 1048.6, "note": ""},
        {"op": "residual+RMSNorm+MXFP8 (cfg 2)", "kernel": "k3h_residual_rms_mxfp8", "shape": "s",
         "bytes": 3 * COPY_BYTES, "launches": 3, "us": 4.0, "us_p10": 3.9, "us_p90": 4.2, "gbs": 786.4,
         "pct_peak": 9.8, "us_dirty": 5.0, "gbs_dirty": 629.1, "note": "n", "cpu_ms": 2.0,
         "cpu_gbs": 1.57, "cpu_threads": 16},
        {"op": "MoE fc2 (MX GEMM, bf16 out)", "kernel": "kern_k3h_moe_gemm_bf16", "shape": "s",
         "bytes": 10, "flops": 1000, "bound": "mfma", "launches": 3, "us": 1.0, "us_p10": 1.0,
         "us_p90": 1.0, "tflops": 0.001, "pct_peak": 0.0, "gbs": 0.01, "us_dirty": 1.5, "note": ""},
    ]
    json.dump(rows, open(path, "w"))
    return rows


def test_counter_values_keep_dispatch_order_per_kernel(tmp_path):
    p = tmp_path / "c.csv"
    _pmc_csv(p, "FETCH_SIZE", [("a", [3.0, 1.0]), ("b", [7.0]), ("a", [2.0])])
    v = bench.counter_values(str(p), "FETCH_SIZE")
    assert v == {"a": [3.0, 1.0, 2.0], "b": [7.0]}
    assert bench.counter_values(str(p), "WRITE_SIZE") == {}


def test_traffic_table_calibrates_on_the_copy(tmp_path):
    # the copy's counters read half (FETCH) and twice (WRITE) its true bytes: the
    # factors 2 and 0.5 must map the fused kernel's counters onto 2 MiB read + 1 MiB written
    kib = COPY_BYTES / 1024
    f, w = tmp_path / "f.csv", tmp_path / "w.csv"
    _pmc_csv(f, "FETCH_SIZE", [("k3h_stream_copy", [kib / 2] * 3), ("k3h_residual_rms_mxfp8", [kib] * 3)])
    _pmc_csv(w, "WRITE_SIZE", [("k3h_stream_copy", [kib * 2] * 3),
                               ("k3h_residual_rms_mxfp8", [kib / 2, kib * 9, kib / 2])])
    ops = tmp_path / "ops.json"
    _ops_json(ops)
    table = bench.traffic_table(str(f), str(w), str(ops))
    assert "FETCH_SIZE x 2.00000, WRITE_SIZE x 0.50000" in table
    row = next(l for l in table.splitlines() if l.startswith("| residual+RMSNorm+MXFP8"))
    cells = [c.strip() for c in row.strip("|").split("|")]
    # read 2 MiB, written = median of (0.25, 4.5, 0.25) MiB = 0.25 MiB
    assert cells[2] == f"{2 * COPY_BYTES:,}" and cells[3] == f"{COPY_BYTES // 4:,}"
    assert cells[-1] == f"{(2 * COPY_BYTES + COPY_BYTES // 4) / (3 * COPY_BYTES):.3f}"


def test_ops_markdown_columns(tmp_path):
    ops = tmp_path / "ops.json"
    rows = _ops_json(ops)
    md = bench.ops_markdown(str(ops)).splitlines()
    hbm = [l for l in md if l.startswith("| residual+RMSNorm+MXFP8")]
    assert len(hbm) == 1
    cells = [c.strip() for c in hbm[0].strip("|").split("|")]
    assert cells[9] == f"{100 * rows[1]['gbs'] / rows[0]['gbs']:.0f}"  # % of the copy row
    assert cells[10] == "5.00" and cells[11] == "629.1"                  # dirty-flush time and rate
    assert cells[12] == "2.0" and cells[13] == "1.57"                    # CPU oracle columns
    assert cells[14] == f"{rows[1]['gbs'] / rows[1]['cpu_gbs']:.0f}x"
    assert any(l.startswith("| MoE fc2") for l in md)                    # MFMA table
    assert not any(l.startswith("| MoE fc2") and "629" in l for l in md)


def test_ops_markdown_graph_columns(tmp_path):
    ops = tmp_path / "ops.json"
    rows = _ops_json(ops)
    rows[1].update({"us_graph": 3.5, "gbs_graph": 898.6})
    json.dump(rows, open(ops, "w"))
    md = bench.ops_markdown(str(ops)).splitlines()
    head = [c.strip() for c in md[0].strip("|").split("|")]
    assert head[12] == "us, graph replay" and head[13] == "GB/s, graph replay"
    assert all(l.count("|") == md[0].count("|") for l in md[:4])     # every row has the columns
    cells = [c.strip() for c in next(l for l in md if l.startswith("| residual+")).strip("|").split("|")]
    assert cells[12] == "3.50" and cells[13] == "898.6" and cells[14] == "2.0"
    copy = [c.strip() for c in next(l for l in md if l.startswith("| stream copy")).strip("|").split("|")]
    assert copy[12] == "" and copy[13] == ""                           # no graph figure: empty cells


def test_ceilings_markdown_rates():
    rows = [
        {"probe": "copy_u4", "op": "copy", "loads_in_flight": 4, "grid": "flat 16", "cache": "non-temporal",
         "bytes": 8_000_000, "us_b2b": 2.0, "gbs_b2b": 4000.0, "us_flushed": 4.0, "gbs_flushed": 2000.0},
        {"probe": "mfma_f8f4", "op": "mfma", "grid": "2 x 256", "flops": 10_000_000, "us_b2b": 2.0,
         "tflops": 5.0},
    ]
    md = bench.ceilings_markdown(rows).splitlines()
    copy = [c.strip() for c in next(l for l in md if l.startswith("| copy_u4")).strip("|").split("|")]
    assert copy[1] == "copy, non-temporal" and copy[6] == "4000" and copy[7] == "50.0"  # % of 8 TB/s
    assert copy[9] == "2000" and copy[10] == "25.0"
    mf = [c.strip() for c in next(l for l in md if l.startswith("| mfma_f8f4")).strip("|").split("|")]
    assert mf[1] == "e4m3 x e2m1" and mf[5] == "5"


def test_trace_table_takes_clean_flush_launches(tmp_path):
    """Dispatch order per kernel: 5 warm-ups, reps clean, reps dirty; multi-kernel
    ops sum their kernels per launch."""
    reps = 3
    ops = [{"op": "stream copy (ceiling)", "kernel": "k3h_stream_copy", "bytes": 8_000_000,
            "launches": 5 + 2 * reps, "us": 9.0},
           {"op": "EP routing tables (count+tables+scatter)", "kernel": "x", "bytes": 1_000,
            "launches": 5 + 2 * reps, "us": 20.0}]
    json.dump(ops, open(tmp_path / "ops.json", "w"))
    spans = {"k3h_stream_copy": [1] * 5 + [2, 4, 3] + [50] * 3,
             "kern_k3_moe_route_count": [1] * 5 + [1, 1, 1] + [9] * 3,
             "kern_k3_moe_route_tables": [1] * 5 + [2, 2, 2] + [9] * 3,
             "kern_k3_moe_route_scatter": [1] * 5 + [3, 5, 4] + [9] * 3}
    with open(tmp_path / "tr.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp"])
        w.writeheader()
        did = 0
        for i in range(5 + 2 * reps):  # interleaved dispatch ids, as in a real trace
            for k, v in spans.items():
                did += 1
                w.writerow({"Dispatch_Id": did, "Kernel_Name": k + "(int*)", "Start_Timestamp": 1000,
                            "End_Timestamp": 1000 + int(v[i] * 1000)})
    md = bench.trace_table(str(tmp_path / "tr.csv"), str(tmp_path / "ops.json")).splitlines()
    cp = [c.strip() for c in next(l for l in md if l.startswith("| stream copy")).strip("|").split("|")]
    assert cp[3] == "3.00" and cp[4] == f"{8_000_000 / 3e-6 / 1e9:.1f}"   # median of 2, 4, 3
    rt = [c.strip() for c in next(l for l in md if l.startswith("| EP routing tables")).strip("|").split("|")]
    assert rt[3] == "7.00"                                                # 1+2+4 (median of 6, 8, 7)


def test_more_than_one_gpu_is_refused():
    """bench.py measures one GPU: --gpus N > 1 exits with status 2 and says so,
    before touching a device."""
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
