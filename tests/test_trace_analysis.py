"""The trace pipeline's analysis (programs/trace_analysis.py) on hand-made rocprofv3 CSV files:
interval statistics against values worked out by hand, lane packing, the validation failures the
reference's analyze.py:25-60 raises (kernel count, copies in the region, API counts per mode), HBM
bytes from counters, and the Chrome trace export."""
import csv
import gzip
import json

import pytest

from programs import trace_analysis as ta

KERNEL_FIELDS = ["Kind", "Agent_Id", "Queue_Id", "Stream_Id", "Thread_Id", "Dispatch_Id", "Kernel_Id", "Kernel_Name",
                 "Correlation_Id", "Start_Timestamp", "End_Timestamp", "Grid_Size_X", "Workgroup_Size_X"]


def write_csv(path, fields, rows):
    with path.open("w", newline="") as handle:
        writer = csv.DictWriter(handle, fieldnames=fields)
        writer.writeheader()
        for row in rows:
            writer.writerow(row)


def kernels(path, spans, names=None, streams=None):
    rows = []
    for k, (start, end) in enumerate(spans):
        rows.append({"Kind": "KERNEL_DISPATCH", "Agent_Id": "Agent 1", "Queue_Id": 1,
                     "Stream_Id": (streams or [0] * len(spans))[k], "Thread_Id": 7, "Dispatch_Id": k + 1,
                     "Kernel_Id": 1, "Kernel_Name": (names or ["ckl_linear_mfma2x1_nt"] * len(spans))[k],
                     "Correlation_Id": k + 1, "Start_Timestamp": start, "End_Timestamp": end, "Grid_Size_X": 256,
                     "Workgroup_Size_X": 256})
    write_csv(path / "run_kernel_trace.csv", KERNEL_FIELDS, rows)


def apis(path, functions):
    rows = [{"Domain": "HIP_RUNTIME_API", "Function": f, "Process_Id": 1, "Thread_Id": 7, "Correlation_Id": k,
             "Start_Timestamp": 1000 * k, "End_Timestamp": 1000 * k + 500} for k, f in enumerate(functions)]
    write_csv(path / "run_hip_api_trace.csv", list(rows[0]) if rows else ["Function"], rows)


def metadata(kernels_, graph_launches=None, mode="stream"):
    return {"complete": True, "case": "small", "requests": 2, "mode": mode, "group": 1, "steps": 1,
            "kernels": kernels_, "graph_launches": graph_launches, "wall_us": 40.0, "span_us": 30.0}


SPANS = [(0, 10_000), (5_000, 15_000), (20_000, 30_000)]     # ns


def test_interval_statistics_and_lanes(tmp_path):
    names = ["ckl_linear_mfma2x1_nt_shared3", "ckl_rope__rope__append_kv__attention_scores__softmax__attention_values_nt",
             "ckl_linear_rowvec_group"]
    kernels(tmp_path, SPANS, names, streams=[1, 2, 1])
    apis(tmp_path, ["hipModuleLaunchKernel"] * 3 + ["hipStreamSynchronize"])
    s = ta.analyze(tmp_path, "run", metadata(3))
    # Union [0, 15) + [20, 30) = 25 us busy over a 30 us span; [5, 10) runs two kernels.
    assert s["span_us"] == 30.0 and s["busy_us"] == 25.0 and s["idle_us"] == 5.0
    assert s["overlap_us"] == 5.0 and s["max_concurrent_kernels"] == 2
    assert s["overlap_fraction"] == pytest.approx(5 / 30)
    assert s["sum_kernel_us"] == 30.0
    assert s["family_kernel_us"] == {"linear": 20.0, "rope__rope__append_kv__attention_scores__softmax__attention_values": 10.0}
    assert s["stream_kernel_us"] == {"1": 20.0, "2": 10.0}
    assert s["hip_api_counts"]["hipModuleLaunchKernel"] == 3
    assert ta.pack_lanes(SPANS) == [0, 1, 0]
    trace = json.loads(gzip.decompress((tmp_path / "run.trace.json.gz").read_bytes()))
    gpu = [e for e in trace["traceEvents"] if e.get("cat") == "GPU kernel"]
    host = [e for e in trace["traceEvents"] if e.get("cat") == "HIP API"]
    assert len(gpu) == 3 and len(host) == 4
    assert [e["tid"] for e in gpu] == [0, 1, 0] and min(e["ts"] for e in gpu + host) == 0.0
    assert gpu[1]["args"]["stream"] == "2"


def test_intervals_summary_nested_and_touching():
    # [0, 10) holds [2, 4) and [3, 8): three at once in [3, 4); [10, 12) only touches [0, 10).
    s = ta.intervals_summary([(0, 10), (2, 4), (3, 8), (10, 12)])
    assert s == {"busy_ns": 12, "overlap_ns": 6, "max_concurrent": 3}


def test_validation_failures(tmp_path):
    kernels(tmp_path, SPANS)
    with pytest.raises(ValueError, match="expected 4 kernel dispatches"):
        ta.analyze(tmp_path, "run", metadata(4))
    apis(tmp_path, ["hipModuleLaunchKernel"] * 2)
    with pytest.raises(ValueError, match="kernel launches"):
        ta.analyze(tmp_path, "run", metadata(3))
    apis(tmp_path, ["hipGraphLaunch"] * 2)
    ta.analyze(tmp_path, "run", metadata(3, graph_launches=2, mode="graph"))
    with pytest.raises(ValueError, match="graph launches"):
        ta.analyze(tmp_path, "run", metadata(3, graph_launches=3, mode="graph"))
    kernels(tmp_path, SPANS + [(40_000, 41_000)], ["ckl_linear_mfma2x1_nt"] * 3 + ["__amd_rocclr_copyBuffer"])
    with pytest.raises(ValueError, match="copy/fill"):
        ta.analyze(tmp_path, "run", metadata(4, graph_launches=2, mode="graph"))
    kernels(tmp_path, [(5, 5)])
    (tmp_path / "run_hip_api_trace.csv").unlink()
    with pytest.raises(ValueError, match="ends before"):
        ta.analyze(tmp_path, "run", metadata(1))


def test_hbm_bytes_from_counters(tmp_path):
    kernels(tmp_path, SPANS[:2], ["ckl_linear_mfma2x1_nt", "ckl_silu__multiply"])
    fields = ["Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]
    write_csv(tmp_path / "run_counter_collection.csv", fields, [
        {"Dispatch_Id": 1, "Kernel_Name": "ckl_linear_mfma2x1_nt", "Counter_Name": "FETCH_SIZE", "Counter_Value": 100},
        {"Dispatch_Id": 1, "Kernel_Name": "ckl_linear_mfma2x1_nt", "Counter_Name": "WRITE_SIZE", "Counter_Value": 10},
        {"Dispatch_Id": 2, "Kernel_Name": "ckl_silu__multiply", "Counter_Name": "FETCH_SIZE", "Counter_Value": 4}])
    s = ta.analyze(tmp_path, "run", metadata(2), fetch_scale=2.0)
    assert s["family_hbm_bytes"] == {"linear": (100 * 2.0 + 10) * 1024, "silu__multiply": 4 * 2.0 * 1024}


@pytest.mark.parametrize("name,expected", [
    ("ckl_linear_mfma4x1_nt_shared2", "linear"), ("ckl_linear_rowvec", "linear"), ("ckl_linear_rowvec_group", "linear"),
    ("ckl_linear_rowvec__add__rms_stats__rms_apply", "linear_rowvec__add__rms_stats__rms_apply"),
    ("ckl_greedy__advance", "greedy__advance"), ("ckl_attention_values_nt", "attention_values"),
    ("__amd_rocclr_copyBuffer", "__amd_rocclr_copyBuffer")])
def test_family_names(name, expected):
    assert ta.family(name) == expected


def test_one_profiler_region_required(tmp_path):
    kernels(tmp_path, SPANS)
    fields = ["Domain", "Function", "Process_Id", "Thread_Id", "Correlation_Id", "Start_Timestamp", "End_Timestamp"]
    row = {"Domain": "MARKER_CONTROL_API", "Process_Id": 1, "Thread_Id": 1, "Correlation_Id": 1,
           "Start_Timestamp": 0, "End_Timestamp": 1}
    write_csv(tmp_path / "run_marker_api_trace.csv", fields,
              [dict(row, Function="roctxProfilerResume"), dict(row, Function="roctxProfilerPause")])
    assert ta.analyze(tmp_path, "run", metadata(3))["kernels"] == 3
    write_csv(tmp_path / "run_marker_api_trace.csv", fields, [dict(row, Function="roctxProfilerPause")])
    with pytest.raises(ValueError, match="one profiler region"):
        ta.analyze(tmp_path, "run", metadata(3))
