"""Validate a rocprofv3 trace of one profiled burst; summarise and export it.

The analysis half of the trace pipeline (benchmarks/decoder/analyze.py:25-113 of the reference,
which reads Nsight SQLite exports). Input: the CSV files rocprofv3 writes with `-o <prefix>`
(`<prefix>_kernel_trace.csv`, and when collected `<prefix>_hip_api_trace.csv`,
`<prefix>_memory_copy_trace.csv`, `<prefix>_marker_api_trace.csv`, `<prefix>_counter_collection.csv`)
and the metadata file `programs/profile_runs.py` wrote for the burst. Standard library only.

Checks: one profiler region (one roctxProfilerResume and one roctxProfilerPause when markers were
traced) holding exactly the burst's kernel dispatches, every interval has end > start,
no copy or fill ran inside the region (runtime copy kernels or memory-copy records), and the HIP
API counts match the mode (one hipGraphLaunch per submission for graph modes, one
hipModuleLaunchKernel per kernel for the others). Summary: GPU span, busy and idle time (union of
kernel intervals), time with two or more kernels running and the most at once, per-family and
per-stream kernel time, the API counts; with hardware counters (FETCH_SIZE, WRITE_SIZE), HBM
bytes per family after scaling FETCH_SIZE by `--fetch-scale`. Export: a Chrome trace
(`<prefix>.trace.json.gz`) with GPU kernels packed into lanes by interval overlap (lanes are a
visualisation, not streams or compute units; the stream and dispatch ids are in each event's
arguments) and host API calls by thread.
"""
from __future__ import annotations

import argparse
import csv
import gzip
import heapq
import json
from collections import Counter, defaultdict
from pathlib import Path

COPY_KERNELS = ("__amd_rocclr_copyBuffer", "__amd_rocclr_fillBuffer")
LAUNCH_APIS = ("hipModuleLaunchKernel", "hipLaunchKernel", "hipExtModuleLaunchKernel")
GRAPH_APIS = ("hipGraphLaunch",)


def family(name: str) -> str:
    """Kernel family: the library entry without the ckl_ prefix and the streaming/group/shared
    suffixes (all linear tilings are one family)."""
    base = name[len("ckl_"):] if name.startswith("ckl_") else name
    for suffix in ("_group",):
        base = base.removesuffix(suffix)
    base = base.split("_shared")[0].removesuffix("_nt")
    return "linear" if base.startswith("linear_") and "__" not in base else base


def read_csv(path: Path) -> list:
    with path.open(newline="") as handle:
        return list(csv.DictReader(handle))


def intervals_summary(spans: list) -> dict:
    """Union and overlap of [start, end) intervals (ns): busy, overlapped (>= 2 active) and the
    largest number active at once."""
    changes = defaultdict(int)
    for start, end in spans:
        changes[start] += 1
        changes[end] -= 1
    active = busy = overlap = most = 0
    previous = None
    for t in sorted(changes):
        if previous is not None:
            busy += (t - previous) if active else 0
            overlap += (t - previous) if active > 1 else 0
        active += changes[t]
        most = max(most, active)
        previous = t
    return {"busy_ns": busy, "overlap_ns": overlap, "max_concurrent": most}


def pack_lanes(spans: list) -> list:
    """Lane of each interval (in start order): the lowest-ending free lane, else a new one."""
    order = sorted(range(len(spans)), key=lambda k: (spans[k][0], spans[k][1]))
    lanes, ends = [0] * len(spans), []
    for k in order:
        start, end = spans[k]
        if ends and ends[0][0] <= start:
            _, lane = heapq.heappop(ends)
        else:
            lane = len(ends)
        heapq.heappush(ends, (end, lane))
        lanes[k] = lane
    return lanes


def analyze(directory: Path, prefix: str, metadata: dict, fetch_scale: float = 1.0) -> dict:
    kernels = read_csv(directory / f"{prefix}_kernel_trace.csv")
    copies = [k for k in kernels if k["Kernel_Name"].startswith(COPY_KERNELS)]
    if copies:
        raise ValueError(f"{len(copies)} runtime copy/fill kernels inside the profiled region")
    memcopy = directory / f"{prefix}_memory_copy_trace.csv"
    if memcopy.exists() and read_csv(memcopy):
        raise ValueError("memory copies inside the profiled region")
    markers = directory / f"{prefix}_marker_api_trace.csv"
    if markers.exists():
        control = Counter(m["Function"] for m in read_csv(markers))
        if control["roctxProfilerResume"] != 1 or control["roctxProfilerPause"] != 1:
            raise ValueError(f"expected one profiler region, found {dict(control)}")
    if len(kernels) != metadata["kernels"]:
        raise ValueError(f"expected {metadata['kernels']} kernel dispatches, found {len(kernels)}")
    spans = [(int(k["Start_Timestamp"]), int(k["End_Timestamp"])) for k in kernels]
    if any(end <= start for start, end in spans):
        raise ValueError("a kernel interval ends before it starts")
    apis = []
    api_path = directory / f"{prefix}_hip_api_trace.csv"
    if api_path.exists():
        apis = read_csv(api_path)
    counts = Counter(a["Function"] for a in apis)
    if apis:
        launches = sum(counts[f] for f in LAUNCH_APIS)
        graphs = sum(counts[f] for f in GRAPH_APIS)
        if metadata["graph_launches"] is None:
            if launches != metadata["kernels"] or graphs:
                raise ValueError(f"expected {metadata['kernels']} kernel launches and no graph launch, "
                                 f"found {launches} and {graphs}")
        elif graphs != metadata["graph_launches"] or launches:
            raise ValueError(f"expected {metadata['graph_launches']} graph launches and no kernel launch, "
                             f"found {graphs} and {launches}")
    origin, stop = min(s for s, _ in spans), max(e for _, e in spans)
    stats = intervals_summary(spans)
    families, streams = defaultdict(float), defaultdict(float)
    for k, (start, end) in zip(kernels, spans):
        families[family(k["Kernel_Name"])] += (end - start) / 1e3
        streams[k.get("Stream_Id", "")] += (end - start) / 1e3
    summary = {
        "case": metadata["case"], "requests": metadata["requests"], "mode": metadata["mode"],
        "group": metadata["group"], "steps": metadata["steps"], "serial": metadata.get("serial", False),
        "kernels": len(kernels), "span_us": (stop - origin) / 1e3, "busy_us": stats["busy_ns"] / 1e3,
        "idle_us": (stop - origin - stats["busy_ns"]) / 1e3, "overlap_us": stats["overlap_ns"] / 1e3,
        "overlap_fraction": stats["overlap_ns"] / (stop - origin), "max_concurrent_kernels": stats["max_concurrent"],
        "sum_kernel_us": sum(families.values()),
        "family_kernel_us": dict(sorted(families.items(), key=lambda kv: -kv[1])),
        "stream_kernel_us": dict(streams), "hip_api_counts": dict(counts),
        "burst_wall_us": metadata.get("wall_us"), "burst_span_us": metadata.get("span_us"),
    }
    counters = directory / f"{prefix}_counter_collection.csv"
    if counters.exists():
        hbm = defaultdict(float)
        for row in read_csv(counters):
            value = float(row["Counter_Value"]) * 1024
            if row["Counter_Name"] == "FETCH_SIZE":
                hbm[family(row["Kernel_Name"])] += value * fetch_scale
            elif row["Counter_Name"] == "WRITE_SIZE":
                hbm[family(row["Kernel_Name"])] += value
        summary["family_hbm_bytes"] = dict(hbm)
    # Chrome trace: GPU kernels on packed lanes (pid 1), host API calls by thread (pid 2).
    lanes = pack_lanes(spans)
    events = []
    for k, (start, end), lane in zip(kernels, spans, lanes):
        events.append({"name": family(k["Kernel_Name"]), "cat": "GPU kernel", "ph": "X", "pid": 1, "tid": lane,
                       "ts": (start - origin) / 1e3, "dur": (end - start) / 1e3,
                       "args": {"kernel": k["Kernel_Name"], "stream": k.get("Stream_Id"), "queue": k.get("Queue_Id"),
                                "dispatch": k.get("Dispatch_Id"), "grid": k.get("Grid_Size_X"),
                                "block": k.get("Workgroup_Size_X")}})
    for a in apis:
        events.append({"name": a["Function"], "cat": "HIP API", "ph": "X", "pid": 2, "tid": int(a["Thread_Id"]),
                       "ts": (int(a["Start_Timestamp"]) - origin) / 1e3,
                       "dur": (int(a["End_Timestamp"]) - int(a["Start_Timestamp"])) / 1e3})
    shift = -min((e["ts"] for e in events), default=0.0)
    for e in events:
        e["ts"] += shift
    meta = [{"ph": "M", "name": "process_name", "pid": 1, "args": {"name": "GPU kernels (packed lanes)"}},
            {"ph": "M", "name": "process_name", "pid": 2, "args": {"name": "Host HIP API"}}]
    meta += [{"ph": "M", "name": "thread_name", "pid": 1, "tid": lane, "args": {"name": f"lane {lane}"}}
             for lane in sorted(set(lanes))]
    with gzip.GzipFile(filename=str(directory / f"{prefix}.trace.json.gz"), mode="wb", mtime=0) as handle:
        handle.write(json.dumps({"traceEvents": meta + events, "displayTimeUnit": "us"},
                                separators=(",", ":")).encode())
    return summary


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("directory", type=Path)
    parser.add_argument("--prefix", default="run")
    parser.add_argument("--metadata", type=Path, help="defaults to <directory>/<prefix>.json")
    parser.add_argument("--fetch-scale", type=float, default=1.0,
                        help="factor for FETCH_SIZE (what a copy of known size calibrates it to)")
    args = parser.parse_args()
    metadata = json.loads((args.metadata or args.directory / f"{args.prefix}.json").read_text())
    if not metadata.get("complete"):
        raise SystemExit("incomplete profile metadata")
    summary = analyze(args.directory, args.prefix, metadata, args.fetch_scale)
    (args.directory / f"{args.prefix}.summary.json").write_text(json.dumps(summary, indent=1) + "\n")
    print(json.dumps(summary, indent=1))


if __name__ == "__main__":
    main()
