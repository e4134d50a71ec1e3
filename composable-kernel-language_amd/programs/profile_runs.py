"""One warmed, self-checked decode burst inside a profiler region, for rocprofv3.

The collection half of the trace pipeline (benchmarks/decoder/collect.py:14-93 and the
`--profile` path of experiment.py:110-130 in the reference). The requests of one decoder
configuration are bound to GPU-prefilled state (one request: a single invocation; several:
`programs.harness.RequestGroup`, shared weights, one stream each), the burst (`--steps` decode
steps of every request in `--mode`, `--group` steps per submission) runs once untimed to build
graphs and record the result, then the state is reset and the same burst runs again between
`ckl.profiler_region(True)` and `ckl.profiler_region(False)`. The profiled burst must leave the
unprofiled burst's state bit for bit, so a trace is never taken of a wrong run. A metadata file
beside the trace states what the analysis must find (programs/trace_analysis.py). rocprofv3 (ROCm
7.2) honours the region's roctx calls only when it also traces markers (`--marker-trace`):

    rocprofv3 --selected-regions --marker-trace --kernel-trace --hip-runtime-trace \\
        --memory-copy-trace --output-format csv -d out -o run -- \\
        python3 composable-kernel-language_amd/programs/profile_runs.py --case small --requests 4 \\
        --mode graph --metadata out/run.json
    python3 composable-kernel-language_amd/programs/trace_analysis.py out --prefix run
"""
from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
for path in (HERE.parent / "python", HERE.parent):
    sys.path.insert(0, str(path))

import numpy as np  # noqa: E402

MODES = ("ordinary", "graph", "capture", "branches", "contracted", "stream")


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--case", default="small")
    parser.add_argument("--requests", type=int, default=1)
    parser.add_argument("--mode", choices=MODES, default="graph")
    parser.add_argument("--group", type=int, default=1, help="decode steps per submission")
    parser.add_argument("--steps", type=int, default=16)
    parser.add_argument("--serial", action="store_true", help="requests one after another, not side by side")
    parser.add_argument("--metadata", type=Path, required=True)
    args = parser.parse_args()
    if min(args.requests, args.group, args.steps) < 1 or args.steps % args.group:
        parser.error("positive counts and steps divisible by group are required")

    import ckl
    from programs.decoder_config import CONFIGS, MUTABLE
    from programs.harness import RequestGroup, synthetic_inputs

    c = CONFIGS[args.case]
    device = ckl.Device()
    inputs = [synthetic_inputs(c, 123, prompt_seed=1000 + i) for i in range(args.requests)]
    group = RequestGroup(c, device, [arrays for arrays, _ in inputs])
    group.prefill([prompts for _, prompts in inputs])

    def burst():
        return group.run(mode=args.mode, iterations=args.steps // args.group, batch_size=args.group,
                         serial=args.serial)

    def state():
        return [{k: s.download(k) for k in MUTABLE} for s in group.states]

    group.reset()
    burst()
    expected = state()
    group.reset()
    ckl.profiler_region(True)
    timing = burst()
    ckl.profiler_region(False)
    got = state()
    for a, b in zip(got, expected):
        for k in MUTABLE:
            if not np.array_equal(a[k], b[k]):
                raise AssertionError(f"the profiled burst left a different {k} than the unprofiled one")

    inv = group.invocations[0]
    launches = inv.launch_count(mode=args.mode, batch_size=args.group) * (args.steps // args.group)
    submissions = args.steps // args.group if args.mode != "ordinary" else None
    metadata = {
        "complete": True, "case": args.case, "config": vars(c), "requests": args.requests, "mode": args.mode,
        "group": args.group, "steps": args.steps, "serial": args.serial,
        "kernels_per_request": launches, "kernels": launches * args.requests,
        "graph_launches": None if args.mode in ("ordinary", "stream") else args.requests * submissions,
        "wall_us": timing["wall_us"], "span_us": timing["span_us"],
        "units": [name for name, _ in inv.units()] if args.mode in ("graph", "contracted", "stream") else None,
    }
    args.metadata.parent.mkdir(parents=True, exist_ok=True)
    args.metadata.write_text(json.dumps(metadata, indent=1) + "\n")
    print(f"{args.case} x{args.requests} {args.mode} group {args.group}: {launches * args.requests} kernels, "
          f"burst {timing['wall_us']:.1f} us wall, {timing['span_us']:.1f} us GPU span", flush=True)


if __name__ == "__main__":
    main()
