"""What parallel branches cost and gain in this runtime's DAG graphs.

Two programs launch the same four kernels with the same grids: a root `work` launch, two `work`
launches that read its output, and `join2`, which adds their outputs. In `fork_join` the two middle
launches are independent (a fork and a join in the dependency DAG); in `chain` the second one reads
the first one's output instead of the root's, so the DAG is a chain of four. Each is timed in
run mode "branches" (an explicit hipGraph, one kernel node per dispatch, with the reduced DAG's
edges: where the fork lets the two branches run at once) and "capture" (the launches captured on
one stream), with HIP events over many submissions. With branches that overlap, the fork/join
graph saves up to one `work` launch against the chain; what it saves less than that is the cost of
its fork and join in this runtime.

`work` keeps every thread busy for `rounds` dependent multiply-adds, so its duration is set by
`rounds` and hardly by memory; `--elements` sets how much of the GPU one launch occupies (64: one
wave; 1 << 20: 4096 workgroups of 256 threads, every compute unit busy). Results are checked
against the same arithmetic in NumPy (f32, no contraction).

    python3 composable-kernel-language_amd/programs/branch_cost.py [--elements 64 1048576] [--rounds 2048]
"""
from __future__ import annotations

import argparse
import json
import statistics
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
for path in (HERE.parent / "python", HERE.parent):
    sys.path.insert(0, str(path))

import numpy as np  # noqa: E402

import ckl  # noqa: E402

N = ckl.dim("N")
Line = ckl.Buffer[ckl.f32, (N,)]
THREADS = 256
DECAY, STEP = 0.999, 0.5


@ckl.kernel
def work(src: Line, dst: Line, rounds: ckl.constexpr[ckl.index]) -> None:
    """dst = src after `rounds` applications of v -> v * DECAY + STEP."""
    i = ckl.global_id(0)
    if i < N:
        v = src[i]
        for _ in range(rounds):
            v = v * DECAY + STEP
        dst[i] = v


@ckl.kernel
def join2(a: Line, b: Line, dst: Line) -> None:
    i = ckl.global_id(0)
    if i < N:
        dst[i] = a[i] + b[i]


@ckl.program
def fork_join(src: Line, dst: Line, rounds: ckl.constexpr[ckl.index]) -> None:
    root = ckl.empty_like(src)
    left = ckl.empty_like(src)
    right = ckl.empty_like(src)
    grid = (ckl.cdiv(N, THREADS),)
    ckl.launch(work, src, root, rounds, grid=grid, block=(THREADS,))
    ckl.launch(work, root, left, rounds, grid=grid, block=(THREADS,))
    ckl.launch(work, root, right, rounds, grid=grid, block=(THREADS,))
    ckl.launch(join2, left, right, dst, grid=grid, block=(THREADS,))


@ckl.program
def chain(src: Line, dst: Line, rounds: ckl.constexpr[ckl.index]) -> None:
    root = ckl.empty_like(src)
    left = ckl.empty_like(src)
    right = ckl.empty_like(src)
    grid = (ckl.cdiv(N, THREADS),)
    ckl.launch(work, src, root, rounds, grid=grid, block=(THREADS,))
    ckl.launch(work, root, left, rounds, grid=grid, block=(THREADS,))
    ckl.launch(work, left, right, rounds, grid=grid, block=(THREADS,))
    ckl.launch(join2, left, right, dst, grid=grid, block=(THREADS,))


def expected(x: np.ndarray, rounds: int, kind: str) -> np.ndarray:
    def apply(v):
        v = v.copy()
        for _ in range(rounds):
            v = (v * np.float32(DECAY)).astype(np.float32) + np.float32(STEP)
        return v
    root = apply(x)
    left = apply(root)
    right = apply(root if kind == "fork_join" else left)
    return left + right


def measure(device, elements: int, rounds: int, samples: int, iterations: int) -> dict:
    spec = ckl.BufferSpec((elements,), ckl.f32)
    x = np.random.default_rng(7).uniform(-1, 1, elements).astype(np.float32)
    src, dst = device.empty(spec), device.empty(spec)
    src.copy_from_host(x)
    out = {}
    for label, program in (("fork_join", fork_join), ("chain", chain)):
        compiled = program.lower(signature={"src": spec, "dst": spec}, constants={"rounds": rounds}).compile(
            fuse_pointwise=False)
        inv = compiled.bind(src, dst)
        want = expected(x, rounds, label)
        row = {"edges_branches": inv.edge_count(mode="branches")}
        for mode in ("branches", "capture"):
            inv.run(mode=mode)
            got = np.empty_like(x)
            dst.copy_to_host(got)
            if not np.array_equal(got, want):
                raise AssertionError(f"{label} {mode}: result differs from the NumPy arithmetic")
            inv.benchmark(iterations=iterations, mode=mode)
            runs = [inv.benchmark(iterations=iterations, mode=mode)["stream_us"] for _ in range(samples)]
            row[f"{mode}_us"] = statistics.median(runs)
        # One `work` launch alone: the unit the fork can save.
        row["node_us"] = [inv.time_node(k, iterations) for k in range(inv.node_count)]
        out[label] = row
    fj, ch = out["fork_join"], out["chain"]
    work_us = statistics.median(fj["node_us"][:3] + ch["node_us"][:3])
    out["work_launch_us"] = work_us
    out["saved_by_fork_us"] = ch["branches_us"] - fj["branches_us"]
    out["fork_join_cost_us"] = work_us - out["saved_by_fork_us"]
    return out


def main() -> None:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--elements", type=int, nargs="+", default=[64, 1 << 20])
    parser.add_argument("--rounds", type=int, default=2048)
    parser.add_argument("--samples", type=int, default=7)
    parser.add_argument("--iterations", type=int, default=200)
    args = parser.parse_args()
    device = ckl.Device()
    result = {"rounds": args.rounds, "cases": {}}
    for elements in args.elements:
        result["cases"][str(elements)] = measure(device, elements, args.rounds, args.samples, args.iterations)
        print(json.dumps({str(elements): result["cases"][str(elements)]}), file=sys.stderr, flush=True)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
