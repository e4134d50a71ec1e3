#!/usr/bin/env python3
"""Decode-step benchmark of the CKL MI355X backend (one GPU).

For each decoder configuration (small, wide, deep, large) the decode program is
lowered, compiled with storage reuse off and on, bound to device-resident synthetic state,
prefilled on the GPU (teacher-forced prompt), and timed per variant with the protocol of the
reference harness (benchmarks/decoder/run.py:160-197): every sample resets the mutable state and
times one 16-step generation with HIP events on the invocation stream; samples rotate and reverse
the variant order; the median microseconds per decode step is reported.

Variants (run.py:24-38): sequential/capture/inferred with reuse off and on, and the 16-step
batched capture/inferred graphs. "inferred" executes the DAG-derived graph; "capture" is a
single-stream capture of ordinary launches.

Output: one JSON line on stdout (details per configuration under "configs"); human-readable
progress on stderr. The CPU baseline (NumPy restatement of the reference decoder step) is timed on
this host's cores on the same inputs and is also the checker of the measured runs' tokens.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for path in (ROOT / "composable-kernel-language_amd" / "python", ROOT / "composable-kernel-language_amd", ROOT):
    sys.path.insert(0, str(path))

import numpy as np  # noqa: E402

HBM_PEAK = 8.0e12          # MI355X HBM3E bytes/s
METRIC = "median µs/decode step: inferred hipGraph vs stream capture; scratch bytes"


def log(*parts):
    print(*parts, file=sys.stderr, flush=True)


def variants(steps):
    return [("sequential", False, "ordinary", 1), ("capture", False, "capture", 1), ("inferred", False, "graph", 1),
            ("sequential_reuse", True, "ordinary", 1), ("capture_reuse", True, "capture", 1),
            ("inferred_reuse", True, "graph", 1), ("batched_capture", True, "capture", steps),
            ("batched_inferred", True, "graph", steps)]


def algorithmic_step_bytes(c, position):
    """HBM bytes one decode step must move at `position` (weights + KV read/write + logits +
    embedding gather): 4*[L(4C^2+3CF) + CV + (2L+1)C + BC] + 8*L*B*A*D*(p+1) + 8*L*B*A*D + 4*B*V."""
    b, h, l, f, v, a, d = c.batch, c.hidden, c.layers, c.ffn, c.vocab, c.heads, c.head_dim
    weights = 4 * (l * (4 * h * h + 3 * h * f) + h * v + (2 * l + 1) * h + b * h)
    kv_read = 8 * l * b * a * d * (position + 1)
    kv_write = 8 * l * b * a * d
    return weights + kv_read + kv_write + 4 * b * v


def decoder_node_bytes(c, position):
    """Algorithmic HBM bytes of every dispatch of one decode step at `position`, in plan order
    (the order of the decode program's launches): each kernel's compulsory reads and writes."""
    b, h, f, v, a, d = c.batch, c.hidden, c.ffn, c.vocab, c.heads, c.head_dim
    rows, r = position + 1, d // 2
    hidden = 4 * b * h

    def linear(i, o):
        return ("linear", 4 * (b * i + i * o + b * o))

    nodes = [("embedding", 2 * hidden + 4 * b)]
    for _ in range(c.layers):
        nodes += [("rms_stats", hidden + 4 * b), ("rms_apply", 2 * hidden + 4 * h + 4 * b),
                  linear(h, h), linear(h, h), linear(h, h),
                  ("rope", 2 * hidden + 8 * r), ("rope", 2 * hidden + 8 * r), ("append_kv", 4 * hidden),
                  ("attention_scores", hidden + 4 * b * a * rows * d + 4 * b * a * rows),
                  ("softmax", 8 * b * a * rows),
                  ("attention_values", 4 * b * a * rows + 4 * b * a * rows * d + hidden),
                  linear(h, h), ("add", 3 * hidden), ("rms_stats", hidden + 4 * b),
                  ("rms_apply", 2 * hidden + 4 * h + 4 * b), linear(h, f), linear(h, f),
                  ("silu", 8 * b * f), ("multiply", 12 * b * f), linear(f, h), ("add", 3 * hidden)]
    nodes += [("rms_stats", hidden + 4 * b), ("rms_apply", 2 * hidden + 4 * h + 4 * b), linear(h, v),
              ("greedy", 4 * b * v + 8 * b), ("advance", 8)]
    return nodes


LIGHT_RESET = ("tokens", "position", "history", "logits")


def time_variants(session, c, samples, warmup, log_prefix, only=None):
    """Timing resets restore the small mutable state only: every run rewrites the cache rows it
    reads (positions >= the prefill position) before reading them, with deterministic kernels."""
    state = session.state
    rows = [row for row in variants(c.steps) if not only or row[0] in only]
    metrics = {name: [] for name, *_ in rows}
    setup = {}
    for name, reuse, mode, group in rows:
        inv = session.invocations[reuse]
        state.reset(LIGHT_RESET)
        setup[name] = inv.benchmark(iterations=1, mode=mode, batch_size=group)["graph_setup_ms"]
        for _ in range(warmup):
            state.reset(LIGHT_RESET)
            inv.benchmark(iterations=c.steps // group, mode=mode, batch_size=group)
    results = {}
    for sample in range(samples):
        offset = sample % len(rows)
        order = rows[offset:] + rows[:offset]
        if sample % 2:
            order = list(reversed(order))
        for name, reuse, mode, group in order:
            inv = session.invocations[reuse]
            state.reset(LIGHT_RESET)
            timing = inv.benchmark(iterations=c.steps // group, mode=mode, batch_size=group)
            metrics[name].append(timing["stream_us"])
            results.setdefault(name, []).append(timing["wall_us"])
    table = {}
    for name, reuse, mode, group in rows:
        launches = session.invocations[reuse].launch_count(mode=mode, batch_size=group)
        table[name] = dict(median_us=statistics.median(metrics[name]), min_us=min(metrics[name]),
                           max_us=max(metrics[name]), wall_us=statistics.median(results[name]),
                           graph_setup_ms=setup[name], launches_per_submission=launches, steps_per_submission=group,
                           samples=metrics[name])
        log(f"{log_prefix} {name:18s} {table[name]['median_us']:9.2f} us/step  launches/submission={launches}")
    return table


def run_config(name, c, args, device):
    from programs.harness import DecoderSession, synthetic_inputs
    t0 = time.time()
    arrays, prompts = synthetic_inputs(c, args.seed, init="baseline")
    session = DecoderSession(c, device, arrays=arrays)
    t1 = time.time()
    session.prefill(prompts, mode="ordinary", progress=lambda done, total: log(f"[{name}] prefill {done}/{total}"))
    t2 = time.time()
    log(f"[{name}] inputs+compile+bind {t1 - t0:.1f}s, device prefill of {c.context - 1} steps {t2 - t1:.2f}s")
    table = time_variants(session, c, args.samples, args.warmup, f"[{name}]", args.variants)
    heap = {}
    for reuse, program in session.programs.items():
        heap[str(reuse)] = sum(int(line.split("bytes = ")[1].split(" ")[0]) for line in program.executable_ir.splitlines()
                               if '"ckl_exec.heap"' in line)
    # State after one timed generation (the checker compares it with the CPU oracle).
    session.state.reset()
    session.invocations[True].run(mode="graph" if "batched_inferred" in table else "ordinary", batch_size=c.steps)
    final = {k: session.state.download(k) for k in ("tokens", "history", "position", "logits")}

    def median(variant):
        return table[variant]["median_us"] if variant in table else None

    def ratio(slow, fast):
        return median(slow) / median(fast) if median(slow) and median(fast) else None

    position = c.context - 1
    mean_bytes = statistics.mean(algorithmic_step_bytes(c, position + s) for s in range(c.steps))
    step_us = median("batched_inferred") or min(v["median_us"] for v in table.values())
    result = dict(config=vars(c), steps=c.steps, variants=table,
                  inferred_us=median("inferred"), capture_us=median("capture"), ordinary_us=median("sequential"),
                  inferred_over_capture=ratio("capture", "inferred"),
                  inferred_reuse_over_capture_reuse=ratio("capture_reuse", "inferred_reuse"),
                  scratch_bytes={"reuse_off": heap["False"], "reuse_on": heap["True"]},
                  tokens_per_s=c.batch * 1e6 / step_us,
                  algorithmic_bytes_per_step=mean_bytes,
                  step_hbm_fraction=mean_bytes / (step_us * 1e-6) / HBM_PEAK)
    log(f"[{name}] inferred/capture speedup {result['inferred_over_capture']}; scratch {heap['False']} -> {heap['True']} B; "
        f"step roofline {result['step_hbm_fraction']:.3f} of 8 TB/s")
    return session, result, final


def c_name(c):
    from programs.decoder_config import CONFIGS
    return next((k for k, v in CONFIGS.items() if (v.batch, v.hidden, v.layers, v.vocab) == (c.batch, c.hidden, c.layers, c.vocab)), None)


def measured_traffic(config, family):
    """HBM bytes per launch of `family` on `config` from the committed rocprofv3 FETCH_SIZE and
    WRITE_SIZE passes (profiles/decoder_<config>_hbm_traffic.json, scaled by the copy-kernel
    calibration); None when no such measurement exists."""
    path = ROOT / "profiles" / f"decoder_{config}_hbm_traffic.json"
    if not config or not path.exists():
        return None
    return json.loads(path.read_text()).get("families", {}).get(family)


def unit_family(name):
    """Kernel family of an inferred-step launch: the library family of a plain, grouped or
    shared-operand dispatch ("ckl_linear_mfma1x1_group" -> "linear"), or the chain entry point
    itself (chain entry points join their members' names with "__")."""
    name = name[len("ckl_"):] if name.startswith("ckl_") else name
    name = name[:-len("_group")] if name.endswith("_group") else name
    return "linear" if name.startswith("linear_") and "__" not in name else name


def kernel_roofline(session, c, samples=7):
    """Time every launch of the inferred step (chains contracted, siblings grouped: what the
    headline mode executes) in sequence on the invocation stream, operands as cold as in a graph
    replay: launch k's duration is the difference of the median HIP-event times of the step's
    first k+1 and first k launches (`samples` repeats each). Returns per-family totals and the roofline entry of the dominant family
    (largest total time per step): algorithmic bytes per launch / average launch duration. A
    launch's algorithmic bytes are the sum of its plan nodes' less the hand-offs a chain keeps on
    chip (the attention chain's scores and probabilities, silu's output, the rotated q and k)."""
    inv = session.invocations[False]   # the headline (inferred, storage reuse off) plan
    position = c.context - 1
    nodes = decoder_node_bytes(c, position)
    if len(nodes) != inv.node_count:
        raise AssertionError("plan does not have the decode program's dispatch count")
    units = inv.units()
    session.state.reset(LIGHT_RESET)
    durations = inv.profile_units(samples)
    session.state.reset()
    b, h, f, a, rows = c.batch, c.hidden, c.ffn, c.heads, position + 1
    # Hand-offs a chain keeps on chip (written by one member, read by the next): not HBM traffic.
    on_chip = {"attention_scores__softmax__attention_values": 16 * b * a * rows,   # scores, probs
               "softmax__attention_values": 8 * b * a * rows,                     # probs
               "silu__multiply": 8 * b * f,                                        # activation
               "rope__rope__append_kv": 8 * b * h,                                 # rotated k
               # rotated k, the attention's read of the rotated q, scores, probs
               "rope__rope__append_kv__attention_scores__softmax__attention_values": 12 * b * h + 16 * b * a * rows,
               "linear_rowvec__add__rms_stats__rms_apply": 8 * b * h,                 # linear output
               "linear_rowvec__linear_rowvec__silu__multiply": 24 * b * f,            # gate, up, activation
               # linear output, normalized row; gate, up, activation
               "linear_rowvec__add__rms_stats__rms_apply__linear_rowvec__linear_rowvec__silu__multiply":
                   16 * b * h + 24 * b * f,
               "embedding__rms_stats__rms_apply__linear_rowvec__linear_rowvec__linear_rowvec": 8 * b * h,  # normalized row
               "linear_rowvec__greedy__advance": 4 * b * c.vocab}                  # greedy's read of the logits
    per_kernel = {}
    for index, (name, members) in enumerate(units):
        families = {nodes[m][0] for m in members}
        family = unit_family(name)
        if family == "linear" and families != {"linear"}:
            raise AssertionError(f"launch {index} ({name}) runs non-linear plan nodes")
        if family == "advance":
            continue
        us = durations[index]
        entry = per_kernel.setdefault(family, {"launches": 0, "total_us": 0.0, "bytes": 0, "entries": set(), "nodes": 0})
        entry["launches"] += 1
        entry["nodes"] += len(members)
        entry["total_us"] += us
        entry["bytes"] += sum(nodes[m][1] for m in members) - on_chip.get(family, 0)
        entry["entries"].add(name)
    session.state.reset()
    summary = {k: {"launches": v["launches"], "plan_nodes": v["nodes"], "avg_us": v["total_us"] / v["launches"],
                   "total_us": v["total_us"], "algorithmic_bytes": v["bytes"],
                   "achieved_GBps": v["bytes"] / v["total_us"] / 1e3, "entry_points": sorted(v["entries"])}
               for k, v in sorted(per_kernel.items(), key=lambda kv: -kv[1]["total_us"])}
    dominant = next(iter(summary))
    entry = summary[dominant]
    avg = entry["avg_us"]
    per_launch = entry["algorithmic_bytes"] / entry["launches"]
    achieved = per_launch / (avg * 1e-6)
    roofline = {"bound": "hbm", "kernel": f"ckl_{dominant}", "achieved": achieved / 1e9, "peak": HBM_PEAK / 1e9,
                "unit": "GB/s", "frac": achieved / HBM_PEAK, "traffic": measured_traffic(c_name(c), dominant),
                "algorithmic_bytes_per_launch": per_launch, "avg_launch_us": avg, "launches_per_step": entry["launches"],
                "config": c_name(c), "position": position, "mode": "inferred step launches in sequence (prefix differences)"}
    return summary, dominant, roofline


def cpu_baseline(session, c, final, threads=None):
    """NumPy oracle (restatement of the reference's reference.py step) timed on this host, from the
    same prefilled state; also checks the GPU generation's tokens and logits."""
    from oracle import decoder as oracle
    state = session.state
    initial = {k: (v.copy() if k in oracle.MUTABLE else v) for k, v in state.initial.items()}
    steps = c.steps
    times = []
    reference = None
    samples = 3 if c.hidden >= 1024 else 7
    for _ in range(samples):
        start = time.perf_counter()
        reference = oracle.expected(initial, c, steps)
        times.append((time.perf_counter() - start) / steps * 1e6)
    ok_tokens = np.array_equal(final["history"], reference["history"]) and np.array_equal(final["tokens"], reference["tokens"])
    logits_err = float(np.max(np.abs(final["logits"] - reference["logits"]) / (np.abs(reference["logits"]) + 1e-6)))
    close = bool(np.allclose(final["logits"], reference["logits"], atol=2e-5, rtol=3e-4))
    return dict(value=statistics.median(times), unit="us/step", cores=threads or os.cpu_count(), kind="port",
                sample=f"{samples} x {steps}-step NumPy generations from the GPU-prefilled state, B={c.batch}",
                tokens_match=bool(ok_tokens), logits_allclose=close, logits_max_rel_err=logits_err)


def vector_pipeline(device, samples):
    import ckl
    from programs import vector_pipeline as vp
    n = 1048576
    compiled = {reuse: vp.lower(n).compile(fuse_pointwise=False, reuse_storage=reuse) for reuse in (False, True)}
    spec = ckl.BufferSpec((n,), ckl.f32)
    src, dst = device.empty(spec), device.empty(spec)
    x = np.random.default_rng(123).uniform(-1, 1, n).astype(np.float32)
    src.copy_from_host(x)
    inv = compiled[True].bind(src, dst, 0.5)
    out = {}
    for mode in ("ordinary", "capture", "graph"):
        inv.run(mode=mode)
        got = np.empty_like(x)
        dst.copy_to_host(got)
        assert np.array_equal(got, (x + np.float32(0.5)) + np.float32(0.5))
        inv.benchmark(iterations=20, mode=mode)
        out[mode] = statistics.median(inv.benchmark(iterations=100, mode=mode)["stream_us"] for _ in range(samples))
    heap = {str(r): sum(int(l.split("bytes = ")[1].split(" ")[0]) for l in p.executable_ir.splitlines()
                        if '"ckl_exec.heap"' in l) for r, p in compiled.items()}
    log(f"[vector_pipeline] us/step {out}; heap {heap}")
    return dict(us_per_step=out, heap_bytes=heap, bytes_per_step=16 * n)


def main():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=16, help="decode steps per timed generation (config steps)")
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--samples", type=int, default=7)
    parser.add_argument("--seed", type=int, default=123)
    parser.add_argument("--configs", nargs="+", default=["small", "wide", "deep", "large"])
    parser.add_argument("--variants", nargs="+", default=None, choices=[v[0] for v in variants(16)],
                        help="time only these variants (default: all); kernel timings and the roofline do "
                             "not depend on the run mode")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--output", type=Path, default=None, help="also write the full JSON result here")
    args = parser.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: every box here has one MI355X; "
                          "multi-GPU sharding is a design note (DESIGN.md), not a measured path"}))
        sys.exit(2)
    import dataclasses
    import ckl
    from programs.decoder_config import CONFIGS

    device = ckl.Device()
    log(f"device: {device.name}")
    configs = {}
    headline = None
    for name in args.configs:
        c = dataclasses.replace(CONFIGS[name], steps=args.steps)
        session, result, final = run_config(name, c, args, device)
        summary, dominant, roofline = kernel_roofline(session, c)
        result["kernels"] = summary
        for family, row in summary.items():
            log(f"[{name}] {family:38s} launches={row['launches']:3d} avg={row['avg_us']:9.2f} us "
                f"total={row['total_us']:9.2f} us  {row['achieved_GBps']:8.1f} GB/s")
        # A prefix difference at or below zero is launch-latency noise of a few-microsecond step:
        # no bandwidth is derived from it.
        result["kernel_families"] = {k: {"launches": v["launches"], "avg_us": v["avg_us"],
                                         "achieved_GBps": v["achieved_GBps"] if v["avg_us"] > 0 else None,
                                         "frac": v["achieved_GBps"] * 1e9 / HBM_PEAK if v["avg_us"] > 0 else None}
                                     for k, v in summary.items()}
        if name == "large":
            result["roofline"] = roofline
            log(f"[large] dominant kernel {dominant}: {roofline}")
        if not args.no_cpu_baseline and name in ("small",):
            result["cpu_baseline"] = cpu_baseline(session, c, final)
            log(f"[{name}] cpu baseline {result['cpu_baseline']}")
        configs[name] = result
        if name == "small":
            headline = result
        del session
    vector = vector_pipeline(device, args.samples)
    head = headline or next(iter(configs.values()))
    value = next(v for v in (head["inferred_us"], head["ordinary_us"], head["capture_us"]) if v is not None)
    large = configs.get("large", {})
    line = {
        "metric": METRIC, "value": value, "unit": "us/step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": value / 1000.0, "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded N(0,0.02) weights, random prompts)",
        "config": {"workload": "small decoder (B8 C64 A4x16 L2 F256 V256, ctx 16, 16 greedy steps)",
                   "inferred_us": head["inferred_us"], "capture_us": head["capture_us"],
                   "ordinary_us": head["ordinary_us"], "inferred_over_capture": head["inferred_over_capture"],
                   "scratch_bytes": head["scratch_bytes"], "tokens_per_s": head["tokens_per_s"]},
        "roofline": large.get("roofline"),
        "cpu_baseline": head.get("cpu_baseline"),
        "configs": {k: {kk: vv for kk, vv in v.items() if kk not in ("variants", "kernels")} |
                    {"variants": {vn: {"median_us": vv["median_us"], "launches": vv["launches_per_submission"]}
                                  for vn, vv in v["variants"].items()}} for k, v in configs.items()},
        "vector_pipeline": vector,
        "host": {"cpu": platform.processor() or platform.machine(), "nproc": os.cpu_count(), "numpy": np.__version__},
    }
    if args.output:
        full = dict(line, configs_full=configs)
        args.output.write_text(json.dumps(full, indent=1, default=float) + "\n")
    print(json.dumps(line, default=float))


if __name__ == "__main__":
    main()
