#!/usr/bin/env python3
"""Decode-step benchmark of the CKL MI355X backend (one GPU).

For each decoder configuration (small, wide, deep, large) the decode program is
lowered, compiled with storage reuse off and on, bound to device-resident synthetic state and
prefilled on the GPU (teacher-forced prompt). The NumPy checker (oracle/decoder.py, in a CPU-only
child process) then computes the expected state after 1, 16 and any partial generation's steps
from that prefilled state, and every variant is timed with the protocol of the reference harness
(benchmarks/decoder/run.py:160-197): every sample resets the mutable state and times one
generation with HIP events on the invocation stream; samples rotate and reverse the variant
order; the median microseconds per decode step is reported. Every run is verified
(run.py:172-196): each variant's first generation in full (tokens, history, position, logits,
the cache rows written, the prefill rows and unused suffix unchanged, sentinel tails), every
warmup and timed sample's tokens, history, position and logits, and the weights after all. A timed
sample's state is downloaded right after it and checked once all samples have run, so that no
check leaves the GPU idle between samples (after ~30 ms idle a large step runs ~2% slower).

Variants (run.py:24-38 plus ablations):
  sequential / capture / inferred       ordinary launches, single-stream capture, inferred graph
  branches                              one graph node per dispatch with the reduced DAG's edges
                                        (the reference's inferred graph: branch concurrency only)
  contracted                            the inferred graph's contracted and merged launches
                                        captured on one stream (launch contraction only)
  inferred_stream                       those launches issued on the stream, no graph (the cost
                                        of submitting them as a graph)
  *_reuse                               the same with storage reuse on
  batched_*                             16 steps per graph submission (storage reuse on)

--steps K: decode steps timed per variant, as generations of 16 steps from the prefilled state
and one shorter generation for the remainder (a batched variant rounds its samples up to whole
16-step submissions and reports its own count); --warmup W: untimed warmup steps per variant,
likewise. Each variant's first (verified) generation precedes its warmup, as in run.py:170-178.

Independent requests (`independent_requests`, small and wide): 8 invocations of one compiled
program with shared weights, each on its own stream, bursts of one 16-step generation per request
run side by side (ckl.run_requests), against the batching control (one invocation of 8 x B rows);
every burst's state is checked against the requests run one after another.

Output: one short JSON line on stdout (headline, roofline, CPU baseline, one summary per other
configuration); the full result (every variant's samples, kernel families, setup costs, vector
pipeline, independent requests) goes to --output (default: ckl_bench_detail.json in the system's
temporary directory); progress
on stderr. The headline `value` is the large decoder's inferred-graph median µs/step (the largest
single-GPU configuration of BASELINE.json). The CPU baseline times the same NumPy decoder step in
two child processes started before any GPU call (all cores, then one thread) after the GPU timing.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import shutil
import statistics
import subprocess
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for path in (ROOT / "composable-kernel-language_amd" / "python", ROOT / "composable-kernel-language_amd", ROOT):
    sys.path.insert(0, str(path))

import numpy as np  # noqa: E402

HBM_PEAK = 8.0e12          # MI355X HBM3E bytes/s
METRIC = "median µs/decode step: inferred hipGraph vs stream capture; scratch bytes"
HEADLINE = "large"
GENERATION = 16            # greedy steps per generation
DEFAULT_DETAIL = Path(tempfile.gettempdir()) / "ckl_bench_detail.json"


def log(*parts):
    print(*parts, file=sys.stderr, flush=True)


def variants(steps):
    return [("sequential", False, "ordinary", 1), ("capture", False, "capture", 1), ("inferred", False, "graph", 1),
            ("branches", False, "branches", 1), ("contracted", False, "contracted", 1),
            ("inferred_stream", False, "stream", 1),
            ("sequential_reuse", True, "ordinary", 1), ("capture_reuse", True, "capture", 1),
            ("inferred_reuse", True, "graph", 1), ("batched_capture", True, "capture", steps),
            ("batched_inferred", True, "graph", steps), ("batched_branches", True, "branches", steps)]


def generations(total: int) -> list:
    """Step counts of the generations that make up `total` decode steps: whole generations of
    GENERATION steps, then the remainder."""
    return [GENERATION] * (total // GENERATION) + ([total % GENERATION] if total % GENERATION else [])


def submissions(count: int, group: int) -> int:
    """Submissions of `group` steps that cover a generation of `count` steps."""
    return max(1, math.ceil(count / group))


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


def time_variants(session, c, steps, warmup, expected, log_prefix, only=None):
    """Times every variant over `steps` decode steps (generations(steps)) after `warmup` untimed
    ones, verifying every run against `expected` (step count -> expected state). Timing resets
    restore the small mutable state only: every run rewrites the cache rows it reads (positions
    >= the prefill position) before reading them, with deterministic kernels."""
    state = session.state
    rows = [row for row in variants(c.steps) if not only or row[0] in only]
    metrics = {name: [] for name, *_ in rows}
    walls = {name: [] for name, *_ in rows}
    timed = {name: 0 for name, *_ in rows}
    setup, errors, checked = {}, {name: {} for name, *_ in rows}, {name: 0 for name, *_ in rows}

    def record(name, found):
        for key, value in found.items():
            errors[name][key] = max(errors[name].get(key, 0.0), value)
        checked[name] += 1

    def verify(name, count, full=False):
        record(name, state.verify_generation(expected[count], full=full, longest=c.steps))

    for name, reuse, mode, group in rows:
        inv = session.invocations[reuse]
        state.reset(LIGHT_RESET)
        setup[name] = inv.benchmark(iterations=1, mode=mode, batch_size=group)["graph_setup_ms"]
        verify(name, group, full=True)
        for count in generations(warmup):
            state.reset(LIGHT_RESET)
            k = submissions(count, group)
            inv.benchmark(iterations=k, mode=mode, batch_size=group)
            verify(name, k * group)
    # Timed samples run back to back: each one's final state is downloaded right after it and
    # checked once all samples have run, so the GPU is not left idle for the tens of milliseconds
    # a check takes (an idle GPU starts the next sample below its steady-state clocks).
    captured = []
    for sample, count in enumerate(generations(steps)):
        offset = sample % len(rows)
        order = rows[offset:] + rows[:offset]
        if sample % 2:
            order = list(reversed(order))
        for name, reuse, mode, group in order:
            inv = session.invocations[reuse]
            state.reset(LIGHT_RESET)
            k = submissions(count, group)
            timing = inv.benchmark(iterations=k, mode=mode, batch_size=group)
            metrics[name].append(timing["stream_us"])
            walls[name].append(timing["wall_us"])
            timed[name] += k * group
            captured.append((name, k * group, state.capture()))
    for name, count, capture in captured:
        record(name, state.check_capture(capture, expected[count]))
    state.verify_read_only()
    table = {}
    for name, reuse, mode, group in rows:
        inv = session.invocations[reuse]
        launches = inv.launch_count(mode=mode, batch_size=group)
        edges = inv.edge_count(mode=mode, batch_size=group)
        table[name] = dict(median_us=statistics.median(metrics[name]), min_us=min(metrics[name]),
                           max_us=max(metrics[name]), wall_us=statistics.median(walls[name]),
                           graph_setup_ms=setup[name], launches_per_submission=launches, graph_edges=edges,
                           steps_per_submission=group, timed_steps=timed[name], samples=metrics[name],
                           runs_verified=checked[name], errors=errors[name])
        log(f"{log_prefix} {name:18s} {table[name]['median_us']:9.2f} us/step  launches/submission={launches}"
            f" edges={edges} timed_steps={timed[name]} verified_runs={checked[name]}")
    return table


def heap_bytes(program, op='"ckl_exec.heap"') -> int:
    """Bytes of the plan's temporaries' heaps (or, with op='"ckl_exec.workspace_heap"', of its
    library-workspace heap), read from the executable plan text."""
    return sum(int(line.split("bytes = ")[1].split(" ")[0]) for line in program.executable_ir.splitlines()
               if op in line)


def run_config(name, c, args, device, checker):
    from programs.harness import DecoderSession, synthetic_inputs
    t0 = time.time()
    arrays, prompts = synthetic_inputs(c, args.seed, init="baseline")
    session = DecoderSession(c, device, arrays=arrays)
    bind_allocations = {"reuse_off": session.invocations[False].bind_allocations,
                        "reuse_on": session.invocations[True].bind_allocations}
    t1 = time.time()
    session.prefill(prompts, mode="ordinary", progress=lambda done, total: log(f"[{name}] prefill {done}/{total}"))
    t2 = time.time()
    log(f"[{name}] inputs+compile+bind {t1 - t0:.1f}s, device prefill of {c.context - 1} steps {t2 - t1:.2f}s")
    counts = {1, c.steps} | {n for n in generations(args.steps) + generations(args.warmup)}
    expected = checker.expected(name, session, sorted(counts))
    log(f"[{name}] expected states for {sorted(counts)} steps from the NumPy checker in {time.time() - t2:.1f}s")
    table = time_variants(session, c, args.steps, args.warmup, expected, f"[{name}]", args.variants)
    # Temporaries the inferred graph moved out of storage the plan shares (decided at its first build).
    moved = {"reuse_off": session.invocations[False].private_bytes, "reuse_on": session.invocations[True].private_bytes}
    heap = {str(reuse): heap_bytes(program) for reuse, program in session.programs.items()}

    def median(variant):
        return table[variant]["median_us"] if variant in table else None

    def ratio(slow, fast):
        return median(slow) / median(fast) if median(slow) and median(fast) else None

    position = c.context - 1
    mean_bytes = statistics.mean(algorithmic_step_bytes(c, position + s) for s in range(c.steps))
    step_us = median("inferred") or min(v["median_us"] for v in table.values())
    normwise = max((v["errors"].get("logits_normwise", 0.0) for v in table.values()), default=None)
    result = dict(config=vars(c), steps=c.steps, variants=table,
                  inferred_us=median("inferred"), capture_us=median("capture"), ordinary_us=median("sequential"),
                  branches_us=median("branches"), contracted_us=median("contracted"),
                  stream_us=median("inferred_stream"), inferred_reuse_us=median("inferred_reuse"),
                  batched_inferred_us=median("batched_inferred"),
                  inferred_over_capture=ratio("capture", "inferred"),
                  branches_over_capture=ratio("capture", "branches"),
                  contracted_over_capture=ratio("capture", "contracted"),
                  stream_over_capture=ratio("capture", "inferred_stream"),
                  inferred_over_contracted=ratio("contracted", "inferred"),
                  inferred_reuse_over_capture_reuse=ratio("capture_reuse", "inferred_reuse"),
                  batched_branches_over_batched_capture=ratio("batched_capture", "batched_branches"),
                  scratch_bytes={"reuse_off": heap["False"], "reuse_on": heap["True"]},
                  workspace_bytes={"reuse_off": heap_bytes(session.programs[False], '"ckl_exec.workspace_heap"'),
                                   "reuse_on": heap_bytes(session.programs[True], '"ckl_exec.workspace_heap"')},
                  bind_allocations=bind_allocations,
                  moved_temporary_bytes=moved,
                  tokens_per_s=c.batch * 1e6 / step_us,
                  algorithmic_bytes_per_step=mean_bytes,
                  step_hbm_fraction=mean_bytes / (step_us * 1e-6) / HBM_PEAK,
                  logits_normwise=normwise,
                  runs_verified=sum(v["runs_verified"] for v in table.values()),
                  host_planning_ms={"lower": session.lower_ms, "compile_reuse_off": session.compile_ms[False],
                                    "compile_reuse_on": session.compile_ms[True]})
    log(f"[{name}] inferred/capture {result['inferred_over_capture']}; branches/capture {result['branches_over_capture']}; "
        f"contracted/capture {result['contracted_over_capture']}; scratch {heap['False']} -> {heap['True']} B; "
        f"workspaces {result['workspace_bytes']} B; step roofline {result['step_hbm_fraction']:.3f} of 8 TB/s; "
        f"{result['runs_verified']} runs verified, logits normwise <= {normwise:.2e}")
    return session, result


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
    for suffix in ("_shared2", "_shared3"):
        name = name[:-len(suffix)] if name.endswith(suffix) else name
    name = name[:-len("_nt")] if name.endswith("_nt") else name
    return "linear" if name.startswith("linear_") and "__" not in name else name


def kernel_roofline(session, c, samples=7):
    """Time every launch of the inferred step (chains contracted, siblings grouped: what the
    headline mode executes) in sequence on the invocation stream, operands as cold as in a graph
    replay: launch k's duration is the difference of the median HIP-event times of the step's
    first k+1 and first k launches (`samples` repeats each). Returns per-family totals and the
    roofline entry of the dominant family (largest total time per step): algorithmic bytes per
    launch / average launch duration. A launch's algorithmic bytes are the sum of its plan nodes'
    less the hand-offs a chain keeps on chip (the attention chain's scores and probabilities,
    silu's output, the rotated q and k)."""
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




# ---------------------------------------------------------------------------- CPU side
def cpu_threads() -> int:
    """Cores of this process's share: OMP_NUM_THREADS when set (16 on a one-GPU box), else the
    CPUs it may run on."""
    value = os.environ.get("OMP_NUM_THREADS", "")
    return int(value) if value.isdigit() and int(value) > 0 else len(os.sched_getaffinity(0))


def cpu_description() -> dict:
    model = ""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    blas = "unknown"
    try:
        deps = np.show_config(mode="dicts")["Build Dependencies"]
        blas = f"{deps['blas'].get('name')} {deps['blas'].get('version', '')}".strip()
    except Exception:  # noqa: BLE001 -- numpy builds differ in what show_config reports
        pass
    return {"cpu_model": model or platform.processor() or platform.machine(), "nproc": os.cpu_count(),
            "affinity_cpus": len(os.sched_getaffinity(0)), "numpy": np.__version__, "blas": blas}



def start_cpu_workers(directory: Path, timing: bool):
    """Start the CPU processes now, before this process makes any GPU call (their BLAS threads and
    memory are then not shared with the GPU process): the checker, with BLAS/OpenMP threads = this
    process's cores, which computes expected states on request and, with `timing`, then times the
    decoder step; and with `timing` a 1-thread process that times it single-threaded."""
    workers = {}
    roles = (("all", cpu_threads()), ("single", 1)) if timing else (("all", cpu_threads()),)
    for role, threads in roles:
        env = dict(os.environ, OMP_NUM_THREADS=str(threads), OPENBLAS_NUM_THREADS=str(threads),
                   MKL_NUM_THREADS=str(threads), BLIS_NUM_THREADS=str(threads))
        workers[role] = (threads, subprocess.Popen([sys.executable, str(Path(__file__).resolve()), "--cpu-worker",
                                                   str(directory), "--role", role], env=env))
    return workers


def wait_for(path: Path, alive, limit_s: float) -> bool:
    """Wait until `path` exists; give up when `alive()` turns false or after `limit_s` seconds."""
    deadline = time.time() + limit_s
    while time.time() < deadline:
        if path.exists():
            return True
        if not alive():
            return path.exists()
        time.sleep(0.1)
    return False


def load_state(folder: Path, mutable) -> dict:
    """The saved prefilled state: weights read-only, mutable arrays as copy-on-write views."""
    return {p.stem: np.load(p, mmap_mode="c" if p.stem in mutable else "r") for p in folder.glob("*.npy")}


def check_request(directory: Path, request: Path) -> None:
    """Expected states of one configuration: oracle.decoder.step from the saved prefilled state,
    the tokens, history, position, logits and written cache rows kept after each requested count."""
    from oracle import decoder as oracle
    from programs.decoder_config import Config
    spec = json.loads(request.read_text())
    c = Config(**spec["shape"])
    state = load_state(directory / spec["name"], oracle.MUTABLE)
    start = int(state["position"][0])
    counts = sorted(spec["counts"])
    out = {}
    for n in range(1, counts[-1] + 1):
        oracle.step(state, c)
        if n in counts:
            for key in ("tokens", "history", "position", "logits"):
                out[f"{n}.{key}"] = np.array(state[key])
            for key in ("kc", "vc"):
                out[f"{n}.{key}_rows"] = np.array(state[key][:, :, :, start:start + n])
    partial = directory / f"check.{spec['name']}.tmp.npz"
    np.savez(partial, **out)
    partial.rename(directory / f"check.{spec['name']}.npz")


def cpu_worker(directory: Path, role: str) -> None:
    """The CPU side of the benchmark. The "all" role answers check requests (check.<config>.json)
    as they come, then, on `go`, times oracle.decoder.step (the NumPy restatement of the
    reference's decode step) on each saved prefilled state; the "single" role waits for
    `go_single`. Either ends on `stop` or when the benchmark process is gone."""
    from oracle import decoder as oracle
    from programs.decoder_config import Config
    parent = os.getppid()
    go = directory / ("go" if role == "all" else "go_single")
    answered = set()
    deadline = time.time() + 3 * 3600
    while True:
        if os.getppid() != parent or (directory / "stop").exists() or time.time() > deadline:
            return
        if role == "all":
            for request in sorted(directory.glob("check.*.json")):
                if request.name not in answered:
                    check_request(directory, request)
                    answered.add(request.name)
        if go.exists():
            break
        time.sleep(0.05)
    manifest = json.loads(go.read_text())
    for name in manifest["configs"]:
        plan = manifest["plan"][name][role]
        c = Config(**manifest["shapes"][name])
        times = []
        for sample in range(plan["samples"]):
            state = load_state(directory / name, oracle.MUTABLE)     # each sample from the prefilled state
            start = time.perf_counter()
            for _ in range(plan["steps"]):
                oracle.step(state, c)
            times.append((time.perf_counter() - start) / plan["steps"] * 1e6)
        (directory / f"{name}.{role}.json").write_text(json.dumps(
            {"us_per_step": statistics.median(times), "samples": plan["samples"], "steps": plan["steps"], "times": times}))
    (directory / f"done.{role}").write_text("ok")


class Checker:
    """Expected decoder states from the CPU checker process (oracle/decoder.py run on the
    GPU-prefilled state), and the CPU baseline timing at the end."""

    def __init__(self, directory: Path, workers: dict):
        self.directory, self.workers = directory, workers

    def alive(self, role="all") -> bool:
        return self.workers[role][1].poll() is None

    def expected(self, name: str, session, counts) -> dict:
        folder = self.directory / name
        folder.mkdir(parents=True, exist_ok=True)
        for key, value in session.state.initial.items():
            np.save(folder / f"{key}.npy", np.ascontiguousarray(value))
        request = self.directory / f"check.{name}.json"
        partial = self.directory / f"request.{name}.tmp"
        partial.write_text(json.dumps({"name": name, "shape": vars(session.config), "counts": list(counts)}))
        partial.rename(request)
        answer = self.directory / f"check.{name}.npz"
        if not wait_for(answer, self.alive, 1800):
            raise RuntimeError(f"the NumPy checker gave no expected state for {name}")
        with np.load(answer) as data:
            out = {n: {"steps": n, **{key: data[f"{n}.{key}"] for key in
                                      ("tokens", "history", "position", "logits", "kc_rows", "vc_rows")}}
                   for n in counts}
        answer.unlink()
        return out

    def baselines(self, configs: dict) -> dict:
        """Release the timing processes (all cores, then one thread) and collect their timings."""
        from programs.decoder_config import CONFIGS
        if "single" not in self.workers:
            (self.directory / "stop").write_text("")
            return {}
        names = [n for n in configs if (self.directory / n).exists()]
        plan = {n: {"all": {"samples": 1 if n == "large" else 7, "steps": GENERATION},
                    "single": {"samples": 1 if n == "large" else 3, "steps": 4 if n == "large" else GENERATION}}
                for n in names}
        manifest = json.dumps({"configs": names, "plan": plan, "shapes": {n: vars(CONFIGS[n]) for n in names}})
        out = {}
        (self.directory / "go").write_text(manifest)
        ok = wait_for(self.directory / "done.all", self.alive, 3600)
        (self.directory / "go_single").write_text(manifest)
        ok_single = wait_for(self.directory / "done.single", lambda: self.alive("single"), 3600)
        if not ok:
            log("[cpu] the all-cores CPU baseline did not finish")
            return out
        for n in names:
            row = json.loads((self.directory / f"{n}.all.json").read_text())
            entry = {"value": row["us_per_step"], "unit": "us/step", "cores": self.workers["all"][0], "kind": "port",
                     "sample": f"{row['samples']} x {row['steps']}-step NumPy generation(s) of oracle/decoder.py "
                               f"from the GPU-prefilled state, B={CONFIGS[n].batch}"}
            if ok_single and (self.directory / f"{n}.single.json").exists():
                single = json.loads((self.directory / f"{n}.single.json").read_text())
                entry["single_thread"] = {"value": single["us_per_step"], "unit": "us/step", "cores": 1,
                                          "sample": f"{single['samples']} x {single['steps']}-step generation(s)"}
            out[n] = entry
            log(f"[cpu] {n}: {entry}")
        return out

    def close(self):
        (self.directory / "stop").write_text("")
        for _, process in self.workers.values():
            try:
                process.wait(timeout=30)
            except subprocess.TimeoutExpired:
                process.kill()


# ---------------------------------------------------------------------------- setup cost
def setup_costs(session, samples=5):
    """Host setup measured apart from steady-state decode (benchmarks/decoder/host_setup.py:17-77):
    lowering and compilation (storage reuse off and on), a fresh bind, the first instantiation of
    the inferred graph (one step and 16 steps per launch), and a rebind of the bound invocation
    (ckl_invocation_rebind: argument addresses moved, the graph's kernel nodes updated in place,
    no instantiation) with the graph launch after it. Medians over `samples`; the state is reset
    afterwards."""
    arguments = session.state.arguments()
    out = {"lower_ms": session.lower_ms, "compile_ms": {str(k): v for k, v in session.compile_ms.items()}}
    for reuse, program in session.programs.items():
        rows = {k: [] for k in ("bind_ms", "graph_setup_ms", "graph16_setup_ms", "rebind_ms", "graph_after_rebind_setup_ms")}
        for _ in range(samples):
            start = time.perf_counter()
            inv = program.bind(*arguments)
            rows["bind_ms"].append((time.perf_counter() - start) * 1e3)
            session.state.reset()
            rows["graph_setup_ms"].append(inv.benchmark(iterations=1, mode="graph")["graph_setup_ms"])
            session.state.reset()
            rows["graph16_setup_ms"].append(inv.benchmark(iterations=1, mode="graph", batch_size=GENERATION)["graph_setup_ms"])
            built = inv.graph_instantiations
            start = time.perf_counter()
            inv.rebind(*arguments)
            rows["rebind_ms"].append((time.perf_counter() - start) * 1e3)
            session.state.reset()
            rows["graph_after_rebind_setup_ms"].append(inv.benchmark(iterations=1, mode="graph")["graph_setup_ms"])
            if inv.graph_instantiations != built:
                raise AssertionError("a rebind to buffers of the same layout re-instantiated the graph")
            inv.close()
        out[f"reuse_{'on' if reuse else 'off'}"] = {k: statistics.median(v) for k, v in rows.items()}
    session.state.reset()
    return out


# ---------------------------------------------------------------------------- independent requests
REQUESTS = 8
REQUEST_RUNS = (("serial_inferred", "graph", 1, True), ("ordinary", "ordinary", 1, False),
                ("capture", "capture", 1, False), ("inferred", "graph", 1, False),
                ("inferred_group16", "graph", GENERATION, False), ("inferred_stream", "stream", 1, False))


def request_states(group) -> list:
    return [{k: state.download(k) for k in ("tokens", "history", "position", "logits")} for state in group.states]


def check_requests(group, reference: list, label: str) -> None:
    """Every request's state after a burst equals its state after the same burst run one request
    after another: tokens, history and position exactly, logits within the row-normwise bound."""
    from programs.harness import LOGITS_NORMWISE, normwise_error
    for index, (got, want) in enumerate(zip(request_states(group), reference)):
        for key in ("tokens", "history", "position"):
            if not np.array_equal(got[key], want[key]):
                raise AssertionError(f"requests {label}: request {index} {key} differs from the serial run")
        if normwise_error(got["logits"], want["logits"]) > LOGITS_NORMWISE:
            raise AssertionError(f"requests {label}: request {index} logits differ from the serial run")


def independent_requests(device, names, samples):
    """Independent requests (benchmarks/decoder/experiment.py:20-147; REPORT.md "Independent
    requests and the batching control"): REQUESTS invocations of one compiled decode program with
    shared weights and distinct prompts, GPU-prefilled, each timed 16-step generation burst run
    side by side on their own streams (or one after another: serial_inferred); and the batching
    control, one invocation of the same model with REQUESTS x B rows. Median burst wall and GPU
    span over `samples` rotated/reversed bursts, tokens/s = requests x B x 16 / wall. Every burst
    is checked against the first serial burst."""
    from programs.decoder_config import CONFIGS, Config
    from programs.harness import DecoderSession, RequestGroup, synthetic_inputs
    out = {}
    for name in names:
        c = CONFIGS[name]
        inputs = [synthetic_inputs(c, 123, prompt_seed=1000 + i) for i in range(REQUESTS)]
        group = RequestGroup(c, device, [arrays for arrays, _ in inputs])
        group.prefill([prompts for _, prompts in inputs])
        rows = {label: {"wall_us": [], "span_us": []} for label, *_ in REQUEST_RUNS}
        reference = None
        checked = 0
        for label, mode, batch, serial in REQUEST_RUNS:          # warm: graphs built, clocks up
            group.reset()
            group.run(mode=mode, iterations=GENERATION // batch, batch_size=batch, serial=serial)
            if reference is None:
                reference = request_states(group)
            check_requests(group, reference, label)
            checked += 1
        for sample in range(samples):
            order = list(REQUEST_RUNS[sample % len(REQUEST_RUNS):] + REQUEST_RUNS[:sample % len(REQUEST_RUNS)])
            for label, mode, batch, serial in (order if sample % 2 == 0 else reversed(order)):
                group.reset()
                t = group.run(mode=mode, iterations=GENERATION // batch, batch_size=batch, serial=serial)
                rows[label]["wall_us"].append(t["wall_us"])
                rows[label]["span_us"].append(t["span_us"])
                check_requests(group, reference, label)
                checked += 1
        tokens = REQUESTS * c.batch * GENERATION
        result = {label: {"wall_ms": statistics.median(r["wall_us"]) / 1e3, "span_ms": statistics.median(r["span_us"]) / 1e3,
                          "tokens_per_s": tokens / (statistics.median(r["wall_us"]) * 1e-6)}
                  for label, r in rows.items()}
        del group
        # Batching control: the same model, REQUESTS x B rows in one invocation.
        wide = Config(batch=REQUESTS * c.batch, hidden=c.hidden, heads=c.heads, layers=c.layers, ffn=c.ffn,
                      vocab=c.vocab, context=c.context, steps=c.steps)
        arrays, prompts = synthetic_inputs(wide, 123)
        session = DecoderSession(wide, device, arrays=arrays)
        session.prefill(prompts)
        control = {}
        control_reference = None
        for label, batch in (("batched_inferred", 1), ("batched_inferred_group16", GENERATION)):
            inv = session.invocations[True]
            session.state.reset()
            inv.benchmark(iterations=GENERATION // batch, mode="graph", batch_size=batch)
            runs = []
            for _ in range(samples):
                session.state.reset()
                runs.append(inv.benchmark(iterations=GENERATION // batch, mode="graph", batch_size=batch))
                got = {k: session.state.download(k) for k in ("tokens", "history", "position", "logits")}
                control_reference = control_reference or got
                if not all(np.array_equal(got[k], control_reference[k]) for k in got):
                    raise AssertionError(f"batching control {label}: runs differ")
                checked += 1
            wall = statistics.median(r["wall_us"] for r in runs) * GENERATION
            control[label] = {"wall_ms": wall / 1e3,
                              "span_ms": statistics.median(r["stream_us"] for r in runs) * GENERATION / 1e3,
                              "tokens_per_s": tokens / (wall * 1e-6)}
        del session
        out[name] = {"requests": REQUESTS, "rows_per_request": c.batch, "steps": GENERATION,
                     "independent": result, "batching_control": control, "bursts_verified": checked}
        log(f"[requests] {name}: " + "; ".join(f"{k} {v['wall_ms']:.3f} ms {v['tokens_per_s']:.0f} tok/s"
                                               for k, v in {**result, **control}.items()) + f"; {checked} verified")
    return out


# ---------------------------------------------------------------------------- vector pipeline
def vector_pipeline(device, samples):
    """Config V: dst = (src + 0.5) + 0.5 over N = 1,048,576 f32 (examples/vector_pipeline.py),
    unfused (two `update` launches and one planned 4 MiB temporary, reused across replays) and
    fused (one generated kernel), in every mode; HBM fraction of the fastest submission."""
    import ckl
    from programs import vector_pipeline as vp
    n = 1048576
    spec = ckl.BufferSpec((n,), ckl.f32)
    src, dst = device.empty(spec), device.empty(spec)
    x = np.random.default_rng(123).uniform(-1, 1, n).astype(np.float32)
    src.copy_from_host(x)
    expected = (x + np.float32(0.5)) + np.float32(0.5)
    out = {}
    for label, fuse in (("unfused", False), ("fused", True)):
        compiled = {reuse: vp.lower(n).compile(fuse_pointwise=fuse, reuse_storage=reuse) for reuse in (False, True)}
        inv = compiled[True].bind(src, dst, 0.5)
        timing = {}
        for mode in ("ordinary", "capture", "graph", "stream"):
            inv.run(mode=mode)
            got = np.empty_like(x)
            dst.copy_to_host(got)
            if not np.array_equal(got, expected):
                raise AssertionError(f"vector_pipeline {label} {mode}: result differs from (src + 0.5) + 0.5")
            inv.benchmark(iterations=20, mode=mode)
            runs = [inv.benchmark(iterations=100, mode=mode) for _ in range(samples)]
            timing[mode] = {"stream_us": statistics.median(r["stream_us"] for r in runs),
                            "wall_us": statistics.median(r["wall_us"] for r in runs)}
        heap = {str(r): sum(int(l.split("bytes = ")[1].split(" ")[0]) for l in p.executable_ir.splitlines()
                            if '"ckl_exec.heap"' in l) for r, p in compiled.items()}
        traffic = 16 * n if not fuse else 8 * n
        best = min(v["stream_us"] for v in timing.values())
        out[label] = dict(us_per_step=timing, heap_bytes=heap, algorithmic_bytes=traffic,
                          launches=inv.launch_count(mode="ordinary"), hbm_fraction=traffic / (best * 1e-6) / HBM_PEAK)
        log(f"[vector_pipeline] {label}: {timing}; heap {heap}")
    return out



def summary_line(name, r):
    """The few figures of a non-headline configuration that the stdout line carries."""
    keep = ("inferred_us", "capture_us", "branches_us", "contracted_us", "stream_us", "ordinary_us",
            "inferred_reuse_us", "inferred_over_capture", "branches_over_capture", "scratch_bytes", "workspace_bytes",
            "moved_temporary_bytes", "step_hbm_fraction", "logits_normwise", "runs_verified")
    out = {k: r[k] for k in keep}
    if "cpu_baseline" in r:
        out["cpu_us"] = r["cpu_baseline"]["value"]
    return out


def main():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=7 * GENERATION,
                        help="decode steps timed per variant (generations of 16 steps, then the remainder)")
    parser.add_argument("--warmup", type=int, default=3 * GENERATION, help="untimed warmup decode steps per variant")
    parser.add_argument("--seed", type=int, default=123)
    parser.add_argument("--configs", nargs="+", default=["small", "wide", "deep", "large"])
    parser.add_argument("--variants", nargs="+", default=None, choices=[v[0] for v in variants(GENERATION)],
                        help="time only these variants (default: all)")
    parser.add_argument("--no-cpu-baseline", action="store_true",
                        help="skip the CPU timing (the NumPy checker still verifies every run)")
    parser.add_argument("--no-extras", action="store_true",
                        help="skip the setup-cost, vector-pipeline and independent-request measurements")
    parser.add_argument("--output", type=Path, default=DEFAULT_DETAIL, help="where the full JSON result is written")
    parser.add_argument("--cpu-worker", type=Path, default=None, help=argparse.SUPPRESS)
    parser.add_argument("--role", default="all", help=argparse.SUPPRESS)
    args = parser.parse_args()
    if args.cpu_worker:
        cpu_worker(args.cpu_worker, args.role)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: every box here has one MI355X, and the decode "
                          "step's sharding over requests or heads is a design note, not a measured path"}))
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        parser.error("--steps must be positive and --warmup nonnegative")

    shm = Path("/dev/shm")
    base = shm if shm.is_dir() and shutil.disk_usage(shm).free > 24 << 30 else None
    workdir = Path(tempfile.mkdtemp(prefix="ckl_bench_", dir=base))
    checker = Checker(workdir, start_cpu_workers(workdir, timing=not args.no_cpu_baseline))
    try:
        line = measure(args, checker)
    finally:
        checker.close()
        shutil.rmtree(workdir, ignore_errors=True)
    print(json.dumps(line, default=float), flush=True)


def measure(args, checker):
    import ckl
    from programs.decoder_config import CONFIGS

    device = ckl.Device()
    log(f"device: {device.name}")
    configs = {}
    for name in args.configs:
        c = CONFIGS[name]
        session, result = run_config(name, c, args, device, checker)
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
        result["roofline"] = roofline
        log(f"[{name}] dominant kernel {dominant}: {roofline}")
        if not args.no_extras:
            result["setup"] = setup_costs(session)
            log(f"[{name}] setup: {result['setup']}")
        configs[name] = result
        del session
    extras = {}
    if not args.no_extras:
        extras["vector_pipeline"] = vector_pipeline(device, 7)
        extras["independent_requests"] = independent_requests(device, [n for n in ("small", "wide") if n in args.configs], 7)
    cpu = checker.baselines(configs)
    for name, row in cpu.items():
        configs[name]["cpu_baseline"] = row
    headline = HEADLINE if HEADLINE in configs else list(configs)[-1]
    head = configs[headline]
    c = CONFIGS[headline]
    value = head["inferred_us"] if head["inferred_us"] is not None else min(v["median_us"] for v in head["variants"].values())
    host = cpu_description()
    baseline = None
    if headline in cpu:
        baseline = dict(cpu[headline], cpu_model=host["cpu_model"], blas=host["blas"],
                        planner_ms=head["host_planning_ms"])
    timed = head["variants"]["inferred"]["timed_steps"] if "inferred" in head["variants"] else args.steps
    roofline = {k: head["roofline"][k] for k in ("bound", "kernel", "achieved", "peak", "unit", "frac", "traffic",
                                                 "algorithmic_bytes_per_launch", "avg_launch_us", "launches_per_step")}
    line = {
        "metric": METRIC, "value": value, "unit": "us/step", "n_gpus": 1, "steps": timed,
        "warmup": args.warmup, "ms_per_step": value / 1000.0, "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded N(0,0.02) weights, 1+N(0,0.02) gains, random prompts; GPU teacher-forced prefill)",
        "config": {"workload": f"{headline} decoder (B{c.batch} C{c.hidden} A{c.heads}x{c.head_dim} L{c.layers} "
                               f"F{c.ffn} V{c.vocab}, {c.context}-token prompt -> T {c.capacity}, {c.steps} greedy steps)",
                   **{k: head[k] for k in ("inferred_us", "capture_us", "ordinary_us", "branches_us", "contracted_us",
                                           "stream_us", "inferred_reuse_us", "batched_inferred_us",
                                           "inferred_over_capture", "branches_over_capture",
                                           "contracted_over_capture", "stream_over_capture", "scratch_bytes",
                                           "workspace_bytes", "bind_allocations", "moved_temporary_bytes",
                                           "tokens_per_s", "step_hbm_fraction",
                                           "logits_normwise", "runs_verified")},
                   "verification": "every run of every variant against the NumPy decoder (oracle/decoder.py) from "
                                   "the GPU-prefilled state: tokens, history, position exact; logits atol 2e-5 rtol "
                                   "3e-4 and row-normwise <= 1e-4; first run per variant also cache rows, prefix, "
                                   "suffix, tails; weights after all"},
        "roofline": roofline,
        "cpu_baseline": baseline,
        "other_configs": {k: summary_line(k, v) for k, v in configs.items() if k != headline},
        "detail": str(args.output),
    }
    args.output.parent.mkdir(parents=True, exist_ok=True)
    full = dict(line, host=host, configs=configs, **extras)
    args.output.write_text(json.dumps(full, indent=1, default=float) + "\n")
    return line


if __name__ == "__main__":
    main()
