"""Decoder dependency graph and storage plan against the reference's recorded results
(tests/golden/decoder_reference_results.json, from benchmarks/decoder/results), the Python
restatement of the graph rules (oracle/graph.py) and the reference planner (oracle/_ref)."""
import json
import re
import subprocess
from pathlib import Path

import pytest

from oracle import graph as oracle_graph
from programs.decoder import decode
from programs.decoder_config import CONFIGS, Config, signature, temporary_bytes_without_reuse

GOLDEN = json.loads((Path(__file__).parent / "golden" / "decoder_reference_results.json").read_text())["cases"]
REF_PLANNER = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "ref_planner"


def plan_stats(ir):
    """The reference harness's parser of executable plans (benchmarks/decoder/run.py:66-78)."""
    topology = {}
    for line in ir.splitlines():
        if '"ckl_exec.kernel"' not in line:
            continue
        node = int(re.search(r"\bid = (\d+)", line).group(1))
        match = re.search(r"dependencies = array<i64(?:: ([\d, ]+))?>", line).group(1)
        topology[node] = [int(v) for v in match.split(",")] if match else []
    heaps = [line for line in ir.splitlines() if '"ckl_exec.heap"' in line]
    temporaries = [line for line in ir.splitlines() if '"ckl_exec.resource"' in line and 'kind = "temporary"' in line]
    return dict(nodes=len(topology), edges=sum(map(len, topology.values())), topology=topology,
                temporary_count=len(temporaries),
                temporary_heap_bytes=sum(int(re.search(r"\bbytes = (\d+)", line).group(1)) for line in heaps))


def compiled_stats(config, reuse):
    program = decode.lower(signature=signature(config)).compile(fuse_pointwise=False, reuse_storage=reuse)
    return plan_stats(program.executable_ir)


def oracle_stats(config, reuse):
    c = config
    program = oracle_graph.decoder_program(c.layers, c.batch, c.hidden, c.heads, c.capacity, c.ffn)
    edge_set = oracle_graph.edges(program)
    topology = oracle_graph.reduced_dependencies(program, edge_set)
    _, planned, _ = oracle_graph.decoder_plan(program, edge_set, reuse)
    return topology, planned


@pytest.mark.parametrize("case", GOLDEN, ids=[f"{c['source'].split('/')[0]}-{c['name']}" for c in GOLDEN])
def test_topology_and_heap_match_reference_results(case):
    config = Config(**case["config"])
    for reuse in (False, True):
        stats = compiled_stats(config, reuse)
        golden = case["plans"][str(reuse)]
        assert {str(k): v for k, v in stats["topology"].items()} == golden["topology"]
        for key in ("nodes", "edges", "temporary_count", "temporary_heap_bytes"):
            assert stats[key] == golden[key], key


@pytest.mark.parametrize("case", GOLDEN[:9], ids=[c["name"] for c in GOLDEN[:9]])
def test_oracle_restatement_matches_reference_results(case):
    config = Config(**case["config"])
    for reuse in (False, True):
        topology, planned = oracle_stats(config, reuse)
        assert {str(k): v for k, v in topology.items()} == case["plans"][str(reuse)]["topology"]
        assert planned == case["plans"][str(reuse)]["temporary_heap_bytes"]


@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_baseline_configs(name):
    c = CONFIGS[name]
    topology, planned_on = oracle_stats(c, True)
    _, planned_off = oracle_stats(c, False)
    for reuse, planned in ((False, planned_off), (True, planned_on)):
        stats = compiled_stats(c, reuse)
        assert stats["nodes"] == 21 * c.layers + 6
        assert stats["edges"] == 24 * c.layers + 5
        assert stats["temporary_count"] == 20 * c.layers + 3
        assert stats["topology"] == topology
        assert stats["temporary_heap_bytes"] == planned
    assert planned_off == temporary_bytes_without_reuse(c)
    assert planned_off == {"small": 136448, "wide": 509184, "deep": 532736, "large": 41683200}[name]


@pytest.mark.skipif(not REF_PLANNER.is_file(), reason="reference planner not built (make -C oracle)")
@pytest.mark.parametrize("name", sorted(CONFIGS))
def test_decoder_offsets_match_reference_planner(name):
    """Every temporary's heap offset in the native executable plan equals the reference
    planner's offset for the same graph and resources."""
    c = CONFIGS[name]
    lowered = decode.lower(signature=signature(c))
    text = lowered.analyze("prepare-hip", "build-graph")
    nodes = text.count('"ckl.graph_node"')
    edges = [(int(a), int(b)) for a, b in re.findall(r'"ckl.graph_edge"\(\) <\{from = (\d+) : i64, .*?to = (\d+) : i64\}>', text)]
    resources_text = re.search(r"ckl.resources = \[(.*)\]\} : \(\) -> \(\)", text).group(1)
    resources = []
    for entry in re.findall(r"\{address_space[^{}]*\}", resources_text):
        if 'kind = "temporary"' not in entry:
            continue
        name_ = re.search(r'name = "(alloc\d+)"', entry).group(1)
        users = [int(u) for u in re.search(r"users = array<i64: ([\d, ]+)>", entry).group(1).split(",")]
        resources.append(dict(name=name_, bytes=int(re.search(r"bytes = (\d+)", entry).group(1)), alignment=256, users=users))
    for reuse in (True, False):
        lines = [f"nodes {nodes} reuse {int(reuse)}"] + [f"edge {a} {b}" for a, b in edges]
        lines += [f"resource {r['bytes']} 256 0 0 " + " ".join(map(str, r["users"])) for r in resources]
        out = subprocess.run([str(REF_PLANNER)], input="\n".join(lines) + "\n", capture_output=True, text=True, check=True)
        ref_offsets = {int(row.split()[1]): int(row.split()[3]) for row in out.stdout.splitlines()[1:]}
        ir = lowered.compile(fuse_pointwise=False, reuse_storage=reuse).executable_ir
        mine = {m.group(1): int(m.group(2)) for m in re.finditer(
            r'kind = "temporary", name = "(alloc\d+)", offset = (\d+) : i64', ir)}
        assert len(mine) == len(resources)
        for k, r in enumerate(resources):
            assert mine[r["name"]] == ref_offsets[k], (reuse, r["name"])


def test_sibling_linears_take_their_shared_tiling():
    """The three linears that multiply one x (q, k, v) get the tiling chosen for three siblings in
    every run mode (the prepare step picks the selection's variant per dispatch); o, of the same
    shape and layer but with its own x, keeps the single-linear tiling; gate/up (two siblings) and
    the other projections are unchanged."""
    from ckl.library import linear_tiling
    c = CONFIGS["large"]
    ir = decode.lower(signature=signature(c)).compile(fuse_pointwise=False).executable_ir
    launches = {}
    for line in ir.splitlines():
        if '"ckl_exec.kernel"' in line and "ckl_linear_" in line:
            key = (re.search(r'entry_point = "([^"]+)"', line).group(1), int(re.search(r"\bgrid = array<i64: (\d+)", line).group(1)))
            launches[key] = launches.get(key, 0) + 1
    single = linear_tiling(c.batch, c.hidden, c.hidden)
    siblings = linear_tiling(c.batch, c.hidden, c.hidden, members=3)
    assert siblings["entry"] == "ckl_linear_mfma1x1" and siblings["split"] < single["split"] and single["entry"] == "ckl_linear_mfma2x1"
    gate_up = linear_tiling(c.batch, c.hidden, c.ffn)
    down = linear_tiling(c.batch, c.ffn, c.hidden)
    head = linear_tiling(c.batch, c.hidden, c.vocab)
    expected = {}
    for t, n in ((siblings, 3 * c.layers), (single, c.layers), (gate_up, 2 * c.layers), (down, c.layers), (head, 1)):
        expected[(t["entry"], t["grid"])] = expected.get((t["entry"], t["grid"]), 0) + n
    assert launches == expected


def workspace_plan(ir):
    """(kernels: id -> (dependencies, resource names of its arguments), placements)."""
    kernels = {}
    for line in ir.splitlines():
        if '"ckl_exec.kernel"' not in line:
            continue
        node = int(re.search(r"\bid = (\d+)", line).group(1))
        match = re.search(r"dependencies = array<i64(?:: ([\d, ]+))?>", line).group(1)
        deps = [int(v) for v in match.split(",")] if match else []
        kernels[node] = (deps, re.findall(r'resource = "([^"]+)"', line))
    placements = [dict(kernel=int(m.group(3)), name=m.group(4), offset=int(m.group(5)), bytes=int(m.group(1)),
                       role=m.group(6))
                  for m in re.finditer(r'"ckl_exec.workspace"\(\) <\{bytes = (\d+) : i64, heap = (\d+) : i64, '
                                       r'kernel = (\d+) : i64, name = "(\w+)", offset = (\d+) : i64, role = "(\w+)"', ir)]
    return kernels, placements


@pytest.mark.parametrize("name", ["small", "deep", "large"])
def test_library_workspaces_share_memory_only_between_ordered_lifetimes(name):
    """The workspace heap of the plan (library kernels' state and partial planes, planned apart
    from the temporaries): with storage reuse off nothing overlaps; with it on, two placements
    overlap only if both are partial planes and every reader of the first kernel's outputs
    (kernels taking a resource it writes, from the dependency graph's access list) precedes the
    second kernel in the plan's dependency
    order, so no launch order the dependencies allow can see one kernel's planes overwritten
    while they are still read. Reuse shrinks the large decoder's workspaces to a few layers'
    worth of planes."""
    lowered = decode.lower(signature=signature(CONFIGS[name]))
    graph = lowered.analyze("prepare-hip", "build-graph")
    written = {}
    for node in re.finditer(r'"ckl.graph_node"\(\) <\{accesses = \[(.*?)\], id = (\d+) : i64', graph):
        written[int(node.group(2))] = set(re.findall(r'effects = \[[^\]]*"write"[^\]]*\], region = "\w+", '
                                                     r'resource = "([^"]+)"', node.group(1)))
    sizes = {}
    for reuse in (False, True):
        ir = lowered.compile(fuse_pointwise=False, reuse_storage=reuse).executable_ir
        kernels, placements = workspace_plan(ir)
        heap = [int(m) for m in re.findall(r'"ckl_exec.workspace_heap"\(\) <\{alignment = 256 : i64, bytes = (\d+)', ir)]
        assert len(heap) == 1 and all(p["offset"] + p["bytes"] <= heap[0] for p in placements)
        sizes[reuse] = heap[0]
        reach = {}
        for node in sorted(kernels):
            reach[node] = set(kernels[node][0])
            for d in kernels[node][0]:
                reach[node] |= reach[d]
        for a in placements:
            for b in placements:
                if a is b or a["offset"] >= b["offset"] + b["bytes"] or b["offset"] >= a["offset"] + a["bytes"]:
                    continue
                assert reuse and a["role"] == b["role"] == "partials", (a, b)
                first, second = sorted((a["kernel"], b["kernel"]))
                outputs = written[first]
                assert outputs
                readers = [k for k in kernels if k > first and outputs & set(kernels[k][1])]
                assert all(r in reach[second] for r in [first] + readers), (first, second)
        if not reuse:
            assert sum(p["bytes"] for p in placements) <= heap[0]
    assert sizes[True] <= sizes[False]
    if name == "large":
        assert sizes[False] > 50 << 20 and sizes[True] < 10 << 20
