"""The ckl-opt command-line driver (tools/ckl-opt/ckl-opt.cpp:1-29 of the reference) run as a
subprocess, as the reference's tests run theirs:

- the reference's MLIR fixtures (tests/MLIR/*.mlir and tests/Runtime/*host-plan.mlir, read in place
  from the reference checkout; skipped where it is absent) with the assertions of
  tests/MLIR/test_semantics.py:128-412 restated: effects, diagnostics, graph edges, memory plan,
  executable lowering, control flow, subviews, unknown operations, randomized DAGs;
- the kernel verifier's diagnostics on the invalid kernels of test_semantics.py:155-230;
- the host-entry lowering (the HIP counterpart of tests/MLIR/test_exec_to_llvm.py): exact
  callback order, exact constant bytes, rejected handoffs, and output that parses again;
- command-line behaviour: stdin, -o, pass order, exit codes.
"""
import random
import re
import subprocess
from pathlib import Path

import pytest

from oracle.graph import random_program_expected_edges
from test_graph_semantics import random_program

ROOT = Path(__file__).resolve().parents[1]
TOOL = ROOT / "composable-kernel-language_amd" / "python" / "ckl" / "_lib" / "ckl-opt"
FIXTURES = Path("/root/reference/tests/MLIR")
RUNTIME_FIXTURES = Path("/root/reference/tests/Runtime")
needs_fixtures = pytest.mark.skipif(not FIXTURES.is_dir(), reason="the reference's MLIR fixtures are not present")


def run(source, *arguments):
    """Run ckl-opt on a fixture path or on text through stdin."""
    assert TOOL.exists(), "ckl-opt is not built (python composable-kernel-language_amd/build.py)"
    if isinstance(source, Path):
        return subprocess.run([str(TOOL), str(source), *arguments], text=True, capture_output=True)
    return subprocess.run([str(TOOL), "-", *arguments], input=source, text=True, capture_output=True)


def ok(source, *arguments):
    result = run(source, *arguments)
    assert result.returncode == 0, result.stderr
    return result.stdout


def rejected(source, *arguments):
    result = run(source, *arguments)
    assert result.returncode == 1 and not result.stdout, (result.returncode, result.stdout)
    return result.stderr


def graph_edges(text):
    edges = {}
    for line in text.splitlines():
        if '"ckl.graph_edge"' in line:
            a = int(re.search(r"\bfrom = (\d+)", line).group(1))
            b = int(re.search(r"\bto = (\d+) : i64\}>", line).group(1))
            edges[(a, b)] = set(re.findall(r'\bkind = "([^"]+)"', line))
    return edges


# ------------------------------------------------------------------ the reference's fixtures

@needs_fixtures
def test_effects_fixture():
    out = ok(FIXTURES / "effects.mlir", "--ckl-summarize-effects")
    assert 'effects = ["read"]' in out and 'effects = ["write"]' in out
    assert 'effects = ["read", "write"]' in out, "view did not retain base identity"
    assert "may_alias = [[0, 1]]" in out, "external arguments must conservatively alias"
    assert "func.func @private_allocation() attributes {ckl.effect_summary = {accesses = []" in out
    assert out.count('effects = ["read"]') >= 2, "callee summary was not propagated"
    upstream = out.split("func.func @upstream_interfaces", 1)[1]
    assert 'effects = ["read"]' in upstream and 'effects = ["write"]' in upstream, "memref.copy effects"


@needs_fixtures
def test_dispatch_fixture():
    out = ok(FIXTURES / "dispatch.mlir", "--ckl-summarize-effects")
    assert out.count('effects = ["read"]') >= 2
    assert out.count('effects = ["read", "write"]') >= 2
    assert out.count("synchronizes = true") == 2
    assert out.count('ordering_scopes = ["acq_rel@device", "sync@device"]') == 2


@needs_fixtures
def test_unknown_operation_fixtures():
    source = FIXTURES / "unknown.mlir"
    assert "unregistered dialect 'foreign'" in rejected(source, "--ckl-summarize-effects")
    assert "no complete memory-effect model" in rejected(source, "--allow-unregistered-dialect", "--ckl-summarize-effects")
    out = ok(source, "--allow-unregistered-dialect", "--ckl-summarize-effects=strict=false")
    assert "unknown = true" in out and 'effects = ["read", "write"]' in out and "synchronizes = true" in out
    out = ok(FIXTURES / "unknown-graph.mlir", "--allow-unregistered-dialect", "--ckl-build-graph=strict=false")
    assert "barrier" in graph_edges(out)[(2, 3)], "unknown dispatch did not order an otherwise independent dispatch"
    assert "unknown = true" in out


@needs_fixtures
def test_invalid_fixtures_fail_verification():
    err = rejected(FIXTURES / "invalid-dispatch.mlir")
    assert err.startswith(f"{FIXTURES / 'invalid-dispatch.mlir'}:7:5: error: ") and "requires positive block dimensions" in err
    assert "placement exceeds its heap" in rejected(FIXTURES / "invalid-exec.mlir")


@needs_fixtures
def test_graph_fixture():
    out = ok(FIXTURES / "graph.mlir", "--ckl-build-graph")
    assert out.count('"ckl.graph_node"') == 7 and "digraph" in out
    edges = graph_edges(out)
    assert (2, 3) not in edges, "independent allocations received a false dependency"
    assert "memory" in edges[(2, 4)] and "explicit" in edges[(3, 4)]
    assert "lifetime" in edges[(4, 5)] and "ssa" in edges[(0, 2)]
    assert "from_location" in out and "to_location" in out
    assert "ckl.memory_plan = {assignments =" in out and "ckl.launch_grid = array<i64: 1, 1, 1>" in out
    # capabilities = [] names no argument ABI: lowering must not guess one.
    err = rejected(FIXTURES / "graph.mlir", "--ckl-build-graph", "--ckl-lower-graph-to-exec")
    assert "requires complete launch and ABI metadata" in err


@needs_fixtures
def test_memory_plan_fixture():
    out = ok(FIXTURES / "memory-plan.mlir", "--ckl-build-graph")
    assert "baseline_bytes = 512 : i64" in out and "planned_bytes = 256 : i64" in out
    assert 'resource = "alloc1", shares_with = ["alloc0"], slot = 0 : i64' in out
    offsets = re.findall(r'bytes = 64 : i64, heap = 0 : i64, offset = (\d+) : i64, resource = "alloc[01]", slot = 0 : i64', out)
    assert offsets == ["0", "0"]
    assert 'status = "unavailable"' in out and "requires a static identity-layout integer or float memref" in out


@needs_fixtures
@pytest.mark.parametrize("fixture,kernels,artifact,abi", [
    ("hip-host-plan.mlir", 2, "kernels.hsaco", "bare_pointer"),
    ("host-plan.mlir", 5, "kernels.cubin", "direct_pointer")])
def test_host_plan_fixtures_lower_to_executable_plans(fixture, kernels, artifact, abi):
    out = ok(RUNTIME_FIXTURES / fixture, "--ckl-build-graph", "--ckl-lower-graph-to-exec")
    assert '"ckl.graph"' not in out, "analysis graph was retained"
    assert out.count('"ckl_exec.kernel"') == kernels
    assert "logical_index = 0" in out and "slot = 0" in out and "dependencies = array<i64:" in out
    assert f'packing = "{abi}"' in out and artifact in out
    if abi == "bare_pointer":
        assert "dependencies = array<i64: 0>" in out, "the inferred write conflict was lost"
    ok(out)   # the printed plan parses and verifies again


@needs_fixtures
def test_control_flow_and_subview_fixtures():
    out = ok(FIXTURES / "conditional-dispatch.mlir", "--ckl-build-graph")
    assert 'ckl.execution_control = "unsupported_control_flow"' in out
    err = rejected(FIXTURES / "conditional-dispatch.mlir", "--ckl-build-graph", "--ckl-lower-graph-to-exec")
    assert "does not support graph nodes nested in region or CFG control flow" in err
    out = ok(FIXTURES / "subview-dispatch.mlir", "--ckl-build-graph")
    assert 'packing = "unsupported_view"' in out
    err = rejected(FIXTURES / "subview-dispatch.mlir", "--ckl-build-graph", "--ckl-lower-graph-to-exec")
    assert "does not support view/subview resource arguments" in err


@needs_fixtures
def test_indexed_kernel_fixture():
    source = FIXTURES / "indexed-kernel.mlir"
    out = ok(source, "--ckl-summarize-effects")
    update = out.split("func.func @update", 1)[1].split("func.func @step", 1)[0]
    assert 'effects = ["read"]' in update and 'effects = ["write"]' in update
    assert 'region = "whole"' in update and "unknown = false" in update
    assert 'effects = ["read", "write"]' in out.split("func.func @coordinates", 1)[1]
    assert "memory" in graph_edges(ok(source, "--ckl-build-graph"))[(1, 2)]
    assert ok(source, "--ckl-build-graph", "--ckl-lower-graph-to-exec").count('"ckl_exec.kernel"') == 2


@needs_fixtures
@pytest.mark.parametrize("fixture", sorted(p.name for p in FIXTURES.glob("*.mlir")) if FIXTURES.is_dir() else [])
def test_every_accepted_fixture_round_trips(fixture):
    """What the driver prints for a fixture parses and verifies again (analysis output included)."""
    arguments = ["--allow-unregistered-dialect", "--ckl-build-graph=strict=false"]
    result = run(FIXTURES / fixture, *arguments)
    if result.returncode:
        assert fixture.startswith("invalid-"), result.stderr
        return
    ok(result.stdout, "--allow-unregistered-dialect")


# ------------------------------------------------------------------ kernel verification

def kernel(body, buffer="memref<4xf32>", marker="ckl.kernel"):
    return f'''module {{
  func.func @test(%buffer: {buffer}) attributes {{{marker}}} {{
    %zero = arith.constant 0 : index
    {body}
    func.return
  }}
}}'''


LEAF_LAUNCH = '''module {
  func.func @leaf() attributes {ckl.kernel} { func.return }
  func.func @parent() attributes {ckl.kernel} {
    %done = "ckl.dispatch"() {kernel = @leaf, grid = array<i64: 1, 1, 1>, block = array<i64: 1, 1, 1>,
      shared_memory = 0 : i64, device = "rocm:0", capabilities = [], implementation = "leaf",
      operandSegmentSizes = array<i32: 0, 0>} : () -> !ckl.token
    func.return
  }
}'''

INVALID_KERNELS = [
    (kernel('%i = "ckl.global_id"() {axis = 3 : i32} : () -> index'), "requires axis 0, 1, or 2"),
    (kernel('%i = "ckl.thread_id"() {axis = -1 : i32} : () -> index'), "requires axis 0, 1, or 2"),
    (kernel('%i = "ckl.global_id"() {axis = 0 : i32} : () -> index', marker=""),
     "requires an enclosing func.func marked ckl.kernel"),
    (kernel('%v = "ckl.load_element"(%buffer) : (memref<4xf32>) -> f32'), "requires one index per buffer dimension"),
    (kernel('%v = "ckl.load_element"(%buffer, %zero) : (memref<4xf32>, index) -> i32'),
     "value type must match the buffer element type"),
    (kernel('%v = arith.constant 1 : i32\n    "ckl.store_element"(%v, %buffer, %zero) : (i32, memref<4xf32>, index) -> ()'),
     "value type must match the buffer element type"),
    (kernel('%past = arith.constant 4 : index\n    %v = "ckl.load_element"(%buffer, %past) : (memref<4xf32>, index) -> f32'),
     "constant index is out of bounds for dimension 0"),
    (kernel('%past = arith.constant 3 : index\n    %v = "ckl.load_element"(%buffer, %zero, %past) : (memref<2x3xf32>, index, index) -> f32',
            buffer="memref<2x3xf32>"), "constant index is out of bounds for dimension 1"),
    (kernel('%negative = arith.constant -1 : index\n    %v = arith.constant 1.0 : f32\n'
            '    "ckl.store_element"(%v, %buffer, %negative) : (f32, memref<?xf32>, index) -> ()', buffer="memref<?xf32>"),
     "constant index is out of bounds for dimension 0"),
    (kernel("", buffer="memref<*xf32>"), "ckl.kernel arguments must be numeric scalars or ranked numeric memrefs"),
    (kernel("", marker="ckl.kernel = true"), "ckl.kernel requires a unit attribute on func.func"),
    ("module { func.func private @test() attributes {ckl.kernel} }", "ckl.kernel requires a defined function with no results"),
    ("module { func.func @test() -> i32 attributes {ckl.kernel} {\n  %v = arith.constant 0 : i32\n  func.return %v : i32\n} }",
     "ckl.kernel requires a defined function with no results"),
    (LEAF_LAUNCH, "cannot launch a kernel from a ckl.kernel body"),
]


@pytest.mark.parametrize("source,diagnostic", INVALID_KERNELS, ids=[d for _, d in INVALID_KERNELS])
def test_invalid_kernels_are_rejected(source, diagnostic):
    err = rejected(source)
    assert diagnostic in err and err.startswith("<stdin>:"), err


@pytest.mark.parametrize("source", [
    kernel('%v = "ckl.load_element"(%buffer) : (memref<f32>) -> f32', buffer="memref<f32>"),   # rank 0: no index
    kernel('%v = "ckl.load_element"(%buffer, %zero) : (memref<?xf32>, index) -> f32', buffer="memref<?xf32>")])
def test_rank_zero_and_dynamic_kernels_are_accepted(source):
    ok(source, "--ckl-summarize-effects")


DISPATCH_CASES = [
    ("grid = array<i64: 1, 1, 1>", "grid = array<i64: 1, 1>", "requires exactly three grid dimensions"),
    ("shared_memory = 0 : i64", "shared_memory = -4 : i64", "requires non-negative shared memory"),
    ('implementation = "write.v1"', 'implementation = ""', "requires a stable implementation identity"),
    ("kernel = @write", "kernel = @missing", "references unknown kernel @missing"),
    ('"ckl.dispatch"(%x)', '"ckl.dispatch"(%x, %x)', "operandSegmentSizes"),
]


@pytest.mark.parametrize("old,new,diagnostic", DISPATCH_CASES, ids=[d for *_, d in DISPATCH_CASES])
def test_invalid_dispatches_are_rejected(old, new, diagnostic):
    source = '''module {
  func.func @write(%r: memref<4xf32>) {
    %v = arith.constant 1.0 : f32
    "ckl.store"(%v, %r) : (f32, memref<4xf32>) -> ()
    func.return
  }
  func.func @step(%x: memref<4xf32>) {
    %d = "ckl.dispatch"(%x) {block = array<i64: 64, 1, 1>, capabilities = ["rocm.bare_ptr"], device = "rocm:0",
      grid = array<i64: 1, 1, 1>, implementation = "write.v1", kernel = @write,
      operandSegmentSizes = array<i32: 1, 0>, shared_memory = 0 : i64} : (memref<4xf32>) -> !ckl.token
    func.return
  }
}'''
    ok(source)
    assert old in source
    bad = source.replace(old, new)
    if new.startswith('"ckl.dispatch"(%x, %x)'):
        bad = bad.replace(": (memref<4xf32>) -> !ckl.token", ": (memref<4xf32>, memref<4xf32>) -> !ckl.token")
    assert diagnostic in rejected(bad)


def test_random_programs_through_the_driver():
    """The reference's randomized DAG check (seed 20260927, test_semantics.py:98-125), via the tool."""
    generator = random.Random(20260927)
    for case in range(20):
        text, operations = random_program(generator, 3, 8)
        edges = graph_edges(ok(text, "--ckl-build-graph"))
        actual = {(a - 3, b - 3) for a, b in edges if a >= 3 and b >= 3}
        assert actual == random_program_expected_edges(operations), f"case {case}"


# ------------------------------------------------------------------ host entry lowering

HOST_PLAN = r'''module {
  func.func private @step(memref<4xf32>, f32)
  "ckl_exec.plan"() <{source = @step, name = "step.exec", backend = "rocm"}> ({
    "ckl_exec.heap"() <{id = 0 : i64, bytes = 256 : i64, alignment = 256 : i64, device = 0 : i64, address_space = "global"}> : () -> ()
    "ckl_exec.resource"() <{name = "arg0", kind = "external", device = "rocm:0", address_space = "global",
      alignment = 16 : i64, bytes = 16 : i64}> : () -> ()
    "ckl_exec.resource"() <{name = "scratch", kind = "temporary", device = "rocm:0", address_space = "global",
      alignment = 16 : i64, bytes = 16 : i64, heap = 0 : i64, offset = 0 : i64}> : () -> ()
    "ckl_exec.kernel"() <{id = 2 : i64, kernel = @producer, implementation = "producer.v1", artifact = "module.v1",
      abi = "rocm.bare_ptr", device = "rocm:0", grid = array<i64: 1, 1, 1>, block = array<i64: 64, 1, 1>,
      shared_memory = 0 : i64, dependencies = array<i64>, arguments = [
        {slot = 1 : i64, logical_index = 1 : i64, kind = "scalar", name = "arg1", type = f32},
        {slot = 0 : i64, logical_index = 0 : i64, kind = "resource", resource = "arg0", packing = "bare_pointer", type = memref<4xf32>},
        {slot = 2 : i64, logical_index = 2 : i64, kind = "constant", value = -7 : i64, type = i64},
        {slot = 3 : i64, logical_index = 3 : i64, kind = "constant", value = -0.0 : f64, type = f64},
        {slot = 4 : i64, logical_index = 4 : i64, kind = "bytes", value = array<i8: 0, -1, 1>, type = vector<3xi8>}]}> : () -> ()
    "ckl_exec.kernel"() <{id = 5 : i64, kernel = @consumer, implementation = "consumer.v1", artifact = "module.v1",
      abi = "rocm.bare_ptr", device = "rocm:0", grid = array<i64: 1, 1, 1>, block = array<i64: 64, 1, 1>,
      shared_memory = 0 : i64, dependencies = array<i64: 2>, arguments = [
        {slot = 0 : i64, logical_index = 0 : i64, kind = "resource", resource = "scratch", packing = "bare_pointer", type = memref<4xf32>}]}> : () -> ()
  }) : () -> ()
}
'''


def callees(text):
    return re.findall(r'callee = "([a-z_]+)"', text)


def test_host_entry_order_and_exact_bytes():
    out = ok(HOST_PLAN, "--ckl-lower-exec-to-host")
    assert "ckl_exec." not in out and "func.func" not in out and '"ckl_host.entry"' in out
    assert callees(out) == ["ckl_module", "ckl_heap", "ckl_resource", "ckl_resource", "ckl_kernel", "ckl_argument_resource",
                            *["ckl_argument_value"] * 4, "ckl_commit", "ckl_kernel", "ckl_argument_resource",
                            "ckl_dependency", "ckl_commit"]
    # -7 : i64, -0.0 : f64 and the bytes 00 FF 01, little-endian and exact.
    for data in (r'"\F9\FF\FF\FF\FF\FF\FF\FF"', r'"\00\00\00\00\00\00\00\80"', r'"\00\FF\01"'):
        assert f"bytes = {data}" in out
    assert 'argument = 1 : i64, callee = "ckl_argument_value", size = 4 : i64' in out   # f32 from host argument 1
    ok(out)   # the host entry is valid IR on its own


def test_host_entry_of_a_lowered_program():
    """The pipeline end to end: graph -> plan -> host entry, for the HIP fixture the tool also
    lowers above (two launches, the second waiting on the first)."""
    source = '''module {
  func.func @add_bias(%values: memref<1024xf32>, %count: i32, %bias: f32) {
    %value = "ckl.load"(%values) : (memref<1024xf32>) -> f32
    %updated = arith.addf %value, %bias : f32
    "ckl.store"(%updated, %values) : (f32, memref<1024xf32>) -> ()
    func.return
  }
  func.func @launch(%values: memref<1024xf32>, %count: i32) {
    %one = arith.constant 1.0 : f32
    %a = "ckl.dispatch"(%values, %count, %one) {artifact = "kernels.hsaco", implementation = "add_bias.first",
      kernel = @add_bias, device = "rocm:0", capabilities = ["rocm.bare_ptr"], grid = array<i64: 4, 1, 1>,
      block = array<i64: 256, 1, 1>, shared_memory = 0 : i64, operandSegmentSizes = array<i32: 3, 0>}
      : (memref<1024xf32>, i32, f32) -> !ckl.token
    %b = "ckl.dispatch"(%values, %count, %one) {artifact = "kernels.hsaco", implementation = "add_bias.second",
      kernel = @add_bias, device = "rocm:0", capabilities = ["rocm.bare_ptr"], grid = array<i64: 4, 1, 1>,
      block = array<i64: 256, 1, 1>, shared_memory = 0 : i64, operandSegmentSizes = array<i32: 3, 0>}
      : (memref<1024xf32>, i32, f32) -> !ckl.token
    func.return
  }
}'''
    out = ok(source, "--ckl-build-graph", "--ckl-lower-graph-to-exec", "--ckl-lower-exec-to-host")
    assert callees(out) == ["ckl_module", "ckl_resource", "ckl_kernel", "ckl_argument_resource", "ckl_argument_value",
                            "ckl_argument_value", "ckl_commit", "ckl_kernel", "ckl_argument_resource", "ckl_argument_value",
                            "ckl_argument_value", "ckl_dependency", "ckl_commit"]
    assert r'bytes = "\00\00\80?"' in out   # 1.0f little-endian: 00 00 80 3F ('?')


@pytest.mark.parametrize("old,new,diagnostic", [
    ('backend = "rocm"', 'backend = "cuda"', "requires the rocm backend"),
    ('name = "arg1"', 'name = "arg9"', "original argN bindings"),
    ('name = "arg1"', 'name = "arg0"', "binding type does not match"),
    ('abi = "rocm.bare_ptr", device = "rocm:0", grid = array<i64: 1, 1, 1>, block = array<i64: 64, 1, 1>,\n      shared_memory = 0 : i64, dependencies = array<i64>',
     'abi = "cuda.direct", device = "rocm:0", grid = array<i64: 1, 1, 1>, block = array<i64: 64, 1, 1>,\n      shared_memory = 0 : i64, dependencies = array<i64>',
     "direct_pointer packing"),
    ('device = "rocm:0", grid', 'device = "rocm:1", grid', "requires rocm:0"),
    ("func.func private @step(memref<4xf32>, f32)", "func.func private @step(memref<4xf32>, f32) -> i32",
     "source function declaration with no results"),
    ("func.func private @step", "func.func private @unrelated()\n  func.func private @step", "unexpected operation"),
])
def test_host_lowering_rejects_inconsistent_handoffs(old, new, diagnostic):
    assert old in HOST_PLAN
    assert diagnostic in rejected(HOST_PLAN.replace(old, new, 1), "--ckl-lower-exec-to-host")


def test_bytes_arguments_are_checked():
    bad = HOST_PLAN.replace("type = vector<3xi8>", "type = vector<4xi8>")
    assert "bytes argument requires a non-empty vector<Nxi8> type and N byte values" in rejected(bad)
    bad = HOST_PLAN.replace("value = -7 : i64, type = i64", "value = -7 : i32, type = i64")
    assert "constant argument requires a value matching its type" in rejected(bad)


# ------------------------------------------------------------------ command line

def test_command_line_behaviour(tmp_path):
    source = tmp_path / "in.mlir"
    source.write_text(HOST_PLAN)
    target = tmp_path / "out.mlir"
    result = subprocess.run([str(TOOL), str(source), "--ckl-lower-exec-to-host", "-o", str(target)], capture_output=True, text=True)
    assert result.returncode == 0 and not result.stdout and '"ckl_host.entry"' in target.read_text()
    assert subprocess.run([str(TOOL), "--no-such-flag"], capture_output=True, text=True).returncode == 2
    missing = subprocess.run([str(TOOL), str(tmp_path / "missing.mlir")], capture_output=True, text=True)
    assert missing.returncode == 1 and "cannot open input file" in missing.stderr
    assert "usage: ckl-opt" in subprocess.run([str(TOOL), "--help"], capture_output=True, text=True).stdout
    err = rejected(HOST_PLAN, "--ckl-lower-exec-to-host", "--ckl-summarize-effects")
    assert "lower-exec-to-host must be the last pass" in err
    # A parse error carries its position.
    assert re.match(r"<stdin>:3:\d+: error: ", rejected('module {\n  func.func @f() {\n    %x = "ckl.alloc"( : () -> memref<4xf32>\n  }\n}\n'))
