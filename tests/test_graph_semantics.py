"""Effect summaries, dependency edges with reasons, storage plans and executable lowering on
hand-written IR, restating the behaviours the reference checks in tests/MLIR/test_semantics.py
(graph fixture :281-293, memory-plan fixture :294-312, randomized DAG oracle :50-125, strict vs
conservative unknown effects :257-275, control flow and subviews :356-393)."""
import random
import re

import pytest

from ckl import _native
from oracle.graph import random_program_expected_edges

READ_WRITE = '''
  func.func @read(%resource: memref<16xf32>) {
    %value = "ckl.load"(%resource) : (memref<16xf32>) -> f32
    func.return
  }
  func.func @write(%resource: memref<16xf32>) {
    %value = arith.constant 1.0 : f32
    "ckl.store"(%value, %resource) : (f32, memref<16xf32>) -> ()
    func.return
  }
'''


def dispatch(result, operands, types, kernel, deps=0, device="rocm:0", extra=""):
    return (f'    {result} = "ckl.dispatch"({operands}) {{block = array<i64: 256, 1, 1>, capabilities = ["rocm.bare_ptr"], '
            f'device = "{device}", grid = array<i64: 1, 1, 1>, implementation = "{kernel}.v1", kernel = @{kernel}, '
            f'operandSegmentSizes = array<i32: {len(operands.split(",")) - deps}, {deps}>, shared_memory = 0 : i64{extra}}}'
            f' : ({types}) -> !ckl.token\n')


def graph_edges(text):
    edges = {}
    for line in text.splitlines():
        if '"ckl.graph_edge"' in line:
            a = int(re.search(r"\bfrom = (\d+)", line).group(1))
            b = int(re.search(r"\bto = (\d+) : i64\}>", line).group(1))
            edges[(a, b)] = set(re.findall(r'\bkind = "([^"]+)"', line))
    return edges


def opt(text, *passes):
    return _native.native_opt(text, passes)


GRAPH_PROGRAM = "module {" + READ_WRITE + '''
  func.func @step() {
    %x = "ckl.alloc"() : () -> memref<16xf32>
    %y = memref.alloc() : memref<16xf32>
''' + dispatch("%x_written", "%x", "memref<16xf32>", "write") + dispatch("%y_written", "%y", "memref<16xf32>", "write") + \
    dispatch("%x_read", "%x, %y_written", "memref<16xf32>, !ckl.token", "read", deps=1) + '''
    "ckl.free"(%x) : (memref<16xf32>) -> ()
    memref.dealloc %y : memref<16xf32>
    func.return
  }
}
'''


def test_graph_nodes_edges_and_reasons():
    out = opt(GRAPH_PROGRAM, "build-graph")
    assert out.count('"ckl.graph_node"') == 7
    assert "digraph" in out
    edges = graph_edges(out)
    assert (2, 3) not in edges, "independent allocations received a false dependency"
    assert "memory" in edges[(2, 4)]
    assert "explicit" in edges[(3, 4)]
    assert "lifetime" in edges[(4, 5)]
    assert "ssa" in edges[(0, 2)]
    assert "from_location" in out and "to_location" in out
    assert "ckl.memory_plan = {assignments =" in out
    assert "ckl.launch_grid = array<i64: 1, 1, 1>" in out


MEMORY_PLAN_PROGRAM = "module {" + READ_WRITE + '''
  func.func @read_dynamic(%resource: memref<?xf32>) {
    %value = "ckl.load"(%resource) : (memref<?xf32>) -> f32
    func.return
  }
  func.func @step() {
    %first = "ckl.alloc"() : () -> memref<16xf32>
''' + dispatch("%first_written", "%first", "memref<16xf32>", "write") + \
    dispatch("%first_read", "%first, %first_written", "memref<16xf32>, !ckl.token", "read", deps=1) + '''
    "ckl.free"(%first) : (memref<16xf32>) -> ()
    %second = "ckl.alloc"() : () -> memref<16xf32>
''' + dispatch("%second_written", "%second, %first_read", "memref<16xf32>, !ckl.token", "write", deps=1) + \
    dispatch("%second_read", "%second, %second_written", "memref<16xf32>, !ckl.token", "read", deps=1) + '''
    "ckl.free"(%second) : (memref<16xf32>) -> ()
    func.return
  }
  func.func @dynamic(%size: index) {
    %resource = memref.alloc(%size) : memref<?xf32>
''' + dispatch("%done", "%resource", "memref<?xf32>", "read_dynamic") + '''
    memref.dealloc %resource : memref<?xf32>
    func.return
  }
}
'''


def test_memory_plan_reuses_ordered_temporaries():
    out = opt(MEMORY_PLAN_PROGRAM, "build-graph")
    assert "baseline_bytes = 512 : i64" in out
    assert "planned_bytes = 256 : i64" in out
    assert 'resource = "alloc1", shares_with = ["alloc0"], slot = 0 : i64' in out
    offsets = re.findall(r'bytes = 64 : i64, heap = 0 : i64, offset = (\d+) : i64, resource = "alloc[01]", slot = 0 : i64', out)
    assert offsets == ["0", "0"]
    assert 'status = "unavailable"' in out
    assert "requires a static identity-layout integer or float memref" in out


def random_program(generator, resources, count):
    operations, lines = [], ["module {", '''  func.func @read(%resource: memref<4xf32>) {
    %value = "ckl.load"(%resource) : (memref<4xf32>) -> f32
    func.return
  }
  func.func @write(%resource: memref<4xf32>) {
    %value = arith.constant 1.0 : f32
    "ckl.store"(%value, %resource) : (f32, memref<4xf32>) -> ()
    func.return
  }
  func.func @step() {''']
    for index in range(count):
        resource = generator.randrange(resources)
        effect = generator.choice(("read", "write"))
        dependency = None
        if index and generator.random() < 0.35:
            dependency = generator.randrange(index)
        operations.append((resource, effect, dependency))
    for r in range(resources):
        lines.append(f'    %r{r} = "ckl.alloc"() : () -> memref<4xf32>')
    for index, (resource, effect, dependency) in enumerate(operations):
        operands, types, deps = f"%r{resource}", "memref<4xf32>", 0
        if dependency is not None:
            operands, types, deps = operands + f", %d{dependency}", types + ", !ckl.token", 1
        lines.append(dispatch(f"%d{index}", operands, types, effect, deps=deps).rstrip("\n"))
    lines += ["    func.return", "  }", "}"]
    return "\n".join(lines) + "\n", operations


def test_random_programs_match_closed_form_edges():
    """Seed and generator calls of the reference's randomized check (test_semantics.py:98-125)."""
    generator = random.Random(20260927)
    for case in range(20):
        text, operations = random_program(generator, 3, 8)
        edges = graph_edges(opt(text, "build-graph"))
        actual = {(a - 3, b - 3) for a, b in edges if a >= 3 and b >= 3}
        assert actual == random_program_expected_edges(operations), f"case {case}"


UNKNOWN = '''module {
  func.func @mystery(%resource: memref<4xf32>) {
    "test.opaque"(%resource) : (memref<4xf32>) -> ()
    func.return
  }
  func.func @plain(%resource: memref<4xf32>) {
    %value = "ckl.load"(%resource) : (memref<4xf32>) -> f32
    func.return
  }
  func.func @step() {
    %a = "ckl.alloc"() : () -> memref<4xf32>
    %b = "ckl.alloc"() : () -> memref<4xf32>
''' + dispatch("%d0", "%a", "memref<4xf32>", "mystery") + dispatch("%d1", "%b", "memref<4xf32>", "plain") + '''
    func.return
  }
}
'''


def test_unknown_effects_strict_and_conservative():
    with pytest.raises(RuntimeError, match="unregistered dialect 'test'"):
        opt(UNKNOWN, "summarize-effects")
    with pytest.raises(RuntimeError, match="no complete memory-effect model"):
        opt(UNKNOWN, "allow-unregistered-dialect", "summarize-effects")
    out = opt(UNKNOWN, "allow-unregistered-dialect", "summarize-effects{strict=false}")
    assert "unknown = true" in out and 'effects = ["read", "write"]' in out and "synchronizes = true" in out
    edges = graph_edges(opt(UNKNOWN, "allow-unregistered-dialect", "build-graph{strict=false}"))
    assert "barrier" in edges[(2, 3)], "unknown dispatch did not order an otherwise independent dispatch"


CONDITIONAL = "module {" + READ_WRITE + '''
  func.func @step(%flag: i1) {
    %x = "ckl.alloc"() : () -> memref<16xf32>
    scf.if %flag {
''' + dispatch("%w", "%x", "memref<16xf32>", "write") + '''
    }
    func.return
  }
}
'''


def test_conditional_dispatch_is_not_executable():
    out = opt(CONDITIONAL, "build-graph")
    assert 'ckl.execution_control = "unsupported_control_flow"' in out
    with pytest.raises(RuntimeError, match="does not support graph nodes nested in region or CFG control flow"):
        opt(CONDITIONAL, "build-graph", "lower-graph-to-exec")


SUBVIEW = '''module {
  func.func @write(%resource: memref<4xf32>) {
    %value = arith.constant 1.0 : f32
    "ckl.store"(%value, %resource) : (f32, memref<4xf32>) -> ()
    func.return
  }
  func.func @step(%base: memref<16xf32>) {
    %view = "ckl.subview"(%base) {offset = 4 : i64} : (memref<16xf32>) -> memref<4xf32>
''' + dispatch("%w", "%view", "memref<4xf32>", "write") + '''
    func.return
  }
}
'''


def test_subview_region_and_lowering():
    out = opt(SUBVIEW, "build-graph")
    assert "length = 16 : i64, offset = 16 : i64" in out, "subview byte range was not composed"
    text = opt(SUBVIEW, "build-graph", "lower-graph-to-exec")
    assert "byte_length = 16 : i64" in text and "byte_offset = 16 : i64" in text


INDEXED = '''module {
  func.func @update(%input: memref<257xf32>, %output: memref<257xf32>) attributes {ckl.kernel} {
    %i = "ckl.global_id"() {axis = 0 : i32} : () -> index
    %count = arith.constant 257 : index
    %in_bounds = arith.cmpi ult, %i, %count : index
    scf.if %in_bounds {
      %value = "ckl.load_element"(%input, %i) : (memref<257xf32>, index) -> f32
      %one = arith.constant 1.0 : f32
      %updated = arith.addf %value, %one : f32
      "ckl.store_element"(%updated, %output, %i) : (f32, memref<257xf32>, index) -> ()
    }
    func.return
  }
  func.func @first(%buffer: memref<2x3xi32>) attributes {ckl.kernel} {
    %zero = arith.constant 0 : index
    %two = arith.constant 2 : index
    %value = "ckl.load_element"(%buffer, %zero, %two) : (memref<2x3xi32>, index, index) -> i32
    "ckl.store_element"(%value, %buffer, %zero, %zero) : (i32, memref<2x3xi32>, index, index) -> ()
    func.return
  }
  func.func @step(%input: memref<257xf32>, %output: memref<257xf32>) {
    %temporary = "ckl.alloc"() : () -> memref<257xf32>
''' + dispatch("%a", "%input, %temporary", "memref<257xf32>, memref<257xf32>", "update") + \
    dispatch("%b", "%temporary, %output", "memref<257xf32>, memref<257xf32>", "update") + '''
    "ckl.free"(%temporary) : (memref<257xf32>) -> ()
    func.return
  }
}
'''


def test_indexed_kernel_effects_and_plan():
    out = opt(INDEXED, "summarize-effects")
    update = out.split("func.func @update", 1)[1].split("func.func @first", 1)[0]
    assert 'effects = ["read"]' in update and 'effects = ["write"]' in update
    assert 'region = "whole"' in update and "unknown = false" in update and "may_alias = [[0, 1]]" in update
    first = out.split("func.func @first", 1)[1].split("func.func @step", 1)[0]
    assert "effects = [\"read\", \"write\"], region = {length = 12 : i64, offset = 0 : i64}" in first
    edges = graph_edges(opt(INDEXED, "build-graph"))
    assert "memory" in edges[(1, 2)]
    text = opt(INDEXED, "build-graph", "lower-graph-to-exec")
    assert text.count('"ckl_exec.kernel"') == 2
    assert "dependencies = array<i64: 1>" in text and 'packing = "bare_pointer"' in text
    assert "logical_index = 0" in text and "slot = 0" in text
    assert "bytes = 1280 : i64" in text     # 257 f32 rounded to 256-byte alignment


def test_parse_errors_are_reported_with_position():
    with pytest.raises(RuntimeError, match=r"^\d+:\d+: "):
        opt("module {\n  func.func @f() {\n    %x = \"ckl.alloc\"( : () -> memref<4xf32>\n  }\n}\n")
