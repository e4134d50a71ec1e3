"""Pointwise fusion (the reference's ckl-fuse-pointwise, lib/Transforms/PointwiseFusion.cpp:30-304):
structural checks mirroring tests/Python/test_pointwise_fusion.py -- which launch chains fuse,
which boundaries must survive, and the compile pipeline's fused/unfused programs."""
import re

import pytest

import ckl
from ckl import _native
from fusion_programs import CASES
from programs import vector_pipeline

SPEC = ckl.BufferSpec((257,), ckl.f32)


def fused(text):
    return _native.native_opt(text, ["fuse-pointwise"])


def step_ir():
    return vector_pipeline.lower(257).mlir


def test_two_stage_chain_is_scalarised_deterministically():
    source = step_ir()
    out = fused(source)
    assert out == fused(source)
    assert out.count('"ckl.dispatch"') == 1
    assert out.count('"ckl.load_element"') == 1 and out.count('"ckl.store_element"') == 1
    assert out.count("arith.addf") == 2
    assert "ckl.fusion.requires_disjoint" in out and "ckl.fused_steps = 2" in out
    assert '"ckl.alloc"' not in out and '"ckl.free"' not in out
    assert re.search(r"@kernel_fused_[0-9a-f]{24}\(", out)
    assert fused(out) == out
    executable = _native.native_opt(out, ["prepare-hip", "build-graph", "lower-graph-to-exec"])
    assert executable.count('"ckl_exec.kernel"') == 1 and '"ckl_exec.heap"' not in executable


@pytest.mark.parametrize("name", sorted(CASES))
def test_complete_chains_fuse_but_not_branches_or_stencils(name):
    program, expected = CASES[name]
    signature = {"src": SPEC, "dst": SPEC}
    if name == "fan_out":
        signature["other"] = SPEC
    out = fused(program.lower(signature=signature).mlir)
    assert out.count('"ckl.dispatch"') == expected
    if name == "six_steps":
        assert "ckl.fused_steps = 6" in out and '"ckl.alloc"' not in out


def test_launch_and_guard_mismatches_are_not_fused():
    source = step_ir()
    first = source.index('"ckl.dispatch"')
    second = source.index('"ckl.dispatch"', first + 1)
    line_end = source.index("\n", second)

    def in_second(old, new):
        return source[:second] + source[second:line_end].replace(old, new, 1) + source[line_end:]

    mismatches = [
        in_second("block = array<i64: 256, 1, 1>", "block = array<i64: 128, 1, 1>"),
        source.replace("grid = array<i64: 2, 1, 1>", "grid = array<i64: 2, 2, 1>"),
        source.replace("shared_memory = 0 : i64", "shared_memory = 16 : i64"),
        source.replace("{predicate = 2 : i64}", "{predicate = 3 : i64}"),      # slt -> sle
        source.replace("{value = 257 : index}", "{value = 256 : index}"),
    ]
    for text in mismatches:
        assert text != source
        assert fused(text).count('"ckl.dispatch"') == 2, text


def test_escaping_temporary_and_barrier_keep_the_boundary():
    source = step_ir()
    temporary = re.search(r'(%\d+) = "ckl.alloc"', source).group(1)
    free = re.search(r'    "ckl.free"\([^\n]*\n', source).group(0)
    view = f'    %escaped = "ckl.view"({temporary}) : (memref<257xf32>) -> memref<257xf32>\n'
    assert fused(source.replace(free, view + free)).count('"ckl.dispatch"') == 2
    dispatches = [m.start() for m in re.finditer(r'    %[^\n]*"ckl.dispatch"', source)]
    barrier = '    "ckl.sync"() {scope = "device"} : () -> ()\n'
    assert fused(source[:dispatches[1]] + barrier + source[dispatches[1]:]).count('"ckl.dispatch"') == 2


def test_second_consumer_and_explicit_token_keep_the_boundary():
    source = step_ir()
    lines = re.findall(r'    %[^\n]*"ckl.dispatch"[^\n]*', source)
    extra = re.sub(r"    %\d+ =", "    %extra =", lines[1])
    free = source.index('    "ckl.free"')
    assert fused(source[:free] + extra + "\n" + source[free:]).count('"ckl.dispatch"') == 3
    token = re.match(r"    (%\d+) =", lines[0]).group(1)
    dependent = re.sub(r'("ckl.dispatch"\([^)]*)\)', r"\1, " + token + ")", lines[1])
    dependent = dependent.replace("array<i32: 3, 0>", "array<i32: 3, 1>")
    dependent = dependent.replace("f32) -> !ckl.token", "f32, !ckl.token) -> !ckl.token")
    assert fused(source.replace(lines[1], dependent)).count('"ckl.dispatch"') == 2


def test_prepared_and_prefused_modules_are_rejected():
    prepared = _native.native_opt(step_ir(), ["prepare-hip"])
    with pytest.raises(RuntimeError, match="before HIP preparation"):
        fused(prepared)
    prefused = fused(step_ir())
    lib = _native.native()
    import ctypes
    options = _native.CompileOptions(1, 1, 1, b"gfx950")
    handle = ctypes.c_void_p()
    assert lib.ckl_compile(prefused.encode(), ctypes.byref(options), ctypes.byref(handle)) != 0
    assert b"pre-fused" in lib.ckl_last_error()


def test_compile_keeps_an_unfused_fallback():
    program = vector_pipeline.lower(257).compile()
    assert program.executable_ir.count('"ckl_exec.kernel"') == 1
    assert '"ckl_exec.heap"' not in program.executable_ir
    assert "kernel_fused_" in program.device_ir
    unfused = vector_pipeline.lower(257).compile(fuse_pointwise=False)
    assert unfused.executable_ir.count('"ckl_exec.kernel"') == 2
