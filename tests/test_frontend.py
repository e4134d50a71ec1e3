"""Frontend lowering: deterministic IR and cache keys, source-located diagnostics, no execution
of CKL bodies, constexpr handling, and the node order the graph numbering depends on
(behaviours of tests/Python/test_frontend.py in the reference)."""
import pytest

import ckl
from programs import vector_pipeline

N = ckl.dim("N")
Vec = ckl.Buffer[ckl.f32, (N,)]


@ckl.kernel
def shift(src: Vec, dst: Vec, bias: ckl.f32) -> None:
    i = ckl.global_id(0)
    if i < N:
        dst[i] = src[i] + bias


@ckl.kernel
def scaled(src: Vec, dst: Vec, factor: ckl.constexpr[ckl.f32]) -> None:
    i = ckl.global_id(0)
    if i < N:
        dst[i] = src[i] * factor


@ckl.program
def chain(src: Vec, dst: Vec, bias: ckl.f32) -> None:
    a = ckl.empty_like(src)
    b = ckl.empty_like(src)
    ckl.launch(shift, src, a, bias, grid=(ckl.cdiv(N, 64),), block=(64,))
    ckl.launch(scaled, a, b, 2.0, grid=(ckl.cdiv(N, 64),), block=(64,))
    ckl.launch(shift, b, dst, bias, grid=(ckl.cdiv(N, 64),), block=(64,))


@ckl.program
def bad_loop(src: Vec, dst: Vec, bias: ckl.f32) -> None:
    for item in src:
        ckl.launch(shift, src, dst, bias, grid=(1,), block=(64,))


@ckl.program
def runtime_constexpr(src: Vec, dst: Vec, bias: ckl.f32) -> None:
    ckl.launch(scaled, src, dst, bias, grid=(1,), block=(64,))


SPEC = ckl.BufferSpec((100,), ckl.f32)
SIG = {"src": SPEC, "dst": SPEC, "bias": ckl.f32}


def test_lowering_is_deterministic():
    first, second = chain.lower(signature=SIG), chain.lower(signature=SIG)
    assert first.mlir == second.mlir and first.cache_key == second.cache_key
    other = chain.lower(signature={**SIG, "src": ckl.BufferSpec((101,), ckl.f32), "dst": ckl.BufferSpec((101,), ckl.f32)})
    assert other.cache_key != first.cache_key


def test_node_order_allocs_dispatches_and_reversed_frees():
    text = chain.lower(signature=SIG).mlir
    program = text.split("func.func @program_")[1].split("func.func @kernel_")[0]
    ops = [line.split('"')[1] for line in program.splitlines() if '= "ckl.' in line or line.strip().startswith('"ckl.')]
    assert ops == ["ckl.alloc", "ckl.alloc", "ckl.dispatch", "ckl.dispatch", "ckl.dispatch", "ckl.free", "ckl.free"]
    frees = [line for line in program.splitlines() if '"ckl.free"' in line]
    assert "%1" in frees[0] and "%0" in frees[1]


def test_constexpr_specializes_kernel_and_shares_identical_specializations():
    lowered = chain.lower(signature=SIG)
    assert len(lowered.specializations) == 2           # shift shared by both launches, scaled once
    assert "2.0 : f32" in lowered.mlir                 # constexpr folded into the kernel body


def test_diagnostics_carry_source_positions():
    with pytest.raises(ckl.FrontendError) as error:
        bad_loop.lower(signature=SIG)
    message = str(error.value)
    assert "test_frontend.py:" in message and "for requires a simple induction variable" in message
    assert message.splitlines()[-1].strip() == "^"
    with pytest.raises(ckl.FrontendError, match="constexpr launch arguments must be compile-time constants"):
        runtime_constexpr.lower(signature=SIG)


def test_bodies_are_not_python_callables():
    with pytest.raises(ckl.FrontendError, match="not Python callables"):
        shift(None, None, 0.0)
    with pytest.raises(ckl.FrontendError, match="lower a @ckl.program entry point"):
        shift.lower(signature={})
    with pytest.raises(ckl.FrontendError, match="only valid inside a CKL source definition"):
        ckl.global_id(0)


def test_signature_errors():
    with pytest.raises(ckl.FrontendError, match="dimension N conflicts"):
        chain.lower(signature={**SIG, "dst": ckl.BufferSpec((7,), ckl.f32)})
    with pytest.raises(ckl.FrontendError, match="missing or misplaced runtime signature"):
        chain.lower(signature={"src": SPEC, "dst": SPEC})
    with pytest.raises(ckl.FrontendError, match="unknown specialization arguments"):
        chain.lower(signature={**SIG, "extra": ckl.f32})


def test_vector_pipeline_plan():
    """The vector pipeline's temporary: heap of 1280 bytes at N=257, second launch depends on
    the first (2026-08-29-ckl.md:459-468 of the reference)."""
    compiled = vector_pipeline.lower(257).compile(fuse_pointwise=False)
    ir = compiled.executable_ir
    assert ir.count('"ckl_exec.kernel"') == 2 and "dependencies = array<i64: 1>" in ir
    assert "bytes = 1280 : i64, device = 0 : i64" in ir
    assert "ckl.hip.library.update" in ir
