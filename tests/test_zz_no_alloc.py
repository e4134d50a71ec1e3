"""ckl_bind_static, the no-allocation variant of ckl_bind, against ckl_bind itself through the C
ABI: on two calls in a row (the small decoder, then a smaller one) the statically bound
invocation must leave exactly the state the ordinarily bound one leaves, in every run mode and
for a 16-step graph submission; the first static invocation is superseded by the second bind;
programs larger than the arena are refused."""
import ctypes

import numpy as np
import pytest

import ckl
from ckl import _native
from oracle import decoder as oracle
from programs.decoder_config import CONFIGS, MUTABLE, Config
from programs.harness import DecoderSession

pytestmark = pytest.mark.gpu

SMALLER = Config(batch=3, hidden=48, heads=3, layers=1, ffn=80, vocab=129, context=3, steps=16)


@pytest.fixture(scope="module")
def stream(device):
    hip = ctypes.CDLL("libamdhip64.so")
    handle = ctypes.c_void_p()
    assert hip.hipStreamCreate(ctypes.byref(handle)) == 0
    yield handle.value
    hip.hipStreamSynchronize(handle)
    hip.hipStreamDestroy(handle)


def pack(arguments):
    packed = (_native.Argument * len(arguments))()
    for k, value in enumerate(arguments):
        if isinstance(value, ckl.DeviceBuffer):
            packed[k].kind = 0
            packed[k].buffer = value._native_resource.pointer
        else:
            packed[k].kind = 3          # the decode program's two scalars are f32
            packed[k].real = value
    return packed


def bind_static(program, device, arguments, stream):
    packed = pack(arguments)
    handle = ctypes.c_void_p()
    _native.check(_native.native().ckl_bind_static(program._native_resource.pointer, device._native_resource.pointer,
                                                   packed, len(arguments), stream, ctypes.byref(handle)))
    return handle.value


def run(handle, mode, batch=1):
    _native.check(_native.native().ckl_invocation_run(handle, mode, batch))


def state(session):
    return {name: session.state.download(name) for name in MUTABLE}


def same(a, b):
    return all(np.array_equal(a[k], b[k]) for k in a)


def check_against_ckl_bind(device, stream, c):
    initial, _ = oracle.make_inputs(c, 123, init="baseline")
    session = DecoderSession(c, device, arrays=initial)     # ordinary binds: code objects now resident
    ordinary = session.invocations[True]
    handle = bind_static(session.programs[True], device, session.state.arguments(), stream)
    for mode, name in ((0, "ordinary"), (1, "graph"), (2, "capture"), (3, "branches"), (4, "contracted"), (5, "stream")):
        session.state.reset()
        ordinary.run(mode=name)
        expected = state(session)
        session.state.reset()
        run(handle, mode)
        assert same(state(session), expected), mode
    session.state.reset()
    ordinary.run(mode="graph", batch_size=c.steps)
    expected = state(session)
    session.state.reset()
    run(handle, 1, c.steps)
    assert same(state(session), expected)
    return session, handle


def test_static_bind_matches_ckl_bind_twice(device, stream):
    lib = _native.native()
    assert lib.ckl_static_scratch_bytes() == 64 << 20
    first_session, first = check_against_ckl_bind(device, stream, CONFIGS["small"])
    second_session, second = check_against_ckl_bind(device, stream, SMALLER)
    try:
        with pytest.raises(ValueError, match="taken over"):
            run(first, 1)
        with pytest.raises(ValueError, match="taken over"):
            average = ctypes.c_double()
            _native.check(lib.ckl_invocation_time_node(first, 0, 1, ctypes.byref(average)))
        run(second, 1)
    finally:
        lib.ckl_invocation_release(first)
        lib.ckl_invocation_release(second)


def test_static_bind_refuses_programs_beyond_the_arena(device, stream):
    from programs import vector_pipeline
    n = 20 << 20                        # a 80 MiB temporary: more than the 64 MiB arena
    compiled = vector_pipeline.lower(n).compile(fuse_pointwise=False)
    spec = ckl.BufferSpec((n,), ckl.f32)
    src, dst = device.empty(spec), device.empty(spec)
    compiled.bind(src, dst, 0.5)        # makes its code objects resident
    with pytest.raises(ValueError, match="static arena"):
        packed = (_native.Argument * 3)()
        packed[0].kind, packed[0].buffer = 0, src._native_resource.pointer
        packed[1].kind, packed[1].buffer = 0, dst._native_resource.pointer
        packed[2].kind, packed[2].real = 3, 0.5
        handle = ctypes.c_void_p()
        _native.check(_native.native().ckl_bind_static(compiled._native_resource.pointer,
                                                       device._native_resource.pointer, packed, 3, stream,
                                                       ctypes.byref(handle)))


def memory(handle):
    out = (ctypes.c_uint64 * 3)()
    _native.check(_native.native().ckl_invocation_memory(handle, out))
    return list(out)


def test_static_bind_allocates_no_device_memory(device, stream):
    """A static bind after a warm-up one (same program, same stream) makes no device allocation:
    the binding reports none, and the device's free memory is the same before and after it."""
    hip = ctypes.CDLL("libamdhip64.so")
    lib = _native.native()
    initial, _ = oracle.make_inputs(SMALLER, 123, init="baseline")
    session = DecoderSession(SMALLER, device, arrays=initial)
    assert session.invocations[True].bind_allocations == 1        # one arena for every heap
    program, arguments = session.programs[True], session.state.arguments()
    warm = bind_static(program, device, arguments, stream)
    hip.hipStreamSynchronize(ctypes.c_void_p(stream))
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    before = free.value
    handle = bind_static(program, device, arguments, stream)
    hip.hipStreamSynchronize(ctypes.c_void_p(stream))
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    try:
        assert free.value == before
        heap, private, allocations = memory(handle)
        assert allocations == 0 and heap > 0 and private == 0     # workspaces are planned heap placements
        assert memory(warm)[:2] == [heap, private]
    finally:
        lib.ckl_invocation_release(warm)
        lib.ckl_invocation_release(handle)

