"""The host-entry contract of the C ABI, restating the reference's native program test
(tests/Runtime/NvidiaProgramValidation.cpp:23-109) through `ckl_program_from_entry`.

A ctypes entry stands in for JIT host code: it receives `entry(void*[]{&frame, &values})`,
checks the f32/f64/i64 scalar packing, loads a hand-written gfx950 code object
(tests/kernels/join.hip, a four-parameter kernel), declares one 128-byte heap with one
temporary and three external buffers, and commits two `join` dispatches, the second depending on
the first: temp = 0.625 x + 0.375 y, output = 0.625 temp + 0.375 y = 2.21875 for x = 1, y = 3.
The program then runs in every mode with 2 steps per submission; a scalar of the wrong type is
rejected with ValueError; an entry whose first callback fails reports that first error as
RuntimeError while its later callbacks do nothing.

The metadata validation runs on the CPU; everything that binds needs the GPU.
"""
import ctypes
from pathlib import Path

import numpy as np
import pytest

from ckl import _native

KERNEL = Path(__file__).resolve().parent / "kernels" / "join.gfx950.hsaco"
ENTRY = ctypes.CFUNCTYPE(None, ctypes.POINTER(ctypes.c_void_p))
SIZES = [128, 128, 128, 0, 0, 0, 0]
TYPES = ["", "", "", "i32", "f32", "f64", "i64"]


def from_entry(entry, sizes=SIZES, types=TYPES):
    lib = _native.native()
    count = len(sizes)
    handle = ctypes.c_void_p()
    status = lib.ckl_program_from_entry(
        ctypes.cast(entry, ctypes.c_void_p) if entry is not None else None,
        (ctypes.c_uint64 * max(1, count))(*sizes), (ctypes.c_char_p * max(1, count))(*[t.encode() for t in types]),
        count, None, ctypes.byref(handle))
    _native.check(status)
    return handle.value


# ---------------------------------------------------------------------------------- CPU part
def noop_entry(packed):
    pass


NOOP = ENTRY(noop_entry)


def test_entry_program_metadata_is_validated():
    lib = _native.native()
    handle = from_entry(NOOP)
    lib.ckl_program_release(handle)
    with pytest.raises(ValueError, match="invalid host entry"):
        from_entry(None)
    with pytest.raises(ValueError, match="invalid host entry"):
        from_entry(NOOP, [128, 0], ["", "f16"])      # no such scalar type
    with pytest.raises(ValueError, match="invalid host entry"):
        from_entry(NOOP, [0], [""])                  # neither a buffer nor a scalar
    with pytest.raises(ValueError, match="invalid host entry"):
        from_entry(NOOP, [64], ["f32"])              # a buffer with a scalar type
    out = ctypes.c_void_p()
    with pytest.raises(ValueError, match="invalid host entry"):
        _native.check(lib.ckl_program_from_entry(ctypes.cast(NOOP, ctypes.c_void_p), None, None, 1, None,
                                                 ctypes.byref(out)))


# ---------------------------------------------------------------------------------- GPU part
class JoinEntry:
    """The reference test's `entry`, written against the C ABI."""

    def __init__(self, image: bytes):
        self.image = ctypes.create_string_buffer(image, len(image))
        self.size = len(image)
        self.packing = []
        self.function = ENTRY(self)

    def __call__(self, packed):
        lib = _native.native()
        frame = ctypes.cast(packed[0], ctypes.POINTER(ctypes.c_void_p))[0]
        args = ctypes.cast(packed[1], ctypes.POINTER(ctypes.POINTER(ctypes.c_void_p)))[0]
        self.packing.append((ctypes.cast(args[4], ctypes.POINTER(ctypes.c_float))[0],
                             ctypes.cast(args[5], ctypes.POINTER(ctypes.c_double))[0],
                             ctypes.cast(args[6], ctypes.POINTER(ctypes.c_int64))[0]))
        lib.ckl_begin(frame, self.image, self.size)
        lib.ckl_heap(frame, 0, 128)
        for resource in range(3):
            lib.ckl_resource(frame, resource, 0, 0, args[resource])
        lib.ckl_resource(frame, 3, 0, 0, None)
        for node in (2, 5):
            lib.ckl_kernel(frame, b"join", 1, 1, 1, 32, 1, 1, 0)
            lib.ckl_argument_resource(frame, 0 if node == 2 else 3, 0)
            lib.ckl_argument_resource(frame, 1, 0)
            lib.ckl_argument_resource(frame, 3 if node == 2 else 2, 0)
            lib.ckl_argument_value(frame, args[3], 4)
            if node == 5:
                lib.ckl_dependency(frame, 2)
            lib.ckl_commit(frame, node)


def failing_entry(packed):
    lib = _native.native()
    frame = ctypes.cast(packed[0], ctypes.POINTER(ctypes.c_void_p))[0]
    lib.ckl_argument_resource(frame, 999, 0)   # records an error instead of unwinding
    lib.ckl_argument_resource(frame, 0, 0)     # must stay a no-op


FAILING = ENTRY(failing_entry)


def bind(program, device, arguments):
    lib = _native.native()
    packed = (_native.Argument * len(arguments))()
    for k, (kind, value) in enumerate(arguments):
        packed[k].kind = kind
        if kind == 0:
            packed[k].buffer = value
        elif kind in (1, 2):
            packed[k].integer = value
        else:
            packed[k].real = value
    handle = ctypes.c_void_p()
    _native.check(lib.ckl_bind(program, device, packed, len(arguments), ctypes.byref(handle)))
    return handle.value


@pytest.mark.gpu
def test_entry_program_runs_in_every_mode(device):
    if not KERNEL.exists():
        pytest.fail("tests/kernels/join.gfx950.hsaco is missing: run __graft_entry__.build()")
    lib = _native.native()
    dev = device._native_resource.pointer
    buffers = []
    for values in (np.ones(32, np.float32), np.full(32, 3.0, np.float32), np.zeros(32, np.float32)):
        handle = ctypes.c_void_p()
        _native.check(lib.ckl_buffer_alloc(dev, 128, ctypes.byref(handle)))
        _native.check(lib.ckl_buffer_copy_from_host(handle, values.ctypes.data, 128))
        buffers.append(handle.value)
    entry = JoinEntry(KERNEL.read_bytes())
    program = from_entry(entry.function)
    arguments = [(0, b) for b in buffers] + [(1, 32), (3, 1.25), (4, -2.5), (2, -1234567890123)]
    invocation = bind(program, dev, arguments)
    try:
        assert entry.packing == [(1.25, -2.5, -1234567890123)]
        assert lib.ckl_invocation_node_count(invocation) == 2
        result = np.empty(32, np.float32)
        timing = (ctypes.c_double * 3)()
        for mode in (0, 1, 2, 3, 4):
            _native.check(lib.ckl_buffer_copy_from_host(buffers[2], np.zeros(32, np.float32).ctypes.data, 128))
            _native.check(lib.ckl_invocation_run(invocation, mode, 2))
            _native.check(lib.ckl_buffer_copy_to_host(buffers[2], result.ctypes.data, 128))
            assert np.all(result == np.float32(2.21875)), (mode, result)
            _native.check(lib.ckl_invocation_benchmark(invocation, mode, 2, 2, timing))
            assert all(value >= 0 for value in timing), mode
        count = ctypes.c_uint64()
        _native.check(lib.ckl_invocation_edge_count(invocation, 3, 2, ctypes.byref(count)))
        assert count.value == 3       # 2 -> 5 in each step, and step 2's root after step 1's leaf

        wrong = list(arguments)
        wrong[3] = (3, 32.0)          # an f32 where the program declares i32
        with pytest.raises(ValueError, match="does not match"):
            bind(program, dev, wrong)

        failing = from_entry(FAILING)
        with pytest.raises(RuntimeError, match="999"):
            bind(failing, dev, arguments)
        lib.ckl_program_release(failing)

        again = bind(program, dev, arguments)
        _native.check(lib.ckl_invocation_run(again, 1, 1))
        lib.ckl_invocation_release(again)
    finally:
        lib.ckl_invocation_release(invocation)
        lib.ckl_program_release(program)
        for b in buffers:
            lib.ckl_buffer_release(b)


class CopiedAddressEntry(JoinEntry):
    """JoinEntry, except that resource 0 is declared from the entry's own copy of the first
    argument's address rather than from the packed argument array."""

    def __call__(self, packed):
        args = ctypes.cast(ctypes.cast(packed, ctypes.POINTER(ctypes.c_void_p))[1],
                           ctypes.POINTER(ctypes.POINTER(ctypes.c_void_p)))[0]
        self.copy = ctypes.c_uint64(ctypes.cast(args[0], ctypes.POINTER(ctypes.c_uint64))[0])
        saved = args[0]
        args[0] = ctypes.cast(ctypes.pointer(self.copy), ctypes.c_void_p)
        try:
            super().__call__(packed)
        finally:
            args[0] = saved


def rebind(invocation, arguments):
    packed = (_native.Argument * len(arguments))()
    for k, (kind, value) in enumerate(arguments):
        packed[k].kind = kind
        if kind == 0:
            packed[k].buffer = value
        elif kind in (1, 2):
            packed[k].integer = value
        else:
            packed[k].real = value
    _native.check(_native.native().ckl_invocation_rebind(invocation, packed, len(arguments)))


@pytest.mark.gpu
def test_rebind_follows_packed_arguments_and_refuses_copied_addresses(device):
    """A rebind moves resources the entry declared from the packed argument array to the new
    buffers; one declared from an address the entry copied elsewhere cannot be followed, so the
    rebind is refused with ValueError instead of leaving graphs that write freed memory."""
    lib = _native.native()
    dev = device._native_resource.pointer

    def buffers():
        out = []
        for values in (np.ones(32, np.float32), np.full(32, 3.0, np.float32), np.zeros(32, np.float32)):
            handle = ctypes.c_void_p()
            _native.check(lib.ckl_buffer_alloc(dev, 128, ctypes.byref(handle)))
            _native.check(lib.ckl_buffer_copy_from_host(handle, values.ctypes.data, 128))
            out.append(handle.value)
        return out

    first, second = buffers(), buffers()
    scalars = [(1, 32), (3, 1.25), (4, -2.5), (2, -1234567890123)]
    result = np.empty(32, np.float32)
    held = []
    try:
        for kind in (JoinEntry, CopiedAddressEntry):
            entry = kind(KERNEL.read_bytes())
            program = from_entry(entry.function)
            invocation = bind(program, dev, [(0, b) for b in first] + scalars)
            held.append((invocation, program, entry))
            _native.check(lib.ckl_invocation_run(invocation, 1, 1))
            _native.check(lib.ckl_buffer_copy_to_host(first[2], result.ctypes.data, 128))
            assert np.all(result == np.float32(2.21875)), kind.__name__
            if kind is JoinEntry:
                rebind(invocation, [(0, b) for b in second] + scalars)
                _native.check(lib.ckl_invocation_run(invocation, 1, 1))
                _native.check(lib.ckl_buffer_copy_to_host(second[2], result.ctypes.data, 128))
                assert np.all(result == np.float32(2.21875))
            else:
                with pytest.raises(ValueError, match="outside the packed"):
                    rebind(invocation, [(0, b) for b in second] + scalars)
                # The refused rebind left the binding as it was.
                _native.check(lib.ckl_buffer_copy_from_host(first[2], np.zeros(32, np.float32).ctypes.data, 128))
                _native.check(lib.ckl_invocation_run(invocation, 1, 1))
                _native.check(lib.ckl_buffer_copy_to_host(first[2], result.ctypes.data, 128))
                assert np.all(result == np.float32(2.21875))
    finally:
        for invocation, program, _ in held:
            lib.ckl_invocation_release(invocation)
            lib.ckl_program_release(program)
        for b in first + second:
            lib.ckl_buffer_release(b)
