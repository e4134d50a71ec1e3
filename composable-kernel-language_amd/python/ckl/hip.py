"""HIP runtime API: Device, DeviceBuffer, CompiledProgram and Invocation on MI355X.

Public behaviour mirrors python/ckl/cuda.py:93-300 of the reference (argument validation,
ownership, run modes, benchmark results); execution goes through libckl_hip.so
(include/ckl_hip.h). Compilation selects hand-written gfx950 kernels for recognised kernel
bodies (ckl.library) and JIT-compiles the rest in-process.
"""
from __future__ import annotations

import ctypes
import math
import struct
import weakref
from contextlib import AbstractContextManager
from pathlib import Path

from . import _native
from .compiler import AMDTarget
from .types import BufferSpec, f32, f64, i32, i64

_SCALARS = {f32: ("f", 4), f64: ("d", 8), i32: ("i", 4), i64: ("q", 8)}
_KINDS = {i32: 1, i64: 2, f32: 3, f64: 4}


def _byte_count(spec) -> int:
    if not isinstance(spec, BufferSpec) or spec.dtype not in _SCALARS:
        raise TypeError("device storage requires a numeric BufferSpec")
    size = math.prod(spec.shape) * _SCALARS[spec.dtype][1]
    if not 0 < size < (1 << 64):
        raise ValueError("device storage byte count must fit a positive 64-bit size")
    return size


class _Handle:
    """Owns one native handle and releases it exactly once."""

    def __init__(self, pointer: int, release):
        self.pointer = pointer
        self._finalizer = weakref.finalize(self, release, ctypes.c_void_p(pointer))

    def release(self):
        self._finalizer()


class _ContextManager(AbstractContextManager):
    _resource = None

    @property
    def _native_resource(self):
        if self._resource is None:
            raise RuntimeError(f"{type(self).__name__} is closed")
        return self._resource

    @property
    def closed(self):
        return self._resource is None

    def close(self):
        # Bound invocations keep their own references to native resources.
        self._resource = None

    def __enter__(self):
        _ = self._native_resource
        return self

    def __exit__(self, exc_type, exc_value, traceback):
        self.close()
        return False


def runtime_available() -> bool:
    try:
        return _native.device_count() > 0
    except RuntimeError:
        return False


class Device(_ContextManager):
    """HIP device 0 (the one GPU of an MI355X box). Construction initialises HIP."""

    def __init__(self, ordinal: int = 0):
        lib = _native.native()
        handle = ctypes.c_void_p()
        _native.check(lib.ckl_device_open(ordinal, ctypes.byref(handle)))
        self._resource = _Handle(handle.value, lib.ckl_device_release)

    @property
    def native_library(self) -> Path:
        return _native.library_path().resolve()

    @property
    def name(self) -> str:
        return _native.native().ckl_device_name(self._native_resource.pointer).decode()

    def empty(self, spec: BufferSpec) -> "DeviceBuffer":
        size = _byte_count(spec)
        handle = ctypes.c_void_p()
        _native.check(_native.native().ckl_buffer_alloc(self._native_resource.pointer, size, ctypes.byref(handle)))
        return DeviceBuffer(self, _Handle(handle.value, _native.native().ckl_buffer_release), spec)

    def import_buffer(self, address: int, spec: BufferSpec, *, owner) -> "DeviceBuffer":
        """Borrow device memory; the Python owner stays alive as long as the buffer."""
        size = _byte_count(spec)
        if type(address) is not int or not 0 < address < (1 << 64) or owner is None:
            raise ValueError("imported storage requires a valid address and a live owner")
        handle = ctypes.c_void_p()
        _native.check(_native.native().ckl_buffer_import(self._native_resource.pointer, address, size, ctypes.byref(handle)))
        return DeviceBuffer(self, _Handle(handle.value, _native.native().ckl_buffer_release), spec, owner)


class DeviceBuffer(_ContextManager):
    def __init__(self, device: Device, resource: _Handle, spec: BufferSpec, owner=None):
        self.device, self.spec, self._owner = device, spec, owner
        self._resource = resource

    def close(self):
        super().close()
        self.device = self._owner = None

    @property
    def address(self) -> int:
        return int(_native.native().ckl_buffer_address(self._native_resource.pointer))

    @property
    def nbytes(self) -> int:
        return int(_native.native().ckl_buffer_nbytes(self._native_resource.pointer))

    def subview(self, *, offset: int, shape: tuple) -> "DeviceBuffer":
        """A bounded contiguous view; `offset` counts elements of this buffer."""
        spec = BufferSpec(shape, self.spec.dtype)
        size = _byte_count(spec)
        if type(offset) is not int or offset < 0:
            raise ValueError("subview requires a nonnegative element offset")
        byte_offset = offset * _SCALARS[self.spec.dtype][1]
        if byte_offset > self.nbytes or size > self.nbytes - byte_offset:
            raise ValueError("subview exceeds its source buffer")
        handle = ctypes.c_void_p()
        _native.check(_native.native().ckl_buffer_slice(self._native_resource.pointer, byte_offset, size,
                                                        ctypes.byref(handle)))
        return DeviceBuffer(self.device, _Handle(handle.value, _native.native().ckl_buffer_release), spec, self)

    def copy_from_host(self, source) -> None:
        view = memoryview(source).cast("B")
        if view.nbytes != self.nbytes:
            raise ValueError("host buffer byte count does not match device storage")
        data = (ctypes.c_char * view.nbytes).from_buffer_copy(view) if view.readonly else \
            (ctypes.c_char * view.nbytes).from_buffer(view)
        _native.check(_native.native().ckl_buffer_copy_from_host(self._native_resource.pointer, data, view.nbytes))

    def copy_to_host(self, destination) -> None:
        view = memoryview(destination).cast("B")
        if view.readonly or view.nbytes != self.nbytes:
            raise ValueError("destination must be writable and match device storage byte count")
        data = (ctypes.c_char * view.nbytes).from_buffer(view)
        _native.check(_native.native().ckl_buffer_copy_to_host(self._native_resource.pointer, data, view.nbytes))


class CompiledProgram(_ContextManager):
    """Native executable plan plus its device code (library kernels and JIT code object)."""

    def __init__(self, program, target=None, *, fuse_pointwise=True, reuse_storage=True):
        if type(fuse_pointwise) is not bool:
            raise TypeError("fuse_pointwise must be bool")
        if type(reuse_storage) is not bool:
            raise TypeError("reuse_storage must be bool")
        target = AMDTarget() if target is None else target
        if not isinstance(target, AMDTarget):
            raise ValueError("the HIP backend requires an AMDTarget")
        self.signature, self.target = program.signature, target
        from . import library
        self.selections = library.select(program)
        text = program.mlir
        identity = _native.library_identity()
        if self.selections and identity:
            attribute = library.selection_attribute(self.selections, identity)
            if not text.startswith("module {"):
                raise ValueError("unexpected IR module header")
            text = "module attributes {" + attribute + "} {" + text[len("module {"):]
        elif self.selections:
            raise RuntimeError("the gfx950 kernel library code object (ckl_kernels_gfx950.hsaco, or "
                               "CKL_KERNEL_LIBRARY) is missing; build it with composable-kernel-language_amd/build.py")
        lib = _native.native()
        options = _native.CompileOptions(int(reuse_storage), int(fuse_pointwise), 1, target.chip.encode())
        handle = ctypes.c_void_p()
        _native.check(lib.ckl_compile(text.encode(), ctypes.byref(options), ctypes.byref(handle)))
        self._resource = _Handle(handle.value, lib.ckl_program_release)
        count = ctypes.c_size_t()
        sizes = ctypes.POINTER(ctypes.c_uint64)()
        types = ctypes.POINTER(ctypes.c_char_p)()
        _native.check(lib.ckl_program_signature(handle, ctypes.byref(count), ctypes.byref(sizes), ctypes.byref(types)))
        expected = [_byte_count(p.dtype) if isinstance(p.dtype, BufferSpec) else 0 for p in program.signature.runtime]
        if [sizes[k] for k in range(count.value)] != expected:
            raise RuntimeError("compiled source signature does not match the Python signature")

    def _ir(self, stage: int) -> str:
        text = ctypes.c_char_p()
        size = ctypes.c_size_t()
        _native.check(_native.native().ckl_program_ir(self._native_resource.pointer, stage, ctypes.byref(text),
                                                      ctypes.byref(size)))
        return ctypes.string_at(text, size.value).decode()

    @property
    def prepared_ir(self) -> str:
        return self._ir(0)

    @property
    def executable_ir(self) -> str:
        return self._ir(1)

    @property
    def device_ir(self) -> str:
        """Generated HIP source of the JIT-compiled kernels ("" when all come from the library)."""
        return self._ir(2)

    @property
    def host_ir(self) -> str:
        """The host entry's callback sequence (what the reference compiles to LLVM IR)."""
        return self._ir(3)

    @property
    def fallback_host_ir(self) -> str:
        return self._ir(4)

    def bind(self, *arguments, device: Device = None) -> "Invocation":
        parameters = self.signature.runtime
        if len(arguments) != len(parameters):
            raise TypeError(f"expected {len(parameters)} runtime arguments, got {len(arguments)}")
        buffers = [a for a in arguments if isinstance(a, DeviceBuffer)]
        device = device or (buffers[0].device if buffers else None)
        if device is None:
            raise ValueError("pass a Device for programs without buffer arguments")
        packed = (_native.Argument * max(1, len(arguments)))()
        for k, (parameter, value) in enumerate(zip(parameters, arguments)):
            if isinstance(parameter.dtype, BufferSpec):
                if not isinstance(value, DeviceBuffer) or value.spec != parameter.dtype:
                    raise TypeError(f"{parameter.name} requires {parameter.dtype}")
                if value.device is not device:
                    raise ValueError("all buffers must belong to the selected Device")
                packed[k].kind = 0
                packed[k].buffer = value._native_resource.pointer
                continue
            code, width = _SCALARS[parameter.dtype]
            if parameter.dtype in (i32, i64):
                bits = width * 8
                if type(value) is not int or not -(1 << (bits - 1)) <= value < (1 << (bits - 1)):
                    raise TypeError(f"{parameter.name} requires a {bits}-bit integer")
                packed[k].integer = value
            else:
                if type(value) not in (int, float) or not math.isfinite(float(value)):
                    raise TypeError(f"{parameter.name} requires a finite numeric value")
                try:
                    rounded = struct.unpack(code, struct.pack(code, value))[0]
                except (OverflowError, struct.error):
                    raise ValueError(f"{parameter.name} overflows {parameter.dtype.name}") from None
                if not math.isfinite(rounded):
                    raise ValueError(f"{parameter.name} overflows {parameter.dtype.name}")
                packed[k].real = float(value)
            packed[k].kind = _KINDS[parameter.dtype]
        handle = ctypes.c_void_p()
        _native.check(_native.native().ckl_bind(self._native_resource.pointer, device._native_resource.pointer, packed,
                                                len(arguments), ctypes.byref(handle)))
        return Invocation(self, device, arguments, _Handle(handle.value, _native.native().ckl_invocation_release))

    def run(self, *arguments, graph=False, device=None) -> "Invocation":
        return self.bind(*arguments, device=device).run(graph=graph)


class Invocation(_ContextManager):
    """A bound program: one stream, its planned heaps and cached graphs."""

    # The reference's three modes, plus two ablations of the inferred graph: "branches" is one
    # graph node per dispatch with the reduced DAG's edges (the reference's inferred graph) and
    # "contracted" captures the inferred graph's contracted launches on one stream.
    MODES = {"ordinary": 0, "graph": 1, "capture": 2, "branches": 3, "contracted": 4}

    def __init__(self, program, device, arguments, resource: _Handle):
        self.program, self.device, self.arguments = program, device, arguments
        self._resource = resource

    def close(self):
        super().close()
        self.program = self.device = self.arguments = None

    @classmethod
    def _execution(cls, graph, mode, batch_size) -> int:
        if type(batch_size) is not int or not 0 < batch_size < (1 << 64):
            raise ValueError("batch_size must be a positive 64-bit count")
        if mode is not None and graph:
            raise ValueError("specify either graph or mode")
        if mode is not None and mode not in cls.MODES:
            raise ValueError("mode must be ordinary, graph, capture, branches, or contracted")
        return cls.MODES[mode] if mode is not None else int(bool(graph))

    def run(self, *, graph=False, mode=None, batch_size=1) -> "Invocation":
        execution = self._execution(graph, mode, batch_size)
        _native.check(_native.native().ckl_invocation_run(self._native_resource.pointer, execution, batch_size))
        return self

    @property
    def node_count(self) -> int:
        """Dispatches in the bound plan (including an overlap-triggered fallback)."""
        return int(_native.native().ckl_invocation_node_count(self._native_resource.pointer))

    def launch_count(self, *, mode="graph", batch_size=1) -> int:
        """Device launches one execution submits (graph nodes for graph modes)."""
        count = ctypes.c_uint64()
        _native.check(_native.native().ckl_invocation_launch_count(
            self._native_resource.pointer, self._execution(False, mode, batch_size), batch_size, ctypes.byref(count)))
        return int(count.value)

    def edge_count(self, *, mode="graph", batch_size=1) -> int:
        """Dependency edges of the explicit graph of `mode` ("graph" or "branches"; 0 otherwise)."""
        count = ctypes.c_uint64()
        _native.check(_native.native().ckl_invocation_edge_count(
            self._native_resource.pointer, self._execution(False, mode, batch_size), batch_size, ctypes.byref(count)))
        return int(count.value)

    def node_name(self, index: int) -> str:
        return _native.native().ckl_invocation_node_name(self._native_resource.pointer, index).decode()

    def time_node(self, index: int, iterations: int = 20) -> float:
        """Average microseconds of plan node `index` launched `iterations` times back to back
        (HIP events on the invocation stream). The node's writes are repeated."""
        out = ctypes.c_double()
        _native.check(_native.native().ckl_invocation_time_node(self._native_resource.pointer, index, iterations,
                                                                ctypes.byref(out)))
        return out.value

    def units(self) -> list:
        """The launches of one inferred step (chains contracted, siblings grouped): a list of
        (entry point, plan node indices)."""
        lib = _native.native()
        count = ctypes.c_uint64()
        _native.check(lib.ckl_invocation_unit_count(self._native_resource.pointer, ctypes.byref(count)))
        out = []
        for unit in range(count.value):
            name = ctypes.c_char_p()
            _native.check(lib.ckl_invocation_unit_name(self._native_resource.pointer, unit, ctypes.byref(name)))
            n = ctypes.c_uint64()
            _native.check(lib.ckl_invocation_unit_members(self._native_resource.pointer, unit, None, 0, ctypes.byref(n)))
            members = (ctypes.c_uint64 * max(1, n.value))()
            _native.check(lib.ckl_invocation_unit_members(self._native_resource.pointer, unit, members, n.value,
                                                          ctypes.byref(n)))
            out.append((name.value.decode(), [int(members[k]) for k in range(n.value)]))
        return out

    def time_unit(self, unit: int, iterations: int = 20) -> float:
        """Average microseconds of inferred-step launch `unit` issued `iterations` times back to back."""
        out = ctypes.c_double()
        _native.check(_native.native().ckl_invocation_time_unit(self._native_resource.pointer, unit, iterations,
                                                                ctypes.byref(out)))
        return out.value

    def profile_units(self, repeats: int = 7) -> list:
        """Durations (microseconds, `units()` order) of the inferred step's launches in sequence,
        from the median times of the step's launch-chain prefixes (each issued `repeats` times
        between HIP events; their effects are applied)."""
        lib = _native.native()
        count = ctypes.c_uint64()
        _native.check(lib.ckl_invocation_unit_count(self._native_resource.pointer, ctypes.byref(count)))
        out = (ctypes.c_double * max(1, count.value))()
        _native.check(lib.ckl_invocation_profile_units(self._native_resource.pointer, repeats, out, count.value,
                                                       ctypes.byref(count)))
        return [float(out[k]) for k in range(count.value)]

    def benchmark(self, *, iterations=200, graph=False, mode=None, batch_size=1) -> dict:
        """Time `iterations` submissions of `batch_size` program executions with HIP events on
        the invocation stream; returns per-program stream and wall microseconds plus graph setup."""
        if type(iterations) is not int or not 0 < iterations < (1 << 64):
            raise ValueError("iterations must be a positive 64-bit count")
        execution = self._execution(graph, mode, batch_size)
        out = (ctypes.c_double * 3)()
        _native.check(_native.native().ckl_invocation_benchmark(self._native_resource.pointer, execution, iterations,
                                                                batch_size, out))
        return {"stream_us": out[0], "wall_us": out[1], "graph_setup_ms": out[2]}
