"""Runtime objects of the HIP backend: Device, DeviceBuffer, CompiledProgram and Invocation.

These keep the public surface of the reference's python/ckl/cuda.py:93-300 (names, argument
checks and their messages, ownership, run modes, benchmark results) over libckl_hip.so
(include/ckl_hip.h), bound with ctypes. Compiling a lowered program selects hand-written gfx950
kernels for recognised kernel bodies (ckl.library) and JIT-compiles the others in-process.

Ownership: every native handle belongs to exactly one Python object and is released once, when
that object is garbage-collected; `close()` only detaches the Python object, because bound
invocations hold native references to the programs, devices and buffers they use.
"""
from __future__ import annotations

import ctypes
import math
import struct
import weakref
from pathlib import Path

from . import _native
from .compiler import AMDTarget
from .types import BufferSpec, ScalarType, f32, f64, i32, i64

_MAX_U64 = 1 << 64


class _Handle:
    """One native handle, released exactly once by its release function."""

    def __init__(self, pointer: int, release):
        self.pointer = pointer
        self._finalizer = weakref.finalize(self, release, ctypes.c_void_p(pointer))

    def release(self):
        self._finalizer()


class _Closable:
    """Explicit scope for an object backed by a native handle (`with` closes it)."""

    _resource = None

    @property
    def _native_resource(self) -> _Handle:
        if self._resource is None:
            raise RuntimeError(f"{type(self).__name__} is closed")
        return self._resource

    @property
    def closed(self) -> bool:
        return self._resource is None

    def close(self):
        self._resource = None

    def __enter__(self):
        self._native_resource
        return self

    def __exit__(self, *exc):
        self.close()
        return False


def _nbytes(spec) -> int:
    if not isinstance(spec, BufferSpec):
        raise TypeError("device storage requires a numeric BufferSpec")
    size = spec.nbytes
    if not 0 < size < _MAX_U64:
        raise ValueError("device storage byte count must fit a positive 64-bit size")
    return size


def runtime_available() -> bool:
    try:
        return _native.device_count() > 0
    except RuntimeError:
        return False


# ------------------------------------------------------------------------------ scalar packing
class _ScalarSlot:
    """How a Python value becomes the native argument of one scalar type (CKL_ARG_* kind)."""

    def __init__(self, kind: int, dtype: ScalarType):
        self.kind, self.dtype = kind, dtype

    def encode(self, name: str, value, slot) -> None:
        slot.kind = self.kind
        if self.dtype.is_integer:
            bits = self.dtype.bits
            if type(value) is not int or not -(1 << (bits - 1)) <= value < 1 << (bits - 1):
                raise TypeError(f"{name} requires a {bits}-bit integer")
            slot.integer = value
            return
        if type(value) not in (int, float) or not math.isfinite(float(value)):
            raise TypeError(f"{name} requires a finite numeric value")
        code = "<f" if self.dtype == f32 else "<d"
        try:
            stored = struct.unpack(code, struct.pack(code, value))[0]
        except (OverflowError, struct.error):
            stored = math.inf
        if not math.isfinite(stored):
            raise ValueError(f"{name} overflows {self.dtype.name}")
        slot.real = float(value)


_SLOTS = {dtype: _ScalarSlot(kind, dtype) for kind, dtype in ((1, i32), (2, i64), (3, f32), (4, f64))}


# ------------------------------------------------------------------------------ device and buffers
class Device(_Closable):
    """A HIP device (ordinal 0 is the one GPU of an MI355X box). Construction initialises HIP."""

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

    def _buffer(self, create, spec: BufferSpec, owner=None) -> "DeviceBuffer":
        handle = ctypes.c_void_p()
        _native.check(create(ctypes.byref(handle)))
        return DeviceBuffer(self, _Handle(handle.value, _native.native().ckl_buffer_release), spec, owner)

    def empty(self, spec: BufferSpec) -> "DeviceBuffer":
        size = _nbytes(spec)
        return self._buffer(lambda out: _native.native().ckl_buffer_alloc(self._native_resource.pointer, size, out), spec)

    def import_buffer(self, address: int, spec: BufferSpec, *, owner) -> "DeviceBuffer":
        """Borrow device memory at `address`; `owner` is kept alive as long as the buffer."""
        size = _nbytes(spec)
        if owner is None or type(address) is not int or not 0 < address < _MAX_U64:
            raise ValueError("imported storage requires a valid address and a live owner")
        return self._buffer(
            lambda out: _native.native().ckl_buffer_import(self._native_resource.pointer, address, size, out), spec, owner)


class DeviceBuffer(_Closable):
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
        """A contiguous view `shape` starting `offset` elements into this buffer."""
        spec = BufferSpec(shape, self.spec.dtype)
        size = _nbytes(spec)
        if type(offset) is not int or offset < 0:
            raise ValueError("subview requires a nonnegative element offset")
        start = offset * spec.element_bytes
        if start > self.nbytes or size > self.nbytes - start:
            raise ValueError("subview exceeds its source buffer")
        handle = ctypes.c_void_p()
        _native.check(_native.native().ckl_buffer_slice(self._native_resource.pointer, start, size, ctypes.byref(handle)))
        return DeviceBuffer(self.device, _Handle(handle.value, _native.native().ckl_buffer_release), spec, self)

    def copy_from_host(self, source) -> None:
        view = memoryview(source).cast("B")
        if view.nbytes != self.nbytes:
            raise ValueError("host buffer byte count does not match device storage")
        storage = ctypes.c_char * view.nbytes
        data = storage.from_buffer_copy(view) if view.readonly else storage.from_buffer(view)
        _native.check(_native.native().ckl_buffer_copy_from_host(self._native_resource.pointer, data, view.nbytes))

    def copy_to_host(self, destination) -> None:
        view = memoryview(destination).cast("B")
        if view.readonly or view.nbytes != self.nbytes:
            raise ValueError("destination must be writable and match device storage byte count")
        data = (ctypes.c_char * view.nbytes).from_buffer(view)
        _native.check(_native.native().ckl_buffer_copy_to_host(self._native_resource.pointer, data, view.nbytes))


# ------------------------------------------------------------------------------ programs
class CompiledProgram(_Closable):
    """A program compiled for one MI355X: its executable plan and device code (library kernels
    and a JIT code object for the rest)."""

    def __init__(self, program, target=None, *, fuse_pointwise=True, reuse_storage=True):
        for flag, label in ((fuse_pointwise, "fuse_pointwise"), (reuse_storage, "reuse_storage")):
            if type(flag) is not bool:
                raise TypeError(f"{label} must be bool")
        target = AMDTarget() if target is None else target
        if not isinstance(target, AMDTarget):
            raise ValueError("the HIP backend requires an AMDTarget")
        self.signature, self.target = program.signature, target
        from . import library
        self.selection_report = library.explain(program)
        self.selections = {s: d for s, (kind, d) in self.selection_report.items() if kind == "library"}
        text = self._with_selection(program.mlir, library)
        lib = _native.native()
        options = _native.CompileOptions(int(reuse_storage), int(fuse_pointwise), 1, target.chip.encode())
        handle = ctypes.c_void_p()
        _native.check(lib.ckl_compile(text.encode(), ctypes.byref(options), ctypes.byref(handle)))
        self._resource = _Handle(handle.value, lib.ckl_program_release)
        self._check_signature(program, handle)

    def _with_selection(self, text: str, library) -> str:
        """The IR with the library selections as a module attribute (none: the IR unchanged)."""
        if not self.selections:
            return text
        identity = _native.library_identity()
        if not identity:
            raise RuntimeError("the gfx950 kernel library code object (ckl_kernels_gfx950.hsaco, or "
                               "CKL_KERNEL_LIBRARY) is missing; build it with composable-kernel-language_amd/build.py")
        if not text.startswith("module {"):
            raise ValueError("unexpected IR module header")
        return "module attributes {" + library.selection_attribute(self.selections, identity) + "} {" + \
            text[len("module {"):]

    def _check_signature(self, program, handle) -> None:
        count = ctypes.c_size_t()
        sizes = ctypes.POINTER(ctypes.c_uint64)()
        types = ctypes.POINTER(ctypes.c_char_p)()
        _native.check(_native.native().ckl_program_signature(handle, ctypes.byref(count), ctypes.byref(sizes),
                                                             ctypes.byref(types)))
        expected = [_nbytes(p.dtype) if isinstance(p.dtype, BufferSpec) else 0 for p in program.signature.runtime]
        if [sizes[k] for k in range(count.value)] != expected:
            raise RuntimeError("compiled source signature does not match the Python signature")

    def _ir(self, stage: int) -> str:
        text = ctypes.c_char_p()
        size = ctypes.c_size_t()
        _native.check(_native.native().ckl_program_ir(self._native_resource.pointer, stage, ctypes.byref(text),
                                                      ctypes.byref(size)))
        return ctypes.string_at(text, size.value).decode()

    prepared_ir = property(lambda self: self._ir(0), doc="IR after fusion and HIP preparation")
    executable_ir = property(lambda self: self._ir(1), doc="executable plan (ckl_exec ops)")
    device_ir = property(lambda self: self._ir(2), doc="generated HIP source of JIT kernels ('' when none)")
    host_ir = property(lambda self: self._ir(3), doc="the host entry's callback sequence")
    fallback_host_ir = property(lambda self: self._ir(4), doc="callback sequence of the unfused fallback")

    def _pack(self, arguments, device):
        parameters = self.signature.runtime
        if len(arguments) != len(parameters):
            raise TypeError(f"expected {len(parameters)} runtime arguments, got {len(arguments)}")
        if device is None:
            device = next((a.device for a in arguments if isinstance(a, DeviceBuffer)), None)
        if device is None:
            raise ValueError("pass a Device for programs without buffer arguments")
        packed = (_native.Argument * max(1, len(arguments)))()
        for slot, parameter, value in zip(packed, parameters, arguments):
            if not isinstance(parameter.dtype, BufferSpec):
                _SLOTS[parameter.dtype].encode(parameter.name, value, slot)
                continue
            if not isinstance(value, DeviceBuffer) or value.spec != parameter.dtype:
                raise TypeError(f"{parameter.name} requires {parameter.dtype}")
            if value.device is not device:
                raise ValueError("all buffers must belong to the selected Device")
            slot.kind, slot.buffer = 0, value._native_resource.pointer
        return packed, device

    def bind(self, *arguments, device: Device = None) -> "Invocation":
        packed, device = self._pack(arguments, device)
        handle = ctypes.c_void_p()
        _native.check(_native.native().ckl_bind(self._native_resource.pointer, device._native_resource.pointer, packed,
                                                len(arguments), ctypes.byref(handle)))
        return Invocation(self, device, arguments, _Handle(handle.value, _native.native().ckl_invocation_release))

    def run(self, *arguments, graph=False, device=None) -> "Invocation":
        return self.bind(*arguments, device=device).run(graph=graph)


class Invocation(_Closable):
    """A bound program: its stream, planned heaps and cached graphs."""

    # The reference's three modes, plus three variants of the inferred graph: "branches" is one
    # graph node per dispatch with the reduced DAG's edges (the reference's inferred graph),
    # "contracted" captures the inferred graph's contracted launches on one stream and "stream"
    # issues those launches on the invocation stream with no graph.
    MODES = {"ordinary": 0, "graph": 1, "capture": 2, "branches": 3, "contracted": 4, "stream": 5}

    def __init__(self, program, device, arguments, resource: _Handle):
        self.program, self.device, self.arguments = program, device, arguments
        self._resource = resource

    def close(self):
        super().close()
        self.program = self.device = self.arguments = None

    @classmethod
    def _execution(cls, graph, mode, batch_size) -> int:
        if type(batch_size) is not int or not 0 < batch_size < _MAX_U64:
            raise ValueError("batch_size must be a positive 64-bit count")
        if mode is None:
            return 1 if graph else 0
        if graph:
            raise ValueError("specify either graph or mode")
        if mode not in cls.MODES:
            raise ValueError("mode must be ordinary, graph, capture, branches, contracted, or stream")
        return cls.MODES[mode]

    def _call(self, function, *args):
        _native.check(function(self._native_resource.pointer, *args))

    def run(self, *, graph=False, mode=None, batch_size=1) -> "Invocation":
        self._call(_native.native().ckl_invocation_run, self._execution(graph, mode, batch_size), batch_size)
        return self

    def rebind(self, *arguments) -> "Invocation":
        """The same program on other buffers of the same specs (scalars unchanged), keeping the
        instantiated explicit graphs: their kernel nodes' parameters are updated in place."""
        packed, _ = self.program._pack(arguments, self.device)
        self._call(_native.native().ckl_invocation_rebind, packed, len(arguments))
        self.arguments = arguments
        return self

    @property
    def graph_instantiations(self) -> int:
        """Graph executables built for this invocation so far (a rebind that updates nodes in
        place adds none)."""
        count = ctypes.c_uint64()
        self._call(_native.native().ckl_invocation_graph_instantiations, ctypes.byref(count))
        return int(count.value)

    def _memory(self) -> list:
        out = (ctypes.c_uint64 * 3)()
        self._call(_native.native().ckl_invocation_memory, out)
        return [int(v) for v in out]

    @property
    def heap_bytes(self) -> int:
        """Bytes of the planned heaps this binding placed its temporaries in."""
        return self._memory()[0]

    @property
    def private_bytes(self) -> int:
        """Device memory the binding owns besides its heaps: private workspaces (ckl_workspace) and
        temporaries the inferred graph moved out of storage the plan shares."""
        return self._memory()[1]

    @property
    def bind_allocations(self) -> int:
        """Device allocations the bind made (0 for a static binding)."""
        return self._memory()[2]

    @property
    def node_count(self) -> int:
        """Dispatches in the bound plan (including an overlap-triggered fallback)."""
        return int(_native.native().ckl_invocation_node_count(self._native_resource.pointer))

    def _count(self, function, mode, batch_size) -> int:
        count = ctypes.c_uint64()
        self._call(function, self._execution(False, mode, batch_size), batch_size, ctypes.byref(count))
        return int(count.value)

    def launch_count(self, *, mode="graph", batch_size=1) -> int:
        """Device launches one execution submits (graph nodes for graph modes)."""
        return self._count(_native.native().ckl_invocation_launch_count, mode, batch_size)

    def edge_count(self, *, mode="graph", batch_size=1) -> int:
        """Dependency edges of the explicit graph of `mode` ("graph" or "branches"; 0 otherwise)."""
        return self._count(_native.native().ckl_invocation_edge_count, mode, batch_size)

    def node_name(self, index: int) -> str:
        return _native.native().ckl_invocation_node_name(self._native_resource.pointer, index).decode()

    def _average(self, function, index, iterations) -> float:
        out = ctypes.c_double()
        self._call(function, index, iterations, ctypes.byref(out))
        return out.value

    def time_node(self, index: int, iterations: int = 20) -> float:
        """Average microseconds of plan node `index` launched `iterations` times back to back
        (HIP events on the invocation stream). The node's writes are repeated."""
        return self._average(_native.native().ckl_invocation_time_node, index, iterations)

    def time_unit(self, unit: int, iterations: int = 20) -> float:
        """Average microseconds of inferred-step launch `unit` issued `iterations` times back to back."""
        return self._average(_native.native().ckl_invocation_time_unit, unit, iterations)

    def _unit_count(self) -> int:
        count = ctypes.c_uint64()
        self._call(_native.native().ckl_invocation_unit_count, ctypes.byref(count))
        return count.value

    def units(self) -> list:
        """The launches of one inferred step (chains contracted, siblings grouped): a list of
        (entry point, plan node indices)."""
        lib = _native.native()
        out = []
        for unit in range(self._unit_count()):
            name = ctypes.c_char_p()
            self._call(lib.ckl_invocation_unit_name, unit, ctypes.byref(name))
            n = ctypes.c_uint64()
            self._call(lib.ckl_invocation_unit_members, unit, None, 0, ctypes.byref(n))
            members = (ctypes.c_uint64 * max(1, n.value))()
            self._call(lib.ckl_invocation_unit_members, unit, members, n.value, ctypes.byref(n))
            out.append((name.value.decode(), [int(members[k]) for k in range(n.value)]))
        return out

    def profile_units(self, repeats: int = 7) -> list:
        """Durations (microseconds, `units()` order) of the inferred step's launches in sequence,
        from the median times of the step's launch-chain prefixes (each issued `repeats` times
        between HIP events; their effects are applied)."""
        count = self._unit_count()
        out = (ctypes.c_double * max(1, count))()
        n = ctypes.c_uint64()
        self._call(_native.native().ckl_invocation_profile_units, repeats, out, count, ctypes.byref(n))
        return [float(out[k]) for k in range(n.value)]

    def benchmark(self, *, iterations=200, graph=False, mode=None, batch_size=1) -> dict:
        """Time `iterations` submissions of `batch_size` program executions with HIP events on
        the invocation stream; returns per-program stream and wall microseconds plus graph setup."""
        if type(iterations) is not int or not 0 < iterations < _MAX_U64:
            raise ValueError("iterations must be a positive 64-bit count")
        execution = self._execution(graph, mode, batch_size)
        out = (ctypes.c_double * 3)()
        self._call(_native.native().ckl_invocation_benchmark, execution, iterations, batch_size, out)
        return {"stream_us": out[0], "wall_us": out[1], "graph_setup_ms": out[2]}


def run_requests(invocations, *, mode="graph", iterations=1, batch_size=1, serial=False) -> dict:
    """Independent requests (benchmarks/decoder/experiment.py:53-70): `iterations` runs of
    `batch_size` steps of every invocation in `mode`, each invocation on its own stream, submitted
    from this thread; concurrently (step k of every request before step k+1 of any) or, with
    `serial`, one request after another. The invocations may share read-only buffers; each owns
    its stream, heaps and workspaces. Returns the burst's host wall and GPU span in microseconds."""
    invocations = list(invocations)
    if not invocations or not all(isinstance(i, Invocation) for i in invocations):
        raise ValueError("run_requests takes one or more Invocation objects")
    if type(iterations) is not int or not 0 < iterations < _MAX_U64:
        raise ValueError("iterations must be a positive 64-bit count")
    execution = Invocation._execution(False, mode, batch_size)
    handles = (ctypes.c_void_p * len(invocations))(*[i._native_resource.pointer for i in invocations])
    out = (ctypes.c_double * 2)()
    _native.check(_native.native().ckl_invocations_run(handles, len(invocations), execution, iterations, batch_size,
                                                       1 if serial else 0, out))
    return {"wall_us": out[0], "span_us": out[1]}


def profiler_region(active: bool) -> None:
    """Resume (True) or pause (False) rocprofv3 collection under `--selected-regions`."""
    _native.check(_native.native().ckl_profiler_region(1 if active else 0))

