"""CKL on MI355X: the Composable Kernel Language authoring API with a HIP/gfx950 backend.

Public names follow python/ckl/__init__.py:1-27 of the reference (the NVIDIA target is
replaced by AMDTarget).
"""
from .compiler import AMDTarget, CompilationError, CompiledModule, compile_module
from .frontend import FrontendError, LoweredProgram, block, kernel, program
from .frontend.source import INTRINSICS as _intrinsics
from .hip import CompiledProgram, Device, DeviceBuffer, Invocation, profiler_region, run_requests, runtime_available
from .types import Buffer, BufferSpec, constexpr, dim, f32, f64, i32, i64, index
from .types import bool_ as bool

globals().update(_intrinsics)

__all__ = [
    "AMDTarget", "CompilationError", "CompiledModule", "compile_module",
    "CompiledProgram", "Device", "DeviceBuffer", "Invocation", "profiler_region", "run_requests", "runtime_available",
    "Buffer", "BufferSpec", "constexpr", "dim", "f32", "f64", "i32", "i64", "index", "bool",
    "FrontendError", "LoweredProgram", "block", "kernel", "program", *_intrinsics,
]
