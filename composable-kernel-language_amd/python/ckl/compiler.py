"""Target descriptor and in-process analysis entry points.

The reference's NVIDIATarget and ckl-opt subprocess driver (python/ckl/compiler.py:18-157) are
replaced by an AMD gfx950 target and the native pass driver of libckl_hip.so; nothing here
spawns a process.
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass
from typing import Sequence


class CompilationError(RuntimeError):
    def __init__(self, passes: Sequence[str], message: str):
        self.passes = tuple(passes)
        self.stderr = message
        super().__init__(f"CKL compilation failed: {';'.join(passes)}\n{message}")


@dataclass(frozen=True)
class AMDTarget:
    """MI355X code object target (gfx950, wave64)."""

    chip: str = "gfx950"
    features: str = ""
    binary_format: str = "hsaco"

    def cache_identity(self) -> str:
        return f"amd:{self.chip}:{self.features}:{self.binary_format}"


@dataclass(frozen=True)
class CompiledModule:
    source: str
    mlir: str
    passes: tuple
    cache_key: str


def compile_module(source: str, passes: Sequence[str] = ()) -> CompiledModule:
    """Verify IR text and run native passes over it in-process (summarize-effects, build-graph,
    lower-graph-to-exec, prepare-hip, fuse-pointwise, lower-exec-to-host; options in braces, e.g.
    "build-graph{strict=false}"; the item "allow-unregistered-dialect" admits unknown dialects).
    The ckl-opt executable beside the native library runs the same pipeline from a command line."""
    from ._native import native_opt
    try:
        output = native_opt(source, list(passes))
    except (ValueError, RuntimeError) as error:
        raise CompilationError(list(passes), str(error)) from error
    key = hashlib.sha256(source.encode() + b"\0" + "\0".join(passes).encode()).hexdigest()
    return CompiledModule(source, output, tuple(passes), key)
