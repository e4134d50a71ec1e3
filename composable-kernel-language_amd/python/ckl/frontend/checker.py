"""Specialisation: resolve a definition's annotations and bind them to a concrete signature.

A specialisation fixes every runtime parameter to a BufferSpec or a numeric scalar type and every
`constexpr` parameter to a Python constant that fits its type. Dimensions named in buffer
annotations are unified across parameters (one size per name). The rules and diagnostics are the
reference's (python/ckl/frontend/checker.py:17-142); the implementation is a small binder over
the captured annotations.
"""
from __future__ import annotations

import ast
import math
import struct
from collections.abc import Mapping
from dataclasses import dataclass

from ..types import (Buffer, BufferSpec, BufferType, ConstexprType, Dimension, NUMERIC_TYPES, ScalarType, bool_,
                     constexpr, f32, f64, i32, i64, index)
from .source import Definition, Namespace, UnsupportedBinding


# ------------------------------------------------------------------------- annotations
def resolve(node: ast.AST, definition: Definition):
    """Evaluate an annotation expression against the definition's captured names."""
    if isinstance(node, ast.Constant):
        value = node.value
        if isinstance(value, str):             # a string annotation is parsed and evaluated
            return resolve(ast.parse(value, mode="eval").body, definition)
        if type(value) in (int, float, bool) or value is None:
            return value
    elif isinstance(node, ast.Name):
        if node.id not in definition.bindings:
            raise definition.error(node, f"unknown captured name '{node.id}'")
        value = definition.bindings[node.id]
        if isinstance(value, UnsupportedBinding):
            raise definition.error(node, f"unsupported captured binding '{node.id}'")
        return value
    elif isinstance(node, ast.Attribute):
        namespace = resolve(node.value, definition)
        if isinstance(namespace, Namespace) and node.attr in namespace.values:
            return namespace.values[node.attr]
    elif isinstance(node, ast.Tuple):
        return tuple(resolve(item, definition) for item in node.elts)
    elif isinstance(node, ast.Subscript):
        constructor = resolve(node.value, definition)
        if constructor is Buffer or constructor is constexpr:
            try:
                return constructor[resolve(node.slice, definition)]
            except ValueError as error:
                raise definition.error(node, str(error)) from error
    raise definition.error(node, "unsupported annotation; use CKL types and shape declarations")


def annotation_of(definition: Definition, argument: ast.arg):
    """The CKL type of one parameter: the captured annotation object, or its source expression."""
    captured = definition.annotations.get(argument.arg)
    if captured is not None and not isinstance(captured, str):
        return captured
    if argument.annotation is None:
        raise definition.error(argument, "every CKL parameter requires a type annotation")
    return resolve(argument.annotation, definition)


# ------------------------------------------------------------------------- constants
_INTEGER_BITS = {i32: 32, i64: 64, index: 64}


def _round_f32(value: float) -> float:
    return struct.unpack("<f", struct.pack("<f", value))[0]


def _fits(value, dtype):
    """`value` converted to `dtype`, or None when it does not fit."""
    if dtype == bool_:
        return value if type(value) is bool else None
    if dtype in _INTEGER_BITS:
        half = 1 << (_INTEGER_BITS[dtype] - 1)
        return value if type(value) is int and -half <= value < half else None
    if dtype in (f32, f64) and type(value) in (int, float):
        try:
            converted = float(value)
            if dtype == f32:
                converted = _round_f32(converted)
        except (OverflowError, struct.error):
            return None
        return converted if math.isfinite(converted) else None
    return None


def constant(value, dtype: ScalarType, definition: Definition, node: ast.AST):
    """A Python constant as a value of `dtype` (f32 values rounded to f32); diagnostic if it
    does not fit."""
    converted = _fits(value, dtype)
    if converted is None:
        shown = repr(value) if _is_plain(value) else f"<{type(value).__name__}>"
        raise definition.error(node, f"constant {shown} does not fit {dtype.name}")
    return converted


def _is_plain(value) -> bool:
    return value is None or type(value) in (int, float, bool, str)


# ------------------------------------------------------------------------- signatures
@dataclass(frozen=True)
class BoundParameter:
    """One parameter of a specialisation: runtime (dtype = BufferSpec or scalar type) or
    constant (value set, is_constant True)."""

    name: str
    dtype: object
    value: object = None
    is_constant: bool = False


@dataclass(frozen=True)
class BoundSignature:
    parameters: tuple
    dimensions: tuple          # sorted (dimension name, size) pairs

    @property
    def runtime(self) -> tuple:
        return tuple(p for p in self.parameters if not p.is_constant)


class _Binder:
    def __init__(self, definition: Definition, signature: Mapping, constants: Mapping):
        self.definition, self.signature, self.constants = definition, signature, constants
        self.sizes = {}

    def fail(self, node, message):
        raise self.definition.error(node, message)

    def check_parameter_list(self):
        args = self.definition.tree.args
        if args.posonlyargs or args.vararg or args.kwarg or args.kwonlyargs or args.defaults or args.kw_defaults:
            self.fail(self.definition.tree, "CKL definitions require named positional parameters without defaults")
        unknown = (set(self.signature) | set(self.constants)) - {a.arg for a in args.args}
        if unknown:
            self.fail(self.definition.tree, f"unknown specialization arguments: {sorted(unknown)}")
        return args.args

    def constexpr(self, argument, annotation: ConstexprType) -> BoundParameter:
        name = argument.arg
        if name not in self.constants or name in self.signature:
            self.fail(argument, "constexpr parameters require a constants binding, not a runtime signature")
        value = constant(self.constants[name], annotation.dtype, self.definition, argument)
        return BoundParameter(name, annotation.dtype, value, True)

    def unify(self, argument, expected: BufferType, actual: BufferSpec):
        for declared, size in zip(expected.shape, actual.shape):
            if isinstance(declared, Dimension):
                known = self.sizes.setdefault(declared.name, size)
                if known != size:
                    self.fail(argument, f"dimension {declared.name} conflicts: {known} versus {size}")
            elif declared != size:
                self.fail(argument, f"fixed extent {declared} does not match {size}")

    def runtime(self, argument, annotation) -> BoundParameter:
        name = argument.arg
        if name not in self.signature or name in self.constants:
            self.fail(argument, f"missing or misplaced runtime signature for '{name}'")
        actual = self.signature[name]
        if isinstance(annotation, BufferType):
            if not (isinstance(actual, BufferSpec) and actual.dtype == annotation.dtype
                    and len(actual.shape) == len(annotation.shape)):
                self.fail(argument, f"buffer type/rank mismatch for '{name}'")
            self.unify(argument, annotation, actual)
        elif any(annotation == t for t in NUMERIC_TYPES):
            if not (isinstance(actual, ScalarType) and actual == annotation):
                self.fail(argument, f"scalar type mismatch for '{name}'")
        else:
            self.fail(argument, "runtime parameters require numeric scalars or typed buffers")
        return BoundParameter(name, actual)

    def check_return(self):
        tree = self.definition.tree
        if tree.returns is None or self.definition.kind == "block":   # blocks may return buffers
            return
        declared = self.definition.annotations.get("return")
        if isinstance(declared, str):
            declared = resolve(tree.returns, self.definition)
        if declared is not None:
            self.fail(tree.returns, "CKL entry points have no return values")

    def bind(self) -> BoundSignature:
        bound = []
        for argument in self.check_parameter_list():
            annotation = annotation_of(self.definition, argument)
            if isinstance(annotation, ConstexprType):
                bound.append(self.constexpr(argument, annotation))
            else:
                bound.append(self.runtime(argument, annotation))
        self.check_return()
        return BoundSignature(tuple(bound), tuple(sorted(self.sizes.items())))


def bind(definition: Definition, signature: Mapping, constants: Mapping) -> BoundSignature:
    """Specialise `definition` for `signature` and `constants`."""
    if not isinstance(signature, Mapping) or not isinstance(constants, Mapping):
        raise definition.error(definition.tree, "signature and constants must be mappings")
    return _Binder(definition, signature, constants).bind()
