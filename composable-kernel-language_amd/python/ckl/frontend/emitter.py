"""Typed AST lowering of CKL programs and kernels to CKL IR text.

The lowering rules (what is accepted, which operations are emitted and in which order, how
kernels are specialized per concrete signature) follow python/ckl/frontend/emitter.py:60-749
of the reference. Operation order is significant: allocations are emitted at `ckl.empty*`,
dispatches in source order and frees in reverse allocation order at the end of the program,
which fixes the dependency-graph node numbering. The IR is printed in MLIR generic syntax and
consumed by the native compiler (csrc/core/ir.cpp) instead of MLIR.
"""
from __future__ import annotations

import ast
import hashlib
import json
import math
import operator
from dataclasses import dataclass, field

from ..types import TOKEN, BufferSpec, ConstexprType, Dimension, ScalarType, bool_, f32, f64, i32, i64, index
from .checker import BoundSignature, bind, constant, resolve
from .source import Definition, Intrinsic, Namespace, UnsupportedBinding, fingerprint


# ---------------------------------------------------------------------------- a small SSA IR
class Value:
    __slots__ = ("dtype",)

    def __init__(self, dtype):
        self.dtype = dtype


@dataclass(eq=False)
class Op:
    name: str
    operands: list
    results: list
    attrs: list
    regions: list = field(default_factory=list)   # each region: a Block or None (empty)
    loc: str = ""


@dataclass(eq=False)
class Block:
    args: list = field(default_factory=list)
    ops: list = field(default_factory=list)


def type_text(dtype) -> str:
    if isinstance(dtype, BufferSpec):
        return dtype.mlir
    if dtype is TOKEN or getattr(dtype, "name", None) == "!ckl.token":
        return "!ckl.token"
    return dtype.mlir


def quote(text: str) -> str:
    out = []
    for ch in text:
        code = ord(ch)
        if ch == '"':
            out.append("\\22")
        elif ch == "\\":
            out.append("\\\\")
        elif code < 0x20 or code >= 0x7F:
            out.extend(f"\\{b:02X}" for b in ch.encode())
        else:
            out.append(ch)
    return '"' + "".join(out) + '"'


def int_attr(value: int, dtype) -> str:
    if dtype == bool_:
        return "true" if value else "false"
    return f"{int(value)} : {dtype.mlir}"


def float_attr(value: float, dtype) -> str:
    text = repr(float(value))
    if "." not in text and "e" not in text and "inf" not in text and "nan" not in text:
        text += ".0"
    return f"{text} : {dtype.mlir}"


def dense(values, width=64) -> str:
    values = list(values)
    return f"array<i{width}" + (": " + ", ".join(str(int(v)) for v in values) if values else "") + ">"


class Printer:
    def __init__(self, locations: bool):
        self.locations = locations
        self.names = {}
        self.values = 0
        self.args = 0

    def name(self, value: Value) -> str:
        return self.names[value]

    def define(self, value: Value, argument: bool) -> str:
        if argument:
            text = f"%arg{self.args}"
            self.args += 1
        else:
            text = f"%{self.values}"
            self.values += 1
        self.names[value] = text
        return text

    def op(self, op: Op, indent: int, lines: list):
        pad = "  " * indent
        head = ""
        if op.results:
            head = ", ".join(self.define(r, False) for r in op.results) + " = "
        text = f'{pad}{head}{quote(op.name)}(' + ", ".join(self.name(v) for v in op.operands) + ")"
        if op.regions:
            parts = []
            for region in op.regions:
                inner = []
                if region is not None:
                    if region.args:
                        args = ", ".join(f"{self.define(a, True)}: {type_text(a.dtype)}" for a in region.args)
                        inner.append(f"{pad}  ^bb0({args}):")
                    for child in region.ops:
                        self.op(child, indent + 2, inner)
                parts.append("{\n" + "".join(line + "\n" for line in inner) + pad + "}")
            text += " (" + ", ".join(parts) + ")"
        if op.attrs:
            text += " {" + ", ".join(key if value is None else f"{key} = {value}" for key, value in sorted(op.attrs)) + "}"
        text += " : (" + ", ".join(type_text(v.dtype) for v in op.operands) + ") -> "
        if len(op.results) == 1:
            text += type_text(op.results[0].dtype)
        else:
            text += "(" + ", ".join(type_text(r.dtype) for r in op.results) + ")"
        if self.locations and op.loc:
            text += f" loc({op.loc})"
        lines.append(text)

    def function(self, symbol: str, block: Block, attributes: list, loc: str, lines: list):
        args = ", ".join(f"{self.define(a, True)}: {type_text(a.dtype)}" for a in block.args)
        attrs = f" attributes {{{', '.join(attributes)}}}" if attributes else ""
        lines.append(f"  func.func @{symbol}({args}){attrs} {{")
        for op in block.ops:
            self.op(op, 2, lines)
        tail = f"  }} loc({loc})" if self.locations and loc else "  }"
        lines.append(tail)


@dataclass
class Function:
    symbol: str
    block: Block
    kernel: bool
    loc: str


def print_module(functions: list, locations: bool) -> str:
    lines = ["module {"]
    for fn in functions:
        Printer(locations).function(fn.symbol, fn.block, ["ckl.kernel"] if fn.kernel else [], fn.loc, lines)
    lines.append("}")
    return "\n".join(lines) + "\n"


def print_function(fn: Function, locations: bool = False) -> str:
    lines = []
    Printer(locations).function(fn.symbol, fn.block, ["ckl.kernel"] if fn.kernel else [], fn.loc, lines)
    return "\n".join(lines) + "\n"


# ---------------------------------------------------------------------------- lowering
@dataclass(frozen=True)
class Specialization:
    symbol: str
    identity: str
    signature: BoundSignature
    definition: Definition = field(compare=False, repr=False, default=None)


@dataclass(frozen=True)
class LoweredProgram:
    mlir: str
    signature: BoundSignature
    specializations: tuple
    cache_key: str
    diagnostics: tuple = ()
    kernels: tuple = ()        # canonical (name-free) text per specialization, same order
    extents: tuple = ()        # per specialization: sorted launched (x, y, z) thread extents

    def analyze(self, *passes: str) -> str:
        """Run native analysis passes (e.g. "build-graph") over this IR; no device work."""
        from .._native import native_opt
        return native_opt(self.mlir, passes)

    def verify(self) -> "LoweredProgram":
        self.analyze()
        return self

    def compile(self, *, target=None, fuse_pointwise=True, reuse_storage=True):
        """Compile for the HIP backend: plan in native code, kernels from the gfx950 library or JIT."""
        from ..hip import CompiledProgram
        return CompiledProgram(self, target, fuse_pointwise=fuse_pointwise, reuse_storage=reuse_storage)


def identity(definition: Definition, signature: BoundSignature) -> str:
    payload = [definition.identity, [
        [p.name, fingerprint(p.dtype) if isinstance(p.dtype, ScalarType) else [list(p.dtype.shape), p.dtype.dtype.name,
                                                                               p.dtype.layout],
         p.value, p.is_constant] for p in signature.parameters]]
    return hashlib.sha256(json.dumps(payload, sort_keys=True).encode()).hexdigest()


class ModuleEmitter:
    def __init__(self):
        self.functions: list = []
        self.kernels: dict = {}
        self.extents: dict = {}    # kernel symbol -> set of launched (x, y, z) thread extents

    def specialize(self, definition: Definition, signature: BoundSignature) -> Specialization:
        key = identity(definition, signature)
        if key not in self.kernels:
            spec = Specialization("kernel_" + key[:24], key, signature, definition)
            fn = FunctionEmitter(self, definition, signature).build(spec.symbol)
            self.kernels[key] = (spec, fn)
        return self.kernels[key][0]


STATIC_OPS = {ast.Add: operator.add, ast.Sub: operator.sub, ast.Mult: operator.mul, ast.Div: operator.truediv,
              ast.Lt: operator.lt, ast.LtE: operator.le, ast.Gt: operator.gt, ast.GtE: operator.ge,
              ast.Eq: operator.eq, ast.NotEq: operator.ne}
INT_PREDICATES = {ast.Eq: 0, ast.NotEq: 1, ast.Lt: 2, ast.LtE: 3, ast.Gt: 4, ast.GtE: 5}
FLOAT_PREDICATES = {ast.Eq: 1, ast.Gt: 2, ast.GtE: 3, ast.Lt: 4, ast.LtE: 5, ast.NotEq: 13}


class FunctionEmitter:
    """Lower one typed AST to IR operations (python/ckl/frontend/emitter.py:120-724)."""

    def __init__(self, module: ModuleEmitter, definition: Definition, signature: BoundSignature):
        self.module = module
        self.definition = definition
        self.signature = signature
        self.env: dict = {p.name: p.value for p in signature.parameters if p.is_constant}
        self.temporaries: list = []
        self.local_names = {p.name for p in signature.parameters} | {
            n.id for n in ast.walk(definition.tree) if isinstance(n, ast.Name) and isinstance(n.ctx, ast.Store)}
        self.dimensions = dict(signature.dimensions)
        self.block: Block = None

    # -------------------------------------------------------------- helpers
    def fail(self, node, message):
        raise self.definition.error(node, message)

    def location(self, node) -> str:
        line = self.definition.first_line + getattr(node, "lineno", 1) - 1
        column = self.definition.indentation + getattr(node, "col_offset", 0) + 1
        return f"{quote(self.definition.filename)}:{line}:{column}"

    def operation(self, name, node, *, operands=(), results=(), attrs=(), regions=()) -> Op:
        op = Op(name, list(operands), [Value(t) for t in results], list(attrs), list(regions), self.location(node))
        self.block.ops.append(op)
        return op

    def emit(self, name, dtype, node, *, operands=(), attrs=()) -> Value:
        return self.operation(name, node, operands=operands, results=[dtype], attrs=attrs).results[0]

    def build(self, symbol: str) -> Function:
        block = Block(args=[Value(p.dtype) for p in self.signature.runtime])
        fn = Function(symbol, block, self.definition.kind == "kernel", self.location(self.definition.tree))
        self.module.functions.append(fn)
        for parameter, argument in zip(self.signature.runtime, block.args):
            self.env[parameter.name] = argument
        self.block = block
        self.statements(self.definition.tree.body, top=True)
        for temporary in reversed(self.temporaries):
            self.operation("ckl.free", self.definition.tree, operands=[temporary])
        self.operation("func.return", self.definition.tree)
        return fn

    def typed(self, value, dtype, node) -> Value:
        if isinstance(value, Value):
            if value.dtype != dtype:
                shown = type_text(value.dtype)
                self.fail(node, f"expected {dtype.name}, got {shown}; use ckl.cast explicitly")
            return value
        value = constant(value, dtype, self.definition, node)
        attr = float_attr(value, dtype) if dtype in (f32, f64) else int_attr(int(value), dtype)
        return self.emit("arith.constant", dtype, node, attrs=[("value", attr)])

    def buffer(self, node) -> Value:
        value = self.expression(node)
        if not isinstance(value, Value) or not isinstance(value.dtype, BufferSpec):
            self.fail(node, "expected a typed buffer")
        return value

    def indices(self, buffer: Value, node: ast.Subscript) -> list:
        nodes = node.slice.elts if isinstance(node.slice, ast.Tuple) else [node.slice]
        if len(nodes) != len(buffer.dtype.shape):
            self.fail(node, "requires one index per buffer dimension")
        result = []
        for axis, item in enumerate(nodes):
            value = self.expression(item)
            if type(value) is int and not 0 <= value < buffer.dtype.shape[axis]:
                self.fail(item, f"constant index is out of bounds for dimension {axis}")
            result.append(self.typed(value, index, item))
        return result

    def require_kernel_arithmetic(self, node):
        if self.definition.kind != "kernel":
            self.fail(node, "computed runtime host scalars are unsupported; forward the parameter unchanged")

    # -------------------------------------------------------------- expressions
    def expression(self, node):
        if isinstance(node, ast.Constant) and type(node.value) in (int, float, bool):
            if type(node.value) is float and not math.isfinite(node.value):
                self.fail(node, "non-finite source constants are unsupported")
            return node.value
        if isinstance(node, ast.Name):
            if node.id in self.env:
                return self.env[node.id]
            if node.id in self.local_names:
                self.fail(node, f"local '{node.id}' is not defined on this path")
            if node.id not in self.definition.bindings:
                self.fail(node, f"unknown name '{node.id}'")
            captured = self.definition.bindings[node.id]
            if isinstance(captured, UnsupportedBinding):
                self.fail(node, f"unsupported captured binding '{node.id}'")
            if isinstance(captured, Dimension):
                if captured.name not in self.dimensions:
                    self.fail(node, f"unbound dimension '{captured.name}'")
                return self.dimensions[captured.name]
            return captured
        if isinstance(node, ast.Tuple):
            return tuple(self.expression(item) for item in node.elts)
        if isinstance(node, ast.Attribute):
            base = self.expression(node.value)
            if isinstance(base, Namespace) and node.attr in base.values:
                return base.values[node.attr]
            if isinstance(base, Value) and isinstance(base.dtype, BufferSpec):
                if node.attr == "shape":
                    return base.dtype.shape
                if node.attr == "dtype":
                    return base.dtype.dtype
            self.fail(node, f"unsupported attribute '{node.attr}'")
        if isinstance(node, ast.Subscript):
            base = self.expression(node.value)
            if isinstance(base, Value) and isinstance(base.dtype, BufferSpec):
                if self.definition.kind != "kernel":
                    self.fail(node, "buffer contents can only be accessed inside a kernel")
                return self.emit("ckl.load_element", base.dtype.dtype, node, operands=[base, *self.indices(base, node)])
            if type(base) is tuple:
                position = self.expression(node.slice)
                if type(position) is not int or not 0 <= position < len(base):
                    self.fail(node, "tuple/shape axes require an in-range nonnegative compile-time integer")
                return base[position]
            self.fail(node, "unsupported subscript; slices and negative indexing are not supported")
        if isinstance(node, ast.BinOp):
            return self.binary(node)
        if isinstance(node, ast.UnaryOp) and isinstance(node.op, (ast.USub, ast.UAdd)):
            value = self.expression(node.operand)
            if type(value) in (int, float):
                return -value if isinstance(node.op, ast.USub) else value
            if not isinstance(value, Value) or not isinstance(value.dtype, ScalarType) or value.dtype == bool_:
                self.fail(node, "unary arithmetic requires a numeric scalar")
            self.require_kernel_arithmetic(node)
            if isinstance(node.op, ast.UAdd):
                return value
            if value.dtype in (f32, f64):
                return self.emit("arith.negf", value.dtype, node, operands=[value])
            zero = self.typed(0, value.dtype, node)
            return self.emit("arith.subi", value.dtype, node, operands=[zero, value])
        if isinstance(node, ast.Compare):
            if len(node.ops) != 1:
                self.fail(node, "chained comparisons are not supported")
            return self.binary(node, comparison=True)
        if isinstance(node, ast.Call):
            return self.call(node)
        self.fail(node, f"unsupported expression: {type(node).__name__}")

    def binary(self, node, comparison=False):
        left = self.expression(node.left)
        right = self.expression(node.comparators[0] if comparison else node.right)
        op = node.ops[0] if comparison else node.op
        if type(op) not in STATIC_OPS:
            self.fail(node, f"unsupported numeric operator: {type(op).__name__}")
        if not isinstance(left, Value) and not isinstance(right, Value):
            allowed = (int, float, bool) if comparison else (int, float)
            if type(left) not in allowed or type(right) not in allowed:
                self.fail(node, "numeric expressions require scalar operands")
            try:
                result = STATIC_OPS[type(op)](left, right)
            except (ZeroDivisionError, OverflowError) as error:
                self.fail(node, f"invalid constant expression: {error}")
            if type(result) is float and not math.isfinite(result):
                self.fail(node, "non-finite constant expression")
            return result
        self.require_kernel_arithmetic(node)
        dtype = (left if isinstance(left, Value) else right).dtype
        if not isinstance(dtype, ScalarType) or (dtype == bool_ and type(op) not in (ast.Eq, ast.NotEq)):
            self.fail(node, "numeric expressions require compatible scalar types")
        left, right = self.typed(left, dtype, node), self.typed(right, dtype, node)
        floating = dtype in (f32, f64)
        if comparison:
            predicate = (FLOAT_PREDICATES if floating else INT_PREDICATES)[type(op)]
            return self.emit("arith.cmpf" if floating else "arith.cmpi", bool_, node, operands=[left, right],
                             attrs=[("predicate", f"{predicate} : i64")])
        if isinstance(op, ast.Div) and not floating:
            self.fail(node, "division requires floating operands")
        mnemonic = {ast.Add: "add", ast.Sub: "sub", ast.Mult: "mul", ast.Div: "div"}[type(op)]
        return self.emit(f"arith.{mnemonic}{'f' if floating else 'i'}", dtype, node, operands=[left, right])

    def call(self, node: ast.Call):
        callee = self.expression(node.func)
        if isinstance(callee, Definition):
            self.fail(node, "kernel definitions are not ordinary calls; use ckl.launch")
        if not isinstance(callee, Intrinsic):
            self.fail(node, "calling arbitrary Python functions is unsupported")
        if any(isinstance(a, ast.Starred) for a in node.args) or any(k.arg is None for k in node.keywords):
            self.fail(node, "argument expansion is unsupported")
        name = callee.name
        if name == "launch":
            return self.launch(node)
        args = [self.expression(a) for a in node.args]
        keywords = {k.arg: self.expression(k.value) for k in node.keywords}
        if len(keywords) != len(node.keywords):
            self.fail(node, "duplicate keyword arguments")
        if name in ("global_id", "thread_id", "block_id", "block_dim", "grid_dim"):
            if self.definition.kind != "kernel":
                self.fail(node, "device coordinates are only valid in kernels")
            if len(args) != 1 or keywords or type(args[0]) is not int or not 0 <= args[0] <= 2:
                self.fail(node, "device coordinates require one constant axis 0, 1, or 2")
            return self.emit(f"ckl.{name}", index, node, attrs=[("axis", f"{args[0]} : i32")])
        if name == "cdiv":
            if len(args) != 2 or keywords or any(type(v) is not int for v in args) or args[0] < 0 or args[1] <= 0:
                self.fail(node, "cdiv requires a nonnegative constant extent and positive constant divisor")
            return (args[0] + args[1] - 1) // args[1]
        if name in ("empty", "empty_like"):
            if self.definition.kind != "program":
                self.fail(node, "program temporaries cannot be allocated inside kernels")
            if name == "empty_like":
                if len(args) != 1 or keywords or not isinstance(args[0], Value) or not isinstance(args[0].dtype, BufferSpec):
                    self.fail(node, "empty_like requires one buffer")
                spec = args[0].dtype
            else:
                if len(args) != 1 or set(keywords) != {"dtype"}:
                    self.fail(node, "use empty(shape_tuple, dtype=element_type)")
                try:
                    spec = BufferSpec(args[0], keywords["dtype"])
                except (ValueError, TypeError) as error:
                    self.fail(node, str(error))
            value = self.emit("ckl.alloc", spec, node)
            self.temporaries.append(value)
            return value
        if name == "subview":
            if self.definition.kind != "program":
                self.fail(node, "subview is currently supported only in programs")
            if len(args) != 1 or set(keywords) != {"offset", "shape"} or not isinstance(args[0], Value) or \
                    not isinstance(args[0].dtype, BufferSpec):
                self.fail(node, "use subview(buffer, offset=element_offset, shape=shape_tuple)")
            source, offset = args[0], keywords["offset"]
            try:
                spec = BufferSpec(keywords["shape"], source.dtype.dtype)
            except (TypeError, ValueError) as error:
                self.fail(node, str(error))
            if type(offset) is not int or offset < 0 or offset >= (1 << 63) or \
                    offset + math.prod(spec.shape) > math.prod(source.dtype.shape):
                self.fail(node, "subview offset/shape must be constant and within the source")
            return self.emit("ckl.subview", spec, node, operands=[source], attrs=[("offset", f"{offset} : i64")])
        if name == "cast":
            if len(args) != 2 or keywords or not isinstance(args[1], ScalarType):
                self.fail(node, "use cast(value, scalar_type)")
            return self.cast(args[0], args[1], node)
        if name in ("exp", "rsqrt"):
            self.require_kernel_arithmetic(node)
            if len(args) != 1 or keywords or not isinstance(args[0], Value) or args[0].dtype not in (f32, f64):
                self.fail(node, f"{name} requires one typed floating-point scalar")
            return self.emit(f"math.{name}", args[0].dtype, node, operands=[args[0]])
        if name == "select":
            self.require_kernel_arithmetic(node)
            if len(args) != 3 or keywords:
                self.fail(node, "use select(predicate, true_value, false_value)")
            condition = self.typed(args[0], bool_, node)
            dynamic = next((v for v in args[1:] if isinstance(v, Value)), None)
            if dynamic is None or not isinstance(dynamic.dtype, ScalarType):
                self.fail(node, "select requires a typed scalar alternative")
            lhs, rhs = [self.typed(v, dynamic.dtype, node) for v in args[1:]]
            return self.emit("arith.select", lhs.dtype, node, operands=[condition, lhs, rhs])
        self.fail(node, f"unsupported intrinsic: {name}")

    def cast(self, value, dtype, node):
        if not isinstance(value, Value):
            if dtype in (i32, i64, index) and type(value) is float and math.isfinite(value):
                value = int(value)
            return constant(value, dtype, self.definition, node)
        self.require_kernel_arithmetic(node)
        source = value.dtype
        if source == dtype:
            return value
        if not isinstance(source, ScalarType) or bool_ in (source, dtype):
            self.fail(node, "boolean/buffer casts are unsupported")
        floats, integers = (f32, f64), (i32, i64)
        if source in floats and dtype in floats:
            operation = "extf" if dtype == f64 else "truncf"
        elif source in integers and dtype in integers:
            operation = "extsi" if dtype == i64 else "trunci"
        elif source in floats and dtype in integers:
            operation = "fptosi"
        elif source in integers and dtype in floats:
            operation = "sitofp"
        elif index in (source, dtype) and (source in integers or dtype in integers):
            operation = "index_cast"
        else:
            self.fail(node, "cast through an integer type to convert between index and float")
        return self.emit(f"arith.{operation}", dtype, node, operands=[value])

    # -------------------------------------------------------------- launches
    def launch(self, node: ast.Call):
        if self.definition.kind != "program":
            self.fail(node, "kernels cannot launch other kernels")
        if not node.args:
            self.fail(node, "launch requires a kernel definition")
        definition = self.expression(node.args[0])
        if not isinstance(definition, Definition) or definition.kind != "kernel":
            self.fail(node, "launch requires a @ckl.kernel definition")
        parameters = definition.tree.args.args
        if len(node.args) - 1 != len(parameters):
            self.fail(node, "launch argument count does not match kernel signature")
        keywords = {k.arg: self.expression(k.value) for k in node.keywords}
        if set(keywords) - {"grid", "block", "shared_memory"} or not {"grid", "block"} <= set(keywords):
            self.fail(node, "launch requires grid and block; only shared_memory is optional")
        geometry = []
        for key in ("grid", "block"):
            dims = keywords[key]
            if type(dims) is not tuple or not 1 <= len(dims) <= 3 or \
                    any(type(d) is not int or not 0 < d < (1 << 63) for d in dims):
                self.fail(node, f"{key} requires a tuple of one to three positive compile-time integers")
            geometry.append(dims + (1,) * (3 - len(dims)))
        shared = keywords.get("shared_memory", 0)
        if type(shared) is not int or not 0 <= shared < (1 << 63):
            self.fail(node, "shared_memory requires nonnegative compile-time bytes")
        signature, constants, operands = {}, {}, []
        for parameter, argument in zip(parameters, node.args[1:]):
            annotation = definition.annotations.get(parameter.arg)
            if isinstance(annotation, str) or annotation is None:
                if parameter.annotation is None:
                    self.fail(node, "kernel parameters require annotations")
                annotation = resolve(parameter.annotation, definition)
            actual = self.expression(argument)
            if isinstance(annotation, ConstexprType):
                if isinstance(actual, Value):
                    self.fail(argument, "constexpr launch arguments must be compile-time constants")
                constants[parameter.arg] = actual
                continue
            if isinstance(annotation, ScalarType):
                actual = self.typed(actual, annotation, argument)
            if not isinstance(actual, Value):
                self.fail(argument, "kernel arguments must be typed buffers or scalars")
            signature[parameter.arg] = actual.dtype
            operands.append(actual)
        bound = bind(definition, signature, constants)
        spec = self.module.specialize(definition, bound)
        grid, block = geometry
        self.module.extents.setdefault(spec.symbol, set()).add(tuple(g * b for g, b in zip(grid, block)))
        attrs = [("kernel", f"@{spec.symbol}"), ("grid", dense(grid)), ("block", dense(block)),
                 ("shared_memory", f"{shared} : i64"), ("device", quote("unassigned:0")), ("capabilities", "[]"),
                 ("implementation", quote(spec.identity)), ("operandSegmentSizes", dense([len(operands), 0], 32))]
        # Dependencies are inferred from effects, not chained through completion tokens.
        self.emit("ckl.dispatch", TOKEN, node, operands=operands, attrs=attrs)

    # -------------------------------------------------------------- statements
    def region_block(self, args=()) -> Block:
        return Block(args=list(args))

    def statements(self, nodes, *, top=False, branch_outer=None):
        for position, node in enumerate(nodes):
            if isinstance(node, ast.Return):
                if not top or position != len(nodes) - 1 or node.value is not None:
                    self.fail(node, "only a final bare return is supported; buffers carry outputs")
            elif isinstance(node, ast.Assign):
                if len(node.targets) != 1:
                    self.fail(node, "chained assignment is unsupported")
                target = node.targets[0]
                value = self.expression(node.value)
                if isinstance(target, ast.Name):
                    if value is None:
                        self.fail(node, "launches do not return source values")
                    if branch_outer is not None and target.id in branch_outer:
                        self.fail(target, "runtime branch results are deferred; write buffers or use branch-local variables")
                    old = self.env.get(target.id)
                    if isinstance(old, Value) and isinstance(old.dtype, ScalarType):
                        value = self.typed(value, old.dtype, node.value)
                    self.env[target.id] = value
                elif isinstance(target, ast.Subscript):
                    if self.definition.kind != "kernel":
                        self.fail(target, "buffer writes are only valid in kernels")
                    buffer = self.buffer(target.value)
                    indices = self.indices(buffer, target)
                    value = self.typed(value, buffer.dtype.dtype, node.value)
                    self.operation("ckl.store_element", node, operands=[value, buffer, *indices])
                else:
                    self.fail(target, "assignment requires a local name or indexed buffer element")
            elif isinstance(node, ast.If):
                predicate = self.expression(node.test)
                if type(predicate) is bool:
                    self.statements(node.body if predicate else node.orelse, branch_outer=branch_outer)
                    continue
                if self.definition.kind != "kernel" or not isinstance(predicate, Value) or predicate.dtype != bool_:
                    self.fail(node.test, "if requires a boolean predicate; program control flow must be compile-time")
                outer = self.env.copy()
                then_block = self.region_block()
                else_block = self.region_block() if node.orelse else None
                self.operation("scf.if", node, operands=[predicate], regions=[then_block, else_block])
                parent = self.block
                self.block = then_block
                self.statements(node.body, branch_outer=set(outer))
                self.operation("scf.yield", node)
                self.env = outer.copy()
                if else_block is not None:
                    self.block = else_block
                    self.statements(node.orelse, branch_outer=set(outer))
                    self.operation("scf.yield", node)
                self.block = parent
                self.env = outer
            elif isinstance(node, ast.For):
                self.for_loop(node, branch_outer)
            elif isinstance(node, ast.Expr):
                if isinstance(node.value, ast.Constant) and isinstance(node.value.value, str) and position == 0 and top:
                    continue
                if not isinstance(node.value, ast.Call) or self.expression(node.value) is not None:
                    self.fail(node, "expression statements must be kernel launches")
            elif isinstance(node, ast.Pass):
                continue
            else:
                self.fail(node, f"unsupported statement: {type(node).__name__}")

    def for_loop(self, node: ast.For, branch_outer):
        if node.orelse or not isinstance(node.target, ast.Name) or not isinstance(node.iter, ast.Call):
            self.fail(node, "for requires a simple induction variable and range without else")
        callee = self.expression(node.iter.func)
        if not isinstance(callee, Intrinsic) or callee.name != "range" or node.iter.keywords:
            self.fail(node, "for requires range(start, stop, positive_constant_step)")
        bounds = [self.expression(a) for a in node.iter.args]
        if not 1 <= len(bounds) <= 3:
            self.fail(node, "range requires one to three bounds")
        start, stop, step = (0, bounds[0], 1) if len(bounds) == 1 else \
            (bounds[0], bounds[1], bounds[2] if len(bounds) == 3 else 1)
        if type(step) is not int or step <= 0:
            self.fail(node, "range step must be a positive compile-time integer")
        induction = node.target.id
        outer = self.env.copy()
        if self.definition.kind == "program":
            if type(start) is not int or type(stop) is not int:
                self.fail(node, "program range bounds must be compile-time integers")
            if len(range(start, stop, step)) > 1024:
                self.fail(node, "program unrolling is limited to 1024 iterations")
            for value in range(start, stop, step):
                self.env[induction] = value
                self.statements(node.body, branch_outer=branch_outer)
            if induction in outer:
                self.env[induction] = outer[induction]
            else:
                self.env.pop(induction, None)
            return
        assignments = {n.id for s in node.body for n in ast.walk(s) if isinstance(n, ast.Name) and isinstance(n.ctx, ast.Store)}
        if induction in assignments:
            self.fail(node, "cannot assign to the loop induction variable")
        names = sorted(assignments & outer.keys())
        initials = []
        for name in names:
            if branch_outer is not None and name in branch_outer:
                self.fail(node, "runtime branch results are deferred")
            value = outer[name]
            if not isinstance(value, Value):
                dtype = f32 if type(value) is float else i32 if type(value) is int else bool_
                value = self.typed(value, dtype, node)
            if not isinstance(value.dtype, ScalarType):
                self.fail(node, "loop-carried locals must be scalars")
            initials.append(value)
        lower, upper, stride = [self.typed(v, index, node) for v in (start, stop, step)]
        body = self.region_block([Value(index)] + [Value(v.dtype) for v in initials])
        loop = self.operation("scf.for", node, operands=[lower, upper, stride, *initials],
                              results=[v.dtype for v in initials], regions=[body])
        self.env[induction] = body.args[0]
        self.env.update((name, arg) for name, arg in zip(names, body.args[1:]))
        parent = self.block
        self.block = body
        self.statements(node.body, branch_outer=branch_outer)
        yielded = [self.typed(self.env[name], initial.dtype, node) for name, initial in zip(names, initials)]
        self.operation("scf.yield", node, operands=yielded)
        self.block = parent
        self.env = outer
        for name, result in zip(names, loop.results):
            self.env[name] = result


def lower_program(definition: Definition, signature, constants, *, verify=False) -> LoweredProgram:
    """Lower a program and every kernel it launches; returns the IR text and specializations."""
    bound = bind(definition, signature, constants)
    program_identity = identity(definition, bound)
    module = ModuleEmitter()
    FunctionEmitter(module, definition, bound).build("program_" + program_identity[:24])
    text = print_module(module.functions, locations=True)
    semantic = print_module(module.functions, locations=False)
    key = hashlib.sha256((program_identity + semantic).encode()).hexdigest()
    specs = tuple(spec for spec, _ in module.kernels.values())
    canonical = tuple(canonical_kernel(fn) for _, fn in module.kernels.values())
    extents = tuple(tuple(sorted(module.extents.get(spec.symbol, ()))) for spec in specs)
    result = LoweredProgram(text, bound, specs, key, (), canonical, extents)
    if verify:
        result.verify()
    return result


def canonical_kernel(fn: Function) -> str:
    """Kernel text without its symbol or locations: equal bodies print equal text."""
    return print_function(Function("kernel", fn.block, fn.kernel, ""), locations=False)


def lower_kernel(definition: Definition, signature: BoundSignature) -> str:
    """Canonical text of `definition` specialized for a bound signature (library matching)."""
    module = ModuleEmitter()
    spec = module.specialize(definition, signature)
    return canonical_kernel(module.kernels[spec.identity][1])
