"""Lowering of CKL definitions to CKL IR.

A program is lowered for one concrete signature. Its body runs at compile time in the sense that
every host-side value (shapes, grid sizes, loop bounds, constants) is a Python value computed
here: program loops are unrolled and program `if`s are decided, so the only operations left in
the program function are allocations, subviews, scalar constants handed to kernels, dispatches
and frees. Every kernel a program launches is specialised for the argument types and constants
of that launch (identical specialisations are shared) and lowered to structured IR (`scf.if`,
`scf.for` with loop-carried scalars, arithmetic, element loads and stores).

The accepted language, the order of operations and the diagnostics are the reference's
(python/ckl/frontend/emitter.py:60-749): allocations appear at `ckl.empty*`, dispatches in
source order and frees in reverse allocation order at the end of the program, which fixes the
dependency graph's node numbering. Calls of `@ckl.block` fragments (no reference counterpart)
are expanded in place and leave the same operations their bodies would leave written inline.

Structure: `Lowering` evaluates expressions and statements by node type (`expr_<Node>`,
`stmt_<Node>` methods) and looks intrinsics up in per-class tables; `KernelLowering` and
`ProgramLowering` supply what differs between device bodies and host compositions.
"""
from __future__ import annotations

import ast
import hashlib
import json
import math
import operator
from dataclasses import dataclass, field

from ..types import TOKEN, BufferSpec, ConstexprType, Dimension, ScalarType, bool_, f32, f64, i32, i64, index
from .checker import BoundSignature, annotation_of, bind, constant
from .ir import Block, Function, Op, Value, dense, float_attr, int_attr, print_function, print_module, quote, type_text
from .source import Definition, Intrinsic, Namespace, UnsupportedBinding, fingerprint


# ---------------------------------------------------------------------------- results
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
    """Identity of a specialisation: the definition's identity plus its bound parameters."""
    parameters = []
    for p in signature.parameters:
        if isinstance(p.dtype, ScalarType):
            described = fingerprint(p.dtype)
        else:
            described = [list(p.dtype.shape), p.dtype.dtype.name, p.dtype.layout]
        parameters.append([p.name, described, p.value, p.is_constant])
    return hashlib.sha256(json.dumps([definition.identity, parameters], sort_keys=True).encode()).hexdigest()


class Module:
    """The functions of one lowered program: the program first, then each kernel
    specialisation in the order its first launch is lowered."""

    def __init__(self):
        self.functions = []
        self.specializations = {}     # identity -> (Specialization, Function)
        self.extents = {}             # kernel symbol -> set of launched (x, y, z) thread extents

    def specialize(self, definition: Definition, signature: BoundSignature) -> Specialization:
        key = identity(definition, signature)
        if key not in self.specializations:
            spec = Specialization("kernel_" + key[:24], key, signature, definition)
            self.specializations[key] = (spec, KernelLowering(self, definition, signature).function(spec.symbol))
        return self.specializations[key][0]


# ---------------------------------------------------------------------------- operator tables
_FOLD = {ast.Add: operator.add, ast.Sub: operator.sub, ast.Mult: operator.mul, ast.Div: operator.truediv,
         ast.Lt: operator.lt, ast.LtE: operator.le, ast.Gt: operator.gt, ast.GtE: operator.ge,
         ast.Eq: operator.eq, ast.NotEq: operator.ne}
_ARITH = {ast.Add: "add", ast.Sub: "sub", ast.Mult: "mul", ast.Div: "div"}
# arith.cmpi / arith.cmpf predicate numbers (MLIR's enums; cmpf uses the ordered forms, une for !=)
_CMPI = {ast.Eq: 0, ast.NotEq: 1, ast.Lt: 2, ast.LtE: 3, ast.Gt: 4, ast.GtE: 5}
_CMPF = {ast.Eq: 1, ast.Gt: 2, ast.GtE: 3, ast.Lt: 4, ast.LtE: 5, ast.NotEq: 13}
_COORDINATES = ("global_id", "thread_id", "block_id", "block_dim", "grid_dim")
_CASTS = {  # (source category, target category) -> arith operation, width-dependent ones resolved below
    ("float", "float"): None, ("signed", "signed"): None, ("float", "signed"): "fptosi",
    ("signed", "float"): "sitofp", ("index", "signed"): "index_cast", ("signed", "index"): "index_cast",
}


def _scalar(value) -> bool:
    return isinstance(value, Value) and isinstance(value.dtype, ScalarType)


def _buffer(value) -> bool:
    return isinstance(value, Value) and isinstance(value.dtype, BufferSpec)


class Lowering:
    """Shared machinery: scopes, operation emission, expressions and statements."""

    # intrinsic name -> method name; subclasses extend
    INTRINSICS = {"cdiv": "intrinsic_cdiv", "cast": "intrinsic_cast"}

    def __init__(self, module: Module, definition: Definition, signature: BoundSignature, *, scope=None,
                 temporaries=None):
        self.module, self.definition, self.signature = module, definition, signature
        self.scope = {p.name: p.value for p in signature.parameters if p.is_constant} if scope is None else scope
        self.assigned = {p.name for p in signature.parameters} | {
            n.id for n in ast.walk(definition.tree) if isinstance(n, ast.Name) and isinstance(n.ctx, ast.Store)}
        self.sizes = dict(signature.dimensions)
        self.temporaries = [] if temporaries is None else temporaries
        self.block: Block = None
        self.deferred = None          # names a runtime branch may not rebind (kernels)

    # ---------------------------------------------------------------- emission
    def fail(self, node, message):
        raise self.definition.error(node, message)

    def where(self, node) -> str:
        d = self.definition
        line = d.first_line + getattr(node, "lineno", 1) - 1
        column = d.indentation + getattr(node, "col_offset", 0) + 1
        return f"{quote(d.filename)}:{line}:{column}"

    def op(self, name, node, *, operands=(), results=(), attrs=(), regions=()) -> Op:
        operation = Op(name, list(operands), [Value(t) for t in results], list(attrs), list(regions), self.where(node))
        self.block.ops.append(operation)
        return operation

    def value(self, name, dtype, node, *, operands=(), attrs=()) -> Value:
        return self.op(name, node, operands=operands, results=[dtype], attrs=attrs).results[0]

    def as_type(self, value, dtype, node) -> Value:
        """`value` as an IR value of `dtype`: an existing value must already have that type; a
        Python constant becomes an `arith.constant`."""
        if isinstance(value, Value):
            if value.dtype != dtype:
                self.fail(node, f"expected {dtype.name}, got {type_text(value.dtype)}; use ckl.cast explicitly")
            return value
        folded = constant(value, dtype, self.definition, node)
        text = float_attr(folded, dtype) if dtype in (f32, f64) else int_attr(int(folded), dtype)
        return self.value("arith.constant", dtype, node, attrs=[("value", text)])

    # ---------------------------------------------------------------- hooks for subclasses
    def runtime_arithmetic(self, node):
        """Called before emitting arithmetic on runtime values."""

    def load(self, buffer: Value, node: ast.Subscript):
        self.fail(node, "buffer contents can only be accessed inside a kernel")

    def store(self, target: ast.Subscript, value, node):
        self.fail(target, "buffer writes are only valid in kernels")

    def runtime_if(self, node: ast.If, predicate):
        self.fail(node.test, "if requires a boolean predicate; program control flow must be compile-time")

    def loop(self, node: ast.For, start, stop, step):
        raise NotImplementedError

    def call_definition(self, node: ast.Call, callee: Definition):
        self.fail(node, "kernel definitions are not ordinary calls; use ckl.launch")

    def statement_return(self, node: ast.Return, last: bool, top: bool):
        if not top or not last or node.value is not None:
            self.fail(node, "only a final bare return is supported; buffers carry outputs")

    # ---------------------------------------------------------------- expressions
    def evaluate(self, node):
        handler = getattr(self, "expr_" + type(node).__name__, None)
        if handler is None:
            self.fail(node, f"unsupported expression: {type(node).__name__}")
        return handler(node)

    def expr_Constant(self, node):
        if type(node.value) not in (int, float, bool):
            self.fail(node, "unsupported expression: Constant")
        if type(node.value) is float and not math.isfinite(node.value):
            self.fail(node, "non-finite source constants are unsupported")
        return node.value

    def expr_Name(self, node):
        name = node.id
        if name in self.scope:
            return self.scope[name]
        if name in self.assigned:
            self.fail(node, f"local '{name}' is not defined on this path")
        if name not in self.definition.bindings:
            self.fail(node, f"unknown name '{name}'")
        captured = self.definition.bindings[name]
        if isinstance(captured, UnsupportedBinding):
            self.fail(node, f"unsupported captured binding '{name}'")
        if isinstance(captured, Dimension):
            if captured.name not in self.sizes:
                self.fail(node, f"unbound dimension '{captured.name}'")
            return self.sizes[captured.name]
        return captured

    def expr_Tuple(self, node):
        return tuple(self.evaluate(item) for item in node.elts)

    def expr_Attribute(self, node):
        base = self.evaluate(node.value)
        if isinstance(base, Namespace) and node.attr in base.values:
            return base.values[node.attr]
        if _buffer(base) and node.attr in ("shape", "dtype"):
            return base.dtype.shape if node.attr == "shape" else base.dtype.dtype
        self.fail(node, f"unsupported attribute '{node.attr}'")

    def expr_Subscript(self, node):
        base = self.evaluate(node.value)
        if _buffer(base):
            return self.load(base, node)
        if type(base) is tuple:
            position = self.evaluate(node.slice)
            if type(position) is not int or not 0 <= position < len(base):
                self.fail(node, "tuple/shape axes require an in-range nonnegative compile-time integer")
            return base[position]
        self.fail(node, "unsupported subscript; slices and negative indexing are not supported")

    def element_indices(self, buffer: Value, node: ast.Subscript) -> list:
        items = node.slice.elts if isinstance(node.slice, ast.Tuple) else [node.slice]
        if len(items) != len(buffer.dtype.shape):
            self.fail(node, "requires one index per buffer dimension")
        out = []
        for axis, item in enumerate(items):
            value = self.evaluate(item)
            if type(value) is int and not 0 <= value < buffer.dtype.shape[axis]:
                self.fail(item, f"constant index is out of bounds for dimension {axis}")
            out.append(self.as_type(value, index, item))
        return out

    def expr_UnaryOp(self, node):
        if not isinstance(node.op, (ast.USub, ast.UAdd)):
            self.fail(node, "unsupported expression: UnaryOp")
        operand = self.evaluate(node.operand)
        negate = isinstance(node.op, ast.USub)
        if type(operand) in (int, float):
            return -operand if negate else operand
        if not _scalar(operand) or operand.dtype == bool_:
            self.fail(node, "unary arithmetic requires a numeric scalar")
        self.runtime_arithmetic(node)
        if not negate:
            return operand
        if operand.dtype in (f32, f64):
            return self.value("arith.negf", operand.dtype, node, operands=[operand])
        zero = self.as_type(0, operand.dtype, node)
        return self.value("arith.subi", operand.dtype, node, operands=[zero, operand])

    def expr_BinOp(self, node):
        return self.arithmetic(node, node.op, node.left, node.right, comparison=False)

    def expr_Compare(self, node):
        if len(node.ops) != 1:
            self.fail(node, "chained comparisons are not supported")
        return self.arithmetic(node, node.ops[0], node.left, node.comparators[0], comparison=True)

    def arithmetic(self, node, op, left_node, right_node, *, comparison):
        left, right = self.evaluate(left_node), self.evaluate(right_node)
        if type(op) not in _FOLD:
            self.fail(node, f"unsupported numeric operator: {type(op).__name__}")
        if not isinstance(left, Value) and not isinstance(right, Value):
            return self.fold(node, op, left, right, comparison)
        self.runtime_arithmetic(node)
        dtype = (left if isinstance(left, Value) else right).dtype
        if not isinstance(dtype, ScalarType) or (dtype == bool_ and type(op) not in (ast.Eq, ast.NotEq)):
            self.fail(node, "numeric expressions require compatible scalar types")
        left, right = self.as_type(left, dtype, node), self.as_type(right, dtype, node)
        floating = dtype in (f32, f64)
        if comparison:
            predicate = (_CMPF if floating else _CMPI)[type(op)]
            return self.value("arith.cmpf" if floating else "arith.cmpi", bool_, node, operands=[left, right],
                              attrs=[("predicate", f"{predicate} : i64")])
        if isinstance(op, ast.Div) and not floating:
            self.fail(node, "division requires floating operands")
        suffix = "f" if floating else "i"
        return self.value(f"arith.{_ARITH[type(op)]}{suffix}", dtype, node, operands=[left, right])

    def fold(self, node, op, left, right, comparison):
        allowed = (int, float, bool) if comparison else (int, float)
        if type(left) not in allowed or type(right) not in allowed:
            self.fail(node, "numeric expressions require scalar operands")
        try:
            result = _FOLD[type(op)](left, right)
        except (ZeroDivisionError, OverflowError) as error:
            self.fail(node, f"invalid constant expression: {error}")
        if type(result) is float and not math.isfinite(result):
            self.fail(node, "non-finite constant expression")
        return result

    def expr_Call(self, node):
        callee = self.evaluate(node.func)
        if isinstance(callee, Definition):
            return self.call_definition(node, callee)
        if not isinstance(callee, Intrinsic):
            self.fail(node, "calling arbitrary Python functions is unsupported")
        if any(isinstance(a, ast.Starred) for a in node.args) or any(k.arg is None for k in node.keywords):
            self.fail(node, "argument expansion is unsupported")
        if callee.name == "launch":
            return self.intrinsic_launch(node)
        args = [self.evaluate(a) for a in node.args]
        keywords = {k.arg: self.evaluate(k.value) for k in node.keywords}
        if len(keywords) != len(node.keywords):
            self.fail(node, "duplicate keyword arguments")
        method = self.INTRINSICS.get(callee.name) or self.misplaced_intrinsic(callee.name)
        if method is None:
            self.fail(node, f"unsupported intrinsic: {callee.name}")
        return getattr(self, method)(node, callee.name, args, keywords)

    def misplaced_intrinsic(self, name):
        """Name of the method reporting intrinsics this kind of definition does not support."""
        return None

    def intrinsic_launch(self, node):
        self.fail(node, "kernels cannot launch other kernels")

    def intrinsic_cdiv(self, node, name, args, keywords):
        if len(args) != 2 or keywords or any(type(v) is not int for v in args) or args[0] < 0 or args[1] <= 0:
            self.fail(node, "cdiv requires a nonnegative constant extent and positive constant divisor")
        return -(-args[0] // args[1])

    def intrinsic_cast(self, node, name, args, keywords):
        if len(args) != 2 or keywords or not isinstance(args[1], ScalarType):
            self.fail(node, "use cast(value, scalar_type)")
        value, dtype = args
        if not isinstance(value, Value):
            if dtype in (i32, i64, index) and type(value) is float and math.isfinite(value):
                value = int(value)
            return constant(value, dtype, self.definition, node)
        self.runtime_arithmetic(node)
        source = value.dtype
        if source == dtype:
            return value
        if not isinstance(source, ScalarType) or bool_ in (source, dtype):
            self.fail(node, "boolean/buffer casts are unsupported")
        kinds = (source.category, dtype.category)
        if kinds not in _CASTS:
            self.fail(node, "cast through an integer type to convert between index and float")
        operation = _CASTS[kinds]
        if operation is None:       # same category, different width
            wider = dtype.bits > source.bits
            operation = ("extf" if wider else "truncf") if kinds[0] == "float" else ("extsi" if wider else "trunci")
        return self.value(f"arith.{operation}", dtype, node, operands=[value])

    # ---------------------------------------------------------------- statements
    def statements(self, nodes, *, top=False):
        for position, node in enumerate(nodes):
            handler = getattr(self, "stmt_" + type(node).__name__, None)
            if handler is None:
                self.fail(node, f"unsupported statement: {type(node).__name__}")
            handler(node, position == len(nodes) - 1, position == 0 and top, top)

    def stmt_Pass(self, node, last, first, top):
        pass

    def stmt_Return(self, node, last, first, top):
        self.statement_return(node, last, top)

    def stmt_Expr(self, node, last, first, top):
        if first and isinstance(node.value, ast.Constant) and isinstance(node.value.value, str):
            return                                     # docstring
        if not isinstance(node.value, ast.Call) or self.evaluate(node.value) is not None:
            self.fail(node, "expression statements must be kernel launches")

    def stmt_Assign(self, node, last, first, top):
        if len(node.targets) != 1:
            self.fail(node, "chained assignment is unsupported")
        target = node.targets[0]
        value = self.evaluate(node.value)
        if isinstance(target, ast.Name):
            self.bind_name(target, value, node)
        elif isinstance(target, ast.Subscript):
            self.store(target, value, node)
        elif isinstance(target, ast.Tuple) and all(isinstance(t, ast.Name) for t in target.elts):
            # Destructuring of a compile-time tuple (a shape, or the buffers a block returns).
            if type(value) is not tuple or len(value) != len(target.elts):
                self.fail(target, "tuple assignment requires a tuple of the same length")
            for name, item in zip(target.elts, value):
                self.bind_name(name, item, node)
        else:
            self.fail(target, "assignment requires a local name or indexed buffer element")

    def bind_name(self, target: ast.Name, value, node):
        if value is None:
            self.fail(node, "launches do not return source values")
        if self.deferred is not None and target.id in self.deferred:
            self.fail(target, "runtime branch results are deferred; write buffers or use branch-local variables")
        previous = self.scope.get(target.id)
        if _scalar(previous):
            value = self.as_type(value, previous.dtype, node.value)
        self.scope[target.id] = value

    def stmt_If(self, node, last, first, top):
        predicate = self.evaluate(node.test)
        if type(predicate) is bool:
            self.statements(node.body if predicate else node.orelse)
        else:
            self.runtime_if(node, predicate)

    def stmt_For(self, node, last, first, top):
        if node.orelse or not isinstance(node.target, ast.Name) or not isinstance(node.iter, ast.Call):
            self.fail(node, "for requires a simple induction variable and range without else")
        callee = self.evaluate(node.iter.func)
        if not isinstance(callee, Intrinsic) or callee.name != "range" or node.iter.keywords:
            self.fail(node, "for requires range(start, stop, positive_constant_step)")
        bounds = [self.evaluate(a) for a in node.iter.args]
        if not 1 <= len(bounds) <= 3:
            self.fail(node, "range requires one to three bounds")
        start, stop, step = (0, bounds[0], 1) if len(bounds) == 1 else (bounds[0], bounds[1], (bounds[2:] or [1])[0])
        if type(step) is not int or step <= 0:
            self.fail(node, "range step must be a positive compile-time integer")
        self.loop(node, start, stop, step)


# ---------------------------------------------------------------------------- kernels
class KernelLowering(Lowering):
    """A device body: runtime arithmetic, element loads and stores, structured control flow."""

    INTRINSICS = dict(Lowering.INTRINSICS, exp="intrinsic_math", rsqrt="intrinsic_math", select="intrinsic_select",
                      **{name: "intrinsic_coordinate" for name in _COORDINATES})

    def misplaced_intrinsic(self, name):
        return {"empty": "intrinsic_host_only", "empty_like": "intrinsic_host_only",
                "subview": "intrinsic_host_only"}.get(name)

    def function(self, symbol: str) -> Function:
        block = Block(args=[Value(p.dtype) for p in self.signature.runtime])
        fn = Function(symbol, block, True, self.where(self.definition.tree))
        self.module.functions.append(fn)
        self.scope.update((p.name, arg) for p, arg in zip(self.signature.runtime, block.args))
        self.block = block
        self.statements(self.definition.tree.body, top=True)
        self.op("func.return", self.definition.tree)
        return fn

    def load(self, buffer, node):
        return self.value("ckl.load_element", buffer.dtype.dtype, node, operands=[buffer, *self.element_indices(buffer, node)])

    def store(self, target, value, node):
        buffer = self.evaluate(target.value)
        if not _buffer(buffer):
            self.fail(target.value, "expected a typed buffer")
        indices = self.element_indices(buffer, target)
        stored = self.as_type(value, buffer.dtype.dtype, node.value)
        self.op("ckl.store_element", node, operands=[stored, buffer, *indices])

    def region(self, body, outer: dict, args=()) -> Block:
        """Lower `body` into a new region block with the names of `outer` frozen for rebinding."""
        block, parent, deferred = Block(args=list(args)), self.block, self.deferred
        self.block, self.deferred = block, set(outer)
        try:
            self.statements(body)
        finally:
            self.block, self.deferred = parent, deferred
        return block

    def runtime_if(self, node, predicate):
        if not (isinstance(predicate, Value) and predicate.dtype == bool_):
            self.fail(node.test, "if requires a boolean predicate; program control flow must be compile-time")
        outer = dict(self.scope)
        then_block, else_block = Block(), Block() if node.orelse else None
        self.op("scf.if", node, operands=[predicate], regions=[then_block, else_block])
        for block, body in ((then_block, node.body), (else_block, node.orelse)):
            if block is None:
                continue
            self.scope = dict(outer)
            parent, deferred = self.block, self.deferred
            self.block, self.deferred = block, set(outer)
            try:
                self.statements(body)
                self.op("scf.yield", node)
            finally:
                self.block, self.deferred = parent, deferred
        self.scope = outer

    def loop(self, node, start, stop, step):
        induction = node.target.id
        outer = dict(self.scope)
        written = {n.id for s in node.body for n in ast.walk(s) if isinstance(n, ast.Name) and isinstance(n.ctx, ast.Store)}
        if induction in written:
            self.fail(node, "cannot assign to the loop induction variable")
        carried = sorted(written & outer.keys())
        initial = []
        for name in carried:
            if self.deferred is not None and name in self.deferred:
                self.fail(node, "runtime branch results are deferred")
            value = outer[name]
            if not isinstance(value, Value):
                value = self.as_type(value, f32 if type(value) is float else i32 if type(value) is int else bool_, node)
            if not isinstance(value.dtype, ScalarType):
                self.fail(node, "loop-carried locals must be scalars")
            initial.append(value)
        bounds = [self.as_type(v, index, node) for v in (start, stop, step)]
        body = Block(args=[Value(index)] + [Value(v.dtype) for v in initial])
        loop = self.op("scf.for", node, operands=[*bounds, *initial], results=[v.dtype for v in initial], regions=[body])
        self.scope[induction] = body.args[0]
        self.scope.update(zip(carried, body.args[1:]))
        parent = self.block
        self.block = body
        self.statements(node.body)
        yielded = [self.as_type(self.scope[name], v.dtype, node) for name, v in zip(carried, initial)]
        self.op("scf.yield", node, operands=yielded)
        self.block = parent
        self.scope = outer
        self.scope.update(zip(carried, loop.results))

    def intrinsic_coordinate(self, node, name, args, keywords):
        if len(args) != 1 or keywords or type(args[0]) is not int or not 0 <= args[0] <= 2:
            self.fail(node, "device coordinates require one constant axis 0, 1, or 2")
        return self.value(f"ckl.{name}", index, node, attrs=[("axis", f"{args[0]} : i32")])

    def intrinsic_math(self, node, name, args, keywords):
        if len(args) != 1 or keywords or not isinstance(args[0], Value) or args[0].dtype not in (f32, f64):
            self.fail(node, f"{name} requires one typed floating-point scalar")
        return self.value(f"math.{name}", args[0].dtype, node, operands=[args[0]])

    def intrinsic_select(self, node, name, args, keywords):
        if len(args) != 3 or keywords:
            self.fail(node, "use select(predicate, true_value, false_value)")
        condition = self.as_type(args[0], bool_, node)
        typed = next((v for v in args[1:] if isinstance(v, Value)), None)
        if not _scalar(typed):
            self.fail(node, "select requires a typed scalar alternative")
        first, second = (self.as_type(v, typed.dtype, node) for v in args[1:])
        return self.value("arith.select", first.dtype, node, operands=[condition, first, second])

    def intrinsic_host_only(self, node, name, args, keywords):
        if name == "subview":
            self.fail(node, "subview is currently supported only in programs")
        self.fail(node, "program temporaries cannot be allocated inside kernels")


# ---------------------------------------------------------------------------- programs and blocks
class ProgramLowering(Lowering):
    """A host composition, evaluated while lowering: allocations, subviews and dispatches."""

    INTRINSICS = dict(Lowering.INTRINSICS, empty="intrinsic_empty", empty_like="intrinsic_empty",
                      subview="intrinsic_subview")
    HOST_ONLY_MESSAGE = "computed runtime host scalars are unsupported; forward the parameter unchanged"

    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        self.returned = None

    def misplaced_intrinsic(self, name):
        if name in _COORDINATES:
            return "intrinsic_device_only"
        if name in ("exp", "rsqrt", "select"):
            return "intrinsic_device_arithmetic"
        return None

    def function(self, symbol: str) -> Function:
        block = Block(args=[Value(p.dtype) for p in self.signature.runtime])
        fn = Function(symbol, block, False, self.where(self.definition.tree))
        self.module.functions.append(fn)
        self.scope.update((p.name, arg) for p, arg in zip(self.signature.runtime, block.args))
        self.block = block
        self.statements(self.definition.tree.body, top=True)
        for temporary in reversed(self.temporaries):
            self.op("ckl.free", self.definition.tree, operands=[temporary])
        self.op("func.return", self.definition.tree)
        return fn

    def runtime_arithmetic(self, node):
        self.fail(node, self.HOST_ONLY_MESSAGE)

    def loop(self, node, start, stop, step):
        if type(start) is not int or type(stop) is not int:
            self.fail(node, "program range bounds must be compile-time integers")
        if len(range(start, stop, step)) > 1024:
            self.fail(node, "program unrolling is limited to 1024 iterations")
        induction = node.target.id
        missing = object()
        saved = self.scope.get(induction, missing)
        for value in range(start, stop, step):
            self.scope[induction] = value
            self.statements(node.body)
        if saved is missing:
            self.scope.pop(induction, None)
        else:
            self.scope[induction] = saved

    def intrinsic_device_only(self, node, name, args, keywords):
        self.fail(node, "device coordinates are only valid in kernels")

    def intrinsic_device_arithmetic(self, node, name, args, keywords):
        self.runtime_arithmetic(node)

    def intrinsic_empty(self, node, name, args, keywords):
        if name == "empty_like":
            if len(args) != 1 or keywords or not _buffer(args[0]):
                self.fail(node, "empty_like requires one buffer")
            spec = args[0].dtype
        else:
            if len(args) != 1 or set(keywords) != {"dtype"}:
                self.fail(node, "use empty(shape_tuple, dtype=element_type)")
            try:
                spec = BufferSpec(args[0], keywords["dtype"])
            except (TypeError, ValueError) as error:
                self.fail(node, str(error))
        allocation = self.value("ckl.alloc", spec, node)
        self.temporaries.append(allocation)
        return allocation

    def intrinsic_subview(self, node, name, args, keywords):
        if len(args) != 1 or set(keywords) != {"offset", "shape"} or not _buffer(args[0]):
            self.fail(node, "use subview(buffer, offset=element_offset, shape=shape_tuple)")
        source, offset = args[0], keywords["offset"]
        try:
            spec = BufferSpec(keywords["shape"], source.dtype.dtype)
        except (TypeError, ValueError) as error:
            self.fail(node, str(error))
        if type(offset) is not int or not 0 <= offset < (1 << 63) or offset + spec.elements > source.dtype.elements:
            self.fail(node, "subview offset/shape must be constant and within the source")
        return self.value("ckl.subview", spec, node, operands=[source], attrs=[("offset", f"{offset} : i64")])

    def geometry(self, node, keywords, key):
        dims = keywords[key]
        if type(dims) is not tuple or not 1 <= len(dims) <= 3 or \
                any(type(d) is not int or not 0 < d < (1 << 63) for d in dims):
            self.fail(node, f"{key} requires a tuple of one to three positive compile-time integers")
        return dims + (1,) * (3 - len(dims))

    def intrinsic_launch(self, node):
        if not node.args:
            self.fail(node, "launch requires a kernel definition")
        kernel = self.evaluate(node.args[0])
        if not isinstance(kernel, Definition) or kernel.kind != "kernel":
            self.fail(node, "launch requires a @ckl.kernel definition")
        parameters = kernel.tree.args.args
        if len(node.args) - 1 != len(parameters):
            self.fail(node, "launch argument count does not match kernel signature")
        keywords = {k.arg: self.evaluate(k.value) for k in node.keywords}
        if set(keywords) - {"grid", "block", "shared_memory"} or not {"grid", "block"} <= set(keywords):
            self.fail(node, "launch requires grid and block; only shared_memory is optional")
        grid, block = self.geometry(node, keywords, "grid"), self.geometry(node, keywords, "block")
        shared = keywords.get("shared_memory", 0)
        if type(shared) is not int or not 0 <= shared < (1 << 63):
            self.fail(node, "shared_memory requires nonnegative compile-time bytes")
        runtime, constants, operands = {}, {}, []
        for parameter, argument in zip(parameters, node.args[1:]):
            captured = kernel.annotations.get(parameter.arg)
            if (captured is None or isinstance(captured, str)) and parameter.annotation is None:
                self.fail(node, "kernel parameters require annotations")
            annotation = annotation_of(kernel, parameter)
            actual = self.evaluate(argument)
            if isinstance(annotation, ConstexprType):
                if isinstance(actual, Value):
                    self.fail(argument, "constexpr launch arguments must be compile-time constants")
                constants[parameter.arg] = actual
                continue
            if isinstance(annotation, ScalarType):
                actual = self.as_type(actual, annotation, argument)
            if not isinstance(actual, Value):
                self.fail(argument, "kernel arguments must be typed buffers or scalars")
            runtime[parameter.arg] = actual.dtype
            operands.append(actual)
        spec = self.module.specialize(kernel, bind(kernel, runtime, constants))
        self.module.extents.setdefault(spec.symbol, set()).add(tuple(g * b for g, b in zip(grid, block)))
        attrs = [("kernel", f"@{spec.symbol}"), ("grid", dense(grid)), ("block", dense(block)),
                 ("shared_memory", f"{shared} : i64"), ("device", quote("unassigned:0")), ("capabilities", "[]"),
                 ("implementation", quote(spec.identity)), ("operandSegmentSizes", dense([len(operands), 0], 32))]
        # Dependencies come from the kernels' effects, not from completion tokens.
        self.value("ckl.dispatch", TOKEN, node, operands=operands, attrs=attrs)

    # ---------------------------------------------------------------- blocks
    def call_definition(self, node, callee):
        if callee.kind != "block":
            self.fail(node, "kernel definitions are not ordinary calls; use ckl.launch")
        if node.keywords or any(isinstance(a, ast.Starred) for a in node.args):
            self.fail(node, "blocks take positional arguments only")
        parameters = callee.tree.args.args
        if len(node.args) != len(parameters):
            self.fail(node, "block argument count does not match its signature")
        runtime, constants, values = {}, {}, {}
        for parameter, argument in zip(parameters, node.args):
            actual = self.evaluate(argument)
            annotation = annotation_of(callee, parameter)
            if isinstance(annotation, ConstexprType):
                if isinstance(actual, Value):
                    self.fail(argument, "constexpr block arguments must be compile-time constants")
                constants[parameter.arg] = actual
            elif isinstance(actual, Value):
                runtime[parameter.arg] = actual.dtype
                values[parameter.arg] = actual
            else:
                self.fail(argument, "block arguments must be buffers, program scalars or compile-time constants")
        bound = bind(callee, runtime, constants)
        scope = {p.name: (p.value if p.is_constant else values[p.name]) for p in bound.parameters}
        inner = ProgramLowering(self.module, callee, bound, scope=scope, temporaries=self.temporaries)
        inner.block = self.block
        inner.statements(callee.tree.body, top=True)
        return inner.returned

    def statement_return(self, node, last, top):
        if self.definition.kind != "block":
            return super().statement_return(node, last, top)
        if not top or not last:
            self.fail(node, "a block returns only from the end of its body")
        self.returned = None if node.value is None else self.evaluate(node.value)


# ---------------------------------------------------------------------------- entry points
def lower_program(definition: Definition, signature, constants, *, verify=False) -> LoweredProgram:
    """Lower a program and every kernel it launches; returns the IR text and specializations."""
    bound = bind(definition, signature, constants)
    program_identity = identity(definition, bound)
    module = Module()
    ProgramLowering(module, definition, bound).function("program_" + program_identity[:24])
    text = print_module(module.functions, locations=True)
    semantic = print_module(module.functions, locations=False)
    key = hashlib.sha256((program_identity + semantic).encode()).hexdigest()
    entries = list(module.specializations.values())
    specs = tuple(spec for spec, _ in entries)
    canonical = tuple(canonical_kernel(fn) for _, fn in entries)
    extents = tuple(tuple(sorted(module.extents.get(spec.symbol, ()))) for spec in specs)
    result = LoweredProgram(text, bound, specs, key, (), canonical, extents)
    return result.verify() if verify else result


def canonical_kernel(fn: Function) -> str:
    """Kernel text without its symbol or locations: equal bodies print equal text."""
    return print_function(Function("kernel", fn.block, fn.kernel, ""), locations=False)


def lower_kernel(definition: Definition, signature: BoundSignature) -> str:
    """Canonical text of `definition` specialized for a bound signature (library matching)."""
    module = Module()
    spec = module.specialize(definition, signature)
    return canonical_kernel(module.specializations[spec.identity][1])
