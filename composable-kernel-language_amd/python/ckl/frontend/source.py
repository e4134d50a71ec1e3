"""Capture of CKL definitions from Python source, without running them.

`@ckl.kernel`, `@ckl.program` and `@ckl.block` read the decorated function's source text and
parse it; the body is never executed. Every name the body or its annotations use is looked up
once, in the function's globals and closure, and classified: compile-time constants (ints,
floats, bools, strings, None and tuples of them), CKL types and dimensions, other definitions,
intrinsics, the `ckl` module and modules of CKL definitions are kept; anything else is recorded
as unsupported and
reported only if the body actually evaluates it. A definition's identity is a SHA-256 over its
syntax tree and those captured values, so edits to a kernel or to a constant it reads change it.

Behaviour, including the wording and `file:line:col` form of diagnostics, follows the
reference's python/ckl/frontend/source.py:17-236. `@ckl.block` has no counterpart there: it
marks a program fragment that programs call like a function and that the frontend expands in
place.
"""
from __future__ import annotations

import ast
import hashlib
import inspect
import json
import textwrap
from types import MappingProxyType, ModuleType

from ..types import Buffer, BufferType, ConstexprType, Dimension, ScalarType, constexpr

KINDS = ("kernel", "program", "block")


class FrontendError(ValueError):
    """A diagnostic: `file:line:col: message`, the offending source line and a caret."""


class Intrinsic:
    """A `ckl.<name>` operation; it exists only inside CKL source."""

    __slots__ = ("name",)

    def __init__(self, name: str):
        object.__setattr__(self, "name", name)

    def __setattr__(self, key, value):
        raise AttributeError("intrinsics are immutable")

    def __eq__(self, other):
        return isinstance(other, Intrinsic) and other.name == self.name

    def __hash__(self):
        return hash(("Intrinsic", self.name))

    def __repr__(self) -> str:
        return f"ckl.{self.name}"

    def __call__(self, *args, **kwargs):
        raise FrontendError(f"ckl.{self.name} is only valid inside a CKL source definition")


_INTRINSIC_NAMES = ("global_id", "thread_id", "block_id", "block_dim", "grid_dim", "launch", "empty_like", "empty",
                    "cdiv", "cast", "exp", "rsqrt", "select", "subview")
INTRINSICS = {name: Intrinsic(name) for name in _INTRINSIC_NAMES}
RANGE = Intrinsic("range")


class Namespace:
    """A module as a definition sees it (`ckl`, or a module of kernels): its CKL members."""

    def __init__(self, values):
        self.values = MappingProxyType(dict(values))


class UnsupportedBinding:
    """A captured name whose value CKL cannot use (reported when the body reads it)."""

    def __init__(self, name: str):
        self.name = name


# ---------------------------------------------------------------------------------- capture
def _is_constant(value) -> bool:
    if type(value) is tuple:
        return all(_is_constant(item) for item in value)
    return value is None or type(value) in (int, float, bool, str)


def _is_ckl_value(value) -> bool:
    return (isinstance(value, (ScalarType, BufferType, ConstexprType, Dimension, Definition, Intrinsic))
            or value is Buffer or value is constexpr)


def _module_namespace(module: ModuleType) -> Namespace:
    """The `ckl` module exposes its scalar types, intrinsics and annotation syntax; any other
    module exposes the CKL values and constants it defines (kernels, blocks, dimensions, types),
    so `module.kernel_name` works in launches."""
    exported = {}
    for key, item in vars(module).items():
        if key.startswith("__"):
            continue
        if isinstance(item, (ScalarType, Intrinsic)) or item is Buffer or item is constexpr:
            exported[key] = item
        elif module.__name__ != "ckl" and (_is_ckl_value(item) or _is_constant(item)):
            exported[key] = item
    return Namespace(exported)


def classify(name: str, value):
    """What a definition keeps for the Python value `value` bound to `name`."""
    if value is range:
        return RANGE
    if _is_constant(value) or _is_ckl_value(value):
        return value
    if isinstance(value, ModuleType):
        return _module_namespace(value)
    return UnsupportedBinding(name)


def fingerprint(value):
    """A JSON-serialisable description of a captured value, for identities."""
    if isinstance(value, Definition):
        return ["definition", value.identity]
    if isinstance(value, Namespace):
        return ["namespace", sorted([key, fingerprint(item)] for key, item in value.values.items())]
    if value is Buffer or value is constexpr:
        return ["type_constructor", value.__name__]
    if isinstance(value, (ScalarType, Dimension, Intrinsic, UnsupportedBinding)):
        return [type(value).__name__, value.name]
    if isinstance(value, BufferType):
        return ["BufferType", fingerprint(value.dtype), fingerprint(value.shape)]
    if isinstance(value, ConstexprType):
        return ["ConstexprType", fingerprint(value.dtype)]
    if type(value) is tuple:
        return ["tuple", [fingerprint(item) for item in value]]
    return [type(value).__name__, repr(value)]


def _names_in(node: ast.AST) -> set:
    return {n.id for n in ast.walk(node) if isinstance(n, ast.Name)}


class Definition:
    """A captured kernel, program or block: its syntax tree, where it came from, the values of
    the names it reads and its identity."""

    def __init__(self, kind, name, tree, source, filename, first_line, indentation, bindings, annotations, identity):
        self.kind, self.name, self.tree, self.source = kind, name, tree, source
        self.filename, self.first_line, self.indentation = filename, first_line, indentation
        self.bindings, self.annotations, self.identity = bindings, annotations, identity

    def __repr__(self) -> str:
        return f"<ckl.{self.kind} {self.name}>"

    def error(self, node: ast.AST, message: str) -> FrontendError:
        """A FrontendError pointing at `node` in this definition's file."""
        row = getattr(node, "lineno", 1)
        column = getattr(node, "col_offset", 0)
        lines = self.source.splitlines()
        text = lines[row - 1] if 0 < row <= len(lines) else ""
        where = f"{self.filename}:{self.first_line + row - 1}:{self.indentation + column + 1}"
        return FrontendError(f"{where}: {message}\n{text}\n{' ' * column}^")

    def __call__(self, *args, **kwargs):
        if self.kind == "kernel":
            hint = "use ckl.launch inside a program"
        elif self.kind == "block":
            hint = "call blocks from a program body"
        else:
            hint = "use .lower(signature=...)"
        raise self.error(self.tree, f"CKL {self.kind} bodies are not Python callables; {hint}")

    def lower(self, *, signature, constants=None, verify=False):
        """Specialise this program for `signature` (argument name -> BufferSpec or scalar type)
        and `constants` (constexpr name -> value) and lower it to CKL IR."""
        if self.kind != "program":
            raise self.error(self.tree, "lower a @ckl.program entry point")
        from .emitter import lower_program
        return lower_program(self, signature, dict(constants or {}), verify=verify)


def capture(function, kind: str) -> Definition:
    if kind not in KINDS:
        raise ValueError(f"unknown definition kind {kind!r}")
    try:
        lines, first_line = inspect.getsourcelines(function)
        filename = inspect.getsourcefile(function) or "<unknown>"
    except (OSError, TypeError) as error:
        raise FrontendError("CKL definitions require retrievable source in a Python file") from error
    source = textwrap.dedent("".join(lines))
    tree = next((node for node in ast.parse(source).body if isinstance(node, ast.FunctionDef)), None)
    if tree is None:
        raise FrontendError("CKL requires a synchronous function definition")

    scope = {"range": range, **function.__globals__, **inspect.getclosurevars(function).nonlocals}
    used = _names_in(tree)
    for annotation in function.__annotations__.values():
        if isinstance(annotation, str):
            used |= _names_in(ast.parse(annotation, mode="eval"))
    bindings = {name: classify(name, scope[name]) for name in sorted(used) if name in scope}
    annotations = {name: value if isinstance(value, str) else classify(name, value)
                   for name, value in function.__annotations__.items()}

    digest = hashlib.sha256()
    for part in ("ckl.definition/2", kind, ast.dump(tree, include_attributes=False),
                 json.dumps([[name, fingerprint(value)] for name, value in bindings.items()]),
                 json.dumps([[name, fingerprint(value)] for name, value in sorted(annotations.items())])):
        digest.update(part.encode())
        digest.update(b"\0")
    indentation = len(lines[0]) - len(lines[0].lstrip())
    return Definition(kind, function.__name__, tree, source, filename, first_line, indentation,
                      MappingProxyType(bindings), MappingProxyType(annotations), digest.hexdigest())


def kernel(function) -> Definition:
    """`@ckl.kernel`: a device body launched by programs over a grid of threads."""
    return capture(function, "kernel")


def program(function) -> Definition:
    """`@ckl.program`: a host composition of temporaries and launches, lowered per signature."""
    return capture(function, "program")


def block(function) -> Definition:
    """`@ckl.block`: a program fragment, expanded in place where a program (or another block)
    calls it; it may allocate temporaries, launch kernels and return buffers."""
    return capture(function, "block")
