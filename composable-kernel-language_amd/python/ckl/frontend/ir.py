"""In-memory CKL IR (SSA values, operations with attributes and regions, functions) and its
printer. The text is MLIR's generic operation syntax, which the native compiler
(csrc/core/ir.cpp) parses; MLIR itself is not needed.
"""
from __future__ import annotations

from dataclasses import dataclass, field

from ..types import TOKEN, BufferSpec, bool_


class Value:
    """An SSA value: a function or region argument, or an operation result."""

    __slots__ = ("dtype",)

    def __init__(self, dtype):
        self.dtype = dtype


@dataclass(eq=False)
class Op:
    name: str
    operands: list
    results: list
    attrs: list                                    # (key, printed value or None) pairs
    regions: list = field(default_factory=list)   # one Block, or None for an empty region, each
    loc: str = ""


@dataclass(eq=False)
class Block:
    args: list = field(default_factory=list)
    ops: list = field(default_factory=list)


@dataclass
class Function:
    symbol: str
    block: Block
    kernel: bool
    loc: str


def type_text(dtype) -> str:
    if isinstance(dtype, BufferSpec):
        return dtype.mlir
    if dtype == TOKEN:
        return "!ckl.token"
    return dtype.mlir


def quote(text: str) -> str:
    """An MLIR string literal: quotes, backslashes and non-printable bytes escaped as \\XX."""
    pieces = []
    for ch in text:
        if ch == '"':
            pieces.append("\\22")
        elif ch == "\\":
            pieces.append("\\\\")
        elif 0x20 <= ord(ch) < 0x7F:
            pieces.append(ch)
        else:
            pieces.extend(f"\\{byte:02X}" for byte in ch.encode())
    return '"' + "".join(pieces) + '"'


def int_attr(value: int, dtype) -> str:
    if dtype == bool_:
        return "true" if value else "false"
    return f"{int(value)} : {dtype.mlir}"


def float_attr(value: float, dtype) -> str:
    text = repr(float(value))
    if not any(marker in text for marker in (".", "e", "inf", "nan")):
        text += ".0"
    return f"{text} : {dtype.mlir}"


def dense(values, width: int = 64) -> str:
    items = [str(int(v)) for v in values]
    return f"array<i{width}" + (": " + ", ".join(items) if items else "") + ">"


class Printer:
    """Names values in print order (%argN for arguments, %N for results)."""

    def __init__(self, locations: bool):
        self.locations = locations
        self.names = {}
        self.results = 0
        self.arguments = 0

    def name(self, value: Value) -> str:
        return self.names[value]

    def define(self, value: Value, argument: bool) -> str:
        if argument:
            text, self.arguments = f"%arg{self.arguments}", self.arguments + 1
        else:
            text, self.results = f"%{self.results}", self.results + 1
        self.names[value] = text
        return text

    def region(self, block, indent: int) -> str:
        pad = "  " * indent
        lines = []
        if block is not None:
            if block.args:
                args = ", ".join(f"{self.define(a, True)}: {type_text(a.dtype)}" for a in block.args)
                lines.append(f"{pad}  ^bb0({args}):")
            for child in block.ops:
                self.op(child, indent + 2, lines)
        return "{\n" + "".join(line + "\n" for line in lines) + pad + "}"

    def op(self, op: Op, indent: int, lines: list) -> None:
        pad = "  " * indent
        results = ", ".join(self.define(r, False) for r in op.results)
        text = f"{pad}{results + ' = ' if results else ''}{quote(op.name)}("
        text += ", ".join(self.name(v) for v in op.operands) + ")"
        if op.regions:
            text += " (" + ", ".join(self.region(r, indent) for r in op.regions) + ")"
        if op.attrs:
            text += " {" + ", ".join(k if v is None else f"{k} = {v}" for k, v in sorted(op.attrs)) + "}"
        text += " : (" + ", ".join(type_text(v.dtype) for v in op.operands) + ") -> "
        if len(op.results) == 1:
            text += type_text(op.results[0].dtype)
        else:
            text += "(" + ", ".join(type_text(r.dtype) for r in op.results) + ")"
        if self.locations and op.loc:
            text += f" loc({op.loc})"
        lines.append(text)

    def function(self, fn: Function, lines: list) -> None:
        args = ", ".join(f"{self.define(a, True)}: {type_text(a.dtype)}" for a in fn.block.args)
        attributes = " attributes {ckl.kernel}" if fn.kernel else ""
        lines.append(f"  func.func @{fn.symbol}({args}){attributes} {{")
        for op in fn.block.ops:
            self.op(op, 2, lines)
        lines.append(f"  }} loc({fn.loc})" if self.locations and fn.loc else "  }")


def print_module(functions: list, locations: bool) -> str:
    lines = ["module {"]
    for fn in functions:
        Printer(locations).function(fn, lines)
    lines.append("}")
    return "\n".join(lines) + "\n"


def print_function(fn: Function, locations: bool = False) -> str:
    lines = []
    Printer(locations).function(fn, lines)
    return "\n".join(lines) + "\n"
