"""CKL scalar types, symbolic dimensions, typed buffers and specialization descriptors.

Public names and validation rules follow python/ckl/types.py:7-90 of the reference.
"""
from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class ScalarType:
    name: str

    @property
    def mlir(self) -> str:
        return "i1" if self.name == "bool" else self.name


f32 = ScalarType("f32")
f64 = ScalarType("f64")
i32 = ScalarType("i32")
i64 = ScalarType("i64")
index = ScalarType("index")
bool_ = ScalarType("bool")
NUMERIC_TYPES = (f32, f64, i32, i64)
SCALAR_TYPES = (*NUMERIC_TYPES, index, bool_)
TOKEN = ScalarType("!ckl.token")


@dataclass(frozen=True)
class Dimension:
    name: str

    def __post_init__(self) -> None:
        if not isinstance(self.name, str) or not self.name.isidentifier():
            raise ValueError("dimension names must be Python identifiers")


def dim(name: str) -> Dimension:
    return Dimension(name)


def _valid_extent(extent) -> bool:
    return isinstance(extent, Dimension) or (type(extent) is int and 0 < extent < (1 << 63))


@dataclass(frozen=True)
class BufferType:
    dtype: ScalarType
    shape: tuple

    def __post_init__(self) -> None:
        if self.dtype not in NUMERIC_TYPES:
            raise ValueError("buffer elements must be f32, f64, i32, or i64")
        if not isinstance(self.shape, tuple) or not all(_valid_extent(d) for d in self.shape):
            raise ValueError("buffer shapes must be tuples of positive extents within i64 or dimensions")


class Buffer:
    """`Buffer[element_type, shape]` annotation constructor."""

    def __class_getitem__(cls, arguments):
        if not isinstance(arguments, tuple) or len(arguments) != 2:
            raise ValueError("use Buffer[element_type, shape_tuple]")
        return BufferType(*arguments)


@dataclass(frozen=True)
class ConstexprType:
    dtype: ScalarType

    def __post_init__(self) -> None:
        if self.dtype not in SCALAR_TYPES:
            raise ValueError("constexpr requires a CKL scalar type")


class constexpr:
    """`constexpr[scalar_type]` marks a compile-time specialization parameter."""

    def __class_getitem__(cls, dtype):
        return ConstexprType(dtype)


@dataclass(frozen=True)
class BufferSpec:
    """Concrete, contiguous (identity layout) buffer shape and element type."""

    shape: tuple
    dtype: ScalarType
    layout: str = "identity"

    def __post_init__(self) -> None:
        BufferType(self.dtype, self.shape)
        if any(type(d) is not int for d in self.shape):
            raise ValueError("BufferSpec requires concrete integer extents")
        if self.layout != "identity":
            raise ValueError("only contiguous identity-layout buffers are supported")

    @property
    def mlir(self) -> str:
        return "memref<" + "".join(f"{d}x" for d in self.shape) + self.dtype.mlir + ">"

    @property
    def element_bytes(self) -> int:
        return 8 if self.dtype in (f64, i64) else 4

    @property
    def nbytes(self) -> int:
        count = 1
        for d in self.shape:
            count *= d
        return count * self.element_bytes
