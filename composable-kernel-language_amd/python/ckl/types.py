"""The type vocabulary of CKL source: element types, symbolic dimensions, buffer and constexpr
annotations, and the concrete buffer specifications a program is specialised for.

The public names (`f32`, `f64`, `i32`, `i64`, `index`, `bool`, `dim`, `Buffer[...]`,
`constexpr[...]`, `BufferSpec`) and the rules they enforce are those of the reference's
python/ckl/types.py:7-90; the diagnostics keep its wording. Every object here is immutable and
compares by value, so specialisations can be keyed and hashed by them.
"""
from __future__ import annotations

import math


class _Frozen:
    """Value objects: attributes are set once in __init__ and compared as a tuple."""

    __slots__ = ()

    def _fields(self) -> tuple:
        return tuple(getattr(self, name) for name in self.__slots__)

    def _set(self, **values) -> None:
        for name, value in values.items():
            object.__setattr__(self, name, value)

    def __setattr__(self, name, value):
        raise AttributeError(f"{type(self).__name__} objects are immutable")

    def __eq__(self, other):
        return type(other) is type(self) and other._fields() == self._fields()

    def __hash__(self):
        return hash((type(self).__name__, self._fields()))


class ScalarType(_Frozen):
    """An element or scalar type: its CKL name, its width in bits and its category
    ("float", "signed", "index", "predicate", or "opaque" for IR-only types)."""

    __slots__ = ("name", "bits", "category")

    def __init__(self, name: str, bits: int = 0, category: str = "opaque"):
        self._set(name=name, bits=bits, category=category)

    def _fields(self) -> tuple:
        return (self.name,)

    def __repr__(self) -> str:
        return f"ckl.{self.name}"

    @property
    def mlir(self) -> str:
        """Spelling in the IR: the name itself, except the one-bit predicate `i1`."""
        return "i1" if self.category == "predicate" else self.name

    @property
    def is_float(self) -> bool:
        return self.category == "float"

    @property
    def is_integer(self) -> bool:
        return self.category == "signed"


f32 = ScalarType("f32", 32, "float")
f64 = ScalarType("f64", 64, "float")
i32 = ScalarType("i32", 32, "signed")
i64 = ScalarType("i64", 64, "signed")
index = ScalarType("index", 64, "index")
bool_ = ScalarType("bool", 1, "predicate")
NUMERIC_TYPES = (f32, f64, i32, i64)
SCALAR_TYPES = NUMERIC_TYPES + (index, bool_)
TOKEN = ScalarType("!ckl.token")      # completion token of a dispatch (IR only)


class Dimension(_Frozen):
    """A named extent, bound to a concrete size when a definition is specialised."""

    __slots__ = ("name",)

    def __init__(self, name: str):
        if not (isinstance(name, str) and name.isidentifier()):
            raise ValueError("dimension names must be Python identifiers")
        self._set(name=name)

    def __repr__(self) -> str:
        return f"ckl.dim({self.name!r})"


def dim(name: str) -> Dimension:
    return Dimension(name)


_MAX_EXTENT = 1 << 63


def _is_extent(extent) -> bool:
    if isinstance(extent, Dimension):
        return True
    return type(extent) is int and 0 < extent < _MAX_EXTENT


class BufferType(_Frozen):
    """`Buffer[dtype, shape]`: element type plus a shape of positive integers and dimensions."""

    __slots__ = ("dtype", "shape")

    def __init__(self, dtype: ScalarType, shape: tuple):
        if not any(dtype == t for t in NUMERIC_TYPES):
            raise ValueError("buffer elements must be f32, f64, i32, or i64")
        if type(shape) is not tuple or not all(_is_extent(extent) for extent in shape):
            raise ValueError("buffer shapes must be tuples of positive extents within i64 or dimensions")
        self._set(dtype=dtype, shape=shape)

    def __repr__(self) -> str:
        return f"ckl.Buffer[{self.dtype!r}, {self.shape!r}]"


class ConstexprType(_Frozen):
    """`constexpr[dtype]`: a parameter bound at specialisation time, folded into the body."""

    __slots__ = ("dtype",)

    def __init__(self, dtype: ScalarType):
        if not any(dtype == t for t in SCALAR_TYPES):
            raise ValueError("constexpr requires a CKL scalar type")
        self._set(dtype=dtype)

    def __repr__(self) -> str:
        return f"ckl.constexpr[{self.dtype!r}]"


class _AnnotationSyntax:
    """`Name[...]` in annotations; the object itself is never instantiated."""

    def __init__(self, name: str, build):
        self.__name__ = name
        self._build = build

    def __getitem__(self, item):
        return self._build(item)

    def __call__(self, *args, **kwargs):
        raise TypeError(f"ckl.{self.__name__} is used as ckl.{self.__name__}[...] in annotations")

    def __repr__(self) -> str:
        return f"ckl.{self.__name__}"


def _buffer_annotation(item) -> BufferType:
    if type(item) is not tuple or len(item) != 2:
        raise ValueError("use Buffer[element_type, shape_tuple]")
    return BufferType(item[0], item[1])


Buffer = _AnnotationSyntax("Buffer", _buffer_annotation)
constexpr = _AnnotationSyntax("constexpr", ConstexprType)


class BufferSpec(_Frozen):
    """A concrete, contiguous buffer: integer shape, element type and the identity layout."""

    __slots__ = ("shape", "dtype", "layout")

    def __init__(self, shape: tuple, dtype: ScalarType, layout: str = "identity"):
        BufferType(dtype, shape)
        if not all(type(extent) is int for extent in shape):
            raise ValueError("BufferSpec requires concrete integer extents")
        if layout != "identity":
            raise ValueError("only contiguous identity-layout buffers are supported")
        self._set(shape=shape, dtype=dtype, layout=layout)

    def __repr__(self) -> str:
        return f"ckl.BufferSpec({self.shape!r}, {self.dtype!r})"

    @property
    def mlir(self) -> str:
        """The buffer's IR type, e.g. `memref<8x64xf32>`."""
        return "memref<" + "".join(f"{extent}x" for extent in self.shape) + self.dtype.mlir + ">"

    @property
    def element_bytes(self) -> int:
        return self.dtype.bits // 8

    @property
    def elements(self) -> int:
        return math.prod(self.shape)

    @property
    def nbytes(self) -> int:
        return self.elements * self.element_bytes
