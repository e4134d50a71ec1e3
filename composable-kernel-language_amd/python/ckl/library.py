"""Selection of hand-written gfx950 kernels for CKL kernel specializations.

Each library entry names the CKL kernel body it implements (its contract, from
ckl.decoder_kernels) and how to launch its gfx950 implementation (csrc/kernels/library.hip). A
specialization uses the library kernel only when

  1. its kernel IR, printed canonically, is identical to the contract body lowered with the
     same concrete signature (same shapes, dtypes and constexpr values), and
  2. every launch of it covers exactly the thread domain the library kernel computes
     (for example `linear` must be launched over y = B rows and x >= O columns).

Otherwise the kernel is compiled from its own IR (csrc/runtime/codegen.cpp), and `explain`
says why; a kernel that carries a library kernel's name without its body draws a warning. The
dependency graph is always derived from the CKL body, never from the library kernel; the
reference allows several implementations of one kernel when their observable effects agree
(specs/mlir-layout-aware-gpu-compiler-spec.md:241).
"""
from __future__ import annotations

import warnings
from dataclasses import dataclass
from typing import Callable, Optional

from .decoder_kernels import (add, advance, append_kv, attention_scores, attention_values, embedding, greedy, linear,
                              multiply, rms_apply, rms_stats, rope, silu, softmax, update)
from .frontend.checker import BoundSignature, bind
from .frontend.emitter import lower_kernel
from .frontend.source import Definition, FrontendError
from .types import BufferSpec


# ---------------------------------------------------------------------------- launches
BLOCK = 256
VALUES_BLOCK = 512      # kValuesBlock: attention_values workgroup (one per (b, h))
GREEDY_CHUNK = 4096     # kGreedyChunk: logits per greedy workgroup
GREEDY_ROW_THREADS = 1024   # one workgroup per row of at most 8 float4 per thread (kGreedyRowLoads)


def _cdiv(a: int, b: int) -> int:
    return (a + b - 1) // b


@dataclass(frozen=True)
class Launch:
    grid: int
    constants: tuple
    block: int = BLOCK
    shared: int = 0
    entry: str = ""          # entry point when the family has several (default ckl_<name>)
    # Device workspace the compiled plan gives the kernel: `workspace` bytes of state that reads
    # zero at every launch (zero page, completion counters), and, when `partials` >= 0, a second
    # pointer to `partials` bytes of split-reduction planes (0: a null pointer) that live only
    # until the kernel's readers have run, so the plan may share them between kernels.
    workspace: int = 0
    partials: int = -1
    # (members, Launch): the launch a dispatch takes instead when at least `members` dispatches
    # of the kernel in its block multiply the same first operand (siblings the inferred graph
    # runs as one shared-operand launch); the native prepare step picks it per dispatch, so every
    # run mode launches the same tiling.
    variants: tuple = ()


def _elementwise(count: int, inner: int) -> int:
    return _cdiv(count // 4 if inner % 4 == 0 else count, BLOCK)


def _embedding(shapes, consts, ext):
    (b,), (v, c) = shapes[0], shapes[1]
    return Launch(_elementwise(b * c, c), (b, c, v)) if ext[0] >= c and ext[1:] == (b, 1) else None


def _rms_stats(shapes, consts, ext):
    b, c = shapes[0]
    return Launch(b, (b, c)) if ext[0] >= b and ext[1:] == (1, 1) else None      # one workgroup per row


def _rms_apply(shapes, consts, ext):
    (b, c), (g, _c) = shapes[0], shapes[2]
    layer = consts[4]
    if not (0 <= layer < g) or not (ext[0] >= c and ext[1:] == (b, 1)):
        return None
    return Launch(_elementwise(b * c, c), (b, c, layer))


# Tiling of the linear family (csrc/kernels/library.hip, "linear"): output tiles of 64 columns
# (vector path) or 32*J columns (f32 MFMA path, 32 batch rows per tile), reduction slices of
# k_chunk rows shared by the 4 waves of a workgroup, and k_split slices combined through the
# workspace. A B = 32 f32 GEMV costs 16 MFMA FLOP per weight byte, so the MFMA work is two thirds
# of the HBM time and has to hide under the loads. Measured inside the large decode step on
# MI355X (weights not cached), it does so only with one workgroup (one wave per SIMD) per CU:
# with two or three workgroups per CU the MFMA and load phases of the waves sharing a SIMD stop
# overlapping and a launch costs close to the sum of its MFMA-only and load-only times (gate/up
# 33.6 us at 704 workgroups; 25.0 us on 176 workgroups), and a grid just over the CU count
# doubles. So the MFMA path picks, in the order J = 2, 4, 1, the first tiling whose grid fills at
# least LINEAR_MIN_FILL of LINEAR_TARGET_GROUPS workgroups without exceeding it (splitting K into
# slices of at least LINEAR_MIN_CHUNK rows), else the fullest. Sibling linears that multiply the
# same x (q/k/v, gate/up) then run in the inferred graph as one launch of the same grid in which
# every workgroup serves all of them (ckl_linear_mfma<J>x1_shared<M>, csrc/runtime/runtime.cpp).
# The inferred graph hands the split combine to the consuming chain kernel
# (csrc/runtime/chains.cpp), so splits there cost only their partial planes. The vector path
# (B <= 16, latency-bound) runs one workgroup per (64-column tile, batch row) whose up to 16
# waves take 64 reduction rows each, all loaded in one round trip; it splits only beyond 1024
# rows.
# Three or more siblings (q/k/v) try J = 1 first: each member then contributes 2 KB to a wave's
# stage (6 KB for three), and the grid of the same size splits K into half as many slices, so
# the launch writes half the partial planes and its consumer adds half as many. Measured on the
# large decoder's projections alone (cold weights, in sequence): q/k/v 14.7 us with J = 1 against
# 16.1-16.4 us with J = 2, while a single projection of the same shape is slower with J = 1
# (6.5 us against 7.2 us) and the gate/up pair is no faster with J = 2 (24.2 against 24.4 us).
LINEAR_TARGET_GROUPS = 256    # MI355X compute units
LINEAR_EPILOGUE_COLUMN_BYTES = 4 * 16 * 64 * 4   # LDS per weight column of a lane (4 waves x 16 registers)
LINEAR_MIN_FILL = 0.85
LINEAR_MIN_CHUNK = 256
LINEAR_ZERO_PAGE = 256    # kZeroPage: leading workspace bytes that stay zero
LINEAR_VECTOR_ROWS = 16
LINEAR_VECTOR_WAVES = 16      # waves per vector-path workgroup at most (1024 threads)
LINEAR_VECTOR_WAVE_ROWS = 64  # kVectorRows: reduction rows per wave


LINEAR_SHARED_J1_MEMBERS = 3   # siblings from which the MFMA path tries J = 1 first


def linear_tiling(b: int, i: int, o: int, members: int = 1) -> dict:
    """Tiling of one linear (`members` = how many sibling linears of this shape multiply the same
    x and run as one shared-operand launch)."""
    if b > LINEAR_VECTOR_ROWS and i % 4 == 0 and o % 4 == 0:
        row_tiles = _cdiv(b, 32)
        best = None
        for j in ((1, 2, 4) if members >= LINEAR_SHARED_J1_MEMBERS else (2, 4, 1)):
            tiles = _cdiv(o, 32 * j)
            split = max(1, min(LINEAR_TARGET_GROUPS // (row_tiles * tiles), i // LINEAR_MIN_CHUNK))
            chunk = _cdiv(_cdiv(i, split), 16) * 16
            split = _cdiv(i, chunk)
            grid = row_tiles * tiles * split
            fill = grid / LINEAR_TARGET_GROUPS if grid <= LINEAR_TARGET_GROUPS else 0.5
            if best is None or fill > best[0]:
                best = (fill, j, tiles, split, chunk)
            if fill >= LINEAR_MIN_FILL:
                best = (fill, j, tiles, split, chunk)
                break
        _, j, tiles, split, chunk = best
        rows = row_tiles * 32
        shared = j * LINEAR_EPILOGUE_COLUMN_BYTES      # the 4 waves' accumulator tiles, one pass
        entry = f"ckl_linear_mfma{j}x1"
        block = BLOCK
    elif b <= LINEAR_VECTOR_ROWS:
        tiles = _cdiv(o, 64)
        waves = min(LINEAR_VECTOR_WAVES, _cdiv(i, LINEAR_VECTOR_WAVE_ROWS))
        chunk = LINEAR_VECTOR_WAVE_ROWS                   # rows per wave (kVectorRows)
        split = _cdiv(i, waves * chunk)
        rows, row_tiles = b, b                            # one workgroup per batch row
        shared = 0
        entry = "ckl_linear_rowvec"
        block = 64 * waves
    else:
        return None
    workspace, partials = LINEAR_ZERO_PAGE, 0
    if split > 1:
        counters = row_tiles * tiles if entry != "ckl_linear_rowvec" else b * tiles
        workspace += _cdiv(4 * counters, 256) * 256
        partials = 4 * split * rows * o
    return dict(grid=row_tiles * split * tiles, tiles=tiles, split=split, chunk=chunk, shared=shared, entry=entry,
                workspace=workspace, partials=partials, block=block)


def _linear(shapes, consts, ext):
    (b, i), (w, _i, o) = shapes[0], shapes[1]
    layer = consts[3]
    if not (0 <= layer < w) or not (ext[0] >= o and ext[1:] == (b, 1)):
        return None
    def launch(t, variants=()):
        return Launch(t["grid"], (b, i, o, layer, t["tiles"], t["split"], t["chunk"], 0), block=t["block"],
                      shared=t["shared"], entry=t["entry"], workspace=t["workspace"], partials=t["partials"],
                      variants=variants)

    t = linear_tiling(b, i, o)
    if t is None:
        return None
    shared = linear_tiling(b, i, o, LINEAR_SHARED_J1_MEMBERS)
    variants = ((LINEAR_SHARED_J1_MEMBERS, launch(shared)),) if shared != t else ()
    return launch(t, variants)


def _rope(shapes, consts, ext):
    (b, c), (t, r, _two) = shapes[0], shapes[1]
    if c % (2 * r):
        return None
    a = c // (2 * r)
    if not (ext[0] >= r and ext[1:] == (a, b)):
        return None
    unit = 1 if r % 2 else 2      # rope_unit: pairs a thread rotates (two: 128-bit accesses)
    return Launch(_cdiv(b * a * (r // unit), BLOCK), (b, a, r, t))


def _append_kv(shapes, consts, ext):
    (b, c), (l, _b, a, t, d) = shapes[0], shapes[2]
    layer = consts[5]
    if a * d != c or not (0 <= layer < l) or not (ext[0] >= d and ext[1:] == (a, b)):
        return None
    return Launch(_elementwise(b * a * d, d), (l, b, a, t, d, layer))


def _scores(shapes, consts, ext):
    (b, c), (l, _b, a, t, d) = shapes[0], shapes[1]
    layer = consts[5]
    if a * d != c or not (0 <= layer < l) or not (ext[0] >= t and ext[1:] == (a, b)):
        return None
    return Launch(b * a * _cdiv(t, BLOCK), (l, b, a, t, d, layer))


def _softmax(shapes, consts, ext):
    b, a, t = shapes[0]
    if not (ext[0] >= b and ext[1:] == (a, 1)):
        return None
    row_threads = 64 if t <= 512 else 256           # one wave per row, or the whole workgroup
    return Launch(_cdiv(b * a, BLOCK // row_threads), (b, a, t, row_threads))


def _values(shapes, consts, ext):
    (b, a, t), (l, _b, _a, _t, d), (_b2, c) = shapes[0], shapes[1], shapes[3]
    layer = consts[4]
    if a * d != c or not (0 <= layer < l) or not (ext[0] >= d and ext[1:] == (a, b)):
        return None
    # Enough row groups to keep ~8 rows in flight per lane over the whole capacity, at least one
    # wave, at most VALUES_BLOCK threads; the D/4 lanes of a row must divide a wave.
    width = d // 4 if d % 4 == 0 and d <= 256 and 64 % (d // 4) == 0 else 64
    block = 64
    while block < VALUES_BLOCK and (block // width) * 8 < t:
        block *= 2
    return Launch(b * a, (l, b, a, t, d, layer), block=block)


def _binary(shapes, consts, ext):
    (b, c) = shapes[0]
    return Launch(_elementwise(b * c, c), (b * c,)) if ext[0] >= c and ext[1:] == (b, 1) else None


def _unary(shapes, consts, ext):
    (b, c) = shapes[0]
    return Launch(_elementwise(b * c, c), (b * c,)) if ext[0] >= c and ext[1:] == (b, 1) else None


def _greedy(shapes, consts, ext):
    (b, v), (t, _b) = shapes[0], shapes[2]
    if not (ext[0] >= b and ext[1:] == (1, 1)):
        return None
    workspace = _cdiv(12 * b + 4, 256) * 256       # keys, counters, row count (greedy -> advance chain)
    if GREEDY_CHUNK < v <= 8 * 4 * GREEDY_ROW_THREADS and v % 4 == 0:
        return Launch(b, (b, v, t, 1), block=GREEDY_ROW_THREADS, workspace=workspace)
    chunks = _cdiv(v, GREEDY_CHUNK)
    return Launch(b * chunks, (b, v, t, chunks), workspace=workspace)


def _advance(shapes, consts, ext):
    return Launch(1, (), block=64) if ext == (1, 1, 1) else None


def _update(shapes, consts, ext):
    (n,) = shapes[0]
    return Launch(_elementwise(n, n), (n,)) if ext[0] >= n and ext[1:] == (1, 1) else None


@dataclass(frozen=True)
class LibraryKernel:
    name: str
    contract: Definition
    launch: Callable
    groupable: bool = False

    @property
    def entry_point(self) -> str:
        return f"ckl_{self.name}"


LIBRARY = (
    LibraryKernel("embedding", embedding, _embedding),
    LibraryKernel("rms_stats", rms_stats, _rms_stats),
    LibraryKernel("rms_apply", rms_apply, _rms_apply),
    LibraryKernel("linear", linear, _linear, groupable=True),
    LibraryKernel("rope", rope, _rope, groupable=True),
    LibraryKernel("append_kv", append_kv, _append_kv),
    LibraryKernel("attention_scores", attention_scores, _scores),
    LibraryKernel("softmax", softmax, _softmax),
    LibraryKernel("attention_values", attention_values, _values),
    LibraryKernel("add", add, _binary),
    LibraryKernel("silu", silu, _unary),
    LibraryKernel("multiply", multiply, _binary),
    LibraryKernel("greedy", greedy, _greedy),
    LibraryKernel("advance", advance, _advance),
    LibraryKernel("update", update, _update),
)


def _rebind(contract: Definition, signature: BoundSignature) -> Optional[BoundSignature]:
    names = [a.arg for a in contract.tree.args.args]
    if len(names) != len(signature.parameters):
        return None
    runtime = {n: p.dtype for n, p in zip(names, signature.parameters) if not p.is_constant}
    constants = {n: p.value for n, p in zip(names, signature.parameters) if p.is_constant}
    try:
        return bind(contract, runtime, constants)
    except FrontendError:
        return None


@dataclass(frozen=True)
class Selection:
    symbol: str
    kernel: LibraryKernel
    launch: Launch


class LibraryNameWarning(UserWarning):
    """A kernel named like a library kernel is compiled from its own body instead."""


def explain(lowered) -> dict:
    """Per kernel symbol of `lowered`: ("library", entry point) when a library kernel serves it,
    ("jit", reason) otherwise."""
    report = {}
    for spec, text, extents in zip(lowered.specializations, lowered.kernels, lowered.extents):
        report[spec.symbol] = ("jit", "no library kernel has this body")
        for entry in LIBRARY:
            bound = _rebind(entry.contract, spec.signature)
            if bound is None or lower_kernel(entry.contract, bound) != text:
                continue
            shapes = [p.dtype.shape if isinstance(p.dtype, BufferSpec) else None for p in spec.signature.parameters]
            consts = [p.value if p.is_constant else None for p in spec.signature.parameters]
            launches = {entry.launch(shapes, consts, ext) for ext in extents}
            if len(launches) == 1 and None not in launches:
                launch = launches.pop()
                report[spec.symbol] = ("library", Selection(spec.symbol, entry, launch))
            else:
                report[spec.symbol] = ("jit", f"body of library kernel {entry.name}, but launched over threads "
                                              f"{sorted(extents)} that its gfx950 kernel does not cover")
            break
        kind, detail = report[spec.symbol]
        named = spec.definition.name if spec.definition is not None else ""
        if kind == "jit" and any(entry.name == named for entry in LIBRARY):
            warnings.warn(f"kernel '{named}' ({spec.symbol}) is compiled from its own IR: {detail}", LibraryNameWarning,
                          stacklevel=3)
    return report


def select(lowered) -> dict:
    """Map kernel symbols of `lowered` to library selections (unselected kernels are JIT-compiled)."""
    return {symbol: detail for symbol, (kind, detail) in explain(lowered).items() if kind == "library"}


def selection_attribute(selections: dict, artifact: str) -> str:
    """Module attribute text `ckl.hip.selection = {...}` consumed by the native prepare step."""
    entries = []
    for symbol, s in sorted(selections.items()):
        fields = [f'artifact = "{artifact}"', f"block = array<i64: {s.launch.block}, 1, 1>",
                  "constants = [" + ", ".join(f"{int(c)} : i32" for c in s.launch.constants) + "]",
                  f'entry_point = "{s.launch.entry or s.kernel.entry_point}"', f"grid = array<i64: {s.launch.grid}, 1, 1>",
                  f'implementation = "ckl.hip.library.{s.kernel.name}"', f"shared_memory = {s.launch.shared} : i64"]
        if s.launch.workspace:
            fields.append(f"workspace = {s.launch.workspace} : i64")
        if s.launch.partials >= 0:
            fields.append(f"partials = {s.launch.partials} : i64")
        if s.launch.variants:
            variants = []
            for members, v in s.launch.variants:
                variant = [f"block = array<i64: {v.block}, 1, 1>",
                           "constants = [" + ", ".join(f"{int(c)} : i32" for c in v.constants) + "]",
                           f'entry_point = "{v.entry or s.kernel.entry_point}"', f"grid = array<i64: {v.grid}, 1, 1>",
                           f"members = {members} : i64", f"shared_memory = {v.shared} : i64",
                           f"workspace = {v.workspace} : i64", f"partials = {v.partials} : i64"]
                variants.append("{" + ", ".join(variant) + "}")
            fields.append("variants = [" + ", ".join(variants) + "]")
        if s.kernel.groupable:
            fields.append(f'group = "{s.kernel.name}"')
        entries.append(f"{symbol} = {{{', '.join(sorted(fields))}}}")
    return "ckl.hip.selection = {" + ", ".join(entries) + "}"
