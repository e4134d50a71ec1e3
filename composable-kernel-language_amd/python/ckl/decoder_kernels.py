"""Contract bodies of the hand-written gfx950 kernels (csrc/kernels/library.hip).

A CKL kernel specialisation runs on a library kernel exactly when its IR, printed canonically
(no names: SSA numbers, argument positions and concrete types only), equals the IR of the body
below with the same name, specialised to the same signature (ckl.library). The bodies therefore
fix the operation sequence of the kernels the decoder benchmark launches (the reference's
benchmarks/decoder/workloads.py:33-188) and of the vector-pipeline example's `update`
(examples/vector_pipeline.py:11-16); tests/golden/workload_ir.json records the canonical IR of
those reference kernels for every specialisation the decode program uses, and
tests/test_contract_ir.py checks these bodies against it. Everything else here (names, aliases,
layout of the source) is this package's own.

Threads: x is the innermost index of the written element, y and z the outer ones; a thread
outside the output's extent does nothing. Arithmetic is f32 in the order written.
"""
from __future__ import annotations

import ckl

BATCH, WIDTH, DEPTH, HEADS, SLOTS, HEAD, VOCAB, PAIRS = (
    ckl.dim(n) for n in ("batch", "width", "depth", "heads", "slots", "head", "vocab", "pairs"))
STACK, FAN_IN, FAN_OUT, LENGTH = (ckl.dim(n) for n in ("stack", "fan_in", "fan_out", "length"))

Activations = ckl.Buffer[ckl.f32, (BATCH, WIDTH)]        # one row of WIDTH features per request
PerRequest = ckl.Buffer[ckl.f32, (BATCH,)]
TokenIds = ckl.Buffer[ckl.i32, (BATCH,)]
Cursor = ckl.Buffer[ckl.i32, (1,)]                        # the decode position
Emitted = ckl.Buffer[ckl.i32, (SLOTS, BATCH)]             # generated tokens by position
Vocabulary = ckl.Buffer[ckl.f32, (VOCAB, WIDTH)]
Gains = ckl.Buffer[ckl.f32, (DEPTH, WIDTH)]
KVCache = ckl.Buffer[ckl.f32, (DEPTH, BATCH, HEADS, SLOTS, HEAD)]
Rotations = ckl.Buffer[ckl.f32, (SLOTS, PAIRS, 2)]        # (cos, sin) per position and pair
HeadRows = ckl.Buffer[ckl.f32, (BATCH, HEADS, SLOTS)]     # one value per cached position
Logits = ckl.Buffer[ckl.f32, (BATCH, VOCAB)]
Inputs = ckl.Buffer[ckl.f32, (BATCH, FAN_IN)]
Outputs = ckl.Buffer[ckl.f32, (BATCH, FAN_OUT)]
Weights = ckl.Buffer[ckl.f32, (STACK, FAN_IN, FAN_OUT)]  # one matrix per layer
Flat = ckl.Buffer[ckl.f32, (LENGTH,)]


@ckl.kernel
def embedding(ids: TokenIds, table: Vocabulary, out: Activations) -> None:
    """out[r, :] = table[ids[r], :]."""
    col = ckl.global_id(0)
    row = ckl.global_id(1)
    if col < WIDTH:
        entry = ckl.cast(ids[row], ckl.index)
        out[row, col] = table[entry, col]


@ckl.kernel
def rms_stats(rows: Activations, inverse: PerRequest, eps: ckl.f32) -> None:
    """inverse[r] = 1 / sqrt(mean of rows[r, :]^2 + eps), one thread a row, columns in order."""
    row = ckl.global_id(0)
    if row < BATCH:
        squares = 0.0
        for col in range(WIDTH):
            squares = squares + rows[row, col] * rows[row, col]
        inverse[row] = ckl.rsqrt(squares / WIDTH + eps)


@ckl.kernel
def rms_apply(rows: Activations, inverse: PerRequest, gains: Gains, out: Activations,
              which: ckl.constexpr[ckl.index]) -> None:
    """out[r, c] = (rows[r, c] * inverse[r]) * gains[which, c]."""
    col = ckl.global_id(0)
    row = ckl.global_id(1)
    if col < WIDTH:
        out[row, col] = rows[row, col] * inverse[row] * gains[which, col]


@ckl.kernel
def linear(source: Inputs, matrices: Weights, out: Outputs, which: ckl.constexpr[ckl.index]) -> None:
    """out[r, o] = sum over i (in order) of source[r, i] * matrices[which, i, o]."""
    col = ckl.global_id(0)
    row = ckl.global_id(1)
    if col < FAN_OUT:
        acc = 0.0
        for k in range(FAN_IN):
            acc = acc + source[row, k] * matrices[which, k, col]
        out[row, col] = acc


@ckl.kernel
def rope(source: Activations, rotations: Rotations, cursor: Cursor, out: Activations) -> None:
    """Rotates feature pair (2j, 2j+1) of head h by the angle of pair j at the cursor."""
    pair = ckl.global_id(0)
    head = ckl.global_id(1)
    row = ckl.global_id(2)
    if pair < PAIRS:
        at = ckl.cast(cursor[0], ckl.index)
        even = head * (2 * PAIRS) + 2 * pair
        re = source[row, even]
        im = source[row, even + 1]
        cos = rotations[at, pair, 0]
        sin = rotations[at, pair, 1]
        out[row, even] = re * cos - im * sin
        out[row, even + 1] = re * sin + im * cos


@ckl.kernel
def append_kv(keys: Activations, values: Activations, key_cache: KVCache, value_cache: KVCache, cursor: Cursor,
              which: ckl.constexpr[ckl.index]) -> None:
    """Stores head h's key and value features of every request at the cursor's slot."""
    lane = ckl.global_id(0)
    head = ckl.global_id(1)
    row = ckl.global_id(2)
    if lane < HEAD:
        at = ckl.cast(cursor[0], ckl.index)
        key_cache[which, row, head, at, lane] = keys[row, head * HEAD + lane]
        value_cache[which, row, head, at, lane] = values[row, head * HEAD + lane]


@ckl.kernel
def attention_scores(query: Activations, key_cache: KVCache, cursor: Cursor, out: HeadRows, scale: ckl.f32,
                     which: ckl.constexpr[ckl.index]) -> None:
    """out[r, h, s] = (query head h . cached key s) * scale for every slot s up to the cursor."""
    slot = ckl.global_id(0)
    head = ckl.global_id(1)
    row = ckl.global_id(2)
    upto = ckl.cast(cursor[0], ckl.index) + 1
    if slot < upto:
        dot = 0.0
        for lane in range(HEAD):
            dot = dot + query[row, head * HEAD + lane] * key_cache[which, row, head, slot, lane]
        out[row, head, slot] = dot * scale


@ckl.kernel
def softmax(logits: HeadRows, cursor: Cursor, out: HeadRows) -> None:
    """out[r, h, :] = exp(x - max) / sum(exp(x - max)) over slots 0..cursor; the maximum is a
    strict `>` scan from slot 0, the sum is taken in slot order."""
    row = ckl.global_id(0)
    head = ckl.global_id(1)
    if row < BATCH:
        upto = ckl.cast(cursor[0], ckl.index) + 1
        peak = logits[row, head, 0]
        for slot in range(1, upto):
            candidate = logits[row, head, slot]
            peak = ckl.select(candidate > peak, candidate, peak)
        norm = 0.0
        for slot in range(upto):
            norm = norm + ckl.exp(logits[row, head, slot] - peak)
        for slot in range(upto):
            out[row, head, slot] = ckl.exp(logits[row, head, slot] - peak) / norm


@ckl.kernel
def attention_values(weights: HeadRows, value_cache: KVCache, cursor: Cursor, out: Activations,
                     which: ckl.constexpr[ckl.index]) -> None:
    """out[r, h*HEAD + d] = sum over slots 0..cursor (in order) of weight * cached value."""
    lane = ckl.global_id(0)
    head = ckl.global_id(1)
    row = ckl.global_id(2)
    if lane < HEAD:
        upto = ckl.cast(cursor[0], ckl.index) + 1
        acc = 0.0
        for slot in range(upto):
            acc = acc + weights[row, head, slot] * value_cache[which, row, head, slot, lane]
        out[row, head * HEAD + lane] = acc


@ckl.kernel
def add(lhs: Activations, rhs: Activations, out: Activations) -> None:
    col = ckl.global_id(0)
    row = ckl.global_id(1)
    if col < WIDTH:
        out[row, col] = lhs[row, col] + rhs[row, col]


@ckl.kernel
def silu(source: Inputs, out: Inputs) -> None:
    """out = x / (1 + exp(-x))."""
    col = ckl.global_id(0)
    row = ckl.global_id(1)
    if col < FAN_IN:
        x = source[row, col]
        out[row, col] = x / (1.0 + ckl.exp(-x))


@ckl.kernel
def multiply(lhs: Inputs, rhs: Inputs, out: Inputs) -> None:
    col = ckl.global_id(0)
    row = ckl.global_id(1)
    if col < FAN_IN:
        out[row, col] = lhs[row, col] * rhs[row, col]


@ckl.kernel
def greedy(logits: Logits, ids: TokenIds, emitted: Emitted, cursor: Cursor) -> None:
    """ids[r] = emitted[cursor, r] = the first index of the largest logit of row r (a strict `>`
    scan from index 0, so NaN never wins and ties keep the earlier index)."""
    row = ckl.global_id(0)
    if row < BATCH:
        best = logits[row, 0]
        choice = ckl.cast(row, ckl.i32) * 0
        for index in range(1, VOCAB):
            candidate = logits[row, index]
            better = candidate > best
            choice = ckl.select(better, ckl.cast(index, ckl.i32), choice)
            best = ckl.select(better, candidate, best)
        at = ckl.cast(cursor[0], ckl.index)
        ids[row] = choice
        emitted[at, row] = choice


@ckl.kernel
def advance(cursor: Cursor) -> None:
    cursor[0] = cursor[0] + 1


@ckl.kernel
def update(source: Flat, out: Flat, shift: ckl.f32) -> None:
    """out[i] = source[i] + shift."""
    i = ckl.global_id(0)
    if i < source.shape[0]:
        out[i] = source[i] + shift
