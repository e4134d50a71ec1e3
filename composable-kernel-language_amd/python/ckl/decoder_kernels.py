"""The decoder kernel set: the CKL kernel bodies that the gfx950 library implements by hand.

These are the kernels of the reference's decoder workload (benchmarks/decoder/workloads.py:33-188)
and of its vector pipeline example (examples/vector_pipeline.py:11-16), restated as the contract
the library is a drop-in for: a kernel specialisation is served by the library exactly when its
IR, printed canonically, equals the IR of the matching body here specialised the same way
(ckl.library). Programs may launch these definitions directly (programs/decoder.py does) or
define bodies of their own; only the IR decides.
"""
from __future__ import annotations

import ckl

_B, _C, _L, _A, _T, _D, _V, _R = [ckl.dim(n) for n in ("B", "C", "L", "A", "T", "D", "V", "R")]
_W, _I, _O, _N = [ckl.dim(n) for n in ("W", "I", "O", "N")]
_Hidden = ckl.Buffer[ckl.f32, (_B, _C)]
_Rows = ckl.Buffer[ckl.f32, (_B,)]
_Tokens = ckl.Buffer[ckl.i32, (_B,)]
_Position = ckl.Buffer[ckl.i32, (1,)]
_History = ckl.Buffer[ckl.i32, (_T, _B)]
_Table = ckl.Buffer[ckl.f32, (_V, _C)]
_Gain = ckl.Buffer[ckl.f32, (_L, _C)]
_Cache = ckl.Buffer[ckl.f32, (_L, _B, _A, _T, _D)]
_SinCos = ckl.Buffer[ckl.f32, (_T, _R, 2)]
_Scores = ckl.Buffer[ckl.f32, (_B, _A, _T)]
_Logits = ckl.Buffer[ckl.f32, (_B, _V)]
_In = ckl.Buffer[ckl.f32, (_B, _I)]
_Out = ckl.Buffer[ckl.f32, (_B, _O)]
_Matrix = ckl.Buffer[ckl.f32, (_W, _I, _O)]
_Vector = ckl.Buffer[ckl.f32, (_N,)]


@ckl.kernel
def embedding(tokens: _Tokens, table: _Table, dst: _Hidden) -> None:
    c = ckl.global_id(0)
    b = ckl.global_id(1)
    if c < _C:
        token = ckl.cast(tokens[b], ckl.index)
        dst[b, c] = table[token, c]


@ckl.kernel
def rms_stats(x: _Hidden, inv: _Rows, epsilon: ckl.f32) -> None:
    b = ckl.global_id(0)
    if b < _B:
        total = 0.0
        for c in range(_C):
            total = total + x[b, c] * x[b, c]
        inv[b] = ckl.rsqrt(total / _C + epsilon)


@ckl.kernel
def rms_apply(x: _Hidden, inv: _Rows, gain: _Gain, dst: _Hidden, layer: ckl.constexpr[ckl.index]) -> None:
    c = ckl.global_id(0)
    b = ckl.global_id(1)
    if c < _C:
        dst[b, c] = x[b, c] * inv[b] * gain[layer, c]


@ckl.kernel
def linear(x: _In, weight: _Matrix, dst: _Out, layer: ckl.constexpr[ckl.index]) -> None:
    o = ckl.global_id(0)
    b = ckl.global_id(1)
    if o < _O:
        total = 0.0
        for i in range(_I):
            total = total + x[b, i] * weight[layer, i, o]
        dst[b, o] = total


@ckl.kernel
def rope(src: _Hidden, table: _SinCos, position: _Position, dst: _Hidden) -> None:
    r = ckl.global_id(0)
    h = ckl.global_id(1)
    b = ckl.global_id(2)
    if r < _R:
        p = ckl.cast(position[0], ckl.index)
        c = h * (2 * _R) + 2 * r
        first = src[b, c]
        second = src[b, c + 1]
        cosine = table[p, r, 0]
        sine = table[p, r, 1]
        dst[b, c] = first * cosine - second * sine
        dst[b, c + 1] = first * sine + second * cosine


@ckl.kernel
def append_kv(k: _Hidden, v: _Hidden, kc: _Cache, vc: _Cache, position: _Position,
              layer: ckl.constexpr[ckl.index]) -> None:
    d = ckl.global_id(0)
    h = ckl.global_id(1)
    b = ckl.global_id(2)
    if d < _D:
        p = ckl.cast(position[0], ckl.index)
        kc[layer, b, h, p, d] = k[b, h * _D + d]
        vc[layer, b, h, p, d] = v[b, h * _D + d]


@ckl.kernel
def attention_scores(q: _Hidden, kc: _Cache, position: _Position, scores: _Scores,
                     scale: ckl.f32, layer: ckl.constexpr[ckl.index]) -> None:
    t = ckl.global_id(0)
    h = ckl.global_id(1)
    b = ckl.global_id(2)
    end = ckl.cast(position[0], ckl.index) + 1
    if t < end:
        total = 0.0
        for d in range(_D):
            total = total + q[b, h * _D + d] * kc[layer, b, h, t, d]
        scores[b, h, t] = total * scale


@ckl.kernel
def softmax(scores: _Scores, position: _Position, probs: _Scores) -> None:
    b = ckl.global_id(0)
    h = ckl.global_id(1)
    if b < _B:
        end = ckl.cast(position[0], ckl.index) + 1
        maximum = scores[b, h, 0]
        for t in range(1, end):
            value = scores[b, h, t]
            maximum = ckl.select(value > maximum, value, maximum)
        total = 0.0
        for t in range(end):
            total = total + ckl.exp(scores[b, h, t] - maximum)
        for t in range(end):
            probs[b, h, t] = ckl.exp(scores[b, h, t] - maximum) / total


@ckl.kernel
def attention_values(probs: _Scores, vc: _Cache, position: _Position, dst: _Hidden,
                     layer: ckl.constexpr[ckl.index]) -> None:
    d = ckl.global_id(0)
    h = ckl.global_id(1)
    b = ckl.global_id(2)
    if d < _D:
        end = ckl.cast(position[0], ckl.index) + 1
        total = 0.0
        for t in range(end):
            total = total + probs[b, h, t] * vc[layer, b, h, t, d]
        dst[b, h * _D + d] = total


@ckl.kernel
def add(x: _Hidden, y: _Hidden, dst: _Hidden) -> None:
    c = ckl.global_id(0)
    b = ckl.global_id(1)
    if c < _C:
        dst[b, c] = x[b, c] + y[b, c]


@ckl.kernel
def silu(src: _In, dst: _In) -> None:
    i = ckl.global_id(0)
    b = ckl.global_id(1)
    if i < _I:
        value = src[b, i]
        dst[b, i] = value / (1.0 + ckl.exp(-value))


@ckl.kernel
def multiply(x: _In, y: _In, dst: _In) -> None:
    i = ckl.global_id(0)
    b = ckl.global_id(1)
    if i < _I:
        dst[b, i] = x[b, i] * y[b, i]


@ckl.kernel
def greedy(logits: _Logits, tokens: _Tokens, history: _History, position: _Position) -> None:
    b = ckl.global_id(0)
    if b < _B:
        maximum = logits[b, 0]
        winner = ckl.cast(b, ckl.i32) * 0
        for v in range(1, _V):
            score = logits[b, v]
            wins = score > maximum
            winner = ckl.select(wins, ckl.cast(v, ckl.i32), winner)
            maximum = ckl.select(wins, score, maximum)
        p = ckl.cast(position[0], ckl.index)
        tokens[b] = winner
        history[p, b] = winner


@ckl.kernel
def advance(position: _Position) -> None:
    position[0] = position[0] + 1


@ckl.kernel
def update(src: _Vector, dst: _Vector, bias: ckl.f32) -> None:
    i = ckl.global_id(0)
    if i < src.shape[0]:
        dst[i] = src[i] + bias
