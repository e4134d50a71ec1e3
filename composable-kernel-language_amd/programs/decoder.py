"""One greedy decode step of a Llama-style decoder, as a CKL program.

The step embeds each request's current token, runs every layer (RMSNorm, q/k/v projections,
rotary embedding of q and k at the current position, the new k and v appended to the layer's
cache, attention of the new query over positions 0..p, output projection with residual, RMSNorm,
SwiGLU MLP with residual), then normalises, projects onto the vocabulary, picks each request's
next token greedily, records it in the history and advances the position.

This is the measured workload of the reference (benchmarks/decoder/workloads.py:191-254): the
same kernels (ckl.decoder_kernels), the same temporaries and the same launch order, so the
dependency graph, the storage plan and the results are the ones the reference plans for it;
tests/test_decoder_plan.py pins the topology and heap sizes against the reference's recorded
plans. The step is written here as @ckl.block fragments, which the frontend expands in place:
the lowered program is one flat sequence of allocations and dispatches.
"""
from __future__ import annotations

import ckl
from ckl import decoder_kernels as k

Batch, Width, Ffn, Vocab = ckl.dim("B"), ckl.dim("C"), ckl.dim("F"), ckl.dim("V")
Layers, Heads, Capacity, HeadDim, Half = ckl.dim("L"), ckl.dim("A"), ckl.dim("T"), ckl.dim("D"), ckl.dim("R")
Gains = ckl.dim("G")

Activations = ckl.Buffer[ckl.f32, (Batch, Width)]
Norms = ckl.Buffer[ckl.f32, (Gains, Width)]
Square = ckl.Buffer[ckl.f32, (Layers, Width, Width)]
Up = ckl.Buffer[ckl.f32, (Layers, Width, Ffn)]
Down = ckl.Buffer[ckl.f32, (Layers, Ffn, Width)]
Cache = ckl.Buffer[ckl.f32, (Layers, Batch, Heads, Capacity, HeadDim)]
Rotary = ckl.Buffer[ckl.f32, (Capacity, Half, 2)]
Position = ckl.Buffer[ckl.i32, (1,)]

ROW_THREADS = 32        # row kernels (rms_stats, softmax, greedy): one thread per row
COLUMN_THREADS = 64     # column kernels: one thread per output column
HEAD_THREADS = 32       # per-head kernels: one thread per rotary pair / head element / position


@ckl.block
def rms_norm(x: Activations, gains: Norms, row: ckl.constexpr[ckl.index], epsilon: ckl.f32) -> Activations:
    """x * rsqrt(mean(x^2) + epsilon) * gains[row]: the statistics, then the scaled copy."""
    inverse = ckl.empty((Batch,), dtype=ckl.f32)
    scaled = ckl.empty_like(x)
    ckl.launch(k.rms_stats, x, inverse, epsilon, grid=(ckl.cdiv(Batch, ROW_THREADS),), block=(ROW_THREADS,))
    ckl.launch(k.rms_apply, x, inverse, gains, scaled, row, grid=(ckl.cdiv(Width, COLUMN_THREADS), Batch),
               block=(COLUMN_THREADS,))
    return scaled


@ckl.block
def qkv(x: Activations, wq: Square, wk: Square, wv: Square, layer: ckl.constexpr[ckl.index]):
    """The three projections of one normalised input (outputs allocated first, as in the workload)."""
    q = ckl.empty_like(x)
    key = ckl.empty_like(x)
    value = ckl.empty_like(x)
    columns = (ckl.cdiv(Width, COLUMN_THREADS), Batch)
    ckl.launch(k.linear, x, wq, q, layer, grid=columns, block=(COLUMN_THREADS,))
    ckl.launch(k.linear, x, wk, key, layer, grid=columns, block=(COLUMN_THREADS,))
    ckl.launch(k.linear, x, wv, value, layer, grid=columns, block=(COLUMN_THREADS,))
    return q, key, value


@ckl.block
def attention(q: Activations, key: Activations, value: Activations, sincos: Rotary, position: Position,
              kc: Cache, vc: Cache, scale: ckl.f32, layer: ckl.constexpr[ckl.index]) -> Activations:
    """Rotate q and k, append k and v at the position, attend over the cache rows 0..position."""
    q_rotated = ckl.empty_like(q)
    k_rotated = ckl.empty_like(key)
    pairs = (ckl.cdiv(Half, HEAD_THREADS), Heads, Batch)
    lanes = (ckl.cdiv(HeadDim, HEAD_THREADS), Heads, Batch)
    ckl.launch(k.rope, q, sincos, position, q_rotated, grid=pairs, block=(HEAD_THREADS,))
    ckl.launch(k.rope, key, sincos, position, k_rotated, grid=pairs, block=(HEAD_THREADS,))
    ckl.launch(k.append_kv, k_rotated, value, kc, vc, position, layer, grid=lanes, block=(HEAD_THREADS,))
    scores = ckl.empty((Batch, Heads, Capacity), dtype=ckl.f32)
    weights = ckl.empty_like(scores)
    ckl.launch(k.attention_scores, q_rotated, kc, position, scores, scale, layer,
               grid=(ckl.cdiv(Capacity, HEAD_THREADS), Heads, Batch), block=(HEAD_THREADS,))
    ckl.launch(k.softmax, scores, position, weights, grid=(ckl.cdiv(Batch, ROW_THREADS), Heads),
               block=(ROW_THREADS,))
    mixed = ckl.empty_like(q)
    ckl.launch(k.attention_values, weights, vc, position, mixed, layer, grid=lanes, block=(HEAD_THREADS,))
    return mixed


@ckl.block
def project_add(residual: Activations, x: Activations, w: Square, layer: ckl.constexpr[ckl.index]) -> Activations:
    """residual + x @ w[layer]."""
    columns = (ckl.cdiv(Width, COLUMN_THREADS), Batch)
    projected = ckl.empty_like(x)
    ckl.launch(k.linear, x, w, projected, layer, grid=columns, block=(COLUMN_THREADS,))
    total = ckl.empty_like(x)
    ckl.launch(k.add, residual, projected, total, grid=columns, block=(COLUMN_THREADS,))
    return total


@ckl.block
def swiglu(x: Activations, residual: Activations, wg: Up, wu: Up, wd: Down,
           layer: ckl.constexpr[ckl.index]) -> Activations:
    """residual + (silu(x @ wg) * (x @ wu)) @ wd, for layer `layer`."""
    gate = ckl.empty((Batch, Ffn), dtype=ckl.f32)
    up = ckl.empty_like(gate)
    hidden = (ckl.cdiv(Ffn, COLUMN_THREADS), Batch)
    ckl.launch(k.linear, x, wg, gate, layer, grid=hidden, block=(COLUMN_THREADS,))
    ckl.launch(k.linear, x, wu, up, layer, grid=hidden, block=(COLUMN_THREADS,))
    activated = ckl.empty_like(gate)
    gated = ckl.empty_like(gate)
    ckl.launch(k.silu, gate, activated, grid=hidden, block=(COLUMN_THREADS,))
    ckl.launch(k.multiply, activated, up, gated, grid=hidden, block=(COLUMN_THREADS,))
    down = ckl.empty_like(x)
    total = ckl.empty_like(x)
    columns = (ckl.cdiv(Width, COLUMN_THREADS), Batch)
    ckl.launch(k.linear, gated, wd, down, layer, grid=columns, block=(COLUMN_THREADS,))
    ckl.launch(k.add, residual, down, total, grid=columns, block=(COLUMN_THREADS,))
    return total


@ckl.program
def decode(tokens: ckl.Buffer[ckl.i32, (Batch,)], position: Position,
           history: ckl.Buffer[ckl.i32, (Capacity, Batch)], emb: ckl.Buffer[ckl.f32, (Vocab, Width)],
           norm1: ckl.Buffer[ckl.f32, (Layers, Width)], norm2: ckl.Buffer[ckl.f32, (Layers, Width)],
           final_norm: ckl.Buffer[ckl.f32, (1, Width)], wq: Square, wk: Square, wv: Square, wo: Square,
           wg: Up, wu: Up, wd: Down, lm: ckl.Buffer[ckl.f32, (1, Width, Vocab)], sincos: Rotary, kc: Cache,
           vc: Cache, logits: ckl.Buffer[ckl.f32, (Batch, Vocab)], epsilon: ckl.f32,
           attention_scale: ckl.f32) -> None:
    x = ckl.empty((Batch, Width), dtype=ckl.f32)
    ckl.launch(k.embedding, tokens, emb, x, grid=(ckl.cdiv(Width, COLUMN_THREADS), Batch), block=(COLUMN_THREADS,))
    for layer in range(Layers):
        normed = rms_norm(x, norm1, layer, epsilon)
        q, key, value = qkv(normed, wq, wk, wv, layer)
        mixed = attention(q, key, value, sincos, position, kc, vc, attention_scale, layer)
        residual = project_add(x, mixed, wo, layer)
        x = swiglu(rms_norm(residual, norm2, layer, epsilon), residual, wg, wu, wd, layer)
    final = rms_norm(x, final_norm, 0, epsilon)
    ckl.launch(k.linear, final, lm, logits, 0, grid=(ckl.cdiv(Vocab, COLUMN_THREADS), Batch), block=(COLUMN_THREADS,))
    ckl.launch(k.greedy, logits, tokens, history, position, grid=(ckl.cdiv(Batch, ROW_THREADS),), block=(ROW_THREADS,))
    ckl.launch(k.advance, position, grid=(1,), block=(1,))
