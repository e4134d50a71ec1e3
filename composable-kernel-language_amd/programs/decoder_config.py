"""Decoder shapes and the program signature for one configuration.

Config fields and derived sizes follow benchmarks/decoder/reference.py:6-29 of the reference
(capacity = context + steps). The five measured configurations are those of BASELINE.json.
"""
from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class Config:
    batch: int = 1
    hidden: int = 64
    heads: int = 4
    layers: int = 2
    ffn: int = 128
    vocab: int = 256
    context: int = 8
    steps: int = 16

    def __post_init__(self):
        if min(vars(self).values()) <= 0 or self.hidden % self.heads or self.head_dim % 2:
            raise ValueError("positive dimensions and an even head dimension dividing hidden are required")

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads

    @property
    def capacity(self) -> int:
        return self.context + self.steps


CONFIGS = {
    "small": Config(batch=8, hidden=64, heads=4, layers=2, ffn=256, vocab=256, context=16, steps=16),
    "wide": Config(batch=8, hidden=256, heads=8, layers=2, ffn=1024, vocab=1024, context=16, steps=16),
    "deep": Config(batch=8, hidden=64, heads=4, layers=8, ffn=256, vocab=256, context=16, steps=16),
    "large": Config(batch=32, hidden=2048, heads=16, layers=4, ffn=5632, vocab=32000, context=1024, steps=16),
}

MUTABLE = ("tokens", "position", "history", "kc", "vc", "logits")
EPSILON = 1e-5


def shapes(c: Config) -> dict:
    """Host argument shapes in program order (dtype 'i32' or 'f32')."""
    b, h, l, t, d, a = c.batch, c.hidden, c.layers, c.capacity, c.head_dim, c.heads
    return {
        "tokens": ((b,), "i32"), "position": ((1,), "i32"), "history": ((t, b), "i32"),
        "emb": ((c.vocab, h), "f32"), "norm1": ((l, h), "f32"), "norm2": ((l, h), "f32"),
        "final_norm": ((1, h), "f32"), "wq": ((l, h, h), "f32"), "wk": ((l, h, h), "f32"),
        "wv": ((l, h, h), "f32"), "wo": ((l, h, h), "f32"), "wg": ((l, h, c.ffn), "f32"),
        "wu": ((l, h, c.ffn), "f32"), "wd": ((l, c.ffn, h), "f32"), "lm": ((1, h, c.vocab), "f32"),
        "sincos": ((t, d // 2, 2), "f32"), "kc": ((l, b, a, t, d), "f32"), "vc": ((l, b, a, t, d), "f32"),
        "logits": ((b, c.vocab), "f32"),
    }


def signature(c: Config) -> dict:
    import ckl
    types = {"i32": ckl.i32, "f32": ckl.f32}
    sig = {name: ckl.BufferSpec(shape, types[dtype]) for name, (shape, dtype) in shapes(c).items()}
    sig.update(epsilon=ckl.f32, attention_scale=ckl.f32)
    return sig


def temporary_bytes_without_reuse(c: Config) -> int:
    """Sum of 256-byte-aligned temporary sizes: the planner's no-reuse heap (closed form)."""
    def aligned(n):
        return (n + 255) // 256 * 256
    b, h, f, t, a = c.batch, c.hidden, c.ffn, c.capacity, c.heads
    per_layer = 2 * aligned(4 * b) + 12 * aligned(4 * b * h) + 2 * aligned(4 * b * a * t) + 4 * aligned(4 * b * f)
    return aligned(4 * b * h) + c.layers * per_layer + aligned(4 * b) + aligned(4 * b * h)
