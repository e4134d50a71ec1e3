"""Config V of the benchmark (the reference's examples/vector_pipeline.py:7-40): dst = (src + bias)
+ bias as two launches of the library's `update` kernel through one program temporary, which the
storage planner places in a heap and reuses across replays (fused into one generated kernel when
pointwise fusion is on)."""
from __future__ import annotations

import ckl
from ckl.decoder_kernels import Flat, update

THREADS = 256


@ckl.program
def step(src: Flat, dst: Flat, bias: ckl.f32) -> None:
    staged = ckl.empty_like(src)
    blocks = (ckl.cdiv(src.shape[0], THREADS),)
    ckl.launch(update, src, staged, bias, grid=blocks, block=(THREADS,))
    ckl.launch(update, staged, dst, bias, grid=blocks, block=(THREADS,))


def lower(n: int = 257):
    """The program specialised for vectors of `n` f32 values."""
    vector = ckl.BufferSpec(shape=(n,), dtype=ckl.f32)
    return step.lower(signature={"src": vector, "dst": vector, "bias": ckl.f32})
