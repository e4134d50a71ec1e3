"""NumPy decoder oracle (TEST INFRASTRUCTURE; see oracle/__init__.py).

Restates benchmarks/decoder/reference.py:33-114 of the reference:
  rms            reference.py:36-37
  step           reference.py:40-75  (one autoregressive step, mutating persistent state)
  make_inputs    reference.py:78-107 (seeded weights in dict order, RoPE table, prompts,
                                       sentinel-filled caches, prefill of context-1 steps)
  expected       reference.py:110-114
`init="reference"` reproduces the reference's weight scales (embedding N(0, 0.5), matrices
N(0, 0.5/sqrt(fan_in)), gains 1 + N(0, 0.02)); `init="baseline"` is the benchmark's
N(0, 0.02) for the embedding and all matrices with the same draw order.
Parity: pinned against the reference's recorded prompts and generated tokens for its
configurations (tests/test_oracle_decoder.py).
"""
from __future__ import annotations

import numpy as np

MUTABLE = ("tokens", "position", "history", "kc", "vc", "logits")
EPSILON = np.float32(1e-5)
WEIGHTS = ("emb", "norm1", "norm2", "final_norm", "wq", "wk", "wv", "wo", "wg", "wu", "wd", "lm")


def rms(x, gain):
    return x * (1 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + EPSILON)) * gain


def step(a, c):
    """Advance the state `a` (dict of arrays) by exactly one decode step."""
    pos = int(a["position"][0])
    if not 0 <= pos < c.capacity:
        raise ValueError("position exceeds KV/history capacity")
    b, heads, d = c.batch, c.heads, c.head_dim
    x = a["emb"][a["tokens"]].copy()
    cos, sin = a["sincos"][pos, :, 0], a["sincos"][pos, :, 1]

    def rotate(value):
        pairs = value.reshape(b, heads, d // 2, 2)
        out = np.empty_like(pairs)
        out[..., 0] = pairs[..., 0] * cos - pairs[..., 1] * sin
        out[..., 1] = pairs[..., 0] * sin + pairs[..., 1] * cos
        return out.reshape(b, heads, d)

    for layer in range(c.layers):
        n = rms(x, a["norm1"][layer])
        q, k = rotate(n @ a["wq"][layer]), rotate(n @ a["wk"][layer])
        v = (n @ a["wv"][layer]).reshape(b, heads, d)
        a["kc"][layer, :, :, pos, :] = k
        a["vc"][layer, :, :, pos, :] = v
        keys = a["kc"][layer, :, :, :pos + 1, :]
        scores = np.sum(q[:, :, None, :] * keys, axis=-1) * np.float32(d ** -0.5)
        probs = np.exp(scores - scores.max(axis=-1, keepdims=True))
        probs /= probs.sum(axis=-1, keepdims=True)
        values = a["vc"][layer, :, :, :pos + 1, :]
        context = np.sum(probs[..., None] * values, axis=-2).reshape(b, c.hidden)
        residual = x + context @ a["wo"][layer]
        n = rms(residual, a["norm2"][layer])
        gate, up = n @ a["wg"][layer], n @ a["wu"][layer]
        x = residual + (gate / (1 + np.exp(-gate)) * up) @ a["wd"][layer]
    a["logits"][:] = rms(x, a["final_norm"][0]) @ a["lm"][0]
    a["tokens"][:] = a["logits"].argmax(axis=-1).astype(np.int32)
    a["history"][pos] = a["tokens"]
    a["position"][0] += 1


def greedy_scan(logits):
    """Tokens of the CKL decoder's greedy kernel (benchmarks/decoder/workloads.py:170-183): per row,
    a scan from index 0 keeps the running maximum and takes index v only when logit v is strictly
    greater (`>`). So NaN never wins and a NaN logit 0 is never displaced, -0 and +0 tie, and equal
    maxima keep the first index. On rows without NaN this is argmax (reference.py:71)."""
    x = np.asarray(logits, np.float32)
    y = np.where(np.isnan(x), -np.inf, x)
    winner = np.argmax(y == y.max(axis=-1, keepdims=True), axis=-1)
    return np.where(np.isnan(x[..., 0]), 0, winner).astype(np.int32)


def initial_state(c, seed=123, *, init="reference", prompt_seed=None):
    """Weights, RoPE table, prompts and empty state before any prefill step."""
    rng = np.random.default_rng(seed)
    b, h, l, t, d = c.batch, c.hidden, c.layers, c.capacity, c.head_dim
    shapes = dict(emb=(c.vocab, h), norm1=(l, h), norm2=(l, h), final_norm=(1, h),
                  wq=(l, h, h), wk=(l, h, h), wv=(l, h, h), wo=(l, h, h),
                  wg=(l, h, c.ffn), wu=(l, h, c.ffn), wd=(l, c.ffn, h), lm=(1, h, c.vocab))
    arrays = {}
    for name, shape in shapes.items():
        if "norm" in name:
            arrays[name] = (1 + rng.normal(0, 0.02, shape)).astype(np.float32)
        elif init == "reference":
            scale = 0.5 if name == "emb" else 0.5 / np.sqrt(shape[-2])
            arrays[name] = rng.normal(0, scale, shape).astype(np.float32)
        elif init == "baseline":
            arrays[name] = rng.normal(0, 0.02, shape).astype(np.float32)
        else:
            raise ValueError(f"unknown init {init!r}")
    angles = np.arange(t)[:, None] * (10000. ** (-np.arange(0, d, 2) / d))[None, :]
    arrays["sincos"] = np.stack((np.cos(angles), np.sin(angles)), axis=-1).astype(np.float32)
    prompt_rng = rng if prompt_seed is None else np.random.default_rng(prompt_seed)
    prompts = prompt_rng.integers(0, c.vocab, (c.context, b), dtype=np.int32)
    arrays.update(tokens=prompts[0].copy(), position=np.array([0], dtype=np.int32),
                  history=np.full((t, b), -1, dtype=np.int32),
                  kc=np.full((l, b, c.heads, t, d), -12345, dtype=np.float32),
                  vc=np.full((l, b, c.heads, t, d), -12345, dtype=np.float32),
                  logits=np.full((b, c.vocab), -12345, dtype=np.float32))
    return arrays, prompts


def make_inputs(c, seed=123, *, init="reference", prompt_seed=None):
    """Inputs of the first measured step: prefill the first context-1 prompt tokens."""
    arrays, prompts = initial_state(c, seed, init=init, prompt_seed=prompt_seed)
    for i in range(c.context - 1):
        step(arrays, c)
        arrays["tokens"][:] = prompts[i + 1]
    return arrays, prompts


def expected(initial, c, steps):
    result = {name: value.copy() if name in MUTABLE else value for name, value in initial.items()}
    for _ in range(steps):
        step(result, c)
    return result
