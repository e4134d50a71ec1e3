"""Device-side harness for the decoder workload: synthetic inputs, device state with sentinel
tails, compile/bind of the storage ablation, GPU prefill, and state verification.

The verification protocol is that of benchmarks/decoder/run.py:81-132 in the reference:
256-element sentinel tails after every buffer, exact integer state (tokens, history,
position), f32 state within atol 2e-5 / rtol 3e-4, unchanged weights, and unchanged KV-cache
prefix and suffix outside the positions a run writes.
"""
from __future__ import annotations

import time

import numpy as np

import ckl
from programs.decoder import decode
from programs.decoder_config import EPSILON, MUTABLE, Config, shapes, signature

TAIL = 256
SENTINEL = -12345
# The north star's logits tolerance: per request row, max |logits - reference| / max |reference|.
LOGITS_NORMWISE = 1e-4
WEIGHTS = ("emb", "norm1", "norm2", "final_norm", "wq", "wk", "wv", "wo", "wg", "wu", "wd", "lm")


def synthetic_inputs(c: Config, seed: int = 123, *, init: str = "baseline", prompt_seed: int = None):
    """Seeded weights, RoPE table, prompts and empty persistent state (no prefill).

    Draw order and distributions: weights in WEIGHTS order from default_rng(seed) (gains
    1 + N(0, 0.02); embedding and matrices N(0, 0.02) for init="baseline", or N(0, 0.5) and
    N(0, 0.5/sqrt(fan_in)) for init="reference"), then prompts integers(0, V, (context, B)) from
    the same generator, or from default_rng(prompt_seed) when given (independent requests that
    share the weights).
    """
    rng = np.random.default_rng(seed)
    sh = shapes(c)
    arrays = {}
    for name in WEIGHTS:
        shape = sh[name][0]
        if "norm" in name:
            arrays[name] = (1 + rng.normal(0, 0.02, shape)).astype(np.float32)
        elif init == "baseline":
            arrays[name] = rng.normal(0, 0.02, shape).astype(np.float32)
        elif init == "reference":
            arrays[name] = rng.normal(0, 0.5 if name == "emb" else 0.5 / np.sqrt(shape[-2]), shape).astype(np.float32)
        else:
            raise ValueError(f"unknown init {init!r}")
    d, t = c.head_dim, c.capacity
    angles = np.arange(t)[:, None] * (10000. ** (-np.arange(0, d, 2) / d))[None, :]
    arrays["sincos"] = np.stack((np.cos(angles), np.sin(angles)), axis=-1).astype(np.float32)
    prompt_rng = rng if prompt_seed is None else np.random.default_rng(prompt_seed)
    prompts = prompt_rng.integers(0, c.vocab, (c.context, c.batch), dtype=np.int32)
    arrays.update(tokens=prompts[0].copy(), position=np.array([0], dtype=np.int32),
                  history=np.full(sh["history"][0], -1, dtype=np.int32),
                  kc=np.full(sh["kc"][0], SENTINEL, dtype=np.float32),
                  vc=np.full(sh["vc"][0], SENTINEL, dtype=np.float32),
                  logits=np.full(sh["logits"][0], SENTINEL, dtype=np.float32))
    return arrays, prompts


def normwise_error(actual: np.ndarray, reference: np.ndarray) -> float:
    """max over rows of max|actual - reference| / max|reference| (rows of a [B, V] array)."""
    actual = np.asarray(actual, dtype=np.float64).reshape(reference.shape[0], -1)
    reference = np.asarray(reference, dtype=np.float64).reshape(reference.shape[0], -1)
    scale = np.max(np.abs(reference), axis=1)
    if np.any(scale == 0):
        raise AssertionError("a reference logits row is all zero; the normwise tolerance is undefined")
    return float(np.max(np.max(np.abs(actual - reference), axis=1) / scale))


class DecoderState:
    """Device copies of every program argument, each followed by a sentinel tail. With `shared`
    (another request's state), the read-only inputs (weights, RoPE table) are that state's
    buffers, which must hold the same values (benchmarks/decoder/run.py:81-101)."""

    def __init__(self, device: ckl.Device, c: Config, arrays: dict, *, shared: "DecoderState" = None):
        self.device, self.config = device, c
        self.initial = {k: v for k, v in arrays.items()}
        self.owners, self.buffers, self.host = {}, {}, {}
        for name, (shape, dtype) in shapes(c).items():
            values = arrays[name]
            if tuple(values.shape) != tuple(shape):
                raise ValueError(f"{name}: shape {values.shape} != {shape}")
            if shared is not None and name not in MUTABLE:
                if not np.array_equal(values, shared.initial[name]):
                    raise ValueError(f"cannot share different read-only input {name}")
                self.owners[name], self.host[name] = shared.owners[name], shared.host[name]
                self.buffers[name] = shared.buffers[name]
                continue
            host = np.full(values.size + TAIL, SENTINEL, dtype=values.dtype)
            host[:values.size] = values.ravel()
            kind = ckl.i32 if dtype == "i32" else ckl.f32
            owner = device.empty(ckl.BufferSpec(host.shape, kind))
            owner.copy_from_host(host)
            self.owners[name], self.host[name] = owner, host
            self.buffers[name] = device.import_buffer(owner.address, ckl.BufferSpec(tuple(shape), kind), owner=owner)

    def arguments(self):
        c = self.config
        args = [self.buffers[name] for name in shapes(c)]
        return args + [float(np.float32(EPSILON)), float(c.head_dim ** -0.5)]

    def reset(self, names=MUTABLE):
        for name in names:
            self.owners[name].copy_from_host(self.host[name])

    def set_tokens(self, tokens: np.ndarray):
        self.buffers["tokens"].copy_from_host(np.ascontiguousarray(tokens, dtype=np.int32))

    def download(self, name: str, *, with_tail=False) -> np.ndarray:
        out = np.empty_like(self.host[name])
        self.owners[name].copy_to_host(out)
        if with_tail:
            return out
        return out[:self.initial[name].size].reshape(self.initial[name].shape)

    def snapshot(self):
        """Make the current device state the reset point (after a device prefill)."""
        for name in MUTABLE:
            full = self.download(name, with_tail=True)
            self.host[name] = full
            self.initial[name] = full[:self.initial[name].size].reshape(self.initial[name].shape).copy()

    def verify(self, reference: dict, *, check_weights=True) -> float:
        """Compare device state with `reference` (arrays after the same steps). Returns the
        maximum f32 error; raises AssertionError on any violation. Besides run.py:124's
        elementwise allclose, the logits must agree per row within LOGITS_NORMWISE relative to the
        row's largest reference magnitude; that figure is kept in `self.logits_normwise`."""
        errors = {}
        self.logits_normwise = None
        start, end = int(self.initial["position"][0]), int(reference["position"][0])
        for name in shapes(self.config):
            if name not in MUTABLE and not check_weights:
                continue
            actual = self.download(name, with_tail=True)
            size = self.initial[name].size
            if not np.all(actual[size:] == SENTINEL):
                raise AssertionError(f"{name}: tail overwritten")
            actual = actual[:size].reshape(self.initial[name].shape)
            if name not in MUTABLE:
                if not np.array_equal(actual, self.initial[name]):
                    raise AssertionError(f"{name}: model weights/input metadata changed")
            elif actual.dtype == np.int32:
                if not np.array_equal(actual, reference[name]):
                    raise AssertionError(f"{name}: token/history/position mismatch\n{actual}\n{reference[name]}")
            else:
                if not np.all(np.isfinite(actual)) or not np.allclose(actual, reference[name], atol=2e-5, rtol=3e-4):
                    raise AssertionError(f"{name}: numerical mismatch, max error {np.max(np.abs(actual - reference[name]))}")
                errors[name] = float(np.max(np.abs(actual - reference[name])))
                if name == "logits":
                    self.logits_normwise = normwise_error(actual, reference[name])
                    if self.logits_normwise > LOGITS_NORMWISE:
                        raise AssertionError(f"logits: row-normwise error {self.logits_normwise:.3e} > {LOGITS_NORMWISE}")
                if name in ("kc", "vc"):
                    if not np.array_equal(actual[:, :, :, :start], self.initial[name][:, :, :, :start]):
                        raise AssertionError(f"{name}: prefilled cache changed")
                    if not np.array_equal(actual[:, :, :, end:], self.initial[name][:, :, :, end:]):
                        raise AssertionError(f"{name}: unused cache suffix changed")
        return max(errors.values(), default=0.0)

    def verify_generation(self, expected: dict, *, full: bool, longest: int) -> dict:
        """Check the state after a generation of `expected["steps"]` steps from the reset point
        (the checks of benchmarks/decoder/run.py:107-132 that a timed sample can fail): tokens,
        history and position exact; logits finite, within atol 2e-5 / rtol 3e-4 and the
        row-normwise LOGITS_NORMWISE; those buffers' sentinel tails intact. With `full`, also the
        cache rows the generation wrote (same tolerance), the prefill rows before them and every
        row past the longest generation (`longest` steps) unchanged, and the caches' tails.
        `expected` holds tokens, history, position, logits and the written cache rows
        (kc_rows, vc_rows: [L, B, A, steps, D]). Returns the largest errors."""
        out = self.check_capture(self.capture(), expected)
        if not full:
            return out
        return {**out, **self._verify_caches(expected, longest)}

    def capture(self) -> dict:
        """Download what every generation is checked on (tokens, history, position, logits, with
        their sentinel tails), so that the check can run later (check_capture)."""
        return {name: self.download(name, with_tail=True) for name in ("tokens", "history", "position", "logits")}

    def check_capture(self, captured: dict, expected: dict) -> dict:
        """The checks of verify_generation without `full` on a capture() taken after the
        generation. Returns the largest logits errors."""
        out = {}
        for name in ("tokens", "history", "position", "logits"):
            actual = captured[name]
            size = self.initial[name].size
            if not np.all(actual[size:] == SENTINEL):
                raise AssertionError(f"{name}: tail overwritten")
            actual = actual[:size].reshape(self.initial[name].shape)
            if name != "logits":
                if not np.array_equal(actual, expected[name]):
                    raise AssertionError(f"{name}: mismatch after {expected['steps']} steps")
                continue
            if not np.all(np.isfinite(actual)) or not np.allclose(actual, expected[name], atol=2e-5, rtol=3e-4):
                raise AssertionError(f"logits: numerical mismatch, max error {np.max(np.abs(actual - expected[name]))}")
            out["logits_max_abs"] = float(np.max(np.abs(actual - expected[name])))
            out["logits_normwise"] = normwise_error(actual, expected[name])
            if out["logits_normwise"] > LOGITS_NORMWISE:
                raise AssertionError(f"logits: row-normwise error {out['logits_normwise']:.3e} > {LOGITS_NORMWISE}")
        return out

    def _verify_caches(self, expected: dict, longest: int) -> dict:
        out = {}
        start, steps = int(self.initial["position"][0]), int(expected["steps"])
        for name in ("kc", "vc"):
            actual = self.download(name, with_tail=True)
            size = self.initial[name].size
            if not np.all(actual[size:] == SENTINEL):
                raise AssertionError(f"{name}: tail overwritten")
            actual = actual[:size].reshape(self.initial[name].shape)
            initial = self.initial[name]
            for layer in range(actual.shape[0]):      # one layer at a time bounds the temporaries
                if not np.array_equal(actual[layer, :, :, :start], initial[layer, :, :, :start]):
                    raise AssertionError(f"{name}: prefilled cache changed (layer {layer})")
                if not np.array_equal(actual[layer, :, :, start + longest:], initial[layer, :, :, start + longest:]):
                    raise AssertionError(f"{name}: unused cache suffix changed (layer {layer})")
            rows = actual[:, :, :, start:start + steps]
            reference = expected[f"{name}_rows"]
            if not np.all(np.isfinite(rows)) or not np.allclose(rows, reference, atol=2e-5, rtol=3e-4):
                raise AssertionError(f"{name}: written rows differ, max error {np.max(np.abs(rows - reference))}")
            out[f"{name}_max_abs"] = float(np.max(np.abs(rows - reference)))
        return out

    def verify_read_only(self) -> None:
        """Weights, RoPE table and every sentinel tail unchanged (run.py:114-120)."""
        for name in shapes(self.config):
            actual = self.download(name, with_tail=True)
            size = self.initial[name].size
            if not np.all(actual[size:] == SENTINEL):
                raise AssertionError(f"{name}: tail overwritten")
            if name not in MUTABLE and not np.array_equal(actual[:size].reshape(self.initial[name].shape),
                                                          self.initial[name]):
                raise AssertionError(f"{name}: model weights/input metadata changed")


class DecoderSession:
    """Lowered decode program compiled with storage reuse off and on, bound to one state."""

    def __init__(self, c: Config, device: ckl.Device = None, *, arrays=None, seed=123, init="baseline"):
        self.config = c
        self.device = device or ckl.Device()
        if arrays is None:
            arrays, self.prompts = synthetic_inputs(c, seed, init=init)
        else:
            self.prompts = None
        start = time.perf_counter()
        self.lowered = decode.lower(signature=signature(c))
        lowered = time.perf_counter()
        self.programs = {}
        self.compile_ms = {}
        for reuse in (False, True):
            begin = time.perf_counter()
            self.programs[reuse] = self.lowered.compile(fuse_pointwise=False, reuse_storage=reuse)
            self.compile_ms[reuse] = (time.perf_counter() - begin) * 1e3
        # Host planning cost (frontend lowering; native graph, storage plan and executable plan).
        self.lower_ms = (lowered - start) * 1e3
        self.state = DecoderState(self.device, c, arrays)
        self.invocations = {reuse: p.bind(*self.state.arguments()) for reuse, p in self.programs.items()}
        expected_nodes = 21 * c.layers + 6
        for inv in self.invocations.values():
            if inv.node_count != expected_nodes:
                raise AssertionError("unexpected decoder dispatch count")
        if self.programs[False].prepared_ir != self.programs[True].prepared_ir:
            raise AssertionError("storage ablation changed the prepared device kernels")

    def prefill(self, prompts: np.ndarray, *, mode="graph", progress=None):
        """Teacher-forced device prefill of context-1 steps (reference.py:102-106 semantics):
        each step runs the decode program, then the next prompt token replaces the argmax.
        `progress(done, total)` is called every 128 steps when given."""
        inv = self.invocations[True]
        total = self.config.context - 1
        for i in range(total):
            inv.run(mode=mode)
            self.state.set_tokens(prompts[i + 1])
            if progress and (i + 1) % 128 == 0:
                progress(i + 1, total)
        self.state.snapshot()


class RequestGroup:
    """Independent requests of one configuration (benchmarks/decoder/experiment.py:20-50): one
    compiled decode program; the read-only weights and RoPE table allocated once and shared; per
    request its own prompt and mutable state (tokens, position, history, caches, logits) and an
    invocation with its own stream, heaps and workspaces."""

    def __init__(self, c: Config, device: ckl.Device, arrays: list, *, reuse: bool = True):
        self.config, self.device = c, device
        self.states = []
        for values in arrays:
            self.states.append(DecoderState(device, c, values, shared=self.states[0] if self.states else None))
        self.program = decode.lower(signature=signature(c)).compile(fuse_pointwise=False, reuse_storage=reuse)
        self.invocations = [self.program.bind(*state.arguments()) for state in self.states]

    def reset(self):
        for state in self.states:
            state.reset()

    def run(self, *, mode="graph", iterations=1, batch_size=1, serial=False) -> dict:
        return ckl.run_requests(self.invocations, mode=mode, iterations=iterations, batch_size=batch_size,
                                serial=serial)

    def prefill(self, prompts: list):
        """Teacher-forced device prefill of every request (context-1 steps, the requests side by
        side), then the prefilled state becomes each request's reset point."""
        for i in range(self.config.context - 1):
            self.run(mode="graph")
            for state, p in zip(self.states, prompts):
                state.set_tokens(p[i + 1])
        for state in self.states:
            state.snapshot()

