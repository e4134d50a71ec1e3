"""Rebinding without re-instantiation (NvidiaGraphExecutable::updateKernel, lib/Runtime/
NvidiaRuntime.cpp:466-496; tested by tests/Runtime/NvidiaRuntimeValidation.cpp:279-289, which
checks an updated graph against ordinary launches of the updated plan): an invocation moved to
other buffers keeps its explicit graphs, whose kernel nodes get the new parameters in place, and
computes exactly what a fresh bind to those buffers computes."""
import numpy as np
import pytest

import ckl
from oracle import decoder as oracle
from programs import vector_pipeline
from programs.decoder_config import CONFIGS, MUTABLE
from programs.harness import DecoderState
from programs.decoder import decode
from programs.decoder_config import signature

pytestmark = pytest.mark.gpu


def vector_buffers(device, n, seed):
    spec = ckl.BufferSpec((n,), ckl.f32)
    src, dst = device.empty(spec), device.empty(spec)
    x = np.random.default_rng(seed).uniform(-1, 1, n).astype(np.float32)
    src.copy_from_host(x)
    dst.copy_from_host(np.full(n, -12345, np.float32))
    return src, dst, x


def read(buffer, n):
    out = np.empty(n, np.float32)
    buffer.copy_to_host(out)
    return out


@pytest.mark.parametrize("fuse", [False, True], ids=["unfused", "fused"])
def test_vector_pipeline_rebind_updates_graph_nodes(device, fuse):
    n = 1 << 16
    compiled = vector_pipeline.lower(n).compile(fuse_pointwise=fuse)
    src, dst, x = vector_buffers(device, n, 1)
    src2, dst2, x2 = vector_buffers(device, n, 2)
    inv = compiled.bind(src, dst, 0.5)
    for mode in ("graph", "branches", "capture"):
        inv.run(mode=mode)
    assert inv.graph_instantiations == 3
    assert np.array_equal(read(dst, n), (x + np.float32(0.5)) + np.float32(0.5))
    inv.rebind(src2, dst2, 0.5)
    before = read(dst, n)
    for mode in ("graph", "branches"):
        dst2.copy_from_host(np.full(n, -12345, np.float32))
        inv.run(mode=mode)
        assert np.array_equal(read(dst2, n), (x2 + np.float32(0.5)) + np.float32(0.5)), mode
    assert inv.graph_instantiations == 3, "explicit graphs are updated in place"
    dst2.copy_from_host(np.full(n, -12345, np.float32))
    inv.run(mode="capture")                       # captured graph: rebuilt for the new buffers
    assert inv.graph_instantiations == 4
    assert np.array_equal(read(dst2, n), (x2 + np.float32(0.5)) + np.float32(0.5))
    assert np.array_equal(read(dst, n), before), "the old buffers are no longer written"
    with pytest.raises(ValueError):
        inv.rebind(src, dst, 0.25)                # scalars are part of the plan: bind again
    inv.rebind(src, dst, 0.5)                     # and back
    inv.run(mode="graph")
    assert np.array_equal(read(dst, n), (x + np.float32(0.5)) + np.float32(0.5))


def test_fused_rebind_refuses_a_different_overlap(device):
    n = 4096
    compiled = vector_pipeline.lower(n).compile(fuse_pointwise=True)
    src, dst, _ = vector_buffers(device, n, 3)
    inv = compiled.bind(src, dst, 0.5)
    with pytest.raises(ValueError):
        inv.rebind(src, src, 0.5)                 # in place: the unfused fallback program


def test_decoder_rebind_matches_the_oracle(device):
    c = CONFIGS["small"]
    initial = [oracle.make_inputs(c, 123, init="baseline", prompt_seed=123 + i)[0] for i in range(2)]
    first = DecoderState(device, c, initial[0])
    second = DecoderState(device, c, initial[1])       # its own copies of every buffer
    program = decode.lower(signature=signature(c)).compile(fuse_pointwise=False)
    inv = program.bind(*first.arguments())
    references = [oracle.expected(s.initial, c, c.steps) for s in (first, second)]
    for mode in ("graph", "branches"):
        first.reset()
        inv.run(mode=mode, batch_size=c.steps)
        first.verify(references[0])
    built = inv.graph_instantiations
    inv.rebind(*second.arguments())
    for mode in ("graph", "branches"):
        second.reset()
        inv.run(mode=mode, batch_size=c.steps)
        second.verify(references[1])
        assert second.logits_normwise <= 1e-4
    assert inv.graph_instantiations == built, "the decode graphs keep their structure and are updated"
    fresh = program.bind(*second.arguments())
    second.reset()
    fresh.run(mode="graph", batch_size=c.steps)
    expected = {k: second.download(k) for k in MUTABLE}
    second.reset()
    inv.run(mode="graph", batch_size=c.steps)
    for k in MUTABLE:
        assert np.array_equal(second.download(k), expected[k]), k
