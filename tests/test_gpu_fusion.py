"""Fused pointwise chains on the GPU (tests/Runtime/test_pointwise_fusion.py of the reference):
exact results of the fused kernel against the unfused program, the bind-time fallback to the
unfused program when external buffers overlap (shifted or identical), adjacent disjoint slices
keeping the fused topology, and f32 rounding kept across the removed store (no contraction)."""
import numpy as np
import pytest

import ckl
from fusion_programs import scale_offset
from programs import vector_pipeline

pytestmark = pytest.mark.gpu
SENTINEL = np.float32(-12345)


@pytest.mark.parametrize("n", [257, 1048576])
def test_fused_vector_pipeline_and_overlap_fallback(device, n):
    spec = ckl.BufferSpec((n,), ckl.f32)
    module = vector_pipeline.lower(n)
    fused, baseline = module.compile(), module.compile(fuse_pointwise=False)
    initial = ((np.arange(n) % 97) / 128).astype(np.float32)
    expected = (initial + np.float32(0.125)) + np.float32(0.125)
    src, dst = device.empty(spec), device.empty(spec)
    for compiled, nodes in ((fused, 1), (baseline, 2)):
        src.copy_from_host(initial)
        invocation = compiled.bind(src, dst, 0.125)
        assert invocation.node_count == nodes
        for mode in ("ordinary", "graph", "capture"):
            dst.copy_from_host(np.zeros(n, np.float32))
            invocation.run(mode=mode)
            actual = np.empty(n, np.float32)
            dst.copy_to_host(actual)
            assert np.array_equal(actual, expected), (nodes, mode)

    # dst shifted one element past src inside one allocation: the original two launches run.
    owner = device.empty(ckl.BufferSpec((n + 2,), ckl.f32))
    overlap_src = device.import_buffer(owner.address, spec, owner=owner)
    overlap_dst = device.import_buffer(owner.address + 4, spec, owner=owner)
    full = np.concatenate([initial, [SENTINEL, SENTINEL]]).astype(np.float32)
    wanted = np.concatenate([initial[:1], expected, [SENTINEL]]).astype(np.float32)
    overlap = fused.bind(overlap_src, overlap_dst, 0.125)
    assert overlap.node_count == 2
    for mode in ("ordinary", "graph"):
        owner.copy_from_host(full)
        overlap.run(mode=mode)
        got = np.empty(n + 2, np.float32)
        owner.copy_to_host(got)
        assert np.array_equal(got, wanted), mode

    # Adjacent disjoint slices of one allocation keep the fused topology.
    adjacent_owner = device.empty(ckl.BufferSpec((2 * n,), ckl.f32))
    adjacent_src = device.import_buffer(adjacent_owner.address, spec, owner=adjacent_owner)
    adjacent_dst = device.import_buffer(adjacent_owner.address + 4 * n, spec, owner=adjacent_owner)
    adjacent_src.copy_from_host(initial)
    adjacent = fused.bind(adjacent_src, adjacent_dst, 0.125)
    assert adjacent.node_count == 1
    adjacent.run(mode="graph")
    got = np.empty(n, np.float32)
    adjacent_dst.copy_to_host(got)
    assert np.array_equal(got, expected)

    # The same buffer as source and destination.
    exact = fused.bind(src, src, 0.125)
    assert exact.node_count == 2
    src.copy_from_host(initial)
    exact.run(mode="graph")
    src.copy_to_host(got)
    assert np.array_equal(got, expected)


def test_fusion_keeps_f32_rounding_of_the_removed_store(device):
    """(1 + 2^-23)(1 - 2^-23) rounds to 1 in f32, so the fused multiply-then-shift by -1 gives
    exactly 0; a contracted fma would give -2^-46."""
    spec = ckl.BufferSpec((257,), ckl.f32)
    program = scale_offset.lower(signature={"src": spec, "dst": spec, "factor": ckl.f32, "bias": ckl.f32}).compile()
    src, dst = device.empty(spec), device.empty(spec)
    src.copy_from_host(np.full(257, 1 + 2 ** -23, np.float32))
    invocation = program.bind(src, dst, 1 - 2 ** -23, -1.0)
    assert invocation.node_count == 1
    for mode in ("ordinary", "graph"):
        dst.copy_from_host(np.ones(257, np.float32))
        invocation.run(mode=mode)
        got = np.empty(257, np.float32)
        dst.copy_to_host(got)
        assert got.tobytes() == np.zeros(257, np.float32).tobytes(), mode
