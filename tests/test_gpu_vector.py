"""vector_pipeline on the GPU: dst = (src + bias) + bias, exact in f32, through every run mode,
with storage reuse of the temporary (tests/Runtime/test_frontend_runtime.py:63-177 analogue)."""
import numpy as np
import pytest

import ckl
from programs import vector_pipeline

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [257, 1048576])
def test_vector_pipeline_all_modes(device, n):
    compiled = vector_pipeline.lower(n).compile(fuse_pointwise=False)
    assert "ckl.hip.library.update" in compiled.executable_ir
    assert "dependencies = array<i64: 1>" in compiled.executable_ir
    spec = ckl.BufferSpec((n,), ckl.f32)
    full = ckl.BufferSpec((n + 256,), ckl.f32)
    src_owner, dst_owner = device.empty(full), device.empty(full)
    src = device.import_buffer(src_owner.address, spec, owner=src_owner)
    dst = device.import_buffer(dst_owner.address, spec, owner=dst_owner)
    rng = np.random.default_rng(7)
    initial = np.concatenate([rng.uniform(-1, 1, n).astype(np.float32), np.full(256, -12345, np.float32)])
    src_owner.copy_from_host(initial)
    blank = np.full(n + 256, -12345, np.float32)
    for bias in (0.5, -0.125):
        bound = compiled.bind(src, dst, bias)
        assert bound.node_count == 2
        b = np.float32(bias)
        expected = np.concatenate([(initial[:n] + b) + b, blank[n:]])
        for mode in ("ordinary", "graph", "capture", "graph"):
            dst_owner.copy_from_host(blank)
            bound.run(mode=mode)
            actual = np.empty_like(blank)
            dst_owner.copy_to_host(actual)
            assert np.array_equal(actual, expected), mode
        for mode in ("ordinary", "graph", "capture"):
            timing = bound.benchmark(iterations=3, mode=mode, batch_size=2)
            assert timing["stream_us"] > 0 and timing["wall_us"] > 0


def test_vector_pipeline_jit_kernel(device):
    """A kernel body outside the library is compiled from its IR (hipRTC) and runs exactly."""
    N = ckl.dim("N")
    Vec = ckl.Buffer[ckl.f32, (N,)]

    @ckl.kernel
    def scale_shift(src: Vec, dst: Vec, bias: ckl.f32) -> None:
        i = ckl.global_id(0)
        if i < N:
            dst[i] = src[i] * 2.0 + bias

    @ckl.program
    def run(src: Vec, dst: Vec, bias: ckl.f32) -> None:
        ckl.launch(scale_shift, src, dst, bias, grid=(ckl.cdiv(N, 64),), block=(64,))

    spec = ckl.BufferSpec((1000,), ckl.f32)
    compiled = run.lower(signature={"src": spec, "dst": spec, "bias": ckl.f32}).compile()
    assert "__global__" in compiled.device_ir
    src, dst = device.empty(spec), device.empty(spec)
    x = np.linspace(-3, 3, 1000, dtype=np.float32)
    src.copy_from_host(x)
    for mode in ("ordinary", "graph", "capture"):
        compiled.bind(src, dst, 0.25).run(mode=mode)
        out = np.empty_like(x)
        dst.copy_to_host(out)
        assert np.array_equal(out, x * np.float32(2) + np.float32(0.25)), mode
