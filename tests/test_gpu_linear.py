"""The linear kernel family on the GPU (benchmarks/decoder/workloads.py:61-69 body):
dst[b, o] = sum_i x[b, i] * w[layer, i, o], against a float64 NumPy product.

Shapes cover the vector path (B <= 16), the f32 MFMA paths (J = 1, 2 and 4 columns per lane),
split reductions across workgroups (the workspace and its completion counters, replayed so the
self-resetting counters are exercised), ragged K/O/B tails and more than one 32-row batch
tile. Tolerance: fp32 accumulation of I products of N(0, 1) inputs, |err| <= 1e-5 * sqrt(I)
relative to the row scale (the decoder-level check is the oracle comparison in
test_gpu_decoder.py)."""
import numpy as np
import pytest

import ckl
from ckl.library import linear_tiling
from ckl.decoder_kernels import linear

pytestmark = pytest.mark.gpu

SHAPES = [
    (8, 64, 64), (8, 256, 64), (8, 1024, 256), (3, 48, 129), (16, 130, 70),   # vector path
    (32, 2048, 2048), (32, 5632, 2048), (32, 2048, 5632),                    # MFMA, J = 1, split K
    (32, 2048, 32000),                                                        # MFMA, J = 4
    (20, 100, 36), (40, 72, 260), (17, 2052, 20000), (64, 256, 96),          # tails, row tiles
]


_B, _I, _O, _L = ckl.dim("B"), ckl.dim("I"), ckl.dim("O"), ckl.dim("L")
_X = ckl.Buffer[ckl.f32, (_B, _I)]
_W = ckl.Buffer[ckl.f32, (_L, _I, _O)]
_Y = ckl.Buffer[ckl.f32, (_B, _O)]


@ckl.program
def project(x: _X, w: _W, y: _Y, z: _Y, layer: ckl.constexpr[ckl.index]) -> None:
    # Two projections of one x into caller buffers that may alias (so they run in order).
    ckl.launch(linear, x, w, y, layer, grid=(ckl.cdiv(_O, 64), _B), block=(64,))
    ckl.launch(linear, x, w, z, layer, grid=(ckl.cdiv(_O, 64), _B), block=(64,))


def program_for(b, i, o, layers, layer):
    signature = {"x": ckl.BufferSpec((b, i), ckl.f32), "w": ckl.BufferSpec((layers, i, o), ckl.f32),
                 "y": ckl.BufferSpec((b, o), ckl.f32), "z": ckl.BufferSpec((b, o), ckl.f32)}
    return project.lower(signature=signature, constants={"layer": layer}).compile(fuse_pointwise=False)


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_linear_matches_float64(device, shape):
    b, i, o = shape
    layers, layer = 2, 1
    compiled = program_for(b, i, o, layers, layer)
    tiling = linear_tiling(b, i, o)
    assert f'"{tiling["entry"]}"' in compiled.executable_ir
    rng = np.random.default_rng(b * 7919 + i * 31 + o)
    x = rng.standard_normal((b, i)).astype(np.float32)
    w = rng.standard_normal((layers, i, o)).astype(np.float32)
    expected = x.astype(np.float64) @ w[layer].astype(np.float64)
    buffers = {}
    for name, values in (("x", x), ("w", w)):
        buffers[name] = device.empty(ckl.BufferSpec(values.shape, ckl.f32))
        buffers[name].copy_from_host(values)
    for name in ("y", "z"):
        buffers[name] = device.empty(ckl.BufferSpec((b, o), ckl.f32))
    bound = compiled.bind(buffers["x"], buffers["w"], buffers["y"], buffers["z"])
    first = None
    for mode in ("ordinary", "graph", "capture", "graph"):
        for name in ("y", "z"):
            buffers[name].copy_from_host(np.full((b, o), np.nan, np.float32))
        bound.run(mode=mode, batch_size=2)
        for name in ("y", "z"):
            got = np.empty((b, o), np.float32)
            buffers[name].copy_to_host(got)
            scale = np.sqrt(i) * 1e-5 * (1 + np.abs(expected))
            assert np.all(np.abs(got - expected) <= scale), (mode, name, float(np.max(np.abs(got - expected))))
            if first is None:
                first = got
            else:
                assert np.array_equal(got, first), "linear results must be deterministic across runs and modes"
