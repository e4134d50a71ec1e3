"""The add -> rms_stats -> rms_apply chain on rows of every register shape (csrc/kernels/library.hip
row_registers: 1 to 4 float4 per thread, and the loop path past 4096 floats), with both add
operands the partial planes of split linears (B = 32: each MFMA projection of x_j splits its
512-row reduction in two and defers the combine to the chain) or plain rows (B = 5: one-slice
row-parallel projections). The inferred graph (chains, deferred combines) must leave exactly the
bits of the ordinary launches; both must match a float64 NumPy restatement of
benchmarks/decoder/workloads.py:42-69, 145-150 within the fp32 tolerance of a 512-term sum."""
import numpy as np
import pytest

import ckl
from programs.decoder import add, linear, rms_apply, rms_stats

pytestmark = pytest.mark.gpu

_B, _I, _C, _L = ckl.dim("B"), ckl.dim("I"), ckl.dim("C"), ckl.dim("L")
_X = ckl.Buffer[ckl.f32, (_B, _I)]
_W = ckl.Buffer[ckl.f32, (_L, _I, _C)]
_H = ckl.Buffer[ckl.f32, (_B, _C)]
_G = ckl.Buffer[ckl.f32, (_L, _C)]
EPSILON = np.float32(1e-5)


@ckl.program
def residual_norm(x1: _X, w1: _W, x2: _X, w2: _W, h: _H, out: _H, gain: _G, epsilon: ckl.f32,
                  layer: ckl.constexpr[ckl.index]) -> None:
    y1 = ckl.empty_like(h)
    y2 = ckl.empty_like(h)
    ckl.launch(linear, x1, w1, y1, layer, grid=(ckl.cdiv(_C, 64), _B), block=(64,))
    ckl.launch(linear, x2, w2, y2, layer, grid=(ckl.cdiv(_C, 64), _B), block=(64,))
    ckl.launch(add, y1, y2, h, grid=(ckl.cdiv(_C, 64), _B), block=(64,))
    inv = ckl.empty((_B,), dtype=ckl.f32)
    ckl.launch(rms_stats, h, inv, epsilon, grid=(ckl.cdiv(_B, 32),), block=(32,))
    ckl.launch(rms_apply, h, inv, gain, out, layer, grid=(ckl.cdiv(_C, 64), _B), block=(64,))


@pytest.mark.parametrize("b,c", [(32, 1024), (32, 3072), (32, 4096), (32, 4100), (5, 3072)],
                         ids=["planes_r1", "planes_r3", "planes_r4", "planes_loop", "rows_r3"])
def test_add_rms_chain_matches_ordinary_and_float64(device, b, c):
    i, layers, layer = 512, 2, 1
    rng = np.random.default_rng(b * 131 + c)
    arrays = {"x1": rng.standard_normal((b, i)), "w1": rng.standard_normal((layers, i, c)) / np.sqrt(i),
              "x2": rng.standard_normal((b, i)), "w2": rng.standard_normal((layers, i, c)) / np.sqrt(i),
              "gain": 1 + 0.1 * rng.standard_normal((layers, c))}
    arrays = {k: v.astype(np.float32) for k, v in arrays.items()}
    signature = {k: ckl.BufferSpec(v.shape, ckl.f32) for k, v in arrays.items()}
    signature.update(h=ckl.BufferSpec((b, c), ckl.f32), out=ckl.BufferSpec((b, c), ckl.f32),
                     epsilon=ckl.f32)
    compiled = residual_norm.lower(signature=signature, constants={"layer": layer}).compile(fuse_pointwise=False)
    buffers = {k: device.empty(signature[k]) for k in ("x1", "w1", "x2", "w2", "gain", "h", "out")}
    for k, v in arrays.items():
        buffers[k].copy_from_host(v)
    bound = compiled.bind(buffers["x1"], buffers["w1"], buffers["x2"], buffers["w2"], buffers["h"], buffers["out"],
                          buffers["gain"], float(EPSILON))
    assert any(name.startswith("ckl_add__rms_stats__rms_apply") for name, _ in bound.units())
    h64 = (arrays["x1"].astype(np.float64) @ arrays["w1"][layer].astype(np.float64) +
           arrays["x2"].astype(np.float64) @ arrays["w2"][layer].astype(np.float64))
    out64 = h64 / np.sqrt(np.mean(h64 * h64, axis=1, keepdims=True) + float(EPSILON)) * arrays["gain"][layer]
    results = {}
    for mode in ("ordinary", "graph", "graph"):
        for k in ("h", "out"):
            buffers[k].copy_from_host(np.full((b, c), np.nan, np.float32))
        bound.run(mode=mode)
        got = {}
        for k in ("h", "out"):
            got[k] = np.empty((b, c), np.float32)
            buffers[k].copy_to_host(got[k])
        for k, ref in (("h", h64), ("out", out64)):
            assert np.allclose(got[k], ref, rtol=1e-4, atol=1e-4 * np.sqrt(i)), (mode, k, float(np.max(np.abs(got[k] - ref))))
        if mode in results:
            assert all(np.array_equal(got[k], results[mode][k]) for k in got), "graph replays differ"
        results.setdefault(mode, got)
    for k in ("h", "out"):
        assert np.array_equal(results["graph"][k], results["ordinary"][k]), k
