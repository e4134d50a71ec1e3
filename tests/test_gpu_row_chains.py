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
from ckl.decoder_kernels import add, embedding, linear, rms_apply, rms_stats

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


_T = ckl.dim("V")
_E = ckl.Buffer[ckl.f32, (_T, _C)]
_K = ckl.Buffer[ckl.i32, (_B,)]
_Q = ckl.Buffer[ckl.f32, (_L, _C, _C)]


@ckl.program
def embed_project(tokens: _K, table: _E, gain: _G, wq: _Q, wk: _Q, wv: _Q, x: _H, out: _H,
                  epsilon: ckl.f32, layer: ckl.constexpr[ckl.index]) -> None:
    # q, k, v are temporaries (as in the decoder): external outputs would be serialized by the
    # may-alias rule and could not share a launch.
    ckl.launch(embedding, tokens, table, x, grid=(ckl.cdiv(_C, 64), _B), block=(64,))
    inv = ckl.empty((_B,), dtype=ckl.f32)
    normed = ckl.empty_like(x)
    ckl.launch(rms_stats, x, inv, epsilon, grid=(ckl.cdiv(_B, 32),), block=(32,))
    ckl.launch(rms_apply, x, inv, gain, normed, layer, grid=(ckl.cdiv(_C, 64), _B), block=(64,))
    q = ckl.empty_like(x)
    k = ckl.empty_like(x)
    v = ckl.empty_like(x)
    ckl.launch(linear, normed, wq, q, layer, grid=(ckl.cdiv(_C, 64), _B), block=(64,))
    ckl.launch(linear, normed, wk, k, layer, grid=(ckl.cdiv(_C, 64), _B), block=(64,))
    ckl.launch(linear, normed, wv, v, layer, grid=(ckl.cdiv(_C, 64), _B), block=(64,))
    qk = ckl.empty_like(x)
    ckl.launch(add, q, k, qk, grid=(ckl.cdiv(_C, 64), _B), block=(64,))
    ckl.launch(add, qk, v, out, grid=(ckl.cdiv(_C, 64), _B), block=(64,))


@pytest.mark.parametrize("c", [64, 48])
def test_embedding_rms_qkv_launch_matches_ordinary(device, c):
    """embedding -> rms_stats -> rms_apply and the three one-slice row-parallel q, k, v linears run as
    one launch in the inferred graph (C <= 64): the embedded rows and q + k + v, including the NaN
    rows of out-of-range tokens (workloads.py:33-39 writes NaN for them), must be the ordinary
    launches' bits."""
    b, vocab, layers, layer = 7, 50, 2, 1
    rng = np.random.default_rng(c)
    arrays = {"tokens": np.array([3, -1, 49, 50, 0, 17, 3], np.int32),
              "table": rng.standard_normal((vocab, c)).astype(np.float32),
              "gain": (1 + 0.1 * rng.standard_normal((layers, c))).astype(np.float32)}
    for name in ("wq", "wk", "wv"):
        arrays[name] = (rng.standard_normal((layers, c, c)) / np.sqrt(c)).astype(np.float32)
    signature = {k: ckl.BufferSpec(v.shape, ckl.i32 if v.dtype == np.int32 else ckl.f32) for k, v in arrays.items()}
    outputs = ("x", "out")
    signature.update({name: ckl.BufferSpec((b, c), ckl.f32) for name in outputs})
    signature["epsilon"] = ckl.f32
    compiled = embed_project.lower(signature=signature, constants={"layer": layer}).compile(fuse_pointwise=False)
    buffers = {k: device.empty(signature[k]) for k in list(arrays) + list(outputs)}
    for k, value in arrays.items():
        buffers[k].copy_from_host(value)
    order = ("tokens", "table", "gain", "wq", "wk", "wv", "x", "out")
    bound = compiled.bind(*(buffers[n] for n in order), float(EPSILON))
    assert any(name.startswith("ckl_embedding__rms_stats__rms_apply__linear_rowvec") for name, _ in bound.units())
    results = {}
    for mode in ("ordinary", "graph"):
        for name in outputs:
            buffers[name].copy_from_host(np.full((b, c), 7.0, np.float32))
        bound.run(mode=mode)
        results[mode] = {}
        for name in outputs:
            results[mode][name] = np.empty((b, c), np.float32)
            buffers[name].copy_to_host(results[mode][name])
    for name in outputs:
        got, ref = results["graph"][name], results["ordinary"][name]
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), name
    out = results["graph"]["out"]
    assert np.isnan(out[[1, 3]]).all() and not np.isnan(out[[0, 2, 4, 5, 6]]).any()
