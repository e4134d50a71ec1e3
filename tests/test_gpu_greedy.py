"""The greedy and advance kernels on the GPU (benchmarks/decoder/workloads.py:170-188): tokens,
history row and position against the oracle's scan (oracle.decoder.greedy_scan, pinned to the
kernel body's loop on the CPU) on rows with ties, NaN, -0/+0 and -inf. Vocabulary sizes cover
every path of the library kernel: one 256-thread workgroup per row with float4 loads (V = 256),
the scalar path (V = 129), one 1024-thread workgroup per row (V = 32000) and rows cut into
4096-logit slices combined through the workspace (V = 40000, 10 slices). The ordinary launches
run greedy then advance; the inferred graph runs the greedy -> advance chain. Bit-exact."""
import numpy as np
import pytest

import ckl
from oracle import decoder as oracle
from ckl.decoder_kernels import BATCH, advance, greedy, linear
from ckl.decoder_kernels import Cursor as Position, Emitted as History, Logits, TokenIds as Tokens
from test_oracle_decoder import edge_rows

pytestmark = pytest.mark.gpu


@ckl.program
def pick(logits: Logits, tokens: Tokens, history: History, position: Position) -> None:
    ckl.launch(greedy, logits, tokens, history, position, grid=(ckl.cdiv(BATCH, 32),), block=(32,))
    ckl.launch(advance, position, grid=(1,), block=(1,))


@pytest.mark.parametrize("v", [256, 129, 32000, 40000])
def test_greedy_advance_match_the_scan(device, v):
    logits = edge_rows(v, np.random.default_rng(v))
    b, t = logits.shape[0], 6
    signature = {"logits": ckl.BufferSpec((b, v), ckl.f32), "tokens": ckl.BufferSpec((b,), ckl.i32),
                 "history": ckl.BufferSpec((t, b), ckl.i32), "position": ckl.BufferSpec((1,), ckl.i32)}
    compiled = pick.lower(signature=signature).compile(fuse_pointwise=False)
    buffers = {name: device.empty(spec) for name, spec in signature.items()}
    buffers["logits"].copy_from_host(logits)
    bound = compiled.bind(*(buffers[n] for n in ("logits", "tokens", "history", "position")))
    expected = oracle.greedy_scan(logits)
    for mode, start in (("ordinary", 0), ("graph", 2), ("capture", 4)):
        buffers["tokens"].copy_from_host(np.full(b, -7, np.int32))
        buffers["history"].copy_from_host(np.full((t, b), -7, np.int32))
        buffers["position"].copy_from_host(np.array([start], np.int32))
        for _ in range(2):                   # a replay finds the workspace counters reset
            bound.run(mode=mode)
        tokens, history, position = np.empty(b, np.int32), np.empty((t, b), np.int32), np.empty(1, np.int32)
        buffers["tokens"].copy_to_host(tokens)
        buffers["history"].copy_to_host(history)
        buffers["position"].copy_to_host(position)
        assert np.array_equal(tokens, expected), (mode, tokens, expected)
        rows = np.full((t, b), -7, np.int32)
        rows[start:start + 2] = expected
        assert np.array_equal(history, rows), mode
        assert position[0] == start + 2, mode


_BB, _I, _V, _W = ckl.dim("B"), ckl.dim("I"), ckl.dim("V"), ckl.dim("W")


@ckl.program
def project_pick(x: ckl.Buffer[ckl.f32, (_BB, _I)], w: ckl.Buffer[ckl.f32, (_W, _I, _V)],
                 logits: ckl.Buffer[ckl.f32, (_BB, _V)], tokens: ckl.Buffer[ckl.i32, (_BB,)],
                 history: ckl.Buffer[ckl.i32, (ckl.dim("T"), _BB)], position: ckl.Buffer[ckl.i32, (1,)]) -> None:
    ckl.launch(linear, x, w, logits, 0, grid=(ckl.cdiv(_V, 64), _BB), block=(64,))
    ckl.launch(greedy, logits, tokens, history, position, grid=(ckl.cdiv(_BB, 32),), block=(32,))
    ckl.launch(advance, position, grid=(1,), block=(1,))


@pytest.mark.parametrize("v", [256, 70])
def test_linear_greedy_chain_matches_ordinary_and_the_scan(device, v):
    """A single-wave LM head feeding greedy -> advance runs as one workgroup per row in the inferred
    graph (logits in registers); its logits, tokens, history and position must equal the ordinary
    launches' and its tokens the scan of those logits. One-hot x rows pick W rows with a tie at the
    maximum, a +inf column (NaN in the other rows: 0 * inf), a NaN column and -0/+0 entries; one x
    row is all zeros."""
    b, i, t = 6, 64, 5
    rng = np.random.default_rng(v)
    w = rng.standard_normal((1, i, v)).astype(np.float32)
    w[0, 1, [10, v - 6]] = 50.0                     # row picking W[1]: equal maxima
    w[0, 2, 7] = np.inf                             # row picking W[2]: +inf wins; NaN elsewhere
    w[0, 3, 3] = np.nan                             # column 3: NaN in every row
    w[0, 4, :] = -1.0
    w[0, 4, [20, 30]] = [-0.0, 0.0]
    x = np.zeros((b, i), np.float32)
    for row, k in enumerate([0, 1, 2, 4, 5]):
        x[row, k] = 1.0                             # x row 5 stays all zeros
    signature = {"x": ckl.BufferSpec((b, i), ckl.f32), "w": ckl.BufferSpec((1, i, v), ckl.f32),
                 "logits": ckl.BufferSpec((b, v), ckl.f32), "tokens": ckl.BufferSpec((b,), ckl.i32),
                 "history": ckl.BufferSpec((t, b), ckl.i32), "position": ckl.BufferSpec((1,), ckl.i32)}
    compiled = project_pick.lower(signature=signature).compile(fuse_pointwise=False)
    buffers = {name: device.empty(spec) for name, spec in signature.items()}
    buffers["x"].copy_from_host(x)
    buffers["w"].copy_from_host(w)
    bound = compiled.bind(*(buffers[n] for n in ("x", "w", "logits", "tokens", "history", "position")))
    assert any(name.startswith("ckl_linear_rowvec__greedy__advance") for name, _ in bound.units())
    results = {}
    for mode in ("ordinary", "graph"):
        buffers["logits"].copy_from_host(np.full((b, v), -7, np.float32))
        buffers["tokens"].copy_from_host(np.full(b, -7, np.int32))
        buffers["history"].copy_from_host(np.full((t, b), -7, np.int32))
        buffers["position"].copy_from_host(np.array([1], np.int32))
        for _ in range(2):
            bound.run(mode=mode)
        out = {"logits": np.empty((b, v), np.float32), "tokens": np.empty(b, np.int32),
               "history": np.empty((t, b), np.int32), "position": np.empty(1, np.int32)}
        for name, array in out.items():
            buffers[name].copy_to_host(array)
        assert np.array_equal(out["tokens"], oracle.greedy_scan(out["logits"])), mode
        assert out["position"][0] == 3 and np.array_equal(out["history"][1], out["tokens"]), mode
        results[mode] = out
    for name in ("logits", "tokens", "history", "position"):
        assert np.array_equal(results["graph"][name], results["ordinary"][name], equal_nan=name == "logits"), name
