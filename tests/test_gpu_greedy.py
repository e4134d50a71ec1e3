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
from programs.decoder import History, Logits, Position, Tokens, advance, greedy
from programs.decoder import B as _B
from test_oracle_decoder import edge_rows

pytestmark = pytest.mark.gpu


@ckl.program
def pick(logits: Logits, tokens: Tokens, history: History, position: Position) -> None:
    ckl.launch(greedy, logits, tokens, history, position, grid=(ckl.cdiv(_B, 32),), block=(32,))
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
