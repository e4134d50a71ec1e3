"""Library chains in the inferred graph (csrc/runtime/chains.cpp): contracted launches leave exactly
the state the ordinary launches leave, bit for bit, the decode step runs in 4-8 launches per layer
plus 3, and a chain whose buffers overlap in a way row-by-row execution would change runs unfused."""
import numpy as np
import pytest

import ckl
from oracle import decoder as oracle
from ckl.decoder_kernels import rms_apply, rms_stats
from ckl.library import linear_tiling
from programs.decoder_config import CONFIGS, Config
from programs.harness import MUTABLE, DecoderSession

pytestmark = pytest.mark.gpu

REFERENCE_SMALL = Config(batch=1, hidden=64, heads=4, layers=2, ffn=128, vocab=256, context=8, steps=16)
AWKWARD = Config(batch=3, hidden=48, heads=3, layers=1, ffn=80, vocab=129, context=3, steps=16)
# Rows not a multiple of 4 floats (scalar paths of the rms and silu chains), D = 14.
ODD = Config(batch=2, hidden=42, heads=3, layers=2, ffn=31, vocab=70, context=5, steps=6)
# Split reductions whose combine the chains take over: MFMA path (B > 16, splits 2 and 3) and
# vector path (B <= 16, reductions over 1024 rows).
SPLIT_MFMA = Config(batch=20, hidden=1024, heads=8, layers=1, ffn=1536, vocab=300, context=4, steps=3)
SPLIT_VECTOR = Config(batch=5, hidden=1280, heads=10, layers=1, ffn=1536, vocab=300, context=4, steps=3)
# Long cache rows for the other vector layouts of the attention (D = 64: 2 pieces a lane, D = 256:
# 16 lanes a row), so that every wave's key and value streams wrap their rings several times;
# and D = 96, whose rows take the sequential dot product and the scalar values loop.
HEAD64 = Config(batch=2, hidden=128, heads=2, layers=1, ffn=96, vocab=100, context=300, steps=4)
HEAD256 = Config(batch=2, hidden=512, heads=2, layers=1, ffn=64, vocab=100, context=150, steps=4)
HEAD96 = Config(batch=2, hidden=192, heads=2, layers=1, ffn=64, vocab=100, context=40, steps=4)


def whole_rows(b, i, o):
    """Row-parallel linear whose workgroup holds whole output rows (fuses with the row ops after it)."""
    t = linear_tiling(b, i, o)
    return t["entry"] == "ckl_linear_rowvec" and t["tiles"] == 1 and t["split"] == 1


def chained_launches(c):
    # embedding+rms; per layer: QKV, rope pair+append+scores+softmax+values, O, add+rms,
    # gate/up, silu+multiply, down, add+rms (O and down fused with their add+rms, gate/up with
    # silu+multiply, when row-parallel with one slice); then lm head, greedy+advance.
    o = 1 if whole_rows(c.batch, c.hidden, c.hidden) else 2
    down = 1 if whole_rows(c.batch, c.ffn, c.hidden) else 2
    t = linear_tiling(c.batch, c.hidden, c.ffn)
    gate_up = 1 if t["entry"] == "ckl_linear_rowvec" and t["split"] == 1 else 2
    # Both row chains of a layer as one launch when both linears are single-wave (C <= 64).
    single_wave = linear_tiling(c.batch, c.hidden, c.hidden)["block"] == 64 and t["block"] == 64
    merged = 1 if o == 1 and gate_up == 1 and single_wave else 0
    # embedding+rms and layer 0's q/k/v linears as one launch when C <= 64 (C % 4 == 0).
    qkv = linear_tiling(c.batch, c.hidden, c.hidden)
    first = 1 if c.hidden % 4 == 0 and c.hidden <= 64 and qkv["entry"] == "ckl_linear_rowvec" and qkv["split"] == 1 \
        and qkv["block"] == 64 else 0
    # The LM head, greedy and advance as one launch per row when the head is single-wave with at
    # most 16 column tiles.
    head = linear_tiling(c.batch, c.hidden, c.vocab)
    last = 1 if head["entry"] == "ckl_linear_rowvec" and head["split"] == 1 and head["block"] == 64 \
        and head["tiles"] <= 16 else 0
    return 1 + (2 + o + gate_up + down - merged) * c.layers + 2 - first - last


@pytest.mark.parametrize("config", [CONFIGS["small"], REFERENCE_SMALL, AWKWARD, ODD, SPLIT_MFMA, SPLIT_VECTOR, HEAD64,
                                    HEAD256, HEAD96],
                         ids=["small", "reference_small", "awkward", "odd", "split_mfma", "split_vector", "head64",
                              "head256", "head96"])
def test_chained_graph_is_bit_identical_to_ordinary(device, config):
    c = config
    initial, _ = oracle.make_inputs(c, 7, init="reference")
    session = DecoderSession(c, device, arrays=initial)
    reference = oracle.expected(initial, c, c.steps)
    for reuse, inv in session.invocations.items():
        launches = inv.launch_count(mode="graph", batch_size=1)
        # With storage reuse the executor moves a chain output that the plan placed in a chain
        # input's storage to memory of its own, so the same chains are taken; what it moves is
        # at most the temporaries' storage without reuse.
        assert launches == chained_launches(c), reuse
        if reuse:
            assert inv.private_bytes <= session.invocations[False].heap_bytes
        else:
            assert inv.private_bytes == 0
        if c.batch > 16:
            # q/k/v and gate/up multiply one x each: shared-operand launches of the MFMA path.
            names = [name for name, _ in inv.units()]
            assert sum(n.startswith("ckl_linear_mfma") and n.endswith("_shared3") for n in names) == c.layers
            assert sum(n.startswith("ckl_linear_mfma") and n.endswith("_shared2") for n in names) == c.layers
        assert inv.launch_count(mode="graph", batch_size=c.steps) == c.steps * launches
        results = {}
        for mode, group in (("ordinary", 1), ("graph", 1), ("graph", c.steps), ("stream", 1), ("stream", c.steps)):
            session.state.reset()
            for _ in range(c.steps // group):
                inv.run(mode=mode, batch_size=group)
            session.state.verify(reference)
            results[(mode, group)] = {name: session.state.download(name) for name in MUTABLE}
        for key in (("graph", 1), ("graph", c.steps), ("stream", 1), ("stream", c.steps)):
            for name in MUTABLE:
                assert np.array_equal(results[key][name], results[("ordinary", 1)][name]), (reuse, key, name)


_B, _C = ckl.dim("B"), ckl.dim("C")


@ckl.program
def normalize(x: ckl.Buffer[ckl.f32, (_B, _C)], inv: ckl.Buffer[ckl.f32, (_B,)],
              gain: ckl.Buffer[ckl.f32, (1, _C)], dst: ckl.Buffer[ckl.f32, (_B, _C)], eps: ckl.f32) -> None:
    ckl.launch(rms_stats, x, inv, eps, grid=(ckl.cdiv(_B, 32),), block=(32,))
    ckl.launch(rms_apply, x, inv, gain, dst, 0, grid=(ckl.cdiv(_C, 64), _B), block=(64,))


@pytest.mark.parametrize("overlap", [False, True], ids=["disjoint", "inv_aliases_gain"])
def test_rms_chain_respects_overlapping_buffers(device, overlap):
    b, c = 4, 64
    rng = np.random.default_rng(3)
    x = rng.standard_normal((b, c)).astype(np.float32)
    gain = rng.standard_normal((1, c)).astype(np.float32)
    sig = {"x": ckl.BufferSpec((b, c), ckl.f32), "inv": ckl.BufferSpec((b,), ckl.f32),
           "gain": ckl.BufferSpec((1, c), ckl.f32), "dst": ckl.BufferSpec((b, c), ckl.f32), "eps": ckl.f32}
    compiled = normalize.lower(signature=sig).compile(fuse_pointwise=False)
    assert '"ckl_rms_stats"' in compiled.executable_ir and '"ckl_rms_apply"' in compiled.executable_ir
    bx = device.empty(sig["x"])
    bg = device.empty(sig["gain"])
    bd = device.empty(sig["dst"])
    # With overlap, inv is the first B floats of gain: rms_apply must see the gains rms_stats
    # overwrote, which running row by row would not guarantee.
    bi = device.import_buffer(bg.address, sig["inv"], owner=bg) if overlap else device.empty(sig["inv"])
    inv = compiled.bind(bx, bi, bg, bd, 1e-5)
    assert inv.launch_count(mode="graph", batch_size=1) == (2 if overlap else 1)
    outputs = {}
    for mode in ("ordinary", "graph"):
        bx.copy_from_host(x)
        bg.copy_from_host(gain)
        inv.run(mode=mode)
        got = np.empty((b, c), np.float32)
        bd.copy_to_host(got)
        outputs[mode] = got
    assert np.array_equal(outputs["ordinary"], outputs["graph"])
    inverse = 1.0 / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1) + 1e-5)
    g = gain[0].astype(np.float64).copy()
    if overlap:
        g[:b] = inverse.astype(np.float32)
    expected = x * inverse[:, None] * g[None, :]
    assert np.allclose(outputs["ordinary"], expected, rtol=1e-5, atol=1e-6)
