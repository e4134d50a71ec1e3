"""Decoder step on the GPU against the NumPy oracle: exact tokens/history/position, f32 state
within atol 2e-5 / rtol 3e-4 and logits within 1e-4 relative to each row's largest reference
magnitude, for every run mode (ordinary, inferred graph, capture, and the two ablations: one graph
node per dispatch with the reduced DAG's branches, and the contracted launches captured on one
stream), storage reuse on/off and step grouping (benchmarks/decoder/run.py:107-197 protocol)."""
import numpy as np
import pytest

from oracle import decoder as oracle
from programs.decoder_config import CONFIGS, Config
from programs.harness import DecoderSession

pytestmark = pytest.mark.gpu

REFERENCE_SMALL = Config(batch=1, hidden=64, heads=4, layers=2, ffn=128, vocab=256, context=8, steps=16)
AWKWARD = Config(batch=3, hidden=48, heads=3, layers=1, ffn=80, vocab=129, context=3, steps=16)


MODES = ("ordinary", "graph", "capture", "branches", "contracted", "stream")


def run_and_check(device, c, init, steps, modes=MODES, groups=(1,)):
    initial, prompts = oracle.make_inputs(c, 123, init=init)
    session = DecoderSession(c, device, arrays=initial)
    references = {n: oracle.expected(initial, c, n) for n in {1, steps}}
    worst = 0.0
    for reuse, inv in session.invocations.items():
        for mode in modes:
            for group in groups:
                if steps % group:
                    continue
                session.state.reset()
                inv.run(mode=mode, batch_size=1)
                worst = max(worst, session.state.verify(references[1]))
                assert session.state.logits_normwise <= 1e-4
                session.state.reset()
                for _ in range(steps // group):
                    inv.run(mode=mode, batch_size=group)
                worst = max(worst, session.state.verify(references[steps]))
    return worst, session


@pytest.mark.parametrize("name", ["small", "wide", "deep"])
def test_baseline_configs_match_oracle(device, name):
    c = CONFIGS[name]
    worst, _ = run_and_check(device, c, "baseline", c.steps, groups=(1, 16))
    assert worst < 2e-5


@pytest.mark.parametrize("config", [REFERENCE_SMALL, AWKWARD], ids=["reference_small", "awkward"])
def test_reference_configs_match_oracle(device, config):
    worst, _ = run_and_check(device, config, "reference", config.steps, groups=(1, 4))
    assert worst < 2e-5


@pytest.mark.parametrize("name", ["small", "wide", "deep"])
def test_branch_graph_is_the_reduced_dispatch_dag(device, name):
    """Mode "branches" has one kernel node per dispatch (21L + 6) and exactly the reduced DAG's
    dependency edges (24L + 5: 53 small/wide, 197 deep, as recorded by the reference)."""
    c = CONFIGS[name]
    initial, _ = oracle.make_inputs(c, 123, init="baseline")
    session = DecoderSession(c, device, arrays=initial)
    for inv in session.invocations.values():
        assert inv.launch_count(mode="branches") == 21 * c.layers + 6
        assert inv.edge_count(mode="branches") == 24 * c.layers + 5
        assert inv.edge_count(mode="capture") == 0
        assert inv.launch_count(mode="contracted") == inv.launch_count(mode="graph")
        assert inv.launch_count(mode="stream") == inv.launch_count(mode="graph")
        assert inv.edge_count(mode="stream") == 0
